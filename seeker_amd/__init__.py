"""seeker_amd: MI355X (gfx950) speculative-decoding verify path for seeker.

The product is libseeker_hip.so (hand-written HIP kernels behind the C ABI in
include/seeker_hip.h). This package binds it with ctypes and mirrors the
reference's Engine / KvCache / Sampler surface for Python callers and tests.
"""
from . import _native
from ._native import SeekerError, lib
from .inference import Engine, KvCache, Model, QTensor, SamplerConfig, SpecStepOut

__all__ = ["Engine", "KvCache", "Model", "QTensor", "SamplerConfig", "SpecStepOut", "SeekerError", "lib", "_native"]
