"""Synthetic inputs: Llama / Qwen3 / Qwen3-MoE GGUF images with N(0, std)
weights and random prompts.

The configurations of BASELINE.json are reproduced here by name. Weights are
quantized by the generator in csrc/synth.cpp; the reference reads GGUF files
and never quantizes, so these bytes are inputs shared by the GPU path and the
CPU oracle, not a parity target.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _native as N


@dataclass(frozen=True)
class LlamaShape:
    n_layer: int
    n_embd: int
    n_head: int
    n_head_kv: int
    n_ff: int
    n_vocab: int
    n_ctx: int = 8192
    rms_eps: float = 1e-5
    rope_base: float = 10000.0
    weight_std: float = 0.02
    wtype: int = N.GGML_Q4_K
    etype: int = N.GGML_Q4_K
    tied: bool = False
    arch: int = 0            # 0 llama, 1 qwen3, 2 qwen3moe
    head_dim: int = 0        # 0: n_embd / n_head
    n_expert: int = 0
    n_expert_used: int = 0
    expert_ff: int = 0
    norm_jitter: float = 0.0  # norm weights 1 + jitter * N(0, 1) (0: all ones)
    router_std: float = 0.0   # f32 router weights N(0, router_std)
    out_type: int = 0         # output.weight type (0: wtype)
    mix: int = 0              # 1: attn_v / ffn_down(_exps) of even layers in Q6_K (Q4_K_M-style)


# tiny Llama target / 1-layer draft, Q8_0.
TINY_TARGET = LlamaShape(4, 512, 8, 8, 1408, 32000, 1024, 1e-5, 1e4, 0.02, N.GGML_Q8_0, N.GGML_Q8_0)
TINY_DRAFT = LlamaShape(1, 512, 8, 8, 1408, 32000, 1024, 1e-5, 1e4, 0.02, N.GGML_Q8_0, N.GGML_Q8_0)
# Llama-3-8B-shape target, Llama-3.2-1B-shape draft (tied), Q4_K.
L8B_TARGET = LlamaShape(32, 4096, 32, 8, 14336, 128256, 8192, 1e-5, 5e5, 0.02, N.GGML_Q4_K, N.GGML_Q4_K)
L1B_DRAFT = LlamaShape(16, 2048, 32, 8, 8192, 128256, 8192, 1e-5, 5e5, 0.02, N.GGML_Q4_K, N.GGML_Q4_K, True)
# Qwen3-30B-A3B-shape MoE target (router logits ~ N(0, 1): f32 router
# weights N(0, 1/sqrt(n_embd)) against a unit-RMS normalized input) and the
# Qwen3-0.6B-shape draft (tied embeddings), Q4_K.
Q30B_A3B_TARGET = LlamaShape(48, 2048, 32, 4, 0, 151936, 40960, 1e-6, 1e6, 0.02, N.GGML_Q4_K, N.GGML_Q4_K, False,
                             arch=2, head_dim=128, n_expert=128, n_expert_used=8, expert_ff=768, norm_jitter=0.1,
                             router_std=2048 ** -0.5)
Q06B_DRAFT = LlamaShape(28, 1024, 16, 8, 3072, 151936, 40960, 1e-6, 1e6, 0.02, N.GGML_Q4_K, N.GGML_Q4_K, True,
                        arch=1, head_dim=128, norm_jitter=0.1)


class GgufImage:
    """A GGUF byte image owned by the synth library (freed on close)."""

    def __init__(self, shape: LlamaShape, seed: int):
        cfg = N.sh_synth_cfg(
            shape.arch, shape.n_layer, shape.n_embd, shape.n_head, shape.n_head_kv, shape.head_dim, shape.n_ff,
            shape.n_vocab, shape.n_ctx, shape.n_expert, shape.n_expert_used, shape.expert_ff, shape.rms_eps,
            shape.rope_base, shape.weight_std, shape.norm_jitter, shape.router_std, shape.wtype, shape.etype,
            int(shape.tied), seed, shape.out_type, shape.mix)
        ptr = C.POINTER(C.c_uint8)()
        size = C.c_uint64()
        rc = N.synth().sh_synth_gguf(C.byref(cfg), C.byref(ptr), C.byref(size))
        if rc:
            raise N.SeekerError(rc, f"synthetic GGUF generation failed ({shape})")
        self.shape = shape
        self.seed = seed
        self.ptr = ptr
        self.size = size.value

    @property
    def address(self) -> int:
        return C.cast(self.ptr, C.c_void_p).value

    def bytes(self) -> np.ndarray:
        """Zero-copy uint8 view of the image."""
        return np.ctypeslib.as_array(self.ptr, shape=(self.size,))

    def close(self):
        if self.ptr:
            N.synth().sh_synth_free(C.cast(self.ptr, C.c_void_p))
            self.ptr = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def tokens(seed: int, n: int, vocab: int) -> np.ndarray:
    out = np.zeros(n, dtype=np.uint32)
    N.synth().sh_synth_tokens(seed, n, vocab, out.ctypes.data_as(N.U32P))
    return out


def normal_f32(seed: int, stream: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    N.synth().sh_synth_normal_f32(seed, stream, mean, std, n, out.ctypes.data_as(N.F32P))
    return out


def quantize(qtype: int, x: np.ndarray) -> np.ndarray:
    """Quantize a flat f32 array (rows contiguous) to GGUF Q8_0 / Q4_K / Q5_K / Q6_K blocks."""
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    blk, bb = {N.GGML_Q4_K: (256, 144), N.GGML_Q5_K: (256, 176), N.GGML_Q6_K: (256, 210)}.get(qtype, (32, 34))
    out = np.zeros(x.size // blk * bb, dtype=np.uint8)
    rc = N.synth().sh_synth_quantize(qtype, x.ctypes.data_as(N.F32P), x.size,
                                     out.ctypes.data_as(C.POINTER(C.c_uint8)))
    if rc:
        raise N.SeekerError(rc, "quantize: bad size or type")
    return out
