"""ctypes binding of libseeker_hip.so (include/seeker_hip.h) and libseeker_synth.so.

This is the Python face of the C ABI, the same surface a Rust crate binds with
bindgen. Loading fails loudly when the built library is missing: there is no
CPU fallback for any entry point.
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libseeker_hip.so")
SYNTH_PATH = os.path.join(_HERE, "libseeker_synth.so")

# enum sh_status
SH_OK, SH_ERR_ARG, SH_ERR_HIP, SH_ERR_FORMAT, SH_ERR_UNSUPPORTED, SH_ERR_CAPACITY, SH_ERR_STATE = range(7)
# enum sh_sample_mode
SH_SAMPLE_GREEDY, SH_SAMPLE_COMPARE, SH_SAMPLE_REJECTION = 0, 1, 2
GGML_F32, GGML_F16, GGML_Q8_0, GGML_Q4_K, GGML_Q5_K, GGML_Q6_K = 0, 1, 8, 12, 13, 14


class SeekerError(RuntimeError):
    """Raised when a C entry point returns a non-zero status."""

    def __init__(self, status: int, message: str):
        super().__init__(f"[{status}] {message}")
        self.status = status


class sh_sampling(C.Structure):
    _fields_ = [
        ("mode", C.c_uint32),
        ("temperature", C.c_float),
        ("seed", C.c_uint64),
        ("counter", C.c_uint64),
        ("uniforms", C.POINTER(C.c_float)),
        ("top_k", C.c_uint32),
        ("top_p", C.c_float),
        ("min_p", C.c_float),
        ("reserved", C.c_uint32),
    ]


class sh_model_dims(C.Structure):
    _fields_ = [
        ("n_layer", C.c_uint32), ("n_embd", C.c_uint32), ("n_head", C.c_uint32),
        ("n_head_kv", C.c_uint32), ("head_dim", C.c_uint32), ("n_ff", C.c_uint32),
        ("n_vocab", C.c_uint32), ("n_ctx_train", C.c_uint32),
        ("rms_eps", C.c_float), ("rope_freq_base", C.c_float),
        ("weight_type", C.c_int32), ("weight_bytes", C.c_double),
    ]


class sh_kernel_stat(C.Structure):
    _fields_ = [
        ("name", C.c_char * 48),
        ("launches", C.c_uint64),
        ("total_ms", C.c_double),
        ("alg_bytes", C.c_double),
    ]


class sh_synth_cfg(C.Structure):
    _fields_ = [
        ("arch", C.c_uint32),
        ("n_layer", C.c_uint32), ("n_embd", C.c_uint32), ("n_head", C.c_uint32),
        ("n_head_kv", C.c_uint32), ("head_dim", C.c_uint32), ("n_ff", C.c_uint32), ("n_vocab", C.c_uint32),
        ("n_ctx", C.c_uint32), ("n_expert", C.c_uint32), ("n_expert_used", C.c_uint32), ("expert_ff", C.c_uint32),
        ("rms_eps", C.c_float), ("rope_base", C.c_float), ("weight_std", C.c_float),
        ("norm_jitter", C.c_float), ("router_std", C.c_float),
        ("wtype", C.c_uint32), ("etype", C.c_uint32), ("tied", C.c_uint32),
        ("seed", C.c_uint64), ("out_type", C.c_uint32), ("mix", C.c_uint32),
    ]


class sh_synth_llama_cfg(C.Structure):
    _fields_ = [
        ("n_layer", C.c_uint32), ("n_embd", C.c_uint32), ("n_head", C.c_uint32),
        ("n_head_kv", C.c_uint32), ("n_ff", C.c_uint32), ("n_vocab", C.c_uint32),
        ("n_ctx", C.c_uint32),
        ("rms_eps", C.c_float), ("rope_base", C.c_float), ("weight_std", C.c_float),
        ("wtype", C.c_uint32), ("etype", C.c_uint32), ("tied", C.c_uint32),
        ("seed", C.c_uint64),
    ]


P = C.c_void_p
U32P = C.POINTER(C.c_uint32)
I32P = C.POINTER(C.c_int32)
F32P = C.POINTER(C.c_float)
U16P = C.POINTER(C.c_uint16)

# name -> (restype, argtypes); every symbol include/seeker_hip.h declares.
SIGNATURES = {
    "sh_last_error": (C.c_char_p, []),
    "sh_version": (C.c_char_p, []),
    "sh_engine_create": (C.c_int, [C.c_int, C.POINTER(P)]),
    "sh_engine_destroy": (None, [P]),
    "sh_engine_sync": (C.c_int, [P]),
    "sh_engine_set_profiling": (C.c_int, [P, C.c_int]),
    "sh_engine_profile": (C.c_int, [P, C.POINTER(sh_kernel_stat), C.c_uint32, U32P]),
    "sh_engine_profile_reset": (C.c_int, [P]),
    "sh_engine_graph_stats": (C.c_int, [P, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
    "sh_dev_alloc": (C.c_int, [P, C.c_uint64, C.POINTER(P)]),
    "sh_dev_free": (C.c_int, [P, P]),
    "sh_memcpy_h2d": (C.c_int, [P, P, P, C.c_uint64]),
    "sh_memcpy_d2h": (C.c_int, [P, P, P, C.c_uint64]),
    "sh_model_load_gguf": (C.c_int, [P, C.c_char_p, C.POINTER(P)]),
    "sh_model_load_gguf_memory": (C.c_int, [P, P, C.c_uint64, C.POINTER(P)]),
    "sh_model_destroy": (None, [P]),
    "sh_model_info": (C.c_int, [P, C.POINTER(sh_model_dims)]),
    "sh_model_wide_f16": (C.c_int, [P, C.POINTER(C.c_int)]),
    "sh_model_set_wide_f16": (C.c_int, [P, C.c_int]),
    "sh_model_cm1_attention": (C.c_int, [P, C.POINTER(C.c_int)]),
    "sh_model_set_cm1_attention": (C.c_int, [P, C.c_int]),
    "sh_gguf_inspect": (C.c_int, [P, C.c_uint64, C.POINTER(sh_model_dims)]),
    "sh_kv_create": (C.c_int, [P, P, C.c_uint32, C.POINTER(P)]),
    "sh_kv_destroy": (None, [P]),
    "sh_kv_position": (C.c_int, [P, U32P]),
    "sh_kv_truncate": (C.c_int, [P, C.c_uint32]),
    "sh_kv_read_layer": (C.c_int, [P, C.c_uint32, C.c_int, C.c_uint32, U16P]),
    "sh_kv_write_layer": (C.c_int, [P, C.c_uint32, C.c_int, C.c_uint32, U16P]),
    "sh_kv_set_position": (C.c_int, [P, C.c_uint32]),
    "sh_kv_compact": (C.c_int, [P, C.c_uint32, U32P, C.c_uint32]),
    "sh_forward_full": (C.c_int, [P, P, P, U32P, C.c_uint32, C.c_uint32, I32P, C.c_int, F32P, F32P]),
    "sh_verify_greedy": (C.c_int, [P, P, P, U32P, C.c_uint32, C.c_uint32, U32P]),
    "sh_verify_unified": (C.c_int, [P, P, C.POINTER(P), C.c_uint32, U32P, U32P, U32P, I32P, F32P, U32P, F32P]),
    "sh_verify_unified_sampled": (C.c_int, [P, P, C.POINTER(P), C.c_uint32, U32P, U32P, U32P, I32P,
                                            P, F32P, U32P, F32P]),
    "sh_draft_tokens": (C.c_int, [P, P, P, C.c_uint32, C.c_uint32, U32P]),
    "sh_spec_step_forced": (C.c_int, [P, P, P, P, P, C.c_uint32, C.c_uint32, U32P, U32P, C.POINTER(C.c_uint32)]),
    "sh_spec_step_batch": (C.c_int, [P, P, P, C.POINTER(P), C.POINTER(P), C.c_uint32, U32P, C.c_uint32, P, U32P, U32P,
                                     U32P]),
    "sh_spec_step": (C.c_int, [P, P, P, P, P, C.c_uint32, C.c_uint32, C.POINTER(sh_sampling), U32P, U32P, U32P]),
    "sh_spec_step_logits": (C.c_int, [P, F32P, F32P, U32P, U32P]),
    "sh_accept_sample_noalloc": (C.c_int, [P, P, P, P, C.c_uint32, C.c_uint32, C.c_uint32, C.POINTER(sh_sampling),
                                           P, P]),
    "sh_accept_probs": (C.c_int, [P, P, P, P, C.c_uint32, C.c_uint32, C.c_uint32, C.c_float, P]),
    "sh_qtensor_upload": (C.c_int, [P, C.c_int, P, C.c_uint32, C.c_uint32, C.POINTER(P)]),
    "sh_qtensor_destroy": (None, [P]),
    "sh_gemv_quant": (C.c_int, [P, P, P, C.c_uint32, P, C.c_int]),
    "sh_gemm_wide16": (C.c_int, [P, P, P, C.c_uint32, P, C.c_int]),
    "sh_accept_sample": (C.c_int, [P, P, P, P, C.c_uint32, C.c_uint32, C.c_uint32, C.POINTER(sh_sampling), P, P]),
    "sh_tree_accept": (C.c_int, [P, P, P, P, P, C.c_uint32, C.c_uint32, C.c_uint32, C.POINTER(sh_sampling), P, P, P]),
    "sh_tree_verify_step": (C.c_int, [P, P, C.POINTER(P), C.c_uint32, C.c_uint32, U32P, I32P, P,
                                      C.POINTER(sh_sampling), U32P, U32P, U32P]),
}

SYNTH_SIGNATURES = {
    "sh_synth_gguf": (C.c_int, [C.POINTER(sh_synth_cfg), C.POINTER(C.POINTER(C.c_uint8)), C.POINTER(C.c_uint64)]),
    "sh_synth_llama_gguf": (C.c_int, [C.POINTER(sh_synth_llama_cfg), C.POINTER(C.POINTER(C.c_uint8)),
                                      C.POINTER(C.c_uint64)]),
    "sh_synth_free": (None, [P]),
    "sh_synth_tokens": (None, [C.c_uint64, C.c_uint32, C.c_uint32, U32P]),
    "sh_synth_normal_f32": (None, [C.c_uint64, C.c_uint64, C.c_float, C.c_float, C.c_uint64, F32P]),
    "sh_synth_quantize": (C.c_int, [C.c_uint32, F32P, C.c_uint64, C.POINTER(C.c_uint8)]),
}

_lib = None
_synth = None


def _bind(path, sigs):
    if not os.path.exists(path):
        raise SeekerError(SH_ERR_ARG, f"{path} is not built; run __graft_entry__.build() (no CPU fallback exists)")
    lib = C.CDLL(path)
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def lib():
    """The loaded libseeker_hip.so (raises if it is not built)."""
    global _lib
    if _lib is None:
        _lib = _bind(LIB_PATH, SIGNATURES)
    return _lib


def synth():
    global _synth
    if _synth is None:
        _synth = _bind(SYNTH_PATH, SYNTH_SIGNATURES)
    return _synth


def check(status: int):
    if status != SH_OK:
        msg = lib().sh_last_error()
        raise SeekerError(status, msg.decode() if msg else "unknown error")
