"""ctypes wrapper of the CPU oracle (oracle/_build/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker. The product path
(seeker_amd / libseeker_hip.so) never imports or calls it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(_HERE, "_build", "liboracle.so")

P = C.c_void_p
U32P = C.POINTER(C.c_uint32)
I32P = C.POINTER(C.c_int32)
F32P = C.POINTER(C.c_float)
U64P = C.POINTER(C.c_uint64)
U16P = C.POINTER(C.c_uint16)
U8P = C.POINTER(C.c_uint8)


class SamplerCfg(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_uint32), ("top_p", C.c_float), ("min_p", C.c_float)]


_SIGS = {
    "or_f16_to_f32": (C.c_float, [C.c_uint16]),
    "or_f32_to_f16": (C.c_uint16, [C.c_float]),
    "or_philox4x64_10": (None, [U64P, U64P, U64P]),
    "or_philox_word": (C.c_uint64, [C.c_uint64, C.c_uint64, C.c_uint64]),
    "or_unit_f32": (C.c_float, [C.c_uint64]),
    "or_dequant_row": (C.c_int, [C.c_int, U8P, C.c_uint64, C.c_uint64, F32P]),
    "or_gemv": (C.c_int, [C.c_int, U8P, C.c_uint64, C.c_uint64, F32P, C.c_uint32, F32P]),
    "or_gemv16": (C.c_int, [C.c_int, U8P, C.c_uint64, C.c_uint64, F32P, C.c_uint32, F32P]),
    "or_model_set_mm16": (None, [P, C.c_int]),
    "or_model_set_attn_cm1": (None, [P, C.c_int]),
    "or_f64_to_f16": (C.c_uint16, [C.c_double]),
    "or_attn_cm1": (None, [F32P, U16P, U16P, C.c_size_t, C.c_uint32, C.c_uint32, U8P, F32P]),
    "or_attn_cm1_core": (None, [U16P, U16P, U16P, C.c_size_t, C.c_uint32, C.c_uint32, U8P, F32P]),
    "or_model_open": (C.c_int, [P, C.c_uint64, C.POINTER(P)]),
    "or_model_free": (None, [P]),
    "or_model_dims": (None, [P, U32P]),
    "or_model_moe_dims": (None, [P, U32P]),
    "or_moe_route": (None, [F32P, C.c_uint32, C.c_uint32, U32P, F32P]),
    "or_kv_create": (C.c_int, [P, C.c_uint32, C.POINTER(P)]),
    "or_kv_free": (None, [P]),
    "or_kv_position": (C.c_uint32, [P]),
    "or_kv_truncate": (None, [P, C.c_uint32]),
    "or_kv_set_position": (None, [P, C.c_uint32]),
    "or_kv_layer": (U16P, [P, C.c_uint32, C.c_int]),
    "or_kv_compact": (None, [P, C.c_uint32, U32P, C.c_uint32]),
    "or_forward": (C.c_int, [P, P, U32P, C.c_uint32, C.c_uint32, I32P, C.c_int, F32P, F32P]),
    "or_argmax": (C.c_uint32, [F32P, C.c_uint32]),
    "or_softmax": (None, [F32P, C.c_uint32, F32P]),
    "or_sample_one": (C.c_uint32, [F32P, C.c_uint32, C.POINTER(SamplerCfg), C.c_float]),
    "or_sample_vocab_order": (C.c_uint32, [F32P, C.c_uint32, C.c_float, C.c_float]),
    "or_sample_and_compare": (C.c_uint32, [F32P, C.c_uint32, U32P, C.c_uint32, C.POINTER(SamplerCfg), F32P, C.c_int,
                                           U32P]),
    "or_rejection": (C.c_uint32, [F32P, F32P, U32P, C.c_uint32, C.c_uint32, C.c_float, F32P, F32P, U32P]),
    "or_tree_accept": (C.c_int, [F32P, F32P, U32P, I32P, C.c_uint32, C.c_uint32, C.c_float, F32P, U32P, U32P, U32P]),
    "or_probs": (None, [F32P, C.c_uint32, C.c_float, F32P]),
    "or_spec_step_greedy": (C.c_int, [P, P, P, P, C.c_uint32, C.c_uint32, U32P, U32P, U32P, U32P, U32P]),
    "or_spec_draft_token": (C.c_uint32, [C.c_int, F32P, C.c_uint32, C.c_float, C.c_float]),
    "or_spec_accept": (C.c_uint32, [C.c_int, F32P, F32P, U32P, C.c_uint32, C.c_uint32, C.c_float, F32P, U32P]),
    "or_spec_step": (C.c_int, [P, P, P, P, C.c_uint32, C.c_uint32, C.c_int, C.c_float, F32P, U32P, U32P, U32P, U32P,
                               U32P, F32P, F32P]),
}

_lib = None
_lib_fast = None
LIB_FAST = os.path.join(_HERE, "_build", "liboracle_fast.so")


def build():
    subprocess.run(["make", "-s", "-B", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        L = C.CDLL(LIB)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def lib_fast():
    """The timing build (f32 accumulation, -O3 AVX2/FMA) for the CPU baseline; it
    shares the check build's object layouts, so models and caches opened by one
    may be passed to the other."""
    global _lib_fast
    if _lib_fast is None:
        if not os.path.exists(LIB_FAST):
            build()
        L = C.CDLL(LIB_FAST)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib_fast = L
    return _lib_fast


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def dequant_row(qtype: int, raw: np.ndarray, row: int, k: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.empty(k, dtype=np.float32)
    if lib().or_dequant_row(qtype, raw.ctypes.data_as(U8P), row, k, out.ctypes.data_as(F32P)):
        raise ValueError("dequant failed")
    return out


def gemv(qtype: int, w: np.ndarray, M: int, K: int, x: np.ndarray) -> np.ndarray:
    """x [N][K] -> y [N][M] with f64 accumulation."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = _f32(x).reshape(-1, K)
    y = np.empty((x.shape[0], M), dtype=np.float32)
    if lib().or_gemv(qtype, w.ctypes.data_as(U8P), M, K, x.ctypes.data_as(F32P), x.shape[0], y.ctypes.data_as(F32P)):
        raise ValueError("gemv failed")
    return y


def gemv16(qtype: int, w: np.ndarray, M: int, K: int, x: np.ndarray) -> np.ndarray:
    """x [N][K] -> y [N][M] with the wide GEMM's f16 weights and activations
    (or_gemv16), f64 accumulation."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = _f32(x).reshape(-1, K)
    y = np.empty((x.shape[0], M), dtype=np.float32)
    if lib().or_gemv16(qtype, w.ctypes.data_as(U8P), M, K, x.ctypes.data_as(F32P), x.shape[0],
                       y.ctypes.data_as(F32P)):
        raise ValueError("gemv16 failed")
    return y


def philox_block(ctr, key):
    c = (C.c_uint64 * 4)(*ctr)
    k = (C.c_uint64 * 2)(*key)
    o = (C.c_uint64 * 4)()
    lib().or_philox4x64_10(c, k, o)
    return list(o)


def philox_uniforms(seed: int, stream: int, start: int, n: int) -> np.ndarray:
    L = lib()
    return np.array([L.or_unit_f32(L.or_philox_word(seed, stream, start + i)) for i in range(n)], dtype=np.float32)


class Model:
    def __init__(self, image):
        """image: synth.GgufImage (kept alive by the caller)."""
        self.image = image
        h = C.c_void_p()
        rc = lib().or_model_open(C.c_void_p(image.address), image.size, C.byref(h))
        if rc:
            raise ValueError(f"oracle model open failed ({rc})")
        self.h = h
        d = (C.c_uint32 * 7)()
        lib().or_model_dims(h, d)
        self.n_layer, self.d, self.n_head, self.n_kv, self.hd, self.ff, self.V = list(d)
        e = (C.c_uint32 * 4)()
        lib().or_model_moe_dims(h, e)
        self.arch, self.n_expert, self.n_used, self.expert_ff = list(e)
        self.attn_cm1 = False

    def set_mm16(self, mode):
        """Dense matmuls of later forwards with the wide GEMM's f16 operands:
        False / 0 never, True / 1 always, 2 in forward calls of >= 32 columns
        (the reference's dispatch, ops/matmul.rs:433-446)."""
        lib().or_model_set_mm16(self.h, int(mode))

    def set_attn_cm1(self, on):
        """Causal forward calls of more than one column compute attention with
        the reference's cooperative-matrix flash attention arithmetic
        (or_attn_cm1: flash_attn_cm1.slang, ops/flash_attn.rs:442-471)."""
        self.attn_cm1 = bool(on)
        lib().or_model_set_attn_cm1(self.h, int(bool(on)))

    def close(self):
        if self.h:
            lib().or_model_free(self.h)
            self.h = None


def attn_cm1(q, k16, v16, visible=None, staged=False) -> np.ndarray:
    """or_attn_cm1 over keys k16 / v16 [n_keys][hd] (uint16 f16 bits) for one
    query row q [hd]: f32 values staged to f16 by the shader's scale, or (staged)
    the staged f16 bits themselves (or_attn_cm1_core)."""
    k16 = np.ascontiguousarray(k16, dtype=np.uint16)
    v16 = np.ascontiguousarray(v16, dtype=np.uint16)
    n, hd = k16.shape
    out = np.empty(hd, np.float32)
    vis = np.ascontiguousarray(visible, dtype=np.uint8) if visible is not None else None
    vp = vis.ctypes.data_as(U8P) if vis is not None else None
    if staged:
        q16 = np.ascontiguousarray(q, dtype=np.uint16)
        lib().or_attn_cm1_core(q16.ctypes.data_as(U16P), k16.ctypes.data_as(U16P), v16.ctypes.data_as(U16P), hd, hd,
                               n, vp, out.ctypes.data_as(F32P))
    else:
        qq = _f32(q)
        lib().or_attn_cm1(qq.ctypes.data_as(F32P), k16.ctypes.data_as(U16P), v16.ctypes.data_as(U16P), hd, hd, n, vp,
                          out.ctypes.data_as(F32P))
    return out


class KvCache:
    def __init__(self, model: Model, max_seq: int):
        h = C.c_void_p()
        if lib().or_kv_create(model.h, max_seq, C.byref(h)):
            raise MemoryError("oracle kv alloc")
        self.h, self.model, self.max_seq = h, model, max_seq
        self.pending = (C.c_uint32 * 16)()
        self.n_pending = C.c_uint32(0)

    @property
    def position(self):
        return lib().or_kv_position(self.h)

    def truncate(self, p):
        lib().or_kv_truncate(self.h, p)

    def set_position(self, p):
        lib().or_kv_set_position(self.h, p)

    def layer(self, layer: int, is_v: bool, n_pos: int) -> np.ndarray:
        m = self.model
        ptr = lib().or_kv_layer(self.h, layer, int(is_v))
        full = np.ctypeslib.as_array(ptr, shape=(self.max_seq, m.n_kv, m.hd))
        return full[:n_pos]

    def compact(self, base, src):
        s = np.ascontiguousarray(src, dtype=np.uint32)
        lib().or_kv_compact(self.h, base, s.ctypes.data_as(U32P), s.size)

    def close(self):
        if self.h:
            lib().or_kv_free(self.h)
            self.h = None


def forward(model: Model, kv: KvCache, tokens, pos: int, parents=None, logits_mode: int = 2, batched=False):
    """or_forward. batched: the call stands for one sequence of a batched
    verify, whose attention is the reference's scalar kernel
    (ops/flash_attn.rs:819-1016) whatever set_attn_cm1 says."""
    if batched:
        lib().or_model_set_attn_cm1(model.h, 0)
        try:
            return forward(model, kv, tokens, pos, parents, logits_mode)
        finally:
            lib().or_model_set_attn_cm1(model.h, int(bool(model.attn_cm1)))
    t = np.ascontiguousarray(tokens, dtype=np.uint32)
    L = t.size
    cols = L if logits_mode == 2 else (1 if logits_mode == 1 else 0)
    logits = np.empty((max(cols, 1), model.V), dtype=np.float32)
    resid = np.empty((L, model.d), dtype=np.float32)
    par = np.ascontiguousarray(parents, dtype=np.int32) if parents is not None else None
    rc = lib().or_forward(model.h, kv.h, t.ctypes.data_as(U32P), L, pos,
                          par.ctypes.data_as(I32P) if par is not None else None, logits_mode,
                          logits.ctypes.data_as(F32P), resid.ctypes.data_as(F32P))
    if rc:
        raise ValueError(f"oracle forward failed ({rc})")
    return logits[:cols], resid


def moe_route(logits, k: int):
    """or_moe_route: (ids [k], weights [k]) of one column's router logits."""
    lg = _f32(logits)
    ids = np.zeros(k, np.uint32)
    w = np.zeros(k, np.float32)
    lib().or_moe_route(lg.ctypes.data_as(F32P), lg.size, k, ids.ctypes.data_as(U32P), w.ctypes.data_as(F32P))
    return ids, w


def argmax(x) -> int:
    x = _f32(x)
    return int(lib().or_argmax(x.ctypes.data_as(F32P), x.size))


def softmax(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty_like(x)
    lib().or_softmax(x.ctypes.data_as(F32P), x.size, out.ctypes.data_as(F32P))
    return out


def probs(x, temperature: float) -> np.ndarray:
    x = _f32(x)
    out = np.empty_like(x)
    lib().or_probs(x.ctypes.data_as(F32P), x.size, temperature, out.ctypes.data_as(F32P))
    return out


def sample_one(logits, cfg: SamplerCfg, u: float) -> int:
    x = _f32(logits)
    return int(lib().or_sample_one(x.ctypes.data_as(F32P), x.size, C.byref(cfg), u))


def sample_vocab_order(logits, temperature: float, u: float) -> int:
    x = _f32(logits)
    return int(lib().or_sample_vocab_order(x.ctypes.data_as(F32P), x.size, temperature, u))


def sample_and_compare(logits, drafts, cfg: SamplerCfg, uniforms, mode: int = 1):
    lg = _f32(logits)
    n = len(drafts)
    V = lg.shape[-1]
    d = np.ascontiguousarray(drafts, dtype=np.uint32)
    u = _f32(uniforms)
    em = np.zeros(n + 1, dtype=np.uint32)
    ne = lib().or_sample_and_compare(lg.ctypes.data_as(F32P), V, d.ctypes.data_as(U32P), n, C.byref(cfg),
                                     u.ctypes.data_as(F32P), mode, em.ctypes.data_as(U32P))
    return em[:ne].tolist()


def rejection(p_logits, q_logits, drafts, temperature, u_acc, u_res):
    p = _f32(p_logits)
    q = _f32(q_logits)
    k = len(drafts)
    V = p.shape[-1]
    d = np.ascontiguousarray(drafts, dtype=np.uint32)
    ua, ur = _f32(u_acc), _f32(u_res)
    nt = C.c_uint32()
    acc = lib().or_rejection(p.ctypes.data_as(F32P), q.ctypes.data_as(F32P), d.ctypes.data_as(U32P), k, V,
                             temperature, ua.ctypes.data_as(F32P), ur.ctypes.data_as(F32P), C.byref(nt))
    return int(acc), int(nt.value)


def tree_accept(p_logits, q_logits, tokens, parents, temperature, u):
    """Tree acceptance (or_tree_accept): returns (path list of node indices, next token).
    p_logits, q_logits [n][V]; u [n][2] (accept, draw) uniforms; temperature 0 = greedy."""
    p = _f32(p_logits)
    q = _f32(q_logits)
    n, V = p.shape
    t = np.ascontiguousarray(tokens, dtype=np.uint32)
    par = np.ascontiguousarray(parents, dtype=np.int32)
    uu = _f32(u).reshape(-1)
    path = np.zeros(n, dtype=np.uint32)
    plen, nt = C.c_uint32(), C.c_uint32()
    rc = lib().or_tree_accept(p.ctypes.data_as(F32P), q.ctypes.data_as(F32P), t.ctypes.data_as(U32P),
                              par.ctypes.data_as(I32P), n, V, temperature, uu.ctypes.data_as(F32P),
                              path.ctypes.data_as(U32P), C.byref(plen), C.byref(nt))
    if rc:
        raise ValueError("oracle tree_accept: malformed tree")
    return path[: plen.value].tolist(), int(nt.value)


def spec_step_greedy(tgt: Model, drf: Model, tkv: KvCache, dkv: KvCache, last_token: int, n_max: int,
                     fast: bool = False):
    """or_spec_step_greedy; fast=True runs the timing build (f32 accumulation)."""
    em = (C.c_uint32 * 9)()
    dr = (C.c_uint32 * 8)()
    ne = C.c_uint32()
    rc = (lib_fast() if fast else lib()).or_spec_step_greedy(tgt.h, drf.h, tkv.h, dkv.h, last_token, n_max, dkv.pending,
                                   C.byref(dkv.n_pending), em, C.byref(ne), dr)
    if rc:
        raise ValueError(f"oracle spec step failed ({rc})")
    n = min(max(n_max, 1), 8)
    return list(em)[: ne.value], list(dr)[:n]


SPEC_GREEDY, SPEC_COMPARE, SPEC_REJECTION = 0, 1, 2


def spec_uniforms(seed: int, counter: int, n: int) -> np.ndarray:
    """The uniforms a speculative step of n drafts consumes from Philox key
    (seed, 0x5EC) at word counter: 2(n+1) for the verify columns, then n for
    the draft draws (sh_spec_step's layout)."""
    return philox_uniforms(seed, 0x5EC, counter, 3 * n + 2)


def spec_draft_token(mode: int, q_logits, T: float, u: float) -> int:
    q = _f32(q_logits)
    return int(lib().or_spec_draft_token(mode, q.ctypes.data_as(F32P), q.size, T, u))


def spec_accept(mode: int, p_logits, q_logits, drafts, T: float, u) -> list:
    p = _f32(p_logits)
    n = len(drafts)
    V = p.shape[-1]
    q = _f32(q_logits) if q_logits is not None else np.zeros((max(n, 1), V), np.float32)
    d = np.ascontiguousarray(drafts, dtype=np.uint32)
    uu = _f32(u) if u is not None else np.zeros(2 * (n + 1), np.float32)
    em = np.zeros(n + 1, dtype=np.uint32)
    ne = lib().or_spec_accept(mode, p.ctypes.data_as(F32P), q.ctypes.data_as(F32P), d.ctypes.data_as(U32P), n, V, T,
                              uu.ctypes.data_as(F32P), em.ctypes.data_as(U32P))
    return em[:ne].tolist()


def spec_step(tgt: Model, drf: Model, tkv: KvCache, dkv: KvCache, last_token: int, n_max: int, mode: int = 0,
              T: float = 0.0, u=None, want_logits: bool = False):
    """or_spec_step: returns (emitted, drafts) or, with want_logits,
    (emitted, drafts, p_logits [(n+1)][V], q_logits [n][V])."""
    n = min(max(n_max, 1), 8)
    em = (C.c_uint32 * 9)()
    dr = (C.c_uint32 * 8)()
    ne = C.c_uint32()
    uu = _f32(u) if u is not None else None
    p = np.empty((n + 1, tgt.V), np.float32) if want_logits else None
    q = np.empty((n, tgt.V), np.float32) if want_logits else None
    rc = lib().or_spec_step(tgt.h, drf.h, tkv.h, dkv.h, last_token, n_max, mode, T,
                            uu.ctypes.data_as(F32P) if uu is not None else None, dkv.pending,
                            C.byref(dkv.n_pending), em, C.byref(ne), dr,
                            p.ctypes.data_as(F32P) if p is not None else None,
                            q.ctypes.data_as(F32P) if q is not None else None)
    if rc:
        raise ValueError(f"oracle spec step failed ({rc})")
    out = (list(em)[: ne.value], list(dr)[:n])
    return out + (p, q) if want_logits else out
