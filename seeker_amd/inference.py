"""Host-side mirror of seeker-vulkan's spec-decode surface over the C ABI.

Names and argument meaning follow crates/seeker-vulkan/src/inference/mod.rs
(`Engine`), inference/kv_cache.rs (`KvCache`), models/mod.rs (`Model`) and
inference/sample.rs (`SamplerConfig`); errors surface as SeekerError carrying
the C status and message (the reference's Result<_, Box<dyn Error>>). Every
call goes to libseeker_hip.so; nothing here computes on the CPU.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

from . import _native as N


@dataclass
class SpecStepOut:
    """inference/mod.rs:165-178."""
    emitted: list
    accepted: int
    last_token: int
    drafts: list


@dataclass
class VerifyUnifiedOut:
    """models/mod.rs:491-496 + the per-column samples of verify_unified: sampled [N_total],
    logits [N_total][V] and residual [N_total][n_embd] when requested, q_starts [B]."""
    sampled: np.ndarray
    logits: Optional[np.ndarray]
    residual: Optional[np.ndarray]
    q_starts: np.ndarray


@dataclass
class SamplerConfig:
    """Subset of inference/sample.rs:85 used by the verify path: temperature 0
    is greedy; mode selects sample-and-compare or rejection sampling."""
    temperature: float = 0.0
    seed: int = 0
    mode: int = N.SH_SAMPLE_GREEDY

    def to_c(self, counter: int = 0, uniforms: Optional[np.ndarray] = None):
        s = N.sh_sampling()
        s.mode = self.mode if self.temperature > 0 else N.SH_SAMPLE_GREEDY
        s.temperature = self.temperature
        s.seed = self.seed
        s.counter = counter
        s.uniforms = uniforms.ctypes.data_as(N.F32P) if uniforms is not None else None
        return s


class Engine:
    """Engine::new (inference/mod.rs:198): one HIP device, one stream."""

    def __init__(self, device: int = 0):
        self._lib = N.lib()
        h = C.c_void_p()
        N.check(self._lib.sh_engine_create(device, C.byref(h)))
        self.h = h

    def close(self):
        if self.h:
            self._lib.sh_engine_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def sync(self):
        N.check(self._lib.sh_engine_sync(self.h))

    # -- weights / caches ----------------------------------------------------
    def upload_weights(self, gguf) -> "Model":
        """upload_weights + models::open (inference/mod.rs:304, models/mod.rs:537)."""
        h = C.c_void_p()
        if isinstance(gguf, str):
            N.check(self._lib.sh_model_load_gguf(self.h, gguf.encode(), C.byref(h)))
        else:
            N.check(self._lib.sh_model_load_gguf_memory(self.h, C.c_void_p(gguf.address), gguf.size, C.byref(h)))
        return Model(self, h)

    def allocate_kv_cache(self, model: "Model", max_seq_len: int) -> "KvCache":
        """Engine::allocate_kv_cache (inference/mod.rs:318)."""
        h = C.c_void_p()
        N.check(self._lib.sh_kv_create(self.h, model.h, max_seq_len, C.byref(h)))
        return KvCache(self, model, h)

    # -- forward / verify ---------------------------------------------------
    def forward_full_readback(self, model: "Model", cache: "KvCache", tokens: Sequence[int], pos: int,
                              full_logits: bool = True, parents: Optional[Sequence[int]] = None,
                              want_residual: bool = True):
        """Engine::forward_full_readback (inference/mod.rs:2427-2448): returns
        (logits [cols][V], residual [L][d])."""
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        L = t.size
        V, d = model.dims.n_vocab, model.dims.n_embd
        cols = L if full_logits else 1
        logits = np.empty((cols, V), dtype=np.float32)
        resid = np.empty((L, d), dtype=np.float32) if want_residual else None
        par = np.ascontiguousarray(parents, dtype=np.int32) if parents is not None else None
        N.check(self._lib.sh_forward_full(
            self.h, model.h, cache.h, t.ctypes.data_as(N.U32P), L, pos,
            par.ctypes.data_as(N.I32P) if par is not None else None,
            2 if full_logits else 1, logits.ctypes.data_as(N.F32P),
            resid.ctypes.data_as(N.F32P) if resid is not None else None))
        return logits, resid

    def prefill(self, model: "Model", cache: "KvCache", tokens: Sequence[int], pos: int):
        """Forward without logits (KV only; bench.rs feed_kv, :296-317)."""
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        N.check(self._lib.sh_forward_full(self.h, model.h, cache.h, t.ctypes.data_as(N.U32P), t.size, pos, None, 0,
                                          None, None))

    def verify_greedy(self, model: "Model", cache: "KvCache", tokens: Sequence[int], pos: int) -> np.ndarray:
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        out = np.zeros(t.size, dtype=np.uint32)
        N.check(self._lib.sh_verify_greedy(self.h, model.h, cache.h, t.ctypes.data_as(N.U32P), t.size, pos,
                                           out.ctypes.data_as(N.U32P)))
        return out

    def verify_unified(self, model: "Model", caches: Sequence["KvCache"], tokens: Sequence[int],
                       seq_lens: Sequence[int], positions: Optional[Sequence[int]] = None,
                       parents: Optional[Sequence[int]] = None, want_logits: bool = False,
                       want_residual: bool = False, samplers: Optional[Sequence[N.sh_sampling]] = None
                       ) -> VerifyUnifiedOut:
        """Engine::verify_unified (inference/mod.rs:2316-2398): B sequences packed flat, sequence s
        verified against caches[s]. Every column sampled by its sequence's sampler (samplers[s]:
        GREEDY or COMPARE, sh_verify_unified_sampled; None: greedy argmax); logits / residual on
        request. Every cache advances by its seq_len (truncate to the accepted length afterwards);
        each COMPARE sampler's counter advances by its seq_len."""
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        sl = np.ascontiguousarray(seq_lens, dtype=np.uint32)
        n, b = t.size, sl.size
        hs = (C.c_void_p * b)(*[c.h for c in caches])
        pos = None if positions is None else np.ascontiguousarray(positions, dtype=np.uint32)
        par = None if parents is None else np.ascontiguousarray(parents, dtype=np.int32)
        sampled = np.zeros(n, dtype=np.uint32)
        logits = np.zeros((n, model.vocab_size()), dtype=np.float32) if want_logits else None
        resid = np.zeros((n, model.dims.n_embd), dtype=np.float32) if want_residual else None
        args = (self.h, model.h, C.cast(hs, C.POINTER(C.c_void_p)), b, t.ctypes.data_as(N.U32P),
                sl.ctypes.data_as(N.U32P), None if pos is None else pos.ctypes.data_as(N.U32P),
                None if par is None else par.ctypes.data_as(N.I32P))
        outs = (None if logits is None else logits.ctypes.data_as(N.F32P), sampled.ctypes.data_as(N.U32P),
                None if resid is None else resid.ctypes.data_as(N.F32P))
        if samplers is None:
            N.check(self._lib.sh_verify_unified(*args, *outs))
        else:
            arr = (N.sh_sampling * b)(*samplers)
            N.check(self._lib.sh_verify_unified_sampled(*args, C.cast(arr, C.c_void_p), *outs))
            for s_in, s_out in zip(samplers, arr):
                s_in.counter = s_out.counter
        q_starts = np.concatenate([[0], np.cumsum(sl)[:-1]]).astype(np.uint64)
        return VerifyUnifiedOut(sampled, logits, resid, q_starts)

    def tree_verify_step(self, target: "Model", caches: Sequence["KvCache"], tokens: np.ndarray,
                         parents: np.ndarray, q_logits: Optional["DeviceBuffer"], s: N.sh_sampling):
        """One tree verification step (sh_tree_verify_step) for B trees of n nodes:
        returns (paths: list of node-index lists, next_tokens [B]); caches hold the paths."""
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        par = np.ascontiguousarray(parents, dtype=np.int32)
        B, n = t.shape
        hs = (C.c_void_p * B)(*[c.h for c in caches])
        path = np.zeros((B, n), dtype=np.uint32)
        plen = np.zeros(B, dtype=np.uint32)
        nxt = np.zeros(B, dtype=np.uint32)
        N.check(self._lib.sh_tree_verify_step(
            self.h, target.h, C.cast(hs, C.POINTER(C.c_void_p)), B, n, t.ctypes.data_as(N.U32P),
            par.ctypes.data_as(N.I32P), q_logits.ptr if q_logits is not None else None, C.byref(s),
            path.ctypes.data_as(N.U32P), plen.ctypes.data_as(N.U32P), nxt.ctypes.data_as(N.U32P)))
        return [path[b, : plen[b]].tolist() for b in range(B)], nxt

    def decode_speculative(self, target: "Model", draft: "Model", tcache: "KvCache", dcache: "KvCache",
                           last_token: int, n_max: int, sampler: Optional[N.sh_sampling] = None) -> SpecStepOut:
        """Engine::decode_speculative (inference/mod.rs:2108-2297) with a separate draft model."""
        emitted = np.zeros(9, dtype=np.uint32)
        drafts = np.zeros(8, dtype=np.uint32)
        ne = C.c_uint32()
        s = sampler if sampler is not None else N.sh_sampling()
        N.check(self._lib.sh_spec_step(self.h, target.h, draft.h, tcache.h, dcache.h, last_token, n_max,
                                       C.byref(s), emitted.ctypes.data_as(N.U32P), C.byref(ne),
                                       drafts.ctypes.data_as(N.U32P)))
        n = min(max(n_max, 1), 8)
        em = emitted[: ne.value].tolist()
        return SpecStepOut(em, ne.value - 1, em[-1], drafts[:n].tolist())

    def decode_speculative_forced(self, target: "Model", draft: "Model", tcache: "KvCache", dcache: "KvCache",
                                  last_token: int, forced_drafts: Sequence[int]) -> SpecStepOut:
        """sh_spec_step_forced: a greedy step whose drafts are forced_drafts (the
        draft forwards run over them); the forced-acceptance measurement."""
        n = len(forced_drafts)
        fd = np.ascontiguousarray(forced_drafts, dtype=np.uint32)
        emitted = np.zeros(9, dtype=np.uint32)
        ne = C.c_uint32()
        N.check(self._lib.sh_spec_step_forced(self.h, target.h, draft.h, tcache.h, dcache.h, last_token, n,
                                              fd.ctypes.data_as(N.U32P), emitted.ctypes.data_as(N.U32P),
                                              C.byref(ne)))
        em = emitted[: ne.value].tolist()
        return SpecStepOut(em, ne.value - 1, em[-1], fd.tolist())

    def draft_tokens(self, draft: "Model", dcache: "KvCache", last_token: int, n_max: int) -> list:
        """Engine::draft_tokens (inference/mod.rs:2062-2092): greedy drafts of a separate
        draft model from its cache (pending tokens first); the cache advances by
        pending + n and is truncated by the caller to the accepted length."""
        n = min(max(n_max, 1), 8)
        out = np.zeros(n, dtype=np.uint32)
        N.check(self._lib.sh_draft_tokens(self.h, draft.h, dcache.h, last_token, n_max, out.ctypes.data_as(N.U32P)))
        return out.tolist()

    def spec_step_batch(self, target: "Model", draft: "Model", tcaches: Sequence["KvCache"],
                        dcaches: Sequence["KvCache"], last_tokens: Sequence[int], n_max: int,
                        samplers: Optional[Sequence[N.sh_sampling]] = None):
        """The server's batched speculative step (sh_spec_step_batch, server/inference.rs:2777-2924):
        returns (emitted per sequence, drafts per sequence)."""
        B = len(tcaches)
        n = min(max(n_max, 1), 8)
        th = (C.c_void_p * B)(*[c.h for c in tcaches])
        dh = (C.c_void_p * B)(*[c.h for c in dcaches])
        last = np.ascontiguousarray(last_tokens, dtype=np.uint32)
        em = np.zeros((B, n + 1), dtype=np.uint32)
        ne = np.zeros(B, dtype=np.uint32)
        dr = np.zeros((B, n), dtype=np.uint32)
        arr = None
        if samplers is not None:
            arr = (N.sh_sampling * B)(*samplers)
        N.check(self._lib.sh_spec_step_batch(self.h, target.h, draft.h, C.cast(th, C.POINTER(C.c_void_p)),
                                             C.cast(dh, C.POINTER(C.c_void_p)), B, last.ctypes.data_as(N.U32P),
                                             n_max, C.cast(arr, C.c_void_p) if arr is not None else None,
                                             em.ctypes.data_as(N.U32P), ne.ctypes.data_as(N.U32P),
                                             dr.ctypes.data_as(N.U32P)))
        if samplers is not None:
            for s_in, s_out in zip(samplers, arr):
                s_in.counter = s_out.counter
        return [em[s, : ne[s]].tolist() for s in range(B)], [dr[s].tolist() for s in range(B)]

    def spec_step_logits(self):
        """Target logits [(n+1)][V] and draft logits [n][V] of the last stochastic
        decode_speculative on this engine (the reference's tap readback,
        inference/context.rs:136-160)."""
        n, V = C.c_uint32(), C.c_uint32()
        N.check(self._lib.sh_spec_step_logits(self.h, None, None, C.byref(n), C.byref(V)))
        p = np.empty((n.value + 1, V.value), np.float32)
        q = np.empty((n.value, V.value), np.float32)
        N.check(self._lib.sh_spec_step_logits(self.h, p.ctypes.data_as(N.F32P), q.ctypes.data_as(N.F32P),
                                              C.byref(n), C.byref(V)))
        return p, q

    # -- profiling ------------------------------------------------------------
    def set_profiling(self, on: bool):
        N.check(self._lib.sh_engine_set_profiling(self.h, int(on)))

    def graph_stats(self):
        """(graphs captured, graph launches) so far on this engine."""
        c, l = C.c_uint64(), C.c_uint64()
        N.check(self._lib.sh_engine_graph_stats(self.h, C.byref(c), C.byref(l)))
        return c.value, l.value

    def profile(self, reset: bool = False) -> dict:
        n = C.c_uint32()
        N.check(self._lib.sh_engine_profile(self.h, None, 0, C.byref(n)))
        arr = (N.sh_kernel_stat * max(n.value, 1))()
        N.check(self._lib.sh_engine_profile(self.h, arr, n.value, C.byref(n)))
        out = {arr[i].name.decode(): {"launches": arr[i].launches, "ms": arr[i].total_ms,
                                      "bytes": arr[i].alg_bytes} for i in range(n.value)}
        if reset:
            N.check(self._lib.sh_engine_profile_reset(self.h))
        return out

    # -- device buffers (kernel-level entry points) ---------------------------
    def dev_alloc(self, nbytes: int) -> "DeviceBuffer":
        p = C.c_void_p()
        N.check(self._lib.sh_dev_alloc(self.h, nbytes, C.byref(p)))
        return DeviceBuffer(self, p, nbytes)

    def to_device(self, arr: np.ndarray) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        b = self.dev_alloc(arr.nbytes)
        N.check(self._lib.sh_memcpy_h2d(self.h, b.ptr, arr.ctypes.data_as(C.c_void_p), arr.nbytes))
        return b

    def gemv(self, w: "QTensor", x: "DeviceBuffer", n: int, y: "DeviceBuffer", accumulate: bool = False):
        N.check(self._lib.sh_gemv_quant(self.h, w.h, x.ptr, n, y.ptr, int(accumulate)))

    def gemm_wide16(self, w: "QTensor", x: "DeviceBuffer", n: int, y: "DeviceBuffer", accumulate: bool = False):
        """The reference's wide-GEMM arithmetic (f16 weights and activations, f32
        accumulation; ops/matmul.rs:433-446), Q4_K."""
        N.check(self._lib.sh_gemm_wide16(self.h, w.h, x.ptr, n, y.ptr, int(accumulate)))

    def accept_sample(self, p_logits: "DeviceBuffer", q_logits: Optional["DeviceBuffer"], drafts: "DeviceBuffer",
                      B: int, k: int, V: int, s: N.sh_sampling, acc_len: "DeviceBuffer", next_tok: "DeviceBuffer"):
        N.check(self._lib.sh_accept_sample(self.h, p_logits.ptr, q_logits.ptr if q_logits else None, drafts.ptr,
                                           B, k, V, C.byref(s), acc_len.ptr, next_tok.ptr))

    def accept_probs(self, p_logits: "DeviceBuffer", q_logits: "DeviceBuffer", drafts: "DeviceBuffer", B: int, k: int,
                     V: int, temperature: float) -> np.ndarray:
        """sh_accept_probs: [B][k][3] = (p(d), q(d), min(1, p/q)) of each REJECTION accept test."""
        out = self.dev_alloc(B * k * 3 * 8)
        try:
            N.check(self._lib.sh_accept_probs(self.h, p_logits.ptr, q_logits.ptr, drafts.ptr, B, k, V, temperature,
                                              out.ptr))
            return out.read(np.float64, B * k * 3).reshape(B, k, 3)
        finally:
            out.free()

    def tree_accept(self, p_logits: "DeviceBuffer", q_logits: Optional["DeviceBuffer"], tokens: "DeviceBuffer",
                    parents: "DeviceBuffer", B: int, n: int, V: int, s: N.sh_sampling, path: "DeviceBuffer",
                    path_len: "DeviceBuffer", next_tok: "DeviceBuffer"):
        """Tree acceptance (sh_tree_accept) over B trees of n nodes; all buffers on the device."""
        N.check(self._lib.sh_tree_accept(self.h, p_logits.ptr, q_logits.ptr if q_logits else None, tokens.ptr,
                                         parents.ptr, B, n, V, C.byref(s), path.ptr, path_len.ptr, next_tok.ptr))


class DeviceBuffer:
    def __init__(self, engine: Engine, ptr: C.c_void_p, nbytes: int):
        self.engine, self.ptr, self.nbytes = engine, ptr, nbytes

    def read(self, dtype, count: int) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        N.check(self.engine._lib.sh_memcpy_d2h(self.engine.h, out.ctypes.data_as(C.c_void_p), self.ptr, out.nbytes))
        return out

    def write(self, arr: np.ndarray):
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes
        N.check(self.engine._lib.sh_memcpy_h2d(self.engine.h, self.ptr, arr.ctypes.data_as(C.c_void_p), arr.nbytes))

    def free(self):
        if self.ptr:
            N.check(self.engine._lib.sh_dev_free(self.engine.h, self.ptr))
            self.ptr = None


class QTensor:
    """A quantized [M][K] matrix uploaded and repacked for the GEMV."""

    def __init__(self, engine: Engine, qtype: int, blocks: np.ndarray, M: int, K: int):
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
        h = C.c_void_p()
        N.check(engine._lib.sh_qtensor_upload(engine.h, qtype, blocks.ctypes.data_as(C.c_void_p), M, K, C.byref(h)))
        self.engine, self.h, self.M, self.K = engine, h, M, K

    def close(self):
        if self.h:
            self.engine._lib.sh_qtensor_destroy(self.h)
            self.h = None


class Model:
    """Handle to an uploaded Llama model (models/mod.rs `Model`)."""

    def __init__(self, engine: Engine, h: C.c_void_p):
        self.engine, self.h = engine, h
        d = N.sh_model_dims()
        N.check(engine._lib.sh_model_info(h, C.byref(d)))
        self.dims = d

    def vocab_size(self) -> int:
        return self.dims.n_vocab

    @property
    def wide_f16(self) -> bool:
        """Whether forward calls of >= 32 columns take the reference's wide-GEMM
        arithmetic (f16 weights and activations, f32 accumulation;
        ops/matmul.rs:406-446)."""
        on = C.c_int()
        N.check(self.engine._lib.sh_model_wide_f16(self.h, C.byref(on)))
        return bool(on.value)

    @wide_f16.setter
    def wide_f16(self, on: bool):
        N.check(self.engine._lib.sh_model_set_wide_f16(self.h, 1 if on else 0))

    @property
    def cm1_attention(self) -> bool:
        """Causal forward calls of more than one column compute attention with
        the reference's cooperative-matrix flash attention arithmetic
        (flash_attn_cm1.slang via ops/flash_attn.rs:442-471): f16 staged q,
        64-key blocks, f16 P, f16 P V accumulators and output."""
        on = C.c_int()
        N.check(self.engine._lib.sh_model_cm1_attention(self.h, C.byref(on)))
        return bool(on.value)

    @cm1_attention.setter
    def cm1_attention(self, on: bool):
        N.check(self.engine._lib.sh_model_set_cm1_attention(self.h, 1 if on else 0))

    def close(self):
        if self.h:
            self.engine._lib.sh_model_destroy(self.h)
            self.h = None


class KvCache:
    """inference/kv_cache.rs `KvCache`: f16 K/V, cursor position."""

    def __init__(self, engine: Engine, model: Model, h: C.c_void_p):
        self.engine, self.model, self.h = engine, model, h

    @property
    def position(self) -> int:
        p = C.c_uint32()
        N.check(self.engine._lib.sh_kv_position(self.h, C.byref(p)))
        return p.value

    def truncate(self, new_pos: int):
        """KvCache::truncate: position = min(new_pos, position) (kv_cache.rs:587-602)."""
        N.check(self.engine._lib.sh_kv_truncate(self.h, new_pos))

    def set_position(self, pos: int):
        N.check(self.engine._lib.sh_kv_set_position(self.h, pos))

    def read_layer(self, layer: int, is_v: bool, n_pos: int) -> np.ndarray:
        d = self.model.dims
        out = np.zeros((n_pos, d.n_head_kv, d.head_dim), dtype=np.uint16)
        N.check(self.engine._lib.sh_kv_read_layer(self.h, layer, int(is_v), n_pos, out.ctypes.data_as(N.U16P)))
        return out

    def write_layer(self, layer: int, is_v: bool, data: np.ndarray):
        data = np.ascontiguousarray(data, dtype=np.uint16)
        N.check(self.engine._lib.sh_kv_write_layer(self.h, layer, int(is_v), data.shape[0],
                                                   data.ctypes.data_as(N.U16P)))

    def compact(self, base: int, src_rows: Sequence[int]):
        s = np.ascontiguousarray(src_rows, dtype=np.uint32)
        N.check(self.engine._lib.sh_kv_compact(self.h, base, s.ctypes.data_as(N.U32P), s.size))

    def close(self):
        if self.h:
            self.engine._lib.sh_kv_destroy(self.h)
            self.h = None
