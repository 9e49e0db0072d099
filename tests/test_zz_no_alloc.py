"""sh_accept_sample_noalloc (the acceptance kernel with a static device
scratch, for callers that cannot allocate) against sh_accept_sample, through
the C ABI: identical accepted lengths and next tokens on two calls in a row,
the second smaller than the first (the static array keeps the first call's
contents), in both stochastic modes; sizes beyond the array are refused."""
import ctypes as C

import numpy as np
import pytest

from seeker_amd import SeekerError
from seeker_amd import _native as N
from seeker_amd import synth as S
from seeker_amd._native import SH_SAMPLE_COMPARE, SH_SAMPLE_REJECTION, sh_sampling

pytestmark = pytest.mark.gpu


def _inputs(B, k, V, seed):
    p = S.normal_f32(seed, 10, B * (k + 1) * V, 0.0, 3.0).reshape(B, k + 1, V)
    q = (p[:, :k] + S.normal_f32(seed, 11, B * k * V, 0.0, 1.0).reshape(B, k, V)).astype(np.float32)
    rng = np.random.default_rng(seed)
    drafts = rng.integers(0, V, (B, k)).astype(np.uint32)
    drafts[:, ::2] = np.argmax(p[:, : k : 2], axis=-1)  # some drafts likely accepted
    return p, q, drafts


def _run(engine, fn, p, q, drafts, mode, T, seed, counter):
    B, k1, V = p.shape
    k = k1 - 1
    pd, qd, dd = engine.to_device(p), engine.to_device(q), engine.to_device(drafts)
    acc, nxt = engine.dev_alloc(4 * B), engine.dev_alloc(4 * B)
    s = sh_sampling()
    s.mode, s.temperature, s.seed, s.counter = mode, T, seed, counter
    N.check(fn(engine.h, pd.ptr, qd.ptr if mode == SH_SAMPLE_REJECTION else None, dd.ptr, B, k, V, C.byref(s),
               acc.ptr, nxt.ptr))
    engine.sync()
    out = acc.read(np.uint32, B), nxt.read(np.uint32, B)
    for b in (pd, qd, dd, acc, nxt):
        b.free()
    return out


@pytest.mark.parametrize("mode", [SH_SAMPLE_COMPARE, SH_SAMPLE_REJECTION], ids=["compare", "rejection"])
def test_noalloc_matches_allocating_entry(engine, mode):
    lib = N.lib()
    for call, (B, k, V) in enumerate([(32, 8, 128256), (5, 3, 4000)]):
        print(f"no-alloc accept mode {mode} call {call}: B={B} k={k} V={V}", flush=True)
        p, q, drafts = _inputs(B, k, V, seed=40 + call)
        want = _run(engine, lib.sh_accept_sample, p, q, drafts, mode, 0.8, 7, 100 * call)
        got = _run(engine, lib.sh_accept_sample_noalloc, p, q, drafts, mode, 0.8, 7, 100 * call)
        assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1]), call
        if mode == SH_SAMPLE_REJECTION:
            assert want[0].max() > 0  # some drafts accepted: the accept path ran too


def test_noalloc_refuses_oversized_and_explicit_uniforms(engine):
    lib = N.lib()
    B, k, V = 64, 64, 1 << 20  # scratch far beyond the static array
    s = sh_sampling()
    s.mode, s.temperature = SH_SAMPLE_REJECTION, 1.0
    dummy = engine.dev_alloc(16)
    with pytest.raises(SeekerError) as ei:
        N.check(lib.sh_accept_sample_noalloc(engine.h, dummy.ptr, dummy.ptr, dummy.ptr, B, k, V, C.byref(s),
                                             dummy.ptr, dummy.ptr))
    assert ei.value.status == N.SH_ERR_CAPACITY
    u = np.zeros(8, np.float32)
    s.uniforms = u.ctypes.data_as(N.F32P)
    with pytest.raises(SeekerError) as ei:
        N.check(lib.sh_accept_sample_noalloc(engine.h, dummy.ptr, dummy.ptr, dummy.ptr, 1, 1, 16, C.byref(s),
                                             dummy.ptr, dummy.ptr))
    assert ei.value.status == N.SH_ERR_ARG
    dummy.free()
