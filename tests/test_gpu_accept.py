"""GPU acceptance kernel (sh_accept_sample) vs the oracle, configs[1] shapes:
B sequences x k draft positions over vocab V, target logits N(0, 3), draft =
target + N(0, 1), T = 0.8, uniforms from Philox4x64-10 (shared seeds) or
passed explicitly. Accepted lengths and next tokens must be bit-identical.
The accept-test probabilities p(d), q(d) and min(1, p/q) (sh_accept_probs)
must match an independent numpy f64 softmax within 1e-5 absolute (north star)
and 1e-10 relative."""
import numpy as np
import pytest

import oracle as O
from seeker_amd import synth as S
from seeker_amd._native import SH_SAMPLE_COMPARE, SH_SAMPLE_REJECTION, sh_sampling

pytestmark = pytest.mark.gpu


def make_inputs(B, k, V, seed=7):
    p = S.normal_f32(seed, 10, B * (k + 1) * V, 0.0, 3.0).reshape(B, k + 1, V)
    q = (p[:, :k, :] + S.normal_f32(seed, 11, B * k * V, 0.0, 1.0).reshape(B, k, V)).astype(np.float32)
    # drafts d_i ~ q_i (temperature 0.8) using the oracle's inverse CDF and its own Philox stream
    u = O.philox_uniforms(seed, 12, 0, B * k)
    drafts = np.array([[O.sample_vocab_order(q[b, i], 0.8, float(u[b * k + i])) for i in range(k)]
                       for b in range(B)], dtype=np.uint32)
    return p, q, drafts


def run_gpu(engine, p, q, drafts, mode, T, seed, uniforms=None):
    B, k1, V = p.shape
    k = k1 - 1
    pd, qd, dd = engine.to_device(p), engine.to_device(q), engine.to_device(drafts)
    acc, nxt = engine.dev_alloc(4 * B), engine.dev_alloc(4 * B)
    s = sh_sampling()
    s.mode, s.temperature, s.seed, s.counter = mode, T, seed, 0
    keep = None
    if uniforms is not None:
        keep = np.ascontiguousarray(uniforms, np.float32)
        s.uniforms = keep.ctypes.data_as(O.F32P)
    engine.accept_sample(pd, qd if mode == SH_SAMPLE_REJECTION else None, dd, B, k, V, s, acc, nxt)
    a, n = acc.read(np.uint32, B), nxt.read(np.uint32, B)
    for b in (pd, qd, dd, acc, nxt):
        b.free()
    return a, n


def oracle_uniforms(seed, B, k):
    w = O.philox_uniforms(seed, 0x5EC, 0, 2 * B * (k + 1)).reshape(B, k + 1, 2)
    return w


@pytest.mark.parametrize("B,k,V", [(4, 3, 1000), (32, 8, 128256)])
def test_rejection_matches_oracle(engine, B, k, V):
    print(f"rejection B={B} k={k} V={V}", flush=True)
    p, q, drafts = make_inputs(B, k, V)
    a, n = run_gpu(engine, p, q, drafts, SH_SAMPLE_REJECTION, 0.8, seed=7)
    U = oracle_uniforms(7, B, k)
    for b in range(B):
        oa, on = O.rejection(p[b], q[b], drafts[b], 0.8, U[b, :k, 0].copy(), U[b, :, 1].copy())
        assert (a[b], n[b]) == (oa, on), b


@pytest.mark.parametrize("B,k,V", [(4, 3, 1000), (32, 8, 128256)])
def test_compare_matches_oracle(engine, B, k, V):
    print(f"compare B={B} k={k} V={V}", flush=True)
    p, q, drafts = make_inputs(B, k, V, seed=9)
    # make some drafts match the target sample so acceptance lengths vary
    U = oracle_uniforms(9, B, k)
    for b in range(B):
        for i in range(k):
            if (b + i) % 3:
                drafts[b, i] = O.sample_vocab_order(p[b, i], 0.8, float(U[b, i, 1]))
    a, n = run_gpu(engine, p, q, drafts, SH_SAMPLE_COMPARE, 0.8, seed=9)
    cfg = O.SamplerCfg(0.8, 0, 1.0, 0.0)
    for b in range(B):
        em = O.sample_and_compare(p[b], drafts[b], cfg, U[b, :, 1].copy(), mode=1)
        assert a[b] == len(em) - 1 and n[b] == em[-1], b


def test_explicit_uniforms(engine):
    B, k, V = 6, 4, 500
    p, q, drafts = make_inputs(B, k, V, seed=3)
    rng = np.random.default_rng(0)
    U = rng.random((B, k + 1, 2)).astype(np.float32)
    U[0, :, 0] = 0.0          # u = 0 accepts whenever p(d) > 0
    U[1, :, 1] = 0.999999     # resample from the far end of the CDF
    a, n = run_gpu(engine, p, q, drafts, SH_SAMPLE_REJECTION, 0.8, seed=0, uniforms=U)
    for b in range(B):
        oa, on = O.rejection(p[b], q[b], drafts[b], 0.8, U[b, :k, 0].copy(), U[b, :, 1].copy())
        assert (a[b], n[b]) == (oa, on), b


def test_accept_probs_match_numpy_f64(engine):
    B, k, V, T = 8, 5, 128256, 0.8
    print(f"accept probs B={B} k={k} V={V}", flush=True)
    p, q, drafts = make_inputs(B, k, V, seed=17)
    pd, qd, dd = engine.to_device(p), engine.to_device(q), engine.to_device(drafts)
    got = engine.accept_probs(pd, qd, dd, B, k, V, T)
    for b in (pd, qd, dd):
        b.free()

    T32 = float(np.float32(T))  # the kernel's temperature is an f32

    def prob(row, tok):
        z = row.astype(np.float64) / T32
        z = np.exp(z - z.max())
        return z[tok] / z.sum()

    for b in range(B):
        for i in range(k):
            d = int(drafts[b, i])
            want_p, want_q = prob(p[b, i], d), prob(q[b, i], d)
            want = np.array([want_p, want_q, min(1.0, want_p / want_q)])
            assert np.all(np.abs(got[b, i] - want) <= 1e-5), (b, i)
            assert np.allclose(got[b, i], want, rtol=1e-10, atol=0), (b, i, got[b, i], want)
