"""GPU acceptance kernel (sh_accept_sample) vs the oracle, configs[1] shapes:
B sequences x k draft positions over vocab V, target logits N(0, 3), draft =
target + N(0, 1), T = 0.8, uniforms from Philox4x64-10 (shared seeds) or
passed explicitly. Accepted lengths and next tokens must be bit-identical.
The accept-test probabilities p(d), q(d) and min(1, p/q) (sh_accept_probs)
must match an independent numpy f64 softmax within 1e-5 absolute (north star)
and 2e-6 relative: the softmax sums are f64 sums of hardware f32 exp terms
(1 ulp each), the numerators f64."""
import numpy as np
import pytest

import oracle as O
from seeker_amd import synth as S
from parity import record
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


@pytest.mark.parametrize("B,k,V", [(4, 3, 1000), (32, 8, 128256), (260, 2, 300)])
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
            assert np.allclose(got[b, i], want, rtol=2e-6, atol=0), (b, i, got[b, i], want)


def test_rejection_many_seeds(engine):
    """configs[1] (B = 32, k = 8, V = 128256, T = 0.8) over 1000 Philox seeds on
    fixed logits: accepted lengths and next tokens equal a numpy f64 restatement
    of the rejection rule (accept d_i iff u q_i(d_i) < p_i(d_i); first rejection
    i draws from max(0, p_i - q_i), else from p_i; all accepted draws from p_k;
    first v with cumsum > u * total), itself checked against the C oracle on the
    first seeds. A mismatch is allowed only where the f64 reference's own margin
    (|u q - p| / p of the accept test, or the draw target's distance to a CDF
    step) is below 2e-6, the precision of the kernel's softmax sums."""
    B, k, V, T = 32, 8, 128256, 0.8
    n_seeds = 1000
    print(f"rejection x {n_seeds} seeds B={B} k={k} V={V}", flush=True)
    p, q, drafts = make_inputs(B, k, V, seed=21)
    T32 = float(np.float32(T))

    def num(x):  # softmax numerators and sums, f64
        z = x.astype(np.float64) / T32
        z = np.exp(z - z.max(axis=-1, keepdims=True))
        return z, z.sum(axis=-1)

    pd_acc = np.empty((B, k))
    qd_acc = np.empty((B, k))
    rcum = np.empty((B, k, V))  # residual CDFs (unnormalised)
    pcum = np.empty((B, k + 1, V))  # p numerator CDFs
    for b in range(B):
        a, za = num(p[b])
        c, zc = num(q[b])
        idx = drafts[b].astype(np.int64)
        pd_acc[b] = a[np.arange(k), idx] / za[:k]
        qd_acc[b] = c[np.arange(k), idx] / zc
        rcum[b] = np.cumsum(np.maximum(0.0, a[:k] / za[:k, None] - c / zc[:, None]), axis=1)
        pcum[b] = np.cumsum(a, axis=1)

    def ref(U):
        acc = np.full(B, k)
        nxt = np.zeros(B, np.uint32)
        tight = np.zeros(B, bool)
        for b in range(B):
            for i in range(k):
                ua = float(U[b, i, 0])
                if abs(ua * qd_acc[b, i] - pd_acc[b, i]) <= 2e-6 * pd_acc[b, i]:
                    tight[b] = True
                if not ua * qd_acc[b, i] < pd_acc[b, i]:
                    acc[b] = i
                    break
            i = acc[b]
            cum = rcum[b, i] if i < k and rcum[b, i, -1] > 0.0 else pcum[b, i]
            target = float(U[b, i, 1]) * cum[-1]
            v = min(int(np.searchsorted(cum, target, side="right")), V - 1)
            near = min(abs(cum[v] - target), abs(target - (cum[v - 1] if v else 0.0)))
            if near <= 2e-6 * cum[-1]:
                tight[b] = True
            nxt[b] = v
        return acc, nxt, tight

    # the restatement agrees with the C oracle
    for sd in range(2):
        U = oracle_uniforms(1000 + sd, B, k)
        ra, rn, _ = ref(U)
        for b in range(B):
            assert (ra[b], rn[b]) == O.rejection(p[b], q[b], drafts[b], T, U[b, :k, 0].copy(), U[b, :, 1].copy())

    pdv, qdv, ddv = engine.to_device(p), engine.to_device(q), engine.to_device(drafts)
    accd, nxtd = engine.dev_alloc(4 * B), engine.dev_alloc(4 * B)
    s = sh_sampling()
    mism, tight_mism, n_acc = 0, 0, 0
    for sd in range(n_seeds):
        s.mode, s.temperature, s.seed, s.counter = SH_SAMPLE_REJECTION, T, 1000 + sd, 0
        engine.accept_sample(pdv, qdv, ddv, B, k, V, s, accd, nxtd)
        a, n = accd.read(np.uint32, B), nxtd.read(np.uint32, B)
        ra, rn, tight = ref(oracle_uniforms(1000 + sd, B, k))
        bad = (a != ra) | (n != rn)
        mism += int(bad.sum())
        tight_mism += int((bad & tight).sum())
        n_acc += int(a.sum())
        if (sd + 1) % 250 == 0:
            print(f"  {sd + 1} seeds: {mism} mismatches ({tight_mism} at near-ties)", flush=True)
    for x in (pdv, qdv, ddv, accd, nxtd):
        x.free()
    print(f"mean accepted {n_acc / (n_seeds * B):.3f}", flush=True)
    record("rejection_seeds", n_seeds * B, mism)
    assert mism == tight_mism, (mism, tight_mism)
