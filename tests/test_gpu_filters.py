"""GPU sampler chain with candidate filters (SH_SAMPLE_COMPARE with top_k /
top_p / min_p), the reference's chain order (inference/sample.rs:369-473,
ops/sampler.rs:41-132): top_k candidates sorted by logit descending (ties to
the lower id) -> top_p (exclusive cumulative <= p keeps the crossing
candidate) -> min_p (log-space cutoff against the largest) -> 1/T -> softmax
-> first candidate whose cumulative probability reaches u. Every draw must
equal the C oracle's or_sample_one on the same logits and uniform.

Both sides run the top_p cut and the inverse CDF with f64 softmax terms and
f64 running sums; the reference's host chain uses f32 exp, sums and
cumulative sums (inference/sample.rs:420-470, 518-533). At a candidate whose
cumulative probability lies within f32 rounding of top_p, or a uniform within
f32 rounding of a CDF boundary, the reference can pick the neighbouring
token: these tests pin the GPU to the f64 chain, and parity with the
reference's f32 chain is unpinned there."""
import numpy as np
import pytest

import oracle as O
from seeker_amd import SeekerError
from seeker_amd import synth as S
from seeker_amd._native import (SH_ERR_UNSUPPORTED, SH_SAMPLE_COMPARE, SH_SAMPLE_REJECTION, sh_sampling)

pytestmark = pytest.mark.gpu

# (T, top_k, top_p, min_p)
CFGS = [
    (0.8, 40, 1.0, 0.0),
    (0.7, 40, 0.9, 0.05),
    (1.0, 256, 0.5, 0.0),
    (1.3, 1, 1.0, 0.0),
    (0.8, 100, 0.95, 0.1),
    (1.0, 7, 0.3, 0.5),
]


def _sampler(T, top_k, top_p, min_p, seed=5, mode=SH_SAMPLE_COMPARE):
    s = sh_sampling()
    s.mode, s.temperature, s.seed, s.counter = mode, T, seed, 0
    s.top_k, s.top_p, s.min_p = top_k, top_p, min_p
    return s


def _accept(engine, p, drafts, s):
    B, k1, V = p.shape
    k = k1 - 1
    pd, dd = engine.to_device(p), engine.to_device(drafts)
    acc, nxt = engine.dev_alloc(4 * B), engine.dev_alloc(4 * B)
    try:
        engine.accept_sample(pd, None, dd, B, k, V, s, acc, nxt)
        return acc.read(np.uint32, B), nxt.read(np.uint32, B)
    finally:
        for x in (pd, dd, acc, nxt):
            x.free()


def _logits(kind, B, k, V, seed):
    x = S.normal_f32(seed, 30, B * (k + 1) * V, 0.0, 3.0).reshape(B, k + 1, V)
    if kind == "ties":  # integer logits: many candidates tie at the top_k threshold
        x = np.round(x).astype(np.float32)
    elif kind == "masked":  # most of the vocabulary at -inf
        x[..., 20:] = -np.inf
    return np.ascontiguousarray(x, dtype=np.float32)


@pytest.mark.parametrize("kind,V", [("normal", 128256), ("normal", 1000), ("ties", 1000), ("masked", 500),
                                    ("normal", 200)])
@pytest.mark.parametrize("cfg", CFGS, ids=lambda c: "T%g-k%d-p%g-m%g" % c)
def test_filtered_compare_matches_oracle(engine, kind, V, cfg):
    T, top_k, top_p, min_p = cfg
    B, k = 6, 3
    print(f"filters {kind} V={V} cfg={cfg}", flush=True)
    p = _logits(kind, B, k, V, seed=11 + V % 7)
    ocfg = O.SamplerCfg(T, top_k, top_p, min_p)
    U = O.philox_uniforms(5, 0x5EC, 0, 2 * B * (k + 1)).reshape(B, k + 1, 2)
    # drafts: the oracle's own draws at the first positions (so acceptance runs
    # on), a different id at one position per sequence
    drafts = np.zeros((B, k), np.uint32)
    for b in range(B):
        for i in range(k):
            t = O.sample_one(p[b, i], ocfg, float(U[b, i, 1]))
            drafts[b, i] = t if i != b % (k + 1) else (t + 1) % V
    a, n = _accept(engine, p, drafts, _sampler(T, top_k, top_p, min_p))
    for b in range(B):
        em = O.sample_and_compare(p[b], drafts[b], ocfg, U[b, :, 1].copy(), mode=0)
        assert (a[b], n[b]) == (len(em) - 1, em[-1]), (b, a[b], n[b], em)


def test_filtered_draws_follow_the_filtered_distribution(engine):
    """One row, 4000 draws (explicit uniforms through the batched verify rows
    would need a model; here B = 4000 sequences of k = 1 share the row): the
    empirical frequencies of the drawn ids match the chain's probabilities
    (chi^2), and no id outside the kept candidates is ever drawn."""
    V, B, T, top_k, top_p, min_p = 1000, 4000, 0.9, 20, 0.8, 0.02
    row = S.normal_f32(3, 31, V, 0.0, 2.0)
    p = np.broadcast_to(row, (B, 2, V)).copy()
    # the chain's probabilities: the oracle with a fine grid of uniforms
    ocfg = O.SamplerCfg(T, top_k, top_p, min_p)
    grid = (np.arange(20000) + 0.5) / 20000
    ref = np.bincount([O.sample_one(row, ocfg, float(u)) for u in grid], minlength=V) / grid.size
    kept = ref > 0
    # a draft no draw can equal: every next token is the column-0 draw
    drafts = np.full((B, 1), int(np.argmin(row)), np.uint32)
    s = _sampler(T, top_k, top_p, min_p, seed=77)
    a, n = _accept(engine, p, drafts, s)
    assert np.all(a == 0)
    assert kept.sum() <= top_k and np.all(kept[n])
    cnt = np.bincount(n, minlength=V)[kept]
    exp = B * ref[kept]
    chi2 = float(np.sum((cnt - exp) ** 2 / exp))
    print(f"kept {kept.sum()} candidates, chi2 {chi2:.1f}", flush=True)
    assert chi2 < 3.0 * kept.sum() + 30


def test_filter_refusals(engine):
    B, k, V = 2, 2, 1000
    p = _logits("normal", B, k, V, seed=1)
    drafts = np.zeros((B, k), np.uint32)
    for cfg in [(0.8, 300, 1.0, 0.0), (0.8, 0, 0.9, 0.0), (0.8, 0, 1.0, 0.1)]:
        with pytest.raises(SeekerError) as ei:
            _accept(engine, p, drafts, _sampler(*cfg))
        assert ei.value.status == SH_ERR_UNSUPPORTED, cfg
    # REJECTION takes no filters
    pd, qd, dd = engine.to_device(p), engine.to_device(p[:, :k].copy()), engine.to_device(drafts)
    acc, nxt = engine.dev_alloc(4 * B), engine.dev_alloc(4 * B)
    with pytest.raises(SeekerError) as ei:
        engine.accept_sample(pd, qd, dd, B, k, V, _sampler(0.8, 40, 1.0, 0.0, mode=SH_SAMPLE_REJECTION), acc, nxt)
    assert ei.value.status == SH_ERR_UNSUPPORTED
    for x in (pd, qd, dd, acc, nxt):
        x.free()
