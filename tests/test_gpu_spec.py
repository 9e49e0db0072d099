"""GPU speculative decoding (sh_spec_step) vs the oracle on configs[0]:
tiny Llama target (4 layers, d 512, Q8_0) + 1-layer draft, prompt of 64
uniform ids (seed 1234), k = 4, greedy, 128 new tokens.

Invariants: the accepted-token stream is bit-identical to the oracle's and to
plain (non-speculative) greedy decoding (scripts/validate_spec_b1.sh); the KV
positions match after every step; with the draft equal to the target every
draft is accepted (forced acceptance)."""
import numpy as np
import pytest

import oracle as O
from parity import NARROW_REL, WIDE_REL, logits_close, pair, record
from seeker_amd import synth as S

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def models(engine):
    ti = S.GgufImage(S.TINY_TARGET, seed=0)
    di = S.GgufImage(S.TINY_DRAFT, seed=1)
    gt, gd = engine.upload_weights(ti), engine.upload_weights(di)
    ot, od = O.Model(ti), O.Model(di)
    pair(ot, gt)  # the reference's wide-GEMM and cm1 attention arithmetic where the GPU uses them
    pair(od, gd)
    yield gt, gd, ot, od
    for m in (gt, gd, ot, od):
        m.close()
    ti.close()
    di.close()


def _gpu_decode(engine, gt, gd, prompt, n_new, k):
    tkv = engine.allocate_kv_cache(gt, 512)
    dkv = engine.allocate_kv_cache(gd, 512)
    lg, _ = engine.forward_full_readback(gt, tkv, prompt, 0, full_logits=False, want_residual=False)
    engine.forward_full_readback(gd, dkv, prompt, 0, full_logits=False, want_residual=False)
    out = [int(lg[0].argmax())]
    steps = []
    while len(out) < n_new:
        r = engine.decode_speculative(gt, gd, tkv, dkv, out[-1], k)
        steps.append((r.emitted, r.drafts))
        out.extend(r.emitted)
        assert tkv.position == len(prompt) + len(out) - 1
    tkv.close()
    dkv.close()
    return out[:n_new], steps


def _oracle_decode(ot, od, prompt, n_new, k):
    tkv, dkv = O.KvCache(ot, 512), O.KvCache(od, 512)
    lg, _ = O.forward(ot, tkv, prompt, 0, logits_mode=1)
    O.forward(od, dkv, prompt, 0, logits_mode=0)
    out = [O.argmax(lg[0])]
    while len(out) < n_new:
        em, _ = O.spec_step_greedy(ot, od, tkv, dkv, out[-1], k)
        out.extend(em)
    tkv.close(); dkv.close()
    return out[:n_new]


def test_spec_decode_config1_matches_oracle(engine, models):
    gt, gd, ot, od = models
    prompt = S.tokens(1234, 64, gt.dims.n_vocab)
    print("spec decode configs[0]: 128 tokens, k=4", flush=True)
    g, steps = _gpu_decode(engine, gt, gd, prompt, 128, 4)
    o = _oracle_decode(ot, od, prompt, 128, 4)
    assert g == o


def test_spec_decode_k8_two_verify_chunks(engine, models):
    """k = 8: the 9-column verify of the Q8_0 target takes two chunks of the
    8-column path; every column's greedy id must come from its own logits."""
    gt, gd, ot, od = models
    prompt = S.tokens(808, 24, gt.dims.n_vocab)
    print("spec decode k=8 (two verify chunks): 48 tokens", flush=True)
    g, steps = _gpu_decode(engine, gt, gd, prompt, 48, 8)
    assert max(len(d) for _, d in steps) == 8
    o = _oracle_decode(ot, od, prompt, 48, 8)
    assert g == o


def test_spec_decode_lossless_vs_plain_greedy(engine, models):
    """Spec decode emits what plain greedy decoding emits. The invariant is
    exact when the verify computes the same attention as single-token decode:
    with the cm1 attention (the reference's, f16 P and output) the verify's
    logits differ from decode's by f16 roundings, so a near-tie could flip, as
    it could in the reference; the check runs with the switch off."""
    gt, gd, ot, od = models
    gt.cm1_attention = gd.cm1_attention = False
    try:
        _lossless(engine, gt, gd)
    finally:
        gt.cm1_attention = gd.cm1_attention = True


def _lossless(engine, gt, gd):
    prompt = S.tokens(4321, 32, gt.dims.n_vocab)
    kv = engine.allocate_kv_cache(gt, 256)
    lg, _ = engine.forward_full_readback(gt, kv, prompt, 0, full_logits=False, want_residual=False)
    plain = [int(lg[0].argmax())]
    for i in range(40):
        lg, _ = engine.forward_full_readback(gt, kv, [plain[-1]], 32 + i, full_logits=False, want_residual=False)
        plain.append(int(lg[0].argmax()))
    kv.close()
    g, _ = _gpu_decode(engine, gt, gd, prompt, 41, 4)
    assert g == plain


def test_forced_acceptance(engine, models):
    gt, gd, ot, od = models
    prompt = S.tokens(55, 16, gt.dims.n_vocab)
    out, steps = _gpu_decode(engine, gt, gt, prompt, 40, 7)
    assert all(len(em) == 8 for em, _ in steps[:-1])
    o = _oracle_decode(ot, ot, prompt, 40, 7)
    assert out == o


def _stochastic_lockstep(engine, gt, gd, ot, od, mode, T, seed, n_steps, k):
    """Runs GPU stochastic spec steps and, per step, checks against the oracle:
    (1) decisions bit-exact: the oracle's draft draws / argmaxes and its
        acceptance (or_spec_draft_token, or_spec_accept) on the step's own GPU
        logits with the same Philox words reproduce the GPU's drafts and
        emitted tokens;
    (2) numerics: the oracle's forwards of the same tokens (draft: pending +
        last, then d_1..d_{n-1}; target: [last, d_1..d_n]) give logits within
        2e-2 abs / 1e-2 rel (north star) and the bounds of tests/parity.py;
    (3) both caches' positions equal the oracle's after the truncation."""
    from seeker_amd._native import sh_sampling
    prompt = S.tokens(1234, 64, gt.dims.n_vocab)
    V = gt.dims.n_vocab
    gtkv, gdkv = engine.allocate_kv_cache(gt, 512), engine.allocate_kv_cache(gd, 512)
    otkv, odkv = O.KvCache(ot, 512), O.KvCache(od, 512)
    lg, _ = engine.forward_full_readback(gt, gtkv, prompt, 0, full_logits=False, want_residual=False)
    engine.forward_full_readback(gd, gdkv, prompt, 0, full_logits=False, want_residual=False)
    O.forward(ot, otkv, prompt, 0, logits_mode=0)
    O.forward(od, odkv, prompt, 0, logits_mode=0)
    last, pending = int(lg[0].argmax()), []
    s = sh_sampling()
    s.mode, s.temperature, s.seed, s.counter = mode, T, seed, 0
    accepted = 0
    for step in range(n_steps):
        P = gtkv.position
        ctr = s.counter
        r = engine.decode_speculative(gt, gd, gtkv, gdkv, last, k, s)
        n = len(r.drafts)
        assert s.counter == ctr + 3 * n + 2
        pg, qg = engine.spec_step_logits()
        u = O.spec_uniforms(seed, ctr, n)
        for i in range(n):
            assert O.spec_draft_token(mode, qg[i], T, float(u[2 * (n + 1) + i])) == r.drafts[i], (step, i)
        assert O.spec_accept(mode, pg, qg, r.drafts, T, u) == r.emitted, step
        # oracle forwards of the tokens the GPU fed
        feed = pending + [last]
        ql, _ = O.forward(od, odkv, feed, odkv.position, logits_mode=1)
        oq = [ql[0]]
        for i in range(1, n):
            ql, _ = O.forward(od, odkv, [r.drafts[i - 1]], odkv.position, logits_mode=1)
            oq.append(ql[0])
        op, _ = O.forward(ot, otkv, [last] + r.drafts, P, logits_mode=2)
        rel = WIDE_REL if (gt.cm1_attention or gt.wide_f16) else NARROW_REL  # f16 roundings: tests/parity.py
        for got, want in ((qg, np.stack(oq)), (pg, op)):
            err = np.abs(got - want)
            assert np.all(err <= np.maximum(2e-2, 1e-2 * np.abs(want))), float(err.max())
            assert err.max() <= rel * np.abs(want).max(), float(err.max())
        acc = len(r.emitted) - 1
        accepted += acc
        otkv.truncate(P + acc + 1)
        odkv.truncate(P + acc + 1)
        pending = [r.drafts[-1]] if acc == n else []
        assert gtkv.position == otkv.position == P + acc + 1
        assert gdkv.position + len(pending) == gtkv.position and odkv.position == gdkv.position
        last = r.emitted[-1]
    for x in (gtkv, gdkv, otkv, odkv):
        x.close()
    return accepted


@pytest.mark.parametrize("mode", [1, 2], ids=["compare", "rejection"])
def test_stochastic_spec_step_lockstep(engine, models, mode):
    gt, gd, ot, od = models
    print(f"stochastic spec step lockstep, mode {mode}", flush=True)
    acc = _stochastic_lockstep(engine, gt, gd, ot, od, mode, 0.8, seed=21 + mode, n_steps=12, k=4)
    if mode == 2:
        assert acc > 0  # near-uniform p and q: many sampled drafts are accepted


def _stream_vs_own(engine, gt, gd, ot, od, mode, T, seed, k, n_steps):
    """The GPU's stochastic speculative decode against the oracle's own
    (or_spec_step on the oracle's own logits, the same Philox words), step
    after step until the streams part. Returns (steps equal, 1 if they
    parted). A parting step must be a near tie: the two sides' logits of the
    rows that decided it agree within the parity bounds, and the oracle's rule
    on the GPU's own logits gives the GPU's tokens (a draw or accept test
    within rounding of its threshold flips; nothing else may)."""
    from seeker_amd._native import sh_sampling
    prompt = S.tokens(777 + seed, 64, gt.dims.n_vocab)
    gtkv, gdkv = engine.allocate_kv_cache(gt, 512), engine.allocate_kv_cache(gd, 512)
    otkv, odkv = O.KvCache(ot, 512), O.KvCache(od, 512)
    lg, _ = engine.forward_full_readback(gt, gtkv, prompt, 0, full_logits=False, want_residual=False)
    engine.forward_full_readback(gd, gdkv, prompt, 0, full_logits=False, want_residual=False)
    ol, _ = O.forward(ot, otkv, prompt, 0, logits_mode=1)
    O.forward(od, odkv, prompt, 0, logits_mode=0)
    last = int(lg[0].argmax())
    assert last == O.argmax(ol[0])
    s = sh_sampling()
    s.mode, s.temperature, s.seed, s.counter = mode, T, seed, 0
    wide = gt.cm1_attention or gt.wide_f16
    equal, parted = 0, 0
    for step in range(n_steps):
        ctr = s.counter
        r = engine.decode_speculative(gt, gd, gtkv, gdkv, last, k, s)
        pg, qg = engine.spec_step_logits()
        u = O.spec_uniforms(seed, ctr, len(r.drafts))
        em, dr, po, qo = O.spec_step(ot, od, otkv, odkv, last, k, mode, T, u, want_logits=True)
        if em == r.emitted and dr == r.drafts:
            assert gtkv.position == otkv.position
            equal += 1
            last = em[-1]
            continue
        j = next((i for i in range(len(dr)) if dr[i] != r.drafts[i]), len(dr) - 1)
        logits_close(np.asarray(qg[: j + 1]), np.asarray(qo[: j + 1]), wide)
        logits_close(np.asarray(pg[: j + 1]), np.asarray(po[: j + 1]), wide)
        assert O.spec_accept(mode, pg, qg, r.drafts, T, u) == r.emitted, step
        print(f"  seed {seed}: streams part at step {step} (near tie)", flush=True)
        parted = 1
        break
    for x in (gtkv, gdkv, otkv, odkv):
        x.close()
    return equal, parted


@pytest.mark.parametrize("mode", [1, 2], ids=["compare", "rejection"])
def test_stochastic_stream_equals_oracle_own(engine, models, mode):
    """End to end over 4 seeds x 16 steps: the GPU's token stream equals the
    oracle's own stochastic decode up to a near tie (see _stream_vs_own); the
    steps compared and the near ties are recorded in the parity log."""
    gt, gd, ot, od = models
    print(f"stochastic stream vs the oracle's own decode, mode {mode}", flush=True)
    equal = parted = 0
    for seed in range(4):
        e, p = _stream_vs_own(engine, gt, gd, ot, od, mode, 0.8, 31 + 10 * seed + mode, 4, 16)
        equal += e
        parted += p
    record("stochastic_stream_steps", equal + parted, parted)
    assert equal >= 32, (equal, parted)


def test_rejection_spec_step_draft_equals_target(engine, models):
    """Draft == target model: q ~= p, so almost every sampled draft is accepted."""
    gt, gd, ot, od = models
    print("rejection spec step, draft = target", flush=True)
    acc = _stochastic_lockstep(engine, gt, gt, ot, ot, 2, 0.8, seed=5, n_steps=6, k=4)
    assert acc >= 6 * 4 - 2


def test_spec_step_explicit_uniforms(engine, models):
    """sh_sampling.uniforms (3n + 2 floats) gives the same step as the Philox words it replaces."""
    from seeker_amd._native import SH_SAMPLE_REJECTION, sh_sampling
    gt, gd, _, _ = models
    prompt = S.tokens(4242, 32, gt.dims.n_vocab)
    outs = []
    for explicit in (False, True):
        tkv, dkv = engine.allocate_kv_cache(gt, 256), engine.allocate_kv_cache(gd, 256)
        engine.prefill(gt, tkv, prompt, 0)
        engine.prefill(gd, dkv, prompt, 0)
        s = sh_sampling()
        s.mode, s.temperature, s.seed, s.counter = SH_SAMPLE_REJECTION, 0.8, 99, 40
        keep = O.spec_uniforms(99, 40, 4)
        if explicit:
            s.uniforms = keep.ctypes.data_as(O.F32P)
        r = engine.decode_speculative(gt, gd, tkv, dkv, int(prompt[-1]), 4, s)
        outs.append((r.emitted, r.drafts, tkv.position))
        tkv.close(); dkv.close()
    assert outs[0] == outs[1]


def test_batched_spec_step_draft_equals_target(engine, models):
    """sh_spec_step_batch with the draft equal to the target: every draft is
    accepted, so every step emits k + 1 tokens and the draft caches carry d_n
    as pending into the next step's first draft forward. Three sequences with
    different prompt lengths, four steps, equal to the oracle's single-sequence
    greedy steps token for token (attention as the batched path computes it),
    and to plain greedy decoding of each sequence."""
    gt, gd, ot, od = models
    V = gt.dims.n_vocab
    prompts = [S.tokens(900 + b, 20 + 7 * b, V) for b in range(3)]
    ot.set_attn_cm1(False)  # the batched verify's attention: the scalar kernel's arithmetic
    tk, dk, otk = [], [], []
    last = []
    for pr in prompts:
        t, d = engine.allocate_kv_cache(gt, 256), engine.allocate_kv_cache(gt, 256)
        lg, _ = engine.forward_full_readback(gt, t, pr, 0, full_logits=False, want_residual=False)
        engine.forward_full_readback(gt, d, pr, 0, full_logits=False, want_residual=False)
        o = O.KvCache(ot, 256)
        ot.set_attn_cm1(True)  # the prefill: the single-sequence (cm1) attention, as on the GPU
        O.forward(ot, o, pr, 0, logits_mode=0)
        ot.set_attn_cm1(False)
        tk.append(t); dk.append(d); otk.append(o)
        last.append(int(lg[0].argmax()))
    odk = []
    for b, pr in enumerate(prompts):
        o = O.KvCache(ot, 256)
        ot.set_attn_cm1(True)
        O.forward(ot, o, pr, 0, logits_mode=0)
        ot.set_attn_cm1(False)
        odk.append(o)
    for step in range(4):
        em, dr = engine.spec_step_batch(gt, gt, tk, dk, last, 4)
        for b in range(3):
            o_em, o_dr = O.spec_step_greedy(ot, ot, otk[b], odk[b], last[b], 4)
            assert (em[b], dr[b]) == (o_em, o_dr), (step, b)
            assert len(em[b]) == 5 and tk[b].position == otk[b].position
        last = [e[-1] for e in em]
    ot.set_attn_cm1(gt.cm1_attention)
    for x in tk + dk + otk + odk:
        x.close()
