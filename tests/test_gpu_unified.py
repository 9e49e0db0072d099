"""Batched verify (sh_verify_unified, Engine::verify_unified inference/mod.rs:2316-2398)
on the GPU.

Within one kernel path every column's arithmetic is independent of which
other columns share its launch (GEMV columns, per-column RMSNorm and operand
scales, attention splits at absolute key indices, multi-group split-K shapes
that depend on the matrix only). Chunks of up to 8 columns take the 8-column
GEMV kernels; longer chunks of an all-Q4_K model take the multi-group kernel.
So a batch of B sequences gives bit-identical logits, ids, residuals and KV
rows to B separate sh_forward_full calls whenever both take the same path,
however the flat packing cuts sequences across chunks; across the two paths
only the f32 summation order differs (checked to 1e-5 of the logit scale, same
argmax). The separate calls are themselves checked against the C oracle in
test_gpu_forward.py; here the batch is also compared to the oracle per
sequence.
"""
import numpy as np
import pytest

import oracle as O
from parity import WIDE_REL, NARROW_REL, pair
from seeker_amd import SeekerError
from seeker_amd import _native as N
from seeker_amd import synth as S
from seeker_amd._native import GGML_Q4_K, SH_ERR_ARG, SH_ERR_CAPACITY

pytestmark = pytest.mark.gpu

SHAPES = {
    "tiny_q8": S.TINY_TARGET,
    "gqa_q4k": S.LlamaShape(2, 1024, 8, 2, 2048, 4000, 512, 1e-5, 5e5, 0.02, GGML_Q4_K, GGML_Q4_K),
}


@pytest.fixture(scope="module", params=list(SHAPES))
def model(request, engine):
    img = S.GgufImage(SHAPES[request.param], seed=0)
    print(f"model {request.param}", flush=True)
    gm = engine.upload_weights(img)
    yield request.param, img, gm
    gm.close()
    img.close()


def _prefilled(engine, gm, prompt, max_seq=256):
    kv = engine.allocate_kv_cache(gm, max_seq)
    engine.prefill(gm, kv, prompt, 0)
    return kv


def _kv_rows(kv, gm, lo, hi):
    out = []
    for layer in range(gm.dims.n_layer):
        for isv in (False, True):
            out.append(kv.read_layer(layer, isv, hi)[lo:hi])
    return out


# (prefix length, verify length) per sequence; flat packing 5 + 11 + 3 + 9 = 28
# columns cuts sequences 1 and 3 across 8-column chunks.
SEQS = [(20, 5), (37, 11), (5, 3), (12, 9)]


def test_unified_equals_separate_forwards(engine, model):
    name, img, gm = model
    V = gm.vocab_size()
    prompts = [S.tokens(100 + s, p, V) for s, (p, _) in enumerate(SEQS)]
    drafts = [S.tokens(200 + s, n, V) for s, (_, n) in enumerate(SEQS)]
    batch_kv = [_prefilled(engine, gm, pr) for pr in prompts]
    ref_kv = [_prefilled(engine, gm, pr) for pr in prompts]
    toks = np.concatenate(drafts)
    lens = [n for _, n in SEQS]
    positions = np.concatenate([np.arange(p, p + n) for p, n in SEQS])
    out = engine.verify_unified(gm, batch_kv, toks, lens, positions=positions, want_logits=True,
                                want_residual=True)
    assert list(out.q_starts) == [0, 5, 16, 19]
    multi_group = name == "gqa_q4k"  # all-Q4_K: chunks above 8 columns take the multi-group kernel
    batch_mg = multi_group and sum(lens) > 8
    for s, (p, n) in enumerate(SEQS):
        # the batch's attention is the reference's scalar kernel: the separate
        # calls take it too (cm1 attention off)
        gm.cm1_attention = False
        lg, res = engine.forward_full_readback(gm, ref_kv[s], drafts[s], p, full_logits=True, want_residual=True)
        gm.cm1_attention = True
        q = int(out.q_starts[s])
        same_path = batch_mg == (multi_group and n > 8)
        print(f"{name} seq {s}: logits max|d| {np.abs(out.logits[q:q + n] - lg).max():.3e} "
              f"(same path {same_path})", flush=True)
        assert np.array_equal(out.sampled[q:q + n], lg.argmax(axis=1).astype(np.uint32))
        assert batch_kv[s].position == p + n
        rows = zip(_kv_rows(batch_kv[s], gm, p, p + n), _kv_rows(ref_kv[s], gm, p, p + n))
        if same_path:
            assert np.array_equal(out.logits[q:q + n], lg)
            assert np.array_equal(out.residual[q:q + n], res)
            for a, b in rows:
                assert np.array_equal(a, b)
        else:
            # different kernels: the 8-column path's attention (expf, one key
            # block per wave, split combine) and the batched path's (exp2,
            # 64-key tiles, other split boundaries) round differently; both
            # stay within 3e-4 max of the oracle (test_unified_tree_and_chain_vs_oracle)
            assert np.abs(out.logits[q:q + n] - lg).max() <= 5e-5 * np.abs(lg).max()
            assert np.abs(out.residual[q:q + n] - res).max() <= 5e-5 * np.abs(res).max()
            for a, b in rows:
                a, b = a.astype(np.float32), b.astype(np.float32)
                assert np.abs(a - b).max() <= 2e-3 * max(np.abs(b).max(), 1e-3)
    for kv in batch_kv + ref_kv:
        kv.close()


def test_unified_tree_and_chain_vs_oracle(engine, model):
    """One tree sequence (branching 2, 2: 1 + 2 + 4 nodes below the root) next to a
    chain; each compared with its own forward (bit-exactly on the same kernel
    path, else to 1e-5 of the logit scale) and, within the north-star
    tolerance, with the oracle."""
    name, img, gm = model
    V = gm.vocab_size()
    om = O.Model(img)
    wide = pair(om, gm)  # the prefills' arithmetic (wide GEMMs, cm1 attention) where the GPU uses it
    parents_tree = [-1, 0, 0, 1, 1, 2, 2]
    seqs = [(24, S.tokens(301, 7, V), parents_tree), (16, S.tokens(302, 6, V), None)]
    prompts = [S.tokens(400 + s, p, V) for s, (p, _, _) in enumerate(seqs)]
    batch_kv = [_prefilled(engine, gm, pr) for pr in prompts]
    toks = np.concatenate([t for _, t, _ in seqs])
    lens = [len(t) for _, t, _ in seqs]
    parents = np.array(parents_tree + [-1, 0, 1, 2, 3, 4], dtype=np.int32)
    out = engine.verify_unified(gm, batch_kv, toks, lens, parents=parents, want_logits=True)
    for s, (p, t, par) in enumerate(seqs):
        q = int(out.q_starts[s])
        n = len(t)
        ref = _prefilled(engine, gm, prompts[s])
        gm.cm1_attention = False  # the batch's (scalar) attention for the chain
        lg, _ = engine.forward_full_readback(gm, ref, t, p, full_logits=True, parents=par)
        gm.cm1_attention = True
        if name == "gqa_q4k" and sum(lens) > 8 and n <= 8:  # batch multi-group, solo 8-column kernels
            assert np.abs(out.logits[q:q + n] - lg).max() <= 1e-5 * np.abs(lg).max()
            assert np.array_equal(out.logits[q:q + n].argmax(axis=1), lg.argmax(axis=1))
        else:
            assert np.array_equal(out.logits[q:q + n], lg)
        okv = O.KvCache(om, 256)
        O.forward(om, okv, prompts[s], 0, logits_mode=0)
        ol, _ = O.forward(om, okv, t, p, parents=par, logits_mode=2, batched=True)
        tol = np.maximum(2e-2, 1e-2 * np.abs(ol))
        d = np.abs(out.logits[q:q + n] - ol)
        print(f"{name} seq {s}: vs oracle max|d| {d.max():.3e}", flush=True)
        assert np.all(d <= tol) and d.max() <= (WIDE_REL if wide else NARROW_REL) * np.abs(ol).max()
        okv.close()
        ref.close()
    for kv in batch_kv:
        kv.close()
    om.close()


def test_unified_errors(engine, model):
    name, img, gm = model
    V = gm.vocab_size()
    a = _prefilled(engine, gm, S.tokens(1, 8, V), max_seq=32)
    b = _prefilled(engine, gm, S.tokens(2, 8, V), max_seq=32)
    t = S.tokens(3, 4, V)
    with pytest.raises(SeekerError) as ei:
        engine.verify_unified(gm, [a, a], np.concatenate([t, t]), [4, 4])
    assert ei.value.status == SH_ERR_ARG
    with pytest.raises(SeekerError) as ei:
        engine.verify_unified(gm, [a, b], np.concatenate([t, t]), [4, 4], positions=np.arange(8))
    assert ei.value.status == SH_ERR_ARG
    with pytest.raises(SeekerError) as ei:
        engine.verify_unified(gm, [a], S.tokens(4, 30, V), [30])
    assert ei.value.status == SH_ERR_CAPACITY
    assert a.position == 8 and b.position == 8  # failed calls leave the caches alone
    a.close()
    b.close()


def test_tree_verify_step(engine, model):
    """sh_tree_verify_step = verify_unified (device logits) + tree acceptance +
    path compaction: the path equals the oracle's acceptance on the same verify
    logits, and decoding continues from the compacted cache as it does after a
    plain chain forward of the accepted path."""
    from seeker_amd._native import SH_SAMPLE_REJECTION, sh_sampling
    name, img, gm = model
    V = gm.vocab_size()
    par1 = np.array([-1, 0, 0, 1, 1, 2, 2], np.int32)  # branching 2, 2
    B, n = 3, par1.size
    prompts = [S.tokens(500 + b, 12 + 5 * b, V) for b in range(B)]
    tokens = np.stack([np.concatenate([[int(pr[-1])], S.tokens(600 + b, n - 1, V)]) for b, pr in
                       enumerate(prompts)]).astype(np.uint32)
    parents = np.tile(par1, (B, 1))
    # reference logits from a plain batched verify of the same trees
    ref_kv = [_prefilled(engine, gm, pr[:-1]) for pr in prompts]
    out = engine.verify_unified(gm, ref_kv, tokens.reshape(-1), [n] * B, parents=parents.reshape(-1),
                                want_logits=True)
    q = S.normal_f32(9, 9, B * n * V, 0.0, 3.0).reshape(B, n, V)
    q[0] = out.logits[:n]  # q = p: tree 0 accepts the first child at every level (path 0, 1, 3)
    qd = engine.to_device(q)
    s = sh_sampling()
    s.mode, s.temperature, s.seed, s.counter = SH_SAMPLE_REJECTION, 1.0, 17, 0
    U = O.philox_uniforms(17, 0x5EC, 0, 2 * B * n).reshape(B, n, 2)
    kv = [_prefilled(engine, gm, pr[:-1]) for pr in prompts]
    paths, nxt = engine.tree_verify_step(gm, kv, tokens, parents, qd, s)
    for b in range(B):
        lg = out.logits[b * n:(b + 1) * n]
        opath, onext = O.tree_accept(lg, q[b], tokens[b], parents[b], 1.0, U[b])
        print(f"{name} tree {b}: path {paths[b]} next {nxt[b]}", flush=True)
        assert paths[b] == opath and nxt[b] == onext
        if b == 0:
            assert paths[b] == [0, 1, 3]
        base = len(prompts[b]) - 1
        assert kv[b].position == base + len(paths[b])
        # continue after the compacted path vs after a chain forward of it
        chain = _prefilled(engine, gm, prompts[b][:-1])
        gm.cm1_attention = False  # the tree batch's attention: the scalar kernel's arithmetic
        engine.forward_full_readback(gm, chain, tokens[b][paths[b]], base, full_logits=False)
        gm.cm1_attention = True
        a, _ = engine.forward_full_readback(gm, kv[b], [int(nxt[b])], kv[b].position, full_logits=False)
        c, _ = engine.forward_full_readback(gm, chain, [int(nxt[b])], chain.position, full_logits=False)
        d = np.abs(a - c).max()
        assert d <= 3e-4 * np.abs(c).max(), d
        chain.close()
    qd.free()
    for x in kv + ref_kv:
        x.close()


def test_unified_sampled_per_sequence(engine, model):
    """sh_verify_unified_sampled: every column sampled with its own sequence's
    sampler (samplers[col_seq[i]].record_chain, inference/mod.rs:2375-2386).
    Greedy sequences keep the argmax; COMPARE sequences draw column j from
    softmax(l / T) in vocab order with Philox word counter + j of key
    (seed, 0x5EC) or with their explicit uniforms[j], checked against the
    oracle's sampler on the same returned logits (the filtered chain against
    or_sample_one)."""
    from seeker_amd._native import SH_SAMPLE_COMPARE, SH_SAMPLE_GREEDY, SH_SAMPLE_REJECTION, sh_sampling
    name, img, gm = model
    V = gm.vocab_size()
    prompts = [S.tokens(700 + s, p, V) for s, (p, _) in enumerate(SEQS)]
    drafts = [S.tokens(800 + s, n, V) for s, (_, n) in enumerate(SEQS)]
    lens = [n for _, n in SEQS]
    toks = np.concatenate(drafts)
    u_explicit = S.normal_f32(3, 3, lens[2], 0.5, 0.2).clip(0.01, 0.99).astype(np.float32)
    # the last sequence samples through the candidate filters (top_k 50, top_p 0.9, min_p 0.05)
    cfg = [(SH_SAMPLE_GREEDY, 0.0, 0, 0, None), (SH_SAMPLE_COMPARE, 0.8, 5, 7, None),
           (SH_SAMPLE_COMPARE, 1.3, 0, 0, u_explicit), (SH_SAMPLE_COMPARE, 0.5, 9, 0, None)]
    filters = [None, None, None, (50, 0.9, 0.05)]
    samplers = []
    for (mode, t, seed, ctr, u), f in zip(cfg, filters):
        sp = sh_sampling()
        sp.mode, sp.temperature, sp.seed, sp.counter = mode, t, seed, ctr
        if u is not None:
            sp.uniforms = u.ctypes.data_as(N.F32P)
        if f is not None:
            sp.top_k, sp.top_p, sp.min_p = f
        samplers.append(sp)
    kv = [_prefilled(engine, gm, pr) for pr in prompts]
    # a REJECTION sampler is refused before anything runs
    bad = sh_sampling()
    bad.mode, bad.temperature = SH_SAMPLE_REJECTION, 1.0
    with pytest.raises(SeekerError) as ei:
        engine.verify_unified(gm, kv, toks, lens, samplers=[samplers[0], bad, samplers[2], samplers[3]])
    assert ei.value.status == SH_ERR_ARG
    assert [k.position for k in kv] == [p for p, _ in SEQS]
    out = engine.verify_unified(gm, kv, toks, lens, want_logits=True, samplers=samplers)
    differs = 0
    for s, (mode, t, seed, ctr, u) in enumerate(cfg):
        q, n = int(out.q_starts[s]), lens[s]
        lg = out.logits[q:q + n]
        got = out.sampled[q:q + n]
        if mode == SH_SAMPLE_GREEDY:
            want = lg.argmax(axis=1)
            assert samplers[s].counter == 0
        elif filters[s] is not None:
            us = O.philox_uniforms(seed, 0x5EC, ctr, n)
            ocfg = O.SamplerCfg(t, *filters[s])
            want = [O.sample_one(lg[j], ocfg, float(us[j])) for j in range(n)]
            assert samplers[s].counter == ctr + n
        else:
            us = u if u is not None else O.philox_uniforms(seed, 0x5EC, ctr, n)
            want = [O.sample_vocab_order(lg[j], t, float(us[j])) for j in range(n)]
            assert samplers[s].counter == ctr + n
            differs += int(np.sum(got != lg.argmax(axis=1)))
        print(f"{name} seq {s}: sampled {list(got)} want {list(want)}", flush=True)
        assert np.array_equal(got, np.asarray(want, dtype=np.uint32))
        assert kv[s].position == SEQS[s][0] + n
    assert differs > 0  # small random-init logits: temperature sampling leaves the argmax
    for k in kv:
        k.close()
