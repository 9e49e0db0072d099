"""GPU parity of the qwen3 and qwen3moe forwards against the C oracle.

qwen3 (models/qwen3.rs): decoupled head_dim (q width n_head * head_dim above
n_embd), per-head Q/K RMSNorm with learned weights, NEOX RoPE, tied
embeddings. qwen3moe: the same attention with a routed-expert FFN (softmax
router over the experts, top-k with renormalized weights, per-expert SwiGLU;
models/qwen35moe.rs:3117-3182 without the shared expert), run on the
expert-indirect Q4_K GEMM. Chunks of 1, 5, 8, 12 and 64 columns, a tree chunk,
and batched verification of several sequences (pairs of columns and experts
grouped across sequences) are compared with the oracle: logits within 2e-2
abs / 1e-2 rel (north star) and 3e-4 x max|logit|, greedy ids equal.

The last test runs BASELINE configs[4]'s layer shapes (Qwen3-30B-A3B: d 2048,
32 / 4 heads, head_dim 128, 128 experts top-8, expert FFN 768, vocab 151936;
two layers) at batch 8 x 7 columns over 16384 cached keys, with identical
synthetic f16 K/V in both caches, and the Qwen3-0.6B draft layer shape.
"""
import numpy as np
import pytest

import oracle as O
from parity import ids_agree, logits_close, pair
from seeker_amd import synth as S
from seeker_amd._native import GGML_Q4_K

pytestmark = pytest.mark.gpu

QWEN3 = S.LlamaShape(2, 512, 8, 4, 1024, 3000, 1024, 1e-6, 1e6, 0.02, GGML_Q4_K, GGML_Q4_K, True, arch=1,
                     head_dim=128, norm_jitter=0.2)
QWEN3MOE = S.LlamaShape(2, 512, 8, 2, 0, 3000, 1024, 1e-6, 1e6, 0.03, GGML_Q4_K, GGML_Q4_K, False, arch=2,
                        head_dim=128, n_expert=32, n_expert_used=4, expert_ff=512, norm_jitter=0.2,
                        router_std=512 ** -0.5)


def close(a, b, wide=False):
    logits_close(a, b, wide)  # after a wide call: the bounds of tests/parity.py


@pytest.fixture(scope="module", params=["qwen3", "qwen3moe"])
def model(request, engine):
    shape = QWEN3 if request.param == "qwen3" else QWEN3MOE
    img = S.GgufImage(shape, seed=3)
    print(f"model {request.param}", flush=True)
    gm = engine.upload_weights(img)
    om = O.Model(img)
    pair(om, gm)  # the reference's wide-GEMM and cm1 attention arithmetic where the GPU uses them
    yield request.param, gm, om
    gm.close()
    om.close()
    img.close()


def test_dims(model):
    name, gm, om = model
    d = gm.dims
    assert d.head_dim == 128 and d.n_embd == 512 and d.n_head * d.head_dim == 1024


def test_chunks_match_oracle(engine, model):
    name, gm, om = model
    V = gm.dims.n_vocab
    gkv, okv = engine.allocate_kv_cache(gm, 512), O.KvCache(om, 512)
    prompt = S.tokens(70, 40, V)
    # the 40-column prefill (and the 64-column verify): wide GEMMs, cm1 attention
    wide = gm.wide_f16 or gm.cm1_attention
    print(f"{name}: prefill 40", flush=True)
    engine.prefill(gm, gkv, prompt, 0)
    O.forward(om, okv, prompt, 0, logits_mode=0)
    pos = 40
    for n in (1, 5, 8, 12, 64):
        toks = S.tokens(80 + n, n, V)
        print(f"{name}: verify {n} columns at {pos}", flush=True)
        gl, gres = engine.forward_full_readback(gm, gkv, toks, pos)
        ol, ores = O.forward(om, okv, toks, pos)
        close(gl, ol, wide)
        close(gres, ores, wide)
        gkv.truncate(pos)
        ids = engine.verify_greedy(gm, gkv, toks, pos)
        assert np.array_equal(ids, gl.argmax(axis=1))
        ids_agree(gl, ol, wide)
        pos += n
    par = [-1, 0, 0, 1, 1, 2, 3]
    toks = S.tokens(99, len(par), V)
    print(f"{name}: tree of 7 at {pos}", flush=True)
    gl, _ = engine.forward_full_readback(gm, gkv, toks, pos, parents=par)
    ol, _ = O.forward(om, okv, toks, pos, parents=par)
    close(gl, ol, wide)
    gkv.close()
    okv.close()


def test_batched_verify_matches_oracle(engine, model):
    """verify_unified over 4 sequences (3 + 9 + 1 + 14 columns): the MoE pairs of
    all sequences are routed together in one plan per chunk."""
    name, gm, om = model
    V = gm.dims.n_vocab
    seqs = [(20, 3), (33, 9), (7, 1), (15, 14)]
    gk, ok = [], []
    for s, (p, _) in enumerate(seqs):
        pr = S.tokens(300 + s, p, V)
        g, o = engine.allocate_kv_cache(gm, 256), O.KvCache(om, 256)
        engine.prefill(gm, g, pr, 0)
        O.forward(om, o, pr, 0, logits_mode=0)
        gk.append(g)
        ok.append(o)
    drafts = [S.tokens(400 + s, n, V) for s, (_, n) in enumerate(seqs)]
    print(f"{name}: batched verify 4 sequences", flush=True)
    out = engine.verify_unified(gm, gk, np.concatenate(drafts), [n for _, n in seqs], want_logits=True)
    wide = gm.wide_f16 or gm.cm1_attention  # the prefills' f16 roundings
    for s, (p, n) in enumerate(seqs):
        ol, _ = O.forward(om, ok[s], drafts[s], p, batched=True)
        q = int(out.q_starts[s])
        close(out.logits[q:q + n], ol, wide)
        ids_agree(out.logits[q:q + n], ol, wide)
        assert np.array_equal(out.sampled[q:q + n], out.logits[q:q + n].argmax(axis=1))
        assert gk[s].position == p + n
    for x in gk + ok:
        x.close()


T30B_2L = S.LlamaShape(2, 2048, 32, 4, 0, 151936, 40960, 1e-6, 1e6, 0.02, GGML_Q4_K, GGML_Q4_K, False, arch=2,
                       head_dim=128, n_expert=128, n_expert_used=8, expert_ff=768, norm_jitter=0.1,
                       router_std=2048 ** -0.5)
D06B_2L = S.LlamaShape(2, 1024, 16, 8, 3072, 151936, 40960, 1e-6, 1e6, 0.02, GGML_Q4_K, GGML_Q4_K, True, arch=1,
                       head_dim=128, norm_jitter=0.1)


def _seed_kv(gkv, okv, dims, n_pos, rng):
    for layer in range(dims.n_layer):
        for isv in (False, True):
            rows = rng.standard_normal((n_pos, dims.n_head_kv, dims.head_dim)).astype(np.float16).view(np.uint16)
            gkv.write_layer(layer, isv, rows)
            okv.layer(layer, isv, n_pos)[:] = rows
    gkv.set_position(n_pos)
    okv.set_position(n_pos)


@pytest.mark.timeout(900)
def test_config4_moe_verify_b8_l7_at_16384(engine):
    img = S.GgufImage(T30B_2L, seed=0)
    print("configs[4] 2-layer Qwen3-30B-A3B shape", flush=True)
    gm = engine.upload_weights(img)
    om = O.Model(img)
    # the batch of 56 columns is one wide call: its dense matmuls take the
    # wide GEMM's f16 operands (the routed experts keep the f32-level path);
    # the oracle's per-sequence calls of 7 columns then need mode 1
    wide = gm.wide_f16
    om.set_mm16(1 if wide else 0)
    V, P, B, L = gm.dims.n_vocab, 16384, 8, 7
    rng = np.random.default_rng(4)
    gk, ok = [], []
    for b in range(B):
        g, o = engine.allocate_kv_cache(gm, P + 32), O.KvCache(om, P + 32)
        _seed_kv(g, o, gm.dims, P, rng)
        gk.append(g)
        ok.append(o)
    toks = [S.tokens(500 + b, L, V) for b in range(B)]
    print("configs[4] batched verify 8 x 7 at 16384", flush=True)
    out = engine.verify_unified(gm, gk, np.concatenate(toks), [L] * B, want_logits=True)
    for b in range(B):
        ol, _ = O.forward(om, ok[b], toks[b], P, batched=True)
        close(out.logits[b * L:(b + 1) * L], ol, wide)
        ids_agree(out.logits[b * L:(b + 1) * L], ol, wide)
        assert np.array_equal(out.sampled[b * L:(b + 1) * L], out.logits[b * L:(b + 1) * L].argmax(axis=1))
    for x in gk + ok:
        x.close()
    gm.close()
    om.close()
    img.close()


@pytest.mark.timeout(600)
def test_qwen3_06b_draft_shape(engine):
    img = S.GgufImage(D06B_2L, seed=1)
    print("Qwen3-0.6B-shape draft, 2 layers", flush=True)
    gm = engine.upload_weights(img)
    om = O.Model(img)
    wide = pair(om, gm)  # the reference's wide-GEMM and cm1 attention arithmetic where the GPU uses them
    V = gm.dims.n_vocab
    gkv, okv = engine.allocate_kv_cache(gm, 4200), O.KvCache(om, 4200)
    _seed_kv(gkv, okv, gm.dims, 4096, np.random.default_rng(5))
    pos = 4096
    for n in (1, 2, 7):
        toks = S.tokens(600 + n, n, V)
        gl, _ = engine.forward_full_readback(gm, gkv, toks, pos)
        ol, _ = O.forward(om, okv, toks, pos)
        f16 = wide and n > 1 or pos > 4096  # two-column calls and the K/V they shaped: f16 roundings
        close(gl, ol, f16)
        ids_agree(gl, ol, f16)
        pos += n
    for x in (gkv, okv, gm, om):
        x.close()
    img.close()


def test_spec_step_qwen3_draft_moe_target(engine):
    """Greedy speculative steps with a qwen3 draft and a qwen3moe target (the
    configs[4] pairing, small shapes) equal the oracle's, token for token."""
    t_img, d_img = S.GgufImage(QWEN3MOE, seed=7), S.GgufImage(QWEN3, seed=8)
    gt, gd = engine.upload_weights(t_img), engine.upload_weights(d_img)
    ot, od = O.Model(t_img), O.Model(d_img)
    pair(ot, gt)  # the reference's wide-GEMM and cm1 attention arithmetic where the GPU uses them
    pair(od, gd)
    V = gt.dims.n_vocab
    prompt = S.tokens(77, 24, V)
    gtkv, gdkv = engine.allocate_kv_cache(gt, 256), engine.allocate_kv_cache(gd, 256)
    otkv, odkv = O.KvCache(ot, 256), O.KvCache(od, 256)
    lg, _ = engine.forward_full_readback(gt, gtkv, prompt, 0, full_logits=False, want_residual=False)
    engine.prefill(gd, gdkv, prompt, 0)
    O.forward(ot, otkv, prompt, 0, logits_mode=0)
    O.forward(od, odkv, prompt, 0, logits_mode=0)
    last = int(lg[0].argmax())
    for step in range(6):
        r = engine.decode_speculative(gt, gd, gtkv, gdkv, last, 5)
        em, dr = O.spec_step_greedy(ot, od, otkv, odkv, last, 5)
        assert (r.emitted, r.drafts) == (em, dr), step
        assert gtkv.position == otkv.position
        last = em[-1]
    for x in (gtkv, gdkv, otkv, odkv, gt, gd, ot, od):
        x.close()
    t_img.close()
    d_img.close()


@pytest.mark.timeout(900)
def test_config4_batched_spec_step_b8_k6_at_16384(engine):
    """configs[4] as the batch-8 spec decode it is (sh_spec_step_batch, the
    server's step, server/inference.rs:2777-2924): greedy drafts of the
    Qwen3-0.6B-shape draft for all 8 sequences (one batched draft forward per
    position), one batched verify of the Qwen3-30B-A3B-shape MoE target over
    8 x 7 columns at 16384 cached keys (two layers each, the same synthetic
    f16 K/V in both sides' caches; a wide call: f16 dense matmuls), per-sequence
    acceptance and rollback. Three steps equal the oracle's single-sequence
    greedy steps token for token (its attention set to the batched path's
    scalar arithmetic, its target matmuls to the wide GEMM's), with the same
    cache positions."""
    timg, dimg = S.GgufImage(T30B_2L, seed=0), S.GgufImage(D06B_2L, seed=1)
    print("configs[4] batched spec step: 2-layer target and draft", flush=True)
    gt, gd = engine.upload_weights(timg), engine.upload_weights(dimg)
    ot, od = O.Model(timg), O.Model(dimg)
    ot.set_mm16(1 if gt.wide_f16 else 0)  # every target call is the 56-column batched verify: a wide call
    od.set_mm16(0)  # the batched draft forwards: 8 (first position: up to 16) columns
    for om in (ot, od):
        om.set_attn_cm1(False)  # the batched verify's attention: the scalar kernel's arithmetic
    V, P, B, k = gt.dims.n_vocab, 16384, 8, 6
    rng = np.random.default_rng(6)
    gtk, gdk, otk, odk = [], [], [], []
    for b in range(B):
        g, o = engine.allocate_kv_cache(gt, P + 32), O.KvCache(ot, P + 32)
        _seed_kv(g, o, gt.dims, P, rng)
        gtk.append(g)
        otk.append(o)
        g, o = engine.allocate_kv_cache(gd, P + 32), O.KvCache(od, P + 32)
        _seed_kv(g, o, gd.dims, P, rng)
        gdk.append(g)
        odk.append(o)
    last = [int(t) for t in S.tokens(800, B, V)]
    for step in range(3):
        print(f"configs[4] batched spec step {step}", flush=True)
        em, dr = engine.spec_step_batch(gt, gd, gtk, gdk, last, k)
        for b in range(B):
            o_em, o_dr = O.spec_step_greedy(ot, od, otk[b], odk[b], last[b], k)
            assert dr[b] == o_dr, (step, b, dr[b], o_dr)
            assert em[b] == o_em, (step, b, em[b], o_em)
            assert gtk[b].position == otk[b].position == gdk[b].position + len(em[b]) // (k + 1)
        last = [e[-1] for e in em]
    for x in gtk + gdk + otk + odk + [gt, gd, ot, od]:
        x.close()
    timg.close()
    dimg.close()
