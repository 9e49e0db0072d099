"""HIP-graph replay of the speculative step and of the draft loop.

sh_spec_step (every sampling mode) and sh_draft_tokens record one HIP graph per
shape and replay it on later calls, as the reference records a step as one
submit and patches its per-step values (inference/mod.rs:2181-2231,
decode_dyn.rs:25-204). Positions, the Philox key and the uniform-word base are
device words written before each replay.

Checks: a replayed step equals the eager step of the same state bit for bit
(emitted tokens, drafts, and for the stochastic modes both sides' logits); the
replay counters show that the replayed side ran graphs and the eager side
(hipEvent profiling, which launches kernel by kernel) did not; the replayed
drafts of the qwen3 draft model (multi-group path) equal the oracle's greedy
drafts."""
import numpy as np
import pytest

import oracle as O
from parity import pair
from seeker_amd import synth as S
from seeker_amd._native import GGML_Q4_K, sh_sampling

pytestmark = pytest.mark.gpu

QWEN3 = S.LlamaShape(2, 512, 8, 4, 1024, 3000, 1024, 1e-6, 1e6, 0.02, GGML_Q4_K, GGML_Q4_K, True, arch=1,
                     head_dim=128, norm_jitter=0.2)
QWEN3MOE = S.LlamaShape(2, 512, 8, 2, 0, 3000, 1024, 1e-6, 1e6, 0.03, GGML_Q4_K, GGML_Q4_K, False, arch=2,
                        head_dim=128, n_expert=32, n_expert_used=4, expert_ff=512, norm_jitter=0.2,
                        router_std=512 ** -0.5)


def _models(engine, tshape, dshape, tseed, dseed):
    ti, di = S.GgufImage(tshape, seed=tseed), S.GgufImage(dshape, seed=dseed)
    gt, gd = engine.upload_weights(ti), engine.upload_weights(di)
    return ti, di, gt, gd


def _prefilled(engine, gt, gd, prompt, cap=512):
    tkv, dkv = engine.allocate_kv_cache(gt, cap), engine.allocate_kv_cache(gd, cap)
    lg, _ = engine.forward_full_readback(gt, tkv, prompt, 0, full_logits=False, want_residual=False)
    engine.prefill(gd, dkv, prompt, 0)
    return tkv, dkv, int(lg[0].argmax())


def _run_steps(engine, gt, gd, tkv, dkv, last, k, mode, n_steps, eager):
    """n_steps spec steps; eager: with per-launch profiling (no graphs).
    Returns per step (emitted, drafts, logits or None) and the replay-counter
    deltas."""
    s = None
    if mode:
        s = sh_sampling()
        s.mode, s.temperature, s.seed, s.counter = mode, 0.8, 99, 0
    engine.set_profiling(eager)
    c0, l0 = engine.graph_stats()
    out = []
    try:
        for _ in range(n_steps):
            r = engine.decode_speculative(gt, gd, tkv, dkv, last, k, s)
            lg = engine.spec_step_logits() if mode else None
            out.append((r.emitted, r.drafts, lg, tkv.position, dkv.position))
            last = r.emitted[-1]
    finally:
        engine.set_profiling(False)
        engine.profile(reset=True)
    c1, l1 = engine.graph_stats()
    return out, c1 - c0, l1 - l0


def _replay_equals_eager(engine, gt, gd, mode, k, n_steps, prompt_seed):
    V = gt.dims.n_vocab
    prompt = S.tokens(prompt_seed, 40, V)
    tA, dA, last = _prefilled(engine, gt, gd, prompt)
    tB, dB, lastB = _prefilled(engine, gt, gd, prompt)
    assert last == lastB
    eager, ce, le = _run_steps(engine, gt, gd, tA, dA, last, k, mode, n_steps, eager=True)
    replay, cr, lr = _run_steps(engine, gt, gd, tB, dB, last, k, mode, n_steps, eager=False)
    assert (ce, le) == (0, 0)
    assert lr == n_steps and cr >= 1
    for i, (a, b) in enumerate(zip(eager, replay)):
        assert a[0] == b[0] and a[1] == b[1], (i, a[:2], b[:2])
        assert a[3:] == b[3:], i
        if mode:
            for x, y in zip(a[2], b[2]):
                assert np.array_equal(x, y), i
    for x in (tA, dA, tB, dB):
        x.close()
    return replay


@pytest.mark.parametrize("mode", [0, 1, 2], ids=["greedy", "compare", "rejection"])
def test_llama_spec_step_replay_equals_eager(engine, mode):
    print(f"llama spec step replay vs eager, mode {mode}", flush=True)
    ti, di, gt, gd = _models(engine, S.TINY_TARGET, S.TINY_DRAFT, 0, 1)
    _replay_equals_eager(engine, gt, gd, mode, 4, 5, 314)
    for x in (gt, gd, ti, di):
        x.close()


@pytest.mark.parametrize("mode", [0, 2], ids=["greedy", "rejection"])
def test_qwen3_spec_step_replay_equals_eager(engine, mode):
    """The configs[4] pairing at small shapes: qwen3 draft and qwen3moe target
    both on the multi-group path (per-head RMSNorm, NEOX RoPE, routed
    experts), replayed."""
    print(f"qwen3 / qwen3moe spec step replay vs eager, mode {mode}", flush=True)
    ti, di, gt, gd = _models(engine, QWEN3MOE, QWEN3, 7, 8)
    _replay_equals_eager(engine, gt, gd, mode, 5, 4, 2718)
    for x in (gt, gd, ti, di):
        x.close()


@pytest.mark.parametrize("shape", ["tiny_draft", "qwen3"])
def test_draft_tokens_replayed_match_oracle(engine, shape):
    """sh_draft_tokens replays its graph from the second call on; its greedy
    drafts equal the oracle's single-token forwards, and the cache ends where
    the oracle's does."""
    print(f"draft_tokens replay, {shape}", flush=True)
    img = S.GgufImage(S.TINY_DRAFT if shape == "tiny_draft" else QWEN3, seed=11)
    gm = engine.upload_weights(img)
    om = O.Model(img)
    pair(om, gm)
    V = gm.dims.n_vocab
    prompt = S.tokens(5, 30, V)
    gkv, okv = engine.allocate_kv_cache(gm, 256), O.KvCache(om, 256)
    lg, _ = engine.forward_full_readback(gm, gkv, prompt, 0, full_logits=False, want_residual=False)
    O.forward(om, okv, prompt, 0, logits_mode=0)
    last = int(lg[0].argmax())
    c0, l0 = engine.graph_stats()
    for call in range(4):
        n = 6
        dr = engine.draft_tokens(gm, gkv, last, n)
        want = []
        tok = last
        for i in range(n):
            ol, _ = O.forward(om, okv, [tok], okv.position, logits_mode=1)
            tok = O.argmax(ol[0])
            want.append(tok)
        assert dr == want, (call, dr, want)
        assert gkv.position == okv.position  # last, d_1 .. d_{n-1} fed; d_n not
        # keep last and the first 3 drafts (the rest rejected), continue from d_4
        keep = okv.position - n + 4
        gkv.truncate(keep)
        okv.truncate(keep)
        last = dr[3]
    c1, l1 = engine.graph_stats()
    assert l1 - l0 == 4 and c1 - c0 >= 1
    for x in (gkv, okv, gm, om):
        x.close()
    img.close()


@pytest.mark.parametrize("replay", [False, True], ids=["eager", "replay"])
def test_draft_tokens_with_pending_match_oracle(engine, replay):
    """After a fully accepted spec step (draft = target) the draft cache holds
    d_n as a pending token: sh_draft_tokens feeds [d_n, last] as one catch-up
    forward (its last column's logits give d_1), then single tokens. The
    drafts equal the oracle's forwards of the same token chunks."""
    print(f"draft_tokens with a pending token, replay={replay}", flush=True)
    img = S.GgufImage(S.TINY_DRAFT, seed=12)
    gm = engine.upload_weights(img)
    om = O.Model(img)
    pair(om, gm)
    V = gm.dims.n_vocab
    prompt = S.tokens(6, 30, V)
    tkv, dkv = engine.allocate_kv_cache(gm, 256), engine.allocate_kv_cache(gm, 256)
    lg, _ = engine.forward_full_readback(gm, tkv, prompt, 0, full_logits=False, want_residual=False)
    engine.prefill(gm, dkv, prompt, 0)
    okv = O.KvCache(om, 256)
    O.forward(om, okv, prompt, 0, logits_mode=0)
    last = int(lg[0].argmax())
    engine.set_profiling(not replay)
    try:
        r = engine.decode_speculative(gm, gm, tkv, dkv, last, 4)
        assert len(r.emitted) == 5  # all 4 drafts accepted
        assert dkv.position == len(prompt) + 4  # last, d_1..d_3 fed; d_4 pending
        # the oracle's draft cache: the step's draft forwards (last, then d_1..d_3)
        for t in [last] + r.drafts[:3]:
            O.forward(om, okv, [t], okv.position, logits_mode=0)
        c0, l0 = engine.graph_stats()
        dr = engine.draft_tokens(gm, dkv, r.emitted[-1], 5)
        c1, l1 = engine.graph_stats()
    finally:
        engine.set_profiling(False)
        engine.profile(reset=True)
    assert (l1 - l0) == (1 if replay else 0)
    ol, _ = O.forward(om, okv, [r.drafts[3], r.emitted[-1]], okv.position, logits_mode=1)
    want = [O.argmax(ol[0])]
    for _ in range(4):
        ol, _ = O.forward(om, okv, [want[-1]], okv.position, logits_mode=1)
        want.append(O.argmax(ol[0]))
    assert dr == want
    assert dkv.position == okv.position
    for x in (tkv, dkv, okv, gm, om):
        x.close()
    img.close()


def test_forced_drafts_replay_the_greedy_continuation(engine):
    """sh_spec_step_forced with the target's greedy continuation as drafts
    accepts every draft; the emitted stream is that continuation and the
    steps replay graphs (one shape with no pending token, one with)."""
    print("forced-acceptance steps", flush=True)
    ti, di, gt, gd = _models(engine, S.TINY_TARGET, S.TINY_DRAFT, 0, 1)
    V, k = gt.dims.n_vocab, 5
    prompt = S.tokens(77, 40, V)
    # the continuation: single-token greedy forwards of the target
    ckv = engine.allocate_kv_cache(gt, 512)
    lg, _ = engine.forward_full_readback(gt, ckv, prompt, 0, full_logits=False, want_residual=False)
    cont = [int(lg[0].argmax())]
    for i in range(6 * (k + 1) + k):
        cont.append(int(engine.verify_greedy(gt, ckv, [cont[-1]], len(prompt) + i)[0]))
    ckv.close()
    tkv, dkv, last = _prefilled(engine, gt, gd, prompt)
    assert last == cont[0]
    c0, l0 = engine.graph_stats()
    j = 0
    for step in range(6):
        r = engine.decode_speculative_forced(gt, gd, tkv, dkv, cont[j], cont[j + 1:j + 1 + k])
        assert r.emitted == cont[j + 1:j + 2 + k], step
        j += len(r.emitted)
        assert tkv.position == len(prompt) + j
    c1, l1 = engine.graph_stats()
    assert l1 - l0 == 6 and c1 - c0 >= 1
    for x in (tkv, dkv, gt, gd, ti, di):
        x.close()
