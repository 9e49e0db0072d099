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
from seeker_amd import synth as S

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def models(engine):
    ti = S.GgufImage(S.TINY_TARGET, seed=0)
    di = S.GgufImage(S.TINY_DRAFT, seed=1)
    gt, gd = engine.upload_weights(ti), engine.upload_weights(di)
    ot, od = O.Model(ti), O.Model(di)
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


def test_spec_decode_lossless_vs_plain_greedy(engine, models):
    gt, gd, ot, od = models
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
