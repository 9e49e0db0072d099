"""GPU parity against the C oracle at a context where the attention splits
spill past one 16-split merge chunk: 2100 cached keys + the chunk = 17 splits
of 128 keys. One column (and two, with the cm1 attention off) take the
attention merge built into the Wo GEMV's operand (the 17th split loaded with
the first 16); five and eight columns with it off take the two-row-group
attention kernel and the separate combine (two chunks' loads at once). With
it on (the default), calls of two or more columns take the cm1 attention
over 34 64-key blocks: 9 splits of the look-back kernel and the f16 chain. Logits through forward_full, greedy ids through the
graph-replayed verify (whose split grid covers the cache capacity, so the
splits past the live keys exit early).

Tolerances as in test_gpu_forward: logits within 2e-2 absolute or 1e-2
relative and 3e-4 x max|logit|; greedy ids identical.
"""
import numpy as np
import pytest

import oracle as O
from parity import ids_agree, logits_close, pair, record
from seeker_amd import synth as S
from seeker_amd._native import GGML_Q4_K

pytestmark = pytest.mark.gpu

SHAPE = S.LlamaShape(1, 512, 8, 2, 1024, 4000, 4096, 1e-5, 5e5, 0.02, GGML_Q4_K, GGML_Q4_K)
P = 2100


def close(a, b, wide=False):
    logits_close(a, b, wide)  # after a wide prefill: the bounds of tests/parity.py


def test_seventeen_attention_splits(engine):
    img = S.GgufImage(SHAPE, seed=21)
    gm = engine.upload_weights(img)
    om = O.Model(img)
    wide = pair(om, gm)  # the reference's wide-GEMM and cm1 attention arithmetic where the GPU uses them
    V = gm.dims.n_vocab
    gkv = engine.allocate_kv_cache(gm, 2304)
    okv = O.KvCache(om, 2304)
    prompt = S.tokens(31, P, V)
    print(f"prefill {P}", flush=True)
    engine.forward_full_readback(gm, gkv, prompt, 0, full_logits=False)
    O.forward(om, okv, prompt, 0, logits_mode=0)
    # with cm1 attention (the reference's, the default) and without it (the
    # f32-level split kernels and their 17-split combines)
    for cm1, n in [(True, 1), (True, 2), (True, 5), (True, 8), (False, 2), (False, 5), (False, 8)]:
        gm.cm1_attention = cm1
        om.set_attn_cm1(cm1)
        toks = S.tokens(40 + n, n, V)
        print(f"verify {n} columns at {P} (cm1 {cm1})", flush=True)
        gl, _ = engine.forward_full_readback(gm, gkv, toks, P)
        ol, _ = O.forward(om, okv, toks, P)
        close(gl, ol, wide)
        gkv.truncate(P)
        ids = engine.verify_greedy(gm, gkv, toks, P)
        if wide:  # f16 roundings in the prefill: near-ties of the oracle allowed
            bad = np.where(ids != ol.argmax(axis=1))[0]
            assert all(ol[i].max() - ol[i, ids[i]] <= 3e-3 * np.abs(ol).max() for i in bad), (ids, ol.argmax(axis=1))
            record("wide_ids", len(ids), len(bad))
        else:
            assert np.array_equal(ids, ol.argmax(axis=1)), (ids, ol.argmax(axis=1))
        gkv.truncate(P)
        okv.truncate(P)
    gkv.close()
    okv.close()
    gm.close()
    om.close()
    img.close()
