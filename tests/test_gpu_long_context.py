"""GPU parity against the C oracle at a context where the attention splits
spill past one 16-split merge chunk: 2100 cached keys + the chunk = 17 splits
of 128 keys. One and two columns take the attention merge built into the Wo
GEMV's operand (the 17th split loaded with the first 16); five and eight
columns take the two-row-group attention kernel and the separate combine (two
chunks' loads at once). Logits through forward_full, greedy ids through the
graph-replayed verify (whose split grid covers the cache capacity, so the
splits past the live keys exit early).

Tolerances as in test_gpu_forward: logits within 2e-2 absolute or 1e-2
relative and 3e-4 x max|logit|; greedy ids identical.
"""
import numpy as np
import pytest

import oracle as O
from parity import ids_agree, logits_close
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
    om.set_mm16(2 if gm.wide_f16 else 0)  # wide calls: the reference's f16 GEMM arithmetic
    V = gm.dims.n_vocab
    gkv = engine.allocate_kv_cache(gm, 2304)
    okv = O.KvCache(om, 2304)
    prompt = S.tokens(31, P, V)
    print(f"prefill {P}", flush=True)
    engine.forward_full_readback(gm, gkv, prompt, 0, full_logits=False)
    O.forward(om, okv, prompt, 0, logits_mode=0)
    for n in (1, 2, 5, 8):
        toks = S.tokens(40 + n, n, V)
        print(f"verify {n} columns at {P}", flush=True)
        gl, _ = engine.forward_full_readback(gm, gkv, toks, P)
        ol, _ = O.forward(om, okv, toks, P)
        close(gl, ol, gm.wide_f16)
        gkv.truncate(P)
        ids = engine.verify_greedy(gm, gkv, toks, P)
        if gm.wide_f16:  # prefill >= 32 columns: near-ties of the oracle allowed
            bad = np.where(ids != ol.argmax(axis=1))[0]
            assert all(ol[i].max() - ol[i, ids[i]] <= 3e-3 * np.abs(ol).max() for i in bad), (ids, ol.argmax(axis=1))
        else:
            assert np.array_equal(ids, ol.argmax(axis=1)), (ids, ol.argmax(axis=1))
        gkv.truncate(P)
        okv.truncate(P)
    gkv.close()
    okv.close()
    gm.close()
    om.close()
    img.close()
