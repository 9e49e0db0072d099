"""GPU parity against the C oracle on the draft's layer shape (Llama-3.2-1B:
d 2048, 32 heads of 64, 8 kv heads, FFN 8192) at one and two columns, the
draft's own chunk sizes. There the QKV and gate/up GEMVs build their operand
from the residual and the previous GEMV's split partials themselves; the down
GEMV (K = 8192) leaves 16 K-split partials, so the second layer's QKV adds
more than one batch of 8. Two layers, 48 cached tokens, logits and greedy ids.
"""
import numpy as np
import pytest

import oracle as O
from parity import ids_agree, logits_close, pair, record
from seeker_amd import synth as S
from seeker_amd._native import GGML_Q4_K

pytestmark = pytest.mark.gpu

SHAPE = S.LlamaShape(2, 2048, 32, 8, 8192, 4000, 512, 1e-5, 5e5, 0.02, GGML_Q4_K, GGML_Q4_K)


def close(a, b, wide=False):
    logits_close(a, b, wide)  # after a wide prefill: the bounds of tests/parity.py


def test_draft_shape_one_and_two_columns(engine):
    img = S.GgufImage(SHAPE, seed=22)
    gm = engine.upload_weights(img)
    om = O.Model(img)
    wide = pair(om, gm)  # the reference's wide-GEMM and cm1 attention arithmetic where the GPU uses them
    V = gm.dims.n_vocab
    gkv = engine.allocate_kv_cache(gm, 128)
    okv = O.KvCache(om, 128)
    prompt = S.tokens(32, 48, V)
    engine.forward_full_readback(gm, gkv, prompt, 0, full_logits=False)
    O.forward(om, okv, prompt, 0, logits_mode=0)
    for n in (1, 2):
        toks = S.tokens(50 + n, n, V)
        print(f"draft shape: verify {n} columns", flush=True)
        gl, _ = engine.forward_full_readback(gm, gkv, toks, 48)
        ol, _ = O.forward(om, okv, toks, 48)
        close(gl, ol, wide)
        gkv.truncate(48)
        ids = engine.verify_greedy(gm, gkv, toks, 48)
        if wide:  # f16 roundings in the prefill: near-ties of the oracle allowed
            bad = np.where(ids != ol.argmax(axis=1))[0]
            assert all(ol[i].max() - ol[i, ids[i]] <= 3e-3 * np.abs(ol).max() for i in bad), (ids, ol.argmax(axis=1))
            record("wide_ids", len(ids), len(bad))
        else:
            assert np.array_equal(ids, ol.argmax(axis=1)), (ids, ol.argmax(axis=1))
        gkv.truncate(48)
        okv.truncate(48)
    gkv.close()
    okv.close()
    gm.close()
    om.close()
    img.close()
