"""Helper for test_gpu_fusion.py, run as a subprocess (the fusion switch
SH_FUSE is read once per process): writes the logits of 1, 2, 5 and 8-column
verify forwards of two small Q4_K models after a 48-token prefill to argv[1]."""
import os
import sys

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
from seeker_amd import Engine  # noqa: E402
from seeker_amd import synth as S  # noqa: E402
from seeker_amd._native import GGML_Q4_K  # noqa: E402

# GQA shape; one layer of the 8B FFN width (gate/up on the deep-ring kernel)
SHAPES = {
    "gqa": S.LlamaShape(2, 1024, 8, 2, 2048, 4000, 512, 1e-5, 5e5, 0.02, GGML_Q4_K, GGML_Q4_K),
    "ffn": S.LlamaShape(1, 2048, 16, 4, 14336, 4000, 512, 1e-5, 5e5, 0.02, GGML_Q4_K, GGML_Q4_K),
}

out = {}
with Engine(0) as eng:
    for name, shape in SHAPES.items():
        img = S.GgufImage(shape, seed=3)
        m = eng.upload_weights(img)
        V = m.dims.n_vocab
        kv = eng.allocate_kv_cache(m, 256)
        eng.prefill(m, kv, S.tokens(5, 48, V), 0)
        for n in (1, 2, 5, 8):
            lg, _ = eng.forward_full_readback(m, kv, S.tokens(40 + n, n, V), 48, full_logits=True)
            out[f"{name}{n}"] = lg
            kv.truncate(48)
        kv.close()
        m.close()
        img.close()
np.savez(sys.argv[1], **out)
print("saved", sys.argv[1], flush=True)
