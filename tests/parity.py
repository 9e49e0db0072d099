"""Tolerances shared by the GPU-vs-oracle tests.

Narrow forward calls (fewer than 32 columns, or a model without the wide f16
path) keep f32-level operands: logits agree with the oracle's f64 sums to
~1e-5 of their scale, bound 3e-4 x max|logit|.

Wide calls (>= 32 columns on a model with sh_model_wide_f16 on) round every
matmul operand to f16 as the reference's wide GEMM does (ops/matmul.rs:433-446,
mul_mm_cm.slang); the oracle in mode 2 rounds the same operands but sums in
f64, so where the GPU's f32 sum of a row differs from the f64 one in the last
bits, the next matmul's f16 rounding of it can flip by one f16 ulp (2^-11
relative). Those flips leave 5e-4 .. 7e-4 x max|logit| between the two on the
2-layer test models (the same outputs sit 1e-3 .. 1.6e-3 x max from the exact
oracle): bound 1.5e-3 x max, inside the north star's 2e-2 abs / 1e-2 rel.
A test whose caches were filled by a wide call keeps the wide bound for later
narrow calls, which read those K/V rows.

Causal calls of more than one column compute attention with the reference's
cooperative-matrix flash attention arithmetic (flash_attn_cm1.slang via
ops/flash_attn.rs:442-471: f16 staged q, f16 P, f16 P V accumulators and
output) when the model's switch is on (the default), and the oracle follows
with set_attn_cm1: there too an f32-level difference of a score can flip one
f16 rounding, so such calls, and later calls that read the K/V they shaped,
take the wide bounds (pair() returns whether they apply).

Greedy ids: equal, except a column whose oracle top-2 margin is smaller than
twice the largest logit difference seen (a near-tie of the oracle itself).
"""
import os

import numpy as np

# Every near-tie exemption the tests take, for the session summary that
# conftest.py writes when SH_PARITY_LOG names a file: per test, the columns
# compared and those whose greedy id differs (each at a near-tie), and any
# other counted exemption (record()).
EXEMPTIONS = []


def record(kind, compared, differing):
    EXEMPTIONS.append({"test": os.environ.get("PYTEST_CURRENT_TEST", "").split(" ")[0], "kind": kind,
                       "compared": int(compared), "differing": int(differing)})

NARROW_REL = 3e-4
WIDE_REL = 1.5e-3


def logits_close(a, b, wide=False):
    """North-star bound plus the path's tighter bound; returns max|a - b|."""
    err = np.abs(a - b)
    assert np.all(err <= np.maximum(2e-2, 1e-2 * np.abs(b))), float(err.max())
    bound = (WIDE_REL if wide else NARROW_REL) * np.abs(b).max()
    assert err.max() <= bound, (float(err.max()), float(np.abs(b).max()), wide)
    return float(err.max())


def ids_agree(gpu, ref, wide=False, err=None):
    """argmax ids equal up to near-ties of ref; returns the number of columns
    that differ (each at a near-tie)."""
    ga, ra = gpu.argmax(axis=1), ref.argmax(axis=1)
    bad = np.where(ga != ra)[0]
    if err is None:
        err = float(np.abs(gpu - ref).max())
    tie = 2.0 * err if wide else 1e-4
    rows = np.arange(ref.shape[0])
    margin = ref[rows, ra] - ref[rows, ga]
    assert all(margin[i] <= tie for i in bad), (bad, margin[bad], tie)
    # f16 operands widen the near-tie band, so wide calls may flip twice as many
    limit = max(2, ref.shape[0] // 25) if wide else max(1, ref.shape[0] // 50)
    assert len(bad) <= limit, (len(bad), ref.shape[0])
    record("wide_ids" if wide else "narrow_ids", ref.shape[0], len(bad))
    return int(len(bad))


def kv_layer0_ok(g, o, wide=False):
    """Layer-0 f16 cache entries from the same inputs: one ulp where the f32
    value sits on an f16 rounding boundary, or a small fraction of the layer's
    scale near zero (1e-6 narrow; 2e-4 wide, where each input whose f16
    rounding flips moves a projection by |w| x one f16 ulp of the input:
    measured up to 6e-4 of the scale, 1-2 ulps of the largest entries)."""
    floor = (2e-4 if wide else 1e-6) * np.abs(o).max()
    return bool(np.all(np.abs(g - o) <= np.abs(o) * 2.0 ** -10 + floor))


def pair(om, gm):
    """Give the oracle model om the arithmetic of the GPU model gm: the wide
    GEMM's f16 operands for calls of >= 32 columns (mode 2) and the cm1
    attention for causal calls of more than one column. Returns whether the
    wide bounds apply to calls after a multi-column call (f16 roundings in
    play)."""
    om.set_mm16(2 if gm.wide_f16 else 0)
    om.set_attn_cm1(gm.cm1_attention)
    return bool(gm.wide_f16 or gm.cm1_attention)
