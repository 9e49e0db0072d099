"""CPU tests that pin the C oracle before it is trusted as the parity reference.

What pins each oracle function (the reference ships no golden vectors for this
path; its only checks are closed-form inputs + CPU restatements):

  or_f16_to_f32 / or_f32_to_f16  exhaustive / randomized vs numpy float16 (IEEE RNE)
  or_philox4x64_10 / word         numpy.random.Philox raw words (tests/golden fixture)
  or_dequant_row (Q8_0, Q4_K)     independent numpy dequant (tests/ref_numpy.py) +
                                  closed-form special blocks (d=0, sc=1 m=0, q=15)
  or_gemv                         numpy f64 matmul of independently dequantized rows
  or_gemv16 / or_forward mm16     numpy f16 casts of the same rows and inputs; the
                                  mm16 numpy Llama (ref_numpy.RefLlama(mm16=True))
  or_attn_cm1 / forward cm1       closed forms on exactly representable rows (block
                                  rescale, f16 chunk and output accumulators, the
                                  f16 rescale factor), staging by numpy's roundings,
                                  the numpy cm1 Llama (RefLlama(cm1=True))
  or_forward                      independent numpy f64 Llama (ref_numpy.RefLlama),
                                  causal == incremental decode, chain tree == causal,
                                  branch == its own path
  or_argmax / or_softmax          closed forms (ties, NaN, all-masked uniform)
  or_sample_one / vocab order     explicit-uniform inverse CDF on hand-made rows, chi^2
  or_sample_and_compare           hand-made accept / reject patterns
  or_rejection                    q == p always accepts; point-mass q gives accept
                                  rate p(d) and residual p with d removed; chi^2 ~ p
  or_spec_step_greedy             lossless: spec output == plain greedy decode
  or_spec_step (all modes)        GREEDY == or_spec_step_greedy; REJECTION with draft ==
                                  target accepts every draft; chi^2: the first emitted
                                  token of COMPARE and REJECTION steps ~ p (planted
                                  always-accept or reversed-residual mistakes fail it)
"""
import json
import os

import numpy as np
import pytest

import oracle as O
import ref_numpy as R
from seeker_amd import synth as S
from seeker_amd._native import GGML_Q4_K, GGML_Q8_0

HERE = os.path.dirname(os.path.abspath(__file__))


# ------------------------------------------------------------------ f16

def test_f16_to_f32_exhaustive():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([O.lib().or_f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(got[finite], ref[finite])
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(np.isinf(got), np.isinf(ref))


def test_f32_to_f16_rne():
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 20000),
        np.array([0.0, -0.0, 65504, 65519.99, 65520, -65520, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8, 1e-9,
                  np.float32(1 + 2 ** -11), np.float32(1 + 3 * 2 ** -11)], dtype=np.float32),
    ]).astype(np.float32)
    ref = vals.astype(np.float16).view(np.uint16)
    got = np.array([O.lib().or_f32_to_f16(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, ref)


# ------------------------------------------------------------------ philox

def test_philox_numpy_golden():
    g = json.load(open(os.path.join(HERE, "golden", "philox4x64_numpy.json")))
    for case in g["cases"]:
        words = [int(w, 16) for w in case["words"]]
        c0 = case["counter"]
        for i, w in enumerate(words):
            blk = i // 4
            # numpy increments the 256-bit counter before each block
            ctr = list(c0)
            carry = blk + 1
            for j in range(4):
                s = ctr[j] + carry
                ctr[j] = s % (1 << 64)
                carry = s >> 64
            assert O.philox_block(ctr, case["key"])[i % 4] == w
        if case["counter"] == [0, 0, 0, 0]:
            for i, w in enumerate(words):
                assert O.lib().or_philox_word(case["key"][0], case["key"][1], i) == w


def test_unit_f32_range():
    L = O.lib()
    assert L.or_unit_f32(0) == 0.0
    assert L.or_unit_f32(0xFFFFFFFFFFFFFFFF) == np.float32(1 - 2 ** -24)


# ------------------------------------------------------------------ dequant

def _rand_q8(rng, rows, k):
    x = rng.standard_normal(rows * k).astype(np.float32) * 0.02
    return S.quantize(GGML_Q8_0, x), x


def _rand_q4k(rng, rows, k):
    x = rng.standard_normal(rows * k).astype(np.float32) * 0.02
    return S.quantize(GGML_Q4_K, x), x


@pytest.mark.parametrize("qtype", [GGML_Q8_0, GGML_Q4_K])
def test_dequant_matches_numpy(qtype):
    rng = np.random.default_rng(2)
    rows, k = 7, 512
    raw, _ = (_rand_q4k if qtype == GGML_Q4_K else _rand_q8)(rng, rows, k)
    ref = R.dequant(qtype, raw, rows, k)
    for r in range(rows):
        got = O.dequant_row(qtype, raw, r, k)
        np.testing.assert_allclose(got, ref[r], rtol=1e-6, atol=1e-9)


def test_dequant_q4k_special_blocks():
    blk = np.zeros(144, dtype=np.uint8)
    # d = 1.0, dmin = 0.5 (f16 bits), sc=1 / m=0 for sub-block 0, sc=3 / m=2 for sub-block 5
    blk[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blk[2:4] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    sc = [1, 0, 0, 0, 0, 3, 0, 0]
    m = [0, 0, 0, 0, 0, 2, 0, 0]
    for j in range(4):
        blk[4 + j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        blk[8 + j] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        blk[12 + j] = (sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4)
    q = np.arange(256) % 16
    for g in range(4):
        for l in range(32):
            blk[16 + 32 * g + l] = q[64 * g + l] | (q[64 * g + 32 + l] << 4)
    y = O.dequant_row(GGML_Q4_K, blk, 0, 256)
    np.testing.assert_array_equal(y[0:32], q[0:32].astype(np.float32))           # d*1*q - 0
    np.testing.assert_array_equal(y[160:192], (3.0 * q[160:192] - 1.0).astype(np.float32))  # 3q - 0.5*2
    np.testing.assert_array_equal(y[32:64], np.zeros(32, np.float32))             # sc = 0, m = 0
    blk[0:2] = 0  # d = 0 -> only the minimum term survives
    y = O.dequant_row(GGML_Q4_K, blk, 0, 256)
    np.testing.assert_array_equal(y[160:192], np.full(32, -1.0, np.float32))


def test_dequant_q8_special():
    blk = np.zeros(34, dtype=np.uint8)
    blk[0:2] = np.frombuffer(np.float16(0.25).tobytes(), np.uint8)
    blk[2:] = np.array([127, -127, -128, 0] * 8, dtype=np.int8).view(np.uint8)
    y = O.dequant_row(GGML_Q8_0, blk, 0, 32)
    np.testing.assert_array_equal(y[:4], np.array([31.75, -31.75, -32.0, 0.0], np.float32))


def test_quantizer_roundtrip_bounds():
    rng = np.random.default_rng(3)
    x = rng.standard_normal(4096).astype(np.float32) * 0.02
    for qt, tol in [(GGML_Q8_0, 0.02 * 4 / 127), (GGML_Q4_K, 0.02 * 8 / 15)]:
        raw = S.quantize(qt, x)
        y = R.dequant(qt, raw, 1, 4096)[0]
        assert np.max(np.abs(y - x)) < tol


def test_block_layout_sizes():
    # seeker-core/src/gguf/mod.rs:497-511 pins Q4_K = (256, 144); Q8_0 = (32, 34)
    assert S.quantize(GGML_Q4_K, np.zeros(512, np.float32)).size == 2 * 144
    assert S.quantize(GGML_Q8_0, np.zeros(64, np.float32)).size == 2 * 34


@pytest.mark.parametrize("qtype", [GGML_Q8_0, GGML_Q4_K])
def test_gemv_matches_numpy(qtype):
    rng = np.random.default_rng(4)
    M, K, N = 48, 512, 5
    raw, _ = (_rand_q4k if qtype == GGML_Q4_K else _rand_q8)(rng, M, K)
    x = rng.standard_normal((N, K)).astype(np.float32)
    y = O.gemv(qtype, raw, M, K, x)
    ref = x.astype(np.float64) @ R.dequant(qtype, raw, M, K).T
    np.testing.assert_allclose(y, ref, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("qtype", [GGML_Q8_0, GGML_Q4_K])
def test_gemv16_matches_numpy(qtype):
    """The wide-GEMM arithmetic: weights are the f32 dequantized values (exact
    in f64 here, then rounded once to f32) rounded to f16, inputs rounded to
    f16, as numpy's nearest-even casts give them; a mistake that skips either
    rounding moves y by ~1e-4 relative, far above the tolerance."""
    rng = np.random.default_rng(14)
    M, K, N = 40, 512, 3
    raw, _ = (_rand_q4k if qtype == GGML_Q4_K else _rand_q8)(rng, M, K)
    x = rng.standard_normal((N, K)).astype(np.float32)
    y = O.gemv16(qtype, raw, M, K, x)
    w16 = R.dequant(qtype, raw, M, K).astype(np.float32).astype(np.float16).astype(np.float64)
    ref = x.astype(np.float16).astype(np.float64) @ w16.T
    np.testing.assert_allclose(y, ref, rtol=1e-6, atol=1e-7)
    exact = O.gemv(qtype, raw, M, K, x)
    assert np.abs(exact - y).max() > 1e-5 * np.abs(exact).max()  # the roundings are there
    # f16 special cases of the inputs: overflow to inf, subnormals kept
    xs = np.zeros((1, K), np.float32)
    xs[0, 0], xs[0, 1] = 70000.0, 3e-6
    ys = O.gemv16(qtype, raw, M, K, xs)
    w0 = R.dequant(qtype, raw, M, K)[:, 1].astype(np.float32).astype(np.float16).astype(np.float64)
    w00 = R.dequant(qtype, raw, M, K)[:, 0]
    keep = w00 == 0
    np.testing.assert_allclose(ys[0][keep], (w0 * np.float64(np.float16(3e-6)))[keep], rtol=1e-12)
    assert np.all(np.isinf(ys[0][~keep]))


# ------------------------------------------------------------------ forward

SMALL_Q8 = S.LlamaShape(2, 256, 4, 2, 512, 1000, 256, 1e-5, 1e4, 0.02, GGML_Q8_0, GGML_Q8_0)
SMALL_Q4 = S.LlamaShape(2, 256, 4, 2, 512, 1000, 256, 1e-5, 5e5, 0.02, GGML_Q4_K, GGML_Q4_K)


@pytest.fixture(scope="module", params=[SMALL_Q8, SMALL_Q4], ids=["q8", "q4k"])
def small(request):
    img = S.GgufImage(request.param, seed=11)
    yield img
    img.close()


def test_gguf_image_layout(small):
    meta, T, start = R.read_gguf(bytes(small.bytes()))
    sh = small.shape
    assert meta["general.architecture"] == "llama"
    assert meta["llama.block_count"] == sh.n_layer and meta["llama.embedding_length"] == sh.n_embd
    assert start % 32 == 0
    for name in ["token_embd.weight", "output_norm.weight", "output.weight", "blk.0.attn_q.weight",
                 "blk.1.ffn_down.weight"]:
        assert name in T
    assert T["blk.0.attn_k.weight"][0] == [sh.n_embd, sh.n_embd // sh.n_head * sh.n_head_kv]
    assert T["blk.0.ffn_down.weight"][0] == [sh.n_ff, sh.n_embd]


def test_forward_matches_numpy(small):
    ref = R.RefLlama(bytes(small.bytes()))
    m = O.Model(small)
    kv = O.KvCache(m, 64)
    toks = S.tokens(5, 12, m.V)
    lg, res = O.forward(m, kv, toks, 0)
    rl, rr = ref.forward(toks)
    np.testing.assert_allclose(res, rr, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(lg, rl, rtol=1e-4, atol=1e-4 * np.abs(rl).max())
    # next chunk at position 12 (prefix visible, causal within chunk)
    t2 = S.tokens(6, 5, m.V)
    lg2, _ = O.forward(m, kv, t2, 12)
    rl2, _ = ref.forward(t2)
    np.testing.assert_allclose(lg2, rl2, rtol=1e-4, atol=1e-4 * np.abs(rl2).max())
    # KV cache contents: the same f16 values, up to one f16 ulp where the f32 value
    # sits on a rounding boundary (independent f32/f64 arithmetic)
    for li in range(m.n_layer):
        k = kv.layer(li, False, 17).astype(np.int32)
        r = ref.K[li].astype(np.float16).view(np.uint16).astype(np.int32)
        diff = np.abs(k - r)
        assert diff.max() <= 1 and np.mean(diff > 0) < 0.01
    kv.close()
    m.close()


def test_forward_mm16_matches_numpy(small):
    """or_forward with the wide-GEMM operands against the numpy Llama doing the
    same roundings, and away from the exact forward."""
    ref = R.RefLlama(bytes(small.bytes()), mm16=True)
    m = O.Model(small)
    m.set_mm16(True)
    kv = O.KvCache(m, 64)
    toks = S.tokens(5, 12, m.V)
    lg, res = O.forward(m, kv, toks, 0)
    rl, rr = ref.forward(toks)
    # both store the same f32 values at the same points, so they round the
    # same values to f16: equal up to f64 summation order
    np.testing.assert_allclose(res, rr, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(lg, rl, rtol=1e-6, atol=1e-6 * np.abs(rl).max())
    m.set_mm16(False)
    kv2 = O.KvCache(m, 64)
    lg0, _ = O.forward(m, kv2, toks, 0)
    assert np.abs(lg0 - lg).max() > 1e-4 * np.abs(lg0).max()
    kv.close()
    kv2.close()
    m.close()


def test_forward_mm16_auto_follows_call_width(small):
    """Mode 2 (the reference's dispatch, ops/matmul.rs:433-446): a forward call
    of >= 32 columns equals mode 1 exactly, one of fewer columns equals mode 0
    exactly (the width is the call's, so a later narrow call after a wide
    prefill is exact again)."""
    m = O.Model(small)
    out = {}
    for mode in (0, 1, 2):
        m.set_mm16(mode)
        kv = O.KvCache(m, 96)
        wide, _ = O.forward(m, kv, S.tokens(6, 40, m.V), 0)
        narrow, _ = O.forward(m, kv, S.tokens(7, 5, m.V), 40)
        out[mode] = (wide, narrow)
        kv.close()
    assert np.array_equal(out[2][0], out[1][0]) and not np.array_equal(out[2][0], out[0][0])
    # the narrow call reads the wide call's K/V: mode 2 matches mode 1's cache
    # and mode 0's matmuls, so it equals neither whole; rerun it from mode 1's
    # cache with exact matmuls
    m.set_mm16(1)
    kv = O.KvCache(m, 96)
    O.forward(m, kv, S.tokens(6, 40, m.V), 0)
    m.set_mm16(0)
    narrow0, _ = O.forward(m, kv, S.tokens(7, 5, m.V), 40)
    assert np.array_equal(out[2][1], narrow0)
    kv.close()
    m.close()


# ------------------------------------------------------- cm1 attention

def _f16(x):
    return np.asarray(x, np.float16).view(np.uint16)


def _cm1_keys(n, hd, s_of_key, v_of_key):
    """Staged q = e_0 (f16 1.0) and keys whose score is exactly s_of_key[t]
    (K[t][0] = s), values V[t][0] = v_of_key[t] (other d zero)."""
    q16 = _f16(np.eye(1, hd, 0, dtype=np.float32)[0])
    K = np.zeros((n, hd), np.float32)
    V = np.zeros((n, hd), np.float32)
    K[:, 0] = s_of_key
    V[:, 0] = v_of_key
    return q16, _f16(K), _f16(V)


def test_cm1_exact_on_representable_inputs():
    """Integer scores and small integer values keep every intermediate of the
    cm1 arithmetic exact (P = 2^(s - m), every f16 sum representable), so the
    row equals the closed form sum 2^(s_t - M) v_t / sum 2^(s_t - M) bit for
    bit, through four blocks (the last one partial) whose running maximum
    rises in block 2: a dropped or reversed rescale, a dropped chunk or key, or
    a wrong normalisation changes the result."""
    rng = np.random.default_rng(3)
    n, hd = 200, 64
    s = rng.integers(0, 3, n).astype(np.float32)
    s[140] = 4.0  # the maximum arrives in block 2
    v = rng.integers(-2, 3, n).astype(np.float32)
    q16, K, V = _cm1_keys(n, hd, s, v)
    out = O.attn_cm1(q16, K, V, staged=True)
    w = np.exp2(s.astype(np.float64) - 4.0)
    num, den = float(np.sum(w * v)), float(np.sum(w))
    assert out[0] == np.float32(num) * (np.float32(1.0) / np.float32(den))
    assert np.all(out[1:] == 0)
    # keys marked invisible drop out exactly (here: every key with s == 1)
    vis = s != 1
    out2 = O.attn_cm1(q16, K, V, visible=vis.astype(np.uint8), staged=True)
    num2, den2 = float(np.sum((w * v)[vis])), float(np.sum(w[vis]))
    assert out2[0] == np.float32(num2) * (np.float32(1.0) / np.float32(den2))


def test_cm1_f16_accumulators_round():
    """The P V chunk accumulator and the running output are f16 (the reference's
    f16-accumulating MMA and f16 output registers): with all scores 0 (P = 1),
    a block whose chunks add 2048 + 1 + 1 + 3 keeps 2052 (f16 spacing 2 above
    2048, ties to even), and 2048 followed by blocks adding 1 each stays 2048;
    an f32 accumulator would give 2053 and 2050."""
    hd = 64
    v = np.zeros(64, np.float32)
    v[0], v[16], v[32], v[48] = 2048, 1, 1, 3
    q16, K, V = _cm1_keys(64, hd, np.zeros(64, np.float32), v)
    out = O.attn_cm1(q16, K, V, staged=True)
    assert out[0] == np.float32(2052.0) * (np.float32(1.0) / np.float32(64.0))
    v = np.zeros(192, np.float32)
    v[0], v[64], v[128] = 2048, 1, 1
    q16, K, V = _cm1_keys(192, hd, np.zeros(192, np.float32), v)
    out = O.attn_cm1(q16, K, V, staged=True)
    assert out[0] == np.float32(2048.0) * (np.float32(1.0) / np.float32(192.0))


def test_cm1_rescale_factor_is_f16():
    """A running maximum that rises by 0.5 rescales the f16 output by
    f16(2^-0.5) = 0.70703125 (flash_attn_cm1.slang casts the factor to f16),
    not by 0.70710678."""
    hd = 64
    s = np.zeros(128, np.float32)
    s[64] = 0.5
    v = np.zeros(128, np.float32)
    v[0] = 1.0
    q16, K, V = _cm1_keys(128, hd, s, v)
    out = O.attn_cm1(q16, K, V, staged=True)
    e = np.float32(2.0 ** -0.5)
    L = 64.0 * float(e) + 1.0 + 63.0 * float(e)  # block 0 rescaled, block 1: one key at the max
    assert abs(float(out[0]) * L - 0.70703125) < 2e-7
    assert abs(float(out[0]) * L - 2.0 ** -0.5) > 5e-5


def test_cm1_staging_and_distance_from_exact():
    """or_attn_cm1 stages q as f16(q * f32(f32(1/sqrt(hd)) * f32(log2 e)))
    (numpy's own roundings here) and then equals or_attn_cm1_core; on random
    rows it sits within 1e-2 of the exact softmax attention of its relative
    scale, and away from it."""
    rng = np.random.default_rng(5)
    for hd, n in ((64, 70), (128, 300)):
        K = rng.normal(0, 1, (n, hd)).astype(np.float16)
        V = rng.normal(0, 1, (n, hd)).astype(np.float16)
        q = rng.normal(0, 0.5, hd).astype(np.float32)
        qs = np.float32(np.float32(1.0) / np.sqrt(np.float32(hd))) * np.float32(1.4426950408889634)
        q16 = (q * qs).astype(np.float16).view(np.uint16)
        a = O.attn_cm1(q, K.view(np.uint16), V.view(np.uint16))
        b = O.attn_cm1(q16, K.view(np.uint16), V.view(np.uint16), staged=True)
        assert np.array_equal(a, b)
        sc = K.astype(np.float64) @ q.astype(np.float64) / np.sqrt(hd)
        p = np.exp(sc - sc.max())
        ex = p @ V.astype(np.float64) / p.sum()
        d = np.abs(a - ex).max() / np.abs(ex).max()
        assert 1e-6 < d < 1e-2, d


def test_forward_cm1_matches_numpy(small):
    """or_forward with cm1 attention against the numpy Llama doing the same
    roundings (ref_numpy.attn_cm1), and away from the exact forward. The two
    sides store f32 values that differ in their last bits (and ~1 % of their
    f16 K/V entries by one ulp), and the f16 steps turn some of those into
    2^-11 flips: over 70 keys (two 64-key blocks) they agree to ~1.4e-4 of the
    logit scale while each sits 3-4e-4 from the exact forward. A one-column
    call and a tree call are unchanged by the switch."""
    ref = R.RefLlama(bytes(small.bytes()), cm1=True)
    m = O.Model(small)
    m.set_attn_cm1(True)
    kv = O.KvCache(m, 96)
    toks = S.tokens(5, 70, m.V)
    lg, res = O.forward(m, kv, toks, 0)
    rl, rr = ref.forward(toks)
    m.set_attn_cm1(False)
    kv0 = O.KvCache(m, 96)
    lg0, _ = O.forward(m, kv0, toks, 0)
    sc = np.abs(rl).max()
    err, dist = np.abs(lg - rl).max() / sc, np.abs(lg0 - lg).max() / sc
    assert err <= 2.5e-4 and dist >= 2.5e-4 and err <= 0.5 * dist, (err, dist)
    np.testing.assert_allclose(res, rr, rtol=1e-3, atol=5e-4 * np.abs(rr).max())
    # 12 keys (one block, no flips from the KV yet): much closer than to exact
    kv1, kv2 = O.KvCache(m, 96), O.KvCache(m, 96)
    ref1 = R.RefLlama(bytes(small.bytes()), cm1=True)
    m.set_attn_cm1(True)
    a, _ = O.forward(m, kv1, toks[:12], 0)
    b, _ = ref1.forward(toks[:12])
    m.set_attn_cm1(False)
    c, _ = O.forward(m, kv2, toks[:12], 0)
    assert np.abs(a - b).max() <= 0.1 * np.abs(a - c).max()
    kv1.close(); kv2.close()
    # one column / a tree: the exact softmax whatever the switch
    one = {}
    for on in (False, True):
        m.set_attn_cm1(on)
        kv0.set_position(70)
        one[on] = (O.forward(m, kv0, S.tokens(6, 1, m.V), 70)[0],
                   O.forward(m, kv0, S.tokens(7, 3, m.V), 71, parents=[-1, 0, 0])[0])
    assert np.array_equal(one[False][0], one[True][0]) and np.array_equal(one[False][1], one[True][1])
    kv.close(); kv0.close(); m.close()


def test_forward_incremental_equals_batch(small):
    m = O.Model(small)
    toks = S.tokens(7, 9, m.V)
    kv = O.KvCache(m, 64)
    full, _ = O.forward(m, kv, toks, 0)
    kv2 = O.KvCache(m, 64)
    O.forward(m, kv2, toks[:6], 0, logits_mode=0)
    for i in range(6, 9):
        lg, _ = O.forward(m, kv2, toks[i:i + 1], i, logits_mode=1)
        np.testing.assert_allclose(lg[0], full[i], rtol=1e-5, atol=1e-6)
    kv.close(); kv2.close(); m.close()


def test_tree_forward(small):
    m = O.Model(small)
    pre = S.tokens(8, 6, m.V)
    nodes = S.tokens(9, 6, m.V)
    parents = [-1, 0, 0, 1, 2, 2]   # root -> {1, 2}; 1 -> 3; 2 -> {4, 5}
    kv = O.KvCache(m, 64)
    O.forward(m, kv, pre, 0, logits_mode=0)
    tl, _ = O.forward(m, kv, nodes, 6, parents=parents)
    for leaf in [3, 4, 5]:
        path = []
        x = leaf
        while x >= 0:
            path.append(x)
            x = parents[x]
        path = path[::-1]
        kv2 = O.KvCache(m, 64)
        O.forward(m, kv2, pre, 0, logits_mode=0)
        cl, _ = O.forward(m, kv2, nodes[path], 6)
        for j, node in enumerate(path):
            np.testing.assert_allclose(tl[node], cl[j], rtol=1e-5, atol=1e-6)
        kv2.close()
    # chain-shaped tree == causal
    kv3 = O.KvCache(m, 64)
    O.forward(m, kv3, pre, 0, logits_mode=0)
    ch, _ = O.forward(m, kv3, nodes, 6, parents=[-1, 0, 1, 2, 3, 4])
    kv4 = O.KvCache(m, 64)
    O.forward(m, kv4, pre, 0, logits_mode=0)
    ca, _ = O.forward(m, kv4, nodes, 6)
    np.testing.assert_array_equal(ch, ca)
    for k in (kv, kv3, kv4):
        k.close()
    m.close()


def test_kv_compact_then_continue(small):
    """Compacting an accepted tree path then decoding == decoding the path causally."""
    m = O.Model(small)
    pre = S.tokens(10, 5, m.V)
    nodes = S.tokens(11, 4, m.V)
    parents = [-1, 0, 0, 2]
    kv = O.KvCache(m, 64)
    O.forward(m, kv, pre, 0, logits_mode=0)
    O.forward(m, kv, nodes, 5, parents=parents, logits_mode=0)
    kv.compact(5, [0, 2, 3])
    nxt = S.tokens(12, 1, m.V)
    a, _ = O.forward(m, kv, nxt, 8, logits_mode=1)
    kv2 = O.KvCache(m, 64)
    O.forward(m, kv2, np.concatenate([pre, nodes[[0, 2, 3]]]), 0, logits_mode=0)
    b, _ = O.forward(m, kv2, nxt, 8, logits_mode=1)
    np.testing.assert_allclose(a, b, rtol=1e-6, atol=1e-7)
    kv.close(); kv2.close(); m.close()


# ------------------------------------------------------------------ sampler

def test_argmax_ties_and_nan():
    assert O.argmax([1.0, 3.0, 3.0, 2.0]) == 1
    assert O.argmax([np.nan, 1.0, np.nan, 5.0]) == 3
    assert O.argmax([-np.inf, -np.inf]) == 0


def test_softmax_closed_forms():
    p = O.softmax([0.0, np.log(3.0)])
    np.testing.assert_allclose(p, [0.25, 0.75], rtol=1e-6)
    u = O.softmax([-np.inf, -np.inf, -np.inf, -np.inf])
    np.testing.assert_array_equal(u, np.full(4, 0.25, np.float32))


def test_sample_one_inverse_cdf():
    lg = np.log(np.array([0.1, 0.6, 0.3], dtype=np.float64)).astype(np.float32)
    cfg = O.SamplerCfg(1.0, 0, 1.0, 0.0)
    # sorted desc: ids [1, 2, 0] with probs [0.6, 0.3, 0.1]
    assert O.sample_one(lg, cfg, 0.0) == 1
    assert O.sample_one(lg, cfg, 0.59) == 1
    assert O.sample_one(lg, cfg, 0.61) == 2
    assert O.sample_one(lg, cfg, 0.95) == 0
    # vocab order: cumulative [0.1, 0.7, 1.0]
    assert O.sample_vocab_order(lg, 1.0, 0.05) == 0
    assert O.sample_vocab_order(lg, 1.0, 0.5) == 1
    assert O.sample_vocab_order(lg, 1.0, 0.75) == 2
    greedy = O.SamplerCfg(0.0, 0, 1.0, 0.0)
    assert O.sample_one(lg, greedy, 0.99) == 1
    topk1 = O.SamplerCfg(1.0, 1, 1.0, 0.0)
    assert O.sample_one(lg, topk1, 0.99) == 1


def test_sample_vocab_order_chi2():
    rng = np.random.default_rng(5)
    V, T = 12, 0.8
    lg = rng.standard_normal(V).astype(np.float32) * 2
    p = O.probs(lg, T).astype(np.float64)
    n = 6000
    us = rng.random(n).astype(np.float32)
    counts = np.bincount([O.sample_vocab_order(lg, T, float(u)) for u in us], minlength=V)
    chi2 = np.sum((counts - n * p) ** 2 / (n * p))
    assert chi2 < 40.0  # 11 dof, p ~ 1e-4


def test_sample_and_compare_patterns():
    V = 6
    rows = np.full((4, V), -5.0, np.float32)
    for i, t in enumerate([2, 4, 1, 3]):
        rows[i, t] = 5.0
    g = O.SamplerCfg(0.0, 0, 1.0, 0.0)
    assert O.sample_and_compare(rows, [2, 4, 1], g, np.zeros(4)) == [2, 4, 1, 3]   # all accepted + bonus
    assert O.sample_and_compare(rows, [2, 0, 1], g, np.zeros(4)) == [2, 4]         # reject at 1, correction
    assert O.sample_and_compare(rows, [5, 4, 1], g, np.zeros(4)) == [2]


def test_rejection_q_equals_p_always_accepts():
    rng = np.random.default_rng(6)
    k, V = 4, 50
    p = rng.standard_normal((k + 1, V)).astype(np.float32)
    q = p[:k].copy()
    drafts = rng.integers(0, V, k)
    for _ in range(20):
        acc, _ = O.rejection(p, q, drafts, 0.8, rng.random(k).astype(np.float32) * 0.999,
                             rng.random(k + 1).astype(np.float32))
        assert acc == k


def test_rejection_point_mass_q():
    rng = np.random.default_rng(7)
    V, T = 8, 1.0
    p = rng.standard_normal((2, V)).astype(np.float32)
    d = 3
    q = np.full((1, V), -1e30, np.float32)
    q[0, d] = 0.0
    pp = O.probs(p[0], T).astype(np.float64)
    n = 4000
    ua = rng.random(n).astype(np.float32)
    ur = rng.random(n).astype(np.float32)
    accepted = 0
    resid = np.zeros(V)
    for i in range(n):
        acc, tok = O.rejection(p, q, [d], T, ua[i:i + 1], np.array([ur[i], ur[i]], np.float32))
        if acc == 1:
            accepted += 1
        else:
            assert tok != d
            resid[tok] += 1
    assert abs(accepted / n - pp[d]) < 4 * np.sqrt(pp[d] * (1 - pp[d]) / n)
    expect = pp.copy()
    expect[d] = 0
    expect /= expect.sum()
    m = resid.sum()
    nz = expect > 0
    chi2 = np.sum((resid[nz] - m * expect[nz]) ** 2 / (m * expect[nz]))
    assert chi2 < 30.0


def test_rejection_output_distribution_is_p():
    rng = np.random.default_rng(8)
    V, T = 6, 1.0
    p = rng.standard_normal((2, V)).astype(np.float32)
    q = rng.standard_normal((1, V)).astype(np.float32)
    pp = O.probs(p[0], T).astype(np.float64)
    qq = O.probs(q[0], T).astype(np.float64)
    n = 6000
    cnt = np.zeros(V)
    for _ in range(n):
        d = rng.choice(V, p=qq / qq.sum())
        acc, tok = O.rejection(p, q, [d], T, rng.random(1).astype(np.float32), rng.random(2).astype(np.float32))
        cnt[d if acc == 1 else tok] += 1
    chi2 = np.sum((cnt - n * pp) ** 2 / (n * pp))
    assert chi2 < 30.0


# ------------------------------------------------------------------ tree acceptance

def _chain(k):
    return np.arange(-1, k, dtype=np.int32)  # node i's parent is i - 1


def test_tree_accept_chain_equals_rejection():
    """A chain-shaped tree is the single-draft case: with u_acc[i] = u[2(i+1)] and
    u_res[i] = u[2i+1] it must reproduce or_rejection token for token."""
    rng = np.random.default_rng(11)
    V, T = 40, 0.9
    for trial in range(200):
        k = int(rng.integers(1, 6))
        p = (rng.standard_normal((k + 1, V)) * 2).astype(np.float32)
        q = (p + rng.standard_normal((k + 1, V))).astype(np.float32)
        drafts = rng.integers(0, V, k).astype(np.uint32)
        u = rng.random((k + 1, 2)).astype(np.float32)
        acc, nt = O.rejection(p, q[:k], drafts, T, u[1:, 0].copy(), u[:, 1].copy())
        tokens = np.concatenate([[0], drafts]).astype(np.uint32)
        path, nt2 = O.tree_accept(p, q, tokens, _chain(k), T, u)
        assert path == list(range(acc + 1)) and nt2 == nt, (trial, acc, nt, path, nt2)


def test_tree_accept_greedy_walk():
    rng = np.random.default_rng(12)
    V = 7
    parents = np.array([-1, 0, 0, 0, 1, 1, 2, 4, 4], np.int32)
    n = parents.size
    for _ in range(300):
        p = rng.standard_normal((n, V)).astype(np.float32)
        tokens = rng.integers(0, V, n).astype(np.uint32)
        path, nt = O.tree_accept(p, p, tokens, parents, 0.0, np.zeros((n, 2), np.float32))
        v, want = 0, [0]
        while True:
            t = int(np.argmax(p[v]))
            kids = [c for c in range(v + 1, n) if parents[c] == v and tokens[c] == t]
            if not kids:
                break
            v = kids[0]
            want.append(v)
        assert path == want and nt == int(np.argmax(p[v]))


def test_tree_accept_q_equals_p_accepts_first_child():
    rng = np.random.default_rng(13)
    V, T = 30, 1.0
    parents = np.array([-1, 0, 0, 1, 1], np.int32)
    for _ in range(50):
        p = rng.standard_normal((5, V)).astype(np.float32)
        tokens = rng.integers(0, V, 5).astype(np.uint32)
        u = (rng.random((5, 2)) * 0.999).astype(np.float32)
        path, _ = O.tree_accept(p, p, tokens, parents, T, u)
        assert path[:3] == [0, 1, 3]


def test_tree_accept_first_token_distribution_is_p():
    """Losslessness: with m children drawn i.i.d. from q at the root, the first
    token after the root (accepted child or resampled) is distributed as p."""
    rng = np.random.default_rng(14)
    V, T, m = 6, 1.0, 3
    p = np.zeros((m + 1, V), np.float32)
    q = np.zeros((m + 1, V), np.float32)
    p[0] = rng.standard_normal(V)
    q[0] = rng.standard_normal(V)
    pp = O.probs(p[0], T).astype(np.float64)
    qq = O.probs(q[0], T).astype(np.float64)
    parents = np.array([-1] + [0] * m, np.int32)
    n = 8000
    cnt = np.zeros(V)
    for _ in range(n):
        kids = rng.choice(V, size=m, p=qq / qq.sum())
        tokens = np.concatenate([[0], kids]).astype(np.uint32)
        path, nt = O.tree_accept(p, q, tokens, parents, T, rng.random((m + 1, 2)).astype(np.float32))
        cnt[int(tokens[path[1]]) if len(path) > 1 else nt] += 1
    chi2 = np.sum((cnt - n * pp) ** 2 / (n * pp))
    assert chi2 < 30.0, (cnt / n, pp)


# ------------------------------------------------------------------ spec step

def test_spec_greedy_lossless():
    """scripts/validate_spec_b1.sh invariant: spec output == non-spec greedy output."""
    tshape = S.LlamaShape(2, 256, 4, 4, 512, 500, 256, 1e-5, 1e4, 0.02, GGML_Q8_0, GGML_Q8_0)
    dshape = S.LlamaShape(1, 256, 4, 4, 512, 500, 256, 1e-5, 1e4, 0.02, GGML_Q8_0, GGML_Q8_0)
    with S.GgufImage(tshape, 0) as ti, S.GgufImage(dshape, 1) as di:
        tm, dm = O.Model(ti), O.Model(di)
        prompt = S.tokens(1234, 16, tm.V)
        # plain greedy
        kv = O.KvCache(tm, 128)
        lg, _ = O.forward(tm, kv, prompt, 0, logits_mode=1)
        tok = O.argmax(lg[0])
        plain = [tok]
        for i in range(20):
            lg, _ = O.forward(tm, kv, [tok], 16 + i, logits_mode=1)
            tok = O.argmax(lg[0])
            plain.append(tok)
        # spec, draft = separate model, and forced acceptance (draft = target)
        for draft in (dm, tm):
            tkv, dkv = O.KvCache(tm, 128), O.KvCache(draft, 128)
            lg, _ = O.forward(tm, tkv, prompt, 0, logits_mode=1)
            O.forward(draft, dkv, prompt, 0, logits_mode=0)
            out = [O.argmax(lg[0])]
            steps = 0
            while len(out) < 21:
                em, _ = O.spec_step_greedy(tm, draft, tkv, dkv, out[-1], 4)
                out.extend(em)
                steps += 1
                assert tkv.position == 16 + len(out) - 1
            assert out[:21] == plain
            if draft is tm:
                assert steps <= 5  # 5 tokens per step when every draft is accepted
            tkv.close(); dkv.close()
        tm.close(); dm.close()


def _micro_models():
    """A 2-layer target and 1-layer draft small enough for many spec steps (V 64)."""
    tshape = S.LlamaShape(2, 128, 2, 2, 256, 64, 256, 1e-5, 1e4, 0.3, GGML_Q8_0, GGML_Q8_0)
    dshape = S.LlamaShape(1, 128, 2, 2, 256, 64, 256, 1e-5, 1e4, 0.3, GGML_Q8_0, GGML_Q8_0)
    return S.GgufImage(tshape, 5), S.GgufImage(dshape, 6)


def _prefill(tm, dm, prompt, cap=128):
    tkv, dkv = O.KvCache(tm, cap), O.KvCache(dm, cap)
    lg, _ = O.forward(tm, tkv, prompt, 0, logits_mode=1)
    O.forward(dm, dkv, prompt, 0, logits_mode=0)
    return tkv, dkv, O.argmax(lg[0])


def test_spec_step_greedy_mode_equals_greedy_step():
    """or_spec_step in GREEDY mode is or_spec_step_greedy, step for step."""
    ti, di = _micro_models()
    with ti, di:
        tm, dm = O.Model(ti), O.Model(di)
        prompt = S.tokens(77, 12, tm.V)
        a_t, a_d, last_a = _prefill(tm, dm, prompt)
        b_t, b_d, last_b = _prefill(tm, dm, prompt)
        for _ in range(12):
            ea, da = O.spec_step_greedy(tm, dm, a_t, a_d, last_a, 3)
            eb, db = O.spec_step(tm, dm, b_t, b_d, last_b, 3, O.SPEC_GREEDY)
            assert (ea, da) == (eb, db)
            assert a_t.position == b_t.position and a_d.position == b_d.position
            last_a, last_b = ea[-1], eb[-1]
        for x in (a_t, a_d, b_t, b_d, tm, dm):
            x.close()


def test_spec_step_rejection_q_equals_p_accepts_all():
    """Draft == target: q == p exactly, so every sampled draft is accepted and
    each REJECTION step emits n + 1 tokens; the drafts are the draws from q."""
    ti, _ = _micro_models()
    with ti:
        tm = O.Model(ti)
        prompt = S.tokens(78, 10, tm.V)
        tkv, dkv, last = _prefill(tm, tm, prompt)
        ctr = 0
        for step in range(8):
            u = O.spec_uniforms(3, ctr, 4)
            em, dr, p, q = O.spec_step(tm, tm, tkv, dkv, last, 4, O.SPEC_REJECTION, 0.7, u, want_logits=True)
            ctr += 3 * 4 + 2
            assert len(em) == 5 and em[:4] == dr
            assert np.array_equal(p[:4], q)
            for i in range(4):  # each draft is the vocab-order draw from q_i with its own uniform
                assert dr[i] == O.sample_vocab_order(q[i], 0.7, float(u[10 + i]))
            last = em[-1]
        for x in (tkv, dkv, tm):
            x.close()


@pytest.mark.parametrize("mode", [1, 2], ids=["compare", "rejection"])
def test_spec_step_first_token_distribution_is_p(mode):
    """Losslessness of the whole stochastic step: from a fixed state, the first
    emitted token over many seeds is distributed as p_0 = softmax(target / T)
    at the last token (draft and target differ, so rejections happen)."""
    ti, di = _micro_models()
    T = 0.5
    with ti, di:
        tm, dm = O.Model(ti), O.Model(di)
        prompt = S.tokens(79, 8, tm.V)
        tkv, dkv, last = _prefill(tm, dm, prompt)
        P = tkv.position
        n_s = 3000
        cnt = np.zeros(tm.V)
        p0 = None
        rej = 0
        for s in range(n_s):
            u = O.spec_uniforms(100 + s, 0, 3)
            em, dr, p, q = O.spec_step(tm, dm, tkv, dkv, last, 3, mode, T, u, want_logits=True)
            cnt[em[0]] += 1
            rej += em[0] != dr[0]
            p0 = p[0] if p0 is None else p0
            tkv.truncate(P)
            dkv.truncate(P)
            dkv.n_pending.value = 0
        pp = O.probs(p0, T).astype(np.float64)
        pp /= pp.sum()
        e = n_s * pp
        big = e >= 5
        obs = np.append(cnt[big], cnt[~big].sum())
        exp_ = np.append(e[big], e[~big].sum())
        keep = exp_ > 0
        chi2 = np.sum((obs[keep] - exp_[keep]) ** 2 / exp_[keep])
        dof = keep.sum() - 1
        assert rej > 100  # the draft's first token is often rejected
        assert chi2 < dof + 6 * np.sqrt(2 * dof), (chi2, dof)
        for x in (tkv, dkv, tm, dm):
            x.close()


# ------------------------------------------------------------------ qwen3 / qwen3moe

QWEN3_SMALL = S.LlamaShape(2, 256, 4, 2, 512, 700, 256, 1e-6, 1e6, 0.02, GGML_Q4_K, GGML_Q4_K, True, arch=1,
                           head_dim=128, norm_jitter=0.2)
QWEN3MOE_SMALL = S.LlamaShape(2, 256, 4, 2, 0, 700, 256, 1e-6, 1e6, 0.05, GGML_Q4_K, GGML_Q4_K, False, arch=2,
                              head_dim=128, n_expert=16, n_expert_used=4, expert_ff=256, norm_jitter=0.2,
                              router_std=1 / 16)


@pytest.mark.parametrize("shape", [QWEN3_SMALL, QWEN3MOE_SMALL], ids=["qwen3", "qwen3moe"])
def test_qwen_forward_matches_numpy(shape):
    """Decoupled head_dim (q width 512 > n_embd 256), per-head Q/K RMSNorm with
    non-unit weights, NEOX RoPE, and for qwen3moe the routed FFN, against the
    independent numpy f64 forward; then a second chunk (prefix + causal) and a
    tree chunk."""
    with S.GgufImage(shape, seed=12) as img:
        ref = R.RefQwen(bytes(img.bytes()))
        m = O.Model(img)
        assert m.arch == shape.arch and m.hd == 128
        kv = O.KvCache(m, 64)
        toks = S.tokens(5, 10, m.V)
        lg, res = O.forward(m, kv, toks, 0)
        rl, rr = ref.forward(toks)
        # row 0 attends to itself only: f32-level agreement; later rows also see
        # other rows' f16 V, where an f32-level difference occasionally rounds
        # to the neighbouring f16 (one ulp, ~1e-4 of the row after attention)
        np.testing.assert_allclose(res[0], rr[0], rtol=1e-5, atol=1e-5 * np.abs(rr[0]).max())
        np.testing.assert_allclose(lg[0], rl[0], rtol=1e-4, atol=1e-4 * np.abs(rl[0]).max())
        np.testing.assert_allclose(res, rr, rtol=1e-3, atol=5e-4 * np.abs(rr).max())
        np.testing.assert_allclose(lg, rl, rtol=1e-3, atol=1e-3 * np.abs(rl).max())
        par = [-1, 0, 0, 1]
        t2 = S.tokens(6, 4, m.V)
        lg2, _ = O.forward(m, kv, t2, 10, parents=par)
        rl2, _ = ref.forward(t2, parents=par)
        np.testing.assert_allclose(lg2, rl2, rtol=1e-3, atol=1e-3 * np.abs(rl2).max())
        for li in range(m.n_layer):  # layer 0 from the same inputs: one f16 ulp at most
            k = kv.layer(li, False, 14).view(np.float16).astype(np.float64)
            if li == 0:
                r = ref.K[li].astype(np.float16).view(np.uint16).astype(np.int32)
                assert np.abs(kv.layer(li, False, 14).astype(np.int32) - r).max() <= 1
            assert np.abs(k - ref.K[li]).max() <= 1e-3 * np.abs(ref.K[li]).max()
        kv.close()
        m.close()


def test_moe_route_closed_forms():
    rng = np.random.default_rng(3)
    for _ in range(200):
        E, k = 128, 8
        lg = rng.standard_normal(E).astype(np.float32)
        ids, w = O.moe_route(lg, k)
        # top-k of the softmax = top-k of the logits (monotone), in descending order
        want = np.argsort(-lg.astype(np.float64), kind="stable")[:k]
        assert list(ids) == list(want)
        assert abs(float(w.astype(np.float64).sum()) - 1.0) < 1e-6
        assert np.all(np.diff(w) <= 0)
        # weights are softmax restricted to the selection: w_i / w_j = exp(l_i - l_j)
        np.testing.assert_allclose(w[1:] / w[0], np.exp(lg[ids[1:]].astype(np.float64) - lg[ids[0]]), rtol=1e-6)
    # ties go to the lower expert index
    ids, w = O.moe_route(np.array([0.5, 2.0, 2.0, 1.0, 2.0], np.float32), 3)
    assert list(ids) == [1, 2, 4] and np.allclose(w, 1 / 3)


# ------------------------------------------------------------------ Q5_K / Q6_K

GGML_Q5_K, GGML_Q6_K = 13, 14


@pytest.mark.parametrize("qtype,bb", [(GGML_Q5_K, 176), (GGML_Q6_K, 210)], ids=["q5k", "q6k"])
def test_kquant_dequant_random_bytes_match_numpy(qtype, bb):
    """Arbitrary block bytes (every bit pattern of qs / qh / scales) with finite f16
    d / dmin, against the independent numpy dequant."""
    rng = np.random.default_rng(9)
    rows, k = 5, 768
    raw = rng.integers(0, 256, rows * k // 256 * bb, dtype=np.uint8).reshape(rows, k // 256, bb)
    half = np.float16(rng.standard_normal((rows, k // 256, 2)) * 0.01).view(np.uint8).reshape(rows, k // 256, 4)
    if qtype == GGML_Q5_K:
        raw[:, :, 0:4] = half
    else:
        raw[:, :, 208:210] = half[:, :, :2]
    raw = raw.ravel()
    ref = R.dequant(qtype, raw, rows, k)
    for r in range(rows):
        np.testing.assert_allclose(O.dequant_row(qtype, raw, r, k), ref[r], rtol=1e-6, atol=1e-12)


@pytest.mark.parametrize("qtype", [GGML_Q5_K, GGML_Q6_K], ids=["q5k", "q6k"])
def test_kquant_quantizer_roundtrip(qtype):
    rng = np.random.default_rng(10)
    x = rng.standard_normal(4 * 512).astype(np.float32) * 0.02
    y = np.concatenate([O.dequant_row(qtype, S.quantize(qtype, x), r, 512) for r in range(4)])
    step = np.abs(x).max() / (31 if qtype == GGML_Q6_K else 15)  # 5 / 6 bits
    assert np.abs(y - x).max() <= step


def test_q6k_special_block():
    blk = np.zeros(210, dtype=np.uint8)
    blk[208:210] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    blk[192:208] = np.arange(16, dtype=np.int8).view(np.uint8) - 8  # scales -8 .. 7
    blk[0:128] = 0x00
    blk[128:192] = 0xAA            # top bits 2 for every element: q = 32 -> value 0
    assert np.all(O.dequant_row(GGML_Q6_K, blk, 0, 256) == 0.0)
    blk[128:192] = 0xFF            # q = 48 + nibble 0: (48 - 32) = 16
    y = O.dequant_row(GGML_Q6_K, blk, 0, 256)
    np.testing.assert_array_equal(y, 0.5 * 16 * np.repeat(np.arange(16) - 8, 16))


def test_q5k_special_block():
    blk = np.zeros(176, dtype=np.uint8)
    blk[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blk[4] = 1                     # sub-block 0: sc 1, m 0
    blk[16:48] = 0x01              # fifth bit of every element of sub-block 0
    blk[48:80] = 0x0F              # nibble 15 in sub-block 0 (low), 0 in sub-block 1 (high)
    y = O.dequant_row(GGML_Q5_K, blk, 0, 256)
    assert np.all(y[:32] == 31.0) and np.all(y[32:] == 0.0)


MIXED_Q4KM = S.LlamaShape(2, 256, 4, 2, 512, 700, 256, 1e-5, 5e5, 0.02, GGML_Q4_K, GGML_Q4_K, out_type=GGML_Q6_K,
                          mix=1)
MIXED_Q5K = S.LlamaShape(2, 256, 4, 2, 512, 700, 256, 1e-5, 5e5, 0.02, GGML_Q5_K, GGML_Q4_K, out_type=GGML_Q6_K)


@pytest.mark.parametrize("shape", [MIXED_Q4KM, MIXED_Q5K], ids=["q4km_mix", "q5k_base"])
def test_mixed_type_forward_matches_numpy(shape):
    """Q4_K_M-style mixes (attn_v / ffn_down of even layers and output in Q6_K)
    and a Q5_K base with a Q6_K lm_head, against the numpy f64 forward."""
    with S.GgufImage(shape, seed=13) as img:
        meta, T, _ = R.read_gguf(bytes(img.bytes()))
        assert T["output.weight"][1] == GGML_Q6_K
        ref = R.RefLlama(bytes(img.bytes()))
        m = O.Model(img)
        kv = O.KvCache(m, 32)
        toks = S.tokens(5, 8, m.V)
        lg, res = O.forward(m, kv, toks, 0)
        rl, rr = ref.forward(toks)
        np.testing.assert_allclose(res[0], rr[0], rtol=1e-5, atol=1e-5 * np.abs(rr[0]).max())
        np.testing.assert_allclose(lg, rl, rtol=1e-3, atol=1e-3 * np.abs(rl).max())
        kv.close()
        m.close()


def test_sample_one_filters_closed_forms():
    """The host chain's candidate filters (inference/sample.rs:404-473) on rows
    whose filtered distributions are known in closed form."""
    probs = np.array([0.05, 0.5, 0.15, 0.3])  # sorted desc: ids 1, 3, 2, 0
    lg = np.log(probs).astype(np.float32)
    # top_p 0.6: exclusive cumulative 0, 0.5, 0.8 -> ids 1, 3 kept (the crossing one stays),
    # renormalised 0.625 / 0.375
    c = O.SamplerCfg(1.0, 0, 0.6, 0.0)
    assert O.sample_one(lg, c, 0.6) == 1
    assert O.sample_one(lg, c, 0.63) == 3
    assert O.sample_one(lg, c, 0.999) == 3
    # top_p 0.5: exclusive cumulative of id 3 is 0.5, not above 0.5 -> still kept
    assert O.sample_one(lg, O.SamplerCfg(1.0, 0, 0.5, 0.0), 0.999) == 3
    # min_p 0.4: keep p >= 0.4 * 0.5 = 0.2 -> ids 1, 3 (0.15 dropped)
    c = O.SamplerCfg(1.0, 0, 1.0, 0.4)
    assert O.sample_one(lg, c, 0.999) == 3
    assert O.sample_one(lg, c, 0.62) == 1
    # top_k 3 then T = 2: weights sqrt(p) over ids 1, 3, 2
    w = np.sqrt(np.array([0.5, 0.3, 0.15]))
    cum = np.cumsum(w / w.sum())
    c = O.SamplerCfg(2.0, 3, 1.0, 0.0)
    for u, want in [(cum[0] - 1e-3, 1), (cum[0] + 1e-3, 3), (cum[1] + 1e-3, 2), (0.9999, 2)]:
        assert O.sample_one(lg, c, float(u)) == want, u
    # top_p before min_p: top_p 0.6 keeps ids 1, 3; min_p 0.7 then keeps id 1 only
    assert O.sample_one(lg, O.SamplerCfg(1.0, 0, 0.6, 0.7), 0.999) == 1
    # ties at the top_k threshold go to the lower id
    t = np.array([1.0, 2.0, 2.0, 0.0, 2.0], np.float32)
    assert O.sample_one(t, O.SamplerCfg(1.0, 2, 1.0, 0.0), 0.999) == 2
    assert O.sample_one(t, O.SamplerCfg(1.0, 2, 1.0, 0.0), 0.1) == 1
