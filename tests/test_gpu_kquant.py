"""GPU parity of the Q5_K / Q6_K multi-group GEMM and of K-quant-mixed models
against the C oracle.

Formats: Q5_K (llama.cpp block_q5_K: Q4_K's scales and nibbles plus a fifth
bit per element) and Q6_K (run.rs:4257-4291: 6-bit q - 32 times an int8 scale
per 16 elements, mul_mat_vec_q6_k.slang). Matrices are quantized by the
synthetic generator, or are arbitrary block bytes with finite f16 d / dmin
(every bit pattern of the quants and scales), or are special blocks at the
ends of the ranges (Q6_K scales -128 / 127 with q = 0 / 63, the products the
kernel splits as 16 sh + sl; Q5_K scale and min 63 with q = 31). Tolerance as
for Q4_K: 2e-5 x max|y| (the weights are decoded exactly; the error is the
activation's hi + lo f16 split and f32 accumulation), argmax identical.

Models: Q4_K_M-style (attn_v / ffn_down of even layers and output in Q6_K),
Q5_K_M-style (Q5_K base, the same Q6_K layers), a qwen3 with a Q6_K token
embedding tied as lm_head, and a qwen3moe with Q6_K attn_v and
ffn_down_exps on even layers (the expert-indirect GEMM in Q6_K) and a Q6_K
lm_head. They run on the multi-group path at every
chunk width; chunks of 1, 5, 8, 12 and 64 columns, a tree, greedy
verification and greedy speculative steps are
compared with the oracle (logits within 2e-2 abs / 1e-2 rel and 3e-4 x
max|logit|, greedy ids and emitted tokens equal).
"""
import numpy as np
import pytest

import oracle as O
from parity import ids_agree, logits_close, pair
from seeker_amd import QTensor
from seeker_amd import synth as S
from seeker_amd._native import GGML_Q4_K, GGML_Q5_K, GGML_Q6_K

pytestmark = pytest.mark.gpu

BLOCK_BYTES = {GGML_Q5_K: 176, GGML_Q6_K: 210}
KQ = [GGML_Q5_K, GGML_Q6_K]
IDS = ["q5k", "q6k"]


def _gemv(engine, qtype, w, M, K, x, y0=None):
    N = x.shape[0]
    qt = QTensor(engine, qtype, w, M, K)
    xd = engine.to_device(np.ascontiguousarray(x, np.float32))
    yd = engine.to_device(np.zeros((N, M), np.float32) if y0 is None else y0)
    engine.gemv(qt, xd, N, yd, y0 is not None)
    got = yd.read(np.float32, N * M).reshape(N, M)
    xd.free(); yd.free(); qt.close()
    return got


def _check(got, ref, argmax=True):
    err = np.abs(got - ref).max() / np.abs(ref).max()
    assert err < 2e-5, err
    if argmax:
        assert np.array_equal(got.argmax(axis=1), ref.argmax(axis=1))


def _quantized(qtype, M, K, seed):
    return S.quantize(qtype, S.normal_f32(seed, 1, M * K, 0.0, 0.02))


def _random_blocks(qtype, M, K, seed):
    rng = np.random.default_rng(seed)
    bb = BLOCK_BYTES[qtype]
    raw = rng.integers(0, 256, M * K // 256 * bb, dtype=np.uint8).reshape(M, K // 256, bb)
    half = np.float16(rng.standard_normal((M, K // 256, 2)) * 0.01).view(np.uint8).reshape(M, K // 256, 4)
    if qtype == GGML_Q5_K:
        raw[:, :, 0:4] = half
    else:
        raw[:, :, 208:210] = half[:, :, :2]
    return raw.ravel()


@pytest.mark.parametrize("qtype", KQ, ids=IDS)
@pytest.mark.parametrize("N", [1, 3, 8, 13])
def test_kquant_gemv_small(engine, qtype, N):
    print(f"kquant gemv qtype={qtype} 80x512 N={N}", flush=True)
    w = _quantized(qtype, 80, 512, N)
    x = np.random.default_rng(N).standard_normal((N, 512)).astype(np.float32)
    _check(_gemv(engine, qtype, w, 80, 512, x), O.gemv(qtype, w, 80, 512, x))


@pytest.mark.parametrize("qtype", KQ, ids=IDS)
def test_kquant_gemv_random_blocks_ragged_accumulate(engine, qtype):
    """Every bit pattern of quants and scales; 37 rows (a partial tile), 768
    columns (3 superblocks), accumulate into y."""
    print(f"kquant gemv qtype={qtype} random blocks 37x768", flush=True)
    M, K, N = 37, 768, 5
    w = _random_blocks(qtype, M, K, 21)
    rng = np.random.default_rng(22)
    x = rng.standard_normal((N, K)).astype(np.float32)
    y0 = rng.standard_normal((N, M)).astype(np.float32)
    _check(_gemv(engine, qtype, w, M, K, x, y0), O.gemv(qtype, w, M, K, x) + y0, argmax=False)


def test_q6k_extreme_scales(engine):
    """Scales -128 and 127 (the ends of the 16 sh + sl split) times q = 0 and 63:
    weights d * sc * (q - 32) at +-4096 d exactly."""
    print("q6k extreme scales", flush=True)
    M, K = 32, 512
    rng = np.random.default_rng(5)
    raw = np.zeros((M, K // 256, 210), np.uint8)
    for r in range(M):
        for b in range(K // 256):
            sc = rng.choice(np.array([-128, 127, -1, 0, 1, -8, 7, 16], np.int8), 16)
            raw[r, b, 192:208] = sc.view(np.uint8)
            raw[r, b, 0:128] = rng.choice(np.array([0x00, 0xFF, 0x0F, 0xF0], np.uint8), 128)
            raw[r, b, 128:192] = rng.choice(np.array([0x00, 0xFF, 0x55, 0xAA], np.uint8), 64)
            raw[r, b, 208:210] = np.array([2.0 ** rng.integers(-14, -6)], np.float16).view(np.uint8)
    w = raw.ravel()
    x = rng.standard_normal((9, K)).astype(np.float32)
    _check(_gemv(engine, GGML_Q6_K, w, M, K, x), O.gemv(GGML_Q6_K, w, M, K, x), argmax=False)


def test_q5k_extreme_scales(engine):
    """Scale and min 63 on every sub-block with q = 31 (nibble 15 + fifth bit)
    and q = 0 alternating by row."""
    print("q5k extreme scales", flush=True)
    M, K = 32, 512
    raw = np.zeros((M, K // 256, 176), np.uint8)
    raw[:, :, 0:2] = np.array([0.001], np.float16).view(np.uint8)
    raw[:, :, 2:4] = np.array([0.0005], np.float16).view(np.uint8)
    raw[:, :, 4:16] = 0xFF                      # every 6-bit scale and min 63
    raw[0::2, :, 16:48] = 0xFF                  # fifth bits on (even rows)
    raw[0::2, :, 48:176] = 0xFF                 # nibbles 15 (even rows)
    w = raw.ravel()
    x = np.random.default_rng(6).standard_normal((4, K)).astype(np.float32)
    ref = O.gemv(GGML_Q5_K, w, M, K, x)
    deq = O.dequant_row(GGML_Q5_K, w, 0, K)
    assert np.allclose(deq, 0.001 * 63 * 31 - 0.0005 * 63, rtol=1e-3)
    _check(_gemv(engine, GGML_Q5_K, w, M, K, x), ref, argmax=False)


@pytest.mark.parametrize("qtype", KQ, ids=IDS)
@pytest.mark.parametrize("M,K,N", [(4096, 4096, 8), (4096, 14336, 1), (1024, 4096, 64), (6144, 4096, 164)])
def test_kquant_gemv_8b_shapes(engine, qtype, M, K, N):
    print(f"kquant gemv qtype={qtype} {M}x{K} N={N}", flush=True)
    w = _quantized(qtype, M, K, M + N)
    x = np.random.default_rng(M + K + N).standard_normal((N, K)).astype(np.float32)
    _check(_gemv(engine, qtype, w, M, K, x), O.gemv(qtype, w, M, K, x))


def test_q6k_lm_head_shape(engine):
    """The Q4_K_M lm_head: 128256 x 4096 in Q6_K, 8 columns."""
    print("q6k lm_head 128256x4096 N=8", flush=True)
    M, K, N = 128256, 4096, 8
    w = _quantized(GGML_Q6_K, M, K, 3)
    x = np.random.default_rng(3).standard_normal((N, K)).astype(np.float32)
    _check(_gemv(engine, GGML_Q6_K, w, M, K, x), O.gemv(GGML_Q6_K, w, M, K, x))


def test_kquant_columns_independent_of_batch(engine):
    """A column's result does not depend on how many columns share the launch."""
    M, K = 2048, 4096
    w = _quantized(GGML_Q6_K, M, K, 12)
    x = np.random.default_rng(12).standard_normal((64, K)).astype(np.float32)
    outs = [_gemv(engine, GGML_Q6_K, w, M, K, x[:n]) for n in (64, 20, 1)]
    assert np.array_equal(outs[0][:20], outs[1])
    assert np.array_equal(outs[0][:1], outs[2])


# ------------------------------------------------------------------ models


def close(a, b, wide=False):
    logits_close(a, b, wide)  # north star + 3e-4 x max, or the f16-rounding bounds of tests/parity.py


Q4KM = S.LlamaShape(3, 512, 8, 4, 1024, 3000, 1024, 1e-5, 5e5, 0.02, GGML_Q4_K, GGML_Q4_K, out_type=GGML_Q6_K,
                    mix=1)
Q5KM = S.LlamaShape(2, 512, 8, 2, 1024, 3000, 1024, 1e-5, 5e5, 0.02, GGML_Q5_K, GGML_Q5_K, out_type=GGML_Q6_K,
                    mix=1)
QWEN3_Q6E = S.LlamaShape(2, 512, 8, 4, 1024, 3000, 1024, 1e-6, 1e6, 0.02, GGML_Q4_K, GGML_Q6_K, True, arch=1,
                         head_dim=128, norm_jitter=0.2, mix=1)
QWEN3MOE_MIX = S.LlamaShape(2, 512, 8, 2, 0, 3000, 1024, 1e-6, 1e6, 0.03, GGML_Q4_K, GGML_Q4_K, False, arch=2,
                            head_dim=128, n_expert=16, n_expert_used=4, expert_ff=512, norm_jitter=0.2,
                            router_std=512 ** -0.5, out_type=GGML_Q6_K, mix=1)
MODELS = {"q4km": Q4KM, "q5km": Q5KM, "qwen3_q6e": QWEN3_Q6E, "qwen3moe_mix": QWEN3MOE_MIX}


@pytest.fixture(scope="module", params=list(MODELS))
def model(request, engine):
    img = S.GgufImage(MODELS[request.param], seed=31)
    print(f"model {request.param}", flush=True)
    gm = engine.upload_weights(img)
    om = O.Model(img)
    pair(om, gm)  # the reference's wide-GEMM and cm1 attention arithmetic where the GPU uses them
    yield request.param, gm, om
    gm.close()
    om.close()
    img.close()


def test_mixed_chunks_match_oracle(engine, model):
    name, gm, om = model
    V = gm.dims.n_vocab
    gkv, okv = engine.allocate_kv_cache(gm, 512), O.KvCache(om, 512)
    prompt = S.tokens(70, 40, V)
    print(f"{name}: prefill 40", flush=True)
    engine.prefill(gm, gkv, prompt, 0)
    O.forward(om, okv, prompt, 0, logits_mode=0)
    pos = 40
    wide = gm.wide_f16 or gm.cm1_attention  # the prefill's f16 roundings (cm1 attention)
    for n in (1, 5, 8, 12, 64):
        toks = S.tokens(80 + n, n, V)
        print(f"{name}: verify {n} columns at {pos}", flush=True)
        gl, gres = engine.forward_full_readback(gm, gkv, toks, pos)
        ol, ores = O.forward(om, okv, toks, pos)
        close(gl, ol, wide)
        close(gres, ores, wide)
        gkv.truncate(pos)
        assert np.array_equal(engine.verify_greedy(gm, gkv, toks, pos), gl.argmax(axis=1))
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


def test_mixed_spec_steps_match_oracle(engine):
    """Greedy speculative steps, Q4_K_M-style target with a Q5_K_M-style draft."""
    t_img, d_img = S.GgufImage(Q4KM, seed=41), S.GgufImage(Q5KM, seed=42)
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
        print(f"mixed spec step {step}", flush=True)
        r = engine.decode_speculative(gt, gd, gtkv, gdkv, last, 5)
        em, dr = O.spec_step_greedy(ot, od, otkv, odkv, last, 5)
        assert (r.emitted, r.drafts) == (em, dr), step
        assert gtkv.position == otkv.position
        last = em[-1]
    for x in (gtkv, gdkv, otkv, odkv, gt, gd, ot, od):
        x.close()
    t_img.close()
    d_img.close()
