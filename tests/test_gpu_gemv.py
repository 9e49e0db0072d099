"""GPU parity of the quantized GEMV (C ABI sh_gemv_quant) against the oracle.

Tolerance: the kernel keeps ~22 bits of each activation (hi + lo f16) and
accumulates in f32, so results agree with the oracle's f64 sums to ~1e-6 of
the output scale; the bound used is 2e-5 x max|y| (far inside the north-star
2e-2 abs / 1e-2 rel for logits).
"""
import numpy as np
import pytest

import oracle as O
from seeker_amd import QTensor
from seeker_amd import synth as S
from seeker_amd._native import GGML_Q4_K, GGML_Q8_0

pytestmark = pytest.mark.gpu


def _weights(qtype, M, K, seed):
    x = S.normal_f32(seed, 1, M * K, 0.0, 0.02)
    return S.quantize(qtype, x)


def _run(engine, qtype, M, K, N, seed=0, accumulate=False):
    print(f"gemv case qtype={qtype} M={M} K={K} N={N} acc={accumulate}", flush=True)
    w = _weights(qtype, M, K, seed)
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((N, K)).astype(np.float32)
    y0 = rng.standard_normal((N, M)).astype(np.float32) if accumulate else np.zeros((N, M), np.float32)
    qt = QTensor(engine, qtype, w, M, K)
    xd = engine.to_device(x)
    yd = engine.to_device(y0)
    engine.gemv(qt, xd, N, yd, accumulate)
    got = yd.read(np.float32, N * M).reshape(N, M)
    ref = O.gemv(qtype, w, M, K, x) + (y0 if accumulate else 0)
    xd.free(); yd.free(); qt.close()
    return got, ref


@pytest.mark.parametrize("qtype", [GGML_Q8_0, GGML_Q4_K])
@pytest.mark.parametrize("N", [1, 3, 8, 13])
def test_gemv_small(engine, qtype, N):
    got, ref = _run(engine, qtype, 80, 512, N, seed=N)
    err = np.abs(got - ref).max() / np.abs(ref).max()
    assert err < 2e-5, err


@pytest.mark.parametrize("qtype", [GGML_Q8_0, GGML_Q4_K])
def test_gemv_ragged_rows_and_accumulate(engine, qtype):
    got, ref = _run(engine, qtype, 37, 768, 5, seed=3, accumulate=True)
    assert np.abs(got - ref).max() / np.abs(ref).max() < 2e-5


@pytest.mark.parametrize("M,K", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336), (28672, 4096)])
def test_gemv_q4k_8b_shapes(engine, M, K):
    got, ref = _run(engine, GGML_Q4_K, M, K, 8, seed=M + K)
    assert np.abs(got - ref).max() / np.abs(ref).max() < 2e-5
    # greedy-relevant: per-column argmax identical
    assert np.array_equal(got.argmax(axis=1), ref.argmax(axis=1))


@pytest.mark.parametrize("N", [1, 3])
def test_gemv_q4k_deep_ring_columns(engine, N):
    """28672 x 4096 takes the deep-ring kernel (7 tiles per workgroup, 256
    workgroups); fewer than 8 columns leave operand lanes unused."""
    got, ref = _run(engine, GGML_Q4_K, 28672, 4096, N, seed=17 + N)
    assert np.abs(got - ref).max() / np.abs(ref).max() < 2e-5
    assert np.array_equal(got.argmax(axis=1), ref.argmax(axis=1))


def test_gemv_q4k_lm_head_shape(engine):
    got, ref = _run(engine, GGML_Q4_K, 128256, 4096, 8, seed=5)
    assert np.abs(got - ref).max() / np.abs(ref).max() < 2e-5
    assert np.array_equal(got.argmax(axis=1), ref.argmax(axis=1))


# Multi-group kernel (Q4_K, more than 8 columns: up to 64 columns per pass over
# the weights, split-K partials reduced in split order).
@pytest.mark.parametrize("M,K,N", [(4096, 4096, 9), (4096, 4096, 64), (28672, 4096, 40), (4096, 14336, 33),
                                   (6144, 4096, 164)])
def test_gemm_q4k_multi_group(engine, M, K, N):
    got, ref = _run(engine, GGML_Q4_K, M, K, N, seed=M + N)
    assert np.abs(got - ref).max() / np.abs(ref).max() < 2e-5
    assert np.array_equal(got.argmax(axis=1), ref.argmax(axis=1))


def test_gemm_q4k_multi_group_ragged_accumulate(engine):
    got, ref = _run(engine, GGML_Q4_K, 37, 768, 21, seed=4, accumulate=True)
    assert np.abs(got - ref).max() / np.abs(ref).max() < 2e-5


def test_gemm_q4k_columns_independent_of_batch(engine):
    """A column's result does not depend on how many columns share the launch
    (split shapes depend on the matrix only)."""
    M, K = 4096, 4096
    w = _weights(GGML_Q4_K, M, K, 11)
    x = np.random.default_rng(11).standard_normal((64, K)).astype(np.float32)
    qt = QTensor(engine, GGML_Q4_K, w, M, K)
    outs = []
    for n in (64, 20, 9):
        xd = engine.to_device(np.ascontiguousarray(x[:n]))
        yd = engine.to_device(np.zeros((n, M), np.float32))
        engine.gemv(qt, xd, n, yd, False)
        outs.append(yd.read(np.float32, n * M).reshape(n, M))
        xd.free(); yd.free()
    qt.close()
    assert np.array_equal(outs[0][:20], outs[1])
    assert np.array_equal(outs[0][:9], outs[2])
