"""GPU parity of the wide f16 GEMM (C ABI sh_gemm_wide16, the kernels of forward
calls of >= 32 columns) against the oracle's or_gemv16.

The reference computes matmuls of N >= 32 columns with its cooperative-matrix
GEMM (ops/matmul.rs:433-446, mul_mm_cm.slang): weights dequantized in f32 and
rounded to f16, activations rounded to f16, f32 accumulation. or_gemv16 takes
the same f16 operands and sums in f64, so the GPU differs from it only by f32
summation order and by weights whose f16 rounding of the exact a q - b and of
the oracle's twice-rounded f32 value differ in the last bit: bound 2e-5 x
max|y|. The same outputs sit ~1e-4 of max|y| from the exact f64 GEMV (the f16
rounding of the operands), which the test also checks, so a kernel that kept
f32-level operands would fail the first bound.
"""
import numpy as np
import pytest

import oracle as O
from seeker_amd import QTensor
from seeker_amd import synth as S
from seeker_amd._native import GGML_Q4_K, GGML_Q5_K, GGML_Q6_K, GGML_Q8_0

pytestmark = pytest.mark.gpu


def _run(engine, M, K, N, seed=0, accumulate=False):
    print(f"wide16 case M={M} K={K} N={N} acc={accumulate}", flush=True)
    w = S.quantize(GGML_Q4_K, S.normal_f32(seed, 1, M * K, 0.0, 0.02))
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((N, K)).astype(np.float32)
    y0 = rng.standard_normal((N, M)).astype(np.float32) if accumulate else np.zeros((N, M), np.float32)
    qt = QTensor(engine, GGML_Q4_K, w, M, K)
    xd, yd = engine.to_device(x), engine.to_device(y0)
    engine.gemm_wide16(qt, xd, N, yd, accumulate)
    got = yd.read(np.float32, N * M).reshape(N, M)
    add = y0 if accumulate else 0
    ref16 = O.gemv16(GGML_Q4_K, w, M, K, x) + add
    exact = O.gemv(GGML_Q4_K, w, M, K, x) + add
    xd.free(); yd.free(); qt.close()
    return got, ref16, exact


@pytest.mark.parametrize("N", [1, 13, 32, 47, 64, 70, 129, 164, 192, 200])
def test_wide16_small(engine, N):
    got, ref, exact = _run(engine, 80, 512, N, seed=N)
    scale = np.abs(ref).max()
    err, dex = np.abs(got - ref).max() / scale, np.abs(got - exact).max() / scale
    print(f"  vs or_gemv16 {err:.2e}, vs exact {dex:.2e}", flush=True)
    assert err < 2e-5, err
    assert dex > 4 * err


def test_wide16_ragged_rows_and_accumulate(engine):
    got, ref, _ = _run(engine, 37, 768, 40, seed=3, accumulate=True)
    assert np.abs(got - ref).max() / np.abs(ref).max() < 2e-5


@pytest.mark.parametrize("M,K,N", [(6144, 4096, 41), (4096, 4096, 64), (28672, 4096, 48), (4096, 14336, 36),
                                   (128256, 4096, 33), (28672, 4096, 164), (4096, 14336, 164), (6144, 4096, 192),
                                   (128256, 4096, 100)])
def test_wide16_8b_shapes(engine, M, K, N):
    got, ref, exact = _run(engine, M, K, N, seed=M + K + N)
    scale = np.abs(ref).max()
    err, dex = np.abs(got - ref).max() / scale, np.abs(got - exact).max() / scale
    print(f"  vs or_gemv16 {err:.2e}, vs exact {dex:.2e}", flush=True)
    assert err < 2e-5, err
    assert np.array_equal(got.argmax(axis=1), ref.argmax(axis=1))


@pytest.mark.parametrize("qtype", [GGML_Q8_0, GGML_Q5_K, GGML_Q6_K], ids=["q8_0", "q5k", "q6k"])
@pytest.mark.parametrize("M,K,N", [(80, 512, 32), (37, 1536, 70), (512, 1408, 45), (4000, 512, 192)])
def test_wide16_other_formats(engine, qtype, M, K, N):
    """The reference's wide GEMM has Q8_0, Q5_K and Q6_K variants too
    (mmcm_variant, ops/matmul.rs:238-290): f16(f32 dequant) weights in the
    oracle's order of f32 operations, so only the summation order differs from
    or_gemv16."""
    if qtype != GGML_Q8_0 and K % 256:
        K = K // 256 * 256
    print(f"wide16 {qtype} M={M} K={K} N={N}", flush=True)
    w = S.quantize(qtype, S.normal_f32(M + K, 2, M * K, 0.0, 0.02))
    rng = np.random.default_rng(N)
    x = rng.standard_normal((N, K)).astype(np.float32)
    qt = QTensor(engine, qtype, w, M, K)
    xd, yd = engine.to_device(x), engine.to_device(np.zeros((N, M), np.float32))
    engine.gemm_wide16(qt, xd, N, yd, False)
    got = yd.read(np.float32, N * M).reshape(N, M)
    ref = O.gemv16(qtype, w, M, K, x)
    exact = O.gemv(qtype, w, M, K, x)
    xd.free(); yd.free(); qt.close()
    scale = np.abs(ref).max()
    err, dex = np.abs(got - ref).max() / scale, np.abs(got - exact).max() / scale
    print(f"  vs or_gemv16 {err:.2e}, vs exact {dex:.2e}", flush=True)
    assert err < 1e-5, err
    assert dex > 4 * err
