// Device helper shared by the kernels that build the GEMV activation operand.
#pragma once
#include "sh_internal.h"

constexpr int SH_OPERAND_THREADS = 1024;

__device__ __forceinline__ float sh_wave_sum(float v) {
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  return v;
}
__device__ __forceinline__ float sh_wave_max(float v) {
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

// Column `col` of an activation, held as NV float4 per thread of a
// 1024-thread workgroup (element k = 4 * (tid + 1024 i) + t), multiplied by
// `pre` and by the power of two s that puts max|y| in [2^9, 2^10), becomes the
// GEMV operand: B (hi/lo f16, [K/32][64][8], lane 16g + c: hi of column c,
// lane 16g + 8 + c: lo) and XS (per-32 sums, [K/256][64][8], lanes >= 16 stay
// zero). cs[col] = 1/s. `amax` is max|v| over the column (before `pre`).
// Keeping |y| >= 2^9-ish keeps the f16 low halves normal: an f16 subnormal has
// only 2^-24 absolute resolution.
template <int NV>
__device__ __forceinline__ void sh_operand_store(const float4 (&v)[NV], uint32_t K, uint32_t col, float pre,
                                                 float amax, uint16_t* __restrict__ bx, uint16_t* __restrict__ xs,
                                                 float* __restrict__ cs) {
  const uint32_t tid = threadIdx.x, n4 = K / 4;
  const float mx = amax * pre;
  int ex = 0;
  if (mx > 0.f && mx < INFINITY) {
    frexpf(mx, &ex);  // mx = m * 2^ex, m in [0.5, 1)
    ex = ex < -100 ? -100 : (ex > 100 ? 100 : ex);
  }
  const float ps = ldexpf(1.0f, 10 - ex) * pre;
  if (tid == 0) cs[col] = ldexpf(1.0f, ex - 10);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const uint32_t q = tid + SH_OPERAND_THREADS * i;  // every thread joins the shuffles
    const float y[4] = {v[i].x * ps, v[i].y * ps, v[i].z * ps, v[i].w * ps};
    uint16_t hi[4], lo[4];
    float sum = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      // elements 2, 3 of every 4 carry an exact 1/16: the Q4_K kernel decodes
      // their nibbles as 1024 + 16 q (see q4_operand2 in gemv.hip)
      const float yt = t >= 2 ? y[t] * 0.0625f : y[t];
      const _Float16 h = (_Float16)yt;
      hi[t] = __builtin_bit_cast(uint16_t, h);
      lo[t] = __builtin_bit_cast(uint16_t, (_Float16)(yt - (float)h));
      sum += y[t];
    }
    // 8 consecutive threads cover one 32-element sub-block
    sum += __shfl_xor(sum, 1);
    sum += __shfl_xor(sum, 2);
    sum += __shfl_xor(sum, 4);
    if (q < n4) {
      const uint32_t k = 4 * q;
      uint16_t* dst = bx + ((size_t)(k / 32) * 64 + ((k % 32) / 8) * 16 + col) * 8 + (k % 8);
      *(uint2*)dst = *(const uint2*)hi;
      *(uint2*)(dst + 64) = *(const uint2*)lo;
      if ((q & 7) == 0) {
        const uint32_t sb = k / 32;
        const _Float16 sh = (_Float16)sum;
        const size_t xo = ((size_t)(sb / 8) * 64 + col) * 8 + (sb % 8);
        xs[xo] = __builtin_bit_cast(uint16_t, sh);
        xs[xo + 64] = __builtin_bit_cast(uint16_t, (_Float16)(sum - (float)sh));
      }
    }
  }
}
