// Device helpers shared by the kernels that build the GEMV activation operand.
#pragma once
#include "sh_internal.h"

__device__ __forceinline__ float sh_wave_sum(float v) {
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  return v;
}
__device__ __forceinline__ float sh_wave_max(float v) {
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

// Operands of more than 8 columns come in groups of 8: column col lives in
// group col / 8 as lane column col % 8, and group g's B, XS, cs and sums of
// squares start at g times one group's size for this K (sizes below).
__host__ __device__ __forceinline__ size_t sh_grp_bx(uint32_t K) { return (size_t)((K + 255) / 256) * 8 * 512; }
__host__ __device__ __forceinline__ size_t sh_grp_xs(uint32_t K) { return (size_t)((K + 255) / 256) * 512; }
__host__ __device__ __forceinline__ size_t sh_grp_cs(uint32_t K) { return (size_t)((K + 255) / 256) * 8; }

// One wave writes superblock sb (elements 256 sb .. 256 sb + 255) of column
// `col` of the GEMV activation operand; lane l holds y[256 sb + 4l .. +3]
// (zeros past K). The superblock is multiplied by the power of two s that puts
// its max|y| in [2^9, 2^10) and cs[sb * 8 + col] = 1/s, so the f16 low halves
// stay normal (an f16 subnormal has only 2^-24 absolute resolution). Layouts:
// B (hi/lo f16, [K/32][64][8], lane 16g + c: hi of column c, lane 16g + 8 + c:
// lo) and XS (per-32 sums, [K/256][64][8], lanes >= 16 stay zero). Every lane
// of the wave must call this (it shuffles).
__device__ __forceinline__ void sh_operand_store_sb(float4 v, uint32_t K, uint32_t sb, uint32_t col,
                                                    uint16_t* __restrict__ bx, uint16_t* __restrict__ xs,
                                                    float* __restrict__ cs) {
  const uint32_t lane = threadIdx.x & 63;
  {
    const uint32_t g = col / 8;
    bx += g * sh_grp_bx(K);
    xs += g * sh_grp_xs(K);
    cs += g * sh_grp_cs(K);
    col %= 8;
  }
  const float mx = sh_wave_max(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
  int ex = 0;
  if (mx > 0.f && mx < INFINITY) {
    frexpf(mx, &ex);  // mx = m * 2^ex, m in [0.5, 1)
    ex = ex < -100 ? -100 : (ex > 100 ? 100 : ex);
  }
  const float ps = ldexpf(1.0f, 10 - ex);
  if (lane == 0) cs[sb * 8 + col] = ldexpf(1.0f, ex - 10);
  const float y[4] = {v.x * ps, v.y * ps, v.z * ps, v.w * ps};
  uint16_t hi[4], lo[4];
  float sum = 0.f;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    // elements 2, 3 of every 4 carry an exact 1/16: the Q4_K kernels decode
    // their nibbles as 1024 + 16 q and the Q8_0 kernels their bytes as 16 q
    const float yt = t >= 2 ? y[t] * 0.0625f : y[t];
    const _Float16 h = (_Float16)yt;
    hi[t] = __builtin_bit_cast(uint16_t, h);
    lo[t] = __builtin_bit_cast(uint16_t, (_Float16)(yt - (float)h));
    sum += y[t];
  }
  // 8 consecutive lanes cover one 32-element sub-block
  sum += __shfl_xor(sum, 1);
  sum += __shfl_xor(sum, 2);
  sum += __shfl_xor(sum, 4);
  const uint32_t k = 256 * sb + 4 * lane;
  if (k < K) {
    uint16_t* dst = bx + ((size_t)(k / 32) * 64 + ((k % 32) / 8) * 16 + col) * 8 + (k % 8);
    *(uint2*)dst = *(const uint2*)hi;
    *(uint2*)(dst + 64) = *(const uint2*)lo;
    if ((lane & 7) == 0) {
      const uint32_t s = (k % 256) / 32;
      const _Float16 sh = (_Float16)sum;
      const size_t xo = ((size_t)sb * 64 + col) * 8 + s;
      xs[xo] = __builtin_bit_cast(uint16_t, sh);
      xs[xo + 64] = __builtin_bit_cast(uint16_t, (_Float16)(sum - (float)sh));
    }
  }
}
