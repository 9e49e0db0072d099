// Device helpers shared by the kernels that build the GEMV activation operand.
#pragma once
#include "sh_internal.h"

// Cross-lane steps through DPP (no LDS round trip, unlike __shfl_xor):
// quad_perm(1,0,3,2) and quad_perm(2,3,0,1) pair lanes l ^ 1 and l ^ 2;
// row_half_mirror (lane 7 - l of each 8) and row_mirror (15 - l of each 16)
// then pair the quads and the halves of a row once every quad, resp. half,
// holds one value in all its lanes. Every lane of the wave must be active.
template <int CTRL>
__device__ __forceinline__ float sh_dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
constexpr int SH_DPP_XOR1 = 0xB1, SH_DPP_XOR2 = 0x4E, SH_DPP_HALF_MIRROR = 0x141, SH_DPP_MIRROR = 0x140;
__device__ __forceinline__ float sh_lane(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
// Sum over the wave, the same value in every lane: rows of 16 by DPP, then
// the four row sums as (r0 + r1) + (r2 + r3).
__device__ __forceinline__ float sh_wave_sum(float v) {
  v += sh_dpp<SH_DPP_XOR1>(v);
  v += sh_dpp<SH_DPP_XOR2>(v);
  v += sh_dpp<SH_DPP_HALF_MIRROR>(v);
  v += sh_dpp<SH_DPP_MIRROR>(v);
  return (sh_lane(v, 0) + sh_lane(v, 16)) + (sh_lane(v, 32) + sh_lane(v, 48));
}
// Sum of squares of a lane's four elements with explicit FMAs, so every prep
// (kernel or fused into a GEMV) rounds it identically whatever the compiler's
// contraction choices in the surrounding code.
__device__ __forceinline__ float sh_sq4(float4 v) {
  return __builtin_fmaf(v.w, v.w, __builtin_fmaf(v.z, v.z, __builtin_fmaf(v.y, v.y, v.x * v.x)));
}
__device__ __forceinline__ float sh_wave_max(float v) {
  v = fmaxf(v, sh_dpp<SH_DPP_XOR1>(v));
  v = fmaxf(v, sh_dpp<SH_DPP_XOR2>(v));
  v = fmaxf(v, sh_dpp<SH_DPP_HALF_MIRROR>(v));
  v = fmaxf(v, sh_dpp<SH_DPP_MIRROR>(v));
  return fmaxf(fmaxf(sh_lane(v, 0), sh_lane(v, 16)), fmaxf(sh_lane(v, 32), sh_lane(v, 48)));
}

// Operands of more than 8 columns come in groups of 8: column col lives in
// group col / 8 as lane column col % 8, and group g's B, XS, cs and sums of
// squares start at g times one group's size for this K (sizes below).
__host__ __device__ __forceinline__ size_t sh_grp_bx(uint32_t K) { return (size_t)((K + 255) / 256) * 8 * 512; }
__host__ __device__ __forceinline__ size_t sh_grp_xs(uint32_t K) { return (size_t)((K + 255) / 256) * 512; }
__host__ __device__ __forceinline__ size_t sh_grp_cs(uint32_t K) { return (size_t)((K + 255) / 256) * 8; }

// One lane's share of one 256-element superblock of one operand column, for
// any destination: lane l holds y[256 sb + 4l .. +3]. The superblock is
// multiplied by the power of two s that puts its max|y| in [2^9, 2^10) and
// inv = 1/s, so the f16 low halves stay normal (an f16 subnormal has only
// 2^-24 absolute resolution). hi/lo: the four elements as f16 hi + lo (elements
// 2, 3 of every 4 carry an exact 1/16: the Q4_K kernels decode their nibbles as
// 1024 + 16 q and the Q8_0 kernels their bytes as 16 q); shi/slo: the
// 32-element sub-block sum of the lane's 8-lane group, valid in lanes l % 8 = 0.
// Every lane of the wave must call this (cross-lane DPP steps).
struct ShOpndLane {
  uint2 hi, lo;
  uint16_t shi, slo;
  float inv;
};
__device__ __forceinline__ ShOpndLane sh_operand_lane(float4 v) {
  const float mx = sh_wave_max(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
  int ex = 0;
  if (mx > 0.f && mx < INFINITY) {
    frexpf(mx, &ex);  // mx = m * 2^ex, m in [0.5, 1)
    ex = ex < -100 ? -100 : (ex > 100 ? 100 : ex);
  }
  const float ps = ldexpf(1.0f, 10 - ex);
  ShOpndLane o;
  o.inv = ldexpf(1.0f, ex - 10);
  const float y[4] = {v.x * ps, v.y * ps, v.z * ps, v.w * ps};
  uint16_t hi[4], lo[4];
  float sum = 0.f;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const float yt = t >= 2 ? y[t] * 0.0625f : y[t];
    const _Float16 h = (_Float16)yt;
    hi[t] = __builtin_bit_cast(uint16_t, h);
    lo[t] = __builtin_bit_cast(uint16_t, (_Float16)(yt - (float)h));
    sum += y[t];
  }
  // 8 consecutive lanes cover one 32-element sub-block (the pairs of an xor
  // butterfly over lanes l ^ 1, l ^ 2, l ^ 4)
  sum += sh_dpp<SH_DPP_XOR1>(sum);
  sum += sh_dpp<SH_DPP_XOR2>(sum);
  sum += sh_dpp<SH_DPP_HALF_MIRROR>(sum);
  o.hi = *(const uint2*)hi;
  o.lo = *(const uint2*)lo;
  const _Float16 sh = (_Float16)sum;
  o.shi = __builtin_bit_cast(uint16_t, sh);
  o.slo = __builtin_bit_cast(uint16_t, (_Float16)(sum - (float)sh));
  return o;
}

// One wave writes superblock sb (elements 256 sb .. 256 sb + 255) of column
// `col` of the GEMV activation operand in global memory (sh_operand_lane);
// cs[sb * 8 + col] = 1/s. Layouts: B (hi/lo f16, [K/32][64][8], lane 16g + c:
// hi of column c, lane 16g + 8 + c: lo) and XS (per-32 sums, [K/256][64][8],
// lanes >= 16 stay zero). Every lane of the wave must call this.
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
  const ShOpndLane o = sh_operand_lane(v);
  if (lane == 0) cs[sb * 8 + col] = o.inv;
  const uint32_t k = 256 * sb + 4 * lane;
  if (k < K) {
    uint16_t* dst = bx + ((size_t)(k / 32) * 64 + ((k % 32) / 8) * 16 + col) * 8 + (k % 8);
    *(uint2*)dst = o.hi;
    *(uint2*)(dst + 64) = o.lo;
    if ((lane & 7) == 0) {
      const uint32_t s = (k % 256) / 32;
      const size_t xo = ((size_t)sb * 64 + col) * 8 + s;
      xs[xo] = o.shi;
      xs[xo + 64] = o.slo;
    }
  }
}

// Attention split combine for one lane: output elements 256 sb + 4 lane .. +3
// of column col (a 256-wide superblock of heads), merging the n_splits key
// splits of the partial buffer in split order, 16 at a time (the loads of NCH
// such chunks issued before the first is used, one hardware exp2 per split). Partial layout:
// part[((kh * n_layout + split) * rows_pad + rho) * (hd + 4) + {d < hd: O, hd: m,
// hd + 1: l}], rho = (head % gqa) * N + col. Zero for elements past Dq.
template <uint32_t NCH = 1>
__device__ __forceinline__ float4 sh_fa_combine4(const float* __restrict__ part, uint32_t n_layout, uint32_t n_splits,
                                                 uint32_t rows_pad, uint32_t hd, uint32_t n_head, uint32_t gqa,
                                                 uint32_t N, uint32_t sb, uint32_t col) {
  constexpr uint32_t CH = 16;
  const uint32_t lane = threadIdx.x & 63, PS = hd + 4;
  const uint32_t Dq = n_head * hd;
  const size_t sstride = (size_t)rows_pad * PS;
  const uint32_t kk = 256 * sb + 4 * lane;
  const bool valid = kk < Dq;
  const uint32_t k = valid ? kk : 0, head = k / hd, d = k % hd;
  const uint32_t kh = head / gqa, rho = (head % gqa) * N + col;
  const float* p = part + (size_t)kh * n_layout * sstride + (size_t)rho * PS;
  float M = -INFINITY, L = 0.f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  // NCH chunks' loads go out together: with 2, a key length just past a
  // multiple of 16 splits (4104 keys = 17 splits of 256) costs one round trip,
  // not two (the per-chunk arithmetic is the same for any NCH)
  for (uint32_t s00 = 0; s00 < n_splits; s00 += NCH * CH) {
    float4 os[NCH][CH];
    float2 ml[NCH][CH];
#pragma unroll
    for (uint32_t hh = 0; hh < NCH; ++hh)
#pragma unroll
      for (uint32_t j = 0; j < CH; ++j) {
        const float* pp = p + (size_t)min(s00 + CH * hh + j, n_splits - 1) * sstride;
        os[hh][j] = *(const float4*)(pp + d);
        ml[hh][j] = *(const float2*)(pp + hd);
      }
    // NCH == 1: the first split of the next chunk comes with these loads, so a
    // last chunk of one split (4097 keys = 16 splits of 256 + 1) needs no
    // second round trip
    float4 ox = make_float4(0.f, 0.f, 0.f, 0.f);
    float2 mlx = make_float2(-INFINITY, 0.f);
    const bool one_more = NCH == 1 && s00 + CH + 1 == n_splits;
    if (one_more) {
      const float* pp = p + (size_t)(s00 + CH) * sstride;
      ox = *(const float4*)(pp + d);
      mlx = *(const float2*)(pp + hd);
    }
#pragma unroll
    for (uint32_t hh = 0; hh < NCH; ++hh) {
      const uint32_t s0 = s00 + CH * hh;
      if (s0 >= n_splits) break;
      float mc = -INFINITY;
#pragma unroll
      for (uint32_t j = 0; j < CH; ++j) mc = fmaxf(mc, ml[hh][j].x);  // repeats of the last split change nothing
      if (mc == -INFINITY) continue;
      const float mn = fmaxf(M, mc);
      const float a = __builtin_amdgcn_exp2f((M - mn) * 1.4426950408889634f);  // 0 on the first chunk (M = -inf)
      acc.x *= a; acc.y *= a; acc.z *= a; acc.w *= a;
      L *= a;
#pragma unroll
      for (uint32_t j = 0; j < CH; ++j) {
        // 0 for an empty split (m = -inf) and for the clamped repeats past the end
        const float w = s0 + j < n_splits ? __builtin_amdgcn_exp2f((ml[hh][j].x - mn) * 1.4426950408889634f) : 0.0f;
        acc.x += os[hh][j].x * w; acc.y += os[hh][j].y * w; acc.z += os[hh][j].z * w; acc.w += os[hh][j].w * w;
        L += ml[hh][j].y * w;
      }
      M = mn;
    }
    if (one_more) {
      // the one-split chunk as the loop above runs it (its clamped repeats
      // carry weight 0)
      if (mlx.x != -INFINITY) {
        const float mn = fmaxf(M, mlx.x);
        const float a = __builtin_amdgcn_exp2f((M - mn) * 1.4426950408889634f);
        acc.x *= a; acc.y *= a; acc.z *= a; acc.w *= a;
        L *= a;
        const float w = __builtin_amdgcn_exp2f((mlx.x - mn) * 1.4426950408889634f);
        acc.x += ox.x * w; acc.y += ox.y * w; acc.z += ox.z * w; acc.w += ox.w * w;
        L += mlx.y * w;
        M = mn;
      }
      break;
    }
  }
  const float il = L > 0.f ? 1.0f / L : 0.f;
  if (!valid) return make_float4(0.f, 0.f, 0.f, 0.f);
  return make_float4(acc.x * il, acc.y * il, acc.z * il, acc.w * il);
}
