// Quantized GEMV for the verify step: y[j][m] = sum_k deq(W)[m][k] * x[j][k]
// for N <= 8 columns per launch chunk, on gfx950 MFMA.
//
// Semantics: the reference's batched-column matvec (ops/matmul.rs:473-487,
// shaders/compute/mul_mat_vec_q4_k.slang:13-103 for Q4_K, mul_mat_vec.slang:39-100
// for Q8_0), which dequantizes each weight row once and reuses it for all N
// columns. Design here (not a translation):
//   * Weights are repacked once at upload into 16-row tiles so each lane of a
//     wave64 reads its MFMA A-operand bytes with two 16-byte loads.
//   * Q4_K nibbles become exact f16 integers sc*q (<= 945) via the 0x6400 magic
//     exponent and one packed FMA; d and dmin are applied per 256-superblock in f32.
//   * Activations are split x = hi + lo (two f16) and fed as 16 MFMA columns
//     (8 hi + 8 lo), so v_mfma_f32_16x16x32_f16 keeps ~22 bits of x and f32
//     accumulation at no extra MFMA cost for N <= 8.
//   * The Q4_K minimum term dmin * sum_s m_s * sum(x in s) is a ninth MFMA per
//     superblock against per-sub-block column sums (XS).
#include "sh_internal.h"

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

struct alignas(16) u32x4 { uint32_t x, y, z, w; };

__device__ __forceinline__ h2 as_h2(uint32_t v) { return __builtin_bit_cast(h2, v); }
__device__ __forceinline__ uint32_t as_u32(h2 v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ h8 as_h8(u32x4 v) { return __builtin_bit_cast(h8, v); }
__device__ __forceinline__ u32x4 ld16(const void* p) { return *(const u32x4*)p; }

__device__ __forceinline__ f4 mfma16(h8 a, h8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// (v, v) as an f16 pair from a small non-negative integer byte.
__device__ __forceinline__ h2 pair_of(uint32_t word, int byte) {
  float f = (float)((word >> (8 * byte)) & 0xFFu);
  return h2{(_Float16)f, (_Float16)f};
}

// Four f16 pairs (1024 + q) from the nibbles of one repacked word, then
// (1024 + q) * sc - 1024 * sc = sc * q exactly (single rounding of an exact value).
__device__ __forceinline__ h8 q4_operand(uint32_t w, h2 mult, h2 add) {
  u32x4 r;
  r.x = as_u32(__builtin_elementwise_fma(as_h2((w & 0x000F000Fu) | 0x64006400u), mult, add));
  r.y = as_u32(__builtin_elementwise_fma(as_h2(((w >> 4) & 0x000F000Fu) | 0x64006400u), mult, add));
  r.z = as_u32(__builtin_elementwise_fma(as_h2(((w >> 8) & 0x000F000Fu) | 0x64006400u), mult, add));
  r.w = as_u32(__builtin_elementwise_fma(as_h2(((w >> 12) & 0x000F000Fu) | 0x64006400u), mult, add));
  return as_h8(r);
}

// int8 pairs -> f16 exact: (q ^ 0x80) + 1024 as f16, minus 1152. The
// activation operand carries a 1/16 factor at k with t % 4 >= 2 (see
// q4_operand2), so those pairs become 16 q = 16 (1024 + u) - 18432, still exact.
__device__ __forceinline__ h8 q8_operand(uint32_t w0, uint32_t w1) {
  const h2 off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
  const h2 k16 = {(_Float16)16.0f, (_Float16)16.0f};
  const h2 off16 = {(_Float16)-18432.0f, (_Float16)-18432.0f};
  uint32_t a = w0 ^ 0x80808080u, b = w1 ^ 0x80808080u;
  u32x4 r;
  r.x = as_u32(as_h2(((a & 0xFFu) | ((a & 0xFF00u) << 8)) | 0x64006400u) + off);
  r.y = as_u32(__builtin_elementwise_fma(as_h2((((a >> 16) & 0xFFu) | ((a >> 8) & 0xFF0000u)) | 0x64006400u), k16, off16));
  r.z = as_u32(as_h2(((b & 0xFFu) | ((b & 0xFF00u) << 8)) | 0x64006400u) + off);
  r.w = as_u32(__builtin_elementwise_fma(as_h2((((b >> 16) & 0xFFu) | ((b >> 8) & 0xFF0000u)) | 0x64006400u), k16, off16));
  return as_h8(r);
}

// Slot of key kappa (0..31) inside a 32-key V block: the PV MFMA's B operand
// (probabilities) arrives with lane group g holding keys {4g..4g+3, 16+4g..16+4g+3}.
__device__ __forceinline__ uint32_t v_slot(uint32_t kappa) {
  return 8u * ((kappa & 15u) >> 2) + 4u * (kappa >> 4) + (kappa & 3u);
}

// ------------------------------------------------------------------ repack

// Q4_K tile-superblock (2304 B): [0,2048) 64 lanes x 8 words; lane l (row l%16,
// group g=l/16), word m (sub-block m) holds q[32m + 8g + t], t=0..7, pair i=t/2:
// t even at bits 4i, t odd at bits 16+4i. [2048,2112) d|dmin<<16 per row;
// [2112,2304) the 12 packed scale bytes per row.
__global__ void k_repack_q4k(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, uint32_t M,
                             uint32_t nsb, uint32_t dst_tile0, uint32_t tile_stride) {
  const uint32_t tile = blockIdx.x, sb = blockIdx.y, l = threadIdx.x;
  const uint32_t r = l & 15, g = l >> 4, row = tile * 16 + r;
  uint8_t* out = dst + ((size_t)(dst_tile0 + tile * tile_stride) * nsb + sb) * SH_Q4K_TILE_BYTES;
  uint32_t words[8];
  if (row < M) {
    const uint8_t* blk = src + ((size_t)row * nsb + sb) * 144;
    const uint8_t* qs = blk + 16;
    for (int m = 0; m < 8; ++m) {
      uint32_t w = 0;
      for (int t = 0; t < 8; ++t) {
        uint32_t pos = 8 * g + t;
        uint32_t byte = qs[32 * (m >> 1) + pos];
        uint32_t q = (m & 1) ? (byte >> 4) : (byte & 0xF);
        uint32_t shift = (t & 1) ? 16 + 4 * (t >> 1) : 4 * (t >> 1);
        w |= q << shift;
      }
      words[m] = w;
    }
    if (g == 0) {
      uint32_t dd = blk[0] | (blk[1] << 8) | (blk[2] << 16) | ((uint32_t)blk[3] << 24);
      *(uint32_t*)(out + 2048 + 4 * r) = dd;
      for (int i = 0; i < 12; ++i) out[2112 + 12 * r + i] = blk[4 + i];
    }
  } else {
    for (int m = 0; m < 8; ++m) words[m] = 0;
    if (g == 0) {
      *(uint32_t*)(out + 2048 + 4 * r) = 0;
      for (int i = 0; i < 12; ++i) out[2112 + 12 * r + i] = 0;
    }
  }
  uint32_t* o = (uint32_t*)(out + 32 * l);
  for (int m = 0; m < 8; ++m) o[m] = words[m];
}

// Q8_0 tile-block (544 B): [0,512) 64 lanes x 8 int8 (row l%16, k = 32b + 8g + t);
// [512,544) f16 d per row.
__global__ void k_repack_q8(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, uint32_t M,
                            uint32_t nb, uint32_t dst_tile0, uint32_t tile_stride) {
  const uint32_t tile = blockIdx.x, b = blockIdx.y, l = threadIdx.x;
  const uint32_t r = l & 15, g = l >> 4, row = tile * 16 + r;
  uint8_t* out = dst + ((size_t)(dst_tile0 + tile * tile_stride) * nb + b) * SH_Q8_TILE_BYTES;
  if (row < M) {
    const uint8_t* blk = src + ((size_t)row * nb + b) * 34;
    for (int t = 0; t < 8; ++t) out[8 * l + t] = blk[2 + 8 * g + t];
    if (g == 0) { out[512 + 2 * r] = blk[0]; out[513 + 2 * r] = blk[1]; }
  } else {
    for (int t = 0; t < 8; ++t) out[8 * l + t] = 0;
    if (g == 0) { out[512 + 2 * r] = 0; out[513 + 2 * r] = 0; }
  }
}

// ------------------------------------------------------------------ epilogue

__device__ __forceinline__ uint16_t f2h_bits(float x) { return __builtin_bit_cast(uint16_t, (_Float16)x); }

// Final (row, col) value for rows r0..r0+3 (one lane), col < N.
template <int EPI>
__device__ __forceinline__ void epilogue4(const EpiArgs& ea, uint32_t r0, uint32_t col, const float v[4]) {
  if (EPI == EPI_STORE) {
    for (int j = 0; j < 4; ++j)
      if (r0 + j < ea.rows) ea.out[(size_t)col * ea.ldo + r0 + j] = v[j];
  } else if (EPI == EPI_ADD) {
    for (int j = 0; j < 4; ++j) {
      if (r0 + j >= ea.rows) continue;
      float* p = ea.out + (size_t)col * ea.ldo + r0 + j;
      *p = *p + v[j];
    }
  } else if (EPI == EPI_QKV) {
    const int32_t pos = ea.colpos[col & 7];
    const uint32_t slot = ea.slot0 + col;
    if (r0 < ea.Dq) {
      const uint32_t i0 = r0 % ea.hd;
      const float2 cs0 = ea.rope[(size_t)pos * (ea.hd / 2) + i0 / 2];
      const float2 cs1 = ea.rope[(size_t)pos * (ea.hd / 2) + i0 / 2 + 1];
      float* q = ea.out + (size_t)col * ea.Dq + r0;
      q[0] = v[0] * cs0.x - v[1] * cs0.y;
      q[1] = v[0] * cs0.y + v[1] * cs0.x;
      q[2] = v[2] * cs1.x - v[3] * cs1.y;
      q[3] = v[2] * cs1.y + v[3] * cs1.x;
    } else if (r0 < ea.Dq + ea.Dkv) {
      const uint32_t rr = r0 - ea.Dq, kh = rr / ea.hd, i0 = rr % ea.hd;
      const float2 cs0 = ea.rope[(size_t)pos * (ea.hd / 2) + i0 / 2];
      const float2 cs1 = ea.rope[(size_t)pos * (ea.hd / 2) + i0 / 2 + 1];
      float o[4];
      o[0] = v[0] * cs0.x - v[1] * cs0.y;
      o[1] = v[0] * cs0.y + v[1] * cs0.x;
      o[2] = v[2] * cs1.x - v[3] * cs1.y;
      o[3] = v[2] * cs1.y + v[3] * cs1.x;
      uint16_t* k = ea.kc + (((size_t)ea.layer * ea.n_kv + kh) * ea.max_seq + slot) * ea.hd + i0;
      for (int j = 0; j < 4; ++j) k[j] = f2h_bits(o[j]);
    } else {
      const uint32_t rr = r0 - ea.Dq - ea.Dkv, kh = rr / ea.hd, i0 = rr % ea.hd;
      uint16_t* vb = ea.vc + (((size_t)ea.layer * ea.n_kv + kh) * (ea.max_seq / 32) + slot / 32) * ea.hd * 32;
      const uint32_t sl = v_slot(slot & 31);
      for (int j = 0; j < 4; ++j) vb[(size_t)(i0 + j) * 32 + sl] = f2h_bits(v[j]);
    }
  }
}

// ------------------------------------------------------------------ kernels

// One wave's operands for one 16-row tile and one 256-element superblock.
struct Q4Tile {
  u32x4 q0, q1, dd;
  uint32_t s0, s1, s2;
};

__device__ __forceinline__ Q4Tile load_q4_tile(const uint8_t* base, int lane, int g, int r) {
  Q4Tile a;
  a.q0 = ld16(base + 32 * lane);
  a.q1 = ld16(base + 32 * lane + 16);
  a.dd = ld16(base + 2048 + 16 * g);
  const uint32_t* sp = (const uint32_t*)(base + 2112 + 12 * r);
  a.s0 = sp[0];
  a.s1 = sp[1];
  a.s2 = sp[2];
  return a;
}

// (a & mask) | (b & ~mask) in one v_bfi_b32 (the mask lives in an SGPR; a
// VOP3 encoding cannot take two literal constants).
__device__ __forceinline__ uint32_t bfi(uint32_t mask, uint32_t a, uint32_t b) {
  uint32_t r;
  asm volatile("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "s"(mask), "v"(a), "v"(b));
  return r;
}

// Four f16 pairs from one repacked word w (pair i: t = 2i at bits 4i, t = 2i+1
// at bits 16+4i). Pairs 0 and 2 become 1024 + q, pairs 1 and 3 (nibbles in
// bits 4-7 of each half) 1024 + 16q; the activation operand carries a 1/16
// factor at those k (t % 4 >= 2), so one (mult, add) serves all four:
// (1024 + c q) sc - 1024 sc = c sc q exactly (single rounding of an exact value).
__device__ __forceinline__ h8 q4_operand2(uint32_t w, uint32_t magic, h2 mult, h2 add) {
  const uint32_t w8 = w >> 8;
  u32x4 r;
  r.x = as_u32(__builtin_elementwise_fma(as_h2(bfi(0x000F000Fu, w, magic)), mult, add));
  r.y = as_u32(__builtin_elementwise_fma(as_h2(bfi(0x00F000F0u, w, magic)), mult, add));
  r.z = as_u32(__builtin_elementwise_fma(as_h2(bfi(0x000F000Fu, w8, magic)), mult, add));
  r.w = as_u32(__builtin_elementwise_fma(as_h2(bfi(0x00F000F0u, w8, magic)), mult, add));
  return as_h8(r);
}

// f16 pair (1024 + byte_i, 1024 + byte_j) of a word of small integers:
// v_perm picks bytes of {magic, w}; selector 5 is magic's byte 1 (0x64).
__device__ __forceinline__ h2 magic_pair(uint32_t w, uint32_t magic, uint32_t i, uint32_t j) {
  return as_h2(__builtin_amdgcn_perm(magic, w, i | (5u << 8) | (j << 16) | (5u << 24)));
}

// y[j] += d * sum_s sc_s * q.x - dmin * sum_s m_s * xsum_s for rows 4g+j.
__device__ __forceinline__ void q4_tile_mma(const Q4Tile& a, const h8* bq, h8 bm, f4& y) {
  const uint32_t sc03 = a.s0 & 0x3F3F3F3Fu, m03 = a.s1 & 0x3F3F3F3Fu;
  const uint32_t sc47 = (a.s2 & 0x0F0F0F0Fu) | ((a.s0 >> 2) & 0x30303030u);
  const uint32_t m47 = ((a.s2 >> 4) & 0x0F0F0F0Fu) | ((a.s1 >> 2) & 0x30303030u);
  const uint32_t words[8] = {a.q0.x, a.q0.y, a.q0.z, a.q0.w, a.q1.x, a.q1.y, a.q1.z, a.q1.w};
  const uint32_t magic = __builtin_amdgcn_readfirstlane(0x64006400u);  // f16 1024 in both halves
  const h2 k1024 = {(_Float16)-1024.0f, (_Float16)-1024.0f};
  f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    const h2 mult = magic_pair(m < 4 ? sc03 : sc47, magic, m & 3, m & 3) + k1024;  // (sc, sc)
    const h2 add = mult * k1024;
    acc = mfma16(q4_operand2(words[m], magic, mult, add), bq[m], acc);
  }
  // Minimum term: A = m_s (every lane group holds the row's m, but B = XS is
  // zero outside lane group 0, so only k = s of group 0 contributes).
  u32x4 am;
  am.x = as_u32(magic_pair(m03, magic, 0, 1) + k1024);
  am.y = as_u32(magic_pair(m03, magic, 2, 3) + k1024);
  am.z = as_u32(magic_pair(m47, magic, 0, 1) + k1024);
  am.w = as_u32(magic_pair(m47, magic, 2, 3) + k1024);
  const f4 macc = mfma16(as_h8(am), bm, f4{0.f, 0.f, 0.f, 0.f});
  const uint32_t ddw[4] = {a.dd.x, a.dd.y, a.dd.z, a.dd.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float d = (float)as_h2(ddw[j]).x, dmin = (float)as_h2(ddw[j]).y;
    y[j] = y[j] + d * acc[j] - dmin * macc[j];
  }
}

// Q4_K GEMV, streaming form: a workgroup of GW = 8 waves owns T row tiles for
// all of K. Wave w walks superblocks b = w, w + 8, ... and, inside each, the T
// tiles (one activation operand load serves T weight tiles). The next unit's
// weights are always in flight while the current one computes, so a wave pays
// the HBM latency once, not once per unit. The 8 partial sums of each tile meet
// in LDS at the end; no state is shared between workgroups.
constexpr int GW = 8;
template <int T, int EPI>
__global__ __launch_bounds__(64 * GW) void k_gemv_q4s(const uint8_t* __restrict__ Wp, uint32_t tiles, uint32_t nsb,
                                                       const uint16_t* __restrict__ Bx,
                                                       const uint16_t* __restrict__ XS, uint32_t N, EpiArgs ea) {
  constexpr int CH = T < 4 ? T : 4;  // tiles reduced per LDS round
  __shared__ f4 red[CH][GW][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar address math
  const int g = lane >> 4, r = lane & 15;
  const uint32_t tile0 = blockIdx.x * T;
  f4 y[T];
#pragma unroll
  for (int t = 0; t < T; ++t) y[t] = f4{0.f, 0.f, 0.f, 0.f};
  auto a_ptr = [&](uint32_t t, uint32_t b) {
    const uint32_t tile = tile0 + t < tiles ? tile0 + t : tiles - 1;  // clamp keeps loads in bounds
    return Wp + ((size_t)tile * nsb + b) * SH_Q4K_TILE_BYTES;
  };
  // Units run (b, t) with t fastest; two tile buffers alternate so the unit
  // after the current one is always loading. Blocks of superblocks are taken in
  // pairs so each buffer's parity is a compile-time constant.
  const uint32_t nbw = (uint32_t)wave < nsb ? (nsb - 1 - wave) / GW + 1 : 0;
  Q4Tile st[2];
  h8 bq[8], bm;
  auto load_b = [&](uint32_t b) {
#pragma unroll
    for (int m = 0; m < 8; ++m) bq[m] = as_h8(ld16(Bx + ((size_t)(b * 8 + m) * 64 + lane) * 8));
    bm = as_h8(ld16(XS + ((size_t)b * 64 + lane) * 8));
  };
  if (nbw) st[0] = load_q4_tile(a_ptr(0, wave), lane, g, r);
  for (uint32_t i = 0; i < nbw; i += 2) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t bi = i + h;
      if (h == 1 && bi >= nbw) break;
      const uint32_t b = wave + GW * bi;
      load_b(b);
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const int par = (h * T + t) & 1;
        if (t + 1 < T) st[par ^ 1] = load_q4_tile(a_ptr(t + 1, b), lane, g, r);
        else if (bi + 1 < nbw) st[par ^ 1] = load_q4_tile(a_ptr(0, b + GW), lane, g, r);
        q4_tile_mma(st[par], bq, bm, y[t]);
      }
    }
  }
  // Tile partials meet in LDS, CH tiles per round; wave w < CH ends up holding
  // tile (round * CH + w), or with SwiGLU wave w < CH/2 holds the pair
  // (gate, up) = tiles (2w, 2w + 1) of the round.
  const float cs = ea.cs ? ea.cs[r & 7] : 1.0f;
#pragma unroll
  for (int c0 = 0; c0 < T; c0 += CH) {
#pragma unroll
    for (int i = 0; i < CH; ++i) red[i][wave][lane] = y[c0 + i];
    __syncthreads();
    if (EPI == EPI_SWIGLU) {
      if (wave < CH / 2) {
        f4 vg = {0.f, 0.f, 0.f, 0.f}, vu = {0.f, 0.f, 0.f, 0.f};
        for (int w = 0; w < GW; ++w) { vg += red[2 * wave][w][lane]; vu += red[2 * wave + 1][w][lane]; }
        float og[4], ou[4];
        for (int j = 0; j < 4; ++j) {
          og[j] = (vg[j] + __shfl_xor(vg[j], 8)) * cs;
          ou[j] = (vu[j] + __shfl_xor(vu[j], 8)) * cs;
        }
        const uint32_t tg = tile0 + c0 + 2 * wave;
        if (tg < tiles && r < 8 && (uint32_t)r < N) {
          const uint32_t row0 = (tg / 2) * 16 + 4 * g;
          for (int j = 0; j < 4; ++j) {
            const float x = og[j];
            ea.out[(size_t)r * ea.ldo + row0 + j] = (x / (1.0f + expf(-x))) * ou[j];
          }
        }
      }
    } else if (wave < CH) {
      f4 v = {0.f, 0.f, 0.f, 0.f};
      for (int w = 0; w < GW; ++w) v += red[wave][w][lane];
      float o[4];
      for (int j = 0; j < 4; ++j) o[j] = (v[j] + __shfl_xor(v[j], 8)) * cs;
      const uint32_t tile = tile0 + c0 + wave;
      if (tile < tiles && r < 8 && (uint32_t)r < N) epilogue4<EPI>(ea, tile * 16 + 4 * g, (uint32_t)r, o);
    }
    __syncthreads();
  }
}

// Q4_K GEMV: a workgroup of W waves owns R row tiles; wave w takes the
// superblocks b = w, w + W, ... and keeps the next superblock's weights and
// activation operand in flight while it computes the current one. The W
// partial sums meet in LDS; no state is shared between workgroups.
template <int R, int W, int EPI>
__global__ __launch_bounds__(64 * W) void k_gemv_q4k(const uint8_t* __restrict__ Wp, uint32_t tiles, uint32_t nsb,
                                                      const uint16_t* __restrict__ Bx,
                                                      const uint16_t* __restrict__ XS, uint32_t N, EpiArgs ea) {
  __shared__ f4 red[W][R][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const uint32_t tile0 = blockIdx.x * R;
  f4 y[R];
#pragma unroll
  for (int t = 0; t < R; ++t) y[t] = f4{0.f, 0.f, 0.f, 0.f};

  struct Stage {
    h8 bq[8];
    h8 bm;
    Q4Tile a[R];
  };
  auto load = [&](uint32_t b, Stage& st) {
#pragma unroll
    for (int m = 0; m < 8; ++m) st.bq[m] = as_h8(ld16(Bx + ((size_t)(b * 8 + m) * 64 + lane) * 8));
    st.bm = as_h8(ld16(XS + ((size_t)b * 64 + lane) * 8));
#pragma unroll
    for (int t = 0; t < R; ++t) {
      const uint32_t tile = tile0 + t < tiles ? tile0 + t : tiles - 1;  // clamp keeps loads in bounds
      st.a[t] = load_q4_tile(Wp + ((size_t)tile * nsb + b) * SH_Q4K_TILE_BYTES, lane, g, r);
    }
  };
  Stage cur, nxt;
  uint32_t b = wave;
  if (b < nsb) load(b, cur);
  for (; b < nsb; b += W) {
    const bool more = b + W < nsb;
    if (more) load(b + W, nxt);
#pragma unroll
    for (int t = 0; t < R; ++t) q4_tile_mma(cur.a[t], cur.bq, cur.bm, y[t]);
    if (more) cur = nxt;
  }

  if (W > 1) {
#pragma unroll
    for (int t = 0; t < R; ++t) red[wave][t][lane] = y[t];
    __syncthreads();
  }
  // undo the producer's per-column power-of-two activation scale (exact)
  const float cs = ea.cs ? ea.cs[r & 7] : 1.0f;
  if (EPI == EPI_SWIGLU) {
    if (wave >= R / 2) return;
    const int tg = 2 * wave, tu = 2 * wave + 1;
    f4 vg = {0.f, 0.f, 0.f, 0.f}, vu = {0.f, 0.f, 0.f, 0.f};
    if (W > 1) {
      for (int w = 0; w < W; ++w) { vg += red[w][tg][lane]; vu += red[w][tu][lane]; }
    } else {
      vg = y[tg]; vu = y[tu];
    }
    float og[4], ou[4];
    for (int j = 0; j < 4; ++j) {
      og[j] = (vg[j] + __shfl_xor(vg[j], 8)) * cs;
      ou[j] = (vu[j] + __shfl_xor(vu[j], 8)) * cs;
    }
    if (tile0 + tg >= tiles || r >= 8 || (uint32_t)r >= N) return;
    const uint32_t row0 = ((tile0 + tg) / 2) * 16 + 4 * g;
    for (int j = 0; j < 4; ++j) {
      const float x = og[j];
      ea.out[(size_t)r * ea.ldo + row0 + j] = (x / (1.0f + expf(-x))) * ou[j];
    }
    return;
  }
  if (wave >= R) return;
  const uint32_t tile = tile0 + wave;
  f4 v = {0.f, 0.f, 0.f, 0.f};
  if (W > 1) {
    for (int w = 0; w < W; ++w) v += red[w][wave][lane];
  } else {
    v = y[wave];
  }
  float o[4];
  for (int j = 0; j < 4; ++j) o[j] = (v[j] + __shfl_xor(v[j], 8)) * cs;
  if (tile >= tiles || r >= 8 || (uint32_t)r >= N) return;
  epilogue4<EPI>(ea, tile * 16 + 4 * g, (uint32_t)r, o);
}

template <int R, int W, int EPI>
__global__ __launch_bounds__(64 * W) void k_gemv_q8(const uint8_t* __restrict__ Wp, uint32_t tiles, uint32_t nb,
                                                     const uint16_t* __restrict__ Bx, uint32_t N, EpiArgs ea) {
  __shared__ f4 red[W][R][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const uint32_t tile0 = blockIdx.x * R;
  f4 y[R];
#pragma unroll
  for (int t = 0; t < R; ++t) y[t] = f4{0.f, 0.f, 0.f, 0.f};
  for (uint32_t b = wave; b < nb; b += W) {
    const h8 bq = as_h8(ld16(Bx + ((size_t)b * 64 + lane) * 8));
#pragma unroll
    for (int t = 0; t < R; ++t) {
      const uint32_t tile = tile0 + t;
      if (tile >= tiles) break;
      const uint8_t* base = Wp + ((size_t)tile * nb + b) * SH_Q8_TILE_BYTES;
      const uint2 qw = *(const uint2*)(base + 8 * lane);
      const uint2 dw = *(const uint2*)(base + 512 + 8 * g);
      const f4 acc = mfma16(q8_operand(qw.x, qw.y), bq, f4{0.f, 0.f, 0.f, 0.f});
      const float d[4] = {(float)as_h2(dw.x).x, (float)as_h2(dw.x).y, (float)as_h2(dw.y).x,
                          (float)as_h2(dw.y).y};
#pragma unroll
      for (int j = 0; j < 4; ++j) y[t][j] = y[t][j] + d[j] * acc[j];
    }
  }
  if (W > 1) {
#pragma unroll
    for (int t = 0; t < R; ++t) red[wave][t][lane] = y[t];
    __syncthreads();
  }
  // undo the producer's per-column power-of-two activation scale (exact)
  const float cs = ea.cs ? ea.cs[r & 7] : 1.0f;
  if (EPI == EPI_SWIGLU) {
    if (wave >= R / 2) return;
    const int tg = 2 * wave, tu = 2 * wave + 1;
    f4 vg = {0.f, 0.f, 0.f, 0.f}, vu = {0.f, 0.f, 0.f, 0.f};
    if (W > 1) {
      for (int w = 0; w < W; ++w) { vg += red[w][tg][lane]; vu += red[w][tu][lane]; }
    } else {
      vg = y[tg]; vu = y[tu];
    }
    float og[4], ou[4];
    for (int j = 0; j < 4; ++j) {
      og[j] = (vg[j] + __shfl_xor(vg[j], 8)) * cs;
      ou[j] = (vu[j] + __shfl_xor(vu[j], 8)) * cs;
    }
    const uint32_t pair = (tile0 + tg) / 2;
    if (tile0 + tg >= tiles || r >= 8 || (uint32_t)r >= N) return;
    const uint32_t row0 = pair * 16 + 4 * g;
    for (int j = 0; j < 4; ++j) {
      const float x = og[j];
      ea.out[(size_t)r * ea.ldo + row0 + j] = (x / (1.0f + expf(-x))) * ou[j];
    }
    return;
  }
  if (wave >= R) return;
  const uint32_t tile = tile0 + wave;
  f4 v = {0.f, 0.f, 0.f, 0.f};
  if (W > 1) {
    for (int w = 0; w < W; ++w) v += red[w][wave][lane];
  } else {
    v = y[wave];
  }
  float o[4];
  for (int j = 0; j < 4; ++j) o[j] = (v[j] + __shfl_xor(v[j], 8)) * cs;
  if (tile >= tiles || r >= 8 || (uint32_t)r >= N) return;
  epilogue4<EPI>(ea, tile * 16 + 4 * g, (uint32_t)r, o);
}

// ------------------------------------------------------------------ host side

void sh_qmat_free(QMat* m) {
  if (m->d) (void)hipFree(m->d);
  m->d = nullptr;
}

static size_t qrow_bytes(int type, uint32_t K) { return type == GGML_Q4_K ? K / 256 * 144 : K / 32 * 34; }

// Upload nparts row-blocks (each a GGUF [rows][K] matrix) as one packed matrix
// with rows concatenated. Each part's row count must be a multiple of 16.
int sh_repack_upload_cat(sh_engine* e, int type, const uint8_t* const* parts, const uint32_t* rows, int nparts,
                         uint32_t K, QMat* out) {
  SH_CHECK(type == GGML_Q4_K || type == GGML_Q8_0, SH_ERR_UNSUPPORTED,
           "weight type %d not supported (Q4_K=12, Q8_0=8)", type);
  SH_CHECK(K % (type == GGML_Q4_K ? 256 : 32) == 0, SH_ERR_FORMAT, "K=%u not a multiple of the block", K);
  uint32_t M = 0;
  for (int i = 0; i < nparts; ++i) {
    SH_CHECK(nparts == 1 || rows[i] % 16 == 0, SH_ERR_UNSUPPORTED, "concatenated part rows %u %% 16", rows[i]);
    M += rows[i];
  }
  const uint32_t nblk = type == GGML_Q4_K ? K / 256 : K / 32;
  const uint32_t tb = type == GGML_Q4_K ? SH_Q4K_TILE_BYTES : SH_Q8_TILE_BYTES;
  QMat m;
  m.type = type; m.M = M; m.K = K; m.tiles = (M + 15) / 16;
  m.bytes = (size_t)m.tiles * nblk * tb;
  m.alg_bytes = (double)M * qrow_bytes(type, K);
  SH_HIP(hipMalloc(&m.d, m.bytes));
  uint32_t tile0 = 0;
  for (int i = 0; i < nparts; ++i) {
    const size_t bytes = (size_t)rows[i] * qrow_bytes(type, K);
    uint8_t* tmp = nullptr;
    SH_HIP(hipMalloc(&tmp, bytes));
    SH_HIP(hipMemcpyAsync(tmp, parts[i], bytes, hipMemcpyHostToDevice, e->stream));
    const uint32_t ptiles = (rows[i] + 15) / 16;
    dim3 grid(ptiles, nblk);
    if (type == GGML_Q4_K)
      hipLaunchKernelGGL(k_repack_q4k, grid, dim3(64), 0, e->stream, tmp, m.d, rows[i], nblk, tile0, 1u);
    else
      hipLaunchKernelGGL(k_repack_q8, grid, dim3(64), 0, e->stream, tmp, m.d, rows[i], nblk, tile0, 1u);
    SH_HIP(hipGetLastError());
    SH_HIP(hipStreamSynchronize(e->stream));
    SH_HIP(hipFree(tmp));
    tile0 += ptiles;
  }
  *out = m;
  return SH_OK;
}

int sh_repack_upload(sh_engine* e, int type, const uint8_t* host, uint32_t M, uint32_t K, QMat* out) {
  return sh_repack_upload_cat(e, type, &host, &M, 1, K, out);
}

// gate/up: tile t of gate -> packed tile 2t, tile t of up -> 2t+1.
int sh_repack_upload_gu(sh_engine* e, int type, const uint8_t* gate, const uint8_t* up, uint32_t M, uint32_t K,
                        QMat* out) {
  SH_CHECK(type == GGML_Q4_K || type == GGML_Q8_0, SH_ERR_UNSUPPORTED, "weight type %d not supported", type);
  SH_CHECK(M % 32 == 0, SH_ERR_UNSUPPORTED, "n_ff=%u must be a multiple of 32", M);
  const uint32_t nblk = type == GGML_Q4_K ? K / 256 : K / 32;
  const uint32_t tb = type == GGML_Q4_K ? SH_Q4K_TILE_BYTES : SH_Q8_TILE_BYTES;
  QMat m;
  m.type = type; m.M = 2 * M; m.K = K; m.tiles = 2 * (M / 16);
  m.bytes = (size_t)m.tiles * nblk * tb;
  m.alg_bytes = 2.0 * M * qrow_bytes(type, K);
  SH_HIP(hipMalloc(&m.d, m.bytes));
  const size_t bytes = (size_t)M * qrow_bytes(type, K);
  uint8_t* tmp = nullptr;
  SH_HIP(hipMalloc(&tmp, bytes));
  for (int part = 0; part < 2; ++part) {
    SH_HIP(hipMemcpyAsync(tmp, part ? up : gate, bytes, hipMemcpyHostToDevice, e->stream));
    dim3 grid(M / 16, nblk);
    if (type == GGML_Q4_K)
      hipLaunchKernelGGL(k_repack_q4k, grid, dim3(64), 0, e->stream, tmp, m.d, M, nblk, (uint32_t)part, 2u);
    else
      hipLaunchKernelGGL(k_repack_q8, grid, dim3(64), 0, e->stream, tmp, m.d, M, nblk, (uint32_t)part, 2u);
    SH_HIP(hipGetLastError());
    SH_HIP(hipStreamSynchronize(e->stream));
  }
  SH_HIP(hipFree(tmp));
  *out = m;
  return SH_OK;
}

template <int R, int W, int EPI>
static int launch_q4k(sh_engine* e, const QMat& w, const uint16_t* bx, const uint16_t* xs, uint32_t N,
                      const EpiArgs& ea) {
  const uint32_t grid = (w.tiles + R - 1) / R;
  hipLaunchKernelGGL((k_gemv_q4k<R, W, EPI>), dim3(grid), dim3(64 * W), 0, e->stream, w.d, w.tiles, w.K / 256, bx,
                     xs, N, ea);
  return SH_OK;
}
template <int R, int W, int EPI>
static void launch_q8(sh_engine* e, const QMat& w, const uint16_t* bx, uint32_t N, const EpiArgs& ea) {
  const uint32_t grid = (w.tiles + R - 1) / R;
  hipLaunchKernelGGL((k_gemv_q8<R, W, EPI>), dim3(grid), dim3(64 * W), 0, e->stream, w.d, w.tiles, w.K / 32, bx, N,
                     ea);
}

// Shape policy: keep ~1000+ waves in flight. Small-M matrices use one tile per
// workgroup and 8 waves splitting K; large-M ones share each activation stage
// across 2-4 tiles per wave; gate/up waves own (gate, up) tile pairs.
template <int EPI>
static int dispatch_q4k_blocked(sh_engine* e, const QMat& w, const uint16_t* bx, const uint16_t* xs, uint32_t N,
                                const EpiArgs& ea) {
  if (EPI == EPI_SWIGLU) return launch_q4k<2, 8, EPI>(e, w, bx, xs, N, ea);
  if (w.tiles >= 1024) return launch_q4k<2, 4, EPI>(e, w, bx, xs, N, ea);
  return launch_q4k<1, 8, EPI>(e, w, bx, xs, N, ea);
}

template <int T, int EPI>
static int launch_q4s(sh_engine* e, const QMat& w, const uint16_t* bx, const uint16_t* xs, uint32_t N,
                      const EpiArgs& ea) {
  const uint32_t grid = (w.tiles + T - 1) / T;
  hipLaunchKernelGGL((k_gemv_q4s<T, EPI>), dim3(grid), dim3(64 * GW), 0, e->stream, w.d, w.tiles, w.K / 256, bx, xs,
                     N, ea);
  return SH_OK;
}

// Tuning overrides (read once): SH_GEMV_KERNEL=blocked|stream, SH_GEMV_T=1..16.
static int gemv_kernel_choice() {
  static int v = [] {
    const char* s = getenv("SH_GEMV_KERNEL");
    return (s && std::string(s) == "blocked") ? 1 : 0;
  }();
  return v;
}
static uint32_t gemv_t_override() {
  static uint32_t v = [] {
    const char* s = getenv("SH_GEMV_T");
    return s ? (uint32_t)atoi(s) : 0u;
  }();
  return v;
}

// Streaming policy: about 512 workgroups of 8 waves (two per CU), i.e. T =
// tiles / 512 rounded down to a power of two in [1, 16] (even for SwiGLU so a
// workgroup owns whole gate/up pairs).
template <int EPI>
static int dispatch_q4k(sh_engine* e, const QMat& w, const uint16_t* bx, const uint16_t* xs, uint32_t N,
                        const EpiArgs& ea) {
  if (gemv_kernel_choice() == 1) return dispatch_q4k_blocked<EPI>(e, w, bx, xs, N, ea);
  uint32_t t = gemv_t_override();
  if (!t) {
    t = 1;
    while (t < 8 && w.tiles / (2 * t) >= 512) t *= 2;
  }
  if (EPI == EPI_SWIGLU && t < 2) t = 2;
  switch (t) {
    case 1: return launch_q4s<1, EPI>(e, w, bx, xs, N, ea);
    case 2: return launch_q4s<2, EPI>(e, w, bx, xs, N, ea);
    case 4: return launch_q4s<4, EPI>(e, w, bx, xs, N, ea);
    default: return launch_q4s<8, EPI>(e, w, bx, xs, N, ea);
  }
}
template <int EPI>
static void dispatch_q8(sh_engine* e, const QMat& w, const uint16_t* bx, uint32_t N, const EpiArgs& ea) {
  if (EPI == EPI_SWIGLU) launch_q8<2, 4, EPI>(e, w, bx, N, ea);
  else if (w.tiles >= 1024) launch_q8<2, 4, EPI>(e, w, bx, N, ea);
  else launch_q8<1, 4, EPI>(e, w, bx, N, ea);
}

int sh_gemv_launch(sh_engine* e, const QMat& w, const uint16_t* bx, const uint16_t* xs, uint32_t N, EpiKind epi,
                   const EpiArgs& ea, const char* tag) {
  SH_CHECK(N >= 1 && N <= 8, SH_ERR_ARG, "gemv chunk N=%u outside [1,8]", N);
  hipEvent_t ev = nullptr;
  sh_prof_begin(e, &ev);
  if (w.type == GGML_Q4_K) {
    int rc = SH_OK;
    switch (epi) {
      case EPI_STORE: rc = dispatch_q4k<EPI_STORE>(e, w, bx, xs, N, ea); break;
      case EPI_ADD: rc = dispatch_q4k<EPI_ADD>(e, w, bx, xs, N, ea); break;
      case EPI_QKV: rc = dispatch_q4k<EPI_QKV>(e, w, bx, xs, N, ea); break;
      case EPI_SWIGLU: rc = dispatch_q4k<EPI_SWIGLU>(e, w, bx, xs, N, ea); break;
    }
    if (rc) return rc;
  } else if (w.type == GGML_Q8_0) {
    switch (epi) {
      case EPI_STORE: dispatch_q8<EPI_STORE>(e, w, bx, N, ea); break;
      case EPI_ADD: dispatch_q8<EPI_ADD>(e, w, bx, N, ea); break;
      case EPI_QKV: dispatch_q8<EPI_QKV>(e, w, bx, N, ea); break;
      case EPI_SWIGLU: dispatch_q8<EPI_SWIGLU>(e, w, bx, N, ea); break;
    }
  } else {
    SH_CHECK(false, SH_ERR_UNSUPPORTED, "gemv: weight type %d", w.type);
  }
  SH_HIP(hipGetLastError());
  sh_prof_end(e, tag, w.alg_bytes, ev);
  return SH_OK;
}
