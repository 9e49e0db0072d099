// Quantized GEMV for the verify step: y[j][m] = sum_k deq(W)[m][k] * x[j][k]
// for N <= 8 columns per launch chunk, on gfx950 MFMA.
//
// Semantics: the reference's batched-column matvec (ops/matmul.rs:473-487,
// shaders/compute/mul_mat_vec_q4_k.slang:13-103 for Q4_K, mul_mat_vec.slang:39-100
// for Q8_0), which dequantizes each weight row once and reuses it for all N
// columns. Design here (not a translation):
//   * Weights are repacked once at upload into 16-row tiles so each lane of a
//     wave64 reads its MFMA A-operand bytes with two 16-byte loads.
//   * Q4_K nibbles become exact f16 integers c*sc*q (c = 1 or 16) via the
//     0x6400 magic exponent and one packed FMA; d and dmin are applied per
//     256-superblock in f32.
//   * Activations are split x = hi + lo (two f16) and fed as 16 MFMA columns
//     (8 hi + 8 lo), so v_mfma_f32_16x16x32_f16 keeps ~22 bits of x and f32
//     accumulation at no extra MFMA cost for N <= 8. Each superblock of each
//     column carries its own power-of-two scale (cs), undone per superblock.
//   * The Q4_K minimum term dmin * sum_s m_s * sum(x in s) is a ninth MFMA per
//     superblock against per-sub-block column sums (XS).
//   * Two Q4_K kernels: "wide" (8 waves own 8T different row tiles over one
//     K-split whose activation operand sits in LDS, loaded once by direct
//     global->LDS loads and read by all 8 waves; split-K partial sums are
//     finished by the consumer) and "stream" (one workgroup owns T tiles over
//     all of K, its 8 waves split K; for epilogues that need whole sums).
#include <cstdlib>
#include <string>

#include <type_traits>

#include "sh_internal.h"
#include "sh_coherent.h"
#include "sh_dma.h"
#include "sh_operand.h"

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void glb_void_t;

struct alignas(16) u32x4 { uint32_t x, y, z, w; };

// An opaque use of loaded registers: the compiler must finish their loads
// here. The double-buffered GEMMs pin the first tile before their loop: the
// compiler may sink those loads below the preamble's wait, and at the loop
// head, after the asm stage loads it cannot count, it would then wait for
// every load in flight (the prefetch included) before the first use.
__device__ __forceinline__ void pin32(uint32_t& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void pin32(u32x4& v) { pin32(v.x); pin32(v.y); pin32(v.z); pin32(v.w); }
__device__ __forceinline__ void pin32(uint2& v) { pin32(v.x); pin32(v.y); }

__device__ __forceinline__ h2 as_h2(uint32_t v) { return __builtin_bit_cast(h2, v); }
__device__ __forceinline__ uint32_t as_u32(h2 v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ h8 as_h8(u32x4 v) { return __builtin_bit_cast(h8, v); }
__device__ __forceinline__ u32x4 ld16(const void* p) { return *(const u32x4*)p; }

__device__ __forceinline__ f4 mfma16(h8 a, h8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// int8 pairs -> f16 exact: (q ^ 0x80) + 1024 as f16, minus 1152. The
// activation operand carries a 1/16 factor at k with k % 4 >= 2, so those
// pairs become 16 q = 16 (1024 + u) - 18432, still exact.
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

// Q4_K tile-superblock (2304 B): [0,2048) 8 words per lane, words 0-3 of lane l
// at 16 l and words 4-7 at 1024 + 16 l (each 16-byte load of a wave reads 1 KB
// contiguous); lane l (row l%16,
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
  uint32_t* o = (uint32_t*)(out + 16 * l);
  for (int m = 0; m < 4; ++m) o[m] = words[m];
  o = (uint32_t*)(out + 1024 + 16 * l);
  for (int m = 0; m < 4; ++m) o[m] = words[4 + m];
}

// Nibble word m of lane (row, group g) in the Q4_K tile layout from a row's
// 128 packed nibble bytes: element 32 m + 8 g + t is (qs[32 (m / 2) + 8 g + t]
// >> 4 (m % 2)) & 15 (the Q4_K / Q5_K low nibbles; Q6_K maps its quarters onto
// this with its own byte offsets).
__device__ __forceinline__ uint32_t nibble_word(const uint8_t* qs, uint32_t byte0, uint32_t shift) {
  uint32_t w = 0;
  for (int t = 0; t < 8; ++t) {
    const uint32_t q = (qs[byte0 + t] >> shift) & 0xF;
    w |= q << ((t & 1) ? 16 + 4 * (t >> 1) : 4 * (t >> 1));
  }
  return w;
}

// Position, relative to its sub-block's base bit, of the high bits of element
// t of a lane's 8 in the repacked high-bit words: t0 0, t1 16, t2 4, t3 20,
// t4 X, t5 16 + X, t6 4 + X, t7 20 + X, with X = 1 for Q5_K (one bit per
// element) and X = 2 for Q6_K (two bits, at the position and the one above).
// Shifting the word so the base lands on bit 4 puts t0 / t1 on bits 4 / 20 and
// t2 / t3 on 8 / 24, right above the nibbles of the f16 pairs (t0, t1) (nibbles
// at bits 0 / 16) and (t2, t3) (nibbles at 4 / 20); shifting by X less does the
// same for t4..t7.
__device__ __forceinline__ uint32_t hbit_pos(int t, int X) {
  return 16 * (t & 1) + 4 * ((t >> 1) & 1) + X * ((t >> 2) & 1);
}

// Q5_K tile-superblock (2816 B): [0,2048) the low-nibble words as in Q4_K;
// [2048,2560) two high-bit words per lane at 2048 + 8 l, word h holding
// sub-blocks 4h..4h+3 at bases 0, 2, 8, 10 (element t of sub-block m: bit
// base(m) + hbit_pos(t, 1)); [2560,2624) d|dmin<<16 per row; [2624,2816) the 12
// scale bytes per row. GGUF block_q5_K (176 B): d, dmin, scales[12], qh[32],
// qs[128]; element 32 m + p: low nibble as Q4_K, fifth bit (qh[p] >> m) & 1.
__global__ void k_repack_q5k(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, uint32_t M,
                             uint32_t nsb, uint32_t dst_tile0, uint32_t tile_stride) {
  const uint32_t tile = blockIdx.x, sb = blockIdx.y, l = threadIdx.x;
  const uint32_t r = l & 15, g = l >> 4, row = tile * 16 + r;
  uint8_t* out = dst + ((size_t)(dst_tile0 + tile * tile_stride) * nsb + sb) * SH_Q5K_TILE_BYTES;
  uint32_t words[8] = {0, 0, 0, 0, 0, 0, 0, 0}, hw[2] = {0, 0};
  if (row < M) {
    const uint8_t* blk = src + ((size_t)row * nsb + sb) * 176;
    const uint8_t* qh = blk + 16;
    const uint8_t* qs = blk + 48;
    for (int m = 0; m < 8; ++m) {
      words[m] = nibble_word(qs, 32 * (m >> 1) + 8 * g, 4 * (m & 1));
      const uint32_t base = (m & 1) * 2 + ((m >> 1) & 1) * 8;
      for (int t = 0; t < 8; ++t) hw[m >> 2] |= ((qh[8 * g + t] >> m) & 1u) << (base + hbit_pos(t, 1));
    }
  }
  if (g == 0) {
    uint32_t dd = 0;
    uint8_t sc[12] = {0};
    if (row < M) {
      const uint8_t* blk = src + ((size_t)row * nsb + sb) * 176;
      dd = blk[0] | (blk[1] << 8) | (blk[2] << 16) | ((uint32_t)blk[3] << 24);
      for (int i = 0; i < 12; ++i) sc[i] = blk[4 + i];
    }
    *(uint32_t*)(out + 2560 + 4 * r) = dd;
    for (int i = 0; i < 12; ++i) out[2624 + 12 * r + i] = sc[i];
  }
  uint32_t* o = (uint32_t*)(out + 16 * l);
  for (int m = 0; m < 4; ++m) o[m] = words[m];
  o = (uint32_t*)(out + 1024 + 16 * l);
  for (int m = 0; m < 4; ++m) o[m] = words[4 + m];
  o = (uint32_t*)(out + 2048 + 8 * l);
  o[0] = hw[0];
  o[1] = hw[1];
}

// Q6_K tile-superblock (3360 B): [0,2048) the low-nibble words in the Q4_K
// layout; [2048,3072) four high-bit words per lane at 2048 + 16 l, word h
// holding sub-blocks 2h, 2h + 1 at bases 0, 8 (element t: two bits at base +
// hbit_pos(t, 2)); [3072,3328) per
// row 16 int8 scales, the even-indexed 8 then the odd-indexed 8 (lane group g
// reads its 8: scale 2 m + g / 2 for sub-block m); [3328,3360) f16 d per row.
// GGUF block_q6_K (210 B): ql[128], qh[64], scales[16], d; element
// 128 n + 32 s + p: (ql[64 n + 32 (s & 1) + p] >> 4 (s >> 1)) & 15 |
// ((qh[32 n + p] >> 2 s) & 3) << 4, value d * scales[e / 16] * (q - 32).
__global__ void k_repack_q6k(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, uint32_t M,
                             uint32_t nsb, uint32_t dst_tile0, uint32_t tile_stride) {
  const uint32_t tile = blockIdx.x, sb = blockIdx.y, l = threadIdx.x;
  const uint32_t r = l & 15, g = l >> 4, row = tile * 16 + r;
  uint8_t* out = dst + ((size_t)(dst_tile0 + tile * tile_stride) * nsb + sb) * SH_Q6K_TILE_BYTES;
  uint32_t words[8] = {0, 0, 0, 0, 0, 0, 0, 0}, hw[4] = {0, 0, 0, 0};
  const uint8_t* blk = src + ((size_t)(row < M ? row : 0) * nsb + sb) * 210;
  if (row < M) {
    const uint8_t* ql = blk;
    const uint8_t* qh = blk + 128;
    for (int m = 0; m < 8; ++m) {
      const uint32_t n = m >> 2, s = m & 3;
      words[m] = nibble_word(ql, 64 * n + 32 * (s & 1) + 8 * g, 4 * (s >> 1));
      const uint32_t base = 8 * (m & 1);
      for (int t = 0; t < 8; ++t)
        hw[m >> 1] |= ((qh[32 * n + 8 * g + t] >> (2 * s)) & 3u) << (base + hbit_pos(t, 2));
    }
  }
  if (g == 0) {
    const int8_t* sc = (const int8_t*)(blk + 192);
    for (int i = 0; i < 8; ++i) {
      out[3072 + 16 * r + i] = row < M ? (uint8_t)sc[2 * i] : 0;
      out[3072 + 16 * r + 8 + i] = row < M ? (uint8_t)sc[2 * i + 1] : 0;
    }
    out[3328 + 2 * r] = row < M ? blk[208] : 0;
    out[3329 + 2 * r] = row < M ? blk[209] : 0;
  }
  uint32_t* o = (uint32_t*)(out + 16 * l);
  for (int m = 0; m < 4; ++m) o[m] = words[m];
  o = (uint32_t*)(out + 1024 + 16 * l);
  for (int m = 0; m < 4; ++m) o[m] = words[4 + m];
  o = (uint32_t*)(out + 2048 + 16 * l);
  for (int m = 0; m < 4; ++m) o[m] = hw[m];
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

// Rows r0..r0+3 of one column's fused QKV output: q rows are roped into
// qcol, k rows roped and v rows stored as f16 in the column's cache slot
// (V slot-permuted within its 32-key block).
__device__ __forceinline__ void qkv_store4(const EpiArgs& ea, uint32_t r0, const float v[4], int32_t pos,
                                           uint32_t slot, uint32_t ms, uint16_t* kc, uint16_t* vc, float* qcol) {
  if (r0 < ea.Dq) {
    const uint32_t i0 = r0 % ea.hd;
    const float2 cs0 = ea.rope[(size_t)pos * (ea.hd / 2) + i0 / 2];
    const float2 cs1 = ea.rope[(size_t)pos * (ea.hd / 2) + i0 / 2 + 1];
    float* q = qcol + r0;
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
    uint16_t* k = kc + (((size_t)ea.layer * ea.n_kv + kh) * ms + slot) * ea.hd + i0;
    for (int j = 0; j < 4; ++j) k[j] = f2h_bits(o[j]);
  } else {
    const uint32_t rr = r0 - ea.Dq - ea.Dkv, kh = rr / ea.hd, i0 = rr % ea.hd;
    uint16_t* vb = vc + (((size_t)ea.layer * ea.n_kv + kh) * (ms / 32) + slot / 32) * ea.hd * 32;
    const uint32_t sl = v_slot(slot & 31);
    for (int j = 0; j < 4; ++j) vb[(size_t)(i0 + j) * 32 + sl] = f2h_bits(v[j]);
  }
}

// Final (row, col) value for rows r0..r0+3 (one lane), col < N; ks = split.
template <int EPI>
__device__ __forceinline__ void epilogue4(const EpiArgs& ea, uint32_t r0, uint32_t col, const float v[4],
                                          uint32_t ks = 0) {
  if (EPI == EPI_PART) {
    *(float4*)(ea.out + ks * ea.part_stride + (size_t)col * ea.ldo + r0) = make_float4(v[0], v[1], v[2], v[3]);
  } else if (EPI == EPI_STORE) {
    for (int j = 0; j < 4; ++j)
      if (r0 + j < ea.rows) ea.out[(size_t)col * ea.ldo + r0 + j] = v[j];
  } else if (EPI == EPI_ADD) {
    for (int j = 0; j < 4; ++j) {
      if (r0 + j >= ea.rows) continue;
      float* p = ea.out + (size_t)col * ea.ldo + r0 + j;
      *p = *p + v[j];
    }
  } else if (EPI == EPI_QKV) {
    const uint32_t base = ea.dbase ? *ea.dbase : 0u;
    qkv_store4(ea, r0, v, ea.colpos[col & 7] + (int32_t)base, ea.slot[col & 7] + base, ea.mseq[col & 7],
               ea.kc[col & 7], ea.vc[col & 7], ea.out + (size_t)col * ea.Dq);
  }
}

// SwiGLU of a (gate, up) tile pair: h[col][16 pair + 4g + j] = silu(g) * u.
__device__ __forceinline__ void swiglu4(const EpiArgs& ea, uint32_t pair, uint32_t g, uint32_t col, const float og[4],
                                        const float ou[4]) {
  const uint32_t row0 = pair * 16 + 4 * g;
  for (int j = 0; j < 4; ++j) {
    const float x = og[j];
    ea.out[(size_t)col * ea.ldo + row0 + j] = (x / (1.0f + expf(-x))) * ou[j];
  }
}

// ------------------------------------------------------------------ Q4_K core

// One wave's operands for one 16-row tile and one 256-element superblock.
struct Q4Tile {
  u32x4 q0, q1, dd;
  uint32_t s0, s1, s2;
  __device__ void pin() { pin32(q0); pin32(q1); pin32(dd); pin32(s0); pin32(s1); pin32(s2); }
};

// Weight loads are non-temporal (the `nt` hint): every weight byte is read
// once per forward, and the hint keeps the stream from displacing what is read
// again (K/V, operands) in the caches. Measured on the box: the 8B gate/up
// 21.95 -> 21.5 us per launch, the spec step 6.36 -> 6.33 ms, a 512 MB stream
// 94 -> 88 us.
__device__ __forceinline__ u32x4 ldw16(const uint8_t* p) {
  typedef uint32_t u4 __attribute__((ext_vector_type(4)));
  const u4 v = __builtin_nontemporal_load((const u4*)p);
  return u32x4{v[0], v[1], v[2], v[3]};
}
__device__ __forceinline__ uint32_t ldw4(const uint8_t* p) { return __builtin_nontemporal_load((const uint32_t*)p); }
__device__ __forceinline__ Q4Tile load_q4_tile(const uint8_t* base, int lane, int g, int r) {
  Q4Tile a;
  a.q0 = ldw16(base + 16 * lane);
  a.q1 = ldw16(base + 1024 + 16 * lane);
  a.dd = ldw16(base + 2048 + 16 * g);
  const uint8_t* sp = base + 2112 + 12 * r;
  a.s0 = ldw4(sp);
  a.s1 = ldw4(sp + 4);
  a.s2 = ldw4(sp + 8);
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
// factor at those k (k % 4 >= 2), so one (mult, add) serves all four:
// (1024 + c q) sc - 1024 sc = c sc q exactly (single rounding of an exact value).
// `magic` holds f16 1024 in both halves.
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

// y[j] += c * (d * sum_s sc_s * q.x - dmin * sum_s m_s * xsum_s) for rows 4g+j,
// where c undoes the column's activation scale for this superblock.
__device__ __forceinline__ void q4_tile_mma(const Q4Tile& a, const h8* bq, h8 bm, float c, f4& y) {
  const uint32_t sc03 = a.s0 & 0x3F3F3F3Fu, m03 = a.s1 & 0x3F3F3F3Fu;
  const uint32_t sc47 = (a.s2 & 0x0F0F0F0Fu) | ((a.s0 >> 2) & 0x30303030u);
  const uint32_t m47 = ((a.s2 >> 4) & 0x0F0F0F0Fu) | ((a.s1 >> 2) & 0x30303030u);
  const uint32_t words[8] = {a.q0.x, a.q0.y, a.q0.z, a.q0.w, a.q1.x, a.q1.y, a.q1.z, a.q1.w};
  const uint32_t magic = __builtin_amdgcn_readfirstlane(0x64006400u);
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
    y[j] = y[j] + c * (d * acc[j] - dmin * macc[j]);
  }
}

// RMSNorm factor of activation column col, rsqrt(mean(x^2) + eps), from the
// prep's per-superblock sums of squares (added in superblock order); 1 when the
// input is not normalized.
// Called at kernel start so its loads (8 in flight at a time) overlap the weights.
__device__ __forceinline__ float col_rinv(const EpiArgs& ea, uint32_t col) {
  if (!ea.ssq) return 1.0f;
  float ss = 0.f;
  for (uint32_t i0 = 0; i0 < ea.ssq_n; i0 += 8) {
    float t[8];
#pragma unroll
    for (uint32_t j = 0; j < 8; ++j) t[j] = ea.ssq[min(i0 + j, ea.ssq_n - 1) * 8 + col];
#pragma unroll
    for (uint32_t j = 0; j < 8; ++j) ss += i0 + j < ea.ssq_n ? t[j] : 0.0f;
  }
  return 1.0f / sqrtf(ss / (float)ea.norm_K + ea.eps);
}

// The same factor in two steps, so its loads overlap the weights instead of
// delaying them: col_ssq_load at kernel start (the column's first SSQ_PRE
// superblock sums of squares into registers), col_ssq_rinv after the main loop
// (adds them in superblock order, reading any further ones then). Same result
// as col_rinv, bit for bit.
constexpr uint32_t SSQ_PRE = 16;
__device__ __forceinline__ void col_ssq_load(const EpiArgs& ea, uint32_t col, float (&t)[SSQ_PRE]) {
  if (!ea.ssq) return;
#pragma unroll
  for (uint32_t j = 0; j < SSQ_PRE; ++j) t[j] = ea.ssq[min(j, ea.ssq_n - 1) * 8 + col];
}
__device__ __forceinline__ float col_ssq_rinv(const EpiArgs& ea, uint32_t col, float (&t)[SSQ_PRE]) {
  if (!ea.ssq) return 1.0f;
  // opaque here, so the compiler cannot start the sum (and wait on the loads)
  // before the main loop
#pragma unroll
  for (uint32_t j = 0; j < SSQ_PRE; ++j) asm volatile("" : "+v"(t[j]));
  float ss = 0.f;
#pragma unroll
  for (uint32_t j = 0; j < SSQ_PRE; ++j) ss += j < ea.ssq_n ? t[j] : 0.0f;
  for (uint32_t i = SSQ_PRE; i < ea.ssq_n; ++i) ss += ea.ssq[i * 8 + col];
  return 1.0f / sqrtf(ss / (float)ea.norm_K + ea.eps);
}

// Row sums for one lane after the MFMA loop: the hi and lo columns (c, c + 8)
// of the same activation column meet (lane l ^ 8 through DPP row_ror:8),
// times the column's norm factor f. Every lane must call this.
__device__ __forceinline__ void col_sum4(const f4& v, float f, float o[4]) {
  constexpr int ROW_ROR8 = 0x128;
#pragma unroll
  for (int j = 0; j < 4; ++j) o[j] = (v[j] + sh_dpp<ROW_ROR8>(v[j])) * f;
}

// ------------------------------------------------------------------ Q4_K wide

// Workgroup = WV waves; wave w owns row tiles (blockIdx.x * WV + w) * T + t over
// the S superblocks [S * blockIdx.y, S * blockIdx.y + S) of split blockIdx.y. The
// split's activation operand (S superblocks of B and XS, 9 KB each) is copied
// to LDS once with direct global->LDS loads and read there by all waves. A
// wave's S * T weight units (superblock, tile) run as straight-line code with D
// units in flight. No state is shared between workgroups: a split writes its
// partial sums (EPI_PART), or with one split the workgroup finishes the rows.
constexpr int WV = 8;
constexpr uint32_t WIDE_MAX_SB = 7;      // superblocks per split held in LDS (63 KB)
constexpr uint32_t WIDE_MAX_UNITS = 12;  // units per wave (T * S) beyond which registers spill

// With SRC != OPND_STAGED the split's operand is built in LDS by the waves
// (one wave per (superblock, column)): from f32 rows (OPND_ROWS) or by
// combining attention split partials (OPND_FA), with the same arithmetic as
// the prep / combine kernels; the first weight units are already in flight.
// 16-byte agent-coherent store / load of four floats for data that another
// workgroup of the same kernel reads (the protocol of sh_coherent.h).
typedef sh_f4v f4v;
__device__ __forceinline__ void st_coh4(float* p, float4 v) { sh_st_coh16(p, f4v{v.x, v.y, v.z, v.w}); }
__device__ __forceinline__ f4v ld_coh4(const float* p) { return sh_ld_coh16(p); }

// Fused residual prep of output superblock j (the PREP_RESID prep kernel's
// arithmetic: resid + split partials in split order, sums of squares, times
// the norm weight, operand store), one wave per column, by the last workgroup
// to finish j. The partials of the other workgroups are read with
// agent-coherent loads.
__device__ __forceinline__ void fused_prep_sb(const EpiArgs& ea, const PrepFuse& pf, uint32_t j, uint32_t nparts,
                                              uint32_t N) {
  const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (wave >= N) return;  // wave-uniform
  const uint32_t col = wave, k = 256 * j + 4 * lane;
  float* xp = pf.resid + (size_t)col * pf.K + k;
  float4 v = *(const float4*)xp;
  // before the coherent loads: their wait (an asm with a memory clobber) would
  // keep this load behind it, a second round trip
  const float4 wv = *(const float4*)(pf.norm_w + k);
  const float* pc = ea.out + (size_t)col * ea.ldo + k;
  for (uint32_t s0 = 0; s0 < nparts; s0 += 8) {
    f4v t[8];
#pragma unroll
    for (uint32_t i = 0; i < 8; ++i) t[i] = ld_coh4(pc + (size_t)min(s0 + i, nparts - 1) * ea.part_stride);
    asm volatile("s_waitcnt vmcnt(0)"
                 : "+v"(t[0]), "+v"(t[1]), "+v"(t[2]), "+v"(t[3]), "+v"(t[4]), "+v"(t[5]), "+v"(t[6]), "+v"(t[7])
                 :
                 : "memory");
#pragma unroll
    for (uint32_t i = 0; i < 8; ++i) {
      if (s0 + i >= nparts) break;
      v.x += t[i][0]; v.y += t[i][1]; v.z += t[i][2]; v.w += t[i][3];
    }
  }
  *(float4*)xp = v;
  const float ss = sh_wave_sum(sh_sq4(v));
  if (lane == 0) pf.ssq[j * 8 + col] = ss;
  v.x *= wv.x; v.y *= wv.y; v.z *= wv.z; v.w *= wv.w;
  sh_operand_store_sb(v, pf.K, j, col, pf.bx, pf.xs, pf.cs);
}

template <int T, int S, int D, int EPI, int SRC, bool FP = false>
__global__ __launch_bounds__(64 * WV) void k_gemv_q4w(const uint8_t* __restrict__ Wp, uint32_t tiles, uint32_t nsb,
                                                       const uint16_t* __restrict__ Bx,
                                                       const uint16_t* __restrict__ XS,
                                                       const float* __restrict__ CS, uint32_t N, EpiArgs ea,
                                                       OpndSrc src, PrepFuse pf) {
  static_assert(!FP || (EPI == EPI_PART && (SRC == OPND_STAGED || SRC == OPND_ROWS) && (T == 1 || T == 2)),
                "fused prep: split-K partials");
  constexpr int U = S * T;
  __shared__ h8 sB[S * 9 * 64];
  __shared__ float sC[64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4, r = lane & 15;
  const uint32_t ks = blockIdx.y, kb0 = ks * S;
  const uint32_t tile0 = (blockIdx.x * WV + wave) * T;
  float ssq_t[SSQ_PRE];
  col_ssq_load(ea, r & 7, ssq_t);

  if (SRC == OPND_STAGED) {
    // Activation operand of the split -> LDS: 1 KB blocks i = 9 * sb + m (m < 8:
    // B sub-block m, m = 8: XS), one wave instruction each.
#pragma unroll
    for (int i0 = 0; i0 < S * 9; i0 += WV) {
      const uint32_t i = i0 + wave;
      if (i < (uint32_t)(S * 9)) {
        const uint32_t sb = kb0 + i / 9, m = i % 9;
        const uint16_t* src_p = m < 8 ? Bx + ((size_t)(sb * 8 + m) * 64 + lane) * 8 : XS + ((size_t)sb * 64 + lane) * 8;
        __builtin_amdgcn_global_load_lds((glb_void_t*)src_p, (lds_void_t*)(sB + i * 64), 16, 0, 0);
      }
    }
    if (wave == WV - 1) {  // the split's S * 8 scales (lanes past them repeat the last)
      const uint32_t li = (uint32_t)lane < S * 8 ? lane : S * 8 - 1;
      __builtin_amdgcn_global_load_lds((glb_void_t*)(CS + kb0 * 8 + li), (lds_void_t*)sC, 4, 0, 0);
    }
  } else {
    // zero first: XS lanes >= 16 must be 0, and unused columns stay finite
    const h8 z = {0, 0, 0, 0, 0, 0, 0, 0};
    for (uint32_t i = threadIdx.x; i < (uint32_t)(S * 9 * 64); i += 64 * WV) sB[i] = z;
  }

  // Unit u = (superblock u / T, tile u % T); tiles past the end read the last
  // tile (in bounds) and are not written.
  auto unit_ptr = [&](int u) {
    const uint32_t t = tile0 + u % T;
    const uint32_t tile = t < tiles ? t : tiles - 1;
    return Wp + ((size_t)tile * nsb + kb0 + u / T) * SH_Q4K_TILE_BYTES;
  };
  Q4Tile ring[D];
#pragma unroll
  for (int k = 0; k < D && k < U; ++k) ring[k] = load_q4_tile(unit_ptr(k), lane, g, r);

  if (SRC != OPND_STAGED) {
    __syncthreads();  // zero fill done
    const uint32_t K = nsb * 256;
    const uint32_t n_live = SRC == OPND_FA && src.dbase
                                ? (*src.dbase + src.kv_off + src.split_keys - 1) / src.split_keys
                                : src.n_layout;
    // wave-uniform tasks t = wave + WV i; rows are all loaded before any is used
    constexpr int MAXT = (S * 8 + WV - 1) / WV;
    float4 vv[MAXT];
    if (SRC == OPND_ROWS) {
#pragma unroll
      for (int i = 0; i < MAXT; ++i) {
        const uint32_t t = wave + WV * i;
        if (t < (uint32_t)S * N) {
          const uint32_t sb = kb0 + t / N, col = t % N;
          vv[i] = *(const float4*)(src.x + (size_t)col * src.ldx + 256 * sb + 4 * lane);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < MAXT; ++i) {
      const uint32_t t = wave + WV * i;
      if (t >= (uint32_t)S * N) break;
      const uint32_t sbl = t / N, col = t % N, sb = kb0 + sbl;
      const float4 v = SRC == OPND_ROWS ? vv[i]
                                        : sh_fa_combine4(src.fa_part, src.n_layout, n_live, src.rows_pad, src.hd,
                                                         src.n_head, src.gqa, N, sb, col);
      const ShOpndLane o = sh_operand_lane(v);
      if (lane == 0) sC[sbl * 8 + col] = o.inv;
      const uint32_t k = 256 * sb + 4 * lane;
      if (k < K) {
        const uint32_t m = (k % 256) / 32;
        uint16_t* dst = (uint16_t*)(sB + (sbl * 9 + m) * 64 + ((k % 32) / 8) * 16 + col) + (k % 8);
        *(uint2*)dst = o.hi;
        *(uint2*)(dst + 64) = o.lo;
        if ((lane & 7) == 0) {
          uint16_t* xd = (uint16_t*)(sB + (sbl * 9 + 8) * 64 + col) + m;
          xd[0] = o.shi;
          xd[64] = o.slo;
        }
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // the LDS copies (and the first weight units) have landed
  __syncthreads();

  f4 y[T];
#pragma unroll
  for (int t = 0; t < T; ++t) y[t] = f4{0.f, 0.f, 0.f, 0.f};
  h8 bq[8], bm;
  float c = 0.f;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (u % T == 0) {  // next superblock: its operand from LDS
      const h8* sp = sB + (u / T) * 9 * 64 + lane;
#pragma unroll
      for (int m = 0; m < 8; ++m) bq[m] = sp[m * 64];
      bm = sp[8 * 64];
      c = sC[(u / T) * 8 + (lane & 7)];
    }
    const Q4Tile cur = ring[u % D];
    if (u + D < U) ring[u % D] = load_q4_tile(unit_ptr(u + D), lane, g, r);
    q4_tile_mma(cur, bq, bm, c, y[u % T]);
  }
  const float nf = col_ssq_rinv(ea, r & 7, ssq_t);

  if (EPI == EPI_SWIGLU) {
    // (gate, up) = tiles (2i, 2i + 1) of this wave; one split only
#pragma unroll
    for (int i = 0; i < T / 2; ++i) {
      float og[4], ou[4];
      col_sum4(y[2 * i], nf, og);
      col_sum4(y[2 * i + 1], nf, ou);
      const uint32_t tg = tile0 + 2 * i;
      if (tg < tiles && r < 8 && (uint32_t)r < N) swiglu4(ea, tg / 2, g, r, og, ou);
    }
  } else {
#pragma unroll
    for (int t = 0; t < T; ++t) {
      float o[4];
      col_sum4(y[t], nf, o);
      const uint32_t tile = tile0 + t;
      if (tile < tiles && r < 8 && (uint32_t)r < N) {
        if (FP) {  // partials another workgroup will read: agent-coherent stores
          st_coh4(ea.out + ks * ea.part_stride + (size_t)r * ea.ldo + tile * 16 + 4 * g,
                  make_float4(o[0], o[1], o[2], o[3]));
        } else {
          epilogue4<EPI>(ea, tile * 16 + 4 * g, (uint32_t)r, o, ks);
        }
      }
    }
  }
  if (FP) {
    // Arrival: every wave's partial stores have completed; the workgroup that
    // completes output superblock j (row groups x splits) runs its prep.
    __shared__ uint32_t s_last;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    constexpr uint32_t RG_ROWS = 16 * T * WV, RG_PER_SB = 256 / RG_ROWS;
    const uint32_t j = blockIdx.x / RG_PER_SB;
    if (threadIdx.x == 0) {
      const uint32_t arrivals = RG_PER_SB * gridDim.y;
      uint32_t* cnt = pf.cnt + (size_t)j * SH_SB_CNT_STRIDE;
      const uint32_t old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = old + 1 == arrivals;
      if (old + 1 == arrivals) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (s_last) fused_prep_sb(ea, pf, j, gridDim.y, N);
  }
}

// ------------------------------------------------------------------ Q4_K stream

// A workgroup of GW = 8 waves owns T row tiles for all of K. Wave w walks
// superblocks b = w, w + 8, ... and, inside each, the T tiles (one activation
// operand load serves T weight tiles). The next unit's weights are always in
// flight while the current one computes. The 8 partial sums of each tile meet
// in LDS at the end; no state is shared between workgroups.
constexpr int GW = 8;

// acc + p[0] + p[stride] + ... (n terms, in order), 8 loads in flight.
// B partials' loads per round trip (the sum is in split order for any B)
template <uint32_t B = 8>
__device__ __forceinline__ float4 sum_parts4(const float* p, size_t stride, uint32_t n, float4 acc) {
  for (uint32_t i0 = 0; i0 < n; i0 += B) {
    float4 t[B];
#pragma unroll
    for (uint32_t j = 0; j < B; ++j) t[j] = *(const float4*)(p + min(i0 + j, n - 1) * stride);
#pragma unroll
    for (uint32_t j = 0; j < B; ++j)
      if (i0 + j < n) { acc.x += t[j].x; acc.y += t[j].y; acc.z += t[j].z; acc.w += t[j].w; }
  }
  return acc;
}

// SRC = OPND_RESID: before the first superblock, every workgroup builds the
// whole operand in dynamic LDS ([nsb][9][64] h8, then nsb * 8 scales and
// nsb * 8 sums of squares) from the residual and the pending split partials,
// with the prep's arithmetic, and applies the RMS factor itself.
template <int T, int EPI, int SRC>
__global__ __launch_bounds__(64 * GW) void k_gemv_q4s(const uint8_t* __restrict__ Wp, uint32_t tiles, uint32_t nsb,
                                                       const uint16_t* __restrict__ Bx,
                                                       const uint16_t* __restrict__ XS,
                                                       const float* __restrict__ CS, uint32_t N, EpiArgs ea,
                                                       OpndSrc src) {
  constexpr int CH = T < 4 ? T : 4;  // tiles reduced per LDS round
  __shared__ f4 red[CH][GW][64];
  extern __shared__ h8 dynB[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar address math
  const int g = lane >> 4, r = lane & 15;
  const uint32_t tile0 = blockIdx.x * T;
  float ssq_t[SSQ_PRE];
  if (SRC != OPND_RESID) col_ssq_load(ea, r & 7, ssq_t);
  float nf = 1.0f;
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
  float c = 0.f;
  float* sC = (float*)(dynB + (size_t)nsb * 9 * 64);
  float* sQ = sC + nsb * 8;
  auto load_b = [&](uint32_t b) {
    if (SRC == OPND_RESID) {
#pragma unroll
      for (int m = 0; m < 8; ++m) bq[m] = dynB[(b * 9 + m) * 64 + lane];
      bm = dynB[(b * 9 + 8) * 64 + lane];
      c = sC[b * 8 + (lane & 7)];
    } else if (N >= 8) {
#pragma unroll
      for (int m = 0; m < 8; ++m) bq[m] = as_h8(ld16(Bx + ((size_t)(b * 8 + m) * 64 + lane) * 8));
      bm = as_h8(ld16(XS + ((size_t)b * 64 + lane) * 8));
      c = CS[b * 8 + (lane & 7)];
    } else {
      // lanes of columns >= N load nothing (their outputs are never stored):
      // a 1-column launch fetches 1/8 of the operand
      const h8 z = {0, 0, 0, 0, 0, 0, 0, 0};
      const bool live = (uint32_t)(lane & 7) < N;
#pragma unroll
      for (int m = 0; m < 8; ++m) bq[m] = live ? as_h8(ld16(Bx + ((size_t)(b * 8 + m) * 64 + lane) * 8)) : z;
      bm = live ? as_h8(ld16(XS + ((size_t)b * 64 + lane) * 8)) : z;
      c = CS[b * 8 + (lane & 7)];
    }
  };
  if (nbw) st[0] = load_q4_tile(a_ptr(0, wave), lane, g, r);
  if (SRC == OPND_RESID) {
    const h8 z = {0, 0, 0, 0, 0, 0, 0, 0};
    for (uint32_t i = threadIdx.x; i < nsb * 9 * 64; i += 64 * GW) dynB[i] = z;
    __syncthreads();
    const uint32_t K = nsb * 256;
    const size_t pstride = (size_t)8 * src.part_ld;
    for (uint32_t t = wave; t < nsb * N; t += GW) {  // wave-uniform
      const uint32_t sb = t / N, col = t % N, k = 256 * sb + 4 * lane;
      float4 v = *(const float4*)(src.x + (size_t)col * K + k);
      // more than 8 at once (the draft's down leaves 16 K-split partials: two
      // round trips in batches of 8)
      if (src.nparts > 8) v = sum_parts4<16>(src.part + (size_t)col * src.part_ld + k, pstride, src.nparts, v);
      else if (src.nparts) v = sum_parts4(src.part + (size_t)col * src.part_ld + k, pstride, src.nparts, v);
      if (blockIdx.x == 0) *(float4*)(src.rout + (size_t)col * K + k) = v;
      const float ss = sh_wave_sum(sh_sq4(v));
      if (lane == 0) sQ[sb * 8 + col] = ss;
      const float4 wv = *(const float4*)(src.norm_w + k);
      v.x *= wv.x; v.y *= wv.y; v.z *= wv.z; v.w *= wv.w;
      const ShOpndLane o = sh_operand_lane(v);
      if (lane == 0) sC[sb * 8 + col] = o.inv;
      const uint32_t m = (k % 256) / 32;
      uint16_t* dst = (uint16_t*)(dynB + (sb * 9 + m) * 64 + ((k % 32) / 8) * 16 + col) + (k % 8);
      *(uint2*)dst = o.hi;
      *(uint2*)(dst + 64) = o.lo;
      if ((lane & 7) == 0) {
        uint16_t* xd = (uint16_t*)(dynB + (sb * 9 + 8) * 64 + col) + m;
        xd[0] = o.shi;
        xd[64] = o.slo;
      }
    }
    __syncthreads();
    // RMS factor of the lane's column from the superblock sums (added in superblock order)
    const uint32_t cc = (uint32_t)(r & 7) < N ? (uint32_t)(r & 7) : 0u;
    float tot = 0.f;
    for (uint32_t b = 0; b < nsb; ++b) tot += sQ[b * 8 + cc];
    nf = 1.0f / sqrtf(tot / (float)K + src.eps);
  }
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
        q4_tile_mma(st[par], bq, bm, c, y[t]);
      }
    }
  }
  if (SRC != OPND_RESID) nf = col_ssq_rinv(ea, r & 7, ssq_t);
  // Tile partials meet in LDS, CH tiles per round; wave w < CH ends up holding
  // tile (round * CH + w), or with SwiGLU wave w < CH/2 holds the pair
  // (gate, up) = tiles (2w, 2w + 1) of the round.
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
        col_sum4(vg, nf, og);
        col_sum4(vu, nf, ou);
        const uint32_t tg = tile0 + c0 + 2 * wave;
        if (tg < tiles && r < 8 && (uint32_t)r < N) swiglu4(ea, tg / 2, g, r, og, ou);
      }
    } else if (wave < CH) {
      f4 v = {0.f, 0.f, 0.f, 0.f};
      for (int w = 0; w < GW; ++w) v += red[wave][w][lane];
      float o[4];
      col_sum4(v, nf, o);
      const uint32_t tile = tile0 + c0 + wave;
      if (tile < tiles && r < 8 && (uint32_t)r < N) epilogue4<EPI>(ea, tile * 16 + 4 * g, (uint32_t)r, o);
    }
    __syncthreads();
  }
}

// ------------------------------------------------------------------ Q4_K deep ring

// Whole-K GEMV for matrices of exactly 256 * 7 row tiles or more in one round
// (the 8B gate/up: 1792 tiles) whose K is NB * 8 superblocks. A workgroup of GW = 8 waves owns T row tiles for all of
// K; wave w takes superblocks w, w + 8, ... (NB of them) and, inside each, the
// T tiles: NB * T weight units in one fully unrolled sequence with a sliding
// window of D units in flight (unit u + D issued as unit u computes). The
// chip-wide request stream is then steady (D units per wave, ~20 MB in all)
// instead of one burst per superblock, so waves start computing as their first
// units land and the last units arrive just before they are needed. The NB
// activation operands stay in registers. With T = 7 a 1792-tile matrix is 256
// workgroups, one per CU, in a single round. The 8 partial sums of each tile
// meet in LDS in one round. EPI_STORE and EPI_PART (one split) only.
// Fused SwiGLU prep of h superblock j (the PREP_SWIGLU prep kernel's
// arithmetic with one split: h = silu(gate) * up at the packed gate / up rows
// of each element, then the down GEMV's operand), one wave per column, by the
// last workgroup to finish the 32 packed gate / up tiles of j.
__device__ __forceinline__ void fused_swiglu_sb(const EpiArgs& ea, const PrepFuse& pf, uint32_t j, uint32_t N) {
  const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (wave >= N) return;  // wave-uniform
  const uint32_t col = wave, k = 256 * j + 4 * lane;
  const float* pc = ea.out + (size_t)col * ea.ldo + 32 * (k / 16) + k % 16;
  f4v gv = ld_coh4(pc), uv = ld_coh4(pc + 16);
  asm volatile("s_waitcnt vmcnt(0)" : "+v"(gv), "+v"(uv) : : "memory");
  float4 g = make_float4(0.f, 0.f, 0.f, 0.f), u = make_float4(0.f, 0.f, 0.f, 0.f);
  g.x += gv[0]; g.y += gv[1]; g.z += gv[2]; g.w += gv[3];
  u.x += uv[0]; u.y += uv[1]; u.z += uv[2]; u.w += uv[3];
  const float4 v = make_float4((g.x / (1.0f + expf(-g.x))) * u.x, (g.y / (1.0f + expf(-g.y))) * u.y,
                               (g.z / (1.0f + expf(-g.z))) * u.z, (g.w / (1.0f + expf(-g.w))) * u.w);
  sh_operand_store_sb(v, pf.K, j, col, pf.bx, pf.xs, pf.cs);
}

template <int T, int NB, int D, int EPI, bool FS = false, int WV = GW>
__global__ __launch_bounds__(64 * WV) void k_gemv_q4t(const uint8_t* __restrict__ Wp, uint32_t tiles, uint32_t nsb,
                                                       const uint16_t* __restrict__ Bx,
                                                       const uint16_t* __restrict__ XS,
                                                       const float* __restrict__ CS, uint32_t N, EpiArgs ea,
                                                       PrepFuse pf) {
  static_assert(EPI == EPI_STORE || EPI == EPI_PART || EPI == EPI_QKV, "deep-ring GEMV: per-row epilogues only");
  static_assert(!FS || EPI == EPI_PART, "fused SwiGLU prep: gate / up sums");
  constexpr int U = NB * T;
  __shared__ f4 red[T][WV][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4, r = lane & 15;
  const uint32_t tile0 = blockIdx.x * T;
  // the RMS sums of squares: in registers, or staged in LDS by the first
  // threads (16 waves, registers tight; T = 8: 126 instead of 178 VGPRs, two
  // workgroups per CU, the draft's lm_head 38.3 -> 30.5 us); both add them in
  // superblock order
  constexpr bool SSQ_LDS = WV > GW || T == 8;
  __shared__ float s_ssq[SSQ_LDS ? 64 * WV : 1];
  float ssq_t[SSQ_LDS ? 1 : SSQ_PRE];
  if constexpr (SSQ_LDS) {
    if (ea.ssq && threadIdx.x < ea.ssq_n * 8) s_ssq[threadIdx.x] = ea.ssq[threadIdx.x];
  } else {
    col_ssq_load(ea, r & 7, ssq_t);
  }
  // unit u: superblock wave + WV * (u / T), tile tile0 + u % T (clamped in bounds)
  auto unit_ptr = [&](int u) {
    const uint32_t t = tile0 + u % T, tile = t < tiles ? t : tiles - 1;
    return Wp + ((size_t)tile * nsb + wave + WV * (u / T)) * SH_Q4K_TILE_BYTES;
  };
  Q4Tile ring[D];
#pragma unroll
  for (int u = 0; u < D && u < U; ++u) ring[u] = load_q4_tile(unit_ptr(u), lane, g, r);
  h8 bq[NB][8], bm[NB];
  float c[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const uint32_t b = wave + WV * i;
#pragma unroll
    for (int k = 0; k < 8; ++k) bq[i][k] = as_h8(ld16(Bx + ((size_t)(b * 8 + k) * 64 + lane) * 8));
    bm[i] = as_h8(ld16(XS + ((size_t)b * 64 + lane) * 8));
    c[i] = CS[b * 8 + (lane & 7)];
  }
  f4 y[T];
#pragma unroll
  for (int t = 0; t < T; ++t) y[t] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < U; ++u) {
    q4_tile_mma(ring[u % D], bq[u / T], bm[u / T], c[u / T], y[u % T]);
    if (u + D < U) ring[u % D] = load_q4_tile(unit_ptr(u + D), lane, g, r);
  }
  float nf = 1.0f;
  if constexpr (!SSQ_LDS) nf = col_ssq_rinv(ea, r & 7, ssq_t);
#pragma unroll
  for (int t = 0; t < T; ++t) red[t][wave][lane] = y[t];
  __syncthreads();
  if (SSQ_LDS && ea.ssq) {
    float ss = 0.f;
    for (uint32_t i = 0; i < ea.ssq_n; ++i) ss += s_ssq[i * 8 + (r & 7)];
    nf = 1.0f / sqrtf(ss / (float)ea.norm_K + ea.eps);
  }
  if (wave < T) {
    f4 v = {0.f, 0.f, 0.f, 0.f};
    for (int w = 0; w < WV; ++w) v += red[wave][w][lane];
    float o[4];
    col_sum4(v, nf, o);
    const uint32_t tile = tile0 + wave;
    if (tile < tiles && r < 8 && (uint32_t)r < N) {
      if (FS) st_coh4(ea.out + (size_t)r * ea.ldo + tile * 16 + 4 * g, make_float4(o[0], o[1], o[2], o[3]));
      else epilogue4<EPI>(ea, tile * 16 + 4 * g, (uint32_t)r, o);
    }
  }
  if (FS) {
    // Arrival at the (one or two) h superblocks this workgroup's packed tiles
    // touch: packed tile p holds rows of h tile p / 2, so superblock j is
    // packed tiles 32 j .. 32 j + 31, workgroups 32 j / T .. (32 j + 31) / T.
    __shared__ uint32_t s_last[2];
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    const uint32_t j0 = tile0 / 32, j1 = (tile0 + T - 1) / 32;
    if (threadIdx.x < 2) {
      const uint32_t j = threadIdx.x == 0 ? j0 : j1;
      uint32_t last = 0;
      if (threadIdx.x == 0 || j1 != j0) {
        const uint32_t wg_first = 32 * j / T, wg_last = min((32 * j + 31) / T, gridDim.x - 1);
        uint32_t* cnt = pf.cnt + (size_t)j * SH_SB_CNT_STRIDE;
        const uint32_t old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = old + 1 == wg_last - wg_first + 1;
        if (last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      s_last[threadIdx.x] = last;
    }
    __syncthreads();
    if (s_last[0]) fused_swiglu_sb(ea, pf, j0, N);
    if (s_last[1]) fused_swiglu_sb(ea, pf, j1, N);
  }
}

// ------------------------------------------------------------------ Q4_K multi-group

// Decoded state of one weight tile for one superblock: the eight sub-block
// words, the unpacked 6-bit scales and minimums, and d, dmin of the lane's rows.
struct Q4Dec {
  uint32_t w[8];
  uint32_t sc03, sc47, m03, m47;
  float d[4], dmin[4];
};

__device__ __forceinline__ Q4Dec q4_decode_setup(const Q4Tile& a) {
  Q4Dec s;
  s.w[0] = a.q0.x; s.w[1] = a.q0.y; s.w[2] = a.q0.z; s.w[3] = a.q0.w;
  s.w[4] = a.q1.x; s.w[5] = a.q1.y; s.w[6] = a.q1.z; s.w[7] = a.q1.w;
  s.sc03 = a.s0 & 0x3F3F3F3Fu;
  s.m03 = a.s1 & 0x3F3F3F3Fu;
  s.sc47 = (a.s2 & 0x0F0F0F0Fu) | ((a.s0 >> 2) & 0x30303030u);
  s.m47 = ((a.s2 >> 4) & 0x0F0F0F0Fu) | ((a.s1 >> 2) & 0x30303030u);
  const uint32_t ddw[4] = {a.dd.x, a.dd.y, a.dd.z, a.dd.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    s.d[j] = (float)as_h2(ddw[j]).x;
    s.dmin[j] = (float)as_h2(ddw[j]).y;
  }
  return s;
}

// A operand of sub-block m: exact f16 c * sc_m * q (as in q4_tile_mma).
__device__ __forceinline__ h8 q4_frag(const Q4Dec& s, int m, uint32_t magic) {
  const h2 k1024 = {(_Float16)-1024.0f, (_Float16)-1024.0f};
  const h2 mult = magic_pair(m < 4 ? s.sc03 : s.sc47, magic, m & 3, m & 3) + k1024;
  return q4_operand2(s.w[m], magic, mult, mult * k1024);
}

// A operand of the minimum term: m_s at k = s (every lane group).
__device__ __forceinline__ h8 q4_min_frag(const Q4Dec& s, uint32_t magic) {
  const h2 k1024 = {(_Float16)-1024.0f, (_Float16)-1024.0f};
  u32x4 am;
  am.x = as_u32(magic_pair(s.m03, magic, 0, 1) + k1024);
  am.y = as_u32(magic_pair(s.m03, magic, 2, 3) + k1024);
  am.z = as_u32(magic_pair(s.m47, magic, 0, 1) + k1024);
  am.w = as_u32(magic_pair(s.m47, magic, 2, 3) + k1024);
  return as_h8(am);
}

// Norm factor of column c of operand group g (sums of squares of group g
// start at g * ssq_n * 8).
__device__ __forceinline__ float col_rinv_g(const EpiArgs& ea, uint32_t g, uint32_t c) {
  if (!ea.ssq) return 1.0f;
  const float* sq = ea.ssq + (size_t)g * ea.ssq_n * 8;
  float ss = 0.f;
  for (uint32_t i0 = 0; i0 < ea.ssq_n; i0 += 8) {
    float t[8];
#pragma unroll
    for (uint32_t j = 0; j < 8; ++j) t[j] = sq[min(i0 + j, ea.ssq_n - 1) * 8 + c];
#pragma unroll
    for (uint32_t j = 0; j < 8; ++j) ss += i0 + j < ea.ssq_n ? t[j] : 0.0f;
  }
  return 1.0f / sqrtf(ss / (float)ea.norm_K + ea.eps);
}

// ------------------------------------------------------------------ Q5_K / Q6_K fragments

// One wave's operands of one (16-row tile, superblock) of Q5_K: the Q4_K
// words plus two high-bit words per lane (tile layout at k_repack_q5k).
struct Q5Tile {
  u32x4 q0, q1, dd;
  uint32_t h0, h1;
  uint32_t s0, s1, s2;
  __device__ void pin() { pin32(q0); pin32(q1); pin32(dd); pin32(h0); pin32(h1); pin32(s0); pin32(s1); pin32(s2); }
};
struct Q5Dec {
  uint32_t w[8], h[2];
  uint32_t sc03, sc47, m03, m47;
  float d[4], dmin[4];
};
__device__ __forceinline__ Q5Tile load_q5_tile(const uint8_t* base, int lane, int g, int r) {
  Q5Tile a;
  a.q0 = ldw16(base + 16 * lane);
  a.q1 = ldw16(base + 1024 + 16 * lane);
  const uint2 h = *(const uint2*)(base + 2048 + 8 * lane);
  a.h0 = h.x;
  a.h1 = h.y;
  a.dd = ld16(base + 2560 + 16 * g);
  const uint32_t* sp = (const uint32_t*)(base + 2624 + 12 * r);
  a.s0 = sp[0];
  a.s1 = sp[1];
  a.s2 = sp[2];
  return a;
}
__device__ __forceinline__ Q5Dec q5_decode_setup(const Q5Tile& a) {
  Q4Tile b;
  b.q0 = a.q0; b.q1 = a.q1; b.dd = a.dd; b.s0 = a.s0; b.s1 = a.s1; b.s2 = a.s2;
  const Q4Dec q = q4_decode_setup(b);
  Q5Dec s;
#pragma unroll
  for (int m = 0; m < 8; ++m) s.w[m] = q.w[m];
  s.h[0] = a.h0;
  s.h[1] = a.h1;
  s.sc03 = q.sc03; s.sc47 = q.sc47; s.m03 = q.m03; s.m47 = q.m47;
#pragma unroll
  for (int j = 0; j < 4; ++j) { s.d[j] = q.d[j]; s.dmin[j] = q.dmin[j]; }
  return s;
}

// w shifted left by n (n >= 0) or right by -n; n is a constant after unrolling.
__device__ __forceinline__ uint32_t shl_signed(uint32_t w, int n) { return n >= 0 ? w << n : w >> -n; }

// A operand of Q5_K sub-block m: exact f16 c sc_m q5 with q5 = nibble + 16 h.
// The fifth bit goes into the magic's mantissa right above the nibble (bit 4
// of a half for the pairs decoded as 1024 + q, bit 8 for those decoded as
// 1024 + 16 q), so (1024 + c q5) sc - 1024 sc = c sc q5 stays one exact FMA
// (c sc q5 <= 16 * 63 * 31 < 2^15, 11 significant bits).
__device__ __forceinline__ h8 q5_frag(const Q5Dec& s, int m, uint32_t magic) {
  const h2 k1024 = {(_Float16)-1024.0f, (_Float16)-1024.0f};
  const int base = (m & 1) * 2 + ((m >> 1) & 1) * 8;
  const uint32_t hw = s.h[m >> 2];
  const uint32_t hx = shl_signed(hw, 4 - base), hz = shl_signed(hw, 3 - base);
  const uint32_t w = s.w[m], w8 = w >> 8;
  const h2 mult = magic_pair(m < 4 ? s.sc03 : s.sc47, magic, m & 3, m & 3) + k1024;
  const h2 add = mult * k1024;
  u32x4 r;
  r.x = as_u32(__builtin_elementwise_fma(as_h2(bfi(0x000F000Fu, w, bfi(0x00100010u, hx, magic))), mult, add));
  r.y = as_u32(__builtin_elementwise_fma(as_h2(bfi(0x00F000F0u, w, bfi(0x01000100u, hx, magic))), mult, add));
  r.z = as_u32(__builtin_elementwise_fma(as_h2(bfi(0x000F000Fu, w8, bfi(0x00100010u, hz, magic))), mult, add));
  r.w = as_u32(__builtin_elementwise_fma(as_h2(bfi(0x00F000F0u, w8, bfi(0x01000100u, hz, magic))), mult, add));
  return as_h8(r);
}
__device__ __forceinline__ h8 q5_min_frag(const Q5Dec& s, uint32_t magic) {
  Q4Dec q;
  q.m03 = s.m03;
  q.m47 = s.m47;
  return q4_min_frag(q, magic);
}

// One wave's operands of one (16-row tile, superblock) of Q6_K (tile layout at
// k_repack_q6k): the nibble words, four high-bit words, the lane's 8 scales
// (sub-block m: byte m) and d of the lane's 4 output rows.
struct Q6Tile {
  u32x4 q0, q1, h;
  uint2 sc, d;
  __device__ void pin() { pin32(q0); pin32(q1); pin32(h); pin32(sc); pin32(d); }
};
struct Q6Dec {
  uint32_t w[8], h[4];
  uint32_t sl03, sl47, sh03, sh47;
  float d[4];
};
__device__ __forceinline__ Q6Tile load_q6_tile(const uint8_t* base, int lane, int g, int r) {
  Q6Tile a;
  a.q0 = ldw16(base + 16 * lane);
  a.q1 = ldw16(base + 1024 + 16 * lane);
  a.h = ldw16(base + 2048 + 16 * lane);
  a.sc = *(const uint2*)(base + 3072 + 16 * r + 8 * (g >> 1));
  a.d = *(const uint2*)(base + 3328 + 8 * g);
  return a;
}
// A scale sc (int8) is split as 16 sh + sl, sl = sc & 15 in [0, 15] and sh =
// sc >> 4 in [-8, 7]; the bytes below are sl and sh + 8 (the latter as the
// high nibble with its top bit flipped: u ^ 8 = sh + 8 for u = sc >> 4 & 15).
__device__ __forceinline__ Q6Dec q6_decode_setup(const Q6Tile& a) {
  Q6Dec s;
  s.w[0] = a.q0.x; s.w[1] = a.q0.y; s.w[2] = a.q0.z; s.w[3] = a.q0.w;
  s.w[4] = a.q1.x; s.w[5] = a.q1.y; s.w[6] = a.q1.z; s.w[7] = a.q1.w;
  s.h[0] = a.h.x; s.h[1] = a.h.y; s.h[2] = a.h.z; s.h[3] = a.h.w;
  s.sl03 = a.sc.x & 0x0F0F0F0Fu;
  s.sl47 = a.sc.y & 0x0F0F0F0Fu;
  s.sh03 = ((a.sc.x >> 4) & 0x0F0F0F0Fu) ^ 0x08080808u;
  s.sh47 = ((a.sc.y >> 4) & 0x0F0F0F0Fu) ^ 0x08080808u;
  s.d[0] = (float)as_h2(a.d.x).x;
  s.d[1] = (float)as_h2(a.d.x).y;
  s.d[2] = (float)as_h2(a.d.y).x;
  s.d[3] = (float)as_h2(a.d.y).y;
  return s;
}
// The two A operands of Q6_K sub-block m, exact f16 c sl (q - 32) and
// c sh (q - 32), c = 1 or 16 by pair; the sums combine as acc_l + 16 acc_h
// (= sc (q - 32) summed, a product that would need 13 bits in one f16). The
// 6-bit q = nibble + 16 hi2 is decoded as 1024 + q (or 1024 + 16 q, at most
// 2032) with the two high bits in the mantissa above the nibble; the FMA's
// addend -(1024 + 32 c) s removes both offsets: |c s (q - 32)| <= 7680 exactly.
__device__ __forceinline__ void q6_frag(const Q6Dec& s, int m, uint32_t magic, h8 (&a)[2]) {
  const h2 k1024 = {(_Float16)-1024.0f, (_Float16)-1024.0f};
  const h2 k1032 = {(_Float16)-1032.0f, (_Float16)-1032.0f};
  const h2 k1056 = {(_Float16)-1056.0f, (_Float16)-1056.0f};
  const h2 k1536 = {(_Float16)-1536.0f, (_Float16)-1536.0f};
  const int base = (m & 1) * 8;
  const uint32_t hw = s.h[m >> 1];
  const uint32_t hx = shl_signed(hw, 4 - base), hz = shl_signed(hw, 2 - base);
  const uint32_t w = s.w[m], w8 = w >> 8;
  const h2 ml = magic_pair(m < 4 ? s.sl03 : s.sl47, magic, m & 3, m & 3) + k1024;
  const h2 mh = magic_pair(m < 4 ? s.sh03 : s.sh47, magic, m & 3, m & 3) + k1032;
  const h2 px = as_h2(bfi(0x000F000Fu, w, bfi(0x00300030u, hx, magic)));
  const h2 py = as_h2(bfi(0x00F000F0u, w, bfi(0x03000300u, hx, magic)));
  const h2 pz = as_h2(bfi(0x000F000Fu, w8, bfi(0x00300030u, hz, magic)));
  const h2 pw = as_h2(bfi(0x00F000F0u, w8, bfi(0x03000300u, hz, magic)));
  const h2 l1 = ml * k1056, l16 = ml * k1536, h1 = mh * k1056, h16 = mh * k1536;
  u32x4 r;
  r.x = as_u32(__builtin_elementwise_fma(px, ml, l1));
  r.y = as_u32(__builtin_elementwise_fma(py, ml, l16));
  r.z = as_u32(__builtin_elementwise_fma(pz, ml, l1));
  r.w = as_u32(__builtin_elementwise_fma(pw, ml, l16));
  a[0] = as_h8(r);
  r.x = as_u32(__builtin_elementwise_fma(px, mh, h1));
  r.y = as_u32(__builtin_elementwise_fma(py, mh, h16));
  r.z = as_u32(__builtin_elementwise_fma(pz, mh, h1));
  r.w = as_u32(__builtin_elementwise_fma(pw, mh, h16));
  a[1] = as_h8(r);
}

// Weight formats of the multi-group GEMM: tile bytes, one wave's loads of a
// (tile, superblock), the per-superblock decode setup, the A fragments of
// sub-block m (NA per sub-block, each against the same B), whether the
// minimum term (XS operand) applies, and the superblock's contribution
// d * sum - dmin * min for output row j.
struct FmtQ4K {
  static constexpr uint32_t kTile = SH_Q4K_TILE_BYTES;
  static constexpr int NA = 1;
  static constexpr bool kMin = true;
  using Tile = Q4Tile;
  using Dec = Q4Dec;
  static __device__ __forceinline__ Tile load(const uint8_t* b, int lane, int g, int r) {
    return load_q4_tile(b, lane, g, r);
  }
  static __device__ __forceinline__ Dec setup(const Tile& a) { return q4_decode_setup(a); }
  static __device__ __forceinline__ void frag(const Dec& s, int m, uint32_t magic, h8 (&a)[NA]) {
    a[0] = q4_frag(s, m, magic);
  }
  static __device__ __forceinline__ h8 min_frag(const Dec& s, uint32_t magic) { return q4_min_frag(s, magic); }
  static __device__ __forceinline__ float term(const Dec& s, const f4 (&acc)[NA], float macc, int j) {
    return s.d[j] * acc[0][j] - s.dmin[j] * macc;
  }
};
struct FmtQ5K {
  static constexpr uint32_t kTile = SH_Q5K_TILE_BYTES;
  static constexpr int NA = 1;
  static constexpr bool kMin = true;
  using Tile = Q5Tile;
  using Dec = Q5Dec;
  static __device__ __forceinline__ Tile load(const uint8_t* b, int lane, int g, int r) {
    return load_q5_tile(b, lane, g, r);
  }
  static __device__ __forceinline__ Dec setup(const Tile& a) { return q5_decode_setup(a); }
  static __device__ __forceinline__ void frag(const Dec& s, int m, uint32_t magic, h8 (&a)[NA]) {
    a[0] = q5_frag(s, m, magic);
  }
  static __device__ __forceinline__ h8 min_frag(const Dec& s, uint32_t magic) { return q5_min_frag(s, magic); }
  static __device__ __forceinline__ float term(const Dec& s, const f4 (&acc)[NA], float macc, int j) {
    return s.d[j] * acc[0][j] - s.dmin[j] * macc;
  }
};
struct FmtQ6K {
  static constexpr uint32_t kTile = SH_Q6K_TILE_BYTES;
  static constexpr int NA = 2;
  static constexpr bool kMin = false;
  using Tile = Q6Tile;
  using Dec = Q6Dec;
  static __device__ __forceinline__ Tile load(const uint8_t* b, int lane, int g, int r) {
    return load_q6_tile(b, lane, g, r);
  }
  static __device__ __forceinline__ Dec setup(const Tile& a) { return q6_decode_setup(a); }
  static __device__ __forceinline__ void frag(const Dec& s, int m, uint32_t magic, h8 (&a)[NA]) {
    q6_frag(s, m, magic, a);
  }
  static __device__ __forceinline__ h8 min_frag(const Dec&, uint32_t) { return h8{}; }
  static __device__ __forceinline__ float term(const Dec& s, const f4 (&acc)[NA], float, int j) {
    return s.d[j] * __builtin_fmaf(16.0f, acc[1][j], acc[0][j]);
  }
};

// y = W x for G operand groups (up to 64 columns) in one pass over W, W in
// any K-quant format F. A workgroup of 8 waves covers 8 T row tiles (wave w:
// tiles (blockIdx.x * 8 + w) * T + t) over the superblocks [S blockIdx.y,
// S blockIdx.y + S) of split blockIdx.y. Per superblock the G groups' operands
// (B and XS, 9 KB each, and 8 scales) are copied to LDS by direct
// global->LDS loads, two buffers alternating so superblock i + 1 (operands and
// weights) loads while i computes; every decoded weight fragment then feeds G
// MFMAs. The per-superblock sums go through d (and dmin) and the column scale
// in f32 as in the 8-column kernels. EPI_PART writes split partials
// [split][col][row]; EPI_STORE (one split) whole rows.
constexpr uint32_t MG_MAX_G = 8;

template <class F, int T, int G, int EPI>
__global__ __launch_bounds__(512) void k_gemm_kq(const uint8_t* __restrict__ Wp, uint32_t tiles, uint32_t nsb,
                                                  uint32_t S, const uint16_t* __restrict__ Bx,
                                                  const uint16_t* __restrict__ XS, const float* __restrict__ CS,
                                                  uint32_t N, EpiArgs ea) {
  using Tile = typename F::Tile;
  using Dec = typename F::Dec;
  constexpr int NA = F::NA;
  __shared__ h8 sB[2][G * 9 * 64];  // [buffer][group * 9 + fragment][lane]
  __shared__ float sC[2][64];       // [buffer][group * 8 + column]
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g4 = lane >> 4, r = lane & 15;
  const uint32_t ks = blockIdx.y, sb0 = ks * S, sb1 = min(sb0 + S, nsb);
  const uint32_t tile0 = (blockIdx.x * 8 + wave) * T;
  const size_t gB = (size_t)nsb * 8 * 512, gX = (size_t)nsb * 512, gC = (size_t)nsb * 8;
  const uint32_t magic = __builtin_amdgcn_readfirstlane(0x64006400u);
  float nf[G];
#pragma unroll
  for (int g = 0; g < G; ++g) nf[g] = col_rinv_g(ea, g, r & 7);

  auto stage = [&](uint32_t sb, int buf) {
    // fragment f of group g: 1 KB, one wave instruction (XS only with a minimum term)
    for (uint32_t fi = wave; fi < (uint32_t)(G * 9); fi += 8) {
      const uint32_t g = fi / 9, f = fi % 9;
      if (!F::kMin && f == 8) continue;
      const uint16_t* src = f < 8 ? Bx + g * gB + ((size_t)(sb * 8 + f) * 64 + lane) * 8
                                  : XS + g * gX + ((size_t)sb * 64 + lane) * 8;
      sh_dma16(src, &sB[buf][fi * 64]);
    }
    if (wave == 7) {  // the G * 8 scales (lanes past them repeat the last)
      const uint32_t li = (uint32_t)lane < (uint32_t)(G * 8) ? (uint32_t)lane : G * 8 - 1;
      sh_dma4(CS + (li / 8) * gC + sb * 8 + li % 8, sC[buf]);
    }
  };
  auto a_ptr = [&](int t, uint32_t sb) {
    const uint32_t tt = tile0 + t < tiles ? tile0 + t : tiles - 1;  // clamp keeps loads in bounds
    return Wp + ((size_t)tt * nsb + sb) * F::kTile;
  };

  f4 y[T][G];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int g = 0; g < G; ++g) y[t][g] = f4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](const Tile (&at)[T], int buf) {
    Dec dec[T];
#pragma unroll
    for (int t = 0; t < T; ++t) dec[t] = F::setup(at[t]);
    f4 acc[T][G][NA];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int i = 0; i < NA; ++i) acc[t][g][i] = f4{0.f, 0.f, 0.f, 0.f};
    // B fragments one sub-block ahead in registers (the G reads of sub-block
    // m + 1, or the minimum term's after the last, go out before sub-block
    // m's MFMAs): without this each MFMA waited on the LDS read just before it
    h8 bb[2][G];
#pragma unroll
    for (int g = 0; g < G; ++g) bb[0][g] = sB[buf][(g * 9) * 64 + lane];
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const int cur = m & 1;
      if (m < 7 || F::kMin) {
#pragma unroll
        for (int g = 0; g < G; ++g) bb[cur ^ 1][g] = sB[buf][(g * 9 + m + 1) * 64 + lane];
      }
      __builtin_amdgcn_sched_barrier(0);  // keep those reads ahead of this sub-block's MFMAs
      h8 a[T][NA];
#pragma unroll
      for (int t = 0; t < T; ++t) F::frag(dec[t], m, magic, a[t]);
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
          for (int i = 0; i < NA; ++i) acc[t][g][i] = mfma16(a[t][i], bb[cur][g], acc[t][g][i]);
    }
    h8 am[T];
    if constexpr (F::kMin) {
#pragma unroll
      for (int t = 0; t < T; ++t) am[t] = F::min_frag(dec[t], magic);
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const h8 bm = bb[0][g];  // the minimum term's fragment (read during sub-block 7)
      const float c = sC[buf][g * 8 + (lane & 7)];
#pragma unroll
      for (int t = 0; t < T; ++t) {
        f4 macc = f4{0.f, 0.f, 0.f, 0.f};
        if constexpr (F::kMin) macc = mfma16(am[t], bm, f4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
        for (int j = 0; j < 4; ++j) y[t][g][j] = y[t][g][j] + c * F::term(dec[t], acc[t][g], macc[j], j);
      }
    }
  };

  // Superblocks go in pairs so each weight buffer's index is a constant.
  Tile wa[T], wb[T];
  stage(sb0, 0);
#pragma unroll
  for (int t = 0; t < T; ++t) wa[t] = F::load(a_ptr(t, sb0), lane, g4, r);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
#pragma unroll
  for (int t = 0; t < T; ++t) wa[t].pin();
  for (uint32_t sb = sb0; sb < sb1; sb += 2) {
    if (sb + 1 < sb1) {
      stage(sb + 1, 1);
#pragma unroll
      for (int t = 0; t < T; ++t) wb[t] = F::load(a_ptr(t, sb + 1), lane, g4, r);
    }
    compute(wa, 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (sb + 1 >= sb1) break;
    if (sb + 2 < sb1) {
      stage(sb + 2, 0);
#pragma unroll
      for (int t = 0; t < T; ++t) wa[t] = F::load(a_ptr(t, sb + 2), lane, g4, r);
    }
    compute(wb, 1);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }

#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float o[4];
      col_sum4(y[t][g], nf[g], o);
      const uint32_t tile = tile0 + t, col = g * 8 + r;
      if (tile < tiles && r < 8 && col < N) epilogue4<EPI>(ea, tile * 16 + 4 * g4, col, o, ks);
    }
}

// ------------------------------------------------------------------ wide f16 GEMM

// The reference's arithmetic for matmuls of N >= 32 columns
// (ops/matmul.rs:433-446 -> mul_mm_cm.slang): every weight dequantized in f32
// and rounded to f16 (stage_a_tile, the Q4_K line
// f16(dall * sc * nibble - dmin * mb)), every activation rounded to f16,
// products accumulated in f32. Here the activations arrive as f16 rows
// bh[col][k] (k_prep16_*), the weights are decoded from the Q4_K tiles into
// the MFMA A fragment as f16(fma(d sc, q, -dmin m)) (one rounding from the
// exact value; the f32 product then f16 of the reference may differ in the last
// f16 bit), and v_mfma_f32_16x16x32_f16 accumulates over the whole K-split.

// The part of a Q4_K tile-superblock one lane needs for its A row r = lane % 16:
// the eight sub-block words, d | dmin of row r and its 12 scale bytes.
struct Q4TileR {
  u32x4 q0, q1;
  uint32_t dd, s0, s1, s2;
  __device__ void pin() { pin32(q0); pin32(q1); pin32(dd); pin32(s0); pin32(s1); pin32(s2); }
};
__device__ __forceinline__ Q4TileR load_q4_tile_r(const uint8_t* base, int lane, int r) {
  Q4TileR a;
  a.q0 = ldw16(base + 16 * lane);
  a.q1 = ldw16(base + 1024 + 16 * lane);
  a.dd = *(const uint32_t*)(base + 2048 + 4 * r);
  const uint32_t* sp = (const uint32_t*)(base + 2112 + 12 * r);
  a.s0 = sp[0];
  a.s1 = sp[1];
  a.s2 = sp[2];
  return a;
}
// Per superblock: the words and, per sub-block m, the lane row's a_m = d sc_m
// (as 2^24 a_m and 2^20 a_m, exact power-of-two scalings) and b_m = dmin m_m
// (the Q4_K 6-bit unpack of q4_decode_setup).
struct Q4DecR {
  uint32_t w[8];
  float a24[8], a20[8], nb[8];
};
__device__ __forceinline__ Q4DecR q4r_setup(const Q4TileR& t) {
  Q4DecR s;
  s.w[0] = t.q0.x; s.w[1] = t.q0.y; s.w[2] = t.q0.z; s.w[3] = t.q0.w;
  s.w[4] = t.q1.x; s.w[5] = t.q1.y; s.w[6] = t.q1.z; s.w[7] = t.q1.w;
  const uint32_t sc03 = t.s0 & 0x3F3F3F3Fu, m03 = t.s1 & 0x3F3F3F3Fu;
  const uint32_t sc47 = (t.s2 & 0x0F0F0F0Fu) | ((t.s0 >> 2) & 0x30303030u);
  const uint32_t m47 = ((t.s2 >> 4) & 0x0F0F0F0Fu) | ((t.s1 >> 2) & 0x30303030u);
  const float d24 = (float)as_h2(t.dd).x * 16777216.0f, ndmin = -(float)as_h2(t.dd).y;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    s.a24[j] = d24 * (float)((sc03 >> (8 * j)) & 0xFFu);
    s.a24[4 + j] = d24 * (float)((sc47 >> (8 * j)) & 0xFFu);
    s.nb[j] = ndmin * (float)((m03 >> (8 * j)) & 0xFFu);
    s.nb[4 + j] = ndmin * (float)((m47 >> (8 * j)) & 0xFFu);
  }
#pragma unroll
  for (int m = 0; m < 8; ++m) s.a20[m] = s.a24[m] * 0.0625f;
  return s;
}
// A fragment of sub-block m: element t (k = 32 m + 8 g + t) = f16(a_m q_t - b_m).
// A nibble masked in place is an f16 subnormal: q 2^-24 (pairs t = 0, 1 and 4,
// 5, nibbles at bits 0 / 16) or q 2^-20 (t = 2, 3 and 6, 7, at bits 4 / 20),
// which v_fma_mix reads exactly (f16 denormals are kept), so with 2^24 a_m and
// 2^20 a_m every product is a_m q. v_fma_mixlo / mixhi_f16 round the exact
// a q - b once to f16 (written as asm: left to itself the compiler mixes these
// with f32 FMAs plus conversions, which round twice and cost more).
__device__ __forceinline__ uint32_t fma_mix_pair(uint32_t p, float a, float c) {
  uint32_t r;
  asm("v_fma_mixlo_f16 %0, %1, %2, %3 op_sel_hi:[1,0,0]\n\t"
      "v_fma_mixhi_f16 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
      : "=&v"(r)
      : "v"(p), "v"(a), "v"(c));
  return r;
}
__device__ __forceinline__ h8 q4r_frag16(const Q4DecR& s, int m) {
  const uint32_t w = s.w[m], w8 = w >> 8;
  u32x4 r;
  r.x = fma_mix_pair(w & 0x000F000Fu, s.a24[m], s.nb[m]);
  r.y = fma_mix_pair(w & 0x00F000F0u, s.a20[m], s.nb[m]);
  r.z = fma_mix_pair(w8 & 0x000F000Fu, s.a24[m], s.nb[m]);
  r.w = fma_mix_pair(w8 & 0x00F000F0u, s.a20[m], s.nb[m]);
  return as_h8(r);
}

// y = W x over N <= 16 NC columns of f16 rows bh [N][ldb] (K of W), W Q4_K. A
// workgroup of 8 waves covers 8 row tiles (wave w: tile blockIdx.x * 8 + w;
// two waves per SIMD hide each other's decode latencies) over the
// superblocks of split blockIdx.y. Every
// operand goes through a ring of three LDS stages filled by direct
// global->LDS loads two superblocks ahead of the compute: per superblock the
// NC x 8 B fragments (16 columns x 32 k each; columns past N read column
// N - 1, their sums are dropped) and the wave's weight tile (2304 B, as two
// 1 KB and one 256 B load). All of a wave's loads are its own asm
// loads, so the wait for a stage is an exact count of the loads issued after
// it. Each weight tile's f16 fragment feeds NC MFMAs; the sums stay in the
// MFMA accumulators over the whole split. EPI_PART: partials
// [split][col][row]; EPI_STORE (one split): out[col][row], rows < ea.rows.
template <int NC>
struct G16Smem {
  static constexpr int kStages = NC <= 2 ? 4 : 3;       // ring depth within the LDS

  static constexpr uint32_t kB = NC * 8 * 64;           // h8 elements of one stage's B fragments
  static constexpr uint32_t kW = 8 * SH_Q4K_TILE_BYTES;  // bytes of one stage's weight tiles
};

template <int NC, int EPI>
__global__ __launch_bounds__(512) void k_gemm16_q4k(const uint8_t* __restrict__ Wp, uint32_t tiles, uint32_t nsb,
                                                    uint32_t S, const uint16_t* __restrict__ Bh, uint32_t ldb,
                                                    uint32_t N, EpiArgs ea) {
  constexpr int T = 1, WV = 8;
  constexpr uint32_t kB = G16Smem<NC>::kB, kW = G16Smem<NC>::kW;
  constexpr int kLoads = NC + 3 * T;  // one wave's direct loads per stage
  constexpr int G16_STAGES = G16Smem<NC>::kStages;
  __shared__ h8 sB[G16_STAGES][kB];
  __shared__ __attribute__((aligned(16))) uint8_t sW[G16_STAGES][kW];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g4 = lane >> 4, r = lane & 15;
  const uint32_t ks = blockIdx.y, sb0 = ks * S, sb1 = min(sb0 + S, nsb), nst = sb1 - sb0;
  const uint32_t tile0 = (blockIdx.x * WV + wave) * T;

  auto issue = [&](uint32_t sb, int buf) {
    for (uint32_t fi = wave; fi < (uint32_t)(NC * 8); fi += WV) {  // NC per wave
      const uint32_t c = fi >> 3, m = fi & 7;
      const uint32_t col = min(16 * c + (uint32_t)r, N - 1);
      sh_dma16(Bh + (size_t)col * ldb + 256 * sb + 32 * m + 8 * g4, &sB[buf][fi * 64]);
    }
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const uint32_t tt = tile0 + t < tiles ? tile0 + t : tiles - 1;  // clamp keeps loads in bounds
      const uint8_t* src = Wp + ((size_t)tt * nsb + sb) * SH_Q4K_TILE_BYTES;
      uint8_t* dst = &sW[buf][(wave * T + t) * SH_Q4K_TILE_BYTES];
      sh_dma16_nt(src + 16 * lane, dst);
      sh_dma16_nt(src + 1024 + 16 * lane, dst + 1024);
      sh_dma4_nt(src + 2048 + 4 * lane, dst + 2048);
    }
  };

  f4 acc[T][NC];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[t][c] = f4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int buf) {
    Q4DecR dec[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const uint8_t* w = &sW[buf][(wave * T + t) * SH_Q4K_TILE_BYTES];
      Q4TileR a;
      a.q0 = *(const u32x4*)(w + 16 * lane);
      a.q1 = *(const u32x4*)(w + 1024 + 16 * lane);
      a.dd = *(const uint32_t*)(w + 2048 + 4 * r);
      const uint32_t* sp = (const uint32_t*)(w + 2112 + 12 * r);
      a.s0 = sp[0];
      a.s1 = sp[1];
      a.s2 = sp[2];
      dec[t] = q4r_setup(a);
    }
    h8 bb[2][NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) bb[0][c] = sB[buf][(c * 8) * 64 + lane];
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const int cur = m & 1;
      if (m < 7) {
#pragma unroll
        for (int c = 0; c < NC; ++c) bb[cur ^ 1][c] = sB[buf][(c * 8 + m + 1) * 64 + lane];
      }
      __builtin_amdgcn_sched_barrier(0);  // keep those reads ahead of this sub-block's MFMAs
      h8 a[T];
#pragma unroll
      for (int t = 0; t < T; ++t) a[t] = q4r_frag16(dec[t], m);
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int t = 0; t < T; ++t) acc[t][c] = mfma16(a[t], bb[cur][c], acc[t][c]);
    }
  };

  constexpr int kAhead = G16_STAGES - 1;  // stages in flight ahead of the compute
  for (int j = 0; j < kAhead; ++j)
    if ((uint32_t)j < nst) issue(sb0 + j, j);
  for (uint32_t i = 0; i < nst; ++i) {
    // stage i landed (the later ones may still be in flight), and every wave
    // is done with stage i - 1, whose buffer stage i + kAhead now refills
    const uint32_t later = min(nst - 1 - i, (uint32_t)(kAhead - 1));
    if (later >= 2) sh_wait_vm<2 * kLoads>();
    else if (later == 1) sh_wait_vm<kLoads>();
    else sh_wait_vm<0>();
    __syncthreads();
    if (i + kAhead < nst) issue(sb0 + i + kAhead, (i + kAhead) % G16_STAGES);
    compute(i % G16_STAGES);
  }

#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const uint32_t tile = tile0 + t, col = 16 * c + r, row0 = tile * 16 + 4 * g4;
      if (tile >= tiles || col >= N) continue;
      const f4 v = acc[t][c];
      if (EPI == EPI_PART) {
        *(float4*)(ea.out + ks * ea.part_stride + (size_t)col * ea.ldo + row0) = make_float4(v[0], v[1], v[2], v[3]);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (row0 + j < ea.rows) ea.out[(size_t)col * ea.ldo + row0 + j] = v[j];
      }
    }
}

// y = W x over 64 < N <= 16 NC columns (up to 192) of f16 rows bh [N][ldb],
// W Q4_K: one pass over the weights for every column of a wide call. A
// workgroup of 8 waves (two per SIMD) covers 16 row tiles, wave w tiles
// (blockIdx.x * 8 + w) * 2 + t, over the superblocks of split blockIdx.y, in
// stages of half a superblock (sub-blocks 4h .. 4h + 3). A wave decodes each
// of its 2 tiles' f16 fragments once per sub-block and feeds it to NC MFMAs,
// each B fragment read from LDS feeds 2: the decode is ~2.5 VALU instructions
// per MFMA at 192 columns. B goes through two LDS buffers by direct loads and
// the weight words to registers, both one stage ahead of the compute.
template <int NC, int EPI>
__global__ __launch_bounds__(512) void k_gemm16w_q4k(const uint8_t* __restrict__ Wp, uint32_t tiles, uint32_t nsb,
                                                     uint32_t S, const uint16_t* __restrict__ Bh, uint32_t ldb,
                                                     uint32_t N, EpiArgs ea) {
  constexpr int T = 2, WV = 8;
  __shared__ h8 sB[2][NC * 4 * 64];  // [buffer][(column group * 4 + sub-block) * 64 + lane]
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g4 = lane >> 4, r = lane & 15;
  const uint32_t ks = blockIdx.y, sb0 = ks * S, sb1 = min(sb0 + S, nsb), nst = 2 * (sb1 - sb0);
  const uint32_t tile0 = (blockIdx.x * WV + wave) * T;
  const uint8_t* tb[T];
#pragma unroll
  for (int t = 0; t < T; ++t)  // clamped tiles keep the loads in bounds; their sums are dropped
    tb[t] = Wp + (size_t)(tile0 + t < tiles ? tile0 + t : tiles - 1) * nsb * SH_Q4K_TILE_BYTES;

  struct WStage {
    u32x4 q[T];
    uint32_t dd[T], s0[T], s1[T], s2[T];
  };
  auto load_w = [&](uint32_t s, WStage& w) __attribute__((always_inline)) {
    const uint32_t sb = sb0 + (s >> 1), h = s & 1;
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const uint8_t* base = tb[t] + (size_t)sb * SH_Q4K_TILE_BYTES;
      w.q[t] = ldw16(base + 1024 * h + 16 * lane);
      w.dd[t] = *(const uint32_t*)(base + 2048 + 4 * r);
      const uint32_t* sp = (const uint32_t*)(base + 2112 + 12 * r);
      w.s0[t] = sp[0];
      w.s1[t] = sp[1];
      w.s2[t] = sp[2];
    }
  };
  auto issue_b = [&](uint32_t s, int buf) __attribute__((always_inline)) {
    const uint32_t sb = sb0 + (s >> 1), h = s & 1;
    for (uint32_t fi = wave; fi < (uint32_t)(NC * 4); fi += WV) {  // NC / 2 per wave
      const uint32_t c = fi >> 2, mp = fi & 3;
      const uint32_t col = min(16 * c + (uint32_t)r, N - 1);
      sh_dma16(Bh + (size_t)col * ldb + 256 * sb + 32 * (4 * h + mp) + 8 * g4, &sB[buf][fi * 64]);
    }
  };

  f4 acc[T][NC];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[t][c] = f4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](const WStage& w, int buf, int h) __attribute__((always_inline)) {
    // the Q4_K 6-bit unpack of sub-blocks 4h .. 4h + 3 (q4_decode_setup)
    uint32_t scw[T], mw[T];
    float d24[T], ndmin[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      scw[t] = h == 0 ? (w.s0[t] & 0x3F3F3F3Fu) : ((w.s2[t] & 0x0F0F0F0Fu) | ((w.s0[t] >> 2) & 0x30303030u));
      mw[t] = h == 0 ? (w.s1[t] & 0x3F3F3F3Fu) : (((w.s2[t] >> 4) & 0x0F0F0F0Fu) | ((w.s1[t] >> 2) & 0x30303030u));
      d24[t] = (float)as_h2(w.dd[t]).x * 16777216.0f;
      ndmin[t] = -(float)as_h2(w.dd[t]).y;
    }
#pragma unroll
    for (int mp = 0; mp < 4; ++mp) {
      // every B fragment of the sub-block requested before the decode, so the
      // LDS latency overlaps it and the MFMAs below never wait on a read
      h8 bb[NC];
#pragma unroll
      for (int c = 0; c < NC; ++c) bb[c] = sB[buf][(c * 4 + mp) * 64 + lane];
      __builtin_amdgcn_sched_barrier(0);
      h8 a[T];
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const float a24 = d24[t] * (float)((scw[t] >> (8 * mp)) & 0xFFu), a20 = a24 * 0.0625f;
        const float nb = ndmin[t] * (float)((mw[t] >> (8 * mp)) & 0xFFu);
        const uint32_t word = mp == 0 ? w.q[t].x : mp == 1 ? w.q[t].y : mp == 2 ? w.q[t].z : w.q[t].w;
        const uint32_t w8 = word >> 8;
        u32x4 v;
        v.x = fma_mix_pair(word & 0x000F000Fu, a24, nb);
        v.y = fma_mix_pair(word & 0x00F000F0u, a20, nb);
        v.z = fma_mix_pair(w8 & 0x000F000Fu, a24, nb);
        v.w = fma_mix_pair(w8 & 0x00F000F0u, a20, nb);
        a[t] = as_h8(v);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int t = 0; t < T; ++t) acc[t][c] = mfma16(a[t], bb[c], acc[t][c]);
    }
  };

  WStage w0, w1;
  issue_b(0, 0);
  load_w(0, w0);
  auto step = [&](uint32_t s, WStage& cur, WStage& nxt, int u) __attribute__((always_inline)) {
    // B and weights of stage s landed; every wave is done with stage s - 1's
    // B buffer, which stage s + 1 now refills (its weights follow its B)
    sh_wait_vm<0>();
    __syncthreads();
    if (s + 1 < nst) {
      issue_b(s + 1, (u + 1) & 1);
      load_w(s + 1, nxt);
    }
    compute(cur, u & 1, u & 1);
  };
  for (uint32_t s = 0; s < nst; s += 2) {
    step(s, w0, w1, 0);
    if (s + 1 < nst) step(s + 1, w1, w0, 1);
  }

#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const uint32_t tile = tile0 + t, col = 16 * c + r, row0 = tile * 16 + 4 * g4;
      if (tile >= tiles || col >= N) continue;
      const f4 v = acc[t][c];
      if (EPI == EPI_PART) {
        *(float4*)(ea.out + ks * ea.part_stride + (size_t)col * ea.ldo + row0) = make_float4(v[0], v[1], v[2], v[3]);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (row0 + j < ea.rows) ea.out[(size_t)col * ea.ldo + row0 + j] = v[j];
      }
    }
}

// k_gemm16w_q4k with a deeper weight pipeline: the weight words and row
// headers (16 tiles x 1280 B per stage of half a superblock, from HBM) go
// through a ring of three LDS buffers two stages ahead of the compute, B
// through two buffers one stage ahead (from L2). Every load is the wave's own
// direct load, issued per step as B(s + 1), then W(s + 2), so the wait for
// stage s leaves exactly the 2 T weight loads of stage s + 1 in flight.
// LDS: 2 x NC x 4 KB + 3 x 20 KB (156 KB at NC = 12).
template <int NC, int EPI>
__global__ __launch_bounds__(512) void k_gemm16w3_q4k(const uint8_t* __restrict__ Wp, uint32_t tiles, uint32_t nsb,
                                                      uint32_t S, const uint16_t* __restrict__ Bh, uint32_t ldb,
                                                      uint32_t N, EpiArgs ea) {
  constexpr int T = 2, WV = 8, WSTG = 3;
  constexpr uint32_t kTW = 1280;  // one tile's stage: 1 KB of words + the 256 B row header
  __shared__ h8 sB[2][NC * 4 * 64];  // [buffer][(column group * 4 + sub-block) * 64 + lane]
  __shared__ __attribute__((aligned(16))) uint8_t sW[WSTG][WV * T * kTW];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g4 = lane >> 4, r = lane & 15;
  const uint32_t ks = blockIdx.y, sb0 = ks * S, sb1 = min(sb0 + S, nsb), nst = 2 * (sb1 - sb0);
  const uint32_t tile0 = (blockIdx.x * WV + wave) * T;

  auto issue_b = [&](uint32_t s, int buf) __attribute__((always_inline)) {
    const uint32_t sb = sb0 + (s >> 1), h = s & 1;
    for (uint32_t fi = wave; fi < (uint32_t)(NC * 4); fi += WV) {  // NC / 2 per wave
      const uint32_t c = fi >> 2, mp = fi & 3;
      const uint32_t col = min(16 * c + (uint32_t)r, N - 1);
      sh_dma16(Bh + (size_t)col * ldb + 256 * sb + 32 * (4 * h + mp) + 8 * g4, &sB[buf][fi * 64]);
    }
  };
  auto issue_w = [&](uint32_t s, int buf) __attribute__((always_inline)) {
    const uint32_t sb = sb0 + (s >> 1), h = s & 1;
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const uint32_t tt = tile0 + t < tiles ? tile0 + t : tiles - 1;  // clamp keeps loads in bounds
      const uint8_t* src = Wp + ((size_t)tt * nsb + sb) * SH_Q4K_TILE_BYTES;
      uint8_t* dst = &sW[buf][(wave * T + t) * kTW];
      sh_dma16_nt(src + 1024 * h + 16 * lane, dst);
      sh_dma4_nt(src + 2048 + 4 * lane, dst + 1024);
    }
  };

  f4 acc[T][NC];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[t][c] = f4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int bb_buf, int w_buf, uint32_t h) __attribute__((always_inline)) {
    u32x4 q[T];
    uint32_t scw[T], mw[T];
    float d24[T], ndmin[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const uint8_t* wt = &sW[w_buf][(wave * T + t) * kTW];
      q[t] = *(const u32x4*)(wt + 16 * lane);
      const uint32_t dd = *(const uint32_t*)(wt + 1024 + 4 * r);
      const uint32_t* sp = (const uint32_t*)(wt + 1024 + 64 + 12 * r);
      const uint32_t s0 = sp[0], s1 = sp[1], s2 = sp[2];
      // the Q4_K 6-bit unpack of sub-blocks 4h .. 4h + 3 (q4_decode_setup)
      scw[t] = h == 0 ? (s0 & 0x3F3F3F3Fu) : ((s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u));
      mw[t] = h == 0 ? (s1 & 0x3F3F3F3Fu) : (((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u));
      d24[t] = (float)as_h2(dd).x * 16777216.0f;
      ndmin[t] = -(float)as_h2(dd).y;
    }
#pragma unroll
    for (int mp = 0; mp < 4; ++mp) {
      h8 bb[NC];
#pragma unroll
      for (int c = 0; c < NC; ++c) bb[c] = sB[bb_buf][(c * 4 + mp) * 64 + lane];
      __builtin_amdgcn_sched_barrier(0);
      h8 a[T];
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const float a24 = d24[t] * (float)((scw[t] >> (8 * mp)) & 0xFFu), a20 = a24 * 0.0625f;
        const float nb = ndmin[t] * (float)((mw[t] >> (8 * mp)) & 0xFFu);
        const uint32_t word = mp == 0 ? q[t].x : mp == 1 ? q[t].y : mp == 2 ? q[t].z : q[t].w;
        const uint32_t w8 = word >> 8;
        u32x4 v;
        v.x = fma_mix_pair(word & 0x000F000Fu, a24, nb);
        v.y = fma_mix_pair(word & 0x00F000F0u, a20, nb);
        v.z = fma_mix_pair(w8 & 0x000F000Fu, a24, nb);
        v.w = fma_mix_pair(w8 & 0x00F000F0u, a20, nb);
        a[t] = as_h8(v);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int t = 0; t < T; ++t) acc[t][c] = mfma16(a[t], bb[c], acc[t][c]);
    }
  };

  // prologue: W(0), B(0), W(1) (the same order as the steps' B(s + 1), W(s + 2))
  issue_w(0, 0);
  issue_b(0, 0);
  if (nst > 1) issue_w(1, 1);
  for (uint32_t s = 0; s < nst; ++s) {
    // B(s) and W(s) landed (W(s + 1), issued after them, may still be in
    // flight); every wave is done with stage s - 1's buffers, which B(s + 1)
    // and W(s + 2) now refill
    if (s + 1 < nst) sh_wait_vm<2 * T>();
    else sh_wait_vm<0>();
    __syncthreads();
    // the buffer indices as wave-uniform values (the direct loads take their
    // LDS address in M0)
    const int wb = __builtin_amdgcn_readfirstlane((int)(s % WSTG));
    const int bb = __builtin_amdgcn_readfirstlane((int)(s & 1));
    if (s + 1 < nst) issue_b(s + 1, bb ^ 1);
    if (s + 2 < nst) issue_w(s + 2, wb == 0 ? 2 : wb - 1);
    compute(bb, wb, s & 1);
  }

#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const uint32_t tile = tile0 + t, col = 16 * c + r, row0 = tile * 16 + 4 * g4;
      if (tile >= tiles || col >= N) continue;
      const f4 v = acc[t][c];
      if (EPI == EPI_PART) {
        *(float4*)(ea.out + ks * ea.part_stride + (size_t)col * ea.ldo + row0) = make_float4(v[0], v[1], v[2], v[3]);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (row0 + j < ea.rows) ea.out[(size_t)col * ea.ldo + row0 + j] = v[j];
      }
    }
}

// y = W x for 64 < N <= 192 columns in column blocks of 16 NCH columns: a
// workgroup of 8 waves covers 16 row tiles (wave w: tiles 2 (16 rb + w) + t)
// and one column block over the superblocks of split blockIdx.y. The ncb
// column blocks of a row block are 8 workgroups apart, so they run on one XCD
// and the later ones find the weight tiles in its L2. Every operand goes
// through a ring of three LDS stages of half a superblock (B fragments and the
// waves' weight words with their row headers) filled by direct loads two
// stages ahead; all of a wave's loads are its own asm loads, so the wait for
// a stage is an exact count. Each decoded fragment feeds NCH MFMAs, each B
// fragment 2.
template <int NCH, int EPI>
__global__ __launch_bounds__(512) void k_gemm16h_q4k(const uint8_t* __restrict__ Wp, uint32_t tiles, uint32_t nsb,
                                                     uint32_t S, const uint16_t* __restrict__ Bh, uint32_t ldb,
                                                     uint32_t N, uint32_t ncb, EpiArgs ea) {
  constexpr int T = 2, WV = 8, STG = 3;
  constexpr uint32_t kB = NCH * 4 * 64;                  // h8 of one stage's B fragments
  constexpr uint32_t kTW = 1280;                         // one tile's stage: 1 KB of words + the 256 B row header
  constexpr int kLoadsMin = (NCH * 4) / WV + 2 * T;      // fewest direct loads of one wave per stage
  __shared__ h8 sB[STG][kB];
  __shared__ __attribute__((aligned(16))) uint8_t sW[STG][WV * T * kTW];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g4 = lane >> 4, r = lane & 15;
  const uint32_t grp = blockIdx.x / (8 * ncb), within = blockIdx.x % (8 * ncb);
  const uint32_t cb = within / 8, rb = grp * 8 + within % 8;
  if (rb * WV * T >= tiles) return;  // whole workgroup: the last group of 8 row blocks may be short
  const uint32_t tile0 = (rb * WV + wave) * T, col0 = cb * NCH * 16;
  const uint32_t ks = blockIdx.y, sb0 = ks * S, sb1 = min(sb0 + S, nsb), nst = 2 * (sb1 - sb0);

  auto issue = [&](uint32_t s, int buf) __attribute__((always_inline)) {
    const uint32_t sb = sb0 + (s >> 1), h = s & 1;
    for (uint32_t fi = wave; fi < (uint32_t)(NCH * 4); fi += WV) {
      const uint32_t c = fi >> 2, mp = fi & 3;
      const uint32_t col = min(col0 + 16 * c + (uint32_t)r, N - 1);
      sh_dma16(Bh + (size_t)col * ldb + 256 * sb + 32 * (4 * h + mp) + 8 * g4, &sB[buf][fi * 64]);
    }
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const uint32_t tt = tile0 + t < tiles ? tile0 + t : tiles - 1;  // clamp keeps loads in bounds
      const uint8_t* src = Wp + ((size_t)tt * nsb + sb) * SH_Q4K_TILE_BYTES;
      uint8_t* dst = &sW[buf][(wave * T + t) * kTW];
      sh_dma16_nt(src + 1024 * h + 16 * lane, dst);
      sh_dma4_nt(src + 2048 + 4 * lane, dst + 1024);
    }
  };

  f4 acc[T][NCH];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int c = 0; c < NCH; ++c) acc[t][c] = f4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int buf, uint32_t h) __attribute__((always_inline)) {
    u32x4 q[T];
    uint32_t scw[T], mw[T];
    float d24[T], ndmin[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const uint8_t* wt = &sW[buf][(wave * T + t) * kTW];
      q[t] = *(const u32x4*)(wt + 16 * lane);
      const uint32_t dd = *(const uint32_t*)(wt + 1024 + 4 * r);
      const uint32_t* sp = (const uint32_t*)(wt + 1024 + 64 + 12 * r);
      const uint32_t s0 = sp[0], s1 = sp[1], s2 = sp[2];
      // the Q4_K 6-bit unpack of sub-blocks 4h .. 4h + 3 (q4_decode_setup)
      scw[t] = h == 0 ? (s0 & 0x3F3F3F3Fu) : ((s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u));
      mw[t] = h == 0 ? (s1 & 0x3F3F3F3Fu) : (((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u));
      d24[t] = (float)as_h2(dd).x * 16777216.0f;
      ndmin[t] = -(float)as_h2(dd).y;
    }
#pragma unroll
    for (int mp = 0; mp < 4; ++mp) {
      h8 bb[NCH];
#pragma unroll
      for (int c = 0; c < NCH; ++c) bb[c] = sB[buf][(c * 4 + mp) * 64 + lane];
      __builtin_amdgcn_sched_barrier(0);
      h8 a[T];
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const float a24 = d24[t] * (float)((scw[t] >> (8 * mp)) & 0xFFu), a20 = a24 * 0.0625f;
        const float nb = ndmin[t] * (float)((mw[t] >> (8 * mp)) & 0xFFu);
        const uint32_t word = mp == 0 ? q[t].x : mp == 1 ? q[t].y : mp == 2 ? q[t].z : q[t].w;
        const uint32_t w8 = word >> 8;
        u32x4 v;
        v.x = fma_mix_pair(word & 0x000F000Fu, a24, nb);
        v.y = fma_mix_pair(word & 0x00F000F0u, a20, nb);
        v.z = fma_mix_pair(w8 & 0x000F000Fu, a24, nb);
        v.w = fma_mix_pair(w8 & 0x00F000F0u, a20, nb);
        a[t] = as_h8(v);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int c = 0; c < NCH; ++c)
#pragma unroll
        for (int t = 0; t < T; ++t) acc[t][c] = mfma16(a[t], bb[c], acc[t][c]);
    }
  };

#pragma unroll
  for (int j = 0; j < STG - 1; ++j)
    if ((uint32_t)j < nst) issue(j, j);
  for (uint32_t s = 0; s < nst; ++s) {
    // stage s landed (stage s + 1 may still be in flight), and every wave is
    // done with stage s - 1, whose buffer stage s + 2 now refills
    if (s + 1 < nst) sh_wait_vm<kLoadsMin>();
    else sh_wait_vm<0>();
    __syncthreads();
    if (s + STG - 1 < nst) issue(s + STG - 1, (s + STG - 1) % STG);
    compute(s % STG, s & 1);
  }

#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const uint32_t tile = tile0 + t, col = col0 + 16 * c + r, row0 = tile * 16 + 4 * g4;
      if (tile >= tiles || col >= N) continue;
      const f4 v = acc[t][c];
      if (EPI == EPI_PART) {
        *(float4*)(ea.out + ks * ea.part_stride + (size_t)col * ea.ldo + row0) = make_float4(v[0], v[1], v[2], v[3]);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (row0 + j < ea.rows) ea.out[(size_t)col * ea.ldo + row0 + j] = v[j];
      }
    }
}

// QKV from the multi-group kernel's split partials: per column (blockIdx.y) and
// 4 rows per thread, the split sum, then RoPE and the KV-cache writes.
__global__ __launch_bounds__(64) void k_qkv_finish(const float* __restrict__ part, uint32_t nparts,
                                                   size_t part_stride, uint32_t ldp, EpiArgs ea, QkvCols qc) {
  const uint32_t col = blockIdx.y, r0 = qc.row0 + 4 * (blockIdx.x * 64 + threadIdx.x);
  if (r0 >= ea.Dq + 2 * ea.Dkv) return;
  const float* p = part + (size_t)col * ldp + r0;
  if (qc.vpart && r0 >= ea.Dq + ea.Dkv) {  // v rows of their own matrix (4 rows never straddle: hd % 4 == 0)
    p = qc.vpart + (size_t)col * qc.vldp + (r0 - ea.Dq - ea.Dkv);
    nparts = qc.vnparts;
    part_stride = qc.vstride;
  }
  float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
  for (uint32_t k0 = 0; k0 < nparts; k0 += 8) {  // 8 loads in flight, split order kept
    float4 t[8];
#pragma unroll
    for (uint32_t j = 0; j < 8; ++j) t[j] = *(const float4*)(p + min(k0 + j, nparts - 1) * part_stride);
#pragma unroll
    for (uint32_t j = 0; j < 8; ++j)
      if (k0 + j < nparts) { s.x += t[j].x; s.y += t[j].y; s.z += t[j].z; s.w += t[j].w; }
  }
  const float v[4] = {s.x, s.y, s.z, s.w};
  if (qc.tab) {
    const QkvColDev t = qc.tab[col];
    qkv_store4(ea, r0, v, t.pos, t.slot, t.mseq, t.kc, t.vc, ea.out + (size_t)col * ea.Dq);
  } else {
    const uint32_t b0 = ea.dbase ? *ea.dbase : 0u;  // graph replay: offsets from the device base
    qkv_store4(ea, r0, v, qc.pos[col] + (int32_t)b0, qc.slot[col] + b0, qc.mseq[col], qc.kc[col], qc.vc[col],
               ea.out + (size_t)col * ea.Dq);
  }
}

// QKV of a qwen3 layer from split partials (models/qwen3.rs:330-362): one
// workgroup of hd threads per (head, column), thread i owning row i of the
// head. The split sum; for q and k heads the per-head RMSNorm over head_dim
// with weight w[i] (rms_norm.slang:39-55 over rows of head_dim) and RoPE, NEOX
// (pair (i, i + hd/2), rope_funcs.slang rope_neox) or NORM (pair (2j, 2j+1));
// q rows to ea.out [col][Dq], roped k rows and raw v rows to the column's
// cache slot (V slot-permuted within its 32-key block).
__global__ __launch_bounds__(128) void k_qkv_finish_head(const float* __restrict__ part, uint32_t nparts,
                                                          size_t part_stride, uint32_t ldp, EpiArgs ea, QkvCols qc,
                                                          const float* __restrict__ q_norm,
                                                          const float* __restrict__ k_norm, float eps, int neox) {
  __shared__ float sy[128];
  __shared__ float sw[2];
  const uint32_t h = blockIdx.x, col = blockIdx.y, i = threadIdx.x, hd = ea.hd, half = hd / 2;
  const uint32_t nq = ea.Dq / hd, nkv = ea.n_kv;
  const int kind = h < nq ? 0 : (h < nq + nkv ? 1 : 2);  // q, k, v
  const uint32_t hh = kind == 0 ? h : (kind == 1 ? h - nq : h - nq - nkv);
  const uint32_t row = kind == 0 ? hh * hd + i : (kind == 1 ? ea.Dq + hh * hd + i : ea.Dq + ea.Dkv + hh * hd + i);
  const float* p = part + (size_t)col * ldp + row;
  if (kind == 2 && qc.vpart) {  // v rows of their own matrix
    p = qc.vpart + (size_t)col * qc.vldp + hh * hd + i;
    nparts = qc.vnparts;
    part_stride = qc.vstride;
  }
  float v = 0.f;
  for (uint32_t k0 = 0; k0 < nparts; k0 += 8) {  // 8 loads in flight, split order kept
    float t[8];
#pragma unroll
    for (uint32_t j = 0; j < 8; ++j) t[j] = p[(size_t)min(k0 + j, nparts - 1) * part_stride];
#pragma unroll
    for (uint32_t j = 0; j < 8; ++j)
      if (k0 + j < nparts) v += t[j];
  }
  const uint32_t b0 = ea.dbase ? *ea.dbase : 0u;  // graph replay: offsets from the device base
  const int32_t pos = qc.pos[col] + (int32_t)b0;
  const uint32_t slot = qc.slot[col] + b0, ms = qc.mseq[col];
  if (kind == 2) {
    uint16_t* vb = qc.vc[col] + (((size_t)ea.layer * nkv + hh) * (ms / 32) + slot / 32) * hd * 32;
    vb[(size_t)i * 32 + v_slot(slot & 31)] = f2h_bits(v);
    return;  // uniform per workgroup
  }
  const float* w = kind == 0 ? q_norm : k_norm;
  if (w) {
    float ss = v * v;
    for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
    if ((i & 63) == 0) sw[i >> 6] = ss;
    __syncthreads();
    ss = hd > 64 ? sw[0] + sw[1] : sw[0];
    v = v * (1.0f / sqrtf(ss / (float)hd + eps)) * w[i];
  }
  sy[i] = v;
  __syncthreads();
  float o;
  if (neox) {
    const uint32_t j = i < half ? i : i - half;
    const float2 cs = ea.rope[(size_t)pos * half + j];
    o = i < half ? v * cs.x - sy[i + half] * cs.y : sy[i - half] * cs.y + v * cs.x;
  } else {
    const float2 cs = ea.rope[(size_t)pos * half + i / 2];
    o = (i & 1) ? sy[i - 1] * cs.y + v * cs.x : v * cs.x - sy[i + 1] * cs.y;
  }
  if (kind == 0) {
    ea.out[(size_t)col * ea.Dq + row] = o;
  } else {
    qc.kc[col][(((size_t)ea.layer * nkv + hh) * ms + slot) * hd + i] = f2h_bits(o);
  }
}

// ------------------------------------------------------------------ K-quant expert-indirect

// Expert-indirect GEMM of a routed MoE FFN (the MUL_MAT_ID matvec of
// ops/moe.rs:164 / the mul_mat_vec_q*_k shaders' id variant, here batched over
// the columns routed to each expert), W in K-quant format F: E expert slabs of
// tiles_e row tiles.
// Chunk c of the routing plan, info[1 + 3c .. +3] = (expert e, first sorted
// pair p0, n <= 8 pairs), multiplies slab e by the operand columns col[p]
// (the pairs' input columns, gathered lane by lane from the operand groups;
// col == null: column p) and stores the slab's rows for pair p at out[p][row]
// (EPI_STORE, whole K in one workgroup). Grid: max chunks x rb_e row blocks
// of 8 T tiles; workgroups past info[0] chunks exit at once. The superblock
// pipeline (operand fragments staged in LDS by direct loads, two buffers) is
// the multi-group kernel's with one gathered group. T = 2 is held to 128
// VGPRs (4 waves per SIMD: two workgroups per CU; 132 unbounded, one spilled
// register at the bound): the experts' gate/up 2.74 -> 2.50 ms per step of the
// 8 x 7-column Qwen3-30B-A3B-shape verify. Three workgroups of T = 1 per CU
// (80 VGPRs, spills) made the down slower (1.53 -> 1.60 ms).
template <class F, int T>
__global__ __launch_bounds__(512, T == 2 ? 4 : 2) void k_moe_gemm_kq(const uint8_t* __restrict__ Wp, uint32_t tiles_e,
                                                      uint32_t nsb, uint32_t rb_e, const uint16_t* __restrict__ Bx,
                                                      const uint16_t* __restrict__ XS, const float* __restrict__ CS,
                                                      const uint32_t* __restrict__ info,
                                                      const uint32_t* __restrict__ gcol, EpiArgs ea) {
  using Tile = typename F::Tile;
  using Dec = typename F::Dec;
  constexpr int NA = F::NA;
  __shared__ h8 sB[2][9 * 64];
  __shared__ float sC[2][64];
  const uint32_t chunk = blockIdx.x / rb_e, rb = blockIdx.x % rb_e;
  if (chunk >= info[0]) return;  // uniform per workgroup
  const uint32_t e = info[1 + 3 * chunk], p0 = info[2 + 3 * chunk], n = info[3 + 3 * chunk];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g4 = lane >> 4, r = lane & 15;
  const uint32_t tile0 = (rb * 8 + wave) * T;
  const size_t gB = (size_t)nsb * 8 * 512, gX = (size_t)nsb * 512, gC = (size_t)nsb * 8;
  const uint32_t magic = __builtin_amdgcn_readfirstlane(0x64006400u);
  // this lane's column slot (lane & 7) and the operand column it gathers
  const uint32_t slot = (uint32_t)(lane & 7) < n ? (uint32_t)(lane & 7) : n - 1;
  const uint32_t col = gcol ? gcol[p0 + slot] : p0 + slot;
  const uint32_t cg = col / 8, cl = col % 8;
  const float nf = col_rinv_g(ea, cg, cl);
  const uint8_t* We = Wp + (size_t)e * tiles_e * nsb * F::kTile;

  auto stage = [&](uint32_t sb, int buf) {
    for (uint32_t fi = wave; fi < (F::kMin ? 9u : 8u); fi += 8) {
      const uint16_t* src;
      if (fi < 8) {
        src = Bx + cg * gB + ((size_t)(sb * 8 + fi) * 64 + 16 * g4 + cl + 8 * ((lane >> 3) & 1)) * 8;
      } else {  // XS: lanes 0-15 hold the sums (hi, lo), the rest zero
        const uint32_t ls = lane < 16 ? cl + 8 * ((lane >> 3) & 1) : (uint32_t)lane;
        src = XS + cg * gX + ((size_t)sb * 64 + ls) * 8;
      }
      sh_dma16(src, &sB[buf][fi * 64]);
    }
    if (wave == 7)
      sh_dma4(CS + cg * gC + sb * 8 + cl, sC[buf]);
  };
  auto a_ptr = [&](int t, uint32_t sb) {
    const uint32_t tt = tile0 + t < tiles_e ? tile0 + t : tiles_e - 1;  // clamp keeps loads in the slab
    return We + ((size_t)tt * nsb + sb) * F::kTile;
  };
  f4 y[T];
#pragma unroll
  for (int t = 0; t < T; ++t) y[t] = f4{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](const Tile (&at)[T], int buf) {
    Dec dec[T];
#pragma unroll
    for (int t = 0; t < T; ++t) dec[t] = F::setup(at[t]);
    f4 acc[T][NA];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int i = 0; i < NA; ++i) acc[t][i] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const h8 b = sB[buf][m * 64 + lane];
#pragma unroll
      for (int t = 0; t < T; ++t) {
        h8 a[NA];
        F::frag(dec[t], m, magic, a);
#pragma unroll
        for (int i = 0; i < NA; ++i) acc[t][i] = mfma16(a[i], b, acc[t][i]);
      }
    }
    h8 bm;
    if constexpr (F::kMin) bm = sB[buf][8 * 64 + lane];
    const float c = sC[buf][lane & 7];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      f4 macc = f4{0.f, 0.f, 0.f, 0.f};
      if constexpr (F::kMin) macc = mfma16(F::min_frag(dec[t], magic), bm, f4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
      for (int j = 0; j < 4; ++j) y[t][j] = y[t][j] + c * F::term(dec[t], acc[t], macc[j], j);
    }
  };
  Tile wa[T], wb[T];
  stage(0, 0);
#pragma unroll
  for (int t = 0; t < T; ++t) wa[t] = F::load(a_ptr(t, 0), lane, g4, r);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
#pragma unroll
  for (int t = 0; t < T; ++t) wa[t].pin();
  for (uint32_t sb = 0; sb < nsb; sb += 2) {
    if (sb + 1 < nsb) {
      stage(sb + 1, 1);
#pragma unroll
      for (int t = 0; t < T; ++t) wb[t] = F::load(a_ptr(t, sb + 1), lane, g4, r);
    }
    compute(wa, 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (sb + 1 >= nsb) break;
    if (sb + 2 < nsb) {
      stage(sb + 2, 0);
#pragma unroll
      for (int t = 0; t < T; ++t) wa[t] = F::load(a_ptr(t, sb + 2), lane, g4, r);
    }
    compute(wb, 1);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
#pragma unroll
  for (int t = 0; t < T; ++t) {
    float o[4];
    col_sum4(y[t], nf, o);
    const uint32_t tile = tile0 + t;
    if (tile < tiles_e && (uint32_t)r < n) {
      const uint32_t r0 = tile * 16 + 4 * g4;
      float* dst = ea.out + (size_t)(p0 + r) * ea.ldo + r0;
      for (int j = 0; j < 4; ++j)
        if (r0 + j < ea.rows) dst[j] = o[j];
    }
  }
}

// ------------------------------------------------------------------ Q8_0

// Q8_0 GEMV: a workgroup of W waves owns R row tiles; wave w takes the 32-blocks
// b = w, w + W, ...; the W partial sums meet in LDS.
template <int R, int W, int EPI>
__global__ __launch_bounds__(64 * W) void k_gemv_q8(const uint8_t* __restrict__ Wp, uint32_t tiles, uint32_t nb,
                                                     const uint16_t* __restrict__ Bx, const float* __restrict__ CS,
                                                     uint32_t N, EpiArgs ea) {
  __shared__ f4 red[W][R][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const uint32_t tile0 = blockIdx.x * R;
  const float nf = col_rinv(ea, r & 7);
  f4 y[R];
#pragma unroll
  for (int t = 0; t < R; ++t) y[t] = f4{0.f, 0.f, 0.f, 0.f};
  for (uint32_t b = wave; b < nb; b += W) {
    const h8 bq = as_h8(ld16(Bx + ((size_t)b * 64 + lane) * 8));
    const float c = CS[(b / 8) * 8 + (lane & 7)];
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
      for (int j = 0; j < 4; ++j) y[t][j] = y[t][j] + c * (d[j] * acc[j]);
    }
  }
  if (W > 1) {
#pragma unroll
    for (int t = 0; t < R; ++t) red[wave][t][lane] = y[t];
    __syncthreads();
  }
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
    col_sum4(vg, nf, og);
    col_sum4(vu, nf, ou);
    if (tile0 + tg >= tiles || r >= 8 || (uint32_t)r >= N) return;
    swiglu4(ea, (tile0 + tg) / 2, g, r, og, ou);
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
  col_sum4(v, nf, o);
  if (tile >= tiles || r >= 8 || (uint32_t)r >= N) return;
  epilogue4<EPI>(ea, tile * 16 + 4 * g, (uint32_t)r, o);
}

// ------------------------------------------------------------------ host side

void sh_qmat_free(QMat* m) {
  if (m->d) (void)hipFree(m->d);
  m->d = nullptr;
}

static size_t qrow_bytes(int type, uint32_t K) {
  switch (type) {
    case GGML_Q4_K: return (size_t)K / 256 * 144;
    case GGML_Q5_K: return (size_t)K / 256 * 176;
    case GGML_Q6_K: return (size_t)K / 256 * 210;
    default: return (size_t)K / 32 * 34;  // Q8_0
  }
}
static uint32_t q_block_elems(int type) { return type == GGML_Q8_0 ? 32u : 256u; }
static uint32_t q_tile_bytes(int type) {
  switch (type) {
    case GGML_Q4_K: return SH_Q4K_TILE_BYTES;
    case GGML_Q5_K: return SH_Q5K_TILE_BYTES;
    case GGML_Q6_K: return SH_Q6K_TILE_BYTES;
    default: return SH_Q8_TILE_BYTES;
  }
}
static bool q_repackable(int type) { return sh_is_kquant(type) || type == GGML_Q8_0; }

// Repack rows [0, M) of one GGUF matrix (on the device at src) into tiles
// dst_tile0 + t * tile_stride of dst.
static void launch_repack(sh_engine* e, int type, const uint8_t* src, uint8_t* dst, uint32_t M, uint32_t nblk,
                          uint32_t tile0, uint32_t stride) {
  const dim3 grid((M + 15) / 16, nblk);
  switch (type) {
    case GGML_Q4_K: hipLaunchKernelGGL(k_repack_q4k, grid, dim3(64), 0, e->stream, src, dst, M, nblk, tile0, stride); break;
    case GGML_Q5_K: hipLaunchKernelGGL(k_repack_q5k, grid, dim3(64), 0, e->stream, src, dst, M, nblk, tile0, stride); break;
    case GGML_Q6_K: hipLaunchKernelGGL(k_repack_q6k, grid, dim3(64), 0, e->stream, src, dst, M, nblk, tile0, stride); break;
    default: hipLaunchKernelGGL(k_repack_q8, grid, dim3(64), 0, e->stream, src, dst, M, nblk, tile0, stride); break;
  }
}

int sh_repack_upload_cat(sh_engine* e, int type, const uint8_t* const* parts, const uint32_t* rows, int nparts,
                         uint32_t K, QMat* out) {
  SH_CHECK(q_repackable(type), SH_ERR_UNSUPPORTED, "weight type %d not supported (Q4_K=12, Q5_K=13, Q6_K=14, Q8_0=8)",
           type);
  SH_CHECK(K % q_block_elems(type) == 0, SH_ERR_FORMAT, "K=%u not a multiple of the block", K);
  uint32_t M = 0;
  for (int i = 0; i < nparts; ++i) {
    SH_CHECK(nparts == 1 || rows[i] % 16 == 0, SH_ERR_UNSUPPORTED, "concatenated part rows %u %% 16", rows[i]);
    M += rows[i];
  }
  const uint32_t nblk = K / q_block_elems(type);
  QMat m;
  m.type = type; m.M = M; m.K = K; m.tiles = (M + 15) / 16;
  m.bytes = (size_t)m.tiles * nblk * q_tile_bytes(type);
  m.alg_bytes = (double)M * qrow_bytes(type, K);
  SH_HIP(hipMalloc(&m.d, m.bytes));
  uint32_t tile0 = 0;
  for (int i = 0; i < nparts; ++i) {
    const size_t bytes = (size_t)rows[i] * qrow_bytes(type, K);
    uint8_t* tmp = nullptr;
    SH_HIP(hipMalloc(&tmp, bytes));
    SH_HIP(hipMemcpyAsync(tmp, parts[i], bytes, hipMemcpyHostToDevice, e->stream));
    launch_repack(e, type, tmp, m.d, rows[i], nblk, tile0, 1u);
    SH_HIP(hipGetLastError());
    SH_HIP(hipStreamSynchronize(e->stream));
    SH_HIP(hipFree(tmp));
    tile0 += (rows[i] + 15) / 16;
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
  SH_CHECK(q_repackable(type), SH_ERR_UNSUPPORTED, "weight type %d not supported", type);
  SH_CHECK(M % 32 == 0, SH_ERR_UNSUPPORTED, "n_ff=%u must be a multiple of 32", M);
  SH_CHECK(K % q_block_elems(type) == 0, SH_ERR_FORMAT, "K=%u not a multiple of the block", K);
  const uint32_t nblk = K / q_block_elems(type);
  QMat m;
  m.type = type; m.M = 2 * M; m.K = K; m.tiles = 2 * (M / 16);
  m.bytes = (size_t)m.tiles * nblk * q_tile_bytes(type);
  m.alg_bytes = 2.0 * M * qrow_bytes(type, K);
  SH_HIP(hipMalloc(&m.d, m.bytes));
  const size_t bytes = (size_t)M * qrow_bytes(type, K);
  uint8_t* tmp = nullptr;
  SH_HIP(hipMalloc(&tmp, bytes));
  for (int part = 0; part < 2; ++part) {
    SH_HIP(hipMemcpyAsync(tmp, part ? up : gate, bytes, hipMemcpyHostToDevice, e->stream));
    launch_repack(e, type, tmp, m.d, M, nblk, (uint32_t)part, 2u);
    SH_HIP(hipGetLastError());
    SH_HIP(hipStreamSynchronize(e->stream));
  }
  SH_HIP(hipFree(tmp));
  *out = m;
  return SH_OK;
}

// ------------------------------------------------------------------ dispatch

// Tuning overrides (read once): SH_GEMV_KERNEL=stream|wide, SH_GEMV_T (tiles
// per wave, wide: 1|2|4, stream: 1|2|4|8), SH_GEMV_KS (wide: splits).
static int env_u32(const char* name) {
  const char* s = getenv(name);
  return s ? atoi(s) : 0;
}
static int gemv_kernel_choice() {
  static const int v = [] {
    const char* s = getenv("SH_GEMV_KERNEL");
    if (!s) return 0;
    return std::string(s) == "stream" ? 1 : (std::string(s) == "wide" ? 2 : 0);
  }();
  return v;
}
static uint32_t gemv_t_override() {
  static const uint32_t v = (uint32_t)env_u32("SH_GEMV_T");
  return v;
}
static uint32_t gemv_ks_override() {
  static const uint32_t v = (uint32_t)env_u32("SH_GEMV_KS");
  return v;
}

struct WidePlan {
  uint32_t T = 1, S = 1, KS = 1;
};

// Wide-kernel shape for a Q4_K matrix whose consumer finishes split partials:
// T tiles per wave (1 unless overridden) and S superblocks per split, S the
// largest divisor of K/256 up to 7 that still gives >= 256 workgroups (one per
// CU); at most 16 splits.
static bool wide_plan(const QMat& w, WidePlan* p) {
  if (w.type != GGML_Q4_K || gemv_kernel_choice() == 1) return false;
  const uint32_t nsb = w.K / 256;
  uint32_t T = gemv_t_override();
  if (T != 1 && T != 2 && T != 4) T = 1;
  const uint32_t groups = (w.tiles + WV * T - 1) / (WV * T);
  const uint32_t ks_req = gemv_ks_override();
  uint32_t S = 0;
  for (uint32_t s = WIDE_MAX_SB; s >= 1; --s) {
    if (nsb % s || T * s > WIDE_MAX_UNITS) continue;
    const uint32_t ks = nsb / s;
    if (ks > 16) break;
    S = s;
    if (ks_req ? ks >= ks_req : groups * ks >= 256) break;
  }
  if (!S) return false;
  p->T = T;
  p->S = S;
  p->KS = nsb / S;
  return true;
}

size_t sh_gemv_part_floats(const QMat& w) {
  WidePlan p;
  const uint32_t ks = wide_plan(w, &p) ? p.KS : 1;
  return (size_t)ks * 8 * w.tiles * 16;
}

static uint32_t gemv_d_override() {
  static const uint32_t v = (uint32_t)env_u32("SH_GEMV_D");
  return v;
}
// D = weight units in flight per wave (SH_GEMV_D=2|4|8; default 2: the 8B
// down is 6 % faster than at 4 and 15 % faster than at 8, Wo alike).
template <int T, int S, int EPI, int SRC, bool FP>
static void launch_q4w_fp(sh_engine* e, const QMat& w, const uint16_t* bx, const uint16_t* xs, uint32_t N,
                          const EpiArgs& ea, const WidePlan& p, const OpndSrc& src, const PrepFuse& pf) {
  const dim3 grid((w.tiles + WV * T - 1) / (WV * T), p.KS);
  const uint32_t d = gemv_d_override();
  if (d == 4)
    hipLaunchKernelGGL((k_gemv_q4w<T, S, 4, EPI, SRC, FP>), grid, dim3(64 * WV), 0, e->stream, w.d, w.tiles,
                       w.K / 256, bx, xs, ea.cs, N, ea, src, pf);
  else if (d == 8)
    hipLaunchKernelGGL((k_gemv_q4w<T, S, 8, EPI, SRC, FP>), grid, dim3(64 * WV), 0, e->stream, w.d, w.tiles,
                       w.K / 256, bx, xs, ea.cs, N, ea, src, pf);
  else
    hipLaunchKernelGGL((k_gemv_q4w<T, S, 2, EPI, SRC, FP>), grid, dim3(64 * WV), 0, e->stream, w.d, w.tiles,
                       w.K / 256, bx, xs, ea.cs, N, ea, src, pf);
}
template <int T, int S, int EPI, int SRC>
static void launch_q4w_src(sh_engine* e, const QMat& w, const uint16_t* bx, const uint16_t* xs, uint32_t N,
                           const EpiArgs& ea, const WidePlan& p, const OpndSrc& src, const PrepFuse* pf) {
  if constexpr (EPI == EPI_PART && (SRC == OPND_STAGED || SRC == OPND_ROWS) && (T == 1 || T == 2)) {
    if (pf) {
      launch_q4w_fp<T, S, EPI, SRC, true>(e, w, bx, xs, N, ea, p, src, *pf);
      return;
    }
  }
  launch_q4w_fp<T, S, EPI, SRC, false>(e, w, bx, xs, N, ea, p, src, PrepFuse{});
}
template <int T, int S, int EPI>
static void launch_q4w_s(sh_engine* e, const QMat& w, const uint16_t* bx, const uint16_t* xs, uint32_t N,
                         const EpiArgs& ea, const WidePlan& p, const OpndSrc& src, const PrepFuse* pf) {
  if (src.kind == OPND_ROWS) launch_q4w_src<T, S, EPI, OPND_ROWS>(e, w, bx, xs, N, ea, p, src, pf);
  else if (src.kind == OPND_FA) launch_q4w_src<T, S, EPI, OPND_FA>(e, w, bx, xs, N, ea, p, src, nullptr);
  else launch_q4w_src<T, S, EPI, OPND_STAGED>(e, w, bx, xs, N, ea, p, src, pf);
}
template <int T, int S, int EPI>
static void launch_q4w_if(sh_engine* e, const QMat& w, const uint16_t* bx, const uint16_t* xs, uint32_t N,
                          const EpiArgs& ea, const WidePlan& p, const OpndSrc& src, const PrepFuse* pf) {
  if constexpr (T * S <= (int)WIDE_MAX_UNITS) launch_q4w_s<T, S, EPI>(e, w, bx, xs, N, ea, p, src, pf);
}
template <int T, int EPI>
static void launch_q4w(sh_engine* e, const QMat& w, const uint16_t* bx, const uint16_t* xs, uint32_t N,
                       const EpiArgs& ea, const WidePlan& p, const OpndSrc& src, const PrepFuse* pf = nullptr) {
  switch (p.S) {
    case 1: launch_q4w_if<T, 1, EPI>(e, w, bx, xs, N, ea, p, src, pf); break;
    case 2: launch_q4w_if<T, 2, EPI>(e, w, bx, xs, N, ea, p, src, pf); break;
    case 3: launch_q4w_if<T, 3, EPI>(e, w, bx, xs, N, ea, p, src, pf); break;
    case 4: launch_q4w_if<T, 4, EPI>(e, w, bx, xs, N, ea, p, src, pf); break;
    case 5: launch_q4w_if<T, 5, EPI>(e, w, bx, xs, N, ea, p, src, pf); break;
    case 6: launch_q4w_if<T, 6, EPI>(e, w, bx, xs, N, ea, p, src, pf); break;
    default: launch_q4w_if<T, 7, EPI>(e, w, bx, xs, N, ea, p, src, pf); break;
  }
}

bool sh_gemv_prep_fusable(const QMat& w) {
  WidePlan p;
  return wide_plan(w, &p) && (p.T == 1 || p.T == 2) && w.tiles % 16 == 0 && w.tiles / 16 <= SH_SB_CNT;
}

// Dynamic LDS of the OPND_RESID build: the operand, its scales and sums of squares.
static size_t resid_lds_bytes(uint32_t nsb) { return (size_t)nsb * 9 * 64 * 16 + (size_t)nsb * 8 * 4 * 2; }

template <int T, int EPI>
static void launch_q4s(sh_engine* e, const QMat& w, const uint16_t* bx, const uint16_t* xs, uint32_t N,
                       const EpiArgs& ea, const OpndSrc& src) {
  const uint32_t grid = (w.tiles + T - 1) / T, nsb = w.K / 256;
  if (src.kind == OPND_RESID)
    hipLaunchKernelGGL((k_gemv_q4s<T, EPI, OPND_RESID>), dim3(grid), dim3(64 * GW), resid_lds_bytes(nsb), e->stream,
                       w.d, w.tiles, nsb, bx, xs, ea.cs, N, ea, src);
  else
    hipLaunchKernelGGL((k_gemv_q4s<T, EPI, OPND_STAGED>), dim3(grid), dim3(64 * GW), 0, e->stream, w.d, w.tiles, nsb,
                       bx, xs, ea.cs, N, ea, src);
}

// Streaming policy: about 512 workgroups of 8 waves (two per CU), i.e. T =
// tiles / 512 rounded down to a power of two in [1, 8] (even for SwiGLU so a
// workgroup owns whole gate/up pairs); QKV about 128. An OPND_RESID launch
// rebuilds the operand in every workgroup (residual + all pending partials),
// so it aims at about 256 workgroups (draft gate/up, 1024 tiles: T = 4, 25 %
// faster than T = 2, measured).
template <int EPI>
static void dispatch_q4s(sh_engine* e, const QMat& w, const uint16_t* bx, const uint16_t* xs, uint32_t N,
                         const EpiArgs& ea, const OpndSrc& src) {
  uint32_t t = gemv_kernel_choice() == 1 ? gemv_t_override() : 0;
  if (!t) {
    // QKV: every workgroup reads the whole operand (144 KB at K = 4096) for T
    // tiles, so fewer, wider workgroups win: the 8B QKV (384 tiles) is 8 %
    // faster at T = 2 than at 1 (T = 4 is slower).
    const uint32_t target = src.kind == OPND_RESID ? 256 : (EPI == EPI_QKV ? 128 : 512);
    t = 1;
    while (t < 8 && w.tiles / (2 * t) >= target) t *= 2;
  }
  if (EPI == EPI_SWIGLU && t < 2) t = 2;
  switch (t) {
    case 1: launch_q4s<1, EPI>(e, w, bx, xs, N, ea, src); break;
    case 2: launch_q4s<2, EPI>(e, w, bx, xs, N, ea, src); break;
    case 4: launch_q4s<4, EPI>(e, w, bx, xs, N, ea, src); break;
    default: launch_q4s<8, EPI>(e, w, bx, xs, N, ea, src); break;
  }
}

template <int R, int W, int EPI>
static void launch_q8(sh_engine* e, const QMat& w, const uint16_t* bx, uint32_t N, const EpiArgs& ea) {
  const uint32_t grid = (w.tiles + R - 1) / R;
  hipLaunchKernelGGL((k_gemv_q8<R, W, EPI>), dim3(grid), dim3(64 * W), 0, e->stream, w.d, w.tiles, w.K / 32, bx,
                     ea.cs, N, ea);
}
template <int EPI>
static void dispatch_q8(sh_engine* e, const QMat& w, const uint16_t* bx, uint32_t N, const EpiArgs& ea) {
  if (EPI == EPI_SWIGLU) launch_q8<2, 4, EPI>(e, w, bx, N, ea);
  else if (w.tiles >= 1024) launch_q8<2, 4, EPI>(e, w, bx, N, ea);
  else launch_q8<1, 4, EPI>(e, w, bx, N, ea);
}

// Deep-ring policy (K of 8 or 16 superblocks): T = 7 when the tiles split
// evenly into at least 256 workgroups of 7 (one round, one workgroup per CU).
// At K = 4096, matrices that need several rounds (the 8B lm_head) run faster
// on k_gemv_q4s (68 us against 72-77 us for 128256 x 4096), as do small ones.
uint32_t sh_gemv_ring_t(const QMat& w) {
  static const bool off = [] {
    const char* s = getenv("SH_RING");
    return s && std::string(s) == "0";
  }();
  if (off || w.type != GGML_Q4_K || (w.K != 2048 && w.K != 4096)) return 0;  // K = 8 NB superblocks
  if (w.tiles % 7 == 0 && w.tiles / 7 >= 256) return 7;
  // K = 2048 (one superblock per wave) with several rounds of 8 tiles: the
  // draft's tied lm_head, 45 -> 40 us per launch
  if (w.K == 2048 && w.tiles / 8 >= 768) return 8;
  return 0;
}

// Weight units in flight per wave: 2 and 3 time alike on 28672 x 4096
// (16.3 / 16.4 us), 4 and more slower (16.8 us at 4, 19 us at 6).
constexpr int RING_D = 3;
template <int EPI, bool FS = false>
static void launch_q4t(sh_engine* e, const QMat& w, const uint16_t* bx, const uint16_t* xs, uint32_t N,
                       const EpiArgs& ea, uint32_t T, const PrepFuse& pf = PrepFuse{}) {
  if (T == 8 && w.K == 4096) {  // 16 waves of one superblock each
    hipLaunchKernelGGL((k_gemv_q4t<8, 1, RING_D, EPI, FS, 16>), dim3(w.tiles / 8), dim3(64 * 16), 0, e->stream, w.d,
                       w.tiles, 16u, bx, xs, ea.cs, N, ea, pf);
    return;
  }
  if (T == 8) {  // K = 2048
    hipLaunchKernelGGL((k_gemv_q4t<8, 1, RING_D, EPI, FS>), dim3((w.tiles + 7) / 8), dim3(64 * GW), 0, e->stream, w.d,
                       w.tiles, 8u, bx, xs, ea.cs, N, ea, pf);
    return;
  }
  const dim3 grid(w.tiles / 7);
  // K = 4096: 16 waves of one superblock each (4 waves per SIMD; the 8B
  // gate/up 21.5 -> 20.4 us per launch, window 2 and 3 alike) unless
  // SH_RING16=0 (8 waves of two superblocks, 254 VGPRs: 2 waves per SIMD)
  static const bool ring16 = [] {
    const char* s = getenv("SH_RING16");
    return !(s && std::string(s) == "0");
  }();
  if (w.K == 4096 && ring16)
    hipLaunchKernelGGL((k_gemv_q4t<7, 1, 2, EPI, FS, 16>), grid, dim3(64 * 16), 0, e->stream, w.d, w.tiles, 16u, bx,
                       xs, ea.cs, N, ea, pf);
  else if (w.K == 4096)
    hipLaunchKernelGGL((k_gemv_q4t<7, 2, RING_D, EPI, FS>), grid, dim3(64 * GW), 0, e->stream, w.d, w.tiles, 16u, bx,
                       xs, ea.cs, N, ea, pf);
  else
    hipLaunchKernelGGL((k_gemv_q4t<7, 1, RING_D, EPI, FS>), grid, dim3(64 * GW), 0, e->stream, w.d, w.tiles, 8u, bx,
                       xs, ea.cs, N, ea, pf);
}

int sh_gemv_ring_launch(sh_engine* e, const QMat& w, const uint16_t* bx, const uint16_t* xs, uint32_t N,
                        EpiKind epi, const EpiArgs& ea, const char* tag, const PrepFuse* swiglu) {
  SH_CHECK(N >= 1 && N <= 8, SH_ERR_ARG, "gemv chunk N=%u outside [1,8]", N);
  SH_CHECK(ea.cs, SH_ERR_ARG, "gemv: activation scales missing");
  const uint32_t T = sh_gemv_ring_t(w);
  SH_CHECK(T && (epi == EPI_STORE || epi == EPI_PART), SH_ERR_ARG, "gemv: this launch does not take the ring kernel");
  // the 16-wave kernel stages the sums of squares with one thread each
  SH_CHECK(!ea.ssq || ea.ssq_n * 8 <= 64 * 16, SH_ERR_ARG, "gemv: %u superblock sums of squares", ea.ssq_n);
  SH_CHECK(epi != EPI_PART || ea.part_cap >= 1, SH_ERR_CAPACITY, "gemv: no room for the partial sums");
  SH_CHECK(!swiglu || (epi == EPI_PART && swiglu->K * 2 == w.tiles * 16 && swiglu->K % 256 == 0 &&
                       swiglu->K / 256 <= SH_SB_CNT && swiglu->cnt && swiglu->bx && swiglu->xs && swiglu->cs),
           SH_ERR_ARG, "gemv: the fused SwiGLU prep does not fit this launch");
  hipEvent_t ev = nullptr;
  sh_prof_begin(e, &ev);
  if (epi == EPI_STORE) launch_q4t<EPI_STORE>(e, w, bx, xs, N, ea, T);
  else if (swiglu) launch_q4t<EPI_PART, true>(e, w, bx, xs, N, ea, T, *swiglu);
  else launch_q4t<EPI_PART>(e, w, bx, xs, N, ea, T);
  SH_HIP(hipGetLastError());
  sh_prof_end(e, tag, w.alg_bytes, ev);
  return SH_OK;
}

// QKV through k_gemv_q4t at 2 tiles per workgroup (SH_QKV_RING=0: through
// k_gemv_q4s). Measured on the 8B verify (384 tiles, K = 4096): 1, 3 and 4
// tiles per workgroup and windows of 2 or 4 units are all slower.
static bool qkv_ring_enabled() {
  static const bool v = [] {
    const char* s = getenv("SH_QKV_RING");
    return !(s && std::string(s) == "0");
  }();
  return v;
}

template <int T>
static void launch_q4t_qkv(sh_engine* e, const QMat& w, const uint16_t* bx, const uint16_t* xs, uint32_t N,
                           const EpiArgs& ea) {
  const dim3 grid(w.tiles / T);
  // K = 4096: 16 waves of one superblock each (103 VGPRs, 4 waves per SIMD;
  // the 8B verify's QKV 0.55 us faster per layer) unless SH_QKV16=0 (8 waves
  // of two superblocks, 165 VGPRs: 3 waves per SIMD, one workgroup per CU)
  static const bool q16 = [] {
    const char* s = getenv("SH_QKV16");
    return !(s && std::string(s) == "0");
  }();
  if (w.K == 4096 && q16)
    hipLaunchKernelGGL((k_gemv_q4t<T, 1, 2, EPI_QKV, false, 16>), grid, dim3(64 * 16), 0, e->stream, w.d, w.tiles,
                       16u, bx, xs, ea.cs, N, ea, PrepFuse{});
  else if (w.K == 4096)
    hipLaunchKernelGGL((k_gemv_q4t<T, 2, RING_D, EPI_QKV>), grid, dim3(64 * GW), 0, e->stream, w.d, w.tiles, 16u,
                       bx, xs, ea.cs, N, ea, PrepFuse{});
  else
    hipLaunchKernelGGL((k_gemv_q4t<T, 1, RING_D, EPI_QKV>), grid, dim3(64 * GW), 0, e->stream, w.d, w.tiles, 8u, bx,
                       xs, ea.cs, N, ea, PrepFuse{});
}

bool sh_gemv_resid_fusable(const QMat& w, uint32_t N) {
  // the whole-K kernel with its largest reduction buffer (4 tiles x 32 KB / 4) must fit beside the operand
  return w.type == GGML_Q4_K && w.K % 256 == 0 && N <= 2 && resid_lds_bytes(w.K / 256) + 32768 <= 160 * 1024;
}

uint32_t sh_gemv_fusable(const QMat& w) {
  WidePlan p;
  return wide_plan(w, &p) ? p.S : 0;
}

int sh_gemv_launch(sh_engine* e, const QMat& w, const uint16_t* bx, const uint16_t* xs, uint32_t N, EpiKind epi,
                   const EpiArgs& ea, const char* tag, uint32_t* nparts, const OpndSrc* src, const PrepFuse* pf) {
  SH_CHECK(N >= 1 && N <= 8, SH_ERR_ARG, "gemv chunk N=%u outside [1,8]", N);
  SH_CHECK(ea.cs, SH_ERR_ARG, "gemv: activation scales missing");
  const OpndSrc staged;
  const OpndSrc& sr = src ? *src : staged;
  uint32_t np = 1;
  hipEvent_t ev = nullptr;
  sh_prof_begin(e, &ev);
  WidePlan p;
  SH_CHECK(sr.kind == OPND_STAGED ||
               (sr.kind == OPND_RESID ? (epi == EPI_QKV || epi == EPI_SWIGLU) && sh_gemv_resid_fusable(w, N)
                                      : epi == EPI_PART && w.type == GGML_Q4_K && wide_plan(w, &p)),
           SH_ERR_ARG, "gemv: this operand source does not fit this launch");
  SH_CHECK(!pf || (epi == EPI_PART && (sr.kind == OPND_STAGED || sr.kind == OPND_ROWS) && sh_gemv_prep_fusable(w) &&
                   pf->K == w.tiles * 16 &&
                   pf->cnt && pf->resid && pf->norm_w && pf->ssq),
           SH_ERR_ARG, "gemv: the fused residual prep does not fit this launch");
  if (w.type == GGML_Q4_K) {
    if (epi == EPI_PART && wide_plan(w, &p)) {
      SH_CHECK(ea.part_cap >= p.KS, SH_ERR_CAPACITY, "gemv: %u split partials exceed the buffer (%u)", p.KS,
               ea.part_cap);
      np = p.KS;
      if (p.T == 1) launch_q4w<1, EPI_PART>(e, w, bx, xs, N, ea, p, sr, pf);
      else if (p.T == 2) launch_q4w<2, EPI_PART>(e, w, bx, xs, N, ea, p, sr, pf);
      else launch_q4w<4, EPI_PART>(e, w, bx, xs, N, ea, p, sr);
    } else {
      uint32_t rt = sr.kind == OPND_STAGED && epi == EPI_STORE ? sh_gemv_ring_t(w) : 0u;
      // K = 4096 stores of several rounds of 8 tiles (the 8B lm_head): the
      // 16-wave ring, 70 -> 63 us per launch against k_gemv_q4s<8> (228 VGPRs,
      // one workgroup of two waves per SIMD); SH_LM16=0: the stream kernel
      static const bool lm16 = [] {
        const char* s = getenv("SH_LM16");
        return !(s && std::string(s) == "0");
      }();
      if (lm16 && !rt && sr.kind == OPND_STAGED && epi == EPI_STORE && w.type == GGML_Q4_K && w.K == 4096 &&
          w.tiles % 8 == 0 && w.tiles / 8 >= 768)
        rt = 8;
      switch (rt ? -1 : (int)epi) {
        case -1: launch_q4t<EPI_STORE>(e, w, bx, xs, N, ea, rt); break;
        case EPI_STORE: dispatch_q4s<EPI_STORE>(e, w, bx, xs, N, ea, sr); break;
        case EPI_ADD: dispatch_q4s<EPI_ADD>(e, w, bx, xs, N, ea, sr); break;
        case EPI_QKV:
          if (qkv_ring_enabled() && sr.kind == OPND_STAGED && (w.K == 2048 || w.K == 4096) && w.tiles % 2 == 0)
            launch_q4t_qkv<2>(e, w, bx, xs, N, ea);
          else
            dispatch_q4s<EPI_QKV>(e, w, bx, xs, N, ea, sr);
          break;
        case EPI_SWIGLU: dispatch_q4s<EPI_SWIGLU>(e, w, bx, xs, N, ea, sr); break;
        case EPI_PART: dispatch_q4s<EPI_PART>(e, w, bx, xs, N, ea, sr); break;
      }
    }
  } else if (w.type == GGML_Q8_0) {
    switch (epi) {
      case EPI_STORE: dispatch_q8<EPI_STORE>(e, w, bx, N, ea); break;
      case EPI_ADD: dispatch_q8<EPI_ADD>(e, w, bx, N, ea); break;
      case EPI_QKV: dispatch_q8<EPI_QKV>(e, w, bx, N, ea); break;
      case EPI_SWIGLU: dispatch_q8<EPI_SWIGLU>(e, w, bx, N, ea); break;
      case EPI_PART: dispatch_q8<EPI_PART>(e, w, bx, N, ea); break;
    }
  } else {
    SH_CHECK(false, SH_ERR_UNSUPPORTED, "gemv: weight type %d", w.type);
  }
  SH_HIP(hipGetLastError());
  sh_prof_end(e, tag, w.alg_bytes, ev);
  if (nparts) *nparts = np;
  return SH_OK;
}

// ------------------------------------------------------------------ multi-group dispatch

// Multi-group shape: T = 2 tiles per wave for 2 to 4 groups (registers), else 1.
// The splits depend on the matrix only, never on the column count, so a
// column's arithmetic (superblock order within a split, split order in the
// sum) is the same in every multi-group launch: the fewest splits (at most 16)
// whose workgroup count at T = 1 (8 row tiles per workgroup, the launches of
// more than 32 columns) fills the 256 CUs to at least 70 % in its last round
// (one workgroup per CU: up to 148 KB of LDS). Every split costs a round trip
// of [columns][rows] f32 partials through HBM; at 64 columns that outweighs
// the CU fill the T = 2 launches (at most 32 columns) lose to it.
struct MgPlan {
  uint32_t T = 1, S = 1, KS = 1;
};
static MgPlan mg_plan(const QMat& w, uint32_t G, bool one_split) {
  MgPlan p;
  p.T = G >= 2 && G <= 4 ? 2 : 1;
  const uint32_t nsb = w.K / 256, wgx = (w.tiles + 7) / 8, slots = 256;
  uint32_t best_ks = 1;
  double best = -1.0;
  for (uint32_t ks = 1; !one_split && ks <= 16 && ks <= nsb; ++ks) {
    const uint32_t S = (nsb + ks - 1) / ks, k2 = (nsb + S - 1) / S, wgs = wgx * k2;
    const double eff = (double)wgs / (double)(slots * ((wgs + slots - 1) / slots));
    if (eff > best + 1e-9) { best = eff; best_ks = k2; }
    if (eff >= 0.7) break;
  }
  p.S = (nsb + best_ks - 1) / best_ks;
  p.KS = (nsb + p.S - 1) / p.S;
  return p;
}

size_t sh_gemm_part_floats(const QMat& w) {
  if (!sh_is_kquant(w.type)) return 0;
  return (size_t)mg_plan(w, MG_MAX_G, false).KS * SH_MAX_COLS * w.tiles * 16;
}

template <class F, int T, int G, int EPI>
static void launch_mg(sh_engine* e, const QMat& w, const uint16_t* bx, const uint16_t* xs, const float* cs,
                      uint32_t N, const EpiArgs& ea, const MgPlan& p) {
  const dim3 grid((w.tiles + 8 * T - 1) / (8 * T), p.KS);
  hipLaunchKernelGGL((k_gemm_kq<F, T, G, EPI>), grid, dim3(512), 0, e->stream, w.d, w.tiles, w.K / 256, p.S, bx, xs,
                     cs, N, ea);
}
template <class F, int EPI>
static void dispatch_mg(sh_engine* e, const QMat& w, const uint16_t* bx, const uint16_t* xs, const float* cs,
                        uint32_t N, const EpiArgs& ea, const MgPlan& p) {
  // One group: one tile per wave, so the launch has the workgroups the split
  // plan counts on (the Q4_K_M-style 8B's Q6_K down: 22.5 -> 17 us per launch)
  switch ((N + 7) / 8) {
    case 1: launch_mg<F, 1, 1, EPI>(e, w, bx, xs, cs, N, ea, p); break;
    case 2: launch_mg<F, 2, 2, EPI>(e, w, bx, xs, cs, N, ea, p); break;
    case 3: launch_mg<F, 2, 3, EPI>(e, w, bx, xs, cs, N, ea, p); break;
    case 4: launch_mg<F, 2, 4, EPI>(e, w, bx, xs, cs, N, ea, p); break;
    case 5: launch_mg<F, 1, 5, EPI>(e, w, bx, xs, cs, N, ea, p); break;
    case 6: launch_mg<F, 1, 6, EPI>(e, w, bx, xs, cs, N, ea, p); break;
    case 7: launch_mg<F, 1, 7, EPI>(e, w, bx, xs, cs, N, ea, p); break;
    default: launch_mg<F, 1, 8, EPI>(e, w, bx, xs, cs, N, ea, p); break;
  }
}
template <int EPI>
static void dispatch_mg_fmt(sh_engine* e, const QMat& w, const uint16_t* bx, const uint16_t* xs, const float* cs,
                            uint32_t N, const EpiArgs& ea, const MgPlan& p) {
  if (w.type == GGML_Q5_K) dispatch_mg<FmtQ5K, EPI>(e, w, bx, xs, cs, N, ea, p);
  else if (w.type == GGML_Q6_K) dispatch_mg<FmtQ6K, EPI>(e, w, bx, xs, cs, N, ea, p);
  else dispatch_mg<FmtQ4K, EPI>(e, w, bx, xs, cs, N, ea, p);
}

int sh_gemm_launch(sh_engine* e, const QMat& w, const uint16_t* bx, const uint16_t* xs, const float* cs, uint32_t N,
                   EpiKind epi, const EpiArgs& ea, const char* tag, uint32_t* nparts) {
  SH_CHECK(N >= 1 && N <= SH_MAX_COLS, SH_ERR_ARG, "gemm N=%u outside [1, %u]", N, SH_MAX_COLS);
  SH_CHECK(sh_is_kquant(w.type) && w.K % 256 == 0, SH_ERR_UNSUPPORTED,
           "multi-group gemm needs a K-quant (Q4_K / Q5_K / Q6_K; type %d)", w.type);
  SH_CHECK(epi == EPI_PART || epi == EPI_STORE, SH_ERR_ARG, "multi-group gemm epilogue %d", (int)epi);
  const MgPlan p = mg_plan(w, (N + 7) / 8, epi == EPI_STORE);
  if (epi == EPI_PART)
    SH_CHECK(ea.part_cap >= p.KS && ea.part_stride >= (size_t)((N + 7) / 8 * 8) * ea.ldo, SH_ERR_CAPACITY,
             "gemm: %u split partials exceed the buffer (%u)", p.KS, ea.part_cap);
  hipEvent_t ev = nullptr;
  sh_prof_begin(e, &ev);
  if (epi == EPI_PART) dispatch_mg_fmt<EPI_PART>(e, w, bx, xs, cs, N, ea, p);
  else dispatch_mg_fmt<EPI_STORE>(e, w, bx, xs, cs, N, ea, p);
  SH_HIP(hipGetLastError());
  sh_prof_end(e, tag, w.alg_bytes, ev);
  if (nparts) *nparts = p.KS;
  return SH_OK;
}

// K-splits of a wide f16 GEMM: 8-tile workgroups, one per CU (the 150 KB LDS
// ring), at most the splits the multi-group plan sizes the partial buffer for.
// The split count minimises rounds x (superblocks per workgroup + 2), the 2
// standing for the ring's fill before the first superblock computes.
static MgPlan plan16(const QMat& w, bool one_split) {
  MgPlan p;
  p.T = 1;
  const uint32_t nsb = w.K / 256, wgx = (w.tiles + 7) / 8, slots = 256;
  const uint32_t cap = one_split ? 1 : mg_plan(w, MG_MAX_G, false).KS;
  uint32_t best_ks = 1;
  uint64_t best = ~0ull;
  for (uint32_t ks = 1; ks <= cap && ks <= nsb; ++ks) {
    const uint32_t S = (nsb + ks - 1) / ks, k2 = (nsb + S - 1) / S, wgs = wgx * k2;
    const uint64_t cost = (uint64_t)((wgs + slots - 1) / slots) * (S + 2);
    if (cost < best) { best = cost; best_ks = k2; }
  }
  p.S = (nsb + best_ks - 1) / best_ks;
  p.KS = (nsb + p.S - 1) / p.S;
  return p;
}

// K-splits of the wide (more than 64 columns) f16 GEMM: 16-tile workgroups, one
// per CU, at most 16 splits. Estimated time (us): rounds x (superblocks per
// workgroup + 2, the ring's fill) x 0.58 NC (a 16-tile workgroup's superblock
// at NC groups of 16 columns, measured on the 8B gate/up) plus the split
// partials' write and read by the finishing kernel at ~4 TB/s.
static MgPlan plan16w(const QMat& w, bool one_split, uint32_t N) {
  MgPlan p;
  p.T = 2;
  const uint32_t nsb = w.K / 256, wgx = (w.tiles + 15) / 16, slots = 256, NC = (N + 15) / 16;
  const uint32_t cap = one_split ? 1 : 16;
  uint32_t best_ks = 1;
  double best = 1e300;
  for (uint32_t ks = 1; ks <= cap && ks <= nsb; ++ks) {
    const uint32_t S = (nsb + ks - 1) / ks, k2 = (nsb + S - 1) / S, wgs = wgx * k2;
    const double part_us = k2 > 1 ? (double)k2 * ((N + 7) / 8 * 8) * w.tiles * 16 * 8.0 / 4e6 : 0.0;
    const double cost = (double)((wgs + slots - 1) / slots) * (S + 2) * 0.58 * NC + part_us;
    if (cost < best - 1e-9) { best = cost; best_ks = k2; }
  }
  p.S = (nsb + best_ks - 1) / best_ks;
  p.KS = (nsb + p.S - 1) / p.S;
  return p;
}

// Column blocks of the column-block kernel (k_gemm16h_q4k) for N columns: at
// most 6 groups of 16 per block, the blocks as even as the groups allow.
struct G16hShape {
  uint32_t ncb = 1, nch = 1;
};
static G16hShape shape16h(uint32_t N) {
  G16hShape g;
  const uint32_t NC = (N + 15) / 16;
  g.ncb = (NC + 5) / 6;
  g.nch = (NC + g.ncb - 1) / g.ncb;
  return g;
}
// K-splits of the column-block kernel: 16-tile workgroups, one per CU (the
// 132 KB LDS ring), cost as plan16w with the block's groups.
static MgPlan plan16h(const QMat& w, bool one_split, uint32_t N) {
  MgPlan p;
  p.T = 2;
  const G16hShape g = shape16h(N);
  const uint32_t nsb = w.K / 256, wgx = (w.tiles + 15) / 16 * g.ncb, slots = 256;
  const uint32_t cap = one_split ? 1 : 16;
  uint32_t best_ks = 1;
  double best = 1e300;
  for (uint32_t ks = 1; ks <= cap && ks <= nsb; ++ks) {
    const uint32_t S = (nsb + ks - 1) / ks, k2 = (nsb + S - 1) / S, wgs = wgx * k2;
    const double part_us = k2 > 1 ? (double)k2 * ((N + 7) / 8 * 8) * w.tiles * 16 * 8.0 / 4e6 : 0.0;
    const double cost = (double)((wgs + slots - 1) / slots) * (S + 1) * 0.58 * g.nch + part_us;
    if (cost < best - 1e-9) { best = cost; best_ks = k2; }
  }
  p.S = (nsb + best_ks - 1) / best_ks;
  p.KS = (nsb + p.S - 1) / p.S;
  return p;
}
// Which kernel takes a call of more than 64 columns: k_gemm16w_q4k (one pass
// over the weights) unless its split plan leaves more than 40 % of the CUs
// idle (the 8B Wo at 164 columns: 128 workgroups), where the column blocks
// give the 16-tile workgroups twice the parallelism (measured 0.58 vs 0.72 ms
// per tree step; the gate/up, down and QKV shapes are faster one pass).
// SH_G16H=0 / 1 forces either kernel.
static bool use16h(const QMat& w, bool one_split, uint32_t N) {
  static const int forced = [] {
    const char* e = getenv("SH_G16H");
    return e && *e ? atoi(e) : -1;
  }();
  if (forced >= 0) return forced != 0;
  const MgPlan p = plan16w(w, one_split, N);
  return (uint64_t)(w.tiles + 15) / 16 * p.KS * 10 < 256 * 6;
}

size_t sh_gemm16_part_floats(const QMat& w) {
  if (w.type != GGML_Q4_K) return sh_gemm16x_part_floats(w);
  if (w.K % 256) return 0;
  size_t cols = (size_t)plan16(w, false).KS * SH_MAX_COLS;  // split-columns of the widest partial set
  for (uint32_t N = SH_MAX_COLS + 1; N <= SH_MAX_COLS16; ++N)
    cols = std::max({cols, (size_t)plan16w(w, false, N).KS * ((N + 7) / 8 * 8),
                     (size_t)plan16h(w, false, N).KS * ((N + 7) / 8 * 8)});
  return cols * w.tiles * 16;
}

template <int NCH, int EPI>
static void launch16h(sh_engine* e, const QMat& w, const uint16_t* bh, uint32_t ldb, uint32_t N, uint32_t ncb,
                      const EpiArgs& ea, const MgPlan& p) {
  const uint32_t nrb = (w.tiles + 15) / 16;
  const dim3 grid((nrb + 7) / 8 * 8 * ncb, p.KS);
  hipLaunchKernelGGL((k_gemm16h_q4k<NCH, EPI>), grid, dim3(512), 0, e->stream, w.d, w.tiles, w.K / 256, p.S, bh,
                     ldb, N, ncb, ea);
}
template <int EPI>
static void dispatch16h(sh_engine* e, const QMat& w, const uint16_t* bh, uint32_t ldb, uint32_t N,
                        const EpiArgs& ea, const MgPlan& p) {
  const G16hShape g = shape16h(N);
  switch (g.nch) {
    case 4: launch16h<4, EPI>(e, w, bh, ldb, N, g.ncb, ea, p); break;
    case 5: launch16h<5, EPI>(e, w, bh, ldb, N, g.ncb, ea, p); break;
    default: launch16h<6, EPI>(e, w, bh, ldb, N, g.ncb, ea, p); break;
  }
}

template <int NC, int EPI>
static void launch16w(sh_engine* e, const QMat& w, const uint16_t* bh, uint32_t ldb, uint32_t N, const EpiArgs& ea,
                      const MgPlan& p) {
  static const bool deep = [] {
    const char* s = getenv("SH_G16W3");
    return !(s && atoi(s) == 0);
  }();
  const dim3 grid((w.tiles + 15) / 16, p.KS);
  if (deep)
    hipLaunchKernelGGL((k_gemm16w3_q4k<NC, EPI>), grid, dim3(512), 0, e->stream, w.d, w.tiles, w.K / 256, p.S, bh,
                       ldb, N, ea);
  else
    hipLaunchKernelGGL((k_gemm16w_q4k<NC, EPI>), grid, dim3(512), 0, e->stream, w.d, w.tiles, w.K / 256, p.S, bh,
                       ldb, N, ea);
}

template <int NC, int EPI>
static void launch16(sh_engine* e, const QMat& w, const uint16_t* bh, uint32_t ldb, uint32_t N, const EpiArgs& ea,
                     const MgPlan& p) {
  const dim3 grid((w.tiles + 7) / 8, p.KS);
  hipLaunchKernelGGL((k_gemm16_q4k<NC, EPI>), grid, dim3(512), 0, e->stream, w.d, w.tiles, w.K / 256, p.S, bh,
                     ldb, N, ea);
}
template <int EPI>
static void dispatch16(sh_engine* e, const QMat& w, const uint16_t* bh, uint32_t ldb, uint32_t N, const EpiArgs& ea,
                       const MgPlan& p) {
  switch ((N + 15) / 16) {
    case 1: launch16<1, EPI>(e, w, bh, ldb, N, ea, p); break;
    case 2: launch16<2, EPI>(e, w, bh, ldb, N, ea, p); break;
    case 3: launch16<3, EPI>(e, w, bh, ldb, N, ea, p); break;
    case 4: launch16<4, EPI>(e, w, bh, ldb, N, ea, p); break;
    case 5: launch16w<5, EPI>(e, w, bh, ldb, N, ea, p); break;
    case 6: launch16w<6, EPI>(e, w, bh, ldb, N, ea, p); break;
    case 7: launch16w<7, EPI>(e, w, bh, ldb, N, ea, p); break;
    case 8: launch16w<8, EPI>(e, w, bh, ldb, N, ea, p); break;
    case 9: launch16w<9, EPI>(e, w, bh, ldb, N, ea, p); break;
    case 10: launch16w<10, EPI>(e, w, bh, ldb, N, ea, p); break;
    case 11: launch16w<11, EPI>(e, w, bh, ldb, N, ea, p); break;
    default: launch16w<12, EPI>(e, w, bh, ldb, N, ea, p); break;
  }
}

int sh_gemm16_launch(sh_engine* e, const QMat& w, const uint16_t* bh, uint32_t ldb, uint32_t N, EpiKind epi,
                     const EpiArgs& ea, const char* tag, uint32_t* nparts) {
  if (w.type != GGML_Q4_K) return sh_gemm16x_launch(e, w, bh, ldb, N, epi, ea, tag, nparts);  // gemm16x.hip
  SH_CHECK(N >= 1 && N <= SH_MAX_COLS16, SH_ERR_ARG, "f16 gemm N=%u outside [1, %u]", N, SH_MAX_COLS16);
  SH_CHECK(w.type == GGML_Q4_K && w.K % 256 == 0 && ldb >= w.K && ldb % 8 == 0, SH_ERR_UNSUPPORTED,
           "f16 gemm needs Q4_K (type %d) and an operand of at least K = %u halves per column (ldb %u)", w.type, w.K,
           ldb);
  SH_CHECK(epi == EPI_PART || epi == EPI_STORE, SH_ERR_ARG, "f16 gemm epilogue %d", (int)epi);
  const bool h = N > SH_MAX_COLS && use16h(w, epi == EPI_STORE, N);
  const MgPlan p = h ? plan16h(w, epi == EPI_STORE, N)
                     : N > SH_MAX_COLS ? plan16w(w, epi == EPI_STORE, N) : plan16(w, epi == EPI_STORE);
  if (epi == EPI_PART)
    SH_CHECK(ea.part_cap >= p.KS && ea.part_stride >= (size_t)((N + 7) / 8 * 8) * ea.ldo, SH_ERR_CAPACITY,
             "f16 gemm: %u split partials exceed the buffer (%u)", p.KS, ea.part_cap);
  hipEvent_t ev = nullptr;
  sh_prof_begin(e, &ev);
  if (h) {
    if (epi == EPI_PART) dispatch16h<EPI_PART>(e, w, bh, ldb, N, ea, p);
    else dispatch16h<EPI_STORE>(e, w, bh, ldb, N, ea, p);
  } else if (epi == EPI_PART) {
    dispatch16<EPI_PART>(e, w, bh, ldb, N, ea, p);
  } else {
    dispatch16<EPI_STORE>(e, w, bh, ldb, N, ea, p);
  }
  SH_HIP(hipGetLastError());
  sh_prof_end(e, tag, w.alg_bytes, ev);
  if (nparts) *nparts = p.KS;
  return SH_OK;
}

int sh_qkv_finish_launch(sh_engine* e, const float* part, uint32_t nparts, size_t part_stride, uint32_t ldp,
                         uint32_t N, const EpiArgs& ea, const QkvCols& qc) {
  SH_CHECK(N >= 1 && N <= (qc.tab ? (uint32_t)SH_MAX_COLS16 : (uint32_t)SH_MAX_COLS) && ea.hd % 4 == 0, SH_ERR_ARG,
           "qkv finish shape");
  SH_CHECK(!(qc.tab && ea.dbase), SH_ERR_ARG, "qkv finish: a device column table has no graph base");
  SH_CHECK(qc.row0 % 4 == 0 && qc.row0 < ea.Dq + 2 * ea.Dkv && (qc.row0 < ea.Dq + ea.Dkv || qc.vpart), SH_ERR_ARG,
           "qkv finish: first row %u", qc.row0);
  const uint32_t rows = ea.Dq + 2 * ea.Dkv - qc.row0;
  hipEvent_t ev = nullptr;
  sh_prof_begin(e, &ev);
  hipLaunchKernelGGL(k_qkv_finish, dim3((rows / 4 + 63) / 64, N), dim3(64), 0, e->stream, part, nparts, part_stride,
                     ldp, ea, qc);
  SH_HIP(hipGetLastError());
  sh_prof_end(e, "qkv_finish", 0.0, ev);
  return SH_OK;
}

int sh_qkv_finish_head_launch(sh_engine* e, const float* part, uint32_t nparts, size_t part_stride, uint32_t ldp,
                              uint32_t N, const EpiArgs& ea, const QkvCols& qc, const float* q_norm,
                              const float* k_norm, float eps, bool neox) {
  SH_CHECK(!qc.tab && N >= 1 && N <= SH_MAX_COLS && (ea.hd == 64 || ea.hd == 128) && ea.Dq % ea.hd == 0, SH_ERR_ARG,
           "qkv head finish shape");
  const uint32_t heads = ea.Dq / ea.hd + 2 * ea.n_kv;
  hipEvent_t ev = nullptr;
  sh_prof_begin(e, &ev);
  hipLaunchKernelGGL(k_qkv_finish_head, dim3(heads, N), dim3(ea.hd), 0, e->stream, part, nparts, part_stride, ldp, ea,
                     qc, q_norm, k_norm, eps, neox ? 1 : 0);
  SH_HIP(hipGetLastError());
  sh_prof_end(e, "qkv_finish", 0.0, ev);
  return SH_OK;
}

int sh_moe_gemm_launch(sh_engine* e, const QMat& w, uint32_t n_expert, const uint16_t* bx, const uint16_t* xs,
                       const float* cs, uint32_t max_chunks, const uint32_t* info, const uint32_t* gcol,
                       const EpiArgs& ea, const char* tag, double alg_bytes) {
  SH_CHECK(sh_is_kquant(w.type) && w.K % 256 == 0 && n_expert >= 1 && w.tiles % n_expert == 0, SH_ERR_UNSUPPORTED,
           "expert gemm needs K-quant expert slabs of whole tiles");
  SH_CHECK(ea.out && ea.ldo >= w.M / n_expert, SH_ERR_ARG, "expert gemm output");
  const uint32_t tiles_e = w.tiles / n_expert, nsb = w.K / 256;
  hipEvent_t ev = nullptr;
  sh_prof_begin(e, &ev);
  // Q4_K slabs of 8 or more superblocks (the experts' gate/up) with two tiles
  // per wave: twice the weight bytes in flight per wave at one workgroup per
  // CU (132 VGPRs), 2.85 -> 2.72 ms per step of the 8 x 7-column
  // Qwen3-30B-A3B-shape verify; the 768-wide down (3 superblocks) is faster
  // with one (1.52 vs 1.74 ms), four is slower for both
  if (w.type == GGML_Q4_K && nsb >= 8) {
    const uint32_t rb2 = (tiles_e + 15) / 16;
    hipLaunchKernelGGL((k_moe_gemm_kq<FmtQ4K, 2>), dim3(max_chunks * rb2), dim3(512), 0, e->stream, w.d, tiles_e, nsb,
                       rb2, bx, xs, cs, info, gcol, ea);
    SH_HIP(hipGetLastError());
    sh_prof_end(e, tag, alg_bytes, ev);
    return SH_OK;
  }
  constexpr int T = 1;
  const uint32_t rb_e = (tiles_e + 8 * T - 1) / (8 * T);
  const dim3 grid(max_chunks * rb_e);
  if (w.type == GGML_Q5_K)
    hipLaunchKernelGGL((k_moe_gemm_kq<FmtQ5K, T>), grid, dim3(512), 0, e->stream, w.d, tiles_e, nsb, rb_e, bx, xs, cs,
                       info, gcol, ea);
  else if (w.type == GGML_Q6_K)
    hipLaunchKernelGGL((k_moe_gemm_kq<FmtQ6K, T>), grid, dim3(512), 0, e->stream, w.d, tiles_e, nsb, rb_e, bx, xs, cs,
                       info, gcol, ea);
  else
    hipLaunchKernelGGL((k_moe_gemm_kq<FmtQ4K, T>), grid, dim3(512), 0, e->stream, w.d, tiles_e, nsb, rb_e, bx, xs, cs,
                       info, gcol, ea);
  SH_HIP(hipGetLastError());
  sh_prof_end(e, tag, alg_bytes, ev);
  return SH_OK;
}
