// The reference's wide-GEMM arithmetic for the weight formats other than Q4_K.
//
// The reference computes every dense matmul of at least 32 columns with its
// cooperative-matrix GEMM (ops/matmul.rs:433-446 -> mul_mm_cm.slang): each
// weight dequantized in f32 and rounded to f16 (stage_a_tile), each activation
// rounded to f16, f32 accumulation; its variants cover Q8_0, Q5_K and Q6_K as
// well as Q4_K (mmcm_variant, ops/matmul.rs:238-290). Q4_K has its own tuned
// kernels (k_gemm16*_q4k in gemv.hip); this file serves Q8_0, Q5_K and Q6_K
// from the same repacked tiles the f32-level kernels read, with the f32
// dequant of the oracle's or_dequant_row done in the same order (each product
// and difference rounded to f32 as written) and rounded once to f16:
//   Q8_0  f16(d * q)
//   Q5_K  f16((d * sc) * q - dmin * m)
//   Q6_K  f16((d * sc) * (q - 32))
// A workgroup of 8 waves covers 8 row tiles (one per wave) over a K-split of
// 32-column units (a Q8_0 block, a K-quant sub-block); each unit's f16
// fragment (row r, k = 8 g + t of lane (g, r)) feeds one
// v_mfma_f32_16x16x32_f16 per 16 columns, the B fragments read straight from
// the f16 rows (they stay in L2: every wave of the chip reads the same rows).
#include "sh_internal.h"

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
struct alignas(16) u32x4 { uint32_t x, y, z, w; };

__device__ __forceinline__ float h2f(uint32_t bits) { return (float)__builtin_bit_cast(_Float16, (uint16_t)bits); }
// f16 of an f32 value that has been rounded to f32 first (no fused
// multiply-convert across the product)
__device__ __forceinline__ _Float16 r16(float y) {
  asm volatile("" : "+v"(y));
  return (_Float16)y;
}
__device__ __forceinline__ float rf(float y) {
  asm volatile("" : "+v"(y));
  return y;
}
// Element t (k = 8 g + t of a lane's 8) of a nibble word in the Q4_K tile
// layout: even t at bits 4 (t / 2), odd t at 16 + 4 (t / 2).
__device__ __forceinline__ uint32_t nib(uint32_t w, int t) {
  return (w >> ((t & 1) ? 16 + 4 * (t >> 1) : 4 * (t >> 1))) & 0xFu;
}
// Bit position of element t's high bits relative to its sub-block's base in
// the repacked high-bit words (X = 1 for Q5_K, 2 for Q6_K).
__device__ __forceinline__ uint32_t hpos(int t, int X) { return 16 * (t & 1) + 4 * ((t >> 1) & 1) + X * ((t >> 2) & 1); }
// The Q4_K / Q5_K 6-bit (scale, min) unpack of sub-block j from the 12 packed
// bytes (apps/seeker-cli/src/commands/run.rs:4223-4232).
__device__ __forceinline__ void scale_min(const uint8_t* s, int j, int& sc, int& m) {
  if (j < 4) {
    sc = s[j] & 63;
    m = s[j + 4] & 63;
  } else {
    sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
    m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
  }
}
__device__ __forceinline__ uint32_t nib_word(const uint8_t* b, int lane, uint32_t m) {
  return *(const uint32_t*)(b + (m < 4 ? 16 * lane + 4 * m : 1024 + 16 * lane + 4 * (m - 4)));
}

// Q8_0 tile-block (544 B): 64 lanes x 8 int8 (row l % 16, k = 8 g + t), then
// the rows' f16 d.
struct W8 {
  static __device__ __forceinline__ h8 frag(const uint8_t* Wp, uint32_t tile, uint32_t nunits, uint32_t u, int lane,
                                            int g, int r) {
    const uint8_t* b = Wp + ((size_t)tile * nunits + u) * SH_Q8_TILE_BYTES;
    const uint2 q = *(const uint2*)(b + 8 * lane);
    const float d = h2f(*(const uint16_t*)(b + 512 + 2 * r));
    h8 a;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int v = (int8_t)(((t < 4 ? q.x : q.y) >> (8 * (t & 3))) & 0xFFu);
      a[t] = r16(d * (float)v);
    }
    return a;
  }
};
// Q5_K tile-superblock (2816 B, see k_repack_q5k): low nibbles as Q4_K, two
// high-bit words per lane, d | dmin << 16 and the 12 scale bytes per row.
struct W5 {
  static __device__ __forceinline__ h8 frag(const uint8_t* Wp, uint32_t tile, uint32_t nunits, uint32_t u, int lane,
                                            int g, int r) {
    const uint32_t nsb = nunits / 8, sb = u >> 3, m = u & 7;
    const uint8_t* b = Wp + ((size_t)tile * nsb + sb) * SH_Q5K_TILE_BYTES;
    const uint32_t w = nib_word(b, lane, m);
    const uint32_t hw = *(const uint32_t*)(b + 2048 + 8 * lane + 4 * (m >> 2));
    const uint32_t dd = *(const uint32_t*)(b + 2560 + 4 * r);
    int sc, mn;
    scale_min(b + 2624 + 12 * r, (int)m, sc, mn);
    const float d1 = rf(h2f(dd & 0xFFFFu) * (float)sc), m1 = rf(h2f(dd >> 16) * (float)mn);
    const uint32_t base = (m & 1) * 2 + ((m >> 1) & 1) * 8;
    h8 a;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const uint32_t q = nib(w, t) | (((hw >> (base + hpos(t, 1))) & 1u) << 4);
      a[t] = r16(rf(d1 * (float)q) - m1);
    }
    return a;
  }
};
// Q6_K tile-superblock (3360 B, see k_repack_q6k): low nibbles in the Q4_K
// layout, four high-bit words per lane, 16 int8 scales per row (even indices,
// then odd), the rows' f16 d.
struct W6 {
  static __device__ __forceinline__ h8 frag(const uint8_t* Wp, uint32_t tile, uint32_t nunits, uint32_t u, int lane,
                                            int g, int r) {
    const uint32_t nsb = nunits / 8, sb = u >> 3, m = u & 7;
    const uint8_t* b = Wp + ((size_t)tile * nsb + sb) * SH_Q6K_TILE_BYTES;
    const uint32_t w = nib_word(b, lane, m);
    const uint32_t hw = *(const uint32_t*)(b + 2048 + 16 * lane + 4 * (m >> 1));
    const int sc = (int8_t)b[3072 + 16 * r + 8 * (g >> 1) + m];
    const float ds = rf(h2f(*(const uint16_t*)(b + 3328 + 2 * r)) * (float)sc);
    const uint32_t base = 8 * (m & 1);
    h8 a;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int q = (int)(nib(w, t) | (((hw >> (base + hpos(t, 2))) & 3u) << 4)) - 32;
      a[t] = r16(ds * (float)q);
    }
    return a;
  }
};

template <class F, int NC, int EPI>
__global__ __launch_bounds__(512) void k_gemm16x(const uint8_t* __restrict__ Wp, uint32_t tiles, uint32_t nunits,
                                                 uint32_t S, const uint16_t* __restrict__ Bh, uint32_t ldb, uint32_t N,
                                                 EpiArgs ea) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4, r = lane & 15;
  const uint32_t tile = blockIdx.x * 8 + wave, ks = blockIdx.y;
  const uint32_t tt = tile < tiles ? tile : tiles - 1;  // clamped rows compute and are dropped
  const uint32_t u0 = ks * S, u1 = min(u0 + S, nunits);
  f4 acc[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) acc[c] = f4{0.f, 0.f, 0.f, 0.f};
  const uint16_t* brow[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) brow[c] = Bh + (size_t)min(16 * c + (uint32_t)r, N - 1) * ldb + 8 * g;
  for (uint32_t u = u0; u < u1; ++u) {
    const h8 a = F::frag(Wp, tt, nunits, u, lane, g, r);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const h8 b = __builtin_bit_cast(h8, *(const u32x4*)(brow[c] + 32 * u));
      acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[c], 0, 0, 0);
    }
  }
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const uint32_t col = 16 * c + r, row0 = tile * 16 + 4 * g;
    if (tile >= tiles || col >= N) continue;
    const f4 v = acc[c];
    if (EPI == EPI_PART) {
      *(float4*)(ea.out + ks * ea.part_stride + (size_t)col * ea.ldo + row0) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (row0 + j < ea.rows) ea.out[(size_t)col * ea.ldo + row0 + j] = v[j];
    }
  }
}

constexpr uint32_t kMaxSplits = 16;

uint32_t units_of(const QMat& w) { return w.type == GGML_Q8_0 ? w.K / 32 : w.K / 256 * 8; }

// K-splits: enough 8-tile workgroups for about two per CU, at most 16 splits.
void plan(const QMat& w, bool one_split, uint32_t& S, uint32_t& KS) {
  const uint32_t nu = units_of(w), wgx = (w.tiles + 7) / 8;
  uint32_t ks = one_split ? 1u : std::min<uint32_t>(kMaxSplits, std::max<uint32_t>(1u, (512 + wgx - 1) / wgx));
  ks = std::min(ks, nu);
  S = (nu + ks - 1) / ks;
  KS = (nu + S - 1) / S;
}

template <class F, int NC, int EPI>
void launch(sh_engine* e, const QMat& w, const uint16_t* bh, uint32_t ldb, uint32_t N, const EpiArgs& ea, uint32_t S,
            uint32_t KS) {
  hipLaunchKernelGGL((k_gemm16x<F, NC, EPI>), dim3((w.tiles + 7) / 8, KS), dim3(512), 0, e->stream, w.d, w.tiles,
                     units_of(w), S, bh, ldb, N, ea);
}

template <class F, int EPI>
void dispatch(sh_engine* e, const QMat& w, const uint16_t* bh, uint32_t ldb, uint32_t N, const EpiArgs& ea,
              uint32_t S, uint32_t KS) {
  switch ((N + 15) / 16) {
    case 1: launch<F, 1, EPI>(e, w, bh, ldb, N, ea, S, KS); break;
    case 2: launch<F, 2, EPI>(e, w, bh, ldb, N, ea, S, KS); break;
    case 3: launch<F, 3, EPI>(e, w, bh, ldb, N, ea, S, KS); break;
    case 4: launch<F, 4, EPI>(e, w, bh, ldb, N, ea, S, KS); break;
    case 5: launch<F, 5, EPI>(e, w, bh, ldb, N, ea, S, KS); break;
    case 6: launch<F, 6, EPI>(e, w, bh, ldb, N, ea, S, KS); break;
    case 7: launch<F, 7, EPI>(e, w, bh, ldb, N, ea, S, KS); break;
    case 8: launch<F, 8, EPI>(e, w, bh, ldb, N, ea, S, KS); break;
    case 9: launch<F, 9, EPI>(e, w, bh, ldb, N, ea, S, KS); break;
    case 10: launch<F, 10, EPI>(e, w, bh, ldb, N, ea, S, KS); break;
    case 11: launch<F, 11, EPI>(e, w, bh, ldb, N, ea, S, KS); break;
    default: launch<F, 12, EPI>(e, w, bh, ldb, N, ea, S, KS); break;
  }
}

template <int EPI>
void dispatch_fmt(sh_engine* e, const QMat& w, const uint16_t* bh, uint32_t ldb, uint32_t N, const EpiArgs& ea,
                  uint32_t S, uint32_t KS) {
  if (w.type == GGML_Q8_0) dispatch<W8, EPI>(e, w, bh, ldb, N, ea, S, KS);
  else if (w.type == GGML_Q5_K) dispatch<W5, EPI>(e, w, bh, ldb, N, ea, S, KS);
  else dispatch<W6, EPI>(e, w, bh, ldb, N, ea, S, KS);
}

}  // namespace

bool sh_gemm16x_ok(const QMat& w) {
  return (w.type == GGML_Q8_0 && w.K % 32 == 0) || ((w.type == GGML_Q5_K || w.type == GGML_Q6_K) && w.K % 256 == 0);
}

size_t sh_gemm16x_part_floats(const QMat& w) {
  if (!sh_gemm16x_ok(w)) return 0;
  uint32_t S = 0, KS = 0;
  plan(w, false, S, KS);
  return (size_t)KS * SH_MAX_COLS16 * w.tiles * 16;
}

int sh_gemm16x_launch(sh_engine* e, const QMat& w, const uint16_t* bh, uint32_t ldb, uint32_t N, EpiKind epi,
                      const EpiArgs& ea, const char* tag, uint32_t* nparts) {
  SH_CHECK(N >= 1 && N <= SH_MAX_COLS16, SH_ERR_ARG, "f16 gemm N=%u outside [1, %u]", N, SH_MAX_COLS16);
  SH_CHECK(sh_gemm16x_ok(w) && ldb >= w.K && ldb % 8 == 0, SH_ERR_UNSUPPORTED,
           "f16 gemm: type %d with K = %u (ldb %u)", w.type, w.K, ldb);
  SH_CHECK(epi == EPI_PART || epi == EPI_STORE, SH_ERR_ARG, "f16 gemm epilogue %d", (int)epi);
  uint32_t S = 0, KS = 0;
  plan(w, epi == EPI_STORE, S, KS);
  if (epi == EPI_PART)
    SH_CHECK(ea.part_cap >= KS && ea.part_stride >= (size_t)((N + 7) / 8 * 8) * ea.ldo, SH_ERR_CAPACITY,
             "f16 gemm: %u split partials exceed the buffer (%u)", KS, ea.part_cap);
  hipEvent_t ev = nullptr;
  sh_prof_begin(e, &ev);
  if (epi == EPI_PART) dispatch_fmt<EPI_PART>(e, w, bh, ldb, N, ea, S, KS);
  else dispatch_fmt<EPI_STORE>(e, w, bh, ldb, N, ea, S, KS);
  SH_HIP(hipGetLastError());
  sh_prof_end(e, tag, w.alg_bytes, ev);
  if (nparts) *nparts = KS;
  return SH_OK;
}
