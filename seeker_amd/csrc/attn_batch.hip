// Batched verify attention: one launch per layer over every attention segment
// of a forward chunk (B sequences of a batched verify, the B trees of a tree
// verify, the B x (k + 1) columns of a MoE verify), then one combine launch.
//
// Semantics as attn.hip (shaders/compute/flash_attn.slang: online softmax of
// q.K^T * hd^-1/2 over keys [0, kvlen); keys below mask_base always visible,
// keys from mask_base on need their bit in the column's mask: causal chains
// (models/llama.rs:904-955) or ancestor-or-self trees; split-K combine of
// flash_attn_split_k_reduce.slang).
//
// Design (gfx950). A segment has R = gqa x ncol query rows per kv head (up to
// 256). A workgroup of 4 waves owns (segment, key split, kv head) and streams
// the split's keys in tiles (32 keys in a ring of 3 buffers, or 64 keys
// double buffered with KP = 2 below): K (rows of hd f16) and V (32-key blocks,
// [hd][32] each) go global -> LDS by direct 16-byte loads, so the next tiles
// are in flight while tile t is used. The LDS images
// are XOR-swizzled (K: 16-byte chunk c of key row j at c ^ (j % chunks per
// row); V: chunk c of d row at c ^ (d / 2 % 4)), so the 8 lanes of an MFMA
// operand read that share a 128-byte bank window hit 8 different 16-byte slots. Each wave owns RGW groups of 16 query
// rows (rows split over waves, not keys, so every K/V tile is read once from
// HBM for all R rows) and keeps their Q operands (hi + lo f16, a power-of-two
// scale per row) and running (m, l, O) in registers across the split. With
// KP = 2 (segments of at most 32 rows) the two 32-key blocks of a tile go to
// two waves, which write separate partials. Scores run in base 2 (log2(e)
// folded into the scale, v_exp_f32); maxima are stored in natural units so the
// combine of attn.hip's kernels applies unchanged.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <string>
#include <type_traits>
#include <vector>

#include "sh_internal.h"
#include "sh_dma.h"
#include "sh_operand.h"

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void glb_void_t;

namespace {

struct alignas(16) u32x4b { uint32_t x, y, z, w; };

__device__ __forceinline__ f4 mfma16b(h8 a, h8 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
__device__ __forceinline__ h8 lds_h8(const uint16_t* p) { return __builtin_bit_cast(h8, *(const u32x4b*)p); }

__device__ __forceinline__ void split8b(const float* x, h8& hi, h8& lo) {
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const _Float16 h = (_Float16)x[t];
    hi[t] = h;
    lo[t] = (_Float16)(x[t] - (float)h);
  }
}

// Workgroup barrier for LDS hand-offs only. __syncthreads() would also wait
// for every outstanding global load (its fence drains vmcnt), including the
// next tile's prefetch; the direct-LDS loads are waited for explicitly.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

constexpr int kTK = 64;     // keys per tile
constexpr int kWaves = 4;   // waves per workgroup

// TK keys per tile, NS tiles in the LDS ring (NS - 1 in flight while one is
// used). KP = 2 takes 64-key tiles (its two 32-key blocks go to two waves),
// double buffered. KP = 1 takes 32-key tiles in a ring of 3: 48 KB of LDS at
// hd 128 instead of 64 KB, so three workgroups share a CU (three waves per
// SIMD instead of two; the tree verify's attention 2.56 -> 2.12 ms per step,
// where a ring of 4 at two workgroups per CU measured no gain: the waves wait
// on their own MFMA / exp / LDS chains, not on the loads).
template <int HD, int RGW, int KP, int NS = (KP == 2 ? 2 : 3)>
__global__ __launch_bounds__(64 * kWaves, (KP == 1 && RGW == 1) ? (NS == 2 ? 4 : 3) : 2) void k_fab(const FabSeg* __restrict__ segs, const uint32_t* __restrict__ work,
                                                     const float* __restrict__ q, uint32_t n_head, uint32_t gqa,
                                                     uint32_t n_kv, uint32_t layer, uint32_t tps, float scale_log2,
                                                     float* __restrict__ part) {
  // LEAN (2-deep ring, one row group, one key phase): K and V fragments in
  // halves, under 128 VGPRs, so four workgroups share a CU
  constexpr bool LEAN = NS == 2 && KP == 1 && RGW == 1;
  constexpr int TK = KP == 2 ? kTK : 32;  // keys per tile
  constexpr int NB = TK / 32;             // 32-key blocks per tile
  constexpr int NC = HD / 32, DT = HD / 16, CPR = HD / 8;
  constexpr int KI = TK * CPR / 64;    // wave instructions of one K tile (1 KB each)
  constexpr int VI = NB * HD * 4 / 64;  // ... of one V tile
  constexpr int NLD = (KI + VI) / kWaves;  // per wave per tile
  constexpr int WG = kWaves / KP;      // waves per key phase
  constexpr uint32_t PS = sh_fa_part_stride(HD);
  static_assert((KI + VI) % kWaves == 0, "tile loads must spread evenly over the waves");
  static_assert(KP == 1 || NB == 2, "KP = 2 splits a tile's two key blocks over two waves");
  static_assert(NS >= 2 && NS <= 4 && (NS - 1) * NLD < 64, "ring depth");
  // NS buffers, selected at compile time (tiles go in groups of NS)
  __shared__ __align__(16) uint16_t sKr[NS][TK * HD];
  __shared__ __align__(16) uint16_t sVr[NS][NB * HD * 32];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4, r = lane & 15;
  const int kp = wave % KP, wg = wave / KP;
  const uint32_t wi = work[blockIdx.x];
  const uint32_t si = wi >> 20, split = (wi >> 4) & 0xFFFFu, rc = wi & 15u, kh = blockIdx.y;
  const FabSeg& sg = segs[si];
  const uint32_t ncol = sg.ncol, R = gqa * ncol, RG = (R + 15) / 16;
  // row chunk rc: row groups [rc RGc, rc RGc + RGc) of nch balanced chunks
  const uint32_t nch = KP == 1 ? (RG + kWaves * RGW - 1) / (kWaves * RGW) : 1u;
  const uint32_t RGc = (RG + nch - 1) / nch, rg_end = min(RG, (rc + 1) * RGc);
  const uint32_t kvlen = sg.kvlen, mbase = sg.mask_base, max_seq = sg.max_seq;
  const uint32_t key_begin = split * tps * kTK;
  const uint32_t key_end = min(key_begin + tps * kTK, kvlen);
  const uint32_t ntiles = (key_end - key_begin + TK - 1) / TK;
  const size_t lstride = (size_t)n_kv * max_seq * HD;
  const uint16_t* kb = sg.k + layer * lstride + (size_t)kh * max_seq * HD;
  const uint16_t* vb = sg.v + layer * lstride + (size_t)kh * max_seq * HD;

  auto issue = [&](uint32_t t, auto bufc) {
    constexpr int buf = decltype(bufc)::value;
    uint16_t* sK = sKr[buf];
    uint16_t* sV = sVr[buf];
    const uint32_t key0 = key_begin + t * TK;
#pragma unroll
    for (int i = wave; i < KI; i += kWaves) {
      const int qc = 64 * i + lane, row = qc / CPR, c = qc % CPR;
      const uint32_t key = min(key0 + (uint32_t)row, max_seq - 1);  // past the cache: in bounds, masked
      const uint16_t* src = kb + (size_t)key * HD + 8 * (c ^ (row % CPR));
      sh_dma16(src, &sK[512 * i]);
    }
#pragma unroll
    for (int i = wave; i < VI; i += kWaves) {
      const int qc = 64 * i + lane, c = qc & 3, dra = qc >> 2, blk = dra / HD, dr = dra % HD;
      const uint32_t vblk = min(key0 / 32 + (uint32_t)blk, max_seq / 32 - 1);
      const uint16_t* src = vb + ((size_t)vblk * HD + dr) * 32 + 8 * (c ^ ((dr >> 1) & 3));
      sh_dma16(src, &sV[512 * i]);
    }
  };
  // the first NS - 1 tiles (past the split's end: tile 0 again, into an idle
  // buffer, so every path keeps the same count of loads in flight)
  issue(0u, std::integral_constant<int, 0>{});
  if constexpr (NS > 2) issue(1u < ntiles ? 1u : 0u, std::integral_constant<int, 1>{});
  if constexpr (NS > 3) issue(2u < ntiles ? 2u : 0u, std::integral_constant<int, 2>{});

  // The wave's row groups: rgi = rc RGc + wg + WG i. Lane (g, r) holds row
  // 16 rgi + r, d = 32 c + 8 g .. + 7 of the Q^T operand.
  h8 qhi[RGW][NC], qlo[RGW][NC];
  float rs[RGW];
  uint64_t cm[RGW];
  bool live[RGW];
#pragma unroll
  for (int i = 0; i < RGW; ++i) {
    const uint32_t rgi = rc * RGc + wg + WG * i;
    live[i] = wg + WG * i < RGc && rgi < rg_end;  // wave-uniform
    const uint32_t rho = 16 * rgi + r;
    const bool ok = rho < R;
    const uint32_t hq = ok ? rho / ncol : 0, col = ok ? rho % ncol : 0;
    cm[i] = ok ? sg.masks[col] : 0ull;
    const float* qp = q + (size_t)(sg.col0 + col) * n_head * HD + (size_t)(kh * gqa + hq) * HD + 8 * g;
    float x[NC][8];
    float mx = 0.f;
    const float z = ok ? 1.0f : 0.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const float4 a = *(const float4*)(qp + 32 * c), b = *(const float4*)(qp + 32 * c + 4);
      x[c][0] = a.x * z; x[c][1] = a.y * z; x[c][2] = a.z * z; x[c][3] = a.w * z;
      x[c][4] = b.x * z; x[c][5] = b.y * z; x[c][6] = b.z * z; x[c][7] = b.w * z;
#pragma unroll
      for (int t = 0; t < 8; ++t) mx = fmaxf(mx, fabsf(x[c][t]));
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    int ex = 0;
    if (mx > 0.f && mx < INFINITY) {
      frexpf(mx, &ex);
      ex = ex < -100 ? -100 : (ex > 100 ? 100 : ex);
    }
    const float s = ldexpf(1.0f, 10 - ex);
    rs[i] = scale_log2 * ldexpf(1.0f, ex - 10);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
#pragma unroll
      for (int t = 0; t < 8; ++t) x[c][t] *= s;
      split8b(x[c], qhi[i][c], qlo[i][c]);
    }
  }

  f4 o[RGW][DT];
  float mrow[RGW], lrow[RGW];
#pragma unroll
  for (int i = 0; i < RGW; ++i) {
    mrow[i] = -INFINITY;
    lrow[i] = 0.f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[i][dt] = f4{0.f, 0.f, 0.f, 0.f};
  }

  auto step = [&](uint32_t t, auto bufc) {
    constexpr int buf = decltype(bufc)::value;
    const uint16_t* sK = sKr[buf];
    const uint16_t* sV = sVr[buf];
    // Tile t + NS - 1's loads go out unconditionally (past the last tile, tile
    // t again, from L2, into the idle buffer the previous step released): with
    // the same count of loads in flight on every path, the compiler's own
    // waits before the LDS reads stay at (NS - 1) NLD instead of draining the
    // prefetch.
    issue(t + NS - 1 < ntiles ? t + NS - 1 : t, std::integral_constant<int, (buf + NS - 1) % NS>{});
    sh_wait_vm<(NS - 1) * NLD>();
    lds_barrier();
#pragma unroll
    for (int bb = 0; bb < NB; ++bb) {
      if (KP == 2 && bb != kp) continue;
      const uint32_t key0 = key_begin + t * TK + 32 * bb;
      // scores of every row group from the K fragments first, then the V
      // fragments: K and V operands are never live together
      f4 sacc[RGW][2];
      if constexpr (LEAN) {
        // one 16-key tile's K fragments at a time (16 registers, not 32)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
          h8 kop[NC];
          const int row = 32 * bb + 16 * kt + r;
#pragma unroll
          for (int c = 0; c < NC; ++c) kop[c] = lds_h8(&sK[row * HD + 8 * ((4 * c + g) ^ (row % CPR))]);
          f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            acc = mfma16b(kop[c], qhi[0][c], acc);
            acc = mfma16b(kop[c], qlo[0][c], acc);
          }
          sacc[0][kt] = acc;
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {
        h8 kop[2][NC];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
          const int row = 32 * bb + 16 * kt + r;
#pragma unroll
          for (int c = 0; c < NC; ++c) kop[kt][c] = lds_h8(&sK[row * HD + 8 * ((4 * c + g) ^ (row % CPR))]);
        }
#pragma unroll
        for (int i = 0; i < RGW; ++i) {
          if (!live[i]) continue;
#pragma unroll
          for (int kt = 0; kt < 2; ++kt) {
            f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < NC; ++c) {
              acc = mfma16b(kop[kt][c], qhi[i][c], acc);
              acc = mfma16b(kop[kt][c], qlo[i][c], acc);
            }
            sacc[i][kt] = acc;
          }
        }
      }
      // V fragments: all DT, or (LEAN) the first half now, the second after
      // the first half's products
      constexpr int VH = LEAN ? DT / 2 : DT;
      auto load_v = [&](h8* vv, int dt0) {
#pragma unroll
        for (int j = 0; j < VH; ++j) {
          const int dr = 16 * (dt0 + j) + r;
          vv[j] = lds_h8(&sV[(bb * HD + dr) * 32 + 8 * (g ^ ((dr >> 1) & 3))]);
        }
      };
      h8 vop[VH];
      load_v(vop, 0);
      const bool tail = key0 + 32 > key_end || key0 + 32 > mbase;
#pragma unroll
      for (int i = 0; i < RGW; ++i) {
        if (!live[i]) continue;
        float sv[8];
        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            float v = sacc[i][kt][j] * rs[i];
            if (tail) {
              const uint32_t key = key0 + 16 * kt + 4 * g + j;
              bool vis = key < key_end;
              if (vis && key >= mbase) vis = (cm[i] >> (key - mbase)) & 1ull;
              if (!vis) v = -INFINITY;
            }
            sv[4 * kt + j] = v;
            mx = fmaxf(mx, v);
          }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float mnew = fmaxf(mrow[i], mx);
        const bool none = mnew == -INFINITY;  // nothing visible yet: O and l stay zero
        const float alpha = none ? 1.0f : __builtin_amdgcn_exp2f(mrow[i] - mnew);
        // probabilities carry 2^12 (keeps their f16 low halves normal); it
        // cancels in O / l, which are summed from the same values
        const float mb = mnew - 12.0f;
        float p[8], ps = 0.f;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          p[u] = none ? 0.0f : __builtin_amdgcn_exp2f(sv[u] - mb);
          ps += p[u];
        }
        mrow[i] = mnew;
        lrow[i] = lrow[i] * alpha + ps;
        h8 phi, plo;
        split8b(p, phi, plo);
#pragma unroll
        for (int dt = 0; dt < VH; ++dt) {
          o[i][dt] *= alpha;
          o[i][dt] = mfma16b(vop[dt], phi, o[i][dt]);
          o[i][dt] = mfma16b(vop[dt], plo, o[i][dt]);
        }
        if constexpr (LEAN) {
          __builtin_amdgcn_sched_barrier(0);
          load_v(vop, VH);
#pragma unroll
          for (int dt = 0; dt < VH; ++dt) {
            o[i][VH + dt] *= alpha;
            o[i][VH + dt] = mfma16b(vop[dt], phi, o[i][VH + dt]);
            o[i][VH + dt] = mfma16b(vop[dt], plo, o[i][VH + dt]);
          }
        }
      }
    }
    lds_barrier();  // every wave is done with this buffer before it is refilled
  };
  for (uint32_t t = 0; t < ntiles; t += NS) {
    step(t, std::integral_constant<int, 0>{});
    if (t + 1 < ntiles) step(t + 1, std::integral_constant<int, 1>{});
    if constexpr (NS > 2) if (t + 2 < ntiles) step(t + 2, std::integral_constant<int, 2 % NS>{});
    if constexpr (NS > 3) if (t + 3 < ntiles) step(t + 3, std::integral_constant<int, 3 % NS>{});
  }
  sh_wait_vm<0>();  // no LDS write may land after the workgroup ends

  const uint32_t nsv = sg.nsplit * KP, vs = split * KP + kp;
  float* pbase = part + sg.part_off + ((size_t)kh * nsv + vs) * sg.rows_pad * PS;
#pragma unroll
  for (int i = 0; i < RGW; ++i) {
    if (!live[i]) continue;
    float l = lrow[i];
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    const uint32_t rho = 16 * (rc * RGc + wg + WG * i) + r;
    if (rho >= R) continue;
    float* dst = pbase + (size_t)rho * PS;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) *(float4*)(dst + 16 * dt + 4 * g) = make_float4(o[i][dt][0], o[i][dt][1], o[i][dt][2], o[i][dt][3]);
    if (g == 0) *(float4*)(dst + HD) = make_float4(mrow[i] * 0.69314718055994531f, l, 0.f, 0.f);
  }
}

// Split combine per (superblock of the attention output, chunk column): the
// column's segment gives its partials; writes attn [nc][Dq] and the column's
// superblock of the Wo operand (with bh: the f16 row bh[c][Dq] of the wide
// f16 GEMM instead).
// NCH: chunks of 16 partials loaded together (sh_fa_combine4); 1 when no
// segment has more than 17 (half the registers, no clamped repeat loads),
// with bit-identical results.
template <int HD, int NCH>
__global__ __launch_bounds__(64) void k_fab_combine(const FabSeg* __restrict__ segs, const uint32_t* __restrict__ colseg,
                                                    const float* __restrict__ part, uint32_t n_head, uint32_t gqa,
                                                    uint32_t kp, float* __restrict__ attn, uint16_t* __restrict__ bx,
                                                    uint16_t* __restrict__ xs, float* __restrict__ cs,
                                                    uint16_t* __restrict__ bh) {
  const uint32_t sb = blockIdx.x, c = blockIdx.y, lane = threadIdx.x;
  const FabSeg& sg = segs[colseg[c]];
  const uint32_t Dq = n_head * HD, k = 256 * sb + 4 * lane, nsv = sg.nsplit * kp;
  const float4 v = sh_fa_combine4<NCH>(part + sg.part_off, nsv, nsv, sg.rows_pad, HD, n_head, gqa, sg.ncol, sb,
                                     c - sg.col0);
  if (k < Dq) *(float4*)(attn + (size_t)c * Dq + k) = v;
  if (bh) {
    typedef _Float16 hv4 __attribute__((ext_vector_type(4)));
    const hv4 h = {(_Float16)v.x, (_Float16)v.y, (_Float16)v.z, (_Float16)v.w};
    if (k < Dq) *(uint2*)(bh + (size_t)c * Dq + k) = __builtin_bit_cast(uint2, h);
  } else {
    sh_operand_store_sb(v, Dq, sb, c, bx, xs, cs);
  }
}

template <int HD, int RGW, int KP, int NS = (KP == 2 ? 2 : 3)>
void launch_fab(const FabLaunch& fl, hipStream_t st, const float* q, uint32_t n_head, uint32_t gqa, uint32_t n_kv,
                uint32_t layer, float scale_log2, float* part) {
  hipLaunchKernelGGL((k_fab<HD, RGW, KP, NS>), dim3(fl.nwork, n_kv), dim3(64 * kWaves), 0, st, fl.segs, fl.work, q,
                     n_head, gqa, n_kv, layer, fl.tps, scale_log2, part);
}
// One row group per wave, one key phase: the lean variant (2-deep ring, K and
// V fragments in halves, 127 VGPRs, four workgroups per CU) unless
// SH_FAB4=0 (3-deep ring, 147 VGPRs, three per CU). Measured at hd 128:
// the tree step's attention 2.11 -> 1.98 ms, the MoE verify's 2.93 -> 2.81.
static bool fab4() {
  static const bool v = [] {
    const char* s = getenv("SH_FAB4");
    return !(s && std::string(s) == "0");
  }();
  return v;
}

template <int HD>
void launch_fab_hd(const FabLaunch& fl, hipStream_t st, const float* q, uint32_t n_head, uint32_t gqa, uint32_t n_kv,
                   uint32_t layer, float scale_log2, float* part) {
  if (fl.kp == 2) launch_fab<HD, 1, 2>(fl, st, q, n_head, gqa, n_kv, layer, scale_log2, part);
  else if (fl.rgw == 1 && fab4()) launch_fab<HD, 1, 1, 2>(fl, st, q, n_head, gqa, n_kv, layer, scale_log2, part);
  else if (fl.rgw == 1) launch_fab<HD, 1, 1>(fl, st, q, n_head, gqa, n_kv, layer, scale_log2, part);
  else launch_fab<HD, 2, 1>(fl, st, q, n_head, gqa, n_kv, layer, scale_log2, part);
}

}  // namespace

int sh_fab_plan(sh_engine* e, sh_model* m, const FabSegIn* in, uint32_t nseg, uint32_t nc, FabLaunch* out) {
  *out = FabLaunch{};
  SH_CHECK(nseg >= 1 && nseg <= 0xFFF && nc >= 1, SH_ERR_ARG, "batched attention: %u segments, %u columns", nseg, nc);
  SH_CHECK(m->hd == 64 || m->hd == 128, SH_ERR_UNSUPPORTED, "head_dim %u not supported (64, 128)", m->hd);
  const uint32_t gqa = m->n_head / m->n_kv, PS = sh_fa_part_stride(m->hd);
  uint64_t tiles = 0;
  uint32_t max_rg = 0;
  for (uint32_t s = 0; s < nseg; ++s) {
    const FabSegIn& a = in[s];
    SH_CHECK(a.kv && a.ncol >= 1 && a.col0 + a.ncol <= nc && a.ncol <= 64 && a.kvlen >= 1 && a.kvlen <= a.kv->max_seq &&
                 a.hmasks,
             SH_ERR_ARG, "batched attention: segment %u (columns [%u, +%u), %u keys) malformed", s, a.col0, a.ncol,
             a.kvlen);
    SH_CHECK(a.kv->max_seq % 32 == 0 && a.kv->n_kv == m->n_kv && a.kv->hd == m->hd, SH_ERR_ARG,
             "batched attention: segment %u cache does not match the model", s);
    const uint32_t R = gqa * a.ncol;
    SH_CHECK(R <= (uint32_t)SH_FA_MAX_ROWS, SH_ERR_UNSUPPORTED, "%u query rows per kv head above %d", R,
             SH_FA_MAX_ROWS);
    max_rg = std::max(max_rg, (R + 15) / 16);
    tiles += (uint64_t)m->n_kv * ((a.kvlen + kTK - 1) / kTK);
  }
  // Geometry of the launch: rows split over the 4 waves (RGW groups of 16 per
  // wave, segments above 4 RGW groups in row chunks), or the two key blocks of
  // a tile over pairs of waves (KP = 2) when no segment has more than 2 row
  // groups; tiles per split chosen for about 512 workgroups and at least 4
  // keys per split for every row.
  static const int forced_rgw = [] {  // SH_FAB_RGW=1|2: row groups per wave (measurement switch)
    const char* v = getenv("SH_FAB_RGW");
    return v ? atoi(v) : 0;
  }();
  // One row group per wave by default: segments above 4 row groups go in row
  // chunks of 4 whose K/V re-reads hit L2; two per wave (SH_FAB_RGW=2) leaves
  // waves idle at the tile barriers when a chunk's count is not a multiple of 4
  // (tree verify attention 3.8 vs 4.6 ms per step, measured).
  out->kp = max_rg <= 2 ? 2 : 1;
  out->max_nsv = 0;
  out->rgw = (out->kp == 1 && forced_rgw == 2) ? 2 : 1;
  const uint32_t rows_max = 16 * max_rg;
  // (a split's partials are rows x (hd + 4) floats against keys x 2 hd f16 of
  // K/V: keys >= 4 rows keeps them under a quarter of the K/V bytes)
  uint32_t tps = (uint32_t)((tiles + 511) / 512);
  tps = std::max<uint32_t>(tps, (4 * rows_max + kTK - 1) / kTK);
  tps = std::max<uint32_t>(2, std::min<uint32_t>(tps, 64));
  out->tps = tps;
  const uint32_t SK = tps * kTK;
  std::vector<FabSeg> segs(nseg);
  std::vector<uint32_t> work;
  size_t part_floats = 0;
  for (uint32_t s = 0; s < nseg; ++s) {
    const FabSegIn& a = in[s];
    FabSeg& d = segs[s];
    d.k = a.kv->k; d.v = a.kv->v; d.masks = nullptr; d.part_off = part_floats;
    d.max_seq = a.kv->max_seq; d.kvlen = a.kvlen; d.mask_base = a.mask_base; d.col0 = a.col0; d.ncol = a.ncol;
    d.rows_pad = (gqa * a.ncol + 15) / 16 * 16;
    d.nsplit = (a.kvlen + SK - 1) / SK;
    SH_CHECK(d.nsplit <= 0xFFFF, SH_ERR_UNSUPPORTED, "batched attention: %u key splits", d.nsplit);
    out->max_nsv = std::max(out->max_nsv, d.nsplit * out->kp);
    part_floats += (size_t)m->n_kv * d.nsplit * out->kp * d.rows_pad * PS;
    const uint32_t RG = d.rows_pad / 16;
    const uint32_t nch = out->kp == 1 ? (RG + 4 * out->rgw - 1) / (4 * out->rgw) : 1u;
    // The row chunks of one (segment, split) read the same K/V tiles: groups of
    // 8 splits go out chunk by chunk, so a split's chunks are 8 workgroups
    // apart and land on one XCD (workgroups are dealt to the 8 XCDs in turn),
    // where the later chunks find the tiles in that XCD's L2.
    for (uint32_t sp0 = 0; sp0 < d.nsplit; sp0 += 8)
      for (uint32_t rc = 0; rc < nch; ++rc)
        for (uint32_t sp = sp0; sp < std::min<uint32_t>(sp0 + 8, d.nsplit); ++sp)
          work.push_back((s << 20) | (sp << 4) | rc);
  }
  // device tables: segments, work items, column -> segment, masks
  const size_t o_work = ((size_t)nseg * sizeof(FabSeg) + 255) / 256 * 256;
  const size_t o_col = o_work + ((work.size() * 4 + 255) / 256) * 256;
  const size_t o_mask = o_col + ((size_t)nc * 4 + 255) / 256 * 256;
  const size_t bytes = o_mask + (size_t)nc * 8;
  std::vector<uint8_t> host(bytes, 0);
  std::vector<uint32_t> colseg(nc, 0);
  uint64_t* hm = (uint64_t*)(host.data() + o_mask);
  for (uint32_t s = 0; s < nseg; ++s) {
    for (uint32_t j = 0; j < in[s].ncol; ++j) {
      colseg[in[s].col0 + j] = s;
      hm[in[s].col0 + j] = in[s].hmasks[j];
    }
  }
  SH_HIP(hipMallocAsync((void**)&out->dev, bytes, e->stream));
  for (uint32_t s = 0; s < nseg; ++s) segs[s].masks = (const uint64_t*)(out->dev + o_mask) + in[s].col0;
  std::memcpy(host.data(), segs.data(), nseg * sizeof(FabSeg));
  std::memcpy(host.data() + o_work, work.data(), work.size() * 4);
  std::memcpy(host.data() + o_col, colseg.data(), (size_t)nc * 4);
  SH_HIP(hipMemcpyAsync(out->dev, host.data(), bytes, hipMemcpyHostToDevice, e->stream));
  out->segs = (const FabSeg*)out->dev;
  out->work = (const uint32_t*)(out->dev + o_work);
  out->colseg = (const uint32_t*)(out->dev + o_col);
  out->nseg = nseg; out->nwork = (uint32_t)work.size(); out->nc = nc;
  // partial buffer of every segment at once (grown on demand)
  Workspace& w = m->ws;
  if (part_floats > w.fab_part_floats) {
    SH_HIP(hipStreamSynchronize(e->stream));
    SH_HIP(hipFree(w.fab_part));
    w.fab_part = nullptr;
    w.fab_part_floats = 0;
    SH_HIP(hipMalloc(&w.fab_part, part_floats * 4));
    w.fab_part_floats = part_floats;
  }
  out->part = w.fab_part;
  return SH_OK;
}

void sh_fab_free(sh_engine* e, FabLaunch& fl) {
  if (fl.dev) (void)hipFreeAsync(fl.dev, e->stream);
  fl.dev = nullptr;
}

int sh_fab_launch(sh_engine* e, const sh_model* m, const FabLaunch& fl, uint32_t layer, const float* q, float* attn_out,
                  uint16_t* bx, uint16_t* xs, float* cs, uint16_t* bh) {
  const uint32_t gqa = m->n_head / m->n_kv;
  const float scale_log2 = 1.4426950408889634f / sqrtf((float)m->hd);
  hipEvent_t ev = nullptr;
  sh_prof_begin(e, &ev);
  if (m->hd == 128) launch_fab_hd<128>(fl, e->stream, q, m->n_head, gqa, m->n_kv, layer, scale_log2, fl.part);
  else launch_fab_hd<64>(fl, e->stream, q, m->n_head, gqa, m->n_kv, layer, scale_log2, fl.part);
  SH_HIP(hipGetLastError());
  sh_prof_end(e, "attention", 0.0, ev);
  sh_prof_begin(e, &ev);
  const dim3 cgrid((m->n_head * m->hd + 255) / 256, fl.nc);
  const bool one = fl.max_nsv <= 17;
  if (m->hd == 128 && one)
    hipLaunchKernelGGL((k_fab_combine<128, 1>), cgrid, dim3(64), 0, e->stream, fl.segs, fl.colseg, fl.part, m->n_head,
                       gqa, fl.kp, attn_out, bx, xs, cs, bh);
  else if (m->hd == 128)
    hipLaunchKernelGGL((k_fab_combine<128, 2>), cgrid, dim3(64), 0, e->stream, fl.segs, fl.colseg, fl.part, m->n_head,
                       gqa, fl.kp, attn_out, bx, xs, cs, bh);
  else if (one)
    hipLaunchKernelGGL((k_fab_combine<64, 1>), cgrid, dim3(64), 0, e->stream, fl.segs, fl.colseg, fl.part, m->n_head,
                       gqa, fl.kp, attn_out, bx, xs, cs, bh);
  else
    hipLaunchKernelGGL((k_fab_combine<64, 2>), cgrid, dim3(64), 0, e->stream, fl.segs, fl.colseg, fl.part, m->n_head,
                       gqa, fl.kp, attn_out, bx, xs, cs, bh);
  SH_HIP(hipGetLastError());
  sh_prof_end(e, "attn_combine", 0.0, ev);
  return SH_OK;
}
