// Verify-step attention over the f16 KV cache.
//
// Semantics: shaders/compute/flash_attn.slang (online softmax of q.K^T * hd^-1/2
// over keys [0, kvlen); keys below the chunk base are always visible,
// mask_kv_offset :126-129; within-chunk keys follow the [L x L] causal mask of
// models/llama.rs:904-955) and the split-K combine of
// flash_attn_split_k_reduce.slang. Tree verify replaces the causal triangle by
// an ancestor-or-self bitmask per query column (new).
//
// Design (gfx950): one workgroup = (kv head, key split, group of 16*QT query
// rows); each of its W waves takes NH 32-key blocks of the split. A wave issues
// its query loads and then every K and V load of its keys before it waits on
// any of them, so one HBM latency covers the whole split. The GQA rows of one
// kv head (gqa heads x N columns) share every K/V tile, so K and V are read
// once per kv head. S^T = K Q^T and O^T = V^T P^T run on
// v_mfma_f32_16x16x32_f16; Q and P are split into hi + lo f16 halves so the
// products keep ~22 bits (K and V are exact f16). V is stored per 32-key block
// transposed ([hd][32 slots], slot order v_slot()) so the V^T operand is a
// contiguous 16-byte load. A second kernel combines the splits in split order
// (deterministic) per column and builds the Wo activation operand.
#include <cfloat>
#include <cstdlib>
#include <string>

#include "sh_internal.h"
#include "sh_dma.h"
#include "sh_operand.h"

// Scores run in base 2: the score scale carries log2(e), exponentials are the
// hardware exp2 (v_exp_f32), and the split maxima go out in natural units
// (times ln 2), the units the split combine works in.
constexpr float kLog2e = 1.4426950408889634f, kLn2 = 0.69314718055994531f;

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
struct alignas(16) u32x4a { uint32_t x, y, z, w; };
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void glb_void_t;

__device__ __forceinline__ h8 ld_h8(const uint16_t* p) { return __builtin_bit_cast(h8, *(const u32x4a*)p); }
__device__ __forceinline__ f4 mfma16a(h8 a, h8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Workgroup barrier that waits for this wave's LDS accesses only (no vmcnt
// drain, unlike __syncthreads).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Split 8 f32 into hi and lo f16 vectors.
__device__ __forceinline__ void split8(const float* x, h8& hi, h8& lo) {
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    _Float16 h = (_Float16)x[t];
    hi[t] = h;
    lo[t] = (_Float16)(x[t] - (float)h);
  }
}

// colmask[col] by selects: a dynamic index into the kernel arguments would
// become a memory load on the critical path.
__device__ __forceinline__ uint64_t col_mask(const FaArgs& fa, uint32_t col) {
  uint64_t v = fa.colmask[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) v = col == (uint32_t)i ? fa.colmask[i] : v;
  return v;
}

// Partial of split `split` for padded row rho:
// part[((kh * n_splits + split) * n_rows_pad + rho) * PS + {d < HD: O, HD: m, HD+1: l, pad}].
//
// Workgroup = (kv head, key split, group of 16 NQG query rows) of NQG * NKB
// waves; wave w takes key block kb = w % NKB (NH blocks of 32 keys) for row
// group qg = w / NKB (16 query rows). The NQG waves of one key block read the
// same K and V (the second read hits the CU's cache).
template <int HD, int NQG, int NKB, int NH, bool DMASK>
__global__ __launch_bounds__(64 * NQG * NKB) void k_fa(const float* __restrict__ q, const uint16_t* __restrict__ kc,
                                                        const uint16_t* __restrict__ vc, uint32_t max_seq,
                                                        uint32_t n_head, uint32_t N, uint32_t gqa, FaArgs fa,
                                                        float scale, float* __restrict__ part) {
  constexpr int NC = HD / 32;  // d chunks of the QK contraction
  constexpr int DT = HD / 16;  // d tiles of the output
  constexpr int ROWS = 16 * NQG;
  constexpr uint32_t WAVE_KEYS = 32 * NH, SPLIT_KEYS = NKB * WAVE_KEYS, PS = sh_fa_part_stride(HD);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kb = wave % NKB, qg = wave / NKB;
  const int g = lane >> 4, r = lane & 15;
  const uint32_t kh = blockIdx.x, split = blockIdx.y;
  const uint32_t n_splits = gridDim.y;
  // graph replay: live keys and mask base from the device base position
  const uint32_t kbase0 = fa.dbase ? *fa.dbase : 0u;
  const uint32_t kvlen = fa.kvlen + kbase0, mbase = fa.mask_base + kbase0;
  if (fa.dbase && split * (uint32_t)(NKB * 32 * NH) >= kvlen) return;  // uniform: past the live keys
  const uint32_t n_rows = gqa * N;
  const uint32_t n_rows_pad = gridDim.z * ROWS;
  const uint32_t Dq = n_head * HD;

  // This wave's query rows: lane (g, r) holds row rho, d = 32c + 8g .. +8. Rows
  // past n_rows read row 0 and are zeroed.
  const uint32_t rho = blockIdx.z * ROWS + 16 * qg + r;
  const bool ok = rho < n_rows;
  const uint32_t hq = ok ? rho / N : 0, col = ok ? rho % N : 0;
  const float* qp = q + (size_t)col * Dq + (size_t)(kh * gqa + hq) * HD + 8 * g;
  // This wave's keys: blocks past the split's end read clamped (in-bounds) rows
  // and are masked out below.
  const uint32_t k_end = min((split + 1) * SPLIT_KEYS, kvlen);
  const uint32_t kw = split * SPLIT_KEYS + WAVE_KEYS * kb;
  const uint16_t* kbase = kc + (size_t)kh * max_seq * HD;
  const uint16_t* vbase = vc + (size_t)kh * (max_seq / 32) * HD * 32;

  // Every load of the wave's inputs is issued before any is used: Q rows, then
  // K and V. There is no branch between the loads and their uses, and the
  // scheduling barrier keeps them from being sunk, so the split costs one
  // memory latency.
  float4 qraw[NC][2];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    qraw[c][0] = *(const float4*)(qp + 32 * c);
    qraw[c][1] = *(const float4*)(qp + 32 * c + 4);
  }
  h8 kop[NH][2][NC], vop[NH][DT];
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    const uint32_t key0 = min(kw + 32 * h, max_seq - 32);
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int c = 0; c < NC; ++c) kop[h][kt][c] = ld_h8(kbase + (size_t)(key0 + 16 * kt + r) * HD + 8 * g + 32 * c);
    const uint16_t* vp = vbase + (size_t)(key0 / 32) * HD * 32 + (size_t)r * 32 + 8 * g;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) vop[h][dt] = ld_h8(vp + (size_t)dt * 16 * 32);
  }
  const uint64_t cm = DMASK ? fa.masks[col] : col_mask(fa, col);
  __builtin_amdgcn_sched_barrier(0);

  // Q^T operand (B). Each query row is scaled by a power of two (max|q * s| in
  // [2^9, 2^10)) so the f16 low halves stay normal; rscale folds 1/s into the
  // score scale.
  h8 qhi[NC], qlo[NC];
  float rscale;
  {
    const float z = ok ? 1.0f : 0.0f;
    float x[NC][8];
    float mx = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const float4 a = qraw[c][0], b = qraw[c][1];
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
    rscale = scale * ldexpf(1.0f, ex - 10);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
#pragma unroll
      for (int t = 0; t < 8; ++t) x[c][t] *= s;
      split8(x[c], qhi[c], qlo[c]);
    }
  }

  f4 o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] = f4{0.f, 0.f, 0.f, 0.f};
  float mrow = -INFINITY, lrow = 0.f;

#pragma unroll
  for (int h = 0; h < NH; ++h) {
    const uint32_t key0 = kw + 32 * h;
    // S^T[key][rho] for keys key0 + 16*kt + 4g + j.
    f4 sacc[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        acc = mfma16a(kop[h][kt][c], qhi[c], acc);
        acc = mfma16a(kop[h][kt][c], qlo[c], acc);
      }
      sacc[kt] = acc;
    }
    const bool tail = key0 + 32 > k_end || key0 + 32 > mbase;
    float sv[8];
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float v = sacc[kt][j] * rscale;
        if (tail) {
          const uint32_t key = key0 + 16 * kt + 4 * g + j;
          bool vis = key < k_end;
          if (vis && key >= mbase) vis = (cm >> (key - mbase)) & 1ull;
          if (!vis) v = -INFINITY;
        }
        sv[4 * kt + j] = v;
        mx = fmaxf(mx, v);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float mnew = fmaxf(mrow, mx);
    // nothing visible yet: keep O and l (zero) as they are
    const bool none = mnew == -INFINITY;
    const float alpha = none ? 1.0f : __builtin_amdgcn_exp2f(mrow - mnew);
    // probabilities carry a 2^12 factor (keeps their f16 low halves normal);
    // it cancels in O / l because l is summed from the same scaled values
    float p[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) p[t] = none ? 0.0f : __builtin_amdgcn_exp2f(sv[t] - mnew) * 4096.0f;
    mrow = mnew;
    float ps = 0.f;
#pragma unroll
    for (int t = 0; t < 8; ++t) ps += p[t];
    lrow = lrow * alpha + ps;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[dt] *= alpha;
    // P^T operand: lane slot t -> key 4g+t (t<4) or 16+4g+t-4 (t>=4), the order
    // V blocks are stored in.
    h8 phi, plo;
    split8(p, phi, plo);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      o[dt] = mfma16a(vop[h][dt], phi, o[dt]);
      o[dt] = mfma16a(vop[h][dt], plo, o[dt]);
    }
  }
  lrow += __shfl_xor(lrow, 16);
  lrow += __shfl_xor(lrow, 32);

  // Key blocks 1..NKB-1 of each row group park (m, l, O) in LDS (16-byte rows,
  // 132-float stride); key block 0 merges them and writes the split's rows.
  constexpr int KL = NKB > 1 ? NKB - 1 : 1;
  __shared__ float sm[NQG][KL][16], sl[NQG][KL][16];
  __shared__ float4 so[NQG][KL][16][HD / 4 + 1];
  if (NKB > 1) {
    if (kb > 0) {
      if (g == 0) { sm[qg][kb - 1][r] = mrow; sl[qg][kb - 1][r] = lrow; }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) so[qg][kb - 1][r][4 * dt + g] = make_float4(o[dt][0], o[dt][1], o[dt][2], o[dt][3]);
    }
    __syncthreads();
    if (kb > 0) return;
  }
  float M = mrow;
#pragma unroll
  for (int w = 0; w < NKB - 1; ++w) M = fmaxf(M, sm[qg][w][r]);
  const float f0 = mrow == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mrow - M);
  float fw[KL];
  float L = lrow * f0;
#pragma unroll
  for (int w = 0; w < NKB - 1; ++w) {
    fw[w] = sm[qg][w][r] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(sm[qg][w][r] - M);
    L += sl[qg][w][r] * fw[w];
  }
  float* dst = part + (((size_t)kh * n_splits + split) * n_rows_pad + blockIdx.z * ROWS + 16 * qg + r) * PS;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    float4 v = make_float4(o[dt][0] * f0, o[dt][1] * f0, o[dt][2] * f0, o[dt][3] * f0);
#pragma unroll
    for (int w = 0; w < NKB - 1; ++w) {
      const float4 u = so[qg][w][r][4 * dt + g];
      v.x += u.x * fw[w]; v.y += u.y * fw[w]; v.z += u.z * fw[w]; v.w += u.w * fw[w];
    }
    *(float4*)(dst + 16 * dt + 4 * g) = v;
  }
  if (g == 0) *(float4*)(dst + HD) = make_float4(M * kLn2, L, 0.f, 0.f);  // natural units for the combine
}

// Workgroup = (kv head, key split of 32 NKB keys, 32 query rows) of NKB
// waves; wave w takes the 32-key block w of the split for BOTH 16-row groups,
// so each K and V fragment is loaded once and feeds both groups' MFMAs (k_fa
// reads them once per row group). The NKB key blocks then merge in LDS, every
// wave finishing some of the 32 rows, and the split's (O, m, l) rows go to the
// partial buffer in the layout k_fa writes (k_fa_combine reads either).
template <int HD, int NKB, bool DMASK>
__global__ __launch_bounds__(64 * NKB) void k_fa2(const float* __restrict__ q, const uint16_t* __restrict__ kc,
                                                  const uint16_t* __restrict__ vc, uint32_t max_seq, uint32_t n_head,
                                                  uint32_t N, uint32_t gqa, FaArgs fa, float scale,
                                                  float* __restrict__ part) {
  constexpr int NC = HD / 32, DT = HD / 16, ROWS = 32;
  constexpr uint32_t SPLIT_KEYS = 32 * NKB, PS = sh_fa_part_stride(HD);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4, r = lane & 15;
  const uint32_t kh = blockIdx.x, split = blockIdx.y;
  const uint32_t n_splits = gridDim.y;
  const uint32_t kbase0 = fa.dbase ? *fa.dbase : 0u;
  const uint32_t kvlen = fa.kvlen + kbase0, mbase = fa.mask_base + kbase0;
  if (fa.dbase && split * SPLIT_KEYS >= kvlen) return;  // uniform: past the live keys
  const uint32_t n_rows = gqa * N;
  const uint32_t n_rows_pad = gridDim.z * ROWS;
  const uint32_t Dq = n_head * HD;
  const uint32_t k_end = min((split + 1) * SPLIT_KEYS, kvlen);
  const uint32_t key0 = split * SPLIT_KEYS + 32 * wave;
  const uint32_t key0c = min(key0, max_seq - 32);  // blocks past the split's end read in bounds, masked below
  const uint16_t* kbase = kc + (size_t)kh * max_seq * HD;
  const uint16_t* vbase = vc + (size_t)kh * (max_seq / 32) * HD * 32;

  // The workgroup's 32 query rows go to LDS once (one direct global->LDS
  // load of HD floats per row, rows padded to HD + 4 floats), not to every
  // wave; then K and V of the wave's block, all before any wait, so the block
  // costs one memory latency.
  __shared__ __align__(16) float sq[ROWS][HD + 4];
  for (int i = wave; i < ROWS; i += NKB) {
    const uint32_t rho = blockIdx.z * ROWS + i;
    const uint32_t rr = rho < n_rows ? rho : 0;  // rows past the end read row 0 and are zeroed below
    const float* src = q + (size_t)(rr % N) * Dq + (size_t)(kh * gqa + rr / N) * HD + 4 * lane;
    if (lane < HD / 4) sh_dma16(src, &sq[i][0]);
  }
  uint32_t col[2];
  bool ok[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t rho = blockIdx.z * ROWS + 16 * h + r;
    ok[h] = rho < n_rows;
    col[h] = ok[h] ? rho % N : 0;
  }
  h8 kop[2][NC], vop[DT];
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int c = 0; c < NC; ++c) kop[kt][c] = ld_h8(kbase + (size_t)(key0c + 16 * kt + r) * HD + 8 * g + 32 * c);
  {
    const uint16_t* vp = vbase + (size_t)(key0c / 32) * HD * 32 + (size_t)r * 32 + 8 * g;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) vop[dt] = ld_h8(vp + (size_t)dt * 16 * 32);
  }
  uint64_t cm[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) cm[h] = DMASK ? fa.masks[col[h]] : col_mask(fa, col[h]);
  // The query rows (direct LDS loads, which the compiler does not track) were
  // issued before this wave's 2 NC + DT K and V loads (and any mask loads),
  // and loads return in order: with at most 2 NC + DT loads in flight the
  // query rows have landed, while K and V may still be arriving during the
  // query preparation below (the compiler waits for them before their first
  // uses). The barriers until then wait for LDS only; __syncthreads would
  // drain the K and V loads too.
  sh_wait_vm<2 * NC + DT>();
  lds_barrier();

  __shared__ float sm[NKB][ROWS], sl[NKB][ROWS];
  __shared__ float4 so[NKB][ROWS][HD / 4 + 1];
  // Q^T operands, prepared once per workgroup (the waves all use the same 32
  // rows): fragment (h, c) = rows 16 h + r, d = 8 g + 32 c .. + 7 of lane
  // (g, r), each row scaled by a power of two (max|q s| in [2^9, 2^10)) so the
  // f16 low halves stay normal, split hi + lo. Wave w prepares fragments w,
  // w + NKB, ...; partial row maxima and the row factors pass through the
  // merge buffer, the fragments through the query rows' own LDS.
  constexpr int NF = 2 * NC, FPW = (NF + NKB - 1) / NKB;
  float* smx = (float*)&so[0][0][0];  // [NF][64] row maxima of each fragment's 8 d
  float* srs = smx + NF * 64;         // [2][16] row factors
  h8* fq = (h8*)&sq[0][0];            // [NF][hi, lo][64]
  float xq[FPW][8];
#pragma unroll
  for (int i = 0; i < FPW; ++i) {
    const int f = wave + NKB * i;
    if (f < NF) {
      const int h = f / NC, c = f % NC;
      const float z = ok[h] ? 1.0f : 0.0f;
      const float* qs = &sq[16 * h + r][8 * g + 32 * c];
      const float4 a = *(const float4*)qs, b = *(const float4*)(qs + 4);
      xq[i][0] = a.x * z; xq[i][1] = a.y * z; xq[i][2] = a.z * z; xq[i][3] = a.w * z;
      xq[i][4] = b.x * z; xq[i][5] = b.y * z; xq[i][6] = b.z * z; xq[i][7] = b.w * z;
      float mx = 0.f;
#pragma unroll
      for (int t = 0; t < 8; ++t) mx = fmaxf(mx, fabsf(xq[i][t]));
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      smx[f * 64 + lane] = mx;
    }
  }
  lds_barrier();  // partial maxima written; every wave is done reading its f32 rows
#pragma unroll
  for (int i = 0; i < FPW; ++i) {
    const int f = wave + NKB * i;
    if (f < NF) {
      const int h = f / NC, c = f % NC;
      float mx = 0.f;
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) mx = fmaxf(mx, smx[(h * NC + cc) * 64 + lane]);
      int ex = 0;
      if (mx > 0.f && mx < INFINITY) {
        frexpf(mx, &ex);
        ex = ex < -100 ? -100 : (ex > 100 ? 100 : ex);
      }
      const float s = ldexpf(1.0f, 10 - ex);
      if (c == 0 && g == 0) srs[h * 16 + r] = scale * ldexpf(1.0f, ex - 10);
#pragma unroll
      for (int t = 0; t < 8; ++t) xq[i][t] *= s;
      h8 hi, lo;
      split8(xq[i], hi, lo);
      fq[(f * 2) * 64 + lane] = hi;
      fq[(f * 2 + 1) * 64 + lane] = lo;
    }
  }
  lds_barrier();
  h8 qhi2[2][NC], qlo2[2][NC];
  float rscale2[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      qhi2[h][c] = fq[((h * NC + c) * 2) * 64 + lane];
      qlo2[h][c] = fq[((h * NC + c) * 2 + 1) * 64 + lane];
    }
    rscale2[h] = srs[h * 16 + r];
  }
  lds_barrier();  // the merge buffer is free again

  const bool tail = key0 + 32 > k_end || key0 + 32 > mbase;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const h8* qhi = qhi2[h];
    const h8* qlo = qlo2[h];
    const float rscale = rscale2[h];
    // S^T[key][row] for keys key0 + 16 kt + 4 g + j
    f4 sacc[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        acc = mfma16a(kop[kt][c], qhi[c], acc);
        acc = mfma16a(kop[kt][c], qlo[c], acc);
      }
      sacc[kt] = acc;
    }
    float sv[8];
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float v = sacc[kt][j] * rscale;
        if (tail) {
          const uint32_t key = key0 + 16 * kt + 4 * g + j;
          bool vis = key < k_end;
          if (vis && key >= mbase) vis = (cm[h] >> (key - mbase)) & 1ull;
          if (!vis) v = -INFINITY;
        }
        sv[4 * kt + j] = v;
        mx = fmaxf(mx, v);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    // probabilities carry a 2^12 factor (keeps their f16 low halves normal);
    // it cancels in O / l because l is summed from the same scaled values
    const bool none = mx == -INFINITY;
    float p[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) p[t] = none ? 0.0f : __builtin_amdgcn_exp2f(sv[t] - mx) * 4096.0f;
    float ps = 0.f;
#pragma unroll
    for (int t = 0; t < 8; ++t) ps += p[t];
    ps += __shfl_xor(ps, 16);
    ps += __shfl_xor(ps, 32);
    h8 phi, plo;
    split8(p, phi, plo);
    const int row = 16 * h + r;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      f4 o = {0.f, 0.f, 0.f, 0.f};
      o = mfma16a(vop[dt], phi, o);
      o = mfma16a(vop[dt], plo, o);
      so[wave][row][4 * dt + g] = make_float4(o[0], o[1], o[2], o[3]);
    }
    if (g == 0) { sm[wave][row] = mx; sl[wave][row] = ps; }
  }
  __syncthreads();
  // Merge the key blocks in key-block order: a row's d are spread over HD / 8
  // lanes (8 each), RPW rows per wave and pass.
  constexpr int LPR = HD / 8, RPW = 64 / LPR;
  const int dq = 2 * (lane % LPR);
  for (int row = RPW * wave + lane / LPR; row < ROWS; row += RPW * NKB) {
    float M = -INFINITY;
#pragma unroll
    for (int b = 0; b < NKB; ++b) M = fmaxf(M, sm[b][row]);
    float L = 0.f;
    float4 o0 = make_float4(0.f, 0.f, 0.f, 0.f), o1 = o0;
#pragma unroll
    for (int b = 0; b < NKB; ++b) {
      const float mb = sm[b][row];
      const float f = mb == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mb - M);
      L += sl[b][row] * f;
      const float4 a = so[b][row][dq], c = so[b][row][dq + 1];
      o0.x += a.x * f; o0.y += a.y * f; o0.z += a.z * f; o0.w += a.w * f;
      o1.x += c.x * f; o1.y += c.y * f; o1.z += c.z * f; o1.w += c.w * f;
    }
    float* dst = part + (((size_t)kh * n_splits + split) * n_rows_pad + blockIdx.z * ROWS + row) * PS;
    *(float4*)(dst + 4 * dq) = o0;
    *(float4*)(dst + 4 * dq + 4) = o1;
    if (lane % LPR == 0) *(float4*)(dst + HD) = make_float4(M * kLn2, L, 0.f, 0.f);  // natural units
  }
}

// Combine the key splits (in split order) for one 256-wide superblock of the
// attention output of one column, write attn [N][Dq] f32 and that superblock of
// the Wo activation operand (columns col0 + j of the chunk). One wave per
// (superblock, column); lane l owns
// elements 256 sb + 4l .. +3. Splits are read CH at a time (every load issued
// before the first is used); each chunk takes one exp per split.
template <int HD>
__global__ __launch_bounds__(64) void k_fa_combine(const float* __restrict__ part, uint32_t n_layout,
                                                   uint32_t n_rows_pad, uint32_t n_head, uint32_t N, uint32_t gqa,
                                                   uint32_t col0, float* __restrict__ attn,
                                                   uint16_t* __restrict__ bx, uint16_t* __restrict__ xs,
                                                   float* __restrict__ cs, const uint32_t* dbase, uint32_t kv_off,
                                                   uint32_t split_keys) {
  // n_layout splits per kv head in the partial buffer; with dbase (graph
  // replay) only those holding live keys are read
  const uint32_t n_splits = dbase ? (*dbase + kv_off + split_keys - 1) / split_keys : n_layout;
  const uint32_t sb = blockIdx.x, col = blockIdx.y, lane = threadIdx.x;
  const uint32_t Dq = n_head * HD, k = 256 * sb + 4 * lane;
  const float4 v = sh_fa_combine4<2>(part, n_layout, n_splits, n_rows_pad, HD, n_head, gqa, N, sb, col);
  if (k < Dq) *(float4*)(attn + (size_t)(col0 + col) * Dq + k) = v;
  sh_operand_store_sb(v, Dq, sb, col0 + col, bx, xs, cs);
}

// Keys per split: SH_FA_SPLIT=128|256 overrides; by default 256 while that
// still gives >= 128 workgroups of 8 waves (4 waves per CU), else 128.
static uint32_t fa_split_keys(uint32_t n_kv, uint32_t kvlen, uint32_t n_qg) {
  static const uint32_t forced = [] {
    const char* s = getenv("SH_FA_SPLIT");
    const uint32_t v = s ? (uint32_t)atoi(s) : 0u;
    return (v == 128 || v == 256) ? v : 0u;
  }();
  if (forced) return forced;
  return (size_t)n_kv * n_qg * ((kvlen + 255) / 256) >= 128 ? 256 : 128;
}

// Two row groups take k_fa2 (SH_FA=1: k_fa).
static bool fa2_enabled() {
  static const bool v = [] {
    const char* s = getenv("SH_FA");
    return !(s && std::string(s) == "1");
  }();
  return v;
}

template <int HD, int NQG>
static void fa_launch_cfg(uint32_t split_keys, dim3 grid, hipStream_t st, const float* q, const uint16_t* kc,
                          const uint16_t* vc, uint32_t max_seq, uint32_t n_head, uint32_t N, uint32_t gqa,
                          const FaArgs& fa, float scale, float* part) {
  if (NQG == 2 && fa2_enabled()) {
    if (split_keys == 256) {
      if (fa.masks)
        hipLaunchKernelGGL((k_fa2<HD, 8, true>), grid, dim3(512), 0, st, q, kc, vc, max_seq, n_head, N, gqa, fa,
                           scale, part);
      else
        hipLaunchKernelGGL((k_fa2<HD, 8, false>), grid, dim3(512), 0, st, q, kc, vc, max_seq, n_head, N, gqa, fa,
                           scale, part);
    } else {
      if (fa.masks)
        hipLaunchKernelGGL((k_fa2<HD, 4, true>), grid, dim3(256), 0, st, q, kc, vc, max_seq, n_head, N, gqa, fa,
                           scale, part);
      else
        hipLaunchKernelGGL((k_fa2<HD, 4, false>), grid, dim3(256), 0, st, q, kc, vc, max_seq, n_head, N, gqa, fa,
                           scale, part);
    }
    return;
  }
  constexpr int NKB = 4;
  const dim3 block(64 * NQG * NKB);
  if (fa.masks) {  // columns beyond 8: masks from device memory
    if (split_keys == 256)
      hipLaunchKernelGGL((k_fa<HD, NQG, NKB, 2, true>), grid, block, 0, st, q, kc, vc, max_seq, n_head, N, gqa, fa,
                         scale, part);
    else
      hipLaunchKernelGGL((k_fa<HD, NQG, NKB, 1, true>), grid, block, 0, st, q, kc, vc, max_seq, n_head, N, gqa, fa,
                         scale, part);
  } else if (split_keys == 256) {
    hipLaunchKernelGGL((k_fa<HD, NQG, NKB, 2, false>), grid, block, 0, st, q, kc, vc, max_seq, n_head, N, gqa, fa,
                       scale, part);
  } else {
    hipLaunchKernelGGL((k_fa<HD, NQG, NKB, 1, false>), grid, block, 0, st, q, kc, vc, max_seq, n_head, N, gqa, fa,
                       scale, part);
  }
}

int sh_fa_launch(sh_engine* e, const sh_model* m, const sh_kv* kv, const FaArgs& fa, const float* q, float* part,
                 float* attn_out, uint16_t* bx, uint16_t* xs, float* cs, OpndSrc* combine_out) {
  const uint32_t gqa = m->n_head / m->n_kv;
  const uint32_t n_rows = gqa * fa.N;
  const int NQG = n_rows > 16 ? 2 : 1;
  const uint32_t n_qg = (n_rows + 16 * NQG - 1) / (16 * NQG);
  SH_CHECK(n_qg * 16 * NQG <= (uint32_t)SH_FA_MAX_ROWS, SH_ERR_UNSUPPORTED, "%u query rows per kv head above %d",
           n_rows, SH_FA_MAX_ROWS);
  SH_CHECK(fa.kvlen > 0 || fa.dbase, SH_ERR_ARG, "attention over zero keys");
  SH_CHECK(!fa.dbase || fa.kv_cap >= fa.kvlen, SH_ERR_ARG, "attention: graph key capacity below the offset");
  // graph replay: the split size and grid follow the capacity, not the live keys
  const uint32_t kv_grid = fa.dbase ? fa.kv_cap : fa.kvlen;
  const uint32_t split_keys = fa_split_keys(m->n_kv, kv_grid, n_qg);
  const uint32_t n_splits = (kv_grid + split_keys - 1) / split_keys;
  const uint32_t rows_pad = n_qg * 16 * NQG;
  const size_t need = (size_t)m->n_kv * n_splits * rows_pad * sh_fa_part_stride(m->hd);
  SH_CHECK(need <= m->ws.fa_part_floats, SH_ERR_CAPACITY, "attention partial buffer too small (%zu > %zu)", need,
           m->ws.fa_part_floats);
  SH_CHECK(kv->max_seq % 32 == 0 && kv->max_seq >= 32, SH_ERR_ARG, "kv max_seq must be a positive multiple of 32");
  const size_t layer_k = (size_t)m->n_kv * kv->max_seq * m->hd;
  const uint16_t* kc = kv->k + layer_k * fa.layer;
  const uint16_t* vc = kv->v + layer_k * fa.layer;
  SH_CHECK(fa.N >= 1 && (fa.N <= 8 || fa.masks) && fa.col0 + fa.N <= SH_MAX_COLS, SH_ERR_ARG,
           "attention columns [%u, %u) outside the chunk (more than 8 need device masks)", fa.col0, fa.col0 + fa.N);
  const float scale = kLog2e / sqrtf((float)m->hd);  // scores in base 2
  q += (size_t)fa.col0 * m->n_head * m->hd;
  hipEvent_t ev = nullptr;
  sh_prof_begin(e, &ev);
  const dim3 grid(m->n_kv, n_splits, n_qg);
  if (m->hd == 128) {
    if (NQG == 2) fa_launch_cfg<128, 2>(split_keys, grid, e->stream, q, kc, vc, kv->max_seq, m->n_head, fa.N, gqa, fa, scale, part);
    else fa_launch_cfg<128, 1>(split_keys, grid, e->stream, q, kc, vc, kv->max_seq, m->n_head, fa.N, gqa, fa, scale, part);
  } else if (m->hd == 64) {
    if (NQG == 2) fa_launch_cfg<64, 2>(split_keys, grid, e->stream, q, kc, vc, kv->max_seq, m->n_head, fa.N, gqa, fa, scale, part);
    else fa_launch_cfg<64, 1>(split_keys, grid, e->stream, q, kc, vc, kv->max_seq, m->n_head, fa.N, gqa, fa, scale, part);
  } else {
    SH_CHECK(false, SH_ERR_UNSUPPORTED, "head_dim %u not supported (64, 128)", m->hd);
  }
  SH_HIP(hipGetLastError());
  const double kv_bytes = 2.0 * m->n_kv * (double)kv_grid * m->hd * 2.0;
  sh_prof_end(e, "attention", kv_bytes, ev);
  if (combine_out) {
    SH_CHECK(fa.col0 == 0, SH_ERR_ARG, "attention: a deferred combine needs the chunk's first column");
    OpndSrc& o = *combine_out;
    o.kind = OPND_FA; o.fa_part = part; o.n_layout = n_splits; o.rows_pad = rows_pad; o.n_head = m->n_head;
    o.gqa = gqa; o.hd = m->hd; o.split_keys = split_keys; o.kv_off = fa.kvlen; o.dbase = fa.dbase;
    return SH_OK;
  }
  sh_prof_begin(e, &ev);
  const dim3 cgrid((m->n_head * m->hd + 255) / 256, fa.N);
  if (m->hd == 128)
    hipLaunchKernelGGL((k_fa_combine<128>), cgrid, dim3(64), 0, e->stream, part, n_splits, rows_pad, m->n_head, fa.N,
                       gqa, fa.col0, attn_out, bx, xs, cs, fa.dbase, fa.kvlen, split_keys);
  else
    hipLaunchKernelGGL((k_fa_combine<64>), cgrid, dim3(64), 0, e->stream, part, n_splits, rows_pad, m->n_head, fa.N,
                       gqa, fa.col0, attn_out, bx, xs, cs, fa.dbase, fa.kvlen, split_keys);
  SH_HIP(hipGetLastError());
  sh_prof_end(e, "attn_combine", 0.0, ev);
  return SH_OK;
}

// ---------------------------------------------------------------- KV moves

__device__ __forceinline__ uint32_t v_slot_a(uint32_t kappa) {
  return 8u * ((kappa & 15u) >> 2) + 4u * (kappa >> 4) + (kappa & 3u);
}

// Gather rows: dst slot base+i <- src slot base+src[i], every layer / kv head,
// through a staging buffer so overlapping moves are order-independent.
__global__ void k_kv_gather(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, uint16_t* stage,
                            uint32_t max_seq, uint32_t hd, uint32_t base, const uint32_t* src, uint32_t n) {
  const uint32_t lh = blockIdx.x, i = blockIdx.y, d = threadIdx.x;  // lh = layer * n_kv + head
  const uint32_t s = base + src[i];
  const uint16_t* kh = k + (size_t)lh * max_seq * hd;
  const uint16_t* vh = v + (size_t)lh * max_seq * hd;
  uint16_t* st = stage + ((size_t)lh * n + i) * hd * 2;
  st[d] = kh[(size_t)s * hd + d];
  st[hd + d] = vh[((size_t)(s / 32) * hd + d) * 32 + v_slot_a(s & 31)];
}
__global__ void k_kv_scatter(uint16_t* __restrict__ k, uint16_t* __restrict__ v, const uint16_t* stage,
                             uint32_t max_seq, uint32_t hd, uint32_t base, uint32_t n) {
  const uint32_t lh = blockIdx.x, i = blockIdx.y, d = threadIdx.x;
  const uint32_t s = base + i;
  uint16_t* kh = k + (size_t)lh * max_seq * hd;
  uint16_t* vh = v + (size_t)lh * max_seq * hd;
  const uint16_t* st = stage + ((size_t)lh * n + i) * hd * 2;
  kh[(size_t)s * hd + d] = st[d];
  vh[((size_t)(s / 32) * hd + d) * 32 + v_slot_a(s & 31)] = st[hd + d];
}

int sh_kv_compact_launch(sh_engine* e, sh_kv* kv, uint32_t base, const uint32_t* src_dev, uint32_t n) {
  const uint32_t lh = kv->n_layer * kv->n_kv;
  uint16_t* stage = nullptr;
  SH_HIP(hipMallocAsync((void**)&stage, (size_t)lh * n * kv->hd * 2 * 2, e->stream));
  hipLaunchKernelGGL(k_kv_gather, dim3(lh, n), dim3(kv->hd), 0, e->stream, kv->k, kv->v, stage, kv->max_seq, kv->hd,
                     base, src_dev, n);
  hipLaunchKernelGGL(k_kv_scatter, dim3(lh, n), dim3(kv->hd), 0, e->stream, kv->k, kv->v, stage, kv->max_seq,
                     kv->hd, base, n);
  SH_HIP(hipGetLastError());
  SH_HIP(hipFreeAsync(stage, e->stream));
  return SH_OK;
}
