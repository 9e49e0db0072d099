// Verify-step attention over the f16 KV cache.
//
// Semantics: shaders/compute/flash_attn.slang (online softmax of q.K^T * hd^-1/2
// over keys [0, kvlen); keys below the chunk base are always visible,
// mask_kv_offset :126-129; within-chunk keys follow the [L x L] causal mask of
// models/llama.rs:904-955) and the split-K combine of
// flash_attn_split_k_reduce.slang. Tree verify replaces the causal triangle by
// an ancestor-or-self bitmask per query column (new).
//
// Design (gfx950): one workgroup = (kv head, 256-key split, group of 16*QT
// query rows); its 4 waves take 64 keys each and issue all their K and V loads
// up front. The GQA rows of one kv head (gqa heads x N columns) share every K/V
// tile, so K and V are read once per kv head. S^T = K Q^T and O^T = V^T P^T run
// on v_mfma_f32_16x16x32_f16; Q and P are split into hi + lo f16 halves so the
// products keep ~22 bits (K and V are exact f16). V is stored per 32-key block
// transposed ([hd][32 slots], slot order v_slot()) so the V^T operand is a
// contiguous 16-byte load. A second kernel combines the splits in split order
// (deterministic) per column and builds the Wo activation operand.
#include <cfloat>

#include "sh_internal.h"
#include "sh_operand.h"

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
struct alignas(16) u32x4a { uint32_t x, y, z, w; };

__device__ __forceinline__ h8 ld_h8(const uint16_t* p) { return __builtin_bit_cast(h8, *(const u32x4a*)p); }
__device__ __forceinline__ f4 mfma16a(h8 a, h8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Split 8 f32 into hi and lo f16 vectors.
__device__ __forceinline__ void split8(const float* x, h8& hi, h8& lo) {
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    _Float16 h = (_Float16)x[t];
    hi[t] = h;
    lo[t] = (_Float16)(x[t] - (float)h);
  }
}

constexpr uint32_t FA_WAVE_KEYS = 64;
constexpr uint32_t FA_SPLIT_KEYS = 4 * FA_WAVE_KEYS;
static_assert(FA_SPLIT_KEYS == SH_FA_KEYS_PER_SPLIT, "split size");

template <int QT, int HD>
__global__ __launch_bounds__(256) void k_fa(const float* __restrict__ q, const uint16_t* __restrict__ kc,
                                            const uint16_t* __restrict__ vc, uint32_t max_seq, uint32_t n_head,
                                            uint32_t N, uint32_t gqa, FaArgs fa, float scale,
                                            float* __restrict__ part) {
  constexpr int NC = HD / 32;  // d chunks of the QK contraction
  constexpr int DT = HD / 16;  // d tiles of the output
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const uint32_t kh = blockIdx.x, split = blockIdx.y, qg = blockIdx.z;
  const uint32_t n_splits = gridDim.y;
  const uint32_t n_rows = gqa * N;
  const uint32_t n_rows_pad = gridDim.z * 16 * QT;
  const uint32_t Dq = n_head * HD;
  const uint16_t* kbase = kc + (size_t)kh * max_seq * HD;
  const uint16_t* vbase = vc + (size_t)kh * (max_seq / 32) * HD * 32;

  // Issue this wave's K and V loads for its (up to) two 32-key halves first.
  const uint32_t k_end = min((split + 1) * FA_SPLIT_KEYS, fa.kvlen);
  const uint32_t kw = split * FA_SPLIT_KEYS + FA_WAVE_KEYS * wave;
  const bool hv0 = kw < k_end, hv1 = kw + 32 < k_end;
  h8 kop[2][2][NC], vop[2][DT];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    if (h == 0 ? !hv0 : !hv1) continue;
    const uint32_t key0 = kw + 32 * h;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int c = 0; c < NC; ++c) kop[h][kt][c] = ld_h8(kbase + (size_t)(key0 + 16 * kt + r) * HD + 8 * g + 32 * c);
    const uint16_t* vp = vbase + (size_t)(key0 / 32) * HD * 32 + (size_t)r * 32 + 8 * g;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) vop[h][dt] = ld_h8(vp + (size_t)dt * 16 * 32);
  }

  // Q^T operands (B): lane (g, r) holds rho = 16*qt + r, d = 32c + 8g .. +8.
  // Each query row is scaled by a power of two (max|q * s| in [2^9, 2^10)) so
  // the f16 low halves stay normal; rscale folds 1/s into the score scale.
  h8 qhi[QT][NC], qlo[QT][NC];
  uint32_t rowcol[QT];
  float rscale[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const uint32_t rho = qg * 16 * QT + 16 * qt + r;
    const bool ok = rho < n_rows;
    const uint32_t hq = ok ? rho / N : 0, col = ok ? rho % N : 0;
    rowcol[qt] = col;
    const float* qp = q + (size_t)col * Dq + (size_t)(kh * gqa + hq) * HD;
    float x[NC][8];
    float mx = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const float4 a = ok ? *(const float4*)(qp + 32 * c + 8 * g) : make_float4(0.f, 0.f, 0.f, 0.f);
      const float4 b = ok ? *(const float4*)(qp + 32 * c + 8 * g + 4) : make_float4(0.f, 0.f, 0.f, 0.f);
      x[c][0] = a.x; x[c][1] = a.y; x[c][2] = a.z; x[c][3] = a.w;
      x[c][4] = b.x; x[c][5] = b.y; x[c][6] = b.z; x[c][7] = b.w;
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
    rscale[qt] = scale * ldexpf(1.0f, ex - 10);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
#pragma unroll
      for (int t = 0; t < 8; ++t) x[c][t] *= s;
      split8(x[c], qhi[qt][c], qlo[qt][c]);
    }
  }

  f4 o[DT][QT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) o[dt][qt] = f4{0.f, 0.f, 0.f, 0.f};
  float mrow[QT], lrow[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) { mrow[qt] = -INFINITY; lrow[qt] = 0.f; }

#pragma unroll
  for (int h = 0; h < 2; ++h) {
    if (h == 0 ? !hv0 : !hv1) continue;
    const uint32_t key0 = kw + 32 * h;
    // S^T[key][rho] for keys key0 + 16*kt + 4g + j.
    f4 s[2][QT];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          acc = mfma16a(kop[h][kt][c], qhi[qt][c], acc);
          acc = mfma16a(kop[h][kt][c], qlo[qt][c], acc);
        }
        s[kt][qt] = acc;
      }
    const bool tail = key0 + 32 > fa.kvlen || key0 + 32 > fa.mask_base;
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const uint64_t cm = fa.colmask[rowcol[qt] & 7];
      float sv[8];
      float mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float v = s[kt][qt][j] * rscale[qt];
          if (tail) {
            const uint32_t key = key0 + 16 * kt + 4 * g + j;
            bool vis = key < fa.kvlen;
            if (vis && key >= fa.mask_base) vis = (cm >> (key - fa.mask_base)) & 1ull;
            if (!vis) v = -INFINITY;
          }
          sv[4 * kt + j] = v;
          mx = fmaxf(mx, v);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float mnew = fmaxf(mrow[qt], mx);
      float alpha, p[8];
      if (mnew == -INFINITY) {
        alpha = 1.f;
#pragma unroll
        for (int t = 0; t < 8; ++t) p[t] = 0.f;
      } else {
        alpha = expf(mrow[qt] - mnew);
        // probabilities carry a 2^12 factor (keeps their f16 low halves normal);
        // it cancels in O / l because l is summed from the same scaled values
#pragma unroll
        for (int t = 0; t < 8; ++t) p[t] = expf(sv[t] - mnew) * 4096.0f;
      }
      mrow[qt] = mnew;
      float ps = 0.f;
#pragma unroll
      for (int t = 0; t < 8; ++t) ps += p[t];
      lrow[qt] = lrow[qt] * alpha + ps;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) o[dt][qt] *= alpha;
      // P^T operand: lane slot t -> key 4g+t (t<4) or 16+4g+t-4 (t>=4), the order
      // V blocks are stored in.
      h8 phi, plo;
      split8(p, phi, plo);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        o[dt][qt] = mfma16a(vop[h][dt], phi, o[dt][qt]);
        o[dt][qt] = mfma16a(vop[h][dt], plo, o[dt][qt]);
      }
    }
  }
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    lrow[qt] += __shfl_xor(lrow[qt], 16);
    lrow[qt] += __shfl_xor(lrow[qt], 32);
  }

  // Merge the 4 waves through LDS, then write this split's partial:
  // part[((kh * n_splits + split) * n_rows_pad + rho) * (HD + 2) + {d, HD: m, HD+1: l}].
  __shared__ float sm[4][QT * 16], sl[4][QT * 16];
  __shared__ float so[QT * 16][HD + 1];
  if (g == 0) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) { sm[wave][16 * qt + r] = mrow[qt]; sl[wave][16 * qt + r] = lrow[qt]; }
  }
  __syncthreads();
  for (int w = 0; w < 4; ++w) {
    if (wave == w) {
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        const int rho_l = 16 * qt + r;
        float M = sm[0][rho_l];
        for (int v = 1; v < 4; ++v) M = fmaxf(M, sm[v][rho_l]);
        const float f = (mrow[qt] == -INFINITY) ? 0.f : expf(mrow[qt] - M);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            float* dst = &so[rho_l][16 * dt + 4 * g + j];
            *dst = (w == 0 ? 0.f : *dst) + o[dt][qt][j] * f;
          }
      }
    }
    __syncthreads();
  }
  for (int idx = threadIdx.x; idx < QT * 16 * (HD + 2); idx += 256) {
    const int rho_l = idx / (HD + 2), e = idx % (HD + 2);
    float M = sm[0][rho_l];
    for (int w = 1; w < 4; ++w) M = fmaxf(M, sm[w][rho_l]);
    float v;
    if (e < HD) {
      v = so[rho_l][e];
    } else if (e == HD) {
      v = M;
    } else {
      v = 0.f;
      for (int w = 0; w < 4; ++w) v += sm[w][rho_l] == -INFINITY ? 0.f : sl[w][rho_l] * expf(sm[w][rho_l] - M);
    }
    const uint32_t rho = qg * 16 * QT + rho_l;
    part[(((size_t)kh * n_splits + split) * n_rows_pad + rho) * (HD + 2) + e] = v;
  }

}

// Combine the key splits for every head of one column (in split order), write
// attn [N][Dq] f32 and build the Wo activation operand from it. One workgroup
// of 1024 threads per column; thread t owns outputs 4t..4t+3 (+4096 i).
template <int HD, int NV>
__global__ __launch_bounds__(SH_OPERAND_THREADS) void k_fa_combine(const float* __restrict__ part, uint32_t n_splits,
                                                                   uint32_t n_rows_pad, uint32_t n_head, uint32_t N,
                                                                   uint32_t gqa, float* __restrict__ attn,
                                                                   uint16_t* __restrict__ bx,
                                                                   uint16_t* __restrict__ xs, float* __restrict__ cs) {
  __shared__ float red_m[SH_OPERAND_THREADS / 64];
  const uint32_t col = blockIdx.x, tid = threadIdx.x;
  const uint32_t Dq = n_head * HD, n4 = Dq / 4;
  const size_t sstride = (size_t)n_rows_pad * (HD + 2);
  float4 v[NV];
  float mx = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    v[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    const uint32_t q = tid + SH_OPERAND_THREADS * i;
    if (q >= n4) continue;
    const uint32_t k = 4 * q, head = k / HD, d = k % HD;
    const uint32_t kh = head / gqa, rho = (head % gqa) * N + col;
    const float* p = part + (size_t)kh * n_splits * sstride + (size_t)rho * (HD + 2);
    float M = -INFINITY, L = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (uint32_t s = 0; s < n_splits; ++s, p += sstride) {
      const float ms = p[HD];
      if (ms == -INFINITY) continue;
      const float mn = fmaxf(M, ms);
      const float a = expf(M - mn), b = expf(ms - mn);  // M = -inf on the first split: a = 0
      const float4 o = *(const float4*)(p + d);
      acc.x = acc.x * a + o.x * b;
      acc.y = acc.y * a + o.y * b;
      acc.z = acc.z * a + o.z * b;
      acc.w = acc.w * a + o.w * b;
      L = L * a + p[HD + 1] * b;
      M = mn;
    }
    const float il = L > 0.f ? 1.0f / L : 0.f;
    v[i] = make_float4(acc.x * il, acc.y * il, acc.z * il, acc.w * il);
    *(float4*)(attn + (size_t)col * Dq + k) = v[i];
    mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
  }
  mx = sh_wave_max(mx);
  if ((tid & 63) == 0) red_m[tid >> 6] = mx;
  __syncthreads();
  mx = 0.f;
#pragma unroll
  for (int i = 0; i < SH_OPERAND_THREADS / 64; ++i) mx = fmaxf(mx, red_m[i]);
  sh_operand_store<NV>(v, Dq, col, 1.0f, mx, bx, xs, cs);
}

int sh_fa_launch(sh_engine* e, const sh_model* m, const sh_kv* kv, const FaArgs& fa, const float* q, float* part,
                 float* attn_out, uint16_t* bx, uint16_t* xs, float* cs) {
  const uint32_t gqa = m->n_head / m->n_kv;
  const uint32_t n_rows = gqa * fa.N;
  const int QT = n_rows > 16 ? 2 : 1;
  const uint32_t n_qg = (n_rows + 16 * QT - 1) / (16 * QT);
  const uint32_t n_splits = (fa.kvlen + FA_SPLIT_KEYS - 1) / FA_SPLIT_KEYS;
  const size_t need = (size_t)m->n_kv * n_splits * n_qg * 16 * QT * (m->hd + 2);
  SH_CHECK(need <= m->ws.fa_part_floats, SH_ERR_CAPACITY, "attention partial buffer too small (%zu > %zu)", need,
           m->ws.fa_part_floats);
  SH_CHECK(kv->max_seq % 32 == 0, SH_ERR_ARG, "kv max_seq must be a multiple of 32");
  SH_CHECK(m->d <= 4 * SH_OPERAND_THREADS * 2, SH_ERR_UNSUPPORTED, "n_embd %u above 8192", m->d);
  const size_t layer_k = (size_t)m->n_kv * kv->max_seq * m->hd;
  const uint16_t* kc = kv->k + layer_k * fa.layer;
  const uint16_t* vc = kv->v + layer_k * fa.layer;
  const float scale = 1.0f / sqrtf((float)m->hd);
  hipEvent_t ev = nullptr;
  sh_prof_begin(e, &ev);
  dim3 grid(m->n_kv, n_splits, n_qg);
#define FA_LAUNCH(QT_, HD_)                                                                                  \
  hipLaunchKernelGGL((k_fa<QT_, HD_>), grid, dim3(256), 0, e->stream, q, kc, vc, kv->max_seq, m->n_head, fa.N, \
                     gqa, fa, scale, part)
  if (m->hd == 128) {
    if (QT == 2) FA_LAUNCH(2, 128); else FA_LAUNCH(1, 128);
  } else if (m->hd == 64) {
    if (QT == 2) FA_LAUNCH(2, 64); else FA_LAUNCH(1, 64);
  } else {
    SH_CHECK(false, SH_ERR_UNSUPPORTED, "head_dim %u not supported (64, 128)", m->hd);
  }
#undef FA_LAUNCH
  SH_HIP(hipGetLastError());
  const double kv_bytes = 2.0 * m->n_kv * (double)fa.kvlen * m->hd * 2.0;
  sh_prof_end(e, "attention", kv_bytes, ev);
  sh_prof_begin(e, &ev);
  const uint32_t rows_pad = n_qg * 16 * QT;
  const bool two = m->d > 4 * SH_OPERAND_THREADS;
#define FC_LAUNCH(HD_, NV_)                                                                                    \
  hipLaunchKernelGGL((k_fa_combine<HD_, NV_>), dim3(fa.N), dim3(SH_OPERAND_THREADS), 0, e->stream, part, n_splits, \
                     rows_pad, m->n_head, fa.N, gqa, attn_out, bx, xs, cs)
  if (m->hd == 128) {
    if (two) FC_LAUNCH(128, 2); else FC_LAUNCH(128, 1);
  } else {
    if (two) FC_LAUNCH(64, 2); else FC_LAUNCH(64, 1);
  }
#undef FC_LAUNCH
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
