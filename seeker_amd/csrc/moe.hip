// Routed-expert (MoE) FFN of a qwen3moe layer: router + top-k, the routing
// plan that groups (column, expert) pairs by expert, and the weighted sum of
// the experts' outputs into the residual. The expert matrices themselves run
// on the expert-indirect K-quant GEMM (k_moe_gemm_kq in gemv.hip).
//
// Semantics follow the reference's MoE step (models/qwen35moe.rs:3117-3182,
// ops/moe.rs, topk_moe.slang): softmax gating over the experts, the n_used
// most probable kept with ties to the lower expert index, their weights
// renormalized to sum 1 (with_norm), silu(gate_e x) * up_e x through down_e,
// summed with those weights. The shared expert of qwen35moe is absent in
// qwen3moe.
#include <algorithm>

#include "sh_internal.h"

namespace {

constexpr uint32_t kMaxExperts = 1024;

// Orderable key: larger logit first, then the lower expert index; NaN loses.
__device__ __forceinline__ unsigned long long route_key(float v, uint32_t e) {
  if (v != v) return 0ull;
  uint32_t b = __builtin_bit_cast(uint32_t, v);
  b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((unsigned long long)b << 32) | (unsigned long long)(~e);
}
// The logit a (nonzero) key carries.
__device__ __forceinline__ float key_logit(unsigned long long key) {
  const uint32_t b = (uint32_t)(key >> 32);
  return __builtin_bit_cast(float, (b & 0x80000000u) ? (b & 0x7FFFFFFFu) : ~b);
}

// Router logits, one wave per (8 experts, CPW columns): logits[col][e] =
// rinv(col) * sum_i R[e][i] (x[col][i] norm_w[i]), rinv = 1 / sqrt(mean(x^2) +
// eps) (the RMSNorm factor is linear, so it is applied to the dot product).
// Lane l holds elements 4 l + 256 j (j < d / 256) of each of the wave's
// columns in registers; every router row is read as 16-byte loads and the
// sums reduce across the wave. The whole launch spreads the router over
// E / 8 x ceil(N / CPW) waves instead of one workgroup per column walking all
// E rows.
template <int NJ>
__global__ __launch_bounds__(64) void k_moe_logits(const float* __restrict__ x, const float* __restrict__ norm_w,
                                                   const float* __restrict__ R, uint32_t d, uint32_t E, uint32_t N,
                                                   float eps, float* __restrict__ logits) {
  constexpr int CPW = 32 / NJ, EPW = 8;
  const uint32_t lane = threadIdx.x, nj = d / 256;
  const uint32_t e0 = blockIdx.x * EPW, c0 = blockIdx.y * CPW;
  float4 xv[CPW][NJ];
  float rinv[CPW];
#pragma unroll
  for (int c = 0; c < CPW; ++c) {
    const uint32_t col = c0 + c < N ? c0 + c : N - 1;  // past the last column: a clamped (unused) read
    const float* xc = x + (size_t)col * d + 4 * lane;
#pragma unroll
    for (int j = 0; j < NJ; ++j) xv[c][j] = (uint32_t)j < nj ? *(const float4*)(xc + 256 * j) : float4{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int c = 0; c < CPW; ++c) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      ss = __builtin_fmaf(xv[c][j].x, xv[c][j].x, ss);
      ss = __builtin_fmaf(xv[c][j].y, xv[c][j].y, ss);
      ss = __builtin_fmaf(xv[c][j].z, xv[c][j].z, ss);
      ss = __builtin_fmaf(xv[c][j].w, xv[c][j].w, ss);
    }
    for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
    rinv[c] = 1.0f / sqrtf(ss / (float)d + eps);
  }
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    if ((uint32_t)j >= nj) break;
    const float4 w = *(const float4*)(norm_w + 4 * lane + 256 * j);
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
      xv[c][j].x *= w.x; xv[c][j].y *= w.y; xv[c][j].z *= w.z; xv[c][j].w *= w.w;
    }
  }
  // Experts in pairs, both pairs' rows in flight before the first sums.
#pragma unroll
  for (int ep = 0; ep < EPW; ep += 2) {
    float4 rv[2][NJ];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t e = min(e0 + ep + h, E - 1);  // past the last expert: a clamped (unused) read
      const float* r = R + (size_t)e * d + 4 * lane;
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        rv[h][j] = (uint32_t)j < nj ? *(const float4*)(r + 256 * j) : float4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int c = 0; c < CPW; ++c) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          acc = __builtin_fmaf(rv[h][j].x, xv[c][j].x, acc);
          acc = __builtin_fmaf(rv[h][j].y, xv[c][j].y, acc);
          acc = __builtin_fmaf(rv[h][j].z, xv[c][j].z, acc);
          acc = __builtin_fmaf(rv[h][j].w, xv[c][j].w, acc);
        }
        for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off);
        const uint32_t e = e0 + ep + h;
        if (lane == 0 && c0 + c < N && e < E) logits[(size_t)(c0 + c) * E + e] = acc * rinv[c];
      }
  }
}

// Top-k selection and routing plan in one workgroup of 512 threads for
// P = N k <= 512 (column, slot) pairs.
//  * Top-k: wave w takes columns w, w + 8, ...; lane l holds logits l, l + 64,
//    ...; k rounds pick the largest remaining logit (softmax is monotone, so
//    this is the top-k of the probabilities; ties to the lower expert index)
//    and the weights exp(l_j - l_max) / sum over the selection in f64 (the
//    full softmax denominator cancels in the renormalization).
//  * Plan: pair p = column * k + slot has expert ids[p]. Pairs are sorted by
//    expert, within an expert by p: a bitmap of pairs per expert gives each
//    pair's rank by population counts, a wave scan over the experts their
//    offsets. Sorted position s of pair p is slot_of[p] and its input column
//    pair_col[s]. Each expert's run of pairs is cut into chunks of at most 8:
//    info[0] = number of chunks, info[1 + 3c .. +3] = (expert, first sorted
//    pair, count), chunks in expert order.
template <int RL>
__global__ __launch_bounds__(512) void k_moe_plan(const float* __restrict__ logits, uint32_t N, uint32_t E,
                                                  uint32_t k, uint32_t* __restrict__ ids, float* __restrict__ wts,
                                                  uint32_t* __restrict__ info, uint32_t* __restrict__ pair_col,
                                                  uint32_t* __restrict__ slot_of) {
  constexpr uint32_t NW = 16;  // bitmap words per expert: P <= 512
  __shared__ uint32_t sid[512];
  __shared__ uint32_t bm[kMaxExperts * NW];
  __shared__ uint32_t cnt[kMaxExperts], off[kMaxExperts], cbase[kMaxExperts];
  const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const uint32_t P = N * k, nw = (P + 31) / 32;
  for (uint32_t i = t; i < E * NW; i += 512) bm[i] = 0u;
  for (uint32_t col = wave; col < N; col += 8) {
    const float* lg = logits + (size_t)col * E;
    float lv[RL];
#pragma unroll
    for (uint32_t r = 0; r < RL; ++r) lv[r] = lane + 64 * r < E ? lg[lane + 64 * r] : -INFINITY;
    float lmax = 0.f;
    double wsel = 0.0, wsum = 0.0;  // lane j keeps selection j's weight
    for (uint32_t j = 0; j < k; ++j) {
      unsigned long long best = 0ull;
#pragma unroll
      for (uint32_t r = 0; r < RL; ++r)
        if (lane + 64 * r < E) {
          const unsigned long long key = lv[r] == -INFINITY ? 0ull : route_key(lv[r], lane + 64 * r);
          best = key > best ? key : best;
        }
      for (int o = 32; o >= 1; o >>= 1) {
        const unsigned long long ob = __shfl_xor(best, o);
        best = ob > best ? ob : best;
      }
      const uint32_t e = best ? ~(uint32_t)(best & 0xFFFFFFFFull) : 0u;
      const float l = best ? key_logit(best) : lg[e];  // no key: every logit NaN or -inf (expert 0)
      if (j == 0) lmax = l;
#pragma unroll
      for (uint32_t r = 0; r < RL; ++r)
        if (lane + 64 * r == e) lv[r] = -INFINITY;
      const double w = exp((double)l - (double)lmax);
      wsum += w;
      if (lane == j) wsel = w;
      if (lane == 0) {
        ids[(size_t)col * k + j] = e;
        sid[col * k + j] = min(e, E - 1);
      }
    }
    if (lane < k) wts[(size_t)col * k + lane] = (float)(wsel / wsum);
  }
  __syncthreads();
  if (t < P) atomicOr(&bm[sid[t] * NW + (t >> 5)], 1u << (t & 31));
  __syncthreads();
  for (uint32_t x = t; x < E; x += 512) {
    uint32_t n = 0;
    for (uint32_t w = 0; w < nw; ++w) n += __popc(bm[x * NW + w]);
    cnt[x] = n;
  }
  __syncthreads();
  if (wave == 0) {  // exclusive scans of the counts and chunk counts over the experts, E / 64 per lane
    const uint32_t per = (E + 63) / 64, x0 = lane * per;
    uint32_t so = 0, sc = 0;
    for (uint32_t i = 0; i < per; ++i)
      if (x0 + i < E) { so += cnt[x0 + i]; sc += (cnt[x0 + i] + 7) / 8; }
    uint32_t io = so, ic = sc;  // inclusive wave scans
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t ao = __shfl_up(io, o), ac = __shfl_up(ic, o);
      if (lane >= (uint32_t)o) { io += ao; ic += ac; }
    }
    uint32_t o = io - so, c = ic - sc;
    for (uint32_t i = 0; i < per; ++i)
      if (x0 + i < E) {
        off[x0 + i] = o;
        cbase[x0 + i] = c;
        o += cnt[x0 + i];
        c += (cnt[x0 + i] + 7) / 8;
      }
    if (lane == 63) info[0] = ic;
  }
  __syncthreads();
  if (t < P) {
    const uint32_t e = sid[t], wi = t >> 5;
    uint32_t rank = __popc(bm[e * NW + wi] & ((1u << (t & 31)) - 1u));
    for (uint32_t w = 0; w < wi; ++w) rank += __popc(bm[e * NW + w]);
    const uint32_t s = off[e] + rank;
    pair_col[s] = t / k;
    slot_of[t] = s;
  }
  for (uint32_t x = t; x < E; x += 512) {
    const uint32_t n = cnt[x];
    for (uint32_t c = 0; 8 * c < n; ++c) {
      uint32_t* o = info + 1 + 3 * (cbase[x] + c);
      o[0] = x;
      o[1] = off[x] + 8 * c;
      o[2] = min(8u, n - 8 * c);
    }
  }
}

// resid[col][i] += sum_j wts[col][j] * y[slot_of[col k + j]][i], j in selection order.
__global__ __launch_bounds__(256) void k_moe_combine(const float* __restrict__ y, const uint32_t* __restrict__ slot_of,
                                                     const float* __restrict__ wts, uint32_t k, uint32_t d,
                                                     float* __restrict__ resid) {
  const uint32_t col = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
  if (i >= d) return;
  float acc = 0.f;
  for (uint32_t j = 0; j < k; ++j) {
    const uint32_t s = slot_of[(size_t)col * k + j];
    acc = __builtin_fmaf(wts[(size_t)col * k + j], y[(size_t)s * d + i], acc);
  }
  resid[(size_t)col * d + i] += acc;
}

}  // namespace

uint32_t sh_moe_max_chunks(uint32_t P, uint32_t E) { return std::min(P, E) + P / 8 + 1; }

int sh_moe_route_launch(sh_engine* e, const float* x, const float* norm_w, const float* router, uint32_t d, uint32_t E,
                        float eps, uint32_t N, float* logits) {
  SH_CHECK(E >= 1 && E <= kMaxExperts && N >= 1, SH_ERR_ARG, "moe route: E=%u N=%u", E, N);
  SH_CHECK(d % 256 == 0 && d >= 256 && d <= 4096, SH_ERR_UNSUPPORTED,
           "moe route: n_embd %u (a multiple of 256 up to 4096)", d);
  hipEvent_t ev = nullptr;
  sh_prof_begin(e, &ev);
  if (d <= 2048)
    hipLaunchKernelGGL(k_moe_logits<8>, dim3((E + 7) / 8, (N + 3) / 4), dim3(64), 0, e->stream, x, norm_w, router, d,
                       E, N, eps, logits);
  else
    hipLaunchKernelGGL(k_moe_logits<16>, dim3((E + 7) / 8, (N + 1) / 2), dim3(64), 0, e->stream, x, norm_w, router,
                       d, E, N, eps, logits);
  SH_HIP(hipGetLastError());
  sh_prof_end(e, "moe_route", 4.0 * E * d, ev);
  return SH_OK;
}

int sh_moe_plan_launch(sh_engine* e, const float* logits, uint32_t N, uint32_t E, uint32_t k, uint32_t* ids,
                       float* wts, uint32_t* info, uint32_t* pair_col, uint32_t* slot_of) {
  SH_CHECK(N >= 1 && k >= 1 && k <= 64 && k <= E && N * k <= 512 && E <= kMaxExperts, SH_ERR_ARG,
           "moe plan: N=%u k=%u E=%u", N, k, E);
  hipEvent_t ev = nullptr;
  sh_prof_begin(e, &ev);
  if (E <= 128)
    hipLaunchKernelGGL(k_moe_plan<2>, dim3(1), dim3(512), 0, e->stream, logits, N, E, k, ids, wts, info, pair_col,
                       slot_of);
  else if (E <= 256)
    hipLaunchKernelGGL(k_moe_plan<4>, dim3(1), dim3(512), 0, e->stream, logits, N, E, k, ids, wts, info, pair_col,
                       slot_of);
  else
    hipLaunchKernelGGL(k_moe_plan<kMaxExperts / 64>, dim3(1), dim3(512), 0, e->stream, logits, N, E, k, ids, wts,
                       info, pair_col, slot_of);
  SH_HIP(hipGetLastError());
  sh_prof_end(e, "moe_plan", 0.0, ev);
  return SH_OK;
}

int sh_moe_combine_launch(sh_engine* e, const float* y, const uint32_t* slot_of, const float* wts, uint32_t k,
                          uint32_t d, uint32_t N, float* resid) {
  hipEvent_t ev = nullptr;
  sh_prof_begin(e, &ev);
  hipLaunchKernelGGL(k_moe_combine, dim3((d + 255) / 256, N), dim3(256), 0, e->stream, y, slot_of, wts, k, d, resid);
  SH_HIP(hipGetLastError());
  sh_prof_end(e, "moe_combine", 0.0, ev);
  return SH_OK;
}
