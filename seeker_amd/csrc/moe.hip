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

// One column per workgroup (256 threads). x_n = x * rsqrt(mean(x^2) + eps) *
// norm_w in LDS, logits = R x_n (R: f32 [E][d], ffn_gate_inp), then wave 0
// picks the n_used largest logits one at a time (softmax is monotone, so this
// is the top-k of the probabilities) and computes their weights
// exp(l_j - l_max) / sum over the selection in f64: the full softmax
// denominator cancels in the renormalization.
__global__ __launch_bounds__(256) void k_moe_route(const float* __restrict__ x, const float* __restrict__ norm_w,
                                                   const float* __restrict__ R, uint32_t d, uint32_t E, uint32_t k,
                                                   float eps, uint32_t* __restrict__ ids, float* __restrict__ wts) {
  extern __shared__ float smem[];
  float* sx = smem;          // [d]
  float* sl = smem + d;      // [E]
  __shared__ float red[4];
  __shared__ double sw[64];
  const uint32_t col = blockIdx.x, t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const float* xc = x + (size_t)col * d;
  float ss = 0.f;
  for (uint32_t i = t; i < d; i += 256) ss = __builtin_fmaf(xc[i], xc[i], ss);
  for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
  if (lane == 0) red[wave] = ss;
  __syncthreads();
  const float rinv = 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)d + eps);
  for (uint32_t i = t; i < d; i += 256) sx[i] = xc[i] * rinv * norm_w[i];
  __syncthreads();
  for (uint32_t e = wave; e < E; e += 4) {
    const float* r = R + (size_t)e * d;
    float acc = 0.f;
    for (uint32_t i = 4 * lane; i < d; i += 256) {
      const float4 w = *(const float4*)(r + i);
      acc = __builtin_fmaf(w.x, sx[i], acc);
      acc = __builtin_fmaf(w.y, sx[i + 1], acc);
      acc = __builtin_fmaf(w.z, sx[i + 2], acc);
      acc = __builtin_fmaf(w.w, sx[i + 3], acc);
    }
    for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off);
    if (lane == 0) sl[e] = acc;
  }
  __syncthreads();
  if (wave != 0) return;
  // lane l holds logits l, l + 64, ...; a taken expert's logit becomes -inf
  float lv[kMaxExperts / 64];
#pragma unroll
  for (uint32_t r = 0; r < kMaxExperts / 64; ++r) lv[r] = lane + 64 * r < E ? sl[lane + 64 * r] : -INFINITY;
  float lmax = 0.f;
  for (uint32_t j = 0; j < k; ++j) {
    unsigned long long best = 0ull;
#pragma unroll
    for (uint32_t r = 0; r < kMaxExperts / 64; ++r)
      if (lane + 64 * r < E) {
        const unsigned long long key = lv[r] == -INFINITY ? 0ull : route_key(lv[r], lane + 64 * r);
        best = key > best ? key : best;
      }
    for (int off = 32; off >= 1; off >>= 1) {
      const unsigned long long o = __shfl_xor(best, off);
      best = o > best ? o : best;
    }
    const uint32_t e = best ? ~(uint32_t)(best & 0xFFFFFFFFull) : 0u;
    const float l = sl[e];
    if (j == 0) lmax = l;
#pragma unroll
    for (uint32_t r = 0; r < kMaxExperts / 64; ++r)
      if (lane + 64 * r == e) lv[r] = -INFINITY;
    if (lane == 0) {
      ids[(size_t)col * k + j] = e;
      sw[j] = exp((double)l - (double)lmax);
    }
  }
  if (lane == 0) {
    double s = 0.0;
    for (uint32_t j = 0; j < k; ++j) s += sw[j];
    for (uint32_t j = 0; j < k; ++j) wts[(size_t)col * k + j] = (float)(sw[j] / s);
  }
}

// Routing plan, one workgroup of 512 threads for P <= 512 (column, slot)
// pairs, pair p = column * k + slot with expert ids[p]. Pairs are sorted by
// expert, within an expert by p; sorted position s of pair p is slot_of[p]
// and its input column pair_col[s]. Each expert's run of pairs is cut into
// chunks of at most 8: info[0] = number of chunks, info[1 + 3c .. +3] =
// (expert, first sorted pair, count), chunks in expert order.
__global__ __launch_bounds__(512) void k_moe_plan(const uint32_t* __restrict__ ids, uint32_t P, uint32_t E,
                                                  uint32_t k, uint32_t* __restrict__ info,
                                                  uint32_t* __restrict__ pair_col, uint32_t* __restrict__ slot_of) {
  __shared__ uint32_t sid[512];
  __shared__ uint32_t cnt[kMaxExperts], off[kMaxExperts], cbase[kMaxExperts];
  const uint32_t t = threadIdx.x;
  for (uint32_t e = t; e < E; e += 512) cnt[e] = 0;
  if (t < P) sid[t] = min(ids[t], E - 1);  // ids come from the router (< E); the clamp keeps LDS in bounds
  __syncthreads();
  uint32_t rank = 0, e = 0;
  if (t < P) {
    e = sid[t];
    for (uint32_t q = 0; q < t; ++q) rank += sid[q] == e;
    atomicAdd(&cnt[e], 1u);
  }
  __syncthreads();
  if (t == 0) {
    uint32_t o = 0, c = 0;
    for (uint32_t x = 0; x < E; ++x) {
      off[x] = o;
      cbase[x] = c;
      o += cnt[x];
      c += (cnt[x] + 7) / 8;
    }
    info[0] = c;
  }
  __syncthreads();
  if (t < P) {
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
                        uint32_t k, float eps, uint32_t N, uint32_t* ids, float* wts) {
  SH_CHECK(E >= 1 && E <= kMaxExperts && k >= 1 && k <= 64 && k <= E && d % 4 == 0 && N >= 1, SH_ERR_ARG,
           "moe route: E=%u k=%u d=%u N=%u", E, k, d, N);
  const size_t lds = (size_t)(d + E) * sizeof(float);
  SH_CHECK(lds <= 60 * 1024, SH_ERR_UNSUPPORTED, "moe route: n_embd %u + %u experts exceed the LDS staging", d, E);
  hipEvent_t ev = nullptr;
  sh_prof_begin(e, &ev);
  hipLaunchKernelGGL(k_moe_route, dim3(N), dim3(256), lds, e->stream, x, norm_w, router, d, E, k, eps, ids, wts);
  SH_HIP(hipGetLastError());
  sh_prof_end(e, "moe_route", 4.0 * E * d, ev);
  return SH_OK;
}

int sh_moe_plan_launch(sh_engine* e, const uint32_t* ids, uint32_t P, uint32_t E, uint32_t k, uint32_t* info,
                       uint32_t* pair_col, uint32_t* slot_of) {
  SH_CHECK(P >= 1 && P <= 512 && E >= 1 && E <= kMaxExperts && k >= 1, SH_ERR_ARG, "moe plan: P=%u E=%u", P, E);
  hipEvent_t ev = nullptr;
  sh_prof_begin(e, &ev);
  hipLaunchKernelGGL(k_moe_plan, dim3(1), dim3(512), 0, e->stream, ids, P, E, k, info, pair_col, slot_of);
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
