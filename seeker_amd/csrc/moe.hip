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
#include "sh_operand.h"

namespace {

constexpr uint32_t kMaxExperts = 1024;

// Router logits, one wave per (EPW experts, CPW columns): logits[col][e] =
// rinv(col) * sum_i R[e][i] (x[col][i] norm_w[i]), rinv = 1 / sqrt(mean(x^2) +
// eps) (the RMSNorm factor is linear, so it is applied to the dot product).
// Lane l holds elements 4 l + 256 j (j < d / 256) of each of the wave's
// columns and router rows in registers, every load issued at the start (one
// memory latency per wave), and the sums reduce across the wave by DPP steps.
// The launch spreads the router over E / EPW x ceil(N / CPW) waves.
template <int NJ, int EPW, int CPW>
__global__ __launch_bounds__(64) void k_moe_logits(const float* __restrict__ x, const float* __restrict__ norm_w,
                                                   const float* __restrict__ R, uint32_t d, uint32_t E, uint32_t N,
                                                   float eps, float* __restrict__ logits) {
  const uint32_t lane = threadIdx.x, nj = d / 256;
  const uint32_t e0 = blockIdx.x * EPW, c0 = blockIdx.y * CPW;
  float4 xv[CPW][NJ], rv[EPW][NJ];
#pragma unroll
  for (int c = 0; c < CPW; ++c) {
    const uint32_t col = c0 + c < N ? c0 + c : N - 1;  // past the last column: a clamped (unused) read
    const float* xc = x + (size_t)col * d + 4 * lane;
#pragma unroll
    for (int j = 0; j < NJ; ++j) xv[c][j] = (uint32_t)j < nj ? *(const float4*)(xc + 256 * j) : float4{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int ei = 0; ei < EPW; ++ei) {
    const float* r = R + (size_t)min(e0 + ei, E - 1) * d + 4 * lane;  // past the last expert: a clamped (unused) read
#pragma unroll
    for (int j = 0; j < NJ; ++j) rv[ei][j] = (uint32_t)j < nj ? *(const float4*)(r + 256 * j) : float4{0.f, 0.f, 0.f, 0.f};
  }
  float rinv[CPW];
#pragma unroll
  for (int c = 0; c < CPW; ++c) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) ss += sh_sq4(xv[c][j]);
    rinv[c] = 1.0f / sqrtf(sh_wave_sum(ss) / (float)d + eps);
  }
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const float4 w = (uint32_t)j < nj ? *(const float4*)(norm_w + 4 * lane + 256 * j) : float4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
      xv[c][j].x *= w.x; xv[c][j].y *= w.y; xv[c][j].z *= w.z; xv[c][j].w *= w.w;
    }
  }
#pragma unroll
  for (int ei = 0; ei < EPW; ++ei) {
    const uint32_t e = e0 + ei;
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
      float a = 0.f;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        a = __builtin_fmaf(rv[ei][j].x, xv[c][j].x, a);
        a = __builtin_fmaf(rv[ei][j].y, xv[c][j].y, a);
        a = __builtin_fmaf(rv[ei][j].z, xv[c][j].z, a);
        a = __builtin_fmaf(rv[ei][j].w, xv[c][j].w, a);
      }
      const float sum = sh_wave_sum(a);
      if (lane == 0 && c0 + c < N && e < E) logits[(size_t)(c0 + c) * E + e] = sum * rinv[c];
    }
  }
}

// Top-k selection and routing plan in one workgroup of 1024 threads for
// P = N k <= 512 (column, slot) pairs.
//  * Top-k: k rounds pick the largest remaining logit, then the lowest expert
//    index holding it (softmax is monotone, so this is the top-k of the
//    probabilities, ties to the lower expert index), and the weights
//    exp(l_j - l_max) / sum over the selection in f64, summed in selection
//    order (the full softmax denominator cancels in the renormalization).
//    For k <= 8 (G8) an 8-lane group takes a column, so a wave selects for 8
//    columns at once (12 -> ~2 us for 56 columns of 128 experts); otherwise
//    wave w takes columns w, w + 16, ... with lane l holding logits l, l + 64,
//    ... (DPP wave max, then the lowest index by ballot). Both give the same
//    selections and weights.
//  * Plan: pair p = column * k + slot has expert ids[p]. Pairs are sorted by
//    expert, within an expert by p: a bitmap of pairs per expert gives each
//    pair's rank by population counts, a wave scan over the experts their
//    offsets. Sorted position s of pair p is slot_of[p] and its input column
//    pair_col[s]. Each expert's run of pairs is cut into chunks of at most 8:
//    info[0] = number of chunks, info[1 + 3c .. +3] = (expert, first sorted
//    pair, count), chunks in expert order.
template <int SHIFT_CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, SHIFT_CTRL, 0xF, 0xF, false);
}

// G8: top-k by 8-lane groups (k <= 8, E <= 64 RL), else one wave per column.
template <int RL, bool G8>
__global__ __launch_bounds__(1024) void k_moe_plan(const float* __restrict__ logits, uint32_t N, uint32_t E,
                                                  uint32_t k, uint32_t* __restrict__ ids, float* __restrict__ wts,
                                                  uint32_t* __restrict__ info, uint32_t* __restrict__ pair_col,
                                                  uint32_t* __restrict__ slot_of) {
  constexpr uint32_t NW = 16;  // bitmap words per expert: P <= 512
  __shared__ uint32_t sid[512];
  __shared__ uint32_t bm[kMaxExperts * NW];
  __shared__ uint32_t cnt[kMaxExperts], off[kMaxExperts], cbase[kMaxExperts];
  const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const uint32_t P = N * k, nw = (P + 31) / 32;
  for (uint32_t i = t; i < E * NW; i += 1024) bm[i] = 0u;
  if constexpr (G8) {
    // 8 lanes per column, 8 columns per wave: lane q of a group holds experts
    // q, q + 8, ... (VPL of them); a round is a local max, a 3-step DPP max
    // over the group, the lowest index holding it (local search, 3-step DPP
    // min), so all of a wave's columns select at once
    constexpr uint32_t VPL = 8 * RL;  // experts per lane: E <= 8 * VPL
    const uint32_t q = lane & 7, grp = lane >> 3;
    for (uint32_t pass = 0; 128 * pass < N; ++pass) {  // uniform over the wave
      const uint32_t col = 128 * pass + 8 * wave + grp;
      const bool active = col < N;
      // a taken expert (and the padding past E) holds NaN: fmaxf skips it and
      // no comparison matches it; NaN logits rank as -inf
      float lv[VPL];
#pragma unroll
      for (uint32_t r = 0; r < VPL; ++r) {
        const uint32_t ex = q + 8 * r;
        const float v = active && ex < E ? logits[(size_t)col * E + ex] : -INFINITY;
        lv[r] = ex >= E ? __builtin_nanf("") : (v != v ? -INFINITY : v);
      }
      uint32_t sel_e = 0;
      float sel_l = 0.f, l0 = 0.f;
      for (uint32_t j = 0; j < k; ++j) {
        float lm = lv[0];
#pragma unroll
        for (uint32_t r = 1; r < VPL; ++r) lm = fmaxf(lm, lv[r]);
        lm = fmaxf(lm, sh_dpp<SH_DPP_XOR1>(lm));
        lm = fmaxf(lm, sh_dpp<SH_DPP_XOR2>(lm));
        const float m = fmaxf(lm, sh_dpp<SH_DPP_HALF_MIRROR>(lm));
        uint32_t rr = VPL;
#pragma unroll
        for (int r = VPL - 1; r >= 0; --r)
          if (lv[r] == m) rr = (uint32_t)r;
        uint32_t ce = rr < VPL ? q + 8 * rr : 0xFFFFFFFFu;
        ce = min(ce, dpp_u32<SH_DPP_XOR1>(ce));
        ce = min(ce, dpp_u32<SH_DPP_XOR2>(ce));
        const uint32_t e = min(ce, dpp_u32<SH_DPP_HALF_MIRROR>(ce));
#pragma unroll
        for (uint32_t r = 0; r < VPL; ++r)
          if (e == q + 8 * r) lv[r] = __builtin_nanf("");
        if (q == j) { sel_e = e; sel_l = m; }
        if (j == 0) l0 = m;
      }
      // weights exp(l_j - l_0) / sum_j exp(l_j - l_0) in f64, summed in selection order
      const double w = q < k ? exp((double)sel_l - (double)l0) : 0.0;
      double wsum = 0.0;
      for (uint32_t j = 0; j < k; ++j) wsum += __shfl(w, (int)(8 * grp + j));
      if (active && q < k) {
        ids[(size_t)col * k + q] = sel_e;
        wts[(size_t)col * k + q] = (float)(w / wsum);
        sid[col * k + q] = min(sel_e, E - 1);
      }
    }
  } else {
    for (uint32_t cb = wave; cb < N; cb += 64) {  // the wave's next 4 columns cb + 16 i: loads issued together
      float pre[4][RL];
  #pragma unroll
      for (uint32_t i = 0; i < 4; ++i)
  #pragma unroll
        for (uint32_t r = 0; r < RL; ++r) {
          const uint32_t col = cb + 16 * i;
          pre[i][r] = col < N && lane + 64 * r < E ? logits[(size_t)col * E + lane + 64 * r] : -INFINITY;
        }
  #pragma unroll
    for (uint32_t i = 0; i < 4; ++i) {
      const uint32_t col = cb + 16 * i;
      if (col >= N) break;
      // lane l holds experts l, l + 64, ...; NaN ranks as -inf
      float lv[RL];
      bool taken[RL];
  #pragma unroll
      for (uint32_t r = 0; r < RL; ++r) {
        const float v = pre[i][r];
        lv[r] = v != v ? -INFINITY : v;
        taken[r] = lane + 64 * r >= E;
      }
      // round j: the largest value not yet taken (DPP wave max), then the lowest
      // expert index holding it (ballots, lowest r first); lane j keeps it
      uint32_t sel_e = 0;
      float sel_l = 0.f;
      for (uint32_t j = 0; j < k; ++j) {
        float lm = -INFINITY;
  #pragma unroll
        for (uint32_t r = 0; r < RL; ++r) lm = taken[r] ? lm : fmaxf(lm, lv[r]);
        const float m = sh_wave_max(lm);
        uint32_t e = 0;
        bool found = false;
  #pragma unroll
        for (uint32_t r = 0; r < RL; ++r) {
          const unsigned long long b = __ballot(!taken[r] && lv[r] == m);
          if (!found && b) {
            e = 64 * r + (uint32_t)__ffsll((long long)b) - 1;
            found = true;
          }
        }
  #pragma unroll
        for (uint32_t r = 0; r < RL; ++r) taken[r] = taken[r] || lane + 64 * r == e;
        if (lane == j) { sel_e = e; sel_l = m; }
      }
      // weights exp(l_j - l_0) / sum_j exp(l_j - l_0) in f64, summed in selection order
      const float l0 = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, sel_l)));
      const double w = lane < k ? exp((double)sel_l - (double)l0) : 0.0;
      double wsum = 0.0;
      for (uint32_t j = 0; j < k; ++j) {  // lane j's weight, read lane by lane (uniform j)
        const unsigned long long wb = __builtin_bit_cast(unsigned long long, w);
        const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)wb, (int)j);
        const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(wb >> 32), (int)j);
        wsum += __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
      }
      if (lane < k) {
        ids[(size_t)col * k + lane] = sel_e;
        wts[(size_t)col * k + lane] = (float)(w / wsum);
        sid[col * k + lane] = min(sel_e, E - 1);
      }
    }
    }
  }
  __syncthreads();
  if (t < P) atomicOr(&bm[sid[t] * NW + (t >> 5)], 1u << (t & 31));
  __syncthreads();
  for (uint32_t x = t; x < E; x += 1024) {
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
  for (uint32_t x = t; x < E; x += 1024) {
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
  if (d <= 2048)  // 4 experts x 2 columns per wave
    hipLaunchKernelGGL((k_moe_logits<8, 4, 2>), dim3((E + 3) / 4, (N + 1) / 2), dim3(64), 0, e->stream, x, norm_w,
                       router, d, E, N, eps, logits);
  else  // 2 experts x 1 column per wave
    hipLaunchKernelGGL((k_moe_logits<16, 2, 1>), dim3((E + 1) / 2, N), dim3(64), 0, e->stream, x, norm_w, router, d,
                       E, N, eps, logits);
  SH_HIP(hipGetLastError());
  sh_prof_end(e, "moe_route", 4.0 * E * d, ev);
  return SH_OK;
}

// SH_MOE_PLAN=wave: the wave-per-column top-k for every k (measurement switch).
static bool moe_plan_g8() {
  static const bool v = [] {
    const char* s = getenv("SH_MOE_PLAN");
    return !(s && std::string(s) == "wave");
  }();
  return v;
}

int sh_moe_plan_launch(sh_engine* e, const float* logits, uint32_t N, uint32_t E, uint32_t k, uint32_t* ids,
                       float* wts, uint32_t* info, uint32_t* pair_col, uint32_t* slot_of) {
  SH_CHECK(N >= 1 && k >= 1 && k <= 64 && k <= E && N * k <= 512 && E <= kMaxExperts, SH_ERR_ARG,
           "moe plan: N=%u k=%u E=%u", N, k, E);
  hipEvent_t ev = nullptr;
  sh_prof_begin(e, &ev);
  const bool g8 = k <= 8 && moe_plan_g8();
  if (E <= 128 && g8)
    hipLaunchKernelGGL((k_moe_plan<2, true>), dim3(1), dim3(1024), 0, e->stream, logits, N, E, k, ids, wts, info,
                       pair_col, slot_of);
  else if (E <= 256 && g8)
    hipLaunchKernelGGL((k_moe_plan<4, true>), dim3(1), dim3(1024), 0, e->stream, logits, N, E, k, ids, wts, info,
                       pair_col, slot_of);
  else if (E <= 128)
    hipLaunchKernelGGL((k_moe_plan<2, false>), dim3(1), dim3(1024), 0, e->stream, logits, N, E, k, ids, wts, info,
                       pair_col, slot_of);
  else if (E <= 256)
    hipLaunchKernelGGL((k_moe_plan<4, false>), dim3(1), dim3(1024), 0, e->stream, logits, N, E, k, ids, wts, info,
                       pair_col, slot_of);
  else
    hipLaunchKernelGGL((k_moe_plan<kMaxExperts / 64, false>), dim3(1), dim3(1024), 0, e->stream, logits, N, E, k, ids, wts,
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
