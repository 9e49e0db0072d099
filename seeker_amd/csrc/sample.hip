// Acceptance kernels of the verify step.
//
// SH_SAMPLE_COMPARE reproduces the reference's stochastic verify: every verify
// column is sampled independently from softmax(l/T) with its own uniform by
// inverse CDF in vocab-index order (the GPU full-vocab chain,
// inference/ops/sampler.rs:303-368; one uniform per column,
// inference/mod.rs:2181-2231), then drafts are accepted while sample == draft
// (inference/sample.rs:347-361; batched server/inference.rs:2859-2883).
//
// SH_SAMPLE_REJECTION is new (no reference code): speculative sampling of
// Leviathan et al. 2023 / Chen et al. 2023. Draft d_i is accepted iff
// u_acc * q_i(d_i) < p_i(d_i); the first rejected position resamples from
// max(0, p_i - q_i) (p_i if that is all zero), and when all k drafts are
// accepted the bonus token is drawn from p_k. Draws use inverse CDF in vocab
// order, first v with cumsum > u * total.
//
// All probability arithmetic is f64 so that the token a uniform selects does
// not depend on summation order (GPU tree vs CPU sequential).
#include "sh_internal.h"
#include "sh_philox.h"

namespace {

constexpr uint64_t kUniformStream = 0x5EC;

__device__ __forceinline__ double block_sum_d(double v, double* sh) {
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  __syncthreads();
  if (l == 0) sh[w] = v;
  __syncthreads();
  double t = 0.0;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) t += sh[i];
  return t;
}

__device__ __forceinline__ float block_max_f(float v, float* sh) {
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  __syncthreads();
  if (l == 0) sh[w] = v;
  __syncthreads();
  float t = -INFINITY;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) t = fmaxf(t, sh[i]);
  return t;
}

// Row statistics: max and sum of exp((l - max) / T) in f64.
__global__ __launch_bounds__(256) void k_row_stats(const float* __restrict__ p, uint32_t n_p,
                                                   const float* __restrict__ q, uint32_t V, double inv_t,
                                                   double2* __restrict__ stats) {
  __shared__ float shf[4];
  __shared__ double shd[4];
  const uint32_t row = blockIdx.x;
  const float* x = row < n_p ? p + (size_t)row * V : q + (size_t)(row - n_p) * V;
  float mx = -INFINITY;
  for (uint32_t i = threadIdx.x; i < V; i += 256) mx = fmaxf(mx, x[i]);
  mx = block_max_f(mx, shf);
  double s = 0.0;
  for (uint32_t i = threadIdx.x; i < V; i += 256) s += exp(((double)x[i] - (double)mx) * inv_t);
  s = block_sum_d(s, shd);
  if (threadIdx.x == 0) stats[row] = make_double2((double)mx, s);
}

__device__ __forceinline__ float uniform_at(const float* u_dev, uint64_t seed, uint64_t word) {
  if (u_dev) return u_dev[word];
  uint64_t ctr[4] = {word / 4 + 1, 0, 0, 0}, key[2] = {seed, kUniformStream}, out[4];
  sh_philox4x64_10(ctr, key, out);
  return sh_u64_to_unit_f32(out[word % 4]);
}

// Weight of vocab entry v for the inverse CDF: softmax numerator of p, or
// max(0, p - q) with normalised probabilities.
struct RowW {
  const float* p;
  const float* q;  // null: plain p
  double pm, ps, qm, qs, inv_t;
  __device__ __forceinline__ double w(uint32_t v) const {
    const double a = exp(((double)p[v] - pm) * inv_t);
    if (!q) return a;
    const double r = a / ps - exp(((double)q[v] - qm) * inv_t) / qs;
    return r > 0.0 ? r : 0.0;
  }
};

// Workgroup-wide inverse CDF: first v with cumsum(w) >= target (ge = true) or
// > target (ge = false), where target = u * total; falls back to V-1.
// Each thread owns a contiguous chunk, so cumsum order = vocab order.
__device__ uint32_t wg_inverse_cdf(const RowW& rw, uint32_t V, float u, bool ge, double* total_out) {
  __shared__ double part[257];
  __shared__ uint32_t found;
  const uint32_t t = threadIdx.x, C = (V + 255) / 256;
  const uint32_t b0 = min(t * C, V), b1 = min(b0 + C, V);
  double s = 0.0;
  for (uint32_t v = b0; v < b1; ++v) s += rw.w(v);
  __syncthreads();
  part[t] = s;
  __syncthreads();
  if (t == 0) {  // exclusive prefix of the chunk sums, in thread (= vocab) order
    double acc = 0.0;
    for (int i = 0; i < 256; ++i) {
      const double x = part[i];
      part[i] = acc;
      acc += x;
    }
    part[256] = acc;
    found = V - 1;
  }
  __syncthreads();
  const double total = part[256];
  const double target = (double)u * total;
  const double lo = part[t];
  const bool reach = ge ? (lo + s >= target) : (lo + s > target);
  const bool before = t == 0 || (ge ? lo < target : lo <= target);
  if (b0 < b1 && reach && before) {
    double cum = lo;
    uint32_t pick = b1 - 1;
    for (uint32_t v = b0; v < b1; ++v) {
      cum += rw.w(v);
      if (ge ? cum >= target : cum > target) { pick = v; break; }
    }
    atomicMin(&found, pick);
  }
  __syncthreads();
  if (total_out) *total_out = total;
  return found;
}

// COMPARE: sample every column (b, i) independently.
__global__ __launch_bounds__(256) void k_sample_cols(const float* __restrict__ p, const double2* __restrict__ stats,
                                                     uint32_t V, double inv_t, const float* u_dev, uint64_t seed,
                                                     uint64_t counter, uint32_t* __restrict__ out) {
  const uint32_t row = blockIdx.x;
  const double2 st = stats[row];
  RowW rw{p + (size_t)row * V, nullptr, st.x, st.y, 0.0, 1.0, inv_t};
  const float u = uniform_at(u_dev, seed, counter + 2ull * row + 1ull);
  const uint32_t tok = wg_inverse_cdf(rw, V, u, true, nullptr);
  if (threadIdx.x == 0) out[row] = tok;
}

__global__ void k_decide_compare(const uint32_t* __restrict__ samples, const uint32_t* __restrict__ drafts,
                                 uint32_t B, uint32_t k, uint32_t* __restrict__ acc_len,
                                 uint32_t* __restrict__ next_tok) {
  const uint32_t b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  uint32_t i = 0;
  while (i < k && samples[b * (k + 1) + i] == drafts[b * k + i]) ++i;
  acc_len[b] = i;
  next_tok[b] = samples[b * (k + 1) + i];
}

// REJECTION: one workgroup per sequence.
__global__ __launch_bounds__(256) void k_decide_reject(const float* __restrict__ p, const float* __restrict__ q,
                                                       const double2* __restrict__ stats, uint32_t B, uint32_t k,
                                                       uint32_t V, double inv_t, const uint32_t* __restrict__ drafts,
                                                       const float* u_dev, uint64_t seed, uint64_t counter,
                                                       uint32_t* __restrict__ acc_len,
                                                       uint32_t* __restrict__ next_tok) {
  __shared__ uint32_t first_rej;
  const uint32_t b = blockIdx.x, t = threadIdx.x;
  if (t == 0) first_rej = k;
  __syncthreads();
  const double2* sp = stats + (size_t)b * (k + 1);
  const double2* sq = stats + (size_t)B * (k + 1) + (size_t)b * k;
  if (t < k) {
    const uint32_t d = drafts[b * k + t];
    bool accept = false;
    if (d < V) {  // an out-of-vocab draft id is rejected
      const double pd = exp(((double)p[((size_t)b * (k + 1) + t) * V + d] - sp[t].x) * inv_t) / sp[t].y;
      const double qd = exp(((double)q[((size_t)b * k + t) * V + d] - sq[t].x) * inv_t) / sq[t].y;
      const float ua = uniform_at(u_dev, seed, counter + 2ull * (b * (k + 1) + t));
      accept = (double)ua * qd < pd;
    }
    if (!accept) atomicMin(&first_rej, t);
  }
  __syncthreads();
  const uint32_t i = first_rej;
  const float ur = uniform_at(u_dev, seed, counter + 2ull * (b * (k + 1) + i) + 1ull);
  const float* pr = p + ((size_t)b * (k + 1) + i) * V;
  uint32_t tok;
  if (i == k) {
    RowW rw{pr, nullptr, sp[i].x, sp[i].y, 0.0, 1.0, inv_t};
    tok = wg_inverse_cdf(rw, V, ur, false, nullptr);
  } else {
    RowW rw{pr, q + ((size_t)b * k + i) * V, sp[i].x, sp[i].y, sq[i].x, sq[i].y, inv_t};
    double total = 0.0;
    tok = wg_inverse_cdf(rw, V, ur, false, &total);
    if (!(total > 0.0)) {
      RowW rp{pr, nullptr, sp[i].x, sp[i].y, 0.0, 1.0, inv_t};
      tok = wg_inverse_cdf(rp, V, ur, false, nullptr);
    }
  }
  if (t == 0) {
    acc_len[b] = i;
    next_tok[b] = tok;
  }
}

}  // namespace

int sh_accept_launch(sh_engine* e, const float* p_logits, const float* q_logits, const uint32_t* drafts, uint32_t B,
                     uint32_t k, uint32_t V, const sh_sampling* s, uint64_t counter, const float* uniforms_dev,
                     uint32_t* acc_len, uint32_t* next_tok) {
  SH_CHECK(B >= 1 && k >= 1 && k <= 64 && V >= 1, SH_ERR_ARG, "accept: B=%u k=%u V=%u", B, k, V);
  const uint32_t mode = s->mode;
  SH_CHECK(mode == SH_SAMPLE_COMPARE || mode == SH_SAMPLE_REJECTION, SH_ERR_ARG, "accept: mode %u", mode);
  SH_CHECK(s->temperature > 0.f, SH_ERR_ARG, "accept: temperature must be > 0");
  SH_CHECK(mode != SH_SAMPLE_REJECTION || q_logits, SH_ERR_ARG, "REJECTION needs draft logits");
  const double inv_t = 1.0 / (double)s->temperature;
  const uint32_t n_p = B * (k + 1), n_q = mode == SH_SAMPLE_REJECTION ? B * k : 0;
  double2* stats = nullptr;
  SH_HIP(hipMallocAsync((void**)&stats, (size_t)(n_p + n_q) * sizeof(double2), e->stream));
  hipEvent_t ev = nullptr;
  sh_prof_begin(e, &ev);
  hipLaunchKernelGGL(k_row_stats, dim3(n_p + n_q), dim3(256), 0, e->stream, p_logits, n_p, q_logits, V, inv_t, stats);
  SH_HIP(hipGetLastError());
  sh_prof_end(e, "accept_stats", 4.0 * V * (n_p + n_q), ev);
  sh_prof_begin(e, &ev);
  if (mode == SH_SAMPLE_COMPARE) {
    uint32_t* samples = nullptr;
    SH_HIP(hipMallocAsync((void**)&samples, (size_t)n_p * 4, e->stream));
    hipLaunchKernelGGL(k_sample_cols, dim3(n_p), dim3(256), 0, e->stream, p_logits, stats, V, inv_t, uniforms_dev,
                       s->seed, counter, samples);
    hipLaunchKernelGGL(k_decide_compare, dim3((B + 63) / 64), dim3(64), 0, e->stream, samples, drafts, B, k, acc_len,
                       next_tok);
    SH_HIP(hipGetLastError());
    SH_HIP(hipFreeAsync(samples, e->stream));
  } else {
    hipLaunchKernelGGL(k_decide_reject, dim3(B), dim3(256), 0, e->stream, p_logits, q_logits, stats, B, k, V, inv_t,
                       drafts, uniforms_dev, s->seed, counter, acc_len, next_tok);
    SH_HIP(hipGetLastError());
  }
  sh_prof_end(e, "accept_decide", 0.0, ev);
  SH_HIP(hipFreeAsync(stats, e->stream));
  return SH_OK;
}

extern "C" int sh_accept_sample(sh_engine* e, const float* p_logits_dev, const float* q_logits_dev,
                                const uint32_t* drafts_dev, uint32_t B, uint32_t k, uint32_t V, const sh_sampling* s,
                                uint32_t* acc_len_dev, uint32_t* next_tok_dev) {
  SH_CHECK(e && p_logits_dev && drafts_dev && s && acc_len_dev && next_tok_dev, SH_ERR_ARG,
           "sh_accept_sample: NULL argument");
  float* udev = nullptr;
  if (s->uniforms) {
    const size_t n = (size_t)B * (k + 1) * 2;
    SH_HIP(hipMallocAsync((void**)&udev, n * 4, e->stream));
    SH_HIP(hipMemcpyAsync(udev, s->uniforms, n * 4, hipMemcpyHostToDevice, e->stream));
  }
  // explicit uniforms are indexed from 0; Philox words from s->counter
  int rc = sh_accept_launch(e, p_logits_dev, q_logits_dev, drafts_dev, B, k, V, s, udev ? 0 : s->counter, udev,
                            acc_len_dev, next_tok_dev);
  if (udev) (void)hipFreeAsync(udev, e->stream);
  if (rc) return rc;
  SH_HIP(hipStreamSynchronize(e->stream));
  return sh_prof_flush(e);
}
