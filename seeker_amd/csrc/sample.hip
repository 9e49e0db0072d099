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

// Weights held explicitly (the residual of a tree node after rejections).
struct RowR {
  const double* r;
  __device__ __forceinline__ double w(uint32_t v) const { return r[v]; }
};

// Workgroup-wide inverse CDF: first v with cumsum(w) >= target (ge = true) or
// > target (ge = false), where target = u * total; falls back to V-1.
// Each thread owns a contiguous chunk, so cumsum order = vocab order.
template <class W>
__device__ uint32_t wg_inverse_cdf(const W& rw, uint32_t V, float u, bool ge, double* total_out) {
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

// Orderable argmax key: larger float -> larger key, ties -> lower index; NaN loses.
__device__ __forceinline__ unsigned long long tree_amax_key(float v, uint32_t idx) {
  if (v != v) return 0ull;
  uint32_t b = __builtin_bit_cast(uint32_t, v);
  b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((unsigned long long)b << 32) | (unsigned long long)(~idx);
}

// Tree acceptance, one workgroup per tree (b): walk from the root; children of
// the current node v are tried in index order, child c accepted iff
// u * q(tok_c) < cur(tok_c), where cur starts as softmax(p_v / T) and after
// each rejection becomes max(0, cur - q_v) / Z (kept unnormalised in r with its
// sum Z; unchanged if that is all zero). With no child accepted the next token
// is drawn from cur (softmax numerator or r, first v with cumsum > u * total);
// an accepted leaf draws from its own p. Greedy: the child whose token is the
// argmax of p_v. Uniform words: counter + 2 (b n + c) to accept child c,
// counter + 2 (b n + v) + 1 to draw at v.
__global__ __launch_bounds__(256) void k_tree_accept(const float* __restrict__ p, const float* __restrict__ q,
                                                     const uint32_t* __restrict__ tokens,
                                                     const int32_t* __restrict__ parents, uint32_t n, uint32_t V,
                                                     double inv_t, int greedy, const float* u_dev, uint64_t seed,
                                                     uint64_t counter, double* __restrict__ rbuf,
                                                     uint32_t* __restrict__ path_out, uint32_t* __restrict__ path_len,
                                                     uint32_t* __restrict__ next_tok) {
  __shared__ float shf[4];
  __shared__ double shd[4];
  __shared__ unsigned long long shk[4];
  __shared__ int s_acc;
  __shared__ uint32_t s_path[64];
  const uint32_t b = blockIdx.x, t = threadIdx.x;
  const float* P = p + (size_t)b * n * V;
  const float* Q = q ? q + (size_t)b * n * V : nullptr;
  const uint32_t* tok = tokens + (size_t)b * n;
  const int32_t* par = parents + (size_t)b * n;
  double* r = rbuf ? rbuf + (size_t)b * V : nullptr;
  uint32_t v = 0, len = 1, out_tok = 0;
  if (t == 0) s_path[0] = 0;
  for (;;) {
    const float* pv = P + (size_t)v * V;
    int acc = -1;
    if (greedy) {
      unsigned long long best = 0ull;
      for (uint32_t i = t; i < V; i += 256) {
        const unsigned long long k = tree_amax_key(pv[i], i);
        best = k > best ? k : best;
      }
      for (int off = 32; off >= 1; off >>= 1) {
        const unsigned long long o = __shfl_xor(best, off);
        best = o > best ? o : best;
      }
      __syncthreads();
      if ((t & 63) == 0) shk[t >> 6] = best;
      __syncthreads();
      for (int w = 0; w < 4; ++w) best = shk[w] > best ? shk[w] : best;
      const uint32_t am = best == 0ull ? 0u : ~(uint32_t)(best & 0xFFFFFFFFull);
      for (uint32_t c = v + 1; c < n && acc < 0; ++c)
        if (par[c] == (int32_t)v && tok[c] == am) acc = (int)c;
      if (acc < 0) { out_tok = am; break; }
    } else {
      float mx = -INFINITY;
      for (uint32_t i = t; i < V; i += 256) mx = fmaxf(mx, pv[i]);
      const double pm = block_max_f(mx, shf);
      double ssum = 0.0;
      for (uint32_t i = t; i < V; i += 256) ssum += exp(((double)pv[i] - pm) * inv_t);
      const double ps = block_sum_d(ssum, shd);
      const float* qv = Q + (size_t)v * V;
      double qm = 0.0, qs = 1.0, Z = 1.0;
      bool have_q = false, resid = false;
      for (uint32_t c = v + 1; c < n; ++c) {
        if (par[c] != (int32_t)v) continue;
        if (!have_q) {
          float qx = -INFINITY;
          for (uint32_t i = t; i < V; i += 256) qx = fmaxf(qx, qv[i]);
          qm = block_max_f(qx, shf);
          double qsum = 0.0;
          for (uint32_t i = t; i < V; i += 256) qsum += exp(((double)qv[i] - qm) * inv_t);
          qs = block_sum_d(qsum, shd);
          have_q = true;
        }
        if (t == 0) {
          const uint32_t tc = tok[c];
          bool ok = false;
          if (tc < V) {
            const double pc = resid ? r[tc] / Z : exp(((double)pv[tc] - pm) * inv_t) / ps;
            const double qc = exp(((double)qv[tc] - qm) * inv_t) / qs;
            ok = (double)uniform_at(u_dev, seed, counter + 2ull * ((uint64_t)b * n + c)) * qc < pc;
          }
          s_acc = ok ? 1 : 0;
        }
        __syncthreads();
        if (s_acc) { acc = (int)c; break; }
        // reject: cur <- max(0, cur - q) / Z (two passes; r is rewritten only
        // after the sum over the old values is complete)
        double part = 0.0;
        for (uint32_t i = t; i < V; i += 256) {
          const double cur = resid ? r[i] / Z : exp(((double)pv[i] - pm) * inv_t) / ps;
          const double d = cur - exp(((double)qv[i] - qm) * inv_t) / qs;
          part += d > 0.0 ? d : 0.0;
        }
        const double R = block_sum_d(part, shd);
        if (R > 0.0) {
          for (uint32_t i = t; i < V; i += 256) {
            const double cur = resid ? r[i] / Z : exp(((double)pv[i] - pm) * inv_t) / ps;
            const double d = cur - exp(((double)qv[i] - qm) * inv_t) / qs;
            r[i] = d > 0.0 ? d : 0.0;
          }
          __syncthreads();
          Z = R;
          resid = true;
        }
      }
      if (acc < 0) {
        const float ud = uniform_at(u_dev, seed, counter + 2ull * ((uint64_t)b * n + v) + 1ull);
        if (resid) {
          __threadfence_block();
          RowR rr{r};
          out_tok = wg_inverse_cdf(rr, V, ud, false, nullptr);
        } else {
          RowW rw{pv, nullptr, pm, ps, 0.0, 1.0, inv_t};
          out_tok = wg_inverse_cdf(rw, V, ud, false, nullptr);
        }
        break;
      }
    }
    v = (uint32_t)acc;
    if (t == 0) s_path[len] = v;
    ++len;
    __syncthreads();
  }
  if (t == 0) {
    for (uint32_t i = 0; i < len; ++i) path_out[(size_t)b * n + i] = s_path[i];
    path_len[b] = len;
    next_tok[b] = out_tok;
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

extern "C" int sh_tree_accept(sh_engine* e, const float* p_logits_dev, const float* q_logits_dev,
                              const uint32_t* tokens_dev, const int32_t* parents_dev, uint32_t B, uint32_t n,
                              uint32_t V, const sh_sampling* s, uint32_t* path_dev, uint32_t* path_len_dev,
                              uint32_t* next_tok_dev) {
  SH_CHECK(e && p_logits_dev && tokens_dev && parents_dev && s && path_dev && path_len_dev && next_tok_dev,
           SH_ERR_ARG, "sh_tree_accept: NULL argument");
  SH_CHECK(B >= 1 && n >= 1 && n <= 64 && V >= 1, SH_ERR_ARG, "tree_accept: B=%u n=%u V=%u (n <= 64)", B, n, V);
  const bool greedy = s->mode == SH_SAMPLE_GREEDY || !(s->temperature > 0.f);
  SH_CHECK(greedy || s->mode == SH_SAMPLE_REJECTION, SH_ERR_ARG, "tree_accept: mode %u (GREEDY or REJECTION)",
           s->mode);
  SH_CHECK(greedy || q_logits_dev, SH_ERR_ARG, "tree_accept: rejection sampling needs draft logits");
  // tree shape is validated on the host copy (parents[i] < i, parents[0] = -1)
  std::vector<int32_t> par((size_t)B * n);
  SH_HIP(hipMemcpyAsync(par.data(), parents_dev, par.size() * 4, hipMemcpyDeviceToHost, e->stream));
  SH_HIP(hipStreamSynchronize(e->stream));
  for (uint32_t b = 0; b < B; ++b) {
    SH_CHECK(par[(size_t)b * n] == -1, SH_ERR_ARG, "tree_accept: tree %u root parent must be -1", b);
    for (uint32_t i = 1; i < n; ++i)
      SH_CHECK(par[(size_t)b * n + i] >= 0 && par[(size_t)b * n + i] < (int32_t)i, SH_ERR_ARG,
               "tree_accept: tree %u node %u parent %d must precede it", b, i, par[(size_t)b * n + i]);
  }
  float* udev = nullptr;
  double* r = nullptr;
  if (s->uniforms) {
    const size_t nu = (size_t)B * n * 2;
    SH_HIP(hipMallocAsync((void**)&udev, nu * 4, e->stream));
    SH_HIP(hipMemcpyAsync(udev, s->uniforms, nu * 4, hipMemcpyHostToDevice, e->stream));
  }
  if (!greedy) SH_HIP(hipMallocAsync((void**)&r, (size_t)B * V * sizeof(double), e->stream));
  hipEvent_t ev = nullptr;
  sh_prof_begin(e, &ev);
  hipLaunchKernelGGL(k_tree_accept, dim3(B), dim3(256), 0, e->stream, p_logits_dev, greedy ? nullptr : q_logits_dev,
                     tokens_dev, parents_dev, n, V, greedy ? 1.0 : 1.0 / (double)s->temperature, greedy ? 1 : 0,
                     udev, s->seed, udev ? 0ull : s->counter, r, path_dev, path_len_dev, next_tok_dev);
  hipError_t le = hipGetLastError();
  sh_prof_end(e, "tree_accept", 4.0 * V * B * n * (greedy ? 1 : 2), ev);
  if (udev) (void)hipFreeAsync(udev, e->stream);
  if (r) (void)hipFreeAsync(r, e->stream);
  SH_CHECK(le == hipSuccess, SH_ERR_HIP, "tree_accept launch: %s", hipGetErrorString(le));
  SH_HIP(hipStreamSynchronize(e->stream));
  return sh_prof_flush(e);
}
