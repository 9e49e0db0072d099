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
#include <mutex>

#include "sh_internal.h"
#include "sh_coherent.h"
#include "sh_exp.h"
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

// 2^(j/64) for sh_exp_neg; each kernel that calls it copies the table to LDS.
__constant__ double kExp2Tab[64] = SH_EXP2_TABLE_64;

__device__ __forceinline__ void load_exp_table(double* tab) {
  if (threadIdx.x < 64) tab[threadIdx.x] = kExp2Tab[threadIdx.x];
}

__device__ __forceinline__ double wave_sum_d(double v) {
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

__device__ __forceinline__ double wave_max_d(double v) {
  for (int off = 32; off >= 1; off >>= 1) v = fmax(v, __shfl_xor(v, off));
  return v;
}

// Row statistics: max and sum of exp((l - max) / T), in two steps.
// Step 1: the rows are cut into units of 256 E logits (unit c of row r is
// index r * nch + c), one workgroup per unit: every thread keeps its E logits
// in registers (one HBM read), the unit max is reduced, then the exp-sum
// against it. A unit whose logits are all -inf reports (-inf, 0). The terms
// are the hardware exp2 (v_exp_f32, 1 ulp) of (l - max) * log2(e) / T in f32,
// summed in f64: the sum is within ~1e-6 relative of the exact one (it only
// normalises probabilities, whose bound is 1e-5), and one f32 exp per logit
// leaves the kernel bound by HBM. Draws resolve their CDF crossings with f64
// weights computed in the draw kernels themselves, never with these sums.
constexpr int kStatE = 32;

template <bool VEC, int E>
__device__ __forceinline__ void load_unit(const float* __restrict__ p, uint32_t n_p, const float* __restrict__ q,
                                          uint32_t V, uint32_t nch, uint32_t u, float (&v)[E]) {
  const uint32_t row = u / nch, base = (u - row * nch) * 256 * E, t = threadIdx.x;
  const float* x = row < n_p ? p + (size_t)row * V : q + (size_t)(row - n_p) * V;
  if (VEC) {
#pragma unroll
    for (int j = 0; j < E / 4; ++j) {
      const uint32_t i = base + j * 1024 + t * 4;
      float4 f = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
      if (i < V) f = *reinterpret_cast<const float4*>(x + i);  // V % 4 == 0: whole float4 in range
      v[4 * j] = f.x; v[4 * j + 1] = f.y; v[4 * j + 2] = f.z; v[4 * j + 3] = f.w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < E; ++j) {
      const uint32_t i = base + j * 256 + t;
      v[j] = i < V ? x[i] : -INFINITY;
    }
  }
}

template <int E>
__device__ __forceinline__ double2 reduce_unit(const float (&v)[E], double inv_t, float* shf, double* shd) {
  float mx = v[0];
#pragma unroll
  for (int j = 1; j < E; ++j) mx = fmaxf(mx, v[j]);
  mx = block_max_f(mx, shf);
  double s = 0.0;
  if (mx != -INFINITY) {
    const float c = (float)(inv_t * 1.4426950408889634074);  // log2(e) / T
#pragma unroll
    for (int j = 0; j < E; ++j) s += (double)__builtin_amdgcn_exp2f((v[j] - mx) * c);  // -inf -> 0
  }
  return make_double2((double)mx, block_sum_d(s, shd));
}

constexpr uint32_t kCntStride = 64;  // arrival counters 256 bytes apart: no two share a cache line

template <bool VEC, int E>
__global__ __launch_bounds__(256) void k_row_part(const float* __restrict__ p, uint32_t n_p,
                                                  const float* __restrict__ q, uint32_t V, double inv_t,
                                                  uint32_t nch, double2* __restrict__ part,
                                                  const SampRow* __restrict__ rows = nullptr,
                                                  uint32_t* __restrict__ zero_cnt = nullptr, uint32_t nzero = 0) {
  __shared__ float shf[4];
  __shared__ double shd[4];
  // the arrival counters of the kernel that follows start at zero
  if (zero_cnt && blockIdx.x == 0)
    for (uint32_t j = threadIdx.x; j < nzero; j += 256) zero_cnt[(size_t)j * kCntStride] = 0u;
  float v[E];
  load_unit<VEC, E>(p, n_p, q, V, nch, blockIdx.x, v);
  if (rows) inv_t = rows[blockIdx.x / nch].inv_t;  // per-row temperature (a row's units are consecutive)
  const double2 r = reduce_unit<E>(v, inv_t, shf, shd);
  if (threadIdx.x == 0) part[blockIdx.x] = r;
}

// Step 2 (inside the consumers): one wave combines a row's chunk partials into
// (max M, sum of s_c exp((m_c - M) / T)); every lane gets the result.
__device__ double2 wave_row_stat(const double2* __restrict__ part, uint32_t nch, double inv_t, const double* tab) {
  const uint32_t l = threadIdx.x & 63;
  double M = -INFINITY;
  for (uint32_t c = l; c < nch; c += 64) M = fmax(M, part[c].x);
  M = wave_max_d(M);
  double S = 0.0;
  if (M != -INFINITY)
    for (uint32_t c = l; c < nch; c += 64) {
      const double2 pc = part[c];
      if (pc.x != -INFINITY) S += pc.y * sh_exp_neg((pc.x - M) * inv_t, tab);
    }
  return make_double2(M, wave_sum_d(S));
}

// The same combine done by one lane for its own row, all loads of a block of
// 16 partials issued together (blocks after the first rescale the running sum).
__device__ double2 lane_row_stat(const double2* __restrict__ pr, uint32_t nch, double inv_t, const double* tab) {
  double M = -INFINITY, S = 0.0;
  for (uint32_t c0 = 0; c0 < nch; c0 += 16) {
    double2 pc[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) pc[j] = c0 + j < nch ? pr[c0 + j] : make_double2(-INFINITY, 0.0);
    double m = M;
#pragma unroll
    for (int j = 0; j < 16; ++j) m = fmax(m, pc[j].x);
    if (m != -INFINITY) {
      if (M != -INFINITY && M != m) S *= sh_exp_neg((M - m) * inv_t, tab);
#pragma unroll
      for (int j = 0; j < 16; ++j)
        if (pc[j].x != -INFINITY) S += pc[j].y * sh_exp_neg((pc[j].x - m) * inv_t, tab);
    }
    M = m;
  }
  return make_double2(M, S);
}

// Graph replay: the Philox key and word base come from the device words
// rng[0] and rng[1], which the host writes before each replay.
__device__ __forceinline__ void rng_from_dev(const uint64_t* rng, uint64_t& seed, uint64_t& word) {
  if (rng) {
    seed = rng[0];
    word += rng[1];
  }
}

__device__ __forceinline__ float uniform_at(const float* u_dev, uint64_t seed, uint64_t word) {
  if (u_dev) return u_dev[word];
  uint64_t ctr[4] = {word / 4 + 1, 0, 0, 0}, key[2] = {seed, kUniformStream}, out[4];
  sh_philox4x64_10(ctr, key, out);
  return sh_u64_to_unit_f32(out[word % 4]);
}

// Weight of vocab entry v for the inverse CDF: softmax numerator of p, or
// max(0, p - q) with normalised probabilities. raw() loads, wt() computes, so
// callers can issue a block of loads before the arithmetic.
// The residual uses the reciprocals of the two softmax sums (ips, iqs).
struct RowW {
  const float* p;
  const float* q;  // null: plain p
  double pm, ips, qm, iqs, inv_t;
  const double* tab;
  using Raw = float2;
  __device__ __forceinline__ Raw raw(uint32_t v) const { return make_float2(p[v], q ? q[v] : 0.f); }
  __device__ __forceinline__ double num(float pl) const { return sh_exp_neg(((double)pl - pm) * inv_t, tab); }
  // residual weight from the p numerator a and the draft logit ql
  __device__ __forceinline__ double resid(double a, float ql) const {
    const double r = a * ips - sh_exp_neg(((double)ql - qm) * inv_t, tab) * iqs;
    return r > 0.0 ? r : 0.0;
  }
  __device__ __forceinline__ double wt(Raw x) const {
    const double a = num(x.x);
    return q ? resid(a, x.y) : a;
  }
};

// Weights held explicitly (the residual of a tree node after rejections).
struct RowR {
  const double* r;
  using Raw = double;
  __device__ __forceinline__ Raw raw(uint32_t v) const { return r[v]; }
  __device__ __forceinline__ double wt(Raw x) const { return x; }
};

// Sum of the weights of [b0, b1) in index order, 8 loads in flight.
template <class W>
__device__ __forceinline__ double slice_sum(const W& rw, uint32_t b0, uint32_t b1) {
  double s = 0.0;
  for (uint32_t v0 = b0; v0 < b1; v0 += 8) {
    typename W::Raw x[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (v0 + j < b1) x[j] = rw.raw(v0 + j);
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (v0 + j < b1) s += rw.wt(x[j]);
  }
  return s;
}

// First v in [b0, b1) with cum + cumsum(w over [b0, v]) > target (>= if ge);
// b1 - 1 if none.
template <class W>
__device__ __forceinline__ uint32_t slice_find(const W& rw, uint32_t b0, uint32_t b1, double cum, double target,
                                               bool ge) {
  for (uint32_t v0 = b0; v0 < b1; v0 += 8) {
    typename W::Raw x[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (v0 + j < b1) x[j] = rw.raw(v0 + j);
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (v0 + j < b1) {
        cum += rw.wt(x[j]);
        if (ge ? cum >= target : cum > target) return v0 + j;
      }
  }
  return b1 - 1;
}

// Exclusive prefix of x over the 256 threads in thread order, by wave scans:
// ex[t] for thread t, ex[256] = the total.
__device__ void block_exscan_d(double x, double* ex, double* wsum) {
  const uint32_t t = threadIdx.x, l = t & 63, w = t >> 6;
  double inc = x;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const double y = __shfl_up(inc, off);
    if (l >= (uint32_t)off) inc += y;
  }
  double exw = __shfl_up(inc, 1);
  if (l == 0) exw = 0.0;
  __syncthreads();  // earlier readers of ex / wsum are done
  if (l == 63) wsum[w] = inc;
  __syncthreads();
  double base = 0.0;
  for (uint32_t i = 0; i < w; ++i) base += wsum[i];
  ex[t] = base + exw;
  if (t == 255) ex[256] = ((wsum[0] + wsum[1]) + wsum[2]) + wsum[3];
  __syncthreads();
}

// Workgroup-wide inverse CDF over [lo, hi) (256 threads, each owning a
// contiguous slice, so the prefix order is vocab order): the first v with
// off + cumsum(w over [lo, v]) > target (ge = false) or >= target (ge = true).
// rel: target = u * (sum over [lo, hi)) and off = 0. Falls back to hi - 1
// when rounding leaves the sum just short of the target. *total_out (if
// given) receives the sum over [lo, hi).
template <class W>
__device__ uint32_t wg_inverse_cdf(const W& rw, uint32_t lo, uint32_t hi, bool rel, float u, double off,
                                   double target, bool ge, double* total_out) {
  __shared__ double ex[257];
  __shared__ double wsum[4];
  __shared__ uint32_t found;
  const uint32_t t = threadIdx.x, C = (hi - lo + 255) / 256;
  const uint32_t b0 = min(lo + t * C, hi), b1 = min(b0 + C, hi);
  const double s = slice_sum(rw, b0, b1);
  if (t == 0) found = hi - 1;
  block_exscan_d(s, ex, wsum);
  const double total = ex[256];
  if (rel) {
    off = 0.0;
    target = (double)u * total;
  }
  const double a = off + ex[t], z = off + ex[t + 1];
  const bool reach = ge ? z >= target : z > target;
  const bool prior = t == 0 || (ge ? a < target : a <= target);
  if (b0 < b1 && reach && prior) atomicMin(&found, slice_find(rw, b0, b1, a, target, ge));
  __syncthreads();
  if (total_out) *total_out = total;
  return found;
}

// COMPARE: sample every column (b, i) independently; row r takes uniform
// word word0 + wstride * r. The draft draws of a REJECTION speculative step
// use the same sampler.
__global__ __launch_bounds__(256) void k_sample_cols(const float* __restrict__ p, const double2* __restrict__ part,
                                                     uint32_t nch, uint32_t V, double inv_t, const float* u_dev,
                                                     uint64_t seed, uint64_t word0, uint64_t wstride,
                                                     uint32_t* __restrict__ out, const uint64_t* rng) {
  __shared__ double tab[64];
  __shared__ double2 st;
  const uint32_t row = blockIdx.x;
  rng_from_dev(rng, seed, word0);
  load_exp_table(tab);
  __syncthreads();
  if (threadIdx.x < 64) {
    const double2 s = wave_row_stat(part + (size_t)row * nch, nch, inv_t, tab);
    if (threadIdx.x == 0) st = s;
  }
  __syncthreads();
  RowW rw{p + (size_t)row * V, nullptr, st.x, 1.0, 0.0, 1.0, inv_t, tab};
  const float u = uniform_at(u_dev, seed, word0 + wstride * row);
  const uint32_t tok = wg_inverse_cdf(rw, 0, V, true, u, 0.0, 0.0, true, nullptr);
  if (threadIdx.x == 0) out[row] = tok;
}

// Per-row sampling of a batched verify: row r is drawn from softmax(p_r *
// rows[r].inv_t) in vocab order with uniform rows[r].u (explicit) or Philox
// word rows[r].word of key (rows[r].seed, 0x5EC); greedy rows keep the argmax
// already in out[r].
__global__ __launch_bounds__(256) void k_sample_rows_tab(const float* __restrict__ p, const double2* __restrict__ part,
                                                         uint32_t nch, uint32_t V, const SampRow* __restrict__ rows,
                                                         uint32_t* __restrict__ out) {
  __shared__ double tab[64];
  __shared__ double2 st;
  const uint32_t row = blockIdx.x;
  const SampRow sr = rows[row];
  if (sr.greedy || sr.top_k) return;  // uniform: the whole workgroup leaves (filtered rows: k_sample_filtered_tab)
  load_exp_table(tab);
  __syncthreads();
  if (threadIdx.x < 64) {
    const double2 s = wave_row_stat(part + (size_t)row * nch, nch, sr.inv_t, tab);
    if (threadIdx.x == 0) st = s;
  }
  __syncthreads();
  RowW rw{p + (size_t)row * V, nullptr, st.x, 1.0, 0.0, 1.0, sr.inv_t, tab};
  const float u = sr.explicit_u ? sr.u : uniform_at(nullptr, sr.seed, sr.word);
  const uint32_t tok = wg_inverse_cdf(rw, 0, V, true, u, 0.0, 0.0, true, nullptr);
  if (threadIdx.x == 0) out[row] = tok;
}

// ------------------------------------------------------------ filtered sampling
//
// The reference's sampler chain with candidate filters (host order,
// inference/sample.rs:369-473, which the GPU chain mirrors,
// ops/sampler.rs:41-132): the top_k (1..256) largest logits, sorted by logit
// descending with ties to the lower id -> top_p (softmax of the candidates;
// a candidate is dropped once the cumulative probability BEFORE it exceeds
// p, so the crossing one stays) -> min_p (logit below max + ln min_p
// dropped) -> logits times 1/T -> softmax -> the first candidate whose
// cumulative probability reaches u (the last one when rounding leaves the
// sum short). Softmaxes take f64 exps of the f32 logits and f32
// probabilities, cumulative sums in f64 in candidate order, as the C oracle.
//
// One workgroup per row: the top_k-th largest logit by a three-pass radix
// select over orderable keys (11, 11, 10 bits; LDS histograms), one pass to
// collect the candidates (ties at the threshold by index order), a bitonic
// sort of the <= 256 candidates, then the chain on one thread per candidate
// with the order-dependent sums on one thread.
constexpr uint32_t kTopKMax = 256;

struct FiltCfg {
  uint32_t k;        // candidates (1..kTopKMax)
  float top_p;       // used when top_p_on
  float log_min_p;   // ln(min_p), used when min_p_on
  float inv_t;       // 1 / max(T, 1e-9) as f32, used when temp_on
  uint32_t flags;    // 1 top_p_on, 2 min_p_on, 4 temp_on
};

__device__ __forceinline__ uint32_t ord_key(float v) {
  const uint32_t b = __builtin_bit_cast(uint32_t, v);
  if (v != v) return 0u;  // NaN sorts last
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key_value(uint32_t k) {
  return __builtin_bit_cast(float, (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// Exclusive prefix of per-thread counts over the 256 threads (thread order).
__device__ __forceinline__ uint32_t block_exscan_u(uint32_t x, uint32_t* wsum, uint32_t* total) {
  const uint32_t t = threadIdx.x, l = t & 63, w = t >> 6;
  uint32_t inc = x;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t y = __shfl_up(inc, off);
    if (l >= (uint32_t)off) inc += y;
  }
  __syncthreads();
  if (l == 63) wsum[w] = inc;
  __syncthreads();
  uint32_t base = 0;
  for (uint32_t i = 0; i < w; ++i) base += wsum[i];
  if (total) *total = wsum[0] + wsum[1] + wsum[2] + wsum[3];
  return base + inc - x;
}

// softmax of n (<= 256) candidate logits as the C oracle's or_softmax: f64
// exps against the max, summed in order, f32 probabilities. pr[j] for j < n.
__device__ void cand_softmax(const float* kept, uint32_t n, float* pr, double* e, const double* tab) {
  __shared__ double s_sum;
  __shared__ float s_mx;
  const uint32_t t = threadIdx.x;
  if (t == 0) {
    float mx = -INFINITY;
    for (uint32_t j = 0; j < n; ++j) mx = fmaxf(mx, kept[j]);
    s_mx = mx;
  }
  __syncthreads();
  const double mx = (double)s_mx;
  const bool fin = s_mx > -INFINITY && s_mx < INFINITY;
  if (t < n && fin) e[t] = kept[t] == -INFINITY ? 0.0 : sh_exp_neg((double)kept[t] - mx, tab);
  __syncthreads();
  if (t == 0 && fin) {
    double s = 0.0;
    for (uint32_t j = 0; j < n; ++j) s += e[j];
    s_sum = s;
  }
  __syncthreads();
  if (t < n) pr[t] = fin ? (float)(e[t] / s_sum) : 1.0f / (float)n;
  __syncthreads();
}

// The filtered draw of one row (256 threads) with uniform u; returns the id.
__device__ uint32_t sample_filtered_row(const float* __restrict__ x, uint32_t V, const FiltCfg& cf, float u,
                                        const double* tab) {
  __shared__ uint32_t hist[2048];
  __shared__ uint32_t wsum[4];
  __shared__ uint32_t s_prefix, s_need, s_n;
  __shared__ unsigned long long cand[kTopKMax];
  __shared__ float kept[kTopKMax], pr[kTopKMax];
  __shared__ double e[kTopKMax];
  __shared__ uint32_t s_ch;
  const uint32_t t = threadIdx.x, k = cf.k;
  // ---- radix select: the k-th largest key (prefix) and how many of the
  // keys equal to it are taken (need)
  if (t == 0) { s_prefix = 0; s_need = k; }
  constexpr int kShift[3] = {21, 10, 0};
  constexpr int kBits[3] = {11, 11, 10};
#pragma unroll
  for (int ps = 0; ps < 3; ++ps) {
    const uint32_t nb = 1u << kBits[ps];
    for (uint32_t i = t; i < 2048; i += 256) hist[i] = 0;
    __syncthreads();
    const uint32_t hi_shift = kShift[ps] + kBits[ps];  // bits above this digit must match the prefix
    const uint32_t prefix = s_prefix, need = s_need;     // read before this pass's crossing thread writes
    for (uint32_t i = t; i < V; i += 256) {
      const uint32_t key = ord_key(x[i]);
      if (hi_shift == 32 || (key >> hi_shift) == (prefix >> hi_shift))
        atomicAdd(&hist[(key >> kShift[ps]) & (nb - 1)], 1u);
    }
    __syncthreads();
    // thread t owns bins [8 t, 8 t + 8) counted from the top (bin nb - 1 - i)
    const uint32_t per = nb / 256;
    uint32_t c = 0;
    for (uint32_t j = 0; j < per; ++j) c += hist[nb - 1 - (per * t + j)];
    const uint32_t above = block_exscan_u(c, wsum, nullptr);
    if (above < need && above + c >= need) {  // the crossing bin is in this thread's range
      uint32_t a = above;
      for (uint32_t j = 0; j < per; ++j) {
        const uint32_t bin = nb - 1 - (per * t + j), h = hist[bin];
        if (a + h >= need) {
          s_prefix = prefix | (bin << kShift[ps]);
          s_need = need - a;
          break;
        }
        a += h;
      }
    }
    __syncthreads();
  }
  const uint32_t tau = s_prefix, ties = s_need;  // keys > tau: k - ties of them; plus `ties` keys == tau
  // ---- collect: keys above tau in any order, ties at tau by index
  if (t == 0) s_n = 0;
  __syncthreads();
  uint32_t n_eq = 0;
  for (uint32_t i = t; i < V; i += 256) {
    const uint32_t key = ord_key(x[i]);
    if (key > tau) {
      const uint32_t pos = atomicAdd(&s_n, 1u);
      if (pos < kTopKMax) cand[pos] = ((unsigned long long)key << 32) | (unsigned long long)(~i);
    }
    n_eq += key == tau;
  }
  uint32_t eq_total;
  (void)block_exscan_u(n_eq, wsum, &eq_total);
  if (eq_total == ties) {  // every key equal to tau is taken
    for (uint32_t i = t; i < V; i += 256)
      if (ord_key(x[i]) == tau) {
        const uint32_t pos = atomicAdd(&s_n, 1u);
        if (pos < kTopKMax) cand[pos] = ((unsigned long long)tau << 32) | (unsigned long long)(~i);
      }
  } else {  // the first `ties` of them in index order: thread t owns a contiguous slice
    const uint32_t C = (V + 255) / 256, b0 = min(t * C, V), b1 = min(b0 + C, V);
    uint32_t mine = 0;
    for (uint32_t i = b0; i < b1; ++i) mine += ord_key(x[i]) == tau;
    uint32_t rank = block_exscan_u(mine, wsum, nullptr);
    const uint32_t base = k - ties;
    for (uint32_t i = b0; i < b1 && rank < ties; ++i)
      if (ord_key(x[i]) == tau) {
        cand[base + rank] = ((unsigned long long)tau << 32) | (unsigned long long)(~i);
        ++rank;
      }
  }
  __syncthreads();
  // ---- bitonic sort of the k candidates, descending (padding sorts last)
  if (t >= k) cand[t] = 0ull;
  __syncthreads();
  for (uint32_t size = 2; size <= kTopKMax; size <<= 1)
    for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
      const uint32_t j = t ^ stride;
      if (j > t) {
        const unsigned long long a = cand[t], b = cand[j];
        const bool desc = (t & size) == 0;
        if (desc ? a < b : a > b) { cand[t] = b; cand[j] = a; }
      }
      __syncthreads();
    }
  // ---- the chain over the sorted candidates
  if (t < k) kept[t] = key_value((uint32_t)(cand[t] >> 32));
  __syncthreads();
  if (cf.flags & 1u) {  // top_p
    cand_softmax(kept, k, pr, e, tab);
    if (t == 0) {
      double cum = 0.0;
      for (uint32_t j = 0; j < k; ++j) {
        if (cum > (double)cf.top_p) kept[j] = -INFINITY;
        cum += (double)pr[j];
      }
    }
    __syncthreads();
  }
  if (cf.flags & 2u) {  // min_p, against the largest candidate
    const float cut = kept[0] + cf.log_min_p;
    __syncthreads();
    if (t < k && kept[t] < cut) kept[t] = -INFINITY;
    __syncthreads();
  }
  if (cf.flags & 4u) {  // temperature
    if (t < k && kept[t] > -INFINITY && kept[t] < INFINITY) kept[t] *= cf.inv_t;
    __syncthreads();
  }
  cand_softmax(kept, k, pr, e, tab);
  if (t == 0) {
    double cum = 0.0;
    uint32_t ch = k - 1;
    for (uint32_t j = 0; j < k; ++j) {
      cum += (double)pr[j];
      if (cum >= (double)u) { ch = j; break; }
    }
    s_ch = ch;
  }
  __syncthreads();
  return ~(uint32_t)(cand[s_ch] & 0xFFFFFFFFull);
}

// k_sample_cols for rows of many logits, spread over kSampChunks workgroups
// per row (grid (chunk c, row)): each sums its chunk's softmax numerators
// (the weights k_sample_cols sums, in f64) and stores the sum at agent scope;
// the last workgroup of the row to arrive (a counter zeroed by k_row_part,
// reset by that workgroup) scans the chunk sums in vocab order for the first
// chunk whose running sum reaches u * total and draws inside it, as
// k_sample_cols does over the whole row (first v whose running sum reaches
// u * total).
constexpr uint32_t kSampChunks = 64;
__global__ __launch_bounds__(256) void k_sample_chunks(const float* __restrict__ p, const double2* __restrict__ part,
                                                       uint32_t nch, uint32_t V, double inv_t, const float* u_dev,
                                                       uint64_t seed, uint64_t word0, uint64_t wstride,
                                                       double2* __restrict__ csum, uint32_t* __restrict__ cnt,
                                                       uint32_t* __restrict__ out, const uint64_t* rng) {
  static_assert(kSampChunks == 64, "one lane per chunk");
  constexpr int kPer = 8;  // elements per thread per pass
  __shared__ double tab[64];
  __shared__ double2 st;
  __shared__ double shd[4];
  __shared__ uint32_t s_last, s_c;
  __shared__ double s_off, s_target;
  const uint32_t c = blockIdx.x, row = blockIdx.y, t = threadIdx.x;
  rng_from_dev(rng, seed, word0);
  load_exp_table(tab);
  __syncthreads();
  if (t < 64) {
    const double2 s2 = wave_row_stat(part + (size_t)row * nch, nch, inv_t, tab);
    if (t == 0) st = s2;
  }
  __syncthreads();
  const float* pr = p + (size_t)row * V;
  const RowW rw{pr, nullptr, st.x, 1.0, 0.0, 1.0, inv_t, tab};
  const uint32_t CH = (V + kSampChunks - 1) / kSampChunks, lo = min(c * CH, V), hi = min(lo + CH, V);
  double ps = 0.0;
  for (uint32_t v0 = lo; v0 < hi; v0 += 256 * kPer) {
    float x[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const uint32_t v = v0 + j * 256 + t;
      x[j] = v < hi ? pr[v] : -INFINITY;
    }
#pragma unroll
    for (int j = 0; j < kPer; ++j) ps += rw.num(x[j]);
  }
  ps = block_sum_d(ps, shd);
  if (t == 0) {
    sh_st_coh16(csum + (size_t)row * kSampChunks + c, sh_pack_d2(ps, 0.0));
    sh_stores_done();
    uint32_t* cr = cnt + (size_t)row * kCntStride;
    const uint32_t old = __hip_atomic_fetch_add(cr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t last = old + 1 == kSampChunks;
    if (last) __hip_atomic_store(cr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = last;
  }
  __syncthreads();
  if (!s_last) return;  // uniform in the workgroup
  if (t < 64) {
    sh_f4v cv = sh_ld_coh16(csum + (size_t)row * kSampChunks + t);
    sh_coh_wait(cv);
    double w, unused;
    sh_unpack_d2(cv, w, unused);
    double inc = w;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const double y = __shfl_up(inc, off);
      if (t >= (uint32_t)off) inc += y;
    }
    const double total = __shfl(inc, 63);
    const double target = (double)uniform_at(u_dev, seed, word0 + wstride * row) * total;
    const unsigned long long over = __ballot(inc >= target);
    const uint32_t cs = over ? (uint32_t)__builtin_ctzll(over) : 63u;
    double ex = __shfl_up(inc, 1);
    if (t == 0) ex = 0.0;
    ex = __shfl(ex, cs);
    if (t == 0) {
      s_c = cs;
      s_off = ex;
      s_target = target;
    }
  }
  __syncthreads();
  const uint32_t plo = min(s_c * CH, V), phi = min(plo + CH, V);
  const uint32_t tok = wg_inverse_cdf(rw, plo, phi, false, 0.f, s_off, s_target, true, nullptr);
  if (t == 0) out[row] = tok;
}

// COMPARE with filters: row r of p draws with Philox word word0 + wstride r
// (or explicit u_dev[...]), as k_sample_cols.
__global__ __launch_bounds__(256) void k_sample_filtered_cols(const float* __restrict__ p, uint32_t V, FiltCfg cf,
                                                              const float* u_dev, uint64_t seed, uint64_t word0,
                                                              uint64_t wstride, uint32_t* __restrict__ out,
                                                              const uint64_t* rng) {
  __shared__ double tab[64];
  const uint32_t row = blockIdx.x;
  rng_from_dev(rng, seed, word0);
  load_exp_table(tab);
  __syncthreads();
  const float u = uniform_at(u_dev, seed, word0 + wstride * row);
  const uint32_t tok = sample_filtered_row(p + (size_t)row * V, V, cf, u, tab);
  if (threadIdx.x == 0) out[row] = tok;
}

// Batched verify rows with filters (rows[r].top_k > 0); other rows are left alone.
__global__ __launch_bounds__(256) void k_sample_filtered_tab(const float* __restrict__ p, uint32_t V,
                                                             const SampRow* __restrict__ rows,
                                                             uint32_t* __restrict__ out) {
  __shared__ double tab[64];
  const uint32_t row = blockIdx.x;
  const SampRow sr = rows[row];
  if (sr.greedy || sr.top_k == 0) return;  // uniform
  load_exp_table(tab);
  __syncthreads();
  const FiltCfg cf{sr.top_k, sr.top_p, sr.log_min_p, sr.inv_t_f, sr.filt_flags};
  const float u = sr.explicit_u ? sr.u : uniform_at(nullptr, sr.seed, sr.word);
  const uint32_t tok = sample_filtered_row(p + (size_t)row * V, V, cf, u, tab);
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

constexpr uint32_t kDrawChunks = 64;  // vocab chunks of the REJECTION draw

// REJECTION, step 2: one workgroup per sequence b combines the statistics of
// b's 2k + 1 rows (one lane per row), finds the first rejected draft i (k when
// all are accepted; draft i is accepted iff u_acc q_i(d_i) < p_i(d_i)) and
// records i with the statistics of p_i and q_i.
__global__ __launch_bounds__(256) void k_decide_reject(const float* __restrict__ p, const float* __restrict__ q,
                                                       const double2* __restrict__ part, uint32_t nch, uint32_t B,
                                                       uint32_t k, uint32_t V, double inv_t,
                                                       const uint32_t* __restrict__ drafts, const float* u_dev,
                                                       uint64_t seed, uint64_t counter,
                                                       uint32_t* __restrict__ first_rej,
                                                       double2* __restrict__ rstat, double* __restrict__ probs,
                                                       const uint64_t* rng) {
  __shared__ double tab[64];
  __shared__ double2 st[129];  // p rows 0..k, then q rows 0..k-1 (k <= 64)
  __shared__ uint32_t fr;
  const uint32_t b = blockIdx.x, t = threadIdx.x;
  rng_from_dev(rng, seed, counter);
  load_exp_table(tab);
  if (t == 0) fr = k;
  // the draft token's logits for the accept test (lane t < k), loaded with the partials
  uint32_t d = 0;
  float pl = 0.f, ql = 0.f;
  if (t < k) {
    d = drafts[b * k + t];
    if (d < V) {
      pl = p[((size_t)b * (k + 1) + t) * V + d];
      ql = q[((size_t)b * k + t) * V + d];
    }
  }
  __syncthreads();  // table
  if (t < 2 * k + 1) {
    const size_t grow = t <= k ? (size_t)b * (k + 1) + t : (size_t)B * (k + 1) + (size_t)b * k + (t - k - 1);
    st[t] = lane_row_stat(part + grow * nch, nch, inv_t, tab);
  }
  __syncthreads();
  if (t < k) {
    bool accept = false;
    if (d < V) {  // an out-of-vocab draft id is rejected
      const double2 sp = st[t], sq = st[k + 1 + t];
      const double pd = sh_exp_neg(((double)pl - sp.x) * inv_t, tab) / sp.y;
      const double qd = sh_exp_neg(((double)ql - sq.x) * inv_t, tab) / sq.y;
      const float ua = uniform_at(u_dev, seed, counter + 2ull * (b * (k + 1) + t));
      accept = (double)ua * qd < pd;
      if (probs) {  // p_t(d), q_t(d), accept probability min(1, p/q)
        double* o = probs + 3 * ((size_t)b * k + t);
        o[0] = pd;
        o[1] = qd;
        o[2] = qd > 0.0 ? fmin(1.0, pd / qd) : (pd > 0.0 ? 1.0 : 0.0);
      }
    } else if (probs) {
      double* o = probs + 3 * ((size_t)b * k + t);
      o[0] = o[1] = o[2] = 0.0;
    }
    if (!accept) atomicMin(&fr, t);
  }
  __syncthreads();
  if (t == 0) {
    const uint32_t i = fr;
    first_rej[b] = i;
    rstat[2 * b] = st[i];
    rstat[2 * b + 1] = i < k ? st[k + 1 + i] : make_double2(0.0, 1.0);
  }
}

// Step 3: grid (chunk, sequence): sums of the draw weights of row i = first_rej
// over the chunk: .x the residual max(0, p_i - q_i) (i < k only), .y the
// softmax numerator of p_i (the draw when all are accepted or the residual is
// all zero).
__global__ __launch_bounds__(256) void k_draw_chunks(const float* __restrict__ p, const float* __restrict__ q,
                                                     uint32_t k, uint32_t V, double inv_t,
                                                     const uint32_t* __restrict__ first_rej,
                                                     const double2* __restrict__ rstat,
                                                     double2* __restrict__ chunk) {
  constexpr int kPer = 8;  // elements per thread per pass
  __shared__ double tab[64];
  __shared__ double shd[4];
  const uint32_t c = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
  load_exp_table(tab);
  const uint32_t i = first_rej[b];
  const double2 sp = rstat[2 * b], sq = rstat[2 * b + 1];
  const bool resid = i < k;
  const uint32_t CH = (V + kDrawChunks - 1) / kDrawChunks, lo = min(c * CH, V), hi = min(lo + CH, V);
  const float* pr = p + ((size_t)b * (k + 1) + i) * V;
  const float* qr = resid ? q + ((size_t)b * k + i) * V : pr;
  __syncthreads();  // table
  // the same weights as the pick's scan (RowW): the p numerator once per
  // element, the residual from it
  const RowW rres{pr, qr, sp.x, 1.0 / sp.y, sq.x, 1.0 / sq.y, inv_t, tab};
  double rs = 0.0, ps = 0.0;
  for (uint32_t v0 = lo; v0 < hi; v0 += 256 * kPer) {
    float2 x[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const uint32_t v = v0 + j * 256 + t;
      x[j] = make_float2(v < hi ? pr[v] : -INFINITY, v < hi && resid ? qr[v] : -INFINITY);
    }
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const double a = rres.num(x[j].x);
      ps += a;
      if (resid) rs += rres.resid(a, x[j].y);
    }
  }
  rs = block_sum_d(rs, shd);
  ps = block_sum_d(ps, shd);
  if (t == 0) chunk[(size_t)b * kDrawChunks + c] = make_double2(rs, ps);
}

// Step 4: one workgroup per sequence draws the next token: wave 0 scans the
// chunk sums (residual, else p) in vocab order for target = u * total, then
// the inverse CDF inside the crossing chunk. Without a crossing (rounding at
// the end) the last chunk's scan falls back to V - 1, as the sequential draw.
__global__ __launch_bounds__(256) void k_draw_pick(const float* __restrict__ p, const float* __restrict__ q,
                                                   uint32_t k, uint32_t V, double inv_t,
                                                   const uint32_t* __restrict__ first_rej,
                                                   const double2* __restrict__ rstat,
                                                   const double2* __restrict__ chunk, const float* u_dev,
                                                   uint64_t seed, uint64_t counter, uint32_t* __restrict__ acc_len,
                                                   uint32_t* __restrict__ next_tok, const uint64_t* rng) {
  static_assert(kDrawChunks == 64, "one lane per chunk");
  __shared__ double tab[64];
  __shared__ uint32_t s_c;
  __shared__ double s_off, s_target;
  __shared__ int s_use_r;
  const uint32_t b = blockIdx.x, t = threadIdx.x, i = first_rej[b];
  rng_from_dev(rng, seed, counter);
  load_exp_table(tab);
  const double2 sp = rstat[2 * b], sq = rstat[2 * b + 1];
  if (t < 64) {
    const double2 cw = chunk[(size_t)b * kDrawChunks + t];
    const int use_r = i < k && wave_sum_d(cw.x) > 0.0;
    const double w = use_r ? cw.x : cw.y;
    double inc = w;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const double y = __shfl_up(inc, off);
      if (t >= (uint32_t)off) inc += y;
    }
    const double total = __shfl(inc, 63);
    const float u = uniform_at(u_dev, seed, counter + 2ull * (b * (k + 1) + i) + 1ull);
    const double target = (double)u * total;
    const unsigned long long over = __ballot(inc > target);
    const uint32_t cs = over ? (uint32_t)__builtin_ctzll(over) : 63u;
    double ex = __shfl_up(inc, 1);
    if (t == 0) ex = 0.0;
    ex = __shfl(ex, cs);
    if (t == 0) {
      s_c = cs;
      s_off = ex;
      s_target = target;
      s_use_r = use_r;
    }
  }
  __syncthreads();
  const uint32_t CH = (V + kDrawChunks - 1) / kDrawChunks, lo = min(s_c * CH, V), hi = min(lo + CH, V);
  const float* pr = p + ((size_t)b * (k + 1) + i) * V;
  RowW rw{pr, s_use_r ? q + ((size_t)b * k + i) * V : nullptr, sp.x, 1.0 / sp.y, sq.x, 1.0 / sq.y, inv_t, tab};
  const uint32_t tok = wg_inverse_cdf(rw, lo, hi, false, 0.f, s_off, s_target, false, nullptr);
  if (t == 0) {
    acc_len[b] = i;
    next_tok[b] = tok;
  }
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
  __shared__ double tab[64];
  const uint32_t b = blockIdx.x, t = threadIdx.x;
  load_exp_table(tab);  // the first use follows the barriers of block_max_f
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
        const unsigned long long k = sh_amax_key(pv[i], i);
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
      const uint32_t am = sh_amax_index(best);
      for (uint32_t c = v + 1; c < n && acc < 0; ++c)
        if (par[c] == (int32_t)v && tok[c] == am) acc = (int)c;
      if (acc < 0) { out_tok = am; break; }
    } else {
      float mx = -INFINITY;
      for (uint32_t i = t; i < V; i += 256) mx = fmaxf(mx, pv[i]);
      const double pm = block_max_f(mx, shf);
      double ssum = 0.0;
      for (uint32_t i = t; i < V; i += 256) ssum += sh_exp_neg(((double)pv[i] - pm) * inv_t, tab);
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
          for (uint32_t i = t; i < V; i += 256) qsum += sh_exp_neg(((double)qv[i] - qm) * inv_t, tab);
          qs = block_sum_d(qsum, shd);
          have_q = true;
        }
        if (t == 0) {
          const uint32_t tc = tok[c];
          bool ok = false;
          if (tc < V) {
            const double pc = resid ? r[tc] / Z : sh_exp_neg(((double)pv[tc] - pm) * inv_t, tab) / ps;
            const double qc = sh_exp_neg(((double)qv[tc] - qm) * inv_t, tab) / qs;
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
          const double cur = resid ? r[i] / Z : sh_exp_neg(((double)pv[i] - pm) * inv_t, tab) / ps;
          const double d = cur - sh_exp_neg(((double)qv[i] - qm) * inv_t, tab) / qs;
          part += d > 0.0 ? d : 0.0;
        }
        const double R = block_sum_d(part, shd);
        if (R > 0.0) {
          for (uint32_t i = t; i < V; i += 256) {
            const double cur = resid ? r[i] / Z : sh_exp_neg(((double)pv[i] - pm) * inv_t, tab) / ps;
            const double d = cur - sh_exp_neg(((double)qv[i] - qm) * inv_t, tab) / qs;
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
          out_tok = wg_inverse_cdf(rr, 0, V, true, ud, 0.0, 0.0, false, nullptr);
        } else {
          RowW rw{pv, nullptr, pm, 1.0, 0.0, 1.0, inv_t, tab};
          out_tok = wg_inverse_cdf(rw, 0, V, true, ud, 0.0, 0.0, false, nullptr);
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

// ---------------------------------------------------------------- tree REJECTION (multi-workgroup)

// The same walk as k_tree_accept in REJECTION mode, with every full-vocab
// reduction spread over kDrawChunks workgroups per tree. The residual after
// m effective rejections at node v is never stored: cur_m(x) is recomputed
// pointwise from the stored normalizers Z_1..Z_m with the operations of the
// stored form (cur = r / Z, d = cur - q(x), r = max(d, 0)), so each value is
// the one k_tree_accept would hold. A step is k_tree_step (one workgroup per
// tree: finish the previous pass, then accept tests until the next pass is
// needed) followed by k_tree_pass (chunk sums of that pass).
enum : uint32_t { TS_WALK = 0, TS_ZPASS = 1, TS_DRAW = 2, TS_DONE = 3 };
struct TreeState {
  uint32_t v, len, mode, next, m, tok;
  double Z[64];        // normalizers of the effective rejections at v
  uint32_t path[64];
};

// Current distribution at a node: cur_m, the next residual summand and the
// draw weight (softmax numerator without rejections, else the unnormalized
// residual r_m).
struct TreeCur {
  double pm, ps, qm, qs, inv_t;
  const double* Z;
  uint32_t m;
  const double* tab;
  __device__ __forceinline__ double qprob(float qx) const { return sh_exp_neg(((double)qx - qm) * inv_t, tab) / qs; }
  __device__ __forceinline__ double cur(float px, float qx) const {
    double c = sh_exp_neg(((double)px - pm) * inv_t, tab) / ps;
    if (m == 0) return c;
    const double qp = qprob(qx);
    for (uint32_t j = 0; j < m; ++j) {
      const double d = c - qp;
      c = (d > 0.0 ? d : 0.0) / Z[j];
    }
    return c;
  }
  __device__ __forceinline__ double resid_next(float px, float qx) const {
    const double d = cur(px, qx) - qprob(qx);
    return d > 0.0 ? d : 0.0;
  }
  __device__ __forceinline__ double draw_w(float px, float qx) const {
    if (m == 0) return sh_exp_neg(((double)px - pm) * inv_t, tab);
    double c = sh_exp_neg(((double)px - pm) * inv_t, tab) / ps, r = 0.0;
    const double qp = qprob(qx);
    for (uint32_t j = 0; j < m; ++j) {
      const double d = c - qp;
      r = d > 0.0 ? d : 0.0;
      c = r / Z[j];
    }
    return r;
  }
};

struct TreeDrawW {  // RowW-style access for wg_inverse_cdf
  const float* p;
  const float* q;
  TreeCur tc;
  using Raw = float2;
  __device__ __forceinline__ Raw raw(uint32_t v) const { return make_float2(p[v], tc.m ? q[v] : 0.f); }
  __device__ __forceinline__ double wt(Raw x) const { return tc.draw_w(x.x, x.y); }
};

// Statistics of node v of tree b: p row b n + v, q row B n + b n + v.
__device__ __forceinline__ TreeCur tree_cur(const double2* part, uint32_t nch, uint32_t B, uint32_t n, uint32_t b,
                                            uint32_t v, double inv_t, const double* Z, uint32_t m, const double* tab) {
  const double2 sp = lane_row_stat(part + ((size_t)b * n + v) * nch, nch, inv_t, tab);
  const double2 sq = lane_row_stat(part + ((size_t)B * n + (size_t)b * n + v) * nch, nch, inv_t, tab);
  return TreeCur{sp.x, sp.y, sq.x, sq.y, inv_t, Z, m, tab};
}

__global__ __launch_bounds__(256) void k_tree_step(const float* __restrict__ p, const float* __restrict__ q,
                                                   const uint32_t* __restrict__ tokens,
                                                   const int32_t* __restrict__ parents, uint32_t B, uint32_t n,
                                                   uint32_t V, double inv_t, const double2* __restrict__ part,
                                                   uint32_t nch, const float* u_dev, uint64_t seed, uint64_t counter,
                                                   TreeState* __restrict__ state, const double* __restrict__ chunk,
                                                   int first, uint32_t* __restrict__ path_out,
                                                   uint32_t* __restrict__ path_len, uint32_t* __restrict__ next_tok) {
  __shared__ double tab[64];
  __shared__ TreeState s;
  __shared__ TreeCur sc;
  __shared__ uint32_t s_c;
  __shared__ double s_off, s_target;
  const uint32_t b = blockIdx.x, t = threadIdx.x;
  load_exp_table(tab);
  const float* P = p + (size_t)b * n * V;
  const float* Q = q + (size_t)b * n * V;
  if (t == 0) {
    if (first) {
      s.v = 0; s.len = 1; s.mode = TS_WALK; s.next = 1; s.m = 0; s.tok = 0; s.path[0] = 0;
    } else {
      s = state[b];
    }
  }
  __syncthreads();
  if (s.mode == TS_DRAW) {  // draw sums are in: pick the chunk, then the inverse CDF inside it
    if (t == 0) {
      sc = tree_cur(part, nch, B, n, b, s.v, inv_t, s.Z, s.m, tab);
      const double* ch = chunk + (size_t)b * kDrawChunks;
      double total = 0.0;
      for (uint32_t c = 0; c < kDrawChunks; ++c) total += ch[c];
      const float u = uniform_at(u_dev, seed, counter + 2ull * ((uint64_t)b * n + s.v) + 1ull);
      const double target = (double)u * total;
      double off = 0.0;
      uint32_t cs = kDrawChunks - 1;
      for (uint32_t c = 0; c + 1 < kDrawChunks; ++c) {
        if (off + ch[c] > target) { cs = c; break; }
        off += ch[c];
      }
      s_c = cs; s_off = off; s_target = target;
    }
    __syncthreads();
    const uint32_t CH = (V + kDrawChunks - 1) / kDrawChunks, lo = min(s_c * CH, V), hi = min(lo + CH, V);
    TreeCur tc = sc;
    tc.Z = s.Z;
    const TreeDrawW w{P + (size_t)s.v * V, Q + (size_t)s.v * V, tc};
    const uint32_t tok = wg_inverse_cdf(w, lo, hi, false, 0.f, s_off, s_target, false, nullptr);
    if (t == 0) { s.tok = tok; s.mode = TS_DONE; }
  } else if (t == 0 && s.mode == TS_ZPASS) {  // residual sum is in
    const double* ch = chunk + (size_t)b * kDrawChunks;
    double R = 0.0;
    for (uint32_t c = 0; c < kDrawChunks; ++c) R += ch[c];
    if (R > 0.0) s.Z[s.m++] = R;
    s.mode = TS_WALK;
  }
  if (t == 0) {
    const uint32_t* tok = tokens + (size_t)b * n;
    const int32_t* par = parents + (size_t)b * n;
    while (s.mode == TS_WALK) {
      uint32_t c = s.next;
      while (c < n && par[c] != (int32_t)s.v) ++c;
      if (c >= n) { s.mode = TS_DRAW; break; }
      const TreeCur tc = tree_cur(part, nch, B, n, b, s.v, inv_t, s.Z, s.m, tab);
      const uint32_t x = tok[c];
      bool ok = false;
      if (x < V) {
        const float* pv = P + (size_t)s.v * V;
        const float* qv = Q + (size_t)s.v * V;
        const double pc = tc.cur(pv[x], qv[x]), qc = tc.qprob(qv[x]);
        ok = (double)uniform_at(u_dev, seed, counter + 2ull * ((uint64_t)b * n + c)) * qc < pc;
      }
      if (ok) {
        s.v = c; s.path[s.len++] = c; s.m = 0; s.next = c + 1;
      } else {
        s.next = c + 1;
        s.mode = TS_ZPASS;
      }
    }
    state[b] = s;
    if (s.mode == TS_DONE) {
      for (uint32_t i = 0; i < s.len; ++i) path_out[(size_t)b * n + i] = s.path[i];
      path_len[b] = s.len;
      next_tok[b] = s.tok;
    }
  }
}

// Chunk sums of the pass each tree asked for: residual summands (TS_ZPASS) or
// draw weights (TS_DRAW) over chunk blockIdx.x of node v's vocabulary.
__global__ __launch_bounds__(256) void k_tree_pass(const float* __restrict__ p, const float* __restrict__ q,
                                                   uint32_t B, uint32_t n, uint32_t V, double inv_t,
                                                   const double2* __restrict__ part, uint32_t nch,
                                                   const TreeState* __restrict__ state, double* __restrict__ chunk) {
  __shared__ double tab[64];
  __shared__ double shd[4];
  __shared__ TreeCur sc;
  __shared__ double sZ[64];
  const uint32_t c = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
  const uint32_t mode = state[b].mode;
  if (mode != TS_ZPASS && mode != TS_DRAW) return;  // uniform in the workgroup
  load_exp_table(tab);
  const uint32_t v = state[b].v, m = state[b].m;
  if (t < m) sZ[t] = state[b].Z[t];
  __syncthreads();
  if (t == 0) sc = tree_cur(part, nch, B, n, b, v, inv_t, sZ, m, tab);
  __syncthreads();
  const TreeCur tc = sc;
  const float* pv = p + ((size_t)b * n + v) * V;
  const float* qv = q + ((size_t)b * n + v) * V;
  const uint32_t CH = (V + kDrawChunks - 1) / kDrawChunks, lo = min(c * CH, V), hi = min(lo + CH, V);
  double acc = 0.0;
  for (uint32_t x0 = lo; x0 < hi; x0 += 256 * 8) {
    float2 xv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t x = x0 + j * 256 + t;
      xv[j] = x < hi ? make_float2(pv[x], qv[x]) : make_float2(-INFINITY, -INFINITY);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (x0 + j * 256 + t < hi) acc += mode == TS_ZPASS ? tc.resid_next(xv[j].x, xv[j].y) : tc.draw_w(xv[j].x, xv[j].y);
  }
  acc = block_sum_d(acc, shd);
  if (t == 0) chunk[(size_t)b * kDrawChunks + c] = acc;
}

}  // namespace

// Rows of at least this many logits draw through k_sample_chunks.
constexpr uint32_t kChunkedMinV = 8192;
static size_t round256(size_t b) { return (b + 255) / 256 * 256; }
// The chunked draw's chunk sums and arrival counters for nrows rows.
static size_t chunked_bytes(uint32_t nrows) {
  return round256((size_t)nrows * kSampChunks * sizeof(double2)) + (size_t)nrows * kCntStride * 4;
}

size_t sh_accept_scratch_bytes(uint32_t B, uint32_t k, uint32_t V, uint32_t mode) {
  const uint32_t n_p = B * (k + 1), n_q = mode == SH_SAMPLE_REJECTION ? B * k : 0;
  const uint32_t nch = (V + 256 * kStatE - 1) / (256 * kStatE);
  const size_t part_b = (size_t)(n_p + n_q) * nch * sizeof(double2);
  const size_t chunk_b = (size_t)B * kDrawChunks * sizeof(double2), rstat_b = (size_t)B * 2 * sizeof(double2);
  const size_t small_b = mode == SH_SAMPLE_COMPARE ? (size_t)n_p * 4 : (size_t)B * 4;
  const size_t samp_b = mode == SH_SAMPLE_COMPARE && V >= kChunkedMinV ? chunked_bytes(n_p) : 0;
  return round256(part_b + chunk_b + rstat_b + round256(small_b)) + samp_b;
}

size_t sh_sample_rows_scratch_bytes(uint32_t nrows, uint32_t V) {
  const uint32_t nch = (V + 256 * kStatE - 1) / (256 * kStatE);
  return round256((size_t)nrows * nch * sizeof(double2)) + (V >= kChunkedMinV ? chunked_bytes(nrows) : 0);
}

// COMPARE draws of nrows rows of p: over the whole row per workgroup, or for
// wide rows in kSampChunks chunks per row (scratch at samp: chunked_bytes).
static void launch_sample_cols(sh_engine* e, const float* p, const double2* part, uint32_t nch, uint32_t nrows,
                               uint32_t V, double inv_t, const float* u_dev, uint64_t seed, uint64_t word0,
                               uint64_t wstride, char* samp, uint32_t* out, const uint64_t* rng) {
  if (V >= kChunkedMinV) {
    double2* csum = reinterpret_cast<double2*>(samp);
    uint32_t* cnt = reinterpret_cast<uint32_t*>(samp + round256((size_t)nrows * kSampChunks * sizeof(double2)));
    hipLaunchKernelGGL(k_sample_chunks, dim3(kSampChunks, nrows), dim3(256), 0, e->stream, p, part, nch, V, inv_t,
                       u_dev, seed, word0, wstride, csum, cnt, out, rng);
  } else {
    hipLaunchKernelGGL(k_sample_cols, dim3(nrows), dim3(256), 0, e->stream, p, part, nch, V, inv_t, u_dev, seed,
                       word0, wstride, out, rng);
  }
}
// The counters k_row_part zeroes for launch_sample_cols (null: none).
static uint32_t* sample_cols_cnt(char* samp, uint32_t nrows, uint32_t V) {
  return V >= kChunkedMinV ? reinterpret_cast<uint32_t*>(samp + round256((size_t)nrows * kSampChunks *
                                                                                sizeof(double2)))
                           : nullptr;
}

int sh_accept_launch(sh_engine* e, const float* p_logits, const float* q_logits, const uint32_t* drafts, uint32_t B,
                     uint32_t k, uint32_t V, const sh_sampling* s, uint64_t counter, const float* uniforms_dev,
                     uint32_t* acc_len, uint32_t* next_tok, void* scratch_in, double* probs_out,
                     const uint64_t* rng_dev) {
  SH_CHECK(B >= 1 && k >= 1 && k <= 64 && V >= 1, SH_ERR_ARG, "accept: B=%u k=%u V=%u", B, k, V);
  const uint32_t mode = s->mode;
  SH_CHECK(mode == SH_SAMPLE_COMPARE || mode == SH_SAMPLE_REJECTION, SH_ERR_ARG, "accept: mode %u", mode);
  SH_CHECK(s->temperature > 0.f, SH_ERR_ARG, "accept: temperature must be > 0");
  SH_CHECK(mode != SH_SAMPLE_REJECTION || q_logits, SH_ERR_ARG, "REJECTION needs draft logits");
  SampRow filt{};
  if (int rc = sh_samprow_filters(*s, V, filt)) return rc;
  SH_CHECK(!filt.top_k || mode == SH_SAMPLE_COMPARE, SH_ERR_UNSUPPORTED,
           "candidate filters (top_k / top_p / min_p) apply to COMPARE only");
  const double inv_t = 1.0 / (double)s->temperature;
  const uint32_t n_p = B * (k + 1), n_q = mode == SH_SAMPLE_REJECTION ? B * k : 0;
  const uint32_t nch = (V + 256 * kStatE - 1) / (256 * kStatE), nrows = n_p + n_q;
  // one scratch block: unit partials, then per-sequence draw state
  const uint32_t nunits = nrows * nch;
  const size_t part_b = (size_t)nunits * sizeof(double2);
  const size_t chunk_b = (size_t)B * kDrawChunks * sizeof(double2), rstat_b = (size_t)B * 2 * sizeof(double2);
  char* sbuf = static_cast<char*>(scratch_in);
  if (!sbuf) {
    if (int rc = sh_engine_scratch(e, SCR_ACCEPT, sh_accept_scratch_bytes(B, k, V, mode), (void**)&sbuf)) return rc;
  }
  double2* part = reinterpret_cast<double2*>(sbuf);
  double2* chunk = reinterpret_cast<double2*>(sbuf + part_b);
  double2* rstat = reinterpret_cast<double2*>(sbuf + part_b + chunk_b);
  uint32_t* small = reinterpret_cast<uint32_t*>(sbuf + part_b + chunk_b + rstat_b);
  const size_t small_b = mode == SH_SAMPLE_COMPARE ? (size_t)n_p * 4 : (size_t)B * 4;
  char* samp = sbuf + round256(part_b + chunk_b + rstat_b + round256(small_b));  // the chunked COMPARE draw
  uint32_t* zc = mode == SH_SAMPLE_COMPARE ? sample_cols_cnt(samp, n_p, V) : nullptr;
  hipEvent_t ev = nullptr;
  sh_prof_begin(e, &ev);
  if (filt.top_k) {  // the filtered draw reads its rows itself
  } else if (V % 4 == 0) {
    hipLaunchKernelGGL((k_row_part<true, kStatE>), dim3(nunits), dim3(256), 0, e->stream, p_logits, n_p, q_logits,
                       V, inv_t, nch, part, nullptr, zc, n_p);
  } else {
    hipLaunchKernelGGL((k_row_part<false, kStatE>), dim3(nunits), dim3(256), 0, e->stream, p_logits, n_p, q_logits,
                       V, inv_t, nch, part, nullptr, zc, n_p);
  }
  SH_HIP(hipGetLastError());
  sh_prof_end(e, "accept_stats", 4.0 * V * (n_p + n_q), ev);
  sh_prof_begin(e, &ev);
  if (mode == SH_SAMPLE_COMPARE && filt.top_k) {
    const FiltCfg cf{filt.top_k, filt.top_p, filt.log_min_p, filt.inv_t_f, filt.filt_flags};
    hipLaunchKernelGGL(k_sample_filtered_cols, dim3(n_p), dim3(256), 0, e->stream, p_logits, V, cf, uniforms_dev,
                       s->seed, counter + 1ull, 2ull, small, rng_dev);
    hipLaunchKernelGGL(k_decide_compare, dim3((B + 63) / 64), dim3(64), 0, e->stream, small, drafts, B, k, acc_len,
                       next_tok);
  } else if (mode == SH_SAMPLE_COMPARE) {
    launch_sample_cols(e, p_logits, part, nch, n_p, V, inv_t, uniforms_dev, s->seed, counter + 1ull, 2ull, samp,
                       small, rng_dev);
    hipLaunchKernelGGL(k_decide_compare, dim3((B + 63) / 64), dim3(64), 0, e->stream, small, drafts, B, k, acc_len,
                       next_tok);
  } else {
    hipLaunchKernelGGL(k_decide_reject, dim3(B), dim3(256), 0, e->stream, p_logits, q_logits, part, nch, B, k, V,
                       inv_t, drafts, uniforms_dev, s->seed, counter, small, rstat, probs_out, rng_dev);
    hipLaunchKernelGGL(k_draw_chunks, dim3(kDrawChunks, B), dim3(256), 0, e->stream, p_logits, q_logits, k, V, inv_t,
                       small, rstat, chunk);
    hipLaunchKernelGGL(k_draw_pick, dim3(B), dim3(256), 0, e->stream, p_logits, q_logits, k, V, inv_t, small, rstat,
                       chunk, uniforms_dev, s->seed, counter, acc_len, next_tok, rng_dev);
  }
  SH_HIP(hipGetLastError());
  sh_prof_end(e, "accept_decide", 0.0, ev);
  return SH_OK;
}

int sh_sample_rows_launch(sh_engine* e, const float* logits, uint32_t nrows, uint32_t V, float T, const float* u_dev,
                          uint64_t seed, uint64_t word0, uint64_t wstride, void* scratch, size_t scratch_bytes,
                          uint32_t* out, const uint64_t* rng_dev) {
  SH_CHECK(nrows >= 1 && V >= 1 && T > 0.f, SH_ERR_ARG, "sample_rows: nrows=%u V=%u T=%g", nrows, V, (double)T);
  SH_CHECK(sh_sample_rows_scratch_bytes(nrows, V) <= scratch_bytes, SH_ERR_CAPACITY,
           "sample_rows: scratch of %zu bytes below %zu", scratch_bytes, sh_sample_rows_scratch_bytes(nrows, V));
  const double inv_t = 1.0 / (double)T;
  const uint32_t nch = (V + 256 * kStatE - 1) / (256 * kStatE);
  double2* part = static_cast<double2*>(scratch);
  char* samp = static_cast<char*>(scratch) + round256((size_t)nrows * nch * sizeof(double2));
  uint32_t* zc = sample_cols_cnt(samp, nrows, V);
  hipEvent_t ev = nullptr;
  sh_prof_begin(e, &ev);
  if (V % 4 == 0)
    hipLaunchKernelGGL((k_row_part<true, kStatE>), dim3(nrows * nch), dim3(256), 0, e->stream, logits, nrows,
                       nullptr, V, inv_t, nch, part, nullptr, zc, nrows);
  else
    hipLaunchKernelGGL((k_row_part<false, kStatE>), dim3(nrows * nch), dim3(256), 0, e->stream, logits, nrows,
                       nullptr, V, inv_t, nch, part, nullptr, zc, nrows);
  launch_sample_cols(e, logits, part, nch, nrows, V, inv_t, u_dev, seed, word0, wstride, samp, out, rng_dev);
  SH_HIP(hipGetLastError());
  sh_prof_end(e, "sample_rows", 4.0 * V * nrows, ev);
  return SH_OK;
}

int sh_sample_rows_tab_launch(sh_engine* e, const float* logits, uint32_t nrows, uint32_t V, const SampRow* rows_dev,
                              double2* part, uint32_t* out, bool plain, bool filtered) {
  SH_CHECK(nrows >= 1 && V >= 1, SH_ERR_ARG, "sample_rows_tab: nrows=%u V=%u", nrows, V);
  const uint32_t nch = (V + 256 * kStatE - 1) / (256 * kStatE);
  hipEvent_t ev = nullptr;
  sh_prof_begin(e, &ev);
  if (plain) {
    if (V % 4 == 0)
      hipLaunchKernelGGL((k_row_part<true, kStatE>), dim3(nrows * nch), dim3(256), 0, e->stream, logits, nrows,
                         nullptr, V, 1.0, nch, part, rows_dev);
    else
      hipLaunchKernelGGL((k_row_part<false, kStatE>), dim3(nrows * nch), dim3(256), 0, e->stream, logits, nrows,
                         nullptr, V, 1.0, nch, part, rows_dev);
    hipLaunchKernelGGL(k_sample_rows_tab, dim3(nrows), dim3(256), 0, e->stream, logits, part, nch, V, rows_dev, out);
  }
  if (filtered)
    hipLaunchKernelGGL(k_sample_filtered_tab, dim3(nrows), dim3(256), 0, e->stream, logits, V, rows_dev, out);
  SH_HIP(hipGetLastError());
  sh_prof_end(e, "sample_rows", 4.0 * V * nrows, ev);
  return SH_OK;
}

size_t sh_sample_rows_part_bytes(uint32_t nrows, uint32_t V) {
  return (size_t)nrows * ((V + 256 * kStatE - 1) / (256 * kStatE)) * sizeof(double2);
}

int sh_samprow_filters(const sh_sampling& s, uint32_t V, SampRow& r) {
  const bool top_p_on = s.top_p < 1.0f && s.top_p > 0.0f, min_p_on = s.min_p > 0.0f;
  r.top_k = 0;
  r.filt_flags = 0;
  if (s.top_k == 0) {
    SH_CHECK(!top_p_on && !min_p_on, SH_ERR_UNSUPPORTED,
             "top_p / min_p need top_k in 1..%u (the GPU chain filters sorted top_k candidates)", kTopKMax);
    return SH_OK;
  }
  const uint32_t k = s.top_k < V ? s.top_k : V;  // as the host chain (sample.rs:404-409)
  SH_CHECK(k <= kTopKMax, SH_ERR_UNSUPPORTED, "top_k %u (of V = %u) above %u", s.top_k, V, kTopKMax);
  r.top_k = k;
  r.top_p = s.top_p;
  r.log_min_p = min_p_on ? logf(s.min_p) : 0.0f;
  r.inv_t_f = 1.0f / fmaxf(s.temperature, 1e-9f);
  r.filt_flags = (top_p_on ? 1u : 0u) | (min_p_on ? 2u : 0u) | (fabsf(s.temperature - 1.0f) > 1e-9f ? 4u : 0u);
  return SH_OK;
}

extern "C" int sh_accept_sample(sh_engine* e, const float* p_logits_dev, const float* q_logits_dev,
                                const uint32_t* drafts_dev, uint32_t B, uint32_t k, uint32_t V, const sh_sampling* s,
                                uint32_t* acc_len_dev, uint32_t* next_tok_dev) {
  SH_CHECK(e && p_logits_dev && drafts_dev && s && acc_len_dev && next_tok_dev, SH_ERR_ARG,
           "sh_accept_sample: NULL argument");
  SH_CHECK(s->mode == SH_SAMPLE_COMPARE || s->mode == SH_SAMPLE_REJECTION, SH_ERR_ARG, "accept: mode %u", s->mode);
  SH_CHECK(B >= 1 && k >= 1 && k <= 64 && V >= 1, SH_ERR_ARG, "accept: B=%u k=%u V=%u", B, k, V);
  // engine scratch, reused call after call: no allocation once it has grown
  void* sbuf = nullptr;
  int rc = sh_engine_scratch(e, SCR_ACCEPT, sh_accept_scratch_bytes(B, k, V, s->mode), &sbuf);
  if (rc) return rc;
  float* udev = nullptr;
  if (s->uniforms) {
    const size_t n = (size_t)B * (k + 1) * 2;
    if ((rc = sh_engine_scratch(e, SCR_UNIFORMS, n * 4, (void**)&udev))) return rc;
    SH_HIP(hipMemcpyAsync(udev, s->uniforms, n * 4, hipMemcpyHostToDevice, e->stream));
  }
  // explicit uniforms are indexed from 0; Philox words from s->counter
  rc = sh_accept_launch(e, p_logits_dev, q_logits_dev, drafts_dev, B, k, V, s, udev ? 0 : s->counter, udev,
                        acc_len_dev, next_tok_dev, sbuf);
  if (rc) return rc;
  if (udev) SH_HIP(hipStreamSynchronize(e->stream));  // the caller may reuse its uniform array on return
  return sh_prof_flush(e);  // waits for the stream only when profiling
}

extern "C" int sh_accept_probs(sh_engine* e, const float* p_logits_dev, const float* q_logits_dev,
                               const uint32_t* drafts_dev, uint32_t B, uint32_t k, uint32_t V, float temperature,
                               double* probs_dev) {
  SH_CHECK(e && p_logits_dev && q_logits_dev && drafts_dev && probs_dev, SH_ERR_ARG,
           "sh_accept_probs: NULL argument");
  SH_CHECK(B >= 1 && k >= 1 && k <= 64 && V >= 1 && temperature > 0.f, SH_ERR_ARG,
           "accept_probs: B=%u k=%u V=%u T=%g", B, k, V, (double)temperature);
  const double inv_t = 1.0 / (double)temperature;
  const uint32_t n_p = B * (k + 1), nrows = n_p + B * k, nch = (V + 256 * kStatE - 1) / (256 * kStatE);
  const size_t part_b = (size_t)nrows * nch * sizeof(double2), rstat_b = (size_t)B * 2 * sizeof(double2);
  char* sbuf = nullptr;
  SH_HIP(hipMallocAsync((void**)&sbuf, part_b + rstat_b + (size_t)B * 4, e->stream));
  double2* part = reinterpret_cast<double2*>(sbuf);
  double2* rstat = reinterpret_cast<double2*>(sbuf + part_b);
  uint32_t* fr = reinterpret_cast<uint32_t*>(sbuf + part_b + rstat_b);
  if (V % 4 == 0)
    hipLaunchKernelGGL((k_row_part<true, kStatE>), dim3(nrows * nch), dim3(256), 0, e->stream, p_logits_dev, n_p,
                       q_logits_dev, V, inv_t, nch, part);
  else
    hipLaunchKernelGGL((k_row_part<false, kStatE>), dim3(nrows * nch), dim3(256), 0, e->stream, p_logits_dev, n_p,
                       q_logits_dev, V, inv_t, nch, part);
  // the accept tests' probabilities; the uniform (word 0 of seed 0) does not affect them
  hipLaunchKernelGGL(k_decide_reject, dim3(B), dim3(256), 0, e->stream, p_logits_dev, q_logits_dev, part, nch, B, k,
                     V, inv_t, drafts_dev, nullptr, 0ull, 0ull, fr, rstat, probs_dev, nullptr);
  const hipError_t le = hipGetLastError();
  (void)hipFreeAsync(sbuf, e->stream);
  SH_CHECK(le == hipSuccess, SH_ERR_HIP, "accept_probs launch: %s", hipGetErrorString(le));
  SH_HIP(hipStreamSynchronize(e->stream));
  return SH_OK;
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
  SH_CHECK(greedy || (s->top_k == 0 && !(s->top_p > 0.f && s->top_p < 1.f) && !(s->min_p > 0.f)),
           SH_ERR_UNSUPPORTED, "tree_accept: candidate filters (top_k / top_p / min_p) apply to COMPARE only");
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
  hipEvent_t ev = nullptr;
  sh_prof_begin(e, &ev);
  hipError_t le = hipSuccess;
  if (greedy) {
    hipLaunchKernelGGL(k_tree_accept, dim3(B), dim3(256), 0, e->stream, p_logits_dev, nullptr, tokens_dev,
                       parents_dev, n, V, 1.0, 1, udev, s->seed, udev ? 0ull : s->counter, r, path_dev, path_len_dev,
                       next_tok_dev);
    le = hipGetLastError();
  } else {
    // passes any tree can need: at most every child of every node on its path
    // rejected, plus the draw
    uint32_t max_passes = 0;
    std::vector<uint32_t> nch_node(n), acc(n);
    for (uint32_t b = 0; b < B; ++b) {
      std::fill(nch_node.begin(), nch_node.end(), 0u);
      for (uint32_t i = 1; i < n; ++i) ++nch_node[par[(size_t)b * n + i]];
      for (uint32_t i = 0; i < n; ++i) {
        acc[i] = nch_node[i] + (i ? acc[par[(size_t)b * n + i]] : 0u);
        max_passes = std::max(max_passes, acc[i] + 1);
      }
    }
    const double inv_t = 1.0 / (double)s->temperature;
    const uint32_t nch = (V + 256 * kStatE - 1) / (256 * kStatE), nrows = 2 * B * n;
    const uint64_t ctr = udev ? 0ull : s->counter;
    const size_t part_b = (size_t)nrows * nch * sizeof(double2), st_b = (size_t)B * sizeof(TreeState);
    char* sbuf = nullptr;
    SH_HIP(hipMallocAsync((void**)&sbuf, part_b + st_b + (size_t)B * kDrawChunks * sizeof(double), e->stream));
    double2* part = reinterpret_cast<double2*>(sbuf);
    TreeState* st = reinterpret_cast<TreeState*>(sbuf + part_b);
    double* chunk = reinterpret_cast<double*>(sbuf + part_b + st_b);
    if (V % 4 == 0)
      hipLaunchKernelGGL((k_row_part<true, kStatE>), dim3(nrows * nch), dim3(256), 0, e->stream, p_logits_dev,
                         B * n, q_logits_dev, V, inv_t, nch, part);
    else
      hipLaunchKernelGGL((k_row_part<false, kStatE>), dim3(nrows * nch), dim3(256), 0, e->stream, p_logits_dev,
                         B * n, q_logits_dev, V, inv_t, nch, part);
    for (uint32_t step = 0; step <= max_passes; ++step) {
      hipLaunchKernelGGL(k_tree_step, dim3(B), dim3(256), 0, e->stream, p_logits_dev, q_logits_dev, tokens_dev,
                         parents_dev, B, n, V, inv_t, part, nch, udev, s->seed, ctr, st, chunk, step == 0 ? 1 : 0,
                         path_dev, path_len_dev, next_tok_dev);
      if (step < max_passes)
        hipLaunchKernelGGL(k_tree_pass, dim3(kDrawChunks, B), dim3(256), 0, e->stream, p_logits_dev, q_logits_dev,
                           B, n, V, inv_t, part, nch, st, chunk);
    }
    le = hipGetLastError();
    (void)hipFreeAsync(sbuf, e->stream);
  }
  sh_prof_end(e, "tree_accept", 4.0 * V * B * n * (greedy ? 1 : 2), ev);
  if (udev) (void)hipFreeAsync(udev, e->stream);
  if (r) (void)hipFreeAsync(r, e->stream);
  SH_CHECK(le == hipSuccess, SH_ERR_HIP, "tree_accept launch: %s", hipGetErrorString(le));
  SH_HIP(hipStreamSynchronize(e->stream));
  return sh_prof_flush(e);
}

// ------------------------------------------------------------ no-allocation acceptance

// Device scratch of sh_accept_sample_noalloc: one array per GPU, held until
// the process ends. In host code `scratch` names a host-side stand-in, not
// device memory: every host use goes through the per-device address that
// sh_static_scratch_init takes from hipGetSymbolAddress.
constexpr size_t kStaticScratchBytes = (size_t)2 << 20;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
void* g_scratch_dev[kMaxDevices] = {};
// Per device: an event recorded after the last no-alloc call's kernels, which
// the next call's stream waits on, so calls from different streams or
// engines take the array in turn instead of racing on it.
hipEvent_t g_scratch_ev[kMaxDevices] = {};
std::mutex g_scratch_mu;
}  // namespace

int sh_static_scratch_init(int dev) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  SH_CHECK(dev >= 0 && dev < kMaxDevices, SH_ERR_ARG, "static scratch: device %d out of range", dev);
  if (g_scratch_dev[dev]) return SH_OK;
  void* ptr = nullptr;
  const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  SH_CHECK(err == hipSuccess && ptr, SH_ERR_HIP, "static scratch of device %d: hipGetSymbolAddress: %s", dev,
           hipGetErrorString(err));
  hipEvent_t ev = nullptr;
  const hipError_t eerr = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
  SH_CHECK(eerr == hipSuccess, SH_ERR_HIP, "static scratch of device %d: event: %s", dev, hipGetErrorString(eerr));
  g_scratch_ev[dev] = ev;
  g_scratch_dev[dev] = ptr;
  return SH_OK;
}

extern "C" int sh_accept_sample_noalloc(sh_engine* e, const float* p_logits_dev, const float* q_logits_dev,
                                        const uint32_t* drafts_dev, uint32_t B, uint32_t k, uint32_t V,
                                        const sh_sampling* s, uint32_t* acc_len_dev, uint32_t* next_tok_dev) {
  SH_CHECK(e && p_logits_dev && drafts_dev && s && acc_len_dev && next_tok_dev, SH_ERR_ARG,
           "sh_accept_sample_noalloc: NULL argument");
  SH_CHECK(!s->uniforms, SH_ERR_ARG, "sh_accept_sample_noalloc takes Philox uniforms only (uniforms must be NULL)");
  SH_CHECK(s->mode == SH_SAMPLE_COMPARE || s->mode == SH_SAMPLE_REJECTION, SH_ERR_ARG, "accept: mode %u", s->mode);
  SH_CHECK(B >= 1 && k >= 1 && k <= 64 && V >= 1, SH_ERR_ARG, "accept: B=%u k=%u V=%u", B, k, V);
  const size_t need = sh_accept_scratch_bytes(B, k, V, s->mode);
  SH_CHECK(need <= kStaticScratchBytes, SH_ERR_CAPACITY,
           "sh_accept_sample_noalloc: B=%u k=%u V=%u needs %zu scratch bytes, above the static %zu", B, k, V, need,
           kStaticScratchBytes);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  void* ptr = (e->device >= 0 && e->device < kMaxDevices) ? g_scratch_dev[e->device] : nullptr;
  SH_CHECK(ptr, SH_ERR_STATE, "static scratch of device %d is not set up", e->device);
  hipEvent_t ev = g_scratch_ev[e->device];
  // after the previous call's kernels, whichever stream they ran on
  SH_HIP(hipStreamWaitEvent(e->stream, ev, 0));
  // nothing in the scratch needs to start at zero: every kernel writes what it reads
  const int rc = sh_accept_launch(e, p_logits_dev, q_logits_dev, drafts_dev, B, k, V, s, s->counter, nullptr,
                                  acc_len_dev, next_tok_dev, ptr);
  if (rc) return rc;
  SH_HIP(hipEventRecord(ev, e->stream));
  return SH_OK;
}
