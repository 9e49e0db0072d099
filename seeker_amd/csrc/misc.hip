// Small per-column kernels of the verify step: embedding gather, RMSNorm fused
// with the GEMV activation operand build, and greedy per-column argmax.
#include "sh_f16.h"
#include "sh_internal.h"

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t f2hb(float x) { return __builtin_bit_cast(uint16_t, (_Float16)x); }

// ------------------------------------------------------------------ embed

// get_rows of a quantized token_embd (elementwise.rs:873, get_rows_q4_k.slang,
// get_rows_quant.slang): resid[j][i] = deq(token_embd)[tokens[j]][i], with the
// same per-element arithmetic as the Q4_K / Q8_0 dequant (run.rs:4212-4303).
__global__ void k_embed(const uint8_t* __restrict__ embd, int type, uint32_t d, size_t row_bytes,
                        const uint32_t* __restrict__ tokens, uint32_t V, float* __restrict__ resid) {
  const uint32_t j = blockIdx.x;
  uint32_t tok = tokens[j];
  if (tok >= V) tok = V - 1;  // ids are validated on the host; clamp keeps reads in bounds
  const uint8_t* row = embd + (size_t)tok * row_bytes;
  for (uint32_t i = threadIdx.x; i < d; i += blockDim.x) {
    float y;
    if (type == GGML_Q4_K) {
      const uint8_t* blk = row + (size_t)(i / 256) * 144;
      const uint32_t e = i % 256, s = e / 32, l = e % 32;
      const float dd = h2f((uint16_t)(blk[0] | blk[1] << 8));
      const float dmin = h2f((uint16_t)(blk[2] | blk[3] << 8));
      const uint8_t* sc = blk + 4;
      int scv, mv;
      if (s < 4) { scv = sc[s] & 63; mv = sc[s + 4] & 63; }
      else { scv = (sc[s + 4] & 0xF) | ((sc[s - 4] >> 6) << 4); mv = (sc[s + 4] >> 4) | ((sc[s] >> 6) << 4); }
      const uint8_t byte = blk[16 + 32 * (s / 2) + l];
      const uint32_t q = (s & 1) ? (byte >> 4) : (byte & 0xF);
      y = (dd * (float)scv) * (float)q - dmin * (float)mv;
    } else if (type == GGML_Q8_0) {
      const uint8_t* blk = row + (size_t)(i / 32) * 34;
      y = h2f((uint16_t)(blk[0] | blk[1] << 8)) * (float)(int8_t)blk[2 + i % 32];
    } else if (type == GGML_F16) {
      y = h2f(((const uint16_t*)row)[i]);
    } else {
      y = ((const float*)row)[i];
    }
    resid[(size_t)j * d + i] = y;
  }
}

int sh_embed_launch(sh_engine* e, const sh_model* m, const uint32_t* tokens, uint32_t N, float* resid) {
  hipEvent_t ev = nullptr;
  sh_prof_begin(e, &ev);
  hipLaunchKernelGGL(k_embed, dim3(N), dim3(256), 0, e->stream, m->embd_raw, m->embd_type, m->d, m->embd_row_bytes,
                     tokens, m->V, resid);
  SH_HIP(hipGetLastError());
  sh_prof_end(e, "embed", (double)N * m->embd_row_bytes, ev);
  return SH_OK;
}

// ------------------------------------------------------------------ prep

// y = x * rsqrt(mean(x^2) + eps) * w (rms_norm.slang:39-55) when w != null, else
// y = x; then y * s -> GEMV activation operand: B (hi/lo f16, [K/32][64][8]) and
// XS (per-32 sums, [K/256][64][8], lanes >= 16 stay zero), where s is the power
// of two putting max|y * s| in [2^9, 2^10); cs[col] = 1/s. One workgroup per column.
__global__ __launch_bounds__(256) void k_prep(const float* __restrict__ x, uint32_t K, const float* __restrict__ w,
                                              float eps, uint16_t* __restrict__ bx, uint16_t* __restrict__ xs,
                                              float* __restrict__ cs) {
  __shared__ float red[256];
  const uint32_t col = blockIdx.x, tid = threadIdx.x;
  const float* xc = x + (size_t)col * K;
  float scale = 1.f;
  if (w) {
    float ss = 0.f;
    for (uint32_t i = tid; i < K; i += 256) ss += xc[i] * xc[i];
    red[tid] = ss;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
      if ((int)tid < s) red[tid] += red[tid + s];
      __syncthreads();
    }
    scale = 1.0f / sqrtf(red[0] / (float)K + eps);
    __syncthreads();
  }
  float mx = 0.f;
  for (uint32_t i = tid; i < K; i += 256) mx = fmaxf(mx, fabsf(w ? xc[i] * scale * w[i] : xc[i]));
  red[tid] = mx;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if ((int)tid < s) red[tid] = fmaxf(red[tid], red[tid + s]);
    __syncthreads();
  }
  mx = red[0];
  int ex = 0;
  if (mx > 0.f && mx < INFINITY) {
    frexpf(mx, &ex);  // mx = m * 2^ex, m in [0.5, 1)
    ex = ex < -100 ? -100 : (ex > 100 ? 100 : ex);
  }
  const float ps = ldexpf(1.0f, 10 - ex);  // max|y * ps| in [2^9, 2^10)
  if (tid == 0) cs[col] = ldexpf(1.0f, ex - 10);
  const uint32_t c = col;
  for (uint32_t sb = tid; sb < K / 32; sb += 256) {
    float sum = 0.f;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      uint16_t hi[8], lo[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const uint32_t k = sb * 32 + 8 * g + t;
        const float y = (w ? xc[k] * scale * w[k] : xc[k]) * ps;
        sum += y;
        const _Float16 h = (_Float16)y;
        hi[t] = __builtin_bit_cast(uint16_t, h);
        lo[t] = f2hb(y - (float)h);
      }
      uint16_t* dst = bx + ((size_t)sb * 64 + 16 * g + c) * 8;
      *(uint4*)dst = *(uint4*)hi;
      *(uint4*)(dst + 64) = *(uint4*)lo;
    }
    const _Float16 sh = (_Float16)sum;
    const size_t xo = ((size_t)(sb / 8) * 64 + c) * 8 + (sb % 8);
    xs[xo] = __builtin_bit_cast(uint16_t, sh);
    xs[xo + 64] = f2hb(sum - (float)sh);
  }
}

int sh_prep_launch(sh_engine* e, const float* x, uint32_t K, uint32_t N, const float* norm_w, float eps,
                   uint16_t* bx, uint16_t* xs, float* cs) {
  SH_CHECK(K % 32 == 0, SH_ERR_ARG, "prep K=%u not a multiple of 32", K);
  SH_CHECK(N >= 1 && N <= 8, SH_ERR_ARG, "prep N=%u outside [1, 8]", N);
  hipEvent_t ev = nullptr;
  sh_prof_begin(e, &ev);
  hipLaunchKernelGGL(k_prep, dim3(N), dim3(256), 0, e->stream, x, K, norm_w, eps, bx, xs, cs);
  SH_HIP(hipGetLastError());
  sh_prof_end(e, norm_w ? "rmsnorm_prep" : "prep", 0.0, ev);
  return SH_OK;
}

// ------------------------------------------------------------------ argmax

// Orderable key: larger float -> larger key; ties -> lower index wins
// (host argmax semantics, inference/sample.rs:504-514). NaN never wins.
__device__ __forceinline__ unsigned long long amax_key(float v, uint32_t idx) {
  uint32_t b = __builtin_bit_cast(uint32_t, v);
  b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((unsigned long long)b << 32) | (unsigned long long)(~idx);
}

__global__ void k_amax_init(unsigned long long* keys, uint32_t N) {
  if (threadIdx.x < N) keys[threadIdx.x] = 0ull;
}

__global__ __launch_bounds__(256) void k_argmax(const float* __restrict__ logits, uint32_t V,
                                                unsigned long long* keys) {
  const uint32_t col = blockIdx.y;
  const float* row = logits + (size_t)col * V;
  unsigned long long best = 0ull;
  const uint32_t per = 2048;
  const uint32_t i0 = blockIdx.x * per;
  const uint32_t i1 = min(i0 + per, V);
  for (uint32_t i = i0 + threadIdx.x; i < i1; i += 256) {
    const float v = row[i];
    if (v == v) {
      const unsigned long long k = amax_key(v, i);
      best = k > best ? k : best;
    }
  }
  for (int off = 32; off >= 1; off >>= 1) {
    const unsigned long long o = __shfl_xor(best, off);
    best = o > best ? o : best;
  }
  __shared__ unsigned long long wb[4];
  if ((threadIdx.x & 63) == 0) wb[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; ++w) best = wb[w] > best ? wb[w] : best;
    atomicMax(keys + col, best);
  }
}

__global__ void k_amax_finish(const unsigned long long* keys, uint32_t N, uint32_t* out) {
  const uint32_t j = threadIdx.x;
  if (j < N) out[j] = keys[j] == 0ull ? 0u : ~(uint32_t)(keys[j] & 0xFFFFFFFFull);
}

int sh_argmax_launch(sh_engine* e, const float* logits, uint32_t V, uint32_t N, unsigned long long* keys,
                     uint32_t* out_ids) {
  SH_CHECK(N >= 1 && N <= 64, SH_ERR_ARG, "argmax N=%u", N);
  hipEvent_t ev = nullptr;
  sh_prof_begin(e, &ev);
  hipLaunchKernelGGL(k_amax_init, dim3(1), dim3(64), 0, e->stream, keys, N);
  hipLaunchKernelGGL(k_argmax, dim3((V + 2047) / 2048, N), dim3(256), 0, e->stream, logits, V, keys);
  hipLaunchKernelGGL(k_amax_finish, dim3(1), dim3(64), 0, e->stream, keys, N, out_ids);
  SH_HIP(hipGetLastError());
  sh_prof_end(e, "argmax", 4.0 * V * N, ev);
  return SH_OK;
}
