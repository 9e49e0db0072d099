// Small per-column kernels of the verify step: embedding gather, RMSNorm fused
// with the GEMV activation operand build, and greedy per-column argmax.
#include "sh_internal.h"
#include "sh_operand.h"

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

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

constexpr int PREP_THREADS = SH_OPERAND_THREADS;

// y = x * rsqrt(mean(x^2) + eps) * w (rms_norm.slang:39-55) when w != null, else
// y = x; then y * s -> GEMV activation operand: B (hi/lo f16, [K/32][64][8]) and
// XS (per-32 sums, [K/256][64][8], lanes >= 16 stay zero), where s is the power
// of two putting max|y * s| in [2^9, 2^10); cs[col] = 1/s.
// One workgroup of 1024 threads per column; each thread keeps NV float4 of the
// column in registers, so x is read once.
template <int NV>
__global__ __launch_bounds__(PREP_THREADS) void k_prep(const float* __restrict__ x, uint32_t K,
                                                       const float* __restrict__ w, float eps,
                                                       uint16_t* __restrict__ bx, uint16_t* __restrict__ xs,
                                                       float* __restrict__ cs) {
  __shared__ float red_s[PREP_THREADS / 64], red_m[PREP_THREADS / 64];
  const uint32_t col = blockIdx.x, tid = threadIdx.x;
  const float* xc = x + (size_t)col * K;
  const uint32_t n4 = K / 4;
  float4 v[NV];
  float ss = 0.f, mx = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const uint32_t q = tid + PREP_THREADS * i;
    if (q < n4) {
      v[i] = *(const float4*)(xc + 4 * q);
      ss += v[i].x * v[i].x + v[i].y * v[i].y + v[i].z * v[i].z + v[i].w * v[i].w;
      if (w) {
        const float4 wv = *(const float4*)(w + 4 * q);
        v[i].x *= wv.x; v[i].y *= wv.y; v[i].z *= wv.z; v[i].w *= wv.w;  // x*w; the 1/rms factor comes later
      }
      mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
    } else {
      v[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  ss = sh_wave_sum(ss);
  mx = sh_wave_max(mx);
  if ((tid & 63) == 0) { red_s[tid >> 6] = ss; red_m[tid >> 6] = mx; }
  __syncthreads();
  ss = 0.f;
  mx = 0.f;
#pragma unroll
  for (int i = 0; i < PREP_THREADS / 64; ++i) { ss += red_s[i]; mx = fmaxf(mx, red_m[i]); }
  const float scale = w ? 1.0f / sqrtf(ss / (float)K + eps) : 1.0f;
  sh_operand_store<NV>(v, K, col, scale, mx, bx, xs, cs);
}

int sh_prep_launch(sh_engine* e, const float* x, uint32_t K, uint32_t N, const float* norm_w, float eps,
                   uint16_t* bx, uint16_t* xs, float* cs) {
  SH_CHECK(K % 32 == 0, SH_ERR_ARG, "prep K=%u not a multiple of 32", K);
  SH_CHECK(N >= 1 && N <= 8, SH_ERR_ARG, "prep N=%u outside [1, 8]", N);
  const uint32_t nv = (K / 4 + PREP_THREADS - 1) / PREP_THREADS;
  SH_CHECK(nv <= 8, SH_ERR_UNSUPPORTED, "prep K=%u above 32768", K);
  hipEvent_t ev = nullptr;
  sh_prof_begin(e, &ev);
#define PREP(NV_) \
  hipLaunchKernelGGL((k_prep<NV_>), dim3(N), dim3(PREP_THREADS), 0, e->stream, x, K, norm_w, eps, bx, xs, cs)
  if (nv <= 1) PREP(1);
  else if (nv <= 2) PREP(2);
  else if (nv <= 4) PREP(4);
  else PREP(8);
#undef PREP
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
