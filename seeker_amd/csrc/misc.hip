// Small per-column kernels of the verify step: embedding gather, RMSNorm fused
// with the GEMV activation operand build, and greedy per-column argmax.
#include "sh_internal.h"
#include "sh_operand.h"

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// ------------------------------------------------------------------ embed

// get_rows of a quantized token_embd (elementwise.rs:873, get_rows_q4_k.slang,
// get_rows_quant.slang): resid[j][i] = deq(token_embd)[tokens[j]][i], with the
// same per-element arithmetic as the Q4_K / Q6_K / Q8_0 dequant
// (run.rs:4212-4303) and llama.cpp's dequantize_row_q5_K for Q5_K.
__global__ void k_embed(const uint8_t* __restrict__ embd, int type, uint32_t d, size_t row_bytes,
                        const uint32_t* __restrict__ tokens, uint32_t V, float* __restrict__ resid) {
  // workgroup (token j, 256 elements from blockIdx.y): one element per thread,
  // so the row costs one round trip after the token id
  const uint32_t j = blockIdx.x;
  uint32_t tok = tokens[j];
  if (tok >= V) tok = V - 1;  // ids are validated on the host; clamp keeps reads in bounds
  const uint8_t* row = embd + (size_t)tok * row_bytes;
  const uint32_t i = blockIdx.y * 256 + threadIdx.x;
  if (i < d) {
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
    } else if (type == GGML_Q5_K) {
      // Q4_K's scale / min unpack and nibble, fifth bit (qh[l] >> s) & 1
      const uint8_t* blk = row + (size_t)(i / 256) * 176;
      const uint32_t e = i % 256, s = e / 32, l = e % 32;
      const float dd = h2f((uint16_t)(blk[0] | blk[1] << 8));
      const float dmin = h2f((uint16_t)(blk[2] | blk[3] << 8));
      const uint8_t* sc = blk + 4;
      int scv, mv;
      if (s < 4) { scv = sc[s] & 63; mv = sc[s + 4] & 63; }
      else { scv = (sc[s + 4] & 0xF) | ((sc[s - 4] >> 6) << 4); mv = (sc[s + 4] >> 4) | ((sc[s] >> 6) << 4); }
      const uint8_t byte = blk[48 + 32 * (s / 2) + l];
      const uint32_t q = ((s & 1) ? (byte >> 4) : (byte & 0xF)) | (((blk[16 + l] >> s) & 1u) << 4);
      y = (dd * (float)scv) * (float)q - dmin * (float)mv;
    } else if (type == GGML_Q6_K) {
      // element 128 n + 32 s + l: 6-bit q from ql / qh, d * scales[e / 16] * (q - 32)
      const uint8_t* blk = row + (size_t)(i / 256) * 210;
      const uint32_t e = i % 256, n = e / 128, s = (e % 128) / 32, l = e % 32;
      const uint32_t lo = (blk[64 * n + 32 * (s & 1) + l] >> (4 * (s >> 1))) & 0xF;
      const uint32_t hi = (blk[128 + 32 * n + l] >> (2 * s)) & 3;
      const float dd = h2f((uint16_t)(blk[208] | blk[209] << 8));
      y = dd * (float)(int8_t)blk[192 + e / 16] * (float)((int)(lo | hi << 4) - 32);
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
  hipLaunchKernelGGL(k_embed, dim3(N, (m->d + 255) / 256), dim3(256), 0, e->stream, m->embd_raw, m->embd_type, m->d,
                     m->embd_row_bytes, tokens, m->V, resid);
  SH_HIP(hipGetLastError());
  sh_prof_end(e, "embed", (double)N * m->embd_row_bytes, ev);
  return SH_OK;
}

// ------------------------------------------------------------------ prep

// acc + p[0] + p[stride] + ... (n terms, in order). Loads go out 8 at a time
// (indices clamped in bounds, surplus terms dropped) so n partials cost
// ceil(n / 8) memory latencies, not n.
__device__ __forceinline__ float4 sum_parts(const float* p, size_t stride, uint32_t n, float4 acc) {
  for (uint32_t s0 = 0; s0 < n; s0 += 8) {
    float4 t[8];
#pragma unroll
    for (uint32_t j = 0; j < 8; ++j) t[j] = *(const float4*)(p + (size_t)min(s0 + j, n - 1) * stride);
#pragma unroll
    for (uint32_t j = 0; j < 8; ++j) {
      if (s0 + j >= n) break;
      acc.x += t[j].x; acc.y += t[j].y; acc.z += t[j].z; acc.w += t[j].w;
    }
  }
  return acc;
}

// Finish the previous GEMV and build the next one's activation operand, one
// wave per (superblock, column); lane l owns elements 256 sb + 4l .. +3:
//   PREP_PLAIN:  v = x
//   PREP_RESID:  v = x + sum_s part[s] (split partial sums, added in split
//                order); x <- v (the residual stream)
//   PREP_SWIGLU: v = silu(g) * u with g, u = sum_s part[s] at the packed gate /
//                up rows of element i (32 (i / 16) + i % 16 and that + 16)
// With a norm weight w (rms_norm.slang:39-55): ssq[sb][col] = sum v^2 over the
// superblock and y = v * w, the rsqrt(mean + eps) factor being applied by the
// consuming GEMV; else y = v. Then y -> operand (B, XS, cs).
template <int MODE>
__global__ __launch_bounds__(64) void k_prep(PrepArgs a) {
  const uint32_t sb = blockIdx.x, col = blockIdx.y, lane = threadIdx.x;
  const uint32_t k = 256 * sb + 4 * lane;
  const bool valid = k < a.K;
  const size_t pstride = (size_t)a.part_cols * a.part_ld;
  // the norm weight is read first: behind the residual store below it would be
  // a second round trip
  const float4 wv = a.norm_w && valid ? *(const float4*)(a.norm_w + k) : make_float4(1.f, 1.f, 1.f, 1.f);
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  if (valid) {
    if (MODE == PREP_SWIGLU) {
      const float* pc = a.part + (size_t)col * a.part_ld + 32 * (k / 16) + k % 16;
      const float4 g = sum_parts(pc, pstride, a.nparts, make_float4(0.f, 0.f, 0.f, 0.f));
      const float4 u = sum_parts(pc + 16, pstride, a.nparts, make_float4(0.f, 0.f, 0.f, 0.f));
      v = make_float4((g.x / (1.0f + expf(-g.x))) * u.x, (g.y / (1.0f + expf(-g.y))) * u.y,
                      (g.z / (1.0f + expf(-g.z))) * u.z, (g.w / (1.0f + expf(-g.w))) * u.w);
    } else {
      float* xp = a.x + (size_t)col * a.K + k;
      v = *(const float4*)xp;
      if (MODE == PREP_RESID && a.nparts) {
        v = sum_parts(a.part + (size_t)col * a.part_ld + k, pstride, a.nparts, v);
        *(float4*)xp = v;
      }
    }
  }
  if (a.norm_w) {
    const float ss = sh_wave_sum(sh_sq4(v));
    if (lane == 0) a.ssq[(col / 8) * sh_grp_cs(a.K) + sb * 8 + col % 8] = ss;
    if (valid) {
      v.x *= wv.x; v.y *= wv.y; v.z *= wv.z; v.w *= wv.w;
    }
  }
  sh_operand_store_sb(v, a.K, sb, col, a.bx, a.xs, a.cs);
}

__device__ __forceinline__ void store_h4(uint16_t* p, float4 v) {
  typedef _Float16 hv4 __attribute__((ext_vector_type(4)));
  const hv4 h = {(_Float16)v.x, (_Float16)v.y, (_Float16)v.z, (_Float16)v.w};
  *(uint2*)p = __builtin_bit_cast(uint2, h);
}

// Operand of the wide f16 GEMM (the reference's mul_mm_cm input staging,
// mul_mm_cm.slang:969-971: every activation rounded to f16) for
// PREP_PLAIN / PREP_RESID, one 1024-thread workgroup per column (four elements
// per thread and pass, one pass for K <= 4096): v as in k_prep; with a norm
// weight the RMS factor over the whole column first, then
// bh = f16((v * rsqrt(mean + eps)) * w) in rms_norm.slang:39-55's order.
// PREP_MOE_COMBINE adds the routed experts' weighted outputs to x first, as
// k_moe_combine does (moe.hip: per element a fused multiply-add chain over the
// selection order from 0, then one add to x), so the combine and the next
// layer's operand rows are one launch.
template <int MODE>
__global__ __launch_bounds__(1024) void k_prep16_rows(PrepArgs a) {
  const uint32_t col = blockIdx.x, tid = threadIdx.x;
  const size_t pstride = (size_t)a.part_cols * a.part_ld;
  float* xc = a.x + (size_t)col * a.K;
  float ss = 0.f;
  for (uint32_t k = 4 * tid; k < a.K; k += 4096) {
    float4 v = *(const float4*)(xc + k);
    if (MODE == PREP_RESID && a.nparts) {
      v = sum_parts(a.part + (size_t)col * a.part_ld + k, pstride, a.nparts, v);
      *(float4*)(xc + k) = v;
    }
    if (MODE == PREP_MOE_COMBINE) {
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
      for (uint32_t j = 0; j < a.moe_k; ++j) {
        const uint32_t s = a.moe_slot[(size_t)col * a.moe_k + j];
        const float wt = a.moe_wts[(size_t)col * a.moe_k + j];
        const float4 y = *(const float4*)(a.moe_y + (size_t)s * a.K + k);
        acc.x = __builtin_fmaf(wt, y.x, acc.x);
        acc.y = __builtin_fmaf(wt, y.y, acc.y);
        acc.z = __builtin_fmaf(wt, y.z, acc.z);
        acc.w = __builtin_fmaf(wt, y.w, acc.w);
      }
      v.x += acc.x; v.y += acc.y; v.z += acc.z; v.w += acc.w;
      *(float4*)(xc + k) = v;
    }
    ss += sh_sq4(v);
  }
  float rinv = 1.0f;
  if (a.norm_w) {
    __shared__ float s_part[16];
    ss = sh_wave_sum(ss);
    if ((tid & 63) == 0) s_part[tid >> 6] = ss;
    __syncthreads();
    ss = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i += 4) ss += (s_part[i] + s_part[i + 1]) + (s_part[i + 2] + s_part[i + 3]);
    rinv = 1.0f / sqrtf(ss / (float)a.K + a.eps);
  }
  uint16_t* out = a.bh + (size_t)col * a.ldb;
  for (uint32_t k = 4 * tid; k < a.K; k += 4096) {
    float4 v = *(const float4*)(xc + k);  // this thread's own store above, if any
    if (a.norm_w) {
      const float4 w = *(const float4*)(a.norm_w + k);
      v = make_float4((rinv * v.x) * w.x, (rinv * v.y) * w.y, (rinv * v.z) * w.z, (rinv * v.w) * w.w);
    }
    store_h4(out + k, v);
  }
}

// PREP_SWIGLU for the wide f16 GEMM: bh = f16(silu(g) * u), one wave per
// (superblock, column) as in k_prep.
__global__ __launch_bounds__(64) void k_prep16_swiglu(PrepArgs a) {
  const uint32_t sb = blockIdx.x, col = blockIdx.y, lane = threadIdx.x;
  const uint32_t k = 256 * sb + 4 * lane;
  if (k >= a.K) return;
  const size_t pstride = (size_t)a.part_cols * a.part_ld;
  const float* pc = a.part + (size_t)col * a.part_ld + 32 * (k / 16) + k % 16;
  const float4 g = sum_parts(pc, pstride, a.nparts, make_float4(0.f, 0.f, 0.f, 0.f));
  const float4 u = sum_parts(pc + 16, pstride, a.nparts, make_float4(0.f, 0.f, 0.f, 0.f));
  const float4 v = make_float4((g.x / (1.0f + expf(-g.x))) * u.x, (g.y / (1.0f + expf(-g.y))) * u.y,
                               (g.z / (1.0f + expf(-g.z))) * u.z, (g.w / (1.0f + expf(-g.w))) * u.w);
  store_h4(a.bh + (size_t)col * a.ldb + k, v);
}

int sh_prep_launch(sh_engine* e, const PrepArgs& a) {
  SH_CHECK(a.K % 32 == 0, SH_ERR_ARG, "prep K=%u not a multiple of 32", a.K);
  if (a.bh) {
    SH_CHECK(a.N >= 1 && a.N <= SH_MAX_COLS16 && a.ldb >= a.K, SH_ERR_ARG,
             "f16 prep N=%u (at most %u), ldb %u < K %u", a.N, SH_MAX_COLS16, a.ldb, a.K);
    SH_CHECK(a.part_cols >= a.N || a.nparts == 0, SH_ERR_ARG, "prep: partials hold %u columns, N=%u", a.part_cols,
             a.N);
    SH_CHECK(a.mode == PREP_SWIGLU ? (a.part && a.nparts > 0) : a.x != nullptr, SH_ERR_ARG, "prep inputs missing");
    SH_CHECK(a.mode != PREP_RESID || a.nparts == 0 || a.part, SH_ERR_ARG, "prep partials missing");
    SH_CHECK(a.mode != PREP_MOE_COMBINE || (a.moe_y && a.moe_slot && a.moe_wts && a.moe_k >= 1 && a.K % 4 == 0),
             SH_ERR_ARG, "prep: expert outputs missing");
    hipEvent_t ev = nullptr;
    sh_prof_begin(e, &ev);
    if (a.mode == PREP_SWIGLU)
      hipLaunchKernelGGL(k_prep16_swiglu, dim3((a.K + 255) / 256, a.N), dim3(64), 0, e->stream, a);
    else if (a.mode == PREP_RESID)
      hipLaunchKernelGGL((k_prep16_rows<PREP_RESID>), dim3(a.N), dim3(1024), 0, e->stream, a);
    else if (a.mode == PREP_MOE_COMBINE)
      hipLaunchKernelGGL((k_prep16_rows<PREP_MOE_COMBINE>), dim3(a.N), dim3(1024), 0, e->stream, a);
    else
      hipLaunchKernelGGL((k_prep16_rows<PREP_PLAIN>), dim3(a.N), dim3(1024), 0, e->stream, a);
    SH_HIP(hipGetLastError());
    sh_prof_end(e, a.norm_w ? "rmsnorm_prep" : "prep", 0.0, ev);
    return SH_OK;
  }
  SH_CHECK(a.mode != PREP_MOE_COMBINE, SH_ERR_ARG, "prep: the expert combine builds f16 rows only");
  SH_CHECK(a.N >= 1 && a.N <= SH_MAX_PREP_COLS, SH_ERR_ARG, "prep N=%u outside [1, %u]", a.N, SH_MAX_PREP_COLS);
  SH_CHECK(a.part_cols >= a.N || a.nparts == 0, SH_ERR_ARG, "prep: partials hold %u columns, N=%u", a.part_cols, a.N);
  SH_CHECK(a.mode == PREP_SWIGLU ? (a.part && a.nparts > 0) : a.x != nullptr, SH_ERR_ARG, "prep inputs missing");
  SH_CHECK(a.mode != PREP_RESID || a.nparts == 0 || a.part, SH_ERR_ARG, "prep partials missing");
  SH_CHECK(!a.norm_w || a.ssq, SH_ERR_ARG, "prep: norm needs a sum-of-squares buffer");
  hipEvent_t ev = nullptr;
  sh_prof_begin(e, &ev);
  const dim3 grid((a.K + 255) / 256, a.N);
  if (a.mode == PREP_SWIGLU) hipLaunchKernelGGL((k_prep<PREP_SWIGLU>), grid, dim3(64), 0, e->stream, a);
  else if (a.mode == PREP_RESID) hipLaunchKernelGGL((k_prep<PREP_RESID>), grid, dim3(64), 0, e->stream, a);
  else hipLaunchKernelGGL((k_prep<PREP_PLAIN>), grid, dim3(64), 0, e->stream, a);
  SH_HIP(hipGetLastError());
  sh_prof_end(e, a.norm_w ? "rmsnorm_prep" : "prep", 0.0, ev);
  return SH_OK;
}

// y[col][m] (+)= sum_s part[s][col][m] for m < M (split partials, in split order).
// The partials hold part_cols columns per split.
__global__ void k_part_reduce(const float* __restrict__ part, uint32_t nparts, uint32_t part_ld, uint32_t part_cols,
                              uint32_t M, float* __restrict__ y, uint32_t ldy, int accumulate) {
  const uint32_t col = blockIdx.y, m = blockIdx.x * blockDim.x + threadIdx.x;
  if (m >= M) return;
  float s = accumulate ? y[(size_t)col * ldy + m] : 0.f;
  for (uint32_t k = 0; k < nparts; ++k) s += part[((size_t)k * part_cols + col) * part_ld + m];
  y[(size_t)col * ldy + m] = s;
}

int sh_part_reduce_launch(sh_engine* e, const float* part, uint32_t nparts, uint32_t part_ld, uint32_t part_cols,
                          uint32_t M, uint32_t N, float* y, uint32_t ldy, bool accumulate) {
  SH_CHECK(N >= 1 && N <= part_cols && M <= part_ld, SH_ERR_ARG, "partial reduce shape");
  hipLaunchKernelGGL(k_part_reduce, dim3((M + 255) / 256, N), dim3(256), 0, e->stream, part, nparts, part_ld,
                     part_cols, M, y, ldy, accumulate ? 1 : 0);
  SH_HIP(hipGetLastError());
  return SH_OK;
}

// ------------------------------------------------------------------ argmax

// One kernel per argmax: each workgroup folds its 2048-logit block into the
// column's key (atomic max), then counts itself in on its column's counter;
// the column's last workgroup to arrive writes its id and clears the key and
// the counter for the next launch (zero at allocation, so graph replays need
// no memset). The counters follow the SH_MAX_COLS keys, 64 bytes apart (one
// shared counter serialised every workgroup's arrival: 9.9 us for 8 columns).
__global__ __launch_bounds__(256) void k_argmax(const float* __restrict__ logits, uint32_t V, uint32_t N,
                                                unsigned long long* keys, uint32_t* __restrict__ out) {
  const uint32_t col = blockIdx.y;
  const float* row = logits + (size_t)col * V;
  unsigned long long best = 0ull;
  constexpr uint32_t PER_T = 8, per = 256 * PER_T;
  const uint32_t i0 = blockIdx.x * per;
  const uint32_t i1 = min(i0 + per, V);
  // every load of the thread goes out before the first compare (one round trip)
  float v[PER_T];
#pragma unroll
  for (uint32_t j = 0; j < PER_T; ++j) {
    const uint32_t i = i0 + threadIdx.x + 256 * j;
    v[j] = i < i1 ? row[i] : NAN;  // NaN is never selected
  }
#pragma unroll
  for (uint32_t j = 0; j < PER_T; ++j) {
    const unsigned long long k = sh_amax_key(v[j], i0 + threadIdx.x + 256 * j);  // NaN padding: key 0
    best = k > best ? k : best;
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
    // the returned value orders the max before the arrival
    const unsigned long long prev =
        __hip_atomic_fetch_max(keys + col, best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("s_waitcnt vmcnt(0)" : : "v"(prev) : "memory");
    uint32_t* cnt = (uint32_t*)(keys + SH_MAX_COLS + 8 * col);
    const uint32_t arrived = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1;
    const bool last = arrived == gridDim.x;
    if (last) {
      __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const unsigned long long k = __hip_atomic_load(keys + col, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      out[col] = sh_amax_index(k);
      __hip_atomic_store(keys + col, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

int sh_argmax_launch(sh_engine* e, const float* logits, uint32_t V, uint32_t N, unsigned long long* keys,
                     uint32_t* out_ids) {
  SH_CHECK(N >= 1 && N <= SH_MAX_COLS16, SH_ERR_ARG, "argmax N=%u", N);
  hipEvent_t ev = nullptr;
  sh_prof_begin(e, &ev);
  for (uint32_t c0 = 0; c0 < N; c0 += SH_MAX_COLS) {  // SH_MAX_COLS keys: launches of at most that many columns
    const uint32_t n = std::min<uint32_t>(SH_MAX_COLS, N - c0);
    hipLaunchKernelGGL(k_argmax, dim3((V + 2047) / 2048, n), dim3(256), 0, e->stream, logits + (size_t)c0 * V, V, n,
                       keys, out_ids + c0);
  }
  SH_HIP(hipGetLastError());
  sh_prof_end(e, "argmax", 4.0 * V * N, ev);
  return SH_OK;
}
