/* CPU oracle for the seeker speculative-decoding verify path.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py, as the checker, never as the thing measured
 * or shipped. See oracle.h for the numerics contract.
 *
 * Pinning status of each function (what checks it beyond its own formula) is
 * listed in tests/test_oracle.py; functions no check pins are marked
 * "parity unpinned" there.
 */
#include "oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* Accumulation type of the GEMV and attention dot products: f64 in the check
 * build (the parity reference), f32 with vectorized reductions in the timing
 * build (-DOR_FAST: the reference's own arithmetic, FLOAT_TYPE=float in
 * shaders/compute/mul_mat_vec_q4_k.slang:4, used as the CPU baseline). */
#ifdef OR_FAST
typedef float or_acc;
#define OR_SIMD_SUM _Pragma("omp simd reduction(+ : acc)")
#else
typedef double or_acc;
#define OR_SIMD_SUM
#endif

/* ------------------------------------------------------------------ f16 */

/* f16 -> f32 exactly as apps/seeker-cli/src/commands/run.rs:4115-4129
 * (subnormal = mant * 2^-24, exp 31 = inf/nan, normal = (1+m/1024)*2^(e-15)). */
float or_f16_to_f32(uint16_t h) {
  float sign = (h >> 15) & 1 ? -1.0f : 1.0f;
  int e = (h >> 10) & 0x1F;
  float mant = (float)(h & 0x3FF);
  float v;
  if (e == 0) v = mant * ldexpf(1.0f, -24);
  else if (e == 0x1F) v = mant == 0.0f ? INFINITY : NAN;
  else v = (1.0f + mant / 1024.0f) * ldexpf(1.0f, e - 15);
  return sign * v;
}

/* f32 -> f16, IEEE round-to-nearest-even, computed through double arithmetic
 * (independent of the bit-twiddling conversion used by the product). A float
 * widens to double exactly, so this is or_f64_to_f16 of the same value. */
uint16_t or_f32_to_f16(float f) { return or_f64_to_f16((double)f); }

/* double -> f16 with one IEEE round-to-nearest-even rounding of the double value. */
uint16_t or_f64_to_f16(double f) {
  if (isnan(f)) return 0x7E00;
  uint16_t sign = signbit(f) ? 0x8000 : 0;
  double a = fabs(f);
  if (a == 0.0) return sign;
  if (a >= 65520.0) return sign | 0x7C00;
  int e;
  frexp(a, &e);                 /* a = m * 2^e, m in [0.5, 1) */
  int ue = e - 1;               /* a in [2^ue, 2^(ue+1)) */
  if (ue < -14) {               /* subnormal: units of 2^-24 */
    double q = nearbyint(a * 16777216.0);  /* default rounding mode: ties-to-even */
    return sign | (uint16_t)q;             /* q == 1024 gives the min normal bit pattern */
  }
  double q = nearbyint(ldexp(a, 10 - ue)); /* in [1024, 2048] */
  if (q >= 2048.0) { q = 1024.0; ue += 1; }
  if (ue > 15) return sign | 0x7C00;
  return sign | (uint16_t)((ue + 15) << 10) | (uint16_t)((int)q - 1024);
}

/* --------------------------------------------------------------- philox */

/* Philox4x64-10 (Salmon et al. SC'11), the generator numpy.random.Philox
 * implements; pinned against numpy's random_raw(). */
static void mulhilo(uint64_t a, uint64_t b, uint64_t* hi, uint64_t* lo) {
  unsigned __int128 p = (unsigned __int128)a * b;
  *hi = (uint64_t)(p >> 64);
  *lo = (uint64_t)p;
}

void or_philox4x64_10(const uint64_t ctr[4], const uint64_t key[2], uint64_t out[4]) {
  uint64_t x[4] = {ctr[0], ctr[1], ctr[2], ctr[3]};
  uint64_t k[2] = {key[0], key[1]};
  for (int r = 0; r < 10; ++r) {
    if (r) { k[0] += 0x9E3779B97F4A7C15ull; k[1] += 0xBB67AE8584CAA73Bull; }
    uint64_t h0, l0, h1, l1;
    mulhilo(0xD2E7470EE14C6C93ull, x[0], &h0, &l0);
    mulhilo(0xCA5A826395121157ull, x[2], &h1, &l1);
    uint64_t y0 = h1 ^ x[1] ^ k[0], y2 = h0 ^ x[3] ^ k[1];
    x[0] = y0; x[1] = l1; x[2] = y2; x[3] = l0;
  }
  memcpy(out, x, sizeof x);
}

uint64_t or_philox_word(uint64_t k0, uint64_t k1, uint64_t i) {
  uint64_t ctr[4] = {i / 4 + 1, 0, 0, 0}, key[2] = {k0, k1}, out[4];
  or_philox4x64_10(ctr, key, out);
  return out[i % 4];
}

float or_unit_f32(uint64_t w) { return (float)(uint32_t)(w >> 40) / 16777216.0f; }

/* -------------------------------------------------------------- dequant */

/* Q4_K 6-bit (scale, min) unpack: run.rs:4223-4232. */
static void q4k_scale_min(const uint8_t* s, int j, int* sc, int* m) {
  if (j < 4) { *sc = s[j] & 63; *m = s[j + 4] & 63; }
  else {
    *sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
    *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
  }
}

/* run.rs:4212-4303: Q4_K y = (d*sc)*q - (dmin*m) per 32-sub-block, low nibbles
 * of qs[32g..32g+32) are sub-block 2g, high nibbles sub-block 2g+1;
 * Q8_0 y = d*q. F32 / F16 rows copied. */
int or_dequant_row(int type, const uint8_t* raw, uint64_t row, uint64_t k, float* out) {
  if (type == OR_Q4_K) {
    if (k % 256) return 1;
    uint64_t nb = k / 256;
    for (uint64_t b = 0; b < nb; ++b) {
      const uint8_t* blk = raw + (row * nb + b) * 144;
      float d = or_f16_to_f32((uint16_t)(blk[0] | blk[1] << 8));
      float dmin = or_f16_to_f32((uint16_t)(blk[2] | blk[3] << 8));
      const uint8_t* sc = blk + 4;
      const uint8_t* qs = blk + 16;
      float* y = out + b * 256;
      for (int g = 0; g < 4; ++g) {
        int s1, m1, s2, m2;
        q4k_scale_min(sc, 2 * g, &s1, &m1);
        q4k_scale_min(sc, 2 * g + 1, &s2, &m2);
        float d1 = d * (float)s1, mm1 = dmin * (float)m1;
        float d2 = d * (float)s2, mm2 = dmin * (float)m2;
        for (int l = 0; l < 32; ++l) y[64 * g + l] = d1 * (float)(qs[32 * g + l] & 0xF) - mm1;
        for (int l = 0; l < 32; ++l) y[64 * g + 32 + l] = d2 * (float)(qs[32 * g + l] >> 4) - mm2;
      }
    }
    return 0;
  }
  if (type == OR_Q5_K) {
    /* llama.cpp dequantize_row_q5_K (the reference's Q5_K shaders,
     * shaders/compute/mul_mat_vec_q5_k.slang): the Q4_K scale / min unpack,
     * low nibble from qs as in Q4_K, fifth bit (16) = bit s of qh[l] for
     * sub-block s, l = element % 32. */
    if (k % 256) return 1;
    uint64_t nb = k / 256;
    for (uint64_t b = 0; b < nb; ++b) {
      const uint8_t* blk = raw + (row * nb + b) * 176;
      float d = or_f16_to_f32((uint16_t)(blk[0] | blk[1] << 8));
      float dmin = or_f16_to_f32((uint16_t)(blk[2] | blk[3] << 8));
      const uint8_t* sc = blk + 4;
      const uint8_t* qh = blk + 16;
      const uint8_t* qs = blk + 48;
      float* y = out + b * 256;
      for (int s = 0; s < 8; ++s) {
        int scv, mv;
        q4k_scale_min(sc, s, &scv, &mv);
        float d1 = d * (float)scv, m1 = dmin * (float)mv;
        for (int l = 0; l < 32; ++l) {
          int q = (qs[32 * (s / 2) + l] >> (4 * (s % 2))) & 0xF;
          if (qh[l] & (1u << s)) q += 16;
          y[32 * s + l] = d1 * (float)q - m1;
        }
      }
    }
    return 0;
  }
  if (type == OR_Q6_K) {
    /* run.rs:4257-4291: q = low nibble | top two bits << 4, value
     * d * scales[e / 16] * (q - 32). */
    if (k % 256) return 1;
    uint64_t nb = k / 256;
    for (uint64_t b = 0; b < nb; ++b) {
      const uint8_t* blk = raw + (row * nb + b) * 210;
      const uint8_t* ql = blk;
      const uint8_t* qh = blk + 128;
      const int8_t* sc = (const int8_t*)(blk + 192);
      float d = or_f16_to_f32((uint16_t)(blk[208] | blk[209] << 8));
      float* y = out + b * 256;
      for (int n = 0; n < 2; ++n)
        for (int l = 0; l < 32; ++l) {
          const int is = l / 16;
          const int q1 = ((ql[64 * n + l] & 0xF) | ((qh[32 * n + l] & 3) << 4)) - 32;
          const int q2 = ((ql[64 * n + l + 32] & 0xF) | (((qh[32 * n + l] >> 2) & 3) << 4)) - 32;
          const int q3 = ((ql[64 * n + l] >> 4) | (((qh[32 * n + l] >> 4) & 3) << 4)) - 32;
          const int q4 = ((ql[64 * n + l + 32] >> 4) | (((qh[32 * n + l] >> 6) & 3) << 4)) - 32;
          y[128 * n + l] = d * (float)sc[8 * n + is] * (float)q1;
          y[128 * n + l + 32] = d * (float)sc[8 * n + is + 2] * (float)q2;
          y[128 * n + l + 64] = d * (float)sc[8 * n + is + 4] * (float)q3;
          y[128 * n + l + 96] = d * (float)sc[8 * n + is + 6] * (float)q4;
        }
    }
    return 0;
  }
  if (type == OR_Q8_0) {
    if (k % 32) return 1;
    uint64_t nb = k / 32;
    for (uint64_t b = 0; b < nb; ++b) {
      const uint8_t* blk = raw + (row * nb + b) * 34;
      float d = or_f16_to_f32((uint16_t)(blk[0] | blk[1] << 8));
      for (int i = 0; i < 32; ++i) out[b * 32 + i] = d * (float)(int8_t)blk[2 + i];
    }
    return 0;
  }
  if (type == OR_F32) { memcpy(out, raw + row * k * 4, k * 4); return 0; }
  if (type == OR_F16) {
    for (uint64_t i = 0; i < k; ++i) {
      const uint8_t* p = raw + (row * k + i) * 2;
      out[i] = or_f16_to_f32((uint16_t)(p[0] | p[1] << 8));
    }
    return 0;
  }
  return 2;
}

/* Batched-column GEMV, f64 accumulation (semantics of
 * shaders/compute/mul_mat_vec_q4_k.slang:13-103 / mul_mat_vec.slang:39-100,
 * batched columns ops/matmul.rs:473-487). */
int or_gemv(int type, const uint8_t* w, uint64_t M, uint64_t K, const float* x, uint32_t N, float* y) {
  int err = 0;
#pragma omp parallel
  {
    float* row = (float*)malloc(K * sizeof(float));
#pragma omp for schedule(static)
    for (int64_t m = 0; m < (int64_t)M; ++m) {
      if (or_dequant_row(type, w, (uint64_t)m, K, row)) { err = 1; continue; }
      for (uint32_t j = 0; j < N; ++j) {
        const float* xj = x + (uint64_t)j * K;
        or_acc acc = 0;
        OR_SIMD_SUM
        for (uint64_t k = 0; k < K; ++k) acc += (or_acc)row[k] * (or_acc)xj[k];
        y[(uint64_t)j * M + m] = (float)acc;
      }
    }
    free(row);
  }
  return err;
}

/* The reference's wide GEMM (N >= 32 columns, shaders/compute/mul_mm_cm.slang,
 * dispatched by ops/matmul.rs:433-446): every weight dequantized in f32
 * (stage_a_tile, e.g. the Q4_K line dall * sc * nibble - dmin * mb) and
 * rounded to f16, every activation rounded to f16 (the B staging, line 971),
 * products accumulated in f32 by the cooperative matrix; here in f64. The
 * dequantized row of or_dequant_row is that f32 value for every format. */
int or_gemv16(int type, const uint8_t* w, uint64_t M, uint64_t K, const float* x, uint32_t N, float* y) {
  int err = 0;
  double* xh = (double*)malloc((size_t)N * K * sizeof(double));
  for (uint64_t i = 0; i < (uint64_t)N * K; ++i) xh[i] = (double)or_f16_to_f32(or_f32_to_f16(x[i]));
#pragma omp parallel
  {
    float* row = (float*)malloc(K * sizeof(float));
    double* rh = (double*)malloc(K * sizeof(double));
#pragma omp for schedule(static)
    for (int64_t m = 0; m < (int64_t)M; ++m) {
      if (or_dequant_row(type, w, (uint64_t)m, K, row)) { err = 1; continue; }
      for (uint64_t k = 0; k < K; ++k) rh[k] = (double)or_f16_to_f32(or_f32_to_f16(row[k]));
      for (uint32_t j = 0; j < N; ++j) {
        const double* xj = xh + (uint64_t)j * K;
        double acc = 0.0;
        for (uint64_t k = 0; k < K; ++k) acc += rh[k] * xj[k];
        y[(uint64_t)j * M + m] = (float)acc;
      }
    }
    free(row);
    free(rh);
  }
  free(xh);
  return err;
}

/* ----------------------------------------------------------------- GGUF */

typedef struct { const char* name; uint32_t nlen; uint32_t type; uint64_t ne[4]; uint32_t nd; uint64_t off; } or_tensor;

typedef struct {
  const uint8_t* w;
  int type;
  uint64_t rows, cols; /* cols = contracting dim (ne0) */
} or_mat;

typedef struct {
  const float* attn_norm; or_mat wq, wk, wv, wo;
  const float* q_norm; const float* k_norm; /* qwen3 / qwen3moe: per-head RMSNorm weights [hd] */
  const float* ffn_norm; or_mat gate, up, down;
  or_mat gate_inp, gate_exps, up_exps, down_exps; /* qwen3moe: router [E][d]; experts as E stacked slabs */
} or_layer;

enum { OR_ARCH_LLAMA = 0, OR_ARCH_QWEN3 = 1, OR_ARCH_QWEN3MOE = 2 };

struct or_model {
  int arch;
  uint32_t n_layer, d, n_head, n_kv, hd, ff, V, q_dim;
  uint32_t n_expert, n_used, eff;
  float eps, theta;
  or_mat embd, out;
  const float* out_norm;
  or_layer* L;
  int mm16; /* dense matmuls with the wide GEMM's f16 operands (or_gemv16): 0 never,
             * 1 always, 2 in forward calls of >= 32 columns (ops/matmul.rs:433-446) */
  uint32_t call_cols; /* columns of the forward call in progress */
  int attn_cm1; /* causal forward calls of > 1 column: attention with flash_attn_cm1's
                 * f16 arithmetic (or_attn_cm1) instead of the exact softmax */
};

struct or_kv {
  uint32_t n_layer, n_kv, hd, max_seq, pos;
  uint16_t* k; /* [layer][max_seq][n_kv][hd] */
  uint16_t* v;
};

typedef struct { const uint8_t* p; const uint8_t* end; int bad; } rd;

static uint64_t rd_u(rd* r, int n) {
  if (r->p + n > r->end) { r->bad = 1; return 0; }
  uint64_t v = 0;
  for (int i = 0; i < n; ++i) v |= (uint64_t)r->p[i] << (8 * i);
  r->p += n;
  return v;
}

static void rd_skip_value(rd* r, uint32_t t);
static const uint8_t* rd_str(rd* r, uint32_t* len) {
  uint64_t n = rd_u(r, 8);
  *len = 0;
  if (r->bad || r->p + n > r->end) { r->bad = 1; return NULL; }
  const uint8_t* s = r->p;
  r->p += n;
  *len = (uint32_t)n;
  return s;
}
static void rd_skip_value(rd* r, uint32_t t) {
  static const int sz[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
  if (t == 8) { uint32_t l; rd_str(r, &l); return; }
  if (t == 9) {
    uint32_t et = (uint32_t)rd_u(r, 4);
    uint64_t n = rd_u(r, 8);
    for (uint64_t i = 0; i < n && !r->bad; ++i) rd_skip_value(r, et);
    return;
  }
  if (t > 12) { r->bad = 1; return; }
  rd_u(r, sz[t]);
}

static int streq(const uint8_t* s, uint32_t n, const char* z) { return s && strlen(z) == n && memcmp(s, z, n) == 0; }

/* Keys and defaults: models/llama.rs:1038-1048 ("llama."), models/qwen3.rs:
 * 609-638 ("qwen3.": head_dim = attention.key_length, eps 1e-6, theta 1e6),
 * and for "qwen3moe." the expert keys of models/qwen35moe.rs:4127-4129. */
static int key_is(const uint8_t* k, uint32_t kl, const char* arch, const char* suffix) {
  const size_t a = strlen(arch), b = strlen(suffix);
  return kl == a + 1 + b && memcmp(k, arch, a) == 0 && k[a] == '.' && memcmp(k + a + 1, suffix, b) == 0;
}

int or_model_open(const uint8_t* img, uint64_t size, or_model** out) {
  rd r = {img, img + size, 0};
  if (size < 24 || memcmp(img, "GGUF", 4)) return 1;
  r.p += 4;
  uint32_t ver = (uint32_t)rd_u(&r, 4);
  if (ver < 2 || ver > 3) return 2;
  uint64_t nt = rd_u(&r, 8), nkv = rd_u(&r, 8);
  or_model* m = (or_model*)calloc(1, sizeof *m);
  m->arch = -1;
  uint32_t align = 32, n_kv = 0, rope_dim = 0, key_len = 0;
  float theta = -1.f, eps = -1.f;
  const char* A = "";
  for (uint64_t i = 0; i < nkv && !r.bad; ++i) {
    uint32_t kl; const uint8_t* k = rd_str(&r, &kl);
    uint32_t t = (uint32_t)rd_u(&r, 4);
    if (t == 8 && streq(k, kl, "general.architecture")) {
      uint32_t vl; const uint8_t* v = rd_str(&r, &vl);
      if (streq(v, vl, "llama")) { m->arch = OR_ARCH_LLAMA; A = "llama"; }
      else if (streq(v, vl, "qwen3")) { m->arch = OR_ARCH_QWEN3; A = "qwen3"; }
      else if (streq(v, vl, "qwen3moe")) { m->arch = OR_ARCH_QWEN3MOE; A = "qwen3moe"; }
    } else if (t == 4 || t == 6) {
      uint32_t v = (uint32_t)rd_u(&r, 4);
      float f; memcpy(&f, &v, 4);
      if (streq(k, kl, "general.alignment")) align = v;
      else if (key_is(k, kl, A, "block_count")) m->n_layer = v;
      else if (key_is(k, kl, A, "attention.head_count")) m->n_head = v;
      else if (key_is(k, kl, A, "attention.head_count_kv")) n_kv = v;
      else if (key_is(k, kl, A, "attention.key_length")) key_len = v;
      else if (key_is(k, kl, A, "embedding_length")) m->d = v;
      else if (key_is(k, kl, A, "feed_forward_length")) m->ff = v;
      else if (key_is(k, kl, A, "vocab_size")) m->V = v;
      else if (key_is(k, kl, A, "rope.dimension_count")) rope_dim = v;
      else if (key_is(k, kl, A, "rope.freq_base")) theta = f;
      else if (key_is(k, kl, A, "attention.layer_norm_rms_epsilon")) eps = f;
      else if (key_is(k, kl, A, "expert_count")) m->n_expert = v;
      else if (key_is(k, kl, A, "expert_used_count")) m->n_used = v;
      else if (key_is(k, kl, A, "expert_feed_forward_length")) m->eff = v;
    } else {
      rd_skip_value(&r, t);
    }
  }
  if (m->arch < 0) { free(m); return 3; }
  const int qwen = m->arch != OR_ARCH_LLAMA;
  m->n_kv = n_kv ? n_kv : m->n_head;
  m->theta = theta > 0.f ? theta : (qwen ? 1e6f : 1e4f);
  m->eps = eps >= 0.f ? eps : (qwen ? 1e-6f : 1e-5f);
  if (!m->n_layer || !m->n_head || !m->d) { free(m); return 3; }
  m->hd = qwen && key_len ? key_len : m->d / m->n_head;
  m->q_dim = m->n_head * m->hd;
  if (m->arch == OR_ARCH_QWEN3MOE && (!m->n_expert || !m->n_used || !m->eff || m->n_used > m->n_expert)) {
    free(m);
    return 3;
  }
  (void)rope_dim;
  or_tensor* ts = (or_tensor*)calloc(nt, sizeof *ts);
  for (uint64_t i = 0; i < nt && !r.bad; ++i) {
    const uint8_t* s = rd_str(&r, &ts[i].nlen);
    ts[i].name = (const char*)s;
    ts[i].nd = (uint32_t)rd_u(&r, 4);
    ts[i].ne[1] = ts[i].ne[2] = ts[i].ne[3] = 1;
    for (uint32_t j = 0; j < ts[i].nd && j < 4; ++j) ts[i].ne[j] = rd_u(&r, 8);
    ts[i].type = (uint32_t)rd_u(&r, 4);
    ts[i].off = rd_u(&r, 8);
  }
  if (r.bad) { free(ts); free(m); return 4; }
  uint64_t pos = (uint64_t)(r.p - img);
  const uint8_t* data = img + (pos + align - 1) / align * align;
  m->L = (or_layer*)calloc(m->n_layer, sizeof(or_layer));
  int found_out = 0, missing = 0;
  char nm[96];
  /* matrices: rows = ne1 * ne2 (expert slabs stacked), cols = ne0 */
#define FIND(NAME, DST_MAT, DST_F32)                                                       \
  do {                                                                                     \
    int ok = 0;                                                                            \
    for (uint64_t t = 0; t < nt; ++t)                                                      \
      if (streq((const uint8_t*)ts[t].name, ts[t].nlen, NAME)) {                           \
        ok = 1;                                                                            \
        if (DST_MAT) {                                                                     \
          or_mat* mm = DST_MAT;                                                            \
          mm->w = data + ts[t].off; mm->type = (int)ts[t].type;                            \
          mm->cols = ts[t].ne[0]; mm->rows = ts[t].ne[1] * ts[t].ne[2];                    \
        } else {                                                                           \
          *(DST_F32) = (const float*)(data + ts[t].off);                                   \
        }                                                                                  \
      }                                                                                    \
    if (!ok) missing = 1;                                                                  \
  } while (0)
  FIND("token_embd.weight", &m->embd, (const float**)0);
  FIND("output_norm.weight", (or_mat*)0, &m->out_norm);
  for (uint64_t t = 0; t < nt; ++t)
    if (streq((const uint8_t*)ts[t].name, ts[t].nlen, "output.weight")) found_out = 1;
  if (found_out) FIND("output.weight", &m->out, (const float**)0);
  else m->out = m->embd; /* tied: llama.rs:424 / qwen3.rs:673 lm_head = output.unwrap_or(token_embd) */
  for (uint32_t l = 0; l < m->n_layer; ++l) {
    or_layer* L = &m->L[l];
#define NM(S) (snprintf(nm, sizeof nm, "blk.%u." S, l), nm)
    FIND(NM("attn_norm.weight"), (or_mat*)0, &L->attn_norm);
    FIND(NM("attn_q.weight"), &L->wq, (const float**)0);
    FIND(NM("attn_k.weight"), &L->wk, (const float**)0);
    FIND(NM("attn_v.weight"), &L->wv, (const float**)0);
    FIND(NM("attn_output.weight"), &L->wo, (const float**)0);
    FIND(NM("ffn_norm.weight"), (or_mat*)0, &L->ffn_norm);
    if (qwen) {
      FIND(NM("attn_q_norm.weight"), (or_mat*)0, &L->q_norm);
      FIND(NM("attn_k_norm.weight"), (or_mat*)0, &L->k_norm);
    }
    if (m->arch == OR_ARCH_QWEN3MOE) {
      FIND(NM("ffn_gate_inp.weight"), &L->gate_inp, (const float**)0);
      FIND(NM("ffn_gate_exps.weight"), &L->gate_exps, (const float**)0);
      FIND(NM("ffn_up_exps.weight"), &L->up_exps, (const float**)0);
      FIND(NM("ffn_down_exps.weight"), &L->down_exps, (const float**)0);
    } else {
      FIND(NM("ffn_gate.weight"), &L->gate, (const float**)0);
      FIND(NM("ffn_up.weight"), &L->up, (const float**)0);
      FIND(NM("ffn_down.weight"), &L->down, (const float**)0);
    }
#undef NM
  }
#undef FIND
  free(ts);
  if (missing) { free(m->L); free(m); return 5; }
  if (!m->V) m->V = (uint32_t)m->embd.rows;
  *out = m;
  return 0;
}

void or_model_free(or_model* m) { if (m) { free(m->L); free(m); } }

void or_model_dims(const or_model* m, uint32_t d[7]) {
  d[0] = m->n_layer; d[1] = m->d; d[2] = m->n_head; d[3] = m->n_kv; d[4] = m->hd; d[5] = m->ff; d[6] = m->V;
}

void or_model_moe_dims(const or_model* m, uint32_t d[4]) {
  d[0] = (uint32_t)m->arch; d[1] = m->n_expert; d[2] = m->n_used; d[3] = m->eff;
}

/* ------------------------------------------------------------------- KV */

/* KV layout [head_dim, n_head_kv, max_seq_len] token-major per layer
 * (inference/kv_cache.rs:99-111); rollback is a cursor truncate
 * (kv_cache.rs:587-602: position = min(new_pos, position)). */
int or_kv_create(const or_model* m, uint32_t max_seq, or_kv** out) {
  or_kv* kv = (or_kv*)calloc(1, sizeof *kv);
  kv->n_layer = m->n_layer; kv->n_kv = m->n_kv; kv->hd = m->hd; kv->max_seq = max_seq;
  size_t n = (size_t)m->n_layer * max_seq * m->n_kv * m->hd;
  kv->k = (uint16_t*)calloc(n, 2);
  kv->v = (uint16_t*)calloc(n, 2);
  if (!kv->k || !kv->v) { free(kv->k); free(kv->v); free(kv); return 1; }
  *out = kv;
  return 0;
}
void or_kv_free(or_kv* kv) { if (kv) { free(kv->k); free(kv->v); free(kv); } }
uint32_t or_kv_position(const or_kv* kv) { return kv->pos; }
void or_kv_truncate(or_kv* kv, uint32_t p) { if (p < kv->pos) kv->pos = p; }
void or_kv_set_position(or_kv* kv, uint32_t p) { kv->pos = p; }
uint16_t* or_kv_layer(or_kv* kv, uint32_t layer, int is_v) {
  size_t per = (size_t)kv->max_seq * kv->n_kv * kv->hd;
  return (is_v ? kv->v : kv->k) + per * layer;
}
void or_kv_compact(or_kv* kv, uint32_t base, const uint32_t* src, uint32_t n) {
  size_t row = (size_t)kv->n_kv * kv->hd;
  for (uint32_t l = 0; l < kv->n_layer; ++l)
    for (int isv = 0; isv < 2; ++isv) {
      uint16_t* c = or_kv_layer(kv, l, isv);
      for (uint32_t i = 0; i < n; ++i)
        if (src[i] != i) memmove(c + (base + i) * row, c + (base + src[i]) * row, row * 2);
    }
  kv->pos = base + n;
}

/* -------------------------------------------------------------- forward */

/* RMSNorm: y = x * rsqrt(mean(x^2) + eps) * w (shaders/compute/rms_norm.slang:39-55). */
static void rms_norm(const float* x, const float* w, uint32_t n, float eps, float* y) {
  double ss = 0.0;
  for (uint32_t i = 0; i < n; ++i) ss += (double)x[i] * x[i];
  double sc = 1.0 / sqrt(ss / n + (double)eps);
  for (uint32_t i = 0; i < n; ++i) y[i] = (float)((double)x[i] * sc * (double)w[i]);
}

/* RoPE NORM mode (adjacent pairs): theta = pos * base^(-2 i0/n_dims)
 * (shaders/include/rope_funcs.slang:37-61, theta_scale ops/rope.rs:138;
 * freq_scale 1, ext_factor 0, attn_factor 1 per ops/rope.rs:32-45). */
static void rope_norm(float* x, uint32_t n_head, uint32_t hd, uint32_t pos, float base) {
  for (uint32_t h = 0; h < n_head; ++h)
    for (uint32_t i0 = 0; i0 < hd; i0 += 2) {
      double theta = (double)pos * pow((double)base, -(double)i0 / (double)hd);
      double c = cos(theta), s = sin(theta);
      float* p = x + h * hd + i0;
      double x0 = p[0], x1 = p[1];
      p[0] = (float)(x0 * c - x1 * s);
      p[1] = (float)(x0 * s + x1 * c);
    }
}

/* RoPE NEOX mode (qwen3.rs:349-350, rope_funcs.slang rope_neox): the pair
 * (i, i + hd/2) rotated by theta_i = pos * base^(-2i/hd), i < hd/2. */
static void rope_neox(float* x, uint32_t n_head, uint32_t hd, uint32_t pos, float base) {
  const uint32_t half = hd / 2;
  for (uint32_t h = 0; h < n_head; ++h)
    for (uint32_t i = 0; i < half; ++i) {
      double theta = (double)pos * pow((double)base, -2.0 * (double)i / (double)hd);
      double c = cos(theta), s = sin(theta);
      float* p = x + h * hd;
      double x0 = p[i], x1 = p[i + half];
      p[i] = (float)(x0 * c - x1 * s);
      p[i + half] = (float)(x0 * s + x1 * c);
    }
}

static uint64_t row_bytes(int type, uint64_t cols) {
  switch (type) {
    case OR_Q4_K: return cols / 256 * 144;
    case OR_Q5_K: return cols / 256 * 176;
    case OR_Q6_K: return cols / 256 * 210;
    case OR_Q8_0: return cols / 32 * 34;
    case OR_F16: return cols * 2;
    default: return cols * 4;
  }
}

/* MoE gating (topk_moe.slang, GATING_SOFTMAX with_norm as
 * models/qwen35moe.rs:3168-3182): softmax of the E router logits (f64), the
 * k largest probabilities in descending order, ties to the lower expert index,
 * weights = selected probabilities / their sum, rounded to f32. */
void or_moe_route(const float* logits, uint32_t E, uint32_t k, uint32_t* ids, float* w) {
  double mx = -INFINITY, sum = 0.0;
  for (uint32_t e = 0; e < E; ++e) if (logits[e] > mx) mx = logits[e];
  double* p = (double*)malloc(E * sizeof(double));
  for (uint32_t e = 0; e < E; ++e) { p[e] = exp((double)logits[e] - mx); sum += p[e]; }
  for (uint32_t e = 0; e < E; ++e) p[e] /= sum;
  double sel[64], ws = 0.0;
  for (uint32_t j = 0; j < k; ++j) {
    uint32_t best = 0;
    double bv = -1.0;
    for (uint32_t e = 0; e < E; ++e)
      if (p[e] > bv) { bv = p[e]; best = e; }  /* strict >: the lower index wins ties */
    ids[j] = best;
    sel[j] = bv;
    ws += bv;
    p[best] = -2.0;
  }
  for (uint32_t j = 0; j < k; ++j) w[j] = (float)(sel[j] / ws);
  free(p);
}

/* Routed-expert FFN of qwen3moe over L normalized columns xn [L][d] (the
 * MoE step of models/qwen35moe.rs:3117-3182 without the shared expert):
 * router logits = gate_inp xn (f64 accumulation, f32 store), or_moe_route,
 * then per expert over the columns routed to it h = silu(gate_e x) * up_e x
 * (as the dense FFN) and y = down_e h; out[c] = sum_j w_j y_j in selection
 * order (f64 accumulation, f32 store). */
static void moe_ffn(const or_model* m, const or_layer* Ly, const float* xn, uint32_t L, float* out) {
  const uint32_t E = m->n_expert, K = m->n_used, ef = m->eff, d = m->d;
  float* lg = (float*)malloc((size_t)L * E * 4);
  uint32_t* ids = (uint32_t*)malloc((size_t)L * K * 4);
  float* w = (float*)malloc((size_t)L * K * 4);
  float* y = (float*)malloc((size_t)L * K * d * 4);  /* [col][slot][d] */
  float* X = (float*)malloc((size_t)L * d * 4);
  float* G = (float*)malloc((size_t)L * ef * 4);
  float* U = (float*)malloc((size_t)L * ef * 4);
  float* Y = (float*)malloc((size_t)L * d * 4);
  uint32_t* who = (uint32_t*)malloc((size_t)L * 4);
  or_gemv(Ly->gate_inp.type, Ly->gate_inp.w, E, d, xn, L, lg);
  for (uint32_t c = 0; c < L; ++c) or_moe_route(lg + (size_t)c * E, E, K, ids + (size_t)c * K, w + (size_t)c * K);
  const uint64_t gb = row_bytes(Ly->gate_exps.type, d), db = row_bytes(Ly->down_exps.type, ef);
  for (uint32_t e = 0; e < E; ++e) {
    uint32_t n = 0;
    for (uint32_t c = 0; c < L; ++c)
      for (uint32_t j = 0; j < K; ++j)
        if (ids[(size_t)c * K + j] == e) {
          who[n] = c * K + j;
          memcpy(X + (size_t)n * d, xn + (size_t)c * d, (size_t)d * 4);
          ++n;
        }
    if (!n) continue;
    or_gemv(Ly->gate_exps.type, Ly->gate_exps.w + (uint64_t)e * ef * gb, ef, d, X, n, G);
    or_gemv(Ly->up_exps.type, Ly->up_exps.w + (uint64_t)e * ef * gb, ef, d, X, n, U);
    for (size_t i = 0; i < (size_t)n * ef; ++i) {
      double x = G[i];
      G[i] = (float)((x / (1.0 + exp(-x))) * (double)U[i]);
    }
    or_gemv(Ly->down_exps.type, Ly->down_exps.w + (uint64_t)e * d * db, d, ef, G, n, Y);
    for (uint32_t i = 0; i < n; ++i) memcpy(y + (size_t)who[i] * d, Y + (size_t)i * d, (size_t)d * 4);
  }
  for (uint32_t c = 0; c < L; ++c)
    for (uint32_t t = 0; t < d; ++t) {
      double acc = 0.0;
      for (uint32_t j = 0; j < K; ++j) acc += (double)w[(size_t)c * K + j] * (double)y[((size_t)c * K + j) * d + t];
      out[(size_t)c * d + t] = (float)acc;
    }
  free(lg); free(ids); free(w); free(y); free(X); free(G); free(U); free(Y); free(who);
}

static int is_ancestor(const int32_t* parents, uint32_t a, uint32_t j) {
  /* a is ancestor-or-self of j within the chunk */
  int32_t x = (int32_t)j;
  while (x >= 0) {
    if ((uint32_t)x == a) return 1;
    x = parents[x];
  }
  return 0;
}

static void matmul(const or_model* m, const or_mat* W, const float* x, uint32_t N, float* y) {
  if (m->mm16 == 1 || (m->mm16 == 2 && m->call_cols >= 32)) or_gemv16(W->type, W->w, W->rows, W->cols, x, N, y);
  else or_gemv(W->type, W->w, W->rows, W->cols, x, N, y);
}

void or_model_set_mm16(or_model* m, int mode) { m->mm16 = mode >= 0 && mode <= 2 ? mode : 0; }

/* f16 -> f32 table (65536 entries of or_f16_to_f32) for the attention inner loops. */
static float f16_lut[65536];
static int f16_lut_ready = 0;
static void f16_lut_init(void) {
  if (f16_lut_ready) return;
  for (uint32_t i = 0; i < 65536; ++i) f16_lut[i] = or_f16_to_f32((uint16_t)i);
  f16_lut_ready = 1;
}

void or_model_set_attn_cm1(or_model* m, int on) { m->attn_cm1 = on != 0; }

/* The reference's masked attention, shaders/compute/flash_attn_cm1.slang (taken
 * by every forward of L > 1 tokens on an f16 cache, ops/flash_attn.rs:442-471;
 * single pass up to 16384 keys, :1393-1410), for one query row: keys in
 * 64-key blocks from key 0 (Bc, :39); per block the row maximum over its
 * visible keys (:300-312, the running maximum starting at -1e30, :173), the
 * f16 output rescaled by the f16 factor (:314-320), P = exp2(S - M) rounded to
 * f16 (:322-334), P V summed per 16-key chunk into an f16 accumulator (the
 * f16-accumulating coopmat MMA, :349-358) and added to the f16 output
 * (:363-374); O = f32(O16) / L at the end (:398-411). S is the f32 dot product
 * of the staged f16 q (see or_attn_cm1) with the f16 keys, computed here
 * exactly and rounded to f32 once; the order of the reference's sums inside one
 * MMA, of its exp2 and of its L sum are not pinned. L is kept in double. */
#define H2F(h) f16_lut[(uint16_t)(h)]
void or_attn_cm1_core(const uint16_t* q16, const uint16_t* k, const uint16_t* v, size_t kv_stride, uint32_t hd,
                      uint32_t n_keys, const uint8_t* visible, float* out) {
  enum { BC = 64, CH = 16 };
  f16_lut_init();
  uint16_t o16[512];
  float qf[512];
  for (uint32_t e = 0; e < hd; ++e) { o16[e] = 0; qf[e] = H2F(q16[e]); }
  float M = -1.0e30f;
  double L = 0.0;
  for (uint32_t k0 = 0; k0 < n_keys; k0 += BC) {
    float S[BC], P[BC];
    uint16_t p16[BC];
    int vis[BC];
    float rowmax = -1.0e30f;
    for (uint32_t c = 0; c < BC; ++c) {
      const uint32_t t = k0 + c;
      vis[c] = t < n_keys && (!visible || visible[t]);
      S[c] = -INFINITY;
      if (!vis[c]) continue;
      const uint16_t* kr = k + (size_t)t * kv_stride;
      double acc = 0.0;
      for (uint32_t e = 0; e < hd; ++e) acc += (double)qf[e] * (double)H2F(kr[e]);
      S[c] = (float)acc;
      if (S[c] > rowmax) rowmax = S[c];
    }
    const float Mn = rowmax > M ? rowmax : M;
    const float ef = exp2f(M - Mn);
    L = (double)ef * L;
    const double e16 = H2F(or_f32_to_f16(ef));
    for (uint32_t d = 0; d < hd; ++d) o16[d] = or_f64_to_f16(e16 * (double)H2F(o16[d]));
    for (uint32_t c = 0; c < BC; ++c) {
      P[c] = vis[c] ? exp2f(S[c] - Mn) : 0.0f;
      L += P[c];
      p16[c] = or_f32_to_f16(P[c]);
    }
    for (uint32_t d = 0; d < hd; ++d) {
      uint16_t acc16 = 0;
      for (uint32_t c0 = 0; c0 < BC; c0 += CH) {
        double sacc = H2F(acc16);
        for (uint32_t c = c0; c < c0 + CH; ++c)
          if (vis[c]) sacc += (double)H2F(p16[c]) * (double)H2F(v[(size_t)(k0 + c) * kv_stride + d]);
        acc16 = or_f64_to_f16(sacc);
      }
      o16[d] = or_f64_to_f16((double)H2F(o16[d]) + (double)H2F(acc16));
    }
    M = Mn;
  }
  const float Lf = (float)L;
  const float inv = Lf == 0.0f ? 0.0f : 1.0f / Lf;
  for (uint32_t d = 0; d < hd; ++d) out[d] = H2F(o16[d]) * inv;
}

/* Q staging of flash_attn_cm1.slang:155-171: f16(q * (scale * log2 e)) with the
 * f32 product scale * LOG2E (scale = 1 / sqrt(head_dim) in f32,
 * models/llama.rs:237), then the row as or_attn_cm1_core. */
#undef H2F

void or_attn_cm1(const float* q, const uint16_t* k, const uint16_t* v, size_t kv_stride, uint32_t hd, uint32_t n_keys,
                 const uint8_t* visible, float* out) {
  const float scale = 1.0f / sqrtf((float)hd);
  const float qs = scale * 1.44269504088896340736f;
  uint16_t q16[512];
  for (uint32_t e = 0; e < hd; ++e) q16[e] = or_f32_to_f16(q[e] * qs);
  or_attn_cm1_core(q16, k, v, kv_stride, hd, n_keys, visible, out);
}

int or_forward(or_model* m, or_kv* kv, const uint32_t* tokens, uint32_t L, uint32_t pos,
               const int32_t* parents, int logits_mode, float* logits, float* residual_out) {
  f16_lut_init();
  /* Preconditions as models/llama.rs:178-192. */
  if (L == 0) return 1;
  if (kv->pos != pos) return 2;
  if (pos + L > kv->max_seq) return 3;
  m->call_cols = L;
  const uint32_t d = m->d, hd = m->hd, nh = m->n_head, nkv = m->n_kv, ff = m->ff, qd = m->q_dim;
  const uint32_t dkv = hd * nkv, gqa = nh / nkv;
  const uint32_t wide = qd > d ? qd : d;
  uint32_t* qpos = (uint32_t*)malloc(L * sizeof(uint32_t));
  for (uint32_t i = 0; i < L; ++i) {
    uint32_t depth = 0;
    if (parents) { int32_t x = parents[i]; while (x >= 0) { ++depth; x = parents[x]; } }
    else depth = i;
    qpos[i] = pos + depth;
  }
  float* res = (float*)malloc((size_t)L * d * 4);
  float* xn = (float*)malloc((size_t)L * d * 4);
  float* q = (float*)malloc((size_t)L * wide * 4);
  float* k = (float*)malloc((size_t)L * dkv * 4);
  float* v = (float*)malloc((size_t)L * dkv * 4);
  float* att = (float*)malloc((size_t)L * wide * 4);
  float* tmp = (float*)malloc((size_t)L * d * 4);
  float* g = (float*)malloc((size_t)L * (ff ? ff : 1) * 4);
  float* u = (float*)malloc((size_t)L * (ff ? ff : 1) * 4);
  /* get_rows (elementwise.rs:873): dequantized embedding rows. */
  for (uint32_t i = 0; i < L; ++i) or_dequant_row(m->embd.type, m->embd.w, tokens[i], d, res + (size_t)i * d);
  const uint32_t kvlen = pos + L;
  const double scale = 1.0 / sqrt((double)hd);
  for (uint32_t l = 0; l < m->n_layer; ++l) {
    or_layer* Ly = &m->L[l];
    for (uint32_t i = 0; i < L; ++i) rms_norm(res + (size_t)i * d, Ly->attn_norm, d, m->eps, xn + (size_t)i * d);
    matmul(m, &Ly->wq, xn, L, q);
    matmul(m, &Ly->wk, xn, L, k);
    matmul(m, &Ly->wv, xn, L, v);
    if (m->arch != OR_ARCH_LLAMA) {
      /* per-head Q / K RMSNorm over head_dim, then NEOX RoPE (qwen3.rs:340-353) */
      for (uint32_t i = 0; i < L; ++i) {
        for (uint32_t h = 0; h < nh; ++h) {
          float* x = q + (size_t)i * qd + (size_t)h * hd;
          rms_norm(x, Ly->q_norm, hd, m->eps, x);
        }
        for (uint32_t h = 0; h < nkv; ++h) {
          float* x = k + (size_t)i * dkv + (size_t)h * hd;
          rms_norm(x, Ly->k_norm, hd, m->eps, x);
        }
        rope_neox(q + (size_t)i * qd, nh, hd, qpos[i], m->theta);
        rope_neox(k + (size_t)i * dkv, nkv, hd, qpos[i], m->theta);
      }
    } else {
      for (uint32_t i = 0; i < L; ++i) {
        rope_norm(q + (size_t)i * d, nh, hd, qpos[i], m->theta);
        rope_norm(k + (size_t)i * dkv, nkv, hd, qpos[i], m->theta);
      }
    }
    /* cache write f32 -> f16 at slot pos+i (ops/cache_io.rs:191-262). */
    uint16_t* Kc = or_kv_layer(kv, l, 0);
    uint16_t* Vc = or_kv_layer(kv, l, 1);
    for (uint32_t i = 0; i < L; ++i)
      for (uint32_t e = 0; e < dkv; ++e) {
        Kc[(size_t)(pos + i) * dkv + e] = or_f32_to_f16(k[(size_t)i * dkv + e]);
        Vc[(size_t)(pos + i) * dkv + e] = or_f32_to_f16(v[(size_t)i * dkv + e]);
      }
    /* attention: prefix [0,pos) always visible; within-chunk slot pos+a visible to
     * row j iff a <= j (causal, llama.rs:904-955) or a is an ancestor-or-self of j (tree). */
    const int cm1 = m->attn_cm1 && L > 1 && !parents;
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t j = 0; j < (int64_t)L; ++j)
      for (int64_t h = 0; h < (int64_t)nh; ++h) {
        const uint32_t kh = (uint32_t)h / gqa;
        const float* qv = q + (size_t)j * qd + (size_t)h * hd;
        if (cm1) {
          /* row j of the causal chunk sees keys [0, pos + j] */
          or_attn_cm1(qv, Kc + (size_t)kh * hd, Vc + (size_t)kh * hd, dkv, hd, pos + (uint32_t)j + 1, NULL,
                      att + (size_t)j * qd + (size_t)h * hd);
          continue;
        }
        double* s = (double*)malloc(kvlen * sizeof(double));
        double mx = -INFINITY;
        for (uint32_t t = 0; t < kvlen; ++t) {
          int vis = t < pos ? 1 : (parents ? is_ancestor(parents, t - pos, (uint32_t)j) : (t - pos <= (uint32_t)j));
          if (!vis) { s[t] = -INFINITY; continue; }
          const uint16_t* kr = Kc + (size_t)t * dkv + (size_t)kh * hd;
          or_acc acc = 0;
          OR_SIMD_SUM
          for (uint32_t e = 0; e < hd; ++e) acc += (or_acc)qv[e] * (or_acc)f16_lut[kr[e]];
          s[t] = acc * scale;
          if (s[t] > mx) mx = s[t];
        }
        double sum = 0.0;
        for (uint32_t t = 0; t < kvlen; ++t) { s[t] = s[t] == -INFINITY ? 0.0 : exp(s[t] - mx); sum += s[t]; }
        float* o = att + (size_t)j * qd + (size_t)h * hd;
        for (uint32_t e = 0; e < hd; ++e) {
          double acc = 0.0;
          for (uint32_t t = 0; t < kvlen; ++t)
            if (s[t] != 0.0) acc += s[t] * (double)f16_lut[Vc[(size_t)t * dkv + (size_t)kh * hd + e]];
          o[e] = (float)(acc / sum);
        }
        free(s);
      }
    matmul(m, &Ly->wo, att, L, tmp);
    for (size_t i = 0; i < (size_t)L * d; ++i) res[i] = res[i] + tmp[i];
    for (uint32_t i = 0; i < L; ++i) rms_norm(res + (size_t)i * d, Ly->ffn_norm, d, m->eps, xn + (size_t)i * d);
    if (m->arch == OR_ARCH_QWEN3MOE) {
      moe_ffn(m, Ly, xn, L, tmp);
    } else {
      matmul(m, &Ly->gate, xn, L, g);
      matmul(m, &Ly->up, xn, L, u);
      /* silu(x) = x / (1 + exp(-x)) (shaders/compute/silu.slang:21), then * up */
      for (size_t i = 0; i < (size_t)L * ff; ++i) {
        double x = g[i];
        g[i] = (float)((x / (1.0 + exp(-x))) * (double)u[i]);
      }
      matmul(m, &Ly->down, g, L, tmp);
    }
    for (size_t i = 0; i < (size_t)L * d; ++i) res[i] = res[i] + tmp[i];
  }
  if (residual_out) memcpy(residual_out, res, (size_t)L * d * 4);
  if (logits_mode) {
    uint32_t j0 = logits_mode == 1 ? L - 1 : 0, nc = L - j0;
    for (uint32_t i = 0; i < nc; ++i) rms_norm(res + (size_t)(j0 + i) * d, m->out_norm, d, m->eps, xn + (size_t)i * d);
    matmul(m, &m->out, xn, nc, logits);
  }
  kv->pos = pos + L; /* cache_io::advance */
  free(qpos); free(res); free(xn); free(q); free(k); free(v); free(att); free(tmp); free(g); free(u);
  return 0;
}

/* -------------------------------------------------------------- sampler */

/* argmax, lowest index on ties, NaN never selected (inference/sample.rs:504-514). */
uint32_t or_argmax(const float* x, uint32_t n) {
  uint32_t best = 0;
  float bv = -INFINITY;
  for (uint32_t i = 0; i < n; ++i) if (x[i] > bv) { bv = x[i]; best = i; }
  return best;
}

/* softmax with the all-masked uniform fallback (inference/sample.rs:516-533),
 * evaluated in f64. */
void or_softmax(const float* x, uint32_t n, float* out) {
  double mx = -INFINITY;
  for (uint32_t i = 0; i < n; ++i) if (x[i] > mx) mx = x[i];
  if (!isfinite(mx)) { for (uint32_t i = 0; i < n; ++i) out[i] = 1.0f / (float)(n ? n : 1); return; }
  double* e = (double*)malloc(n * sizeof(double));
  double s = 0.0;
  for (uint32_t i = 0; i < n; ++i) { e[i] = exp((double)x[i] - mx); s += e[i]; }
  for (uint32_t i = 0; i < n; ++i) out[i] = (float)(e[i] / s);
  free(e);
}

static const float* g_sort_keys;
static int cmp_desc(const void* a, const void* b) {
  uint32_t i = *(const uint32_t*)a, j = *(const uint32_t*)b;
  float x = g_sort_keys[i], y = g_sort_keys[j];
  if (x > y) return -1;
  if (x < y) return 1;
  return i < j ? -1 : (i > j);
}

/* Host chain (inference/sample.rs:369-474) without bias/penalties:
 * greedy -> argmax; else sort desc (ties by id) -> top_k -> top_p (exclusive
 * cumulative <= p keeps the crossing token) -> min_p (log-space cutoff) ->
 * 1/T -> softmax -> first index with cumulative >= u (clamp to last). */
uint32_t or_sample_one(const float* logits, uint32_t V, const or_sampler_cfg* cfg, float u) {
  if (cfg->temperature <= 0.0f) return or_argmax(logits, V);
  uint32_t* cand = (uint32_t*)malloc(V * sizeof(uint32_t));
  for (uint32_t i = 0; i < V; ++i) cand[i] = i;
  g_sort_keys = logits;
  qsort(cand, V, sizeof(uint32_t), cmp_desc);
  uint32_t k = (cfg->top_k > 0 && cfg->top_k < V) ? cfg->top_k : V;
  float* kept = (float*)malloc(k * sizeof(float));
  float* pr = (float*)malloc(k * sizeof(float));
  for (uint32_t i = 0; i < k; ++i) kept[i] = logits[cand[i]];
  if (cfg->top_p < 1.0f && cfg->top_p > 0.0f) {
    or_softmax(kept, k, pr);
    double cum = 0.0;
    for (uint32_t j = 0; j < k; ++j) { if (cum > cfg->top_p) kept[j] = -INFINITY; cum += pr[j]; }
  }
  if (cfg->min_p > 0.0f) {
    float cut = kept[0] + logf(cfg->min_p);
    for (uint32_t j = 0; j < k; ++j) if (kept[j] < cut) kept[j] = -INFINITY;
  }
  if (fabsf(cfg->temperature - 1.0f) > 1e-9f) {
    float it = 1.0f / fmaxf(cfg->temperature, 1e-9f);
    for (uint32_t j = 0; j < k; ++j) if (isfinite(kept[j])) kept[j] *= it;
  }
  or_softmax(kept, k, pr);
  double cum = 0.0;
  uint32_t ch = k - 1;
  for (uint32_t j = 0; j < k; ++j) { cum += pr[j]; if (cum >= u) { ch = j; break; } }
  uint32_t tok = cand[ch];
  free(cand); free(kept); free(pr);
  return tok;
}

void or_probs(const float* logits, uint32_t V, float T, float* out) {
  double mx = -INFINITY;
  for (uint32_t i = 0; i < V; ++i) if (logits[i] > mx) mx = logits[i];
  double s = 0.0;
  for (uint32_t i = 0; i < V; ++i) s += exp(((double)logits[i] - mx) / (double)T);
  for (uint32_t i = 0; i < V; ++i) out[i] = (float)(exp(((double)logits[i] - mx) / (double)T) / s);
}

/* GPU full-vocab categorical (ops/sampler.rs:303-368): softmax(l/T) in vocab
 * order, idx = first index whose cumulative probability >= u, clamped to V-1. */
uint32_t or_sample_vocab_order(const float* logits, uint32_t V, float T, float u) {
  double mx = -INFINITY;
  for (uint32_t i = 0; i < V; ++i) if (logits[i] > mx) mx = logits[i];
  double s = 0.0;
  for (uint32_t i = 0; i < V; ++i) s += exp(((double)logits[i] - mx) / (double)T);
  double target = (double)u * s, cum = 0.0;
  for (uint32_t i = 0; i < V; ++i) {
    cum += exp(((double)logits[i] - mx) / (double)T);
    if (cum >= target) return i;
  }
  return V - 1;
}

/* sample_and_compare (inference/sample.rs:347-361): emit s_i, continue while
 * i < n and s_i == d_i. One uniform per emitted position. */
uint32_t or_sample_and_compare(const float* logits, uint32_t V, const uint32_t* drafts, uint32_t n,
                               const or_sampler_cfg* cfg, const float* uniforms, int mode,
                               uint32_t* emitted) {
  uint32_t ne = 0;
  for (uint32_t i = 0; i <= n; ++i) {
    const float* row = logits + (size_t)i * V;
    uint32_t t;
    if (cfg->temperature <= 0.0f) t = or_argmax(row, V);
    else if (mode == 1) t = or_sample_vocab_order(row, V, cfg->temperature, uniforms[i]);
    else t = or_sample_one(row, V, cfg, uniforms[i]);
    emitted[ne++] = t;
    if (i < n && t == drafts[i]) continue;
    break;
  }
  return ne;
}

/* Speculative rejection sampling (new; Leviathan et al. 2023, Chen et al. 2023):
 * p_i = softmax(target_i / T), q_i = softmax(draft_i / T) in f64.
 * Accept draft d_i iff u_acc[i] * q_i(d_i) < p_i(d_i). At the first rejection i,
 * draw from r = max(0, p_i - q_i) (fallback p_i when r == 0) in vocab order:
 * first v with cumsum(r)_v > u_res[i] * sum(r). All accepted: draw the bonus from
 * p_k the same way. */
static double row_stats(const float* l, uint32_t V, double T, double* mx_out) {
  double mx = -INFINITY;
  for (uint32_t i = 0; i < V; ++i) if (l[i] > mx) mx = l[i];
  double s = 0.0;
  for (uint32_t i = 0; i < V; ++i) s += exp(((double)l[i] - mx) / T);
  *mx_out = mx;
  return s;
}

uint32_t or_rejection(const float* pl, const float* ql, const uint32_t* drafts, uint32_t k, uint32_t V,
                      float temperature, const float* u_acc, const float* u_res, uint32_t* next_tok) {
  const double T = temperature;
  for (uint32_t i = 0; i <= k; ++i) {
    const float* p = pl + (size_t)i * V;
    double pm, ps = row_stats(p, V, T, &pm);
    if (i == k) {
      double target = (double)u_res[i] * ps, cum = 0.0;
      uint32_t tok = V - 1;
      for (uint32_t v = 0; v < V; ++v) { cum += exp(((double)p[v] - pm) / T); if (cum > target) { tok = v; break; } }
      *next_tok = tok;
      return k;
    }
    const float* q = ql + (size_t)i * V;
    double qm, qs = row_stats(q, V, T, &qm);
    uint32_t dtok = drafts[i];
    double pd = exp(((double)p[dtok] - pm) / T) / ps;
    double qd = exp(((double)q[dtok] - qm) / T) / qs;
    if ((double)u_acc[i] * qd < pd) continue;
    double R = 0.0;
    for (uint32_t v = 0; v < V; ++v) {
      double r = exp(((double)p[v] - pm) / T) / ps - exp(((double)q[v] - qm) / T) / qs;
      if (r > 0.0) R += r;
    }
    uint32_t tok = V - 1;
    if (R > 0.0) {
      double target = (double)u_res[i] * R, cum = 0.0;
      for (uint32_t v = 0; v < V; ++v) {
        double r = exp(((double)p[v] - pm) / T) / ps - exp(((double)q[v] - qm) / T) / qs;
        if (r > 0.0) cum += r;
        if (cum > target) { tok = v; break; }
      }
    } else {
      double target = (double)u_res[i] * ps, cum = 0.0;
      for (uint32_t v = 0; v < V; ++v) { cum += exp(((double)p[v] - pm) / T); if (cum > target) { tok = v; break; } }
    }
    *next_tok = tok;
    return i;
  }
  return k;
}

/* Tree acceptance. The current distribution at a node starts as the target's
 * softmax(p/T); each rejected child replaces it by max(0, cur - q) / Z (kept as
 * the unnormalised r and its sum Z; unchanged when r is all zero). The final
 * draw uses the unnormalised weights (softmax numerator, or r) with the first v
 * whose vocab-order cumsum exceeds u * total, like or_rejection. All in f64. */
int or_tree_accept(const float* pl, const float* ql, const uint32_t* tokens, const int32_t* parents, uint32_t n,
                   uint32_t V, float temperature, const float* u, uint32_t* path, uint32_t* path_len,
                   uint32_t* next_tok) {
  if (n < 1 || parents[0] != -1) return -1;
  for (uint32_t i = 1; i < n; ++i)
    if (parents[i] < 0 || parents[i] >= (int32_t)i) return -1;
  double* r = (double*)malloc((size_t)V * sizeof(double));
  if (!r) return -1;
  uint32_t v = 0, len = 1;
  path[0] = 0;
  for (;;) {
    const float* p = pl + (size_t)v * V;
    int32_t acc = -1;
    if (temperature <= 0.f) {
      const uint32_t t = or_argmax(p, V);
      for (uint32_t c = v + 1; c < n && acc < 0; ++c)
        if (parents[c] == (int32_t)v && tokens[c] == t) acc = (int32_t)c;
      if (acc < 0) { *next_tok = t; break; }
      v = (uint32_t)acc;
      path[len++] = v;
      continue;
    }
    const double T = temperature;
    double pm, ps = row_stats(p, V, T, &pm);
    const float* q = ql + (size_t)v * V;
    double qm = 0.0, qs = 1.0;
    int have_q = 0, resid = 0;
    double Z = 1.0;
    for (uint32_t c = v + 1; c < n && acc < 0; ++c) {
      if (parents[c] != (int32_t)v) continue;
      if (!have_q) { qs = row_stats(q, V, T, &qm); have_q = 1; }
      const uint32_t tok = tokens[c];
      if (tok < V) {
        const double pc = resid ? r[tok] / Z : exp(((double)p[tok] - pm) / T) / ps;
        const double qc = exp(((double)q[tok] - qm) / T) / qs;
        if ((double)u[2 * c] * qc < pc) { acc = (int32_t)c; break; }
      }
      double R = 0.0;
      for (uint32_t x = 0; x < V; ++x) {
        const double cur = resid ? r[x] / Z : exp(((double)p[x] - pm) / T) / ps;
        const double d = cur - exp(((double)q[x] - qm) / T) / qs;
        R += d > 0.0 ? d : 0.0;
      }
      if (R > 0.0) {
        for (uint32_t x = 0; x < V; ++x) {
          const double cur = resid ? r[x] / Z : exp(((double)p[x] - pm) / T) / ps;
          const double d = cur - exp(((double)q[x] - qm) / T) / qs;
          r[x] = d > 0.0 ? d : 0.0;
        }
        Z = R;
        resid = 1;
      }
    }
    if (acc >= 0) {
      v = (uint32_t)acc;
      path[len++] = v;
      continue;
    }
    double total = 0.0;
    for (uint32_t x = 0; x < V; ++x) total += resid ? r[x] : exp(((double)p[x] - pm) / T);
    const double target = (double)u[2 * v + 1] * total;
    double cum = 0.0;
    uint32_t tok = V - 1;
    for (uint32_t x = 0; x < V; ++x) {
      cum += resid ? r[x] : exp(((double)p[x] - pm) / T);
      if (cum > target) { tok = x; break; }
    }
    *next_tok = tok;
    break;
  }
  *path_len = len;
  free(r);
  return 0;
}

/* --------------------------------------------------------- spec step */

/* Engine::decode_speculative (inference/mod.rs:2108-2297), greedy path, with a
 * separate draft model in place of the MTP head. Draft: feed the draft's pending
 * tokens plus last_token, then n-1 greedy steps (mod.rs:2062-2092 drafts greedily).
 * Verify [last, d_1..d_n] with all-position logits, greedy accept (mod.rs:2168-2179),
 * truncate to pos + acc + 1 (mod.rs:2269-2270). */
int or_spec_step_greedy(or_model* tgt, or_model* drf, or_kv* tkv, or_kv* dkv, uint32_t last_token,
                        uint32_t n_max, uint32_t* dpending, uint32_t* n_dpending, uint32_t* emitted,
                        uint32_t* n_emitted, uint32_t* drafts_out) {
  uint32_t n = n_max < 1 ? 1 : (n_max > 8 ? 8 : n_max);
  const uint32_t P = tkv->pos;
  const uint32_t V = tgt->V;
  float* lg = (float*)malloc((size_t)(n + 1) * V * 4);
  uint32_t drafts[8];
  uint32_t feed[16];
  uint32_t nf = 0;
  for (uint32_t i = 0; i < *n_dpending; ++i) feed[nf++] = dpending[i];
  feed[nf++] = last_token;
  if (dkv->pos + nf != P + 1) { free(lg); return 10; }
  int rc = or_forward(drf, dkv, feed, nf, dkv->pos, NULL, 1, lg, NULL);
  if (rc) { free(lg); return rc; }
  drafts[0] = or_argmax(lg, drf->V);
  for (uint32_t i = 1; i < n; ++i) {
    rc = or_forward(drf, dkv, &drafts[i - 1], 1, dkv->pos, NULL, 1, lg, NULL);
    if (rc) { free(lg); return rc; }
    drafts[i] = or_argmax(lg, drf->V);
  }
  uint32_t vt[9];
  vt[0] = last_token;
  for (uint32_t i = 0; i < n; ++i) vt[i + 1] = drafts[i];
  rc = or_forward(tgt, tkv, vt, n + 1, P, NULL, 2, lg, NULL);
  if (rc) { free(lg); return rc; }
  uint32_t ne = 0;
  for (uint32_t i = 0; i <= n; ++i) {
    uint32_t s = or_argmax(lg + (size_t)i * V, V);
    emitted[ne++] = s;
    if (i < n && s == drafts[i]) continue;
    break;
  }
  uint32_t acc = ne - 1;
  or_kv_truncate(tkv, P + acc + 1);
  or_kv_truncate(dkv, P + acc + 1);
  *n_dpending = 0;
  if (acc == n) dpending[(*n_dpending)++] = drafts[n - 1];
  *n_emitted = ne;
  if (drafts_out) memcpy(drafts_out, drafts, n * sizeof(uint32_t));
  free(lg);
  return 0;
}

/* Draft token at one draft position of a speculative step. GREEDY and
 * COMPARE draft greedily, as the reference does (inference/mod.rs:2062-2092,
 * record_greedy); REJECTION draws d ~ q = softmax(q_logits / T) by the
 * vocab-order inverse CDF with uniform u, which speculative sampling needs
 * for its output to follow the target distribution (Leviathan et al. 2023). */
uint32_t or_spec_draft_token(int mode, const float* q_logits, uint32_t V, float T, float u) {
  if (mode == OR_SPEC_REJECTION && T > 0.f) return or_sample_vocab_order(q_logits, V, T, u);
  return or_argmax(q_logits, V);
}

/* Acceptance of one verify of [last, d_1..d_n]. GREEDY: emit argmax p_i while
 * it equals d_{i+1} (host accept, inference/mod.rs:2168-2179). COMPARE: the
 * reference's GPU stochastic path (mod.rs:2181-2231): every column sampled in
 * vocab order with uniform u[2i+1], then sample_and_compare (sample.rs:
 * 347-361). REJECTION: or_rejection with u_acc[i] = u[2i], u_res[i] = u[2i+1].
 * Returns the number emitted (accepted + 1). */
uint32_t or_spec_accept(int mode, const float* p_logits, const float* q_logits, const uint32_t* drafts, uint32_t n,
                        uint32_t V, float T, const float* u, uint32_t* emitted) {
  if (mode == OR_SPEC_GREEDY || !(T > 0.f)) {
    uint32_t ne = 0;
    for (uint32_t i = 0; i <= n; ++i) {
      const uint32_t t = or_argmax(p_logits + (size_t)i * V, V);
      emitted[ne++] = t;
      if (i < n && t == drafts[i]) continue;
      break;
    }
    return ne;
  }
  if (mode == OR_SPEC_COMPARE) {
    float uc[9];
    for (uint32_t i = 0; i <= n; ++i) uc[i] = u[2 * i + 1];
    or_sampler_cfg cfg = {T, 0, 1.0f, 0.0f};
    return or_sample_and_compare(p_logits, V, drafts, n, &cfg, uc, 1, emitted);
  }
  float ua[8], ur[9];
  for (uint32_t i = 0; i <= n; ++i) {
    if (i < n) ua[i] = u[2 * i];
    ur[i] = u[2 * i + 1];
  }
  uint32_t nxt = 0;
  const uint32_t acc = or_rejection(p_logits, q_logits, drafts, n, V, T, ua, ur, &nxt);
  for (uint32_t i = 0; i < acc; ++i) emitted[i] = drafts[i];
  emitted[acc] = nxt;
  return acc + 1;
}

/* Engine::decode_speculative (inference/mod.rs:2108-2297) in all three modes
 * with a separate draft model: feed the draft's pending tokens and last_token,
 * draft n = clamp(n_max, 1, 8) tokens (or_spec_draft_token, draft i with
 * uniform u[2(n+1) + i]), verify [last, d_1..d_n] with all-position logits,
 * accept (or_spec_accept with u[0 .. 2(n+1))), truncate both caches to
 * P + acc + 1 (mod.rs:2269-2270). p_out [(n+1)][V] and q_out [n][V] (either
 * may be NULL) receive the target and draft logits of the step. */
int or_spec_step(or_model* tgt, or_model* drf, or_kv* tkv, or_kv* dkv, uint32_t last_token, uint32_t n_max,
                 int mode, float T, const float* u, uint32_t* dpending, uint32_t* n_dpending, uint32_t* emitted,
                 uint32_t* n_emitted, uint32_t* drafts_out, float* p_out, float* q_out) {
  const uint32_t n = n_max < 1 ? 1 : (n_max > 8 ? 8 : n_max);
  const uint32_t P = tkv->pos, V = tgt->V;
  if (drf->V != V) return 11;
  if (mode != OR_SPEC_GREEDY && !u) return 12;
  float* lg = (float*)malloc((size_t)(n + 1) * V * 4);
  float* ql = (float*)malloc((size_t)n * V * 4);
  uint32_t drafts[8], feed[16], nf = 0;
  for (uint32_t i = 0; i < *n_dpending; ++i) feed[nf++] = dpending[i];
  feed[nf++] = last_token;
  int rc = dkv->pos + nf != P + 1 ? 10 : 0;
  for (uint32_t i = 0; i < n && !rc; ++i) {
    float* q = ql + (size_t)i * V;
    rc = i == 0 ? or_forward(drf, dkv, feed, nf, dkv->pos, NULL, 1, q, NULL)
                : or_forward(drf, dkv, &drafts[i - 1], 1, dkv->pos, NULL, 1, q, NULL);
    if (!rc) drafts[i] = or_spec_draft_token(mode, q, V, T, u ? u[2 * (n + 1) + i] : 0.f);
  }
  uint32_t vt[9];
  vt[0] = last_token;
  for (uint32_t i = 0; i < n; ++i) vt[i + 1] = drafts[i];
  if (!rc) rc = or_forward(tgt, tkv, vt, n + 1, P, NULL, 2, lg, NULL);
  if (!rc) {
    const uint32_t ne = or_spec_accept(mode, lg, ql, drafts, n, V, T, u, emitted);
    const uint32_t acc = ne - 1;
    or_kv_truncate(tkv, P + acc + 1);
    or_kv_truncate(dkv, P + acc + 1);
    *n_dpending = 0;
    if (acc == n) dpending[(*n_dpending)++] = drafts[n - 1];  /* d_n was never fed to the draft */
    *n_emitted = ne;
    if (drafts_out) memcpy(drafts_out, drafts, n * sizeof(uint32_t));
    if (p_out) memcpy(p_out, lg, (size_t)(n + 1) * V * 4);
    if (q_out) memcpy(q_out, ql, (size_t)n * V * 4);
  }
  free(lg);
  free(ql);
  return rc;
}
