// Host runtime of libseeker_hip: engine / model / KV handles, the verify
// forward and the speculative step, behind the C ABI of include/seeker_hip.h.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <functional>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "sh_internal.h"
#include "sh_operand.h"

// Bumped whenever a model or KV cache is destroyed: captured graphs that may
// reference it are dropped (see graph replay below).
static std::atomic<uint64_t> g_graph_gen{1};

// ------------------------------------------------------------------ errors

static thread_local char g_err[1024] = "";

void sh_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
}

extern "C" const char* sh_last_error(void) { return g_err; }
extern "C" const char* sh_version(void) { return "seeker-hip 0.1 (gfx950)"; }

// ------------------------------------------------------------------ profiling

void sh_prof_begin(sh_engine* e, hipEvent_t* a) {
  *a = nullptr;
  if (!e->profiling) return;
  if (e->event_pool.empty()) {
    hipEvent_t ev;
    if (hipEventCreate(&ev) != hipSuccess) return;
    e->event_pool.push_back(ev);
  }
  *a = e->event_pool.back();
  e->event_pool.pop_back();
  (void)hipEventRecord(*a, e->stream);
}

void sh_prof_end(sh_engine* e, const char* name, double bytes, hipEvent_t a) {
  if (!e->profiling || !a) return;
  hipEvent_t b;
  if (e->event_pool.empty()) {
    if (hipEventCreate(&b) != hipSuccess) return;
  } else {
    b = e->event_pool.back();
    e->event_pool.pop_back();
  }
  (void)hipEventRecord(b, e->stream);
  e->pending.push_back({name, bytes, a, b});
}

int sh_prof_flush(sh_engine* e) {
  if (e->pending.empty()) return SH_OK;
  SH_HIP(hipStreamSynchronize(e->stream));
  for (auto& p : e->pending) {
    float ms = 0.f;
    SH_HIP(hipEventElapsedTime(&ms, p.a, p.b));
    KStat& s = e->stats[p.name];
    s.launches += 1;
    s.ms += ms;
    s.bytes += p.bytes;
    e->event_pool.push_back(p.a);
    e->event_pool.push_back(p.b);
  }
  e->pending.clear();
  return SH_OK;
}

// ------------------------------------------------------------------ engine

static void free_spec_bufs(SpecBufs& sb);

extern "C" int sh_engine_create(int dev, sh_engine** out) {
  SH_CHECK(out, SH_ERR_ARG, "sh_engine_create: out is NULL");
  int n = 0;
  SH_HIP(hipGetDeviceCount(&n));
  SH_CHECK(dev >= 0 && dev < n, SH_ERR_ARG, "hip device %d out of range (%d devices)", dev, n);
  SH_HIP(hipSetDevice(dev));
  hipDeviceProp_t prop;
  SH_HIP(hipGetDeviceProperties(&prop, dev));
  SH_CHECK(std::strncmp(prop.gcnArchName, "gfx950", 6) == 0, SH_ERR_UNSUPPORTED,
           "device %d is %s; this library is built for gfx950 only", dev, prop.gcnArchName);
  int rc = sh_static_scratch_init(dev);  // device-side scratch of sh_accept_sample_noalloc
  if (rc) return rc;
  sh_engine* e = new sh_engine();
  e->device = dev;
  hipError_t err = hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking);
  if (err != hipSuccess) {
    delete e;
    sh_set_error("engine setup: %s", hipGetErrorString(err));
    return SH_ERR_HIP;
  }
  *out = e;
  return SH_OK;
}

extern "C" void sh_engine_destroy(sh_engine* e) {
  if (!e) return;
  (void)hipSetDevice(e->device);
  (void)hipStreamSynchronize(e->stream);
  for (auto& p : e->pending) { (void)hipEventDestroy(p.a); (void)hipEventDestroy(p.b); }
  for (auto ev : e->event_pool) (void)hipEventDestroy(ev);
  for (auto& g : e->graphs) (void)hipGraphExecDestroy(g.exec);
  e->graphs.clear();
  free_spec_bufs(e->spec);
  for (void* p : e->scr) (void)hipFree(p);
  (void)hipStreamDestroy(e->stream);
  delete e;
}

extern "C" int sh_engine_sync(sh_engine* e) {
  SH_CHECK(e, SH_ERR_ARG, "engine is NULL");
  SH_HIP(hipStreamSynchronize(e->stream));
  return sh_prof_flush(e);
}

extern "C" int sh_engine_set_profiling(sh_engine* e, int on) {
  SH_CHECK(e, SH_ERR_ARG, "engine is NULL");
  int rc = sh_prof_flush(e);
  if (rc) return rc;
  e->profiling = on != 0;
  return SH_OK;
}

extern "C" int sh_engine_profile(sh_engine* e, sh_kernel_stat* out, uint32_t cap, uint32_t* n_out) {
  SH_CHECK(e && n_out, SH_ERR_ARG, "engine / n_out is NULL");
  int rc = sh_prof_flush(e);
  if (rc) return rc;
  uint32_t n = 0;
  for (auto& kv : e->stats) {
    if (out && n < cap) {
      std::memset(&out[n], 0, sizeof(sh_kernel_stat));
      std::snprintf(out[n].name, sizeof out[n].name, "%s", kv.first.c_str());
      out[n].launches = kv.second.launches;
      out[n].total_ms = kv.second.ms;
      out[n].alg_bytes = kv.second.bytes;
    }
    ++n;
  }
  *n_out = n;
  return SH_OK;
}

extern "C" int sh_engine_profile_reset(sh_engine* e) {
  SH_CHECK(e, SH_ERR_ARG, "engine is NULL");
  int rc = sh_prof_flush(e);
  e->stats.clear();
  return rc;
}

int sh_engine_scratch(sh_engine* e, int slot, size_t bytes, void** out) {
  SH_CHECK(slot >= 0 && slot < 4, SH_ERR_ARG, "scratch slot %d", slot);
  if (bytes > e->scr_bytes[slot]) {
    g_graph_gen.fetch_add(1);  // captured graphs may point into the old block
    SH_HIP(hipStreamSynchronize(e->stream));
    if (e->scr[slot]) SH_HIP(hipFree(e->scr[slot]));
    e->scr[slot] = nullptr;
    e->scr_bytes[slot] = 0;
    const size_t cap = (bytes + 4095) / 4096 * 4096;
    SH_HIP(hipMalloc(&e->scr[slot], cap));
    e->scr_bytes[slot] = cap;
  }
  *out = e->scr[slot];
  return SH_OK;
}

extern "C" int sh_dev_alloc(sh_engine* e, uint64_t bytes, void** out) {
  SH_CHECK(e && out, SH_ERR_ARG, "sh_dev_alloc: NULL argument");
  SH_HIP(hipMalloc(out, bytes ? bytes : 1));
  return SH_OK;
}
extern "C" int sh_dev_free(sh_engine* e, void* p) {
  SH_CHECK(e, SH_ERR_ARG, "engine is NULL");
  if (p) SH_HIP(hipFree(p));
  return SH_OK;
}
extern "C" int sh_memcpy_h2d(sh_engine* e, void* dst, const void* src, uint64_t bytes) {
  SH_CHECK(e && dst && src, SH_ERR_ARG, "sh_memcpy_h2d: NULL argument");
  SH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, e->stream));
  SH_HIP(hipStreamSynchronize(e->stream));
  return SH_OK;
}
extern "C" int sh_memcpy_d2h(sh_engine* e, void* dst, const void* src, uint64_t bytes) {
  SH_CHECK(e && dst && src, SH_ERR_ARG, "sh_memcpy_d2h: NULL argument");
  SH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, e->stream));
  SH_HIP(hipStreamSynchronize(e->stream));
  return sh_prof_flush(e);
}

namespace {

template <class T>
int dalloc(T** p, size_t n) {
  SH_HIP(hipMalloc((void**)p, n * sizeof(T) ? n * sizeof(T) : 1));
  return SH_OK;
}

}  // namespace

// ------------------------------------------------------------------ model

static void free_model(sh_model* m) {
  if (!m) return;
  for (auto& L : m->layers) {
    (void)hipFree(L.attn_norm);
    (void)hipFree(L.ffn_norm);
    sh_qmat_free(&L.wqkv);
    sh_qmat_free(&L.wv);
    sh_qmat_free(&L.wo);
    sh_qmat_free(&L.wgu);
    sh_qmat_free(&L.wdown);
    (void)hipFree(L.q_norm);
    (void)hipFree(L.k_norm);
    (void)hipFree(L.router);
    sh_qmat_free(&L.wgu_exps);
    sh_qmat_free(&L.wdown_exps);
  }
  sh_qmat_free(&m->lm_head);
  (void)hipFree(m->embd_raw);
  (void)hipFree(m->out_norm);
  (void)hipFree(m->rope);
  Workspace& w = m->ws;
  (void)hipFree(w.resid); (void)hipFree(w.resid2); (void)hipFree(w.bx); (void)hipFree(w.xs); (void)hipFree(w.q);
  (void)hipFree(w.attn); (void)hipFree(w.gpart); (void)hipFree(w.h); (void)hipFree(w.logits); (void)hipFree(w.fa_part); (void)hipFree(w.fab_part);
  (void)hipFree(w.tokens); (void)hipFree(w.amax); (void)hipFree(w.cs); (void)hipFree(w.ssq); (void)hipFree(w.bh); (void)hipFree(w.qtab);
  (void)hipFree(w.bx2); (void)hipFree(w.xs2); (void)hipFree(w.cs2); (void)hipFree(w.ssq2); (void)hipFree(w.sb_cnt);
  (void)hipFree(w.moe_logits); (void)hipFree(w.moe_ids); (void)hipFree(w.moe_wts); (void)hipFree(w.moe_info); (void)hipFree(w.moe_col);
  (void)hipFree(w.moe_slot); (void)hipFree(w.moe_hgu); (void)hipFree(w.moe_bx); (void)hipFree(w.moe_xs);
  (void)hipFree(w.moe_cs); (void)hipFree(w.moe_y);
  (void)hipFree(w.fa16_pv); (void)hipFree(w.fa16_ml); (void)hipFree(w.fa16_smax); (void)hipFree(w.fa16_flag);
  delete m;
}

static int ensure_rope(sh_model* m, uint32_t npos) {
  if (npos <= m->rope_max) return SH_OK;
  uint32_t cap = std::max<uint32_t>(npos, 1024);
  cap = (cap + 1023) / 1024 * 1024;
  const uint32_t half = m->hd / 2;
  std::vector<float2> tab((size_t)cap * half);
  // theta = pos * base^(-2 i / n_dims) (rope_funcs.slang:37-61, ops/rope.rs:138),
  // evaluated in double and rounded once.
  for (uint32_t p = 0; p < cap; ++p)
    for (uint32_t i = 0; i < half; ++i) {
      double th = (double)p * std::pow((double)m->theta, -2.0 * i / (double)m->hd);
      tab[(size_t)p * half + i] = make_float2((float)std::cos(th), (float)std::sin(th));
    }
  g_graph_gen.fetch_add(1);  // captured graphs may read the old table
  SH_HIP(hipStreamSynchronize(m->e->stream));
  if (m->rope) SH_HIP(hipFree(m->rope));
  m->rope = nullptr;
  SH_HIP(hipMalloc(&m->rope, tab.size() * sizeof(float2)));
  SH_HIP(hipMemcpy(m->rope, tab.data(), tab.size() * sizeof(float2), hipMemcpyHostToDevice));
  m->rope_max = cap;
  return SH_OK;
}

static int load_model(sh_engine* e, const uint8_t* img, uint64_t size, sh_model** out) {
  SH_CHECK(e && img && out, SH_ERR_ARG, "sh_model_load: NULL argument");
  SH_HIP(hipSetDevice(e->device));
  GFile f;
  ModelDesc md;
  int rc = sh_gguf_parse(img, size, &f);
  if (!rc) rc = sh_gguf_describe(f, &md);
  if (!rc) rc = sh_gguf_supported(md);
  if (rc) return rc;
  sh_model* m = new sh_model();
  m->e = e;
  m->n_layer = md.n_layer; m->n_head = md.n_head; m->n_kv = md.n_kv; m->d = md.d; m->ff = md.ff;
  m->n_ctx = md.n_ctx; m->theta = md.theta; m->eps = md.eps; m->hd = md.hd; m->V = md.V;
  m->arch = md.arch; m->q_dim = md.q_dim(); m->neox = md.neox;
  m->n_expert = md.n_expert; m->n_used = md.n_expert_used; m->eff = md.expert_ff;
  int fail = SH_OK;
#define FAIL(code, ...)                 \
  do {                                  \
    free_model(m);                      \
    SH_CHECK(false, code, __VA_ARGS__); \
  } while (0)
  // embedding (raw rows for the gather)
  const TRef& te = md.tok_embd;
  m->embd_type = (int)te.type;
  m->embd_row_bytes = te.row_bytes;
  if (dalloc(&m->embd_raw, m->embd_row_bytes * m->V)) FAIL(SH_ERR_HIP, "%s", sh_last_error());
  if (hipMemcpy(m->embd_raw, te.data, m->embd_row_bytes * m->V, hipMemcpyHostToDevice) != hipSuccess)
    FAIL(SH_ERR_HIP, "embedding upload failed");
  auto upload_f32 = [&](const TRef& t, float** dst) -> int {
    SH_HIP(hipMalloc(dst, t.cols * 4));
    SH_HIP(hipMemcpy(*dst, t.data, t.cols * 4, hipMemcpyHostToDevice));
    return SH_OK;
  };
  if ((fail = upload_f32(md.out_norm, &m->out_norm))) FAIL(fail, "%s", sh_last_error());
  const TRef& lm = md.output;
  if ((fail = sh_repack_upload(e, (int)lm.type, lm.data, m->V, m->d, &m->lm_head))) FAIL(fail, "%s", sh_last_error());
  m->alg_weight_bytes += m->lm_head.alg_bytes;
  const uint32_t dkv = m->hd * m->n_kv;
  m->layers.resize(m->n_layer);
  for (uint32_t l = 0; l < m->n_layer; ++l) {
    const LayerDesc& D = md.layers[l];
    Layer& L = m->layers[l];
    if ((fail = upload_f32(D.attn_norm, &L.attn_norm)) || (fail = upload_f32(D.ffn_norm, &L.ffn_norm)))
      FAIL(fail, "%s", sh_last_error());
    if (D.q_norm.present() &&
        ((fail = upload_f32(D.q_norm, &L.q_norm)) || (fail = upload_f32(D.k_norm, &L.k_norm))))
      FAIL(fail, "%s", sh_last_error());
    // q and k share a type (checked by the reader); v joins them when its type matches
    const uint8_t* parts[3] = {D.wq.data, D.wk.data, D.wv.data};
    const uint32_t rows[3] = {m->q_dim, dkv, dkv};
    const bool v_own = D.wv.type != D.wq.type;
    if ((fail = sh_repack_upload_cat(e, (int)D.wq.type, parts, rows, v_own ? 2 : 3, m->d, &L.wqkv)))
      FAIL(fail, "%s", sh_last_error());
    if (v_own && (fail = sh_repack_upload(e, (int)D.wv.type, D.wv.data, dkv, m->d, &L.wv)))
      FAIL(fail, "%s", sh_last_error());
    if ((fail = sh_repack_upload(e, (int)D.wo.type, D.wo.data, m->d, m->q_dim, &L.wo)))
      FAIL(fail, "%s", sh_last_error());
    if (m->n_expert) {
      const size_t rb = (size_t)m->n_expert * m->d * 4;
      if (hipMalloc(&L.router, rb) != hipSuccess ||
          hipMemcpy(L.router, D.gate_inp.data, rb, hipMemcpyHostToDevice) != hipSuccess)
        FAIL(SH_ERR_HIP, "router upload failed");
      if ((fail = sh_repack_upload_gu(e, (int)D.gate_exps.type, D.gate_exps.data, D.up_exps.data,
                                      m->n_expert * m->eff, m->d, &L.wgu_exps)))
        FAIL(fail, "%s", sh_last_error());
      if ((fail = sh_repack_upload(e, (int)D.down_exps.type, D.down_exps.data, m->n_expert * m->d, m->eff,
                                   &L.wdown_exps)))
        FAIL(fail, "%s", sh_last_error());
      m->alg_weight_bytes += L.wgu_exps.alg_bytes + L.wdown_exps.alg_bytes + 4.0 * m->n_expert * m->d;
    } else {
      if ((fail = sh_repack_upload_gu(e, (int)D.gate.type, D.gate.data, D.up.data, m->ff, m->d, &L.wgu)))
        FAIL(fail, "%s", sh_last_error());
      if ((fail = sh_repack_upload(e, (int)D.down.type, D.down.data, m->d, m->ff, &L.wdown)))
        FAIL(fail, "%s", sh_last_error());
    }
    m->alg_weight_bytes +=
        L.wqkv.alg_bytes + L.wv.alg_bytes + L.wo.alg_bytes + L.wgu.alg_bytes + L.wdown.alg_bytes + 8.0 * m->d;
  }
  m->alg_weight_bytes += 4.0 * m->d;
  {
    // multi-group path: every matrix a K-quant (the experts included); fused path
    // (llama, <= 8 columns): the layers uniformly Q4_K or Q8_0, lm_head either
    auto kq = [](const QMat& q) { return sh_is_kquant(q.type) && q.K % 256 == 0; };
    bool ok = kq(m->lm_head);
    for (const Layer& L : m->layers)
      ok = ok && kq(L.wqkv) && (!L.wv.d || kq(L.wv)) && kq(L.wo) &&
           (m->n_expert ? kq(L.wgu_exps) && kq(L.wdown_exps) : kq(L.wgu) && kq(L.wdown));
    m->mg_ok = ok;
    // fused path: llama, QKV / Wo / gate-up of every layer uniformly Q4_K or
    // Q8_0; with Q4_K layers (Q4_K_M-style mixes) a V matrix of its own, the
    // down matrices and lm_head may be other K-quants (multi-group GEMM on the
    // same operand)
    const int lt = m->layers[0].wqkv.type;
    const bool q4 = lt == GGML_Q4_K;
    auto side = [&](const QMat& q) { return q.type == lt || (q4 && kq(q)); };
    bool fused = m->arch == ARCH_LLAMA && (lt == GGML_Q4_K || lt == GGML_Q8_0) &&
                 (m->lm_head.type == GGML_Q4_K || m->lm_head.type == GGML_Q8_0 || (q4 && kq(m->lm_head)));
    for (const Layer& L : m->layers)
      fused = fused && L.wqkv.type == lt && L.wo.type == lt && L.wgu.type == lt && side(L.wdown) &&
              (!L.wv.d || (q4 && kq(L.wv)));
    m->fused_ok = fused;
    if (!ok && !fused) FAIL(SH_ERR_UNSUPPORTED, "weight types: neither all K-quants nor uniform Q4_K / Q8_0 layers");
    // wide f16 GEMMs: every dense matrix (the routed experts keep the
    // reference's f32 expert path) in a format the f16 GEMMs take
    auto g16 = [](const QMat& q) { return q.type == GGML_Q4_K ? q.K % 256 == 0 : sh_gemm16x_ok(q); };
    bool w16 = g16(m->lm_head);
    for (const Layer& L : m->layers)
      w16 = w16 && g16(L.wqkv) && (!L.wv.d || g16(L.wv)) && g16(L.wo) &&
            (m->n_expert ? true : g16(L.wgu) && g16(L.wdown));
    m->wide16_ok = w16;
    const char* env16 = getenv("SH_WIDE_F16");
    m->wide16 = w16 && !(env16 && atoi(env16) == 0);
    const char* envcm = getenv("SH_FA_CM");
    m->fa16 = !(envcm && atoi(envcm) == 0);
  }
  // workspace for up to SH_MAX_COLS columns per chunk (operands: 8 groups of 8),
  // SH_MAX_COLS16 for the wide f16 calls of a model that takes them
  Workspace& w = m->ws;
  w.max_cols = m->wide16_ok ? SH_MAX_COLS16 : SH_MAX_COLS;
  const uint32_t kmax = std::max({m->d, m->ff, m->q_dim, m->eff}), ngrp = SH_MAX_COLS / 8;
  const uint32_t wide = std::max(m->d, m->q_dim);  // q and attention rows
  const size_t bx_elems = ngrp * sh_grp_bx(kmax);
  const size_t xs_elems = ngrp * sh_grp_xs(kmax);
  const size_t part_floats =  // grown on demand in forward_dev
      (size_t)m->n_kv * (4096 / SH_FA_MIN_SPLIT_KEYS) * SH_FA_MAX_ROWS * sh_fa_part_stride(m->hd);
  size_t gpart_floats = 0;
  for (const Layer& L : m->layers)
    gpart_floats = std::max({gpart_floats, sh_gemv_part_floats(L.wo), sh_gemv_part_floats(L.wgu),
                             sh_gemv_part_floats(L.wdown), sh_gemv_part_floats(L.wv),
                             sh_gemm_part_floats(L.wqkv) + sh_gemm_part_floats(L.wv),
                             sh_gemm_part_floats(L.wo), sh_gemm_part_floats(L.wgu), sh_gemm_part_floats(L.wdown)});
  if (m->wide16_ok)
    for (const Layer& L : m->layers)
      gpart_floats = std::max({gpart_floats, sh_gemm16_part_floats(L.wqkv), sh_gemm16_part_floats(L.wo),
                               sh_gemm16_part_floats(L.wgu), sh_gemm16_part_floats(L.wdown)});
  const size_t C = w.max_cols;
  if (dalloc(&w.resid, C * m->d) || dalloc(&w.resid2, C * m->d) || dalloc(&w.bx, bx_elems) ||
      dalloc(&w.xs, xs_elems) ||
      dalloc(&w.q, C * wide) || dalloc(&w.attn, C * wide) || dalloc(&w.gpart, gpart_floats) ||
      dalloc(&w.h, C * std::max(m->ff, 1u)) || dalloc(&w.logits, C * m->V) || dalloc(&w.fa_part, part_floats) ||
      dalloc(&w.tokens, C + 64) || dalloc(&w.amax, SH_AMAX_WORDS) || dalloc(&w.cs, ngrp * sh_grp_cs(kmax)) ||
      dalloc(&w.ssq, ngrp * sh_grp_cs(kmax)) || dalloc(&w.bh, C * kmax) || dalloc(&w.qtab, C) || dalloc(&w.bx2, sh_grp_bx(m->d)) || dalloc(&w.xs2, sh_grp_xs(m->d)) ||
      dalloc(&w.cs2, sh_grp_cs(m->d)) || dalloc(&w.ssq2, sh_grp_cs(m->d)) || dalloc(&w.sb_cnt, SH_SB_CNT * SH_SB_CNT_STRIDE))
    FAIL(SH_ERR_HIP, "workspace allocation: %s", sh_last_error());
  w.fa_part_floats = part_floats;
  w.gpart_floats = gpart_floats;
  if (hipMemset(w.xs, 0, xs_elems * 2) != hipSuccess || hipMemset(w.bx, 0, bx_elems * 2) != hipSuccess ||
      hipMemset(w.xs2, 0, sh_grp_xs(m->d) * 2) != hipSuccess || hipMemset(w.bx2, 0, sh_grp_bx(m->d) * 2) != hipSuccess ||
      hipMemset(w.sb_cnt, 0, SH_SB_CNT * SH_SB_CNT_STRIDE * 4) != hipSuccess ||
      hipMemset(w.amax, 0, SH_AMAX_WORDS * 8) != hipSuccess)
    FAIL(SH_ERR_HIP, "workspace clear failed");
  if (m->n_expert) {
    const size_t P = C * m->n_used, ng = (P + 7) / 8;
    const size_t info = 1 + 3 * (size_t)sh_moe_max_chunks((uint32_t)P, m->n_expert);
    if (dalloc(&w.moe_logits, C * m->n_expert) || dalloc(&w.moe_ids, P) || dalloc(&w.moe_wts, P) || dalloc(&w.moe_info, info) || dalloc(&w.moe_col, P) ||
        dalloc(&w.moe_slot, P) || dalloc(&w.moe_hgu, P * 2 * m->eff) || dalloc(&w.moe_bx, ng * sh_grp_bx(m->eff)) ||
        dalloc(&w.moe_xs, ng * sh_grp_xs(m->eff)) || dalloc(&w.moe_cs, ng * sh_grp_cs(m->eff)) ||
        dalloc(&w.moe_y, P * m->d))
      FAIL(SH_ERR_HIP, "moe workspace allocation: %s", sh_last_error());
    if (hipMemset(w.moe_xs, 0, ng * sh_grp_xs(m->eff) * 2) != hipSuccess ||
        hipMemset(w.moe_bx, 0, ng * sh_grp_bx(m->eff) * 2) != hipSuccess)
      FAIL(SH_ERR_HIP, "moe workspace clear failed");
  }
  if ((fail = ensure_rope(m, std::max<uint32_t>(m->n_ctx, 1024)))) FAIL(fail, "%s", sh_last_error());
  if (hipDeviceSynchronize() != hipSuccess) FAIL(SH_ERR_HIP, "model upload failed");
#undef FAIL
  *out = m;
  return SH_OK;
}

extern "C" int sh_model_load_gguf_memory(sh_engine* e, const void* data, uint64_t size, sh_model** out) {
  return load_model(e, (const uint8_t*)data, size, out);
}

extern "C" int sh_model_load_gguf(sh_engine* e, const char* path, sh_model** out) {
  SH_CHECK(path, SH_ERR_ARG, "path is NULL");
  int fd = open(path, O_RDONLY);
  SH_CHECK(fd >= 0, SH_ERR_ARG, "cannot open %s", path);
  struct stat st;
  if (fstat(fd, &st) != 0) { close(fd); SH_CHECK(false, SH_ERR_ARG, "cannot stat %s", path); }
  void* p = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  SH_CHECK(p != MAP_FAILED, SH_ERR_ARG, "mmap %s failed", path);
  int rc = load_model(e, (const uint8_t*)p, (uint64_t)st.st_size, out);
  munmap(p, (size_t)st.st_size);
  return rc;
}

extern "C" void sh_model_destroy(sh_model* m) {
  g_graph_gen.fetch_add(1);
  if (!m) return;
  (void)hipStreamSynchronize(m->e->stream);
  free_model(m);
}

extern "C" int sh_model_info(const sh_model* m, sh_model_dims* o) {
  SH_CHECK(m && o, SH_ERR_ARG, "sh_model_info: NULL argument");
  o->n_layer = m->n_layer; o->n_embd = m->d; o->n_head = m->n_head; o->n_head_kv = m->n_kv;
  o->head_dim = m->hd; o->n_ff = m->ff; o->n_vocab = m->V; o->n_ctx_train = m->n_ctx;
  o->rms_eps = m->eps; o->rope_freq_base = m->theta;
  o->weight_type = m->layers.empty() ? -1 : m->layers[0].wo.type;
  o->weight_bytes = m->alg_weight_bytes;
  return SH_OK;
}

extern "C" int sh_model_wide_f16(const sh_model* m, int* on) {
  SH_CHECK(m && on, SH_ERR_ARG, "sh_model_wide_f16: NULL argument");
  *on = m->wide16 ? 1 : 0;
  return SH_OK;
}

extern "C" int sh_model_set_wide_f16(sh_model* m, int on) {
  SH_CHECK(m, SH_ERR_ARG, "sh_model_set_wide_f16: NULL model");
  SH_CHECK(!on || m->wide16_ok, SH_ERR_UNSUPPORTED,
           "wide f16 GEMMs need a model without routed experts whose matrices are all Q4_K");
  m->wide16 = on != 0;
  return SH_OK;
}

extern "C" int sh_model_cm1_attention(const sh_model* m, int* on) {
  SH_CHECK(m && on, SH_ERR_ARG, "sh_model_cm1_attention: NULL argument");
  *on = m->fa16 ? 1 : 0;
  return SH_OK;
}

extern "C" int sh_model_set_cm1_attention(sh_model* m, int on) {
  SH_CHECK(m, SH_ERR_ARG, "sh_model_set_cm1_attention: NULL model");
  m->fa16 = on != 0;
  return SH_OK;
}

// ------------------------------------------------------------------ KV

extern "C" int sh_kv_create(sh_engine* e, const sh_model* m, uint32_t max_seq, sh_kv** out) {
  SH_CHECK(e && m && out, SH_ERR_ARG, "sh_kv_create: NULL argument");
  SH_CHECK(max_seq >= 1 && max_seq <= (1u << 22), SH_ERR_ARG, "max_seq_len %u out of range", max_seq);
  sh_kv* kv = new sh_kv();
  kv->e = e;
  kv->n_layer = m->n_layer; kv->n_kv = m->n_kv; kv->hd = m->hd;
  kv->max_seq = (max_seq + 31) / 32 * 32;
  const size_t n = (size_t)kv->n_layer * kv->n_kv * kv->max_seq * kv->hd;
  if (hipMalloc(&kv->k, n * 2) != hipSuccess || hipMalloc(&kv->v, n * 2) != hipSuccess) {
    (void)hipFree(kv->k);
    delete kv;
    SH_CHECK(false, SH_ERR_HIP, "KV allocation of %zu bytes failed", n * 4);
  }
  // Zero-fill so never-written slots read as finite zeros.
  SH_HIP(hipMemset(kv->k, 0, n * 2));
  SH_HIP(hipMemset(kv->v, 0, n * 2));
  *out = kv;
  return SH_OK;
}

extern "C" void sh_kv_destroy(sh_kv* kv) {
  g_graph_gen.fetch_add(1);
  if (!kv) return;
  (void)hipStreamSynchronize(kv->e->stream);
  (void)hipFree(kv->k);
  (void)hipFree(kv->v);
  delete kv;
}

extern "C" int sh_kv_position(const sh_kv* kv, uint32_t* pos) {
  SH_CHECK(kv && pos, SH_ERR_ARG, "sh_kv_position: NULL argument");
  *pos = kv->pos;
  return SH_OK;
}

extern "C" int sh_kv_truncate(sh_kv* kv, uint32_t new_pos) {
  SH_CHECK(kv, SH_ERR_ARG, "kv is NULL");
  kv->pos = std::min(new_pos, kv->pos);
  kv->pending.clear();
  return SH_OK;
}

extern "C" int sh_kv_set_position(sh_kv* kv, uint32_t pos) {
  SH_CHECK(kv, SH_ERR_ARG, "kv is NULL");
  SH_CHECK(pos <= kv->max_seq, SH_ERR_CAPACITY, "position %u beyond capacity %u", pos, kv->max_seq);
  kv->pos = pos;
  kv->pending.clear();
  return SH_OK;
}

static inline uint32_t v_slot_host(uint32_t kappa) { return 8u * ((kappa & 15u) >> 2) + 4u * (kappa >> 4) + (kappa & 3u); }

static int kv_xfer(sh_kv* kv, uint32_t layer, int is_v, uint32_t n_pos, uint16_t* host, bool to_host) {
  SH_CHECK(kv && host, SH_ERR_ARG, "sh_kv_*_layer: NULL argument");
  SH_CHECK(layer < kv->n_layer && n_pos <= kv->max_seq, SH_ERR_ARG, "layer %u / n_pos %u out of range", layer, n_pos);
  const size_t per = (size_t)kv->n_kv * kv->max_seq * kv->hd;
  std::vector<uint16_t> buf(per);
  uint16_t* dev = (is_v ? kv->v : kv->k) + per * layer;
  SH_HIP(hipStreamSynchronize(kv->e->stream));
  if (!to_host) SH_HIP(hipMemcpy(buf.data(), dev, per * 2, hipMemcpyDeviceToHost));
  else SH_HIP(hipMemcpy(buf.data(), dev, per * 2, hipMemcpyDeviceToHost));
  for (uint32_t h = 0; h < kv->n_kv; ++h)
    for (uint32_t t = 0; t < n_pos; ++t)
      for (uint32_t d = 0; d < kv->hd; ++d) {
        size_t di = is_v ? (((size_t)h * (kv->max_seq / 32) + t / 32) * kv->hd + d) * 32 + v_slot_host(t & 31)
                         : ((size_t)h * kv->max_seq + t) * kv->hd + d;
        size_t hi = ((size_t)t * kv->n_kv + h) * kv->hd + d;
        if (to_host) host[hi] = buf[di];
        else buf[di] = host[hi];
      }
  if (!to_host) SH_HIP(hipMemcpy(dev, buf.data(), per * 2, hipMemcpyHostToDevice));
  return SH_OK;
}

extern "C" int sh_kv_read_layer(sh_kv* kv, uint32_t layer, int is_v, uint32_t n_pos, uint16_t* out) {
  return kv_xfer(kv, layer, is_v, n_pos, out, true);
}
extern "C" int sh_kv_write_layer(sh_kv* kv, uint32_t layer, int is_v, uint32_t n_pos, const uint16_t* in) {
  return kv_xfer(kv, layer, is_v, n_pos, const_cast<uint16_t*>(in), false);
}

extern "C" int sh_kv_compact(sh_kv* kv, uint32_t base, const uint32_t* src, uint32_t n) {
  SH_CHECK(kv && (src || n == 0), SH_ERR_ARG, "sh_kv_compact: NULL argument");
  SH_CHECK(base + n <= kv->max_seq, SH_ERR_CAPACITY, "compaction beyond capacity");
  for (uint32_t i = 0; i < n; ++i)
    SH_CHECK(base + src[i] < kv->max_seq, SH_ERR_ARG, "compaction source %u out of range", src[i]);
  if (n) {
    sh_engine* e = kv->e;
    uint32_t* d = nullptr;
    SH_HIP(hipMallocAsync((void**)&d, n * 4, e->stream));
    SH_HIP(hipMemcpyAsync(d, src, n * 4, hipMemcpyHostToDevice, e->stream));
    int rc = sh_kv_compact_launch(e, kv, base, d, n);
    if (rc) return rc;
    SH_HIP(hipFreeAsync(d, e->stream));
    SH_HIP(hipStreamSynchronize(e->stream));
  }
  kv->pos = base + n;
  kv->pending.clear();
  return SH_OK;
}

// ------------------------------------------------------------------ forward

// One chunk of nc <= 8 columns whose token ids are already on the device at
// m->ws.tokens[tok_off ..]. Writes K/V at slots slot0 .. slot0+nc, runs every
// layer, and (if want_logits) the final norm + lm_head into ws.logits [nc][V].
// gate/up: SH_GU=split finishes split partials in the down prep (SwiGLU there);
// by default one kernel produces whole sums and applies SwiGLU itself.
static bool swiglu_epilogue() {
  static const bool v = [] {
    const char* s = getenv("SH_GU");
    return !(s && std::string(s) == "split");
  }();
  return v;
}

// One column of a forward chunk: the cache its K/V row goes to, the slot, and
// the RoPE position.
struct ColKv {
  sh_kv* kv = nullptr;
  uint32_t slot = 0;
  int32_t pos = 0;
};
// Attention for columns [col0, col0 + ncol) of a chunk, all of one sequence
// (cache kv): keys [0, kvlen) exist, keys >= mask_base need their colmask bit.
struct FaSeg {
  sh_kv* kv = nullptr;
  uint32_t col0 = 0, ncol = 0, kvlen = 0, mask_base = 0;
  uint64_t colmask[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  const uint64_t* masks = nullptr;  // device masks of the ncol columns (required above 8 columns)
  const uint64_t* hmasks = nullptr;  // host masks of the ncol columns (live for the whole forward)
};

// SH_FAB=0: attention of the multi-group path per segment (k_fa / k_fa2 and
// one combine per segment) instead of one batched launch per layer.
static bool fab_enabled() {
  static const bool v = [] {
    const char* s = getenv("SH_FAB");
    return !(s && std::string(s) == "0");
  }();
  return v;
}

struct FabGuard {  // a chunk's batched-attention plan, freed (stream-ordered) at scope end
  sh_engine* e;
  FabLaunch fl;
  ~FabGuard() { sh_fab_free(e, fl); }
};

static int plan_fab(sh_model* m, const std::vector<FaSeg>& segs, uint32_t nc, FabGuard* g) {
  std::vector<FabSegIn> fin(segs.size());
  for (size_t i = 0; i < segs.size(); ++i) {
    const FaSeg& sg = segs[i];
    fin[i].kv = sg.kv; fin[i].col0 = sg.col0; fin[i].ncol = sg.ncol; fin[i].kvlen = sg.kvlen;
    fin[i].mask_base = sg.mask_base; fin[i].hmasks = sg.hmasks;
  }
  return sh_fab_plan(m->e, m, fin.data(), (uint32_t)fin.size(), nc, &g->fl);
}

// SH_FUSE=0 keeps the separate down prep and attention combine kernels.
static bool fusion_enabled() {
  static const bool v = [] {
    const char* s = getenv("SH_FUSE");
    return !(s && std::string(s) == "0");
  }();
  return v;
}

static int forward_chunk(sh_model* m, const uint32_t* dev_tokens, uint32_t nc, const ColKv* cols,
                         const std::vector<FaSeg>& segs, bool want_logits, bool want_resid) {
  sh_engine* e = m->e;
  Workspace& w = m->ws;
  int rc;
  // For chunks of at most 2 columns (the draft's single-token forwards) the
  // down GEMV builds its operand from h and Wo combines the attention splits
  // itself, when they take the split-K kernel: two fewer kernels per layer.
  // Every row-group workgroup of a split builds that split's operand, which
  // outweighs the saved launch once there are 8 columns (measured).
  const bool fuse = fusion_enabled() && nc <= 2;
  const uint32_t s_wo = m->layers.empty() ? 0 : sh_gemv_fusable(m->layers[0].wo);
  const bool fuse_wo = s_wo && s_wo * nc <= 8;
  // Mixed-type models (Q4_K_M-style): V in a matrix of its own and the down /
  // lm_head matrices in another K-quant take the multi-group GEMM on the same
  // staged operand; the fusions that need the tuned kernels are then decided
  // per layer.
  const int lt = m->layers.empty() ? GGML_Q4_K : m->layers[0].wqkv.type;
  auto tuned = [&](const QMat& q) { return q.type == lt; };
  bool any_wv = false;
  for (const Layer& L : m->layers) any_wv = any_wv || L.wv.d != nullptr;
  if ((rc = sh_embed_launch(e, m, dev_tokens, nc, w.resid))) return rc;
  const uint32_t dkv = m->hd * m->n_kv;
  EpiArgs qkv;
  qkv.out = w.q; qkv.ldo = m->d;
  qkv.Dq = m->d; qkv.Dkv = dkv; qkv.hd = m->hd; qkv.n_kv = m->n_kv;
  qkv.rope = m->rope;
  for (uint32_t j = 0; j < nc; ++j) {
    qkv.colpos[j] = cols[j].pos; qkv.slot[j] = cols[j].slot; qkv.mseq[j] = cols[j].kv->max_seq;
    qkv.kc[j] = cols[j].kv->k; qkv.vc[j] = cols[j].kv->v;
  }
  qkv.dbase = cols[0].kv->graph_base;  // graph capture: one cache per forward
  // Operand the next GEMV reads. The prep kernels and the attention combine
  // write set 0; residual preps fused into the o / down GEMVs write set 1,
  // since other workgroups of the producing kernel may still be staging set 0.
  struct OpSet {
    uint16_t* bx;
    uint16_t* xs;
    float* cs;
    float* ssq;
  };
  const OpSet set0{w.bx, w.xs, w.cs, w.ssq}, set1{w.bx2, w.xs2, w.cs2, w.ssq2};
  OpSet cur = set0;
  // GEMVs whose input is RMS-normalized apply the norm factor to their outputs
  auto set_norm = [&](EpiArgs& ea) {
    ea.cs = cur.cs; ea.ssq = cur.ssq; ea.ssq_n = (m->d + 255) / 256; ea.norm_K = m->d; ea.eps = m->eps;
  };
  // o, gate/up and down write split partial sums, finished by the next prep
  // (residual add, SwiGLU); ld = the matrix's padded (packed) row count. o and
  // down read set 0 (attention combine, SwiGLU prep).
  auto part_args = [&](const QMat& q) {
    EpiArgs pa;
    pa.out = w.gpart; pa.ldo = q.tiles * 16; pa.cs = w.cs;
    pa.part_stride = (size_t)8 * pa.ldo;
    pa.part_cap = (uint32_t)(w.gpart_floats / pa.part_stride);
    return pa;
  };
  EpiArgs sw;
  sw.out = w.h; sw.ldo = m->ff;
  PrepArgs pr;
  pr.N = nc; pr.bx = w.bx; pr.xs = w.xs; pr.cs = w.cs; pr.part = w.gpart; pr.eps = m->eps; pr.ssq = w.ssq;
  // Residual stream: embedding, then + partials of the pending o / down GEMV.
  uint32_t pending = 0, pending_ld = 0;
  auto resid_prep = [&](const float* norm_w) {
    pr.mode = PREP_RESID; pr.x = w.resid; pr.K = m->d; pr.norm_w = norm_w;
    pr.nparts = pending; pr.part_ld = pending_ld;
    pending = 0;
    cur = set0;
    return sh_prep_launch(e, pr);
  };
  // Fused residual preps (<= 2 columns, whole-K kernels whose operand fits in
  // LDS): QKV and gate/up build rmsnorm(resid + pending partials) themselves;
  // the residual alternates between resid and resid2 (resid after each layer).
  // A V matrix of its own needs the staged operand: no fused residual preps.
  const bool fuse_rp = fuse && swiglu_epilogue() && !m->layers.empty() && !any_wv &&
                       sh_gemv_resid_fusable(m->layers[0].wqkv, nc) && sh_gemv_resid_fusable(m->layers[0].wgu, nc);
  auto resid_src = [&](const float* rin, float* rout, const float* norm_w) {
    OpndSrc r;
    r.kind = OPND_RESID; r.x = rin; r.rout = rout; r.part = w.gpart; r.nparts = pending; r.part_ld = pending_ld;
    r.norm_w = norm_w; r.eps = m->eps;
    pending = 0;
    return r;
  };
  // Otherwise the o and down GEMVs finish the residual themselves (the last
  // workgroup of each output superblock runs its prep), writing set 1.
  const bool fuse_pp0 = fusion_enabled() && !fuse_rp;
  bool prepped = false;  // the operand of the next GEMV is built (set 1)
  auto prep_fuse = [&](const float* norm_w) {
    PrepFuse f;
    f.resid = w.resid; f.norm_w = norm_w; f.bx = w.bx2; f.xs = w.xs2; f.cs = w.cs2; f.ssq = w.ssq2;
    f.cnt = w.sb_cnt; f.K = m->d;
    return f;
  };
  // a matrix of the layers' type on the tuned GEMVs, another K-quant on the
  // multi-group GEMM (EPI_PART / EPI_STORE on the staged operand)
  auto gemv_any = [&](const QMat& q, const OpSet& op, EpiKind epi, const EpiArgs& ea, const char* tag,
                      uint32_t* np) {
    return tuned(q) ? sh_gemv_launch(e, q, op.bx, op.xs, nc, epi, ea, tag, np)
                    : sh_gemm_launch(e, q, op.bx, op.xs, op.cs, nc, epi, ea, tag, np);
  };
  for (uint32_t l = 0; l < m->n_layer; ++l) {
    const Layer& L = m->layers[l];
    qkv.layer = l;
    const bool fuse_pp = fuse_pp0 && sh_gemv_prep_fusable(L.wo) && tuned(L.wo);  // Wo's fused residual prep
    const bool fuse_ppd = fuse_pp0 && tuned(L.wdown) && sh_gemv_prep_fusable(L.wdown);  // down's
    const bool fuse_down = tuned(L.wdown) && sh_gemv_fusable(L.wdown) != 0;
    if (fuse_rp) {
      const OpndSrc rs = resid_src(w.resid, w.resid2, L.attn_norm);
      EpiArgs q2 = qkv;
      q2.cs = w.cs;
      q2.ssq = nullptr;  // the kernel applies the RMS factor it computed
      if ((rc = sh_gemv_launch(e, L.wqkv, w.bx, w.xs, nc, EPI_QKV, q2, "gemv_qkv", nullptr, &rs))) return rc;
    } else {
      if (!prepped && (rc = resid_prep(L.attn_norm))) return rc;
      set_norm(qkv);
      if ((rc = sh_gemv_launch(e, L.wqkv, cur.bx, cur.xs, nc, EPI_QKV, qkv, "gemv_qkv"))) return rc;
      if (L.wv.d) {  // V rows from a matrix of their own: split partials, then the cache rows
        EpiArgs pv = part_args(L.wv);
        set_norm(pv);
        uint32_t nv = 0;
        if ((rc = gemv_any(L.wv, cur, EPI_PART, pv, "gemv_v", &nv))) return rc;
        QkvCols qc;
        for (uint32_t j = 0; j < nc; ++j) {
          qc.pos[j] = cols[j].pos; qc.slot[j] = cols[j].slot; qc.mseq[j] = cols[j].kv->max_seq;
          qc.kc[j] = cols[j].kv->k; qc.vc[j] = cols[j].kv->v;
        }
        qc.vpart = pv.out; qc.vnparts = nv; qc.vldp = pv.ldo; qc.vstride = pv.part_stride;
        qc.row0 = m->d + dkv;  // the V rows only: q and k came out of the QKV epilogue
        if ((rc = sh_qkv_finish_launch(e, pv.out, nv, pv.part_stride, pv.ldo, nc, qkv, qc))) return rc;
      }
    }
    prepped = false;
    // one segment covering the chunk: Wo combines the attention splits itself
    // (cm1 attention builds the Wo operand in its own chain kernel)
    const bool fuse_o = !m->call_cm1 && fuse && !fuse_pp && segs.size() == 1 && segs[0].col0 == 0 &&
                        segs[0].ncol == nc && fuse_wo;
    OpndSrc osrc;
    for (const FaSeg& sg : segs) {
      FaArgs fa;
      fa.layer = l; fa.N = sg.ncol; fa.kvlen = sg.kvlen; fa.mask_base = sg.mask_base; fa.col0 = sg.col0;
      for (uint32_t j = 0; j < sg.ncol && j < 8; ++j) fa.colmask[j] = sg.colmask[j];
      fa.masks = sg.masks;
      fa.dbase = sg.kv->graph_base;
      fa.kv_cap = sg.kv->max_seq;
      rc = m->call_cm1 ? sh_fa16_launch(e, m, sg.kv, fa, w.q, w.attn, w.bx, w.xs, w.cs)
                       : sh_fa_launch(e, m, sg.kv, fa, w.q, w.fa_part, w.attn, w.bx, w.xs, w.cs,
                                      fuse_o ? &osrc : nullptr);
      if (rc) return rc;
    }
    EpiArgs po = part_args(L.wo);
    if (fuse_pp) {  // (Wo is always of the layers' type on this path)
      const PrepFuse pf = prep_fuse(L.ffn_norm);
      if ((rc = sh_gemv_launch(e, L.wo, w.bx, w.xs, nc, EPI_PART, po, "gemv_o", nullptr, nullptr, &pf))) return rc;
      pending = 0;
      cur = set1;
      prepped = true;
    } else {
      if ((rc = sh_gemv_launch(e, L.wo, w.bx, w.xs, nc, EPI_PART, po, "gemv_o", &pending, fuse_o ? &osrc : nullptr)))
        return rc;
      pending_ld = po.ldo;
    }
    OpndSrc dsrc;  // down reads h itself when it takes the split-K kernel
    bool down_ready = false;  // the gate/up kernel built the down operand (set 0)
    if (fuse_rp) {
      const OpndSrc rs = resid_src(w.resid2, w.resid, L.ffn_norm);
      EpiArgs s2 = sw;
      s2.cs = w.cs;
      s2.ssq = nullptr;
      if ((rc = sh_gemv_launch(e, L.wgu, w.bx, w.xs, nc, EPI_SWIGLU, s2, "gemv_gate_up", nullptr, &rs))) return rc;
      pr.mode = PREP_PLAIN; pr.x = w.h; pr.nparts = 0;
      if (fuse_down) { dsrc.kind = OPND_ROWS; dsrc.x = w.h; dsrc.ldx = m->ff; }
    } else if (!prepped && (rc = resid_prep(L.ffn_norm))) {
      return rc;
    } else if (swiglu_epilogue() && sh_gemv_ring_t(L.wgu)) {
      // whole sums from the deep-ring kernel (one split); SwiGLU in the down
      // prep, or (reading set 1) in the kernel's own last workgroups, which
      // write the down operand into set 0
      EpiArgs pg = part_args(L.wgu);
      set_norm(pg);
      PrepFuse sf;
      sf.bx = w.bx; sf.xs = w.xs; sf.cs = w.cs; sf.cnt = w.sb_cnt; sf.K = m->ff;
      const bool fuse_sw = prepped;  // gate/up reads set 1 (Wo's fused prep), so its tail may write set 0
      if ((rc = sh_gemv_ring_launch(e, L.wgu, cur.bx, cur.xs, nc, EPI_PART, pg, "gemv_gate_up",
                                    fuse_sw ? &sf : nullptr)))
        return rc;
      pr.mode = PREP_SWIGLU; pr.x = nullptr; pr.nparts = 1; pr.part_ld = pg.ldo;
      down_ready = fuse_sw;
    } else if (swiglu_epilogue()) {
      // whole sums in one kernel, h = silu(gate) * up in its epilogue
      set_norm(sw);
      if ((rc = sh_gemv_launch(e, L.wgu, cur.bx, cur.xs, nc, EPI_SWIGLU, sw, "gemv_gate_up"))) return rc;
      pr.mode = PREP_PLAIN; pr.x = w.h; pr.nparts = 0;
      if (fuse && fuse_down) { dsrc.kind = OPND_ROWS; dsrc.x = w.h; dsrc.ldx = m->ff; }
    } else {
      EpiArgs pg = part_args(L.wgu);
      set_norm(pg);
      uint32_t ngu = 0;
      if ((rc = sh_gemv_launch(e, L.wgu, cur.bx, cur.xs, nc, EPI_PART, pg, "gemv_gate_up", &ngu))) return rc;
      pr.mode = PREP_SWIGLU; pr.x = nullptr; pr.nparts = ngu; pr.part_ld = pg.ldo;
    }
    prepped = false;
    pr.K = m->ff; pr.norm_w = nullptr;
    if (dsrc.kind == OPND_STAGED && !down_ready && (rc = sh_prep_launch(e, pr))) return rc;
    cur = set0;
    EpiArgs pd = part_args(L.wdown);
    const float* next_norm = l + 1 < m->n_layer ? m->layers[l + 1].attn_norm : (want_logits ? m->out_norm : nullptr);
    if (fuse_ppd && next_norm && dsrc.kind == OPND_STAGED) {
      const PrepFuse pf = prep_fuse(next_norm);
      if ((rc = sh_gemv_launch(e, L.wdown, w.bx, w.xs, nc, EPI_PART, pd, "gemv_down", nullptr, nullptr, &pf)))
        return rc;
      pending = 0;
      cur = set1;
      prepped = true;
    } else if (!tuned(L.wdown)) {
      if ((rc = gemv_any(L.wdown, set0, EPI_PART, pd, "gemv_down", &pending))) return rc;
      pending_ld = pd.ldo;
    } else if (fuse_rp && l + 1 == m->n_layer && want_logits && dsrc.kind == OPND_ROWS &&
               sh_gemv_prep_fusable(L.wdown)) {
      // the last down of a 1-2 column chunk finishes the residual and the
      // lm_head's operand itself (set 1): no prep kernel before the lm_head
      const PrepFuse pf = prep_fuse(m->out_norm);
      if ((rc = sh_gemv_launch(e, L.wdown, w.bx, w.xs, nc, EPI_PART, pd, "gemv_down", nullptr, &dsrc, &pf)))
        return rc;
      pending = 0;
      cur = set1;
      prepped = true;
    } else {
      if ((rc = sh_gemv_launch(e, L.wdown, w.bx, w.xs, nc, EPI_PART, pd, "gemv_down", &pending,
                               dsrc.kind == OPND_STAGED ? nullptr : &dsrc)))
        return rc;
      pending_ld = pd.ldo;
    }
  }
  if (want_logits) {
    if (!prepped && (rc = resid_prep(m->out_norm))) return rc;
    EpiArgs st;
    st.out = w.logits; st.ldo = m->V; st.rows = m->V;
    set_norm(st);
    const bool lm_tuned = m->lm_head.type == GGML_Q4_K || m->lm_head.type == GGML_Q8_0;
    if ((rc = lm_tuned ? sh_gemv_launch(e, m->lm_head, cur.bx, cur.xs, nc, EPI_STORE, st, "gemv_lm_head")
                       : sh_gemm_launch(e, m->lm_head, cur.bx, cur.xs, cur.cs, nc, EPI_STORE, st, "gemv_lm_head",
                                        nullptr)))
      return rc;
  } else if (want_resid && pending) {
    if ((rc = sh_part_reduce_launch(e, w.gpart, pending, pending_ld, 8, m->d, nc, w.resid, m->d, true))) return rc;
  }
  return SH_OK;
}

// Routed-expert FFN of a qwen3moe layer over a chunk's nc columns
// (models/qwen35moe.rs:3117-3182 without the shared expert): w.resid holds x
// (attention added) and the staged operand x * ffn_norm with its RMS sums of
// squares. Router + top-k per column, the routing plan (pairs grouped by
// expert), gate/up of every routed expert over its columns (one pass over
// each active expert's slab), SwiGLU + down operand over the pairs, down,
// then the routing-weighted sum added to w.resid. With next_norm on a wide
// call the sum goes in with the next operand's f16 rows (w.bh, RMSNorm by
// next_norm) in one launch.
static int moe_ffn(sh_model* m, const Layer& L, uint32_t nc, const float* next_norm = nullptr) {
  sh_engine* e = m->e;
  Workspace& w = m->ws;
  const uint32_t k = m->n_used, P = nc * k, E = m->n_expert, mc = sh_moe_max_chunks(P, E);
  int rc;
  if ((rc = sh_moe_route_launch(e, w.resid, L.ffn_norm, L.router, m->d, E, m->eps, nc, w.moe_logits))) return rc;
  if ((rc = sh_moe_plan_launch(e, w.moe_logits, nc, E, k, w.moe_ids, w.moe_wts, w.moe_info, w.moe_col, w.moe_slot)))
    return rc;
  EpiArgs gu;
  gu.out = w.moe_hgu; gu.ldo = 2 * m->eff; gu.rows = 2 * m->eff;
  gu.ssq = w.ssq; gu.ssq_n = (m->d + 255) / 256; gu.norm_K = m->d; gu.eps = m->eps;
  if ((rc = sh_moe_gemm_launch(e, L.wgu_exps, E, w.bx, w.xs, w.cs, mc, w.moe_info, w.moe_col, gu, "moe_gate_up", 0.0)))
    return rc;
  PrepArgs pr;
  pr.mode = PREP_SWIGLU; pr.part = w.moe_hgu; pr.nparts = 1; pr.part_ld = 2 * m->eff; pr.part_cols = P;
  pr.K = m->eff; pr.N = P; pr.bx = w.moe_bx; pr.xs = w.moe_xs; pr.cs = w.moe_cs;
  if ((rc = sh_prep_launch(e, pr))) return rc;
  EpiArgs dn;
  dn.out = w.moe_y; dn.ldo = m->d; dn.rows = m->d;
  if ((rc = sh_moe_gemm_launch(e, L.wdown_exps, E, w.moe_bx, w.moe_xs, w.moe_cs, mc, w.moe_info, nullptr, dn,
                               "moe_down", 0.0)))
    return rc;
  if (next_norm && m->call16) {
    PrepArgs pc;
    pc.mode = PREP_MOE_COMBINE; pc.x = w.resid; pc.K = m->d; pc.N = nc; pc.norm_w = next_norm; pc.eps = m->eps;
    pc.bh = w.bh; pc.ldb = m->d;
    pc.moe_y = w.moe_y; pc.moe_slot = w.moe_slot; pc.moe_wts = w.moe_wts; pc.moe_k = k;
    return sh_prep_launch(e, pc);
  }
  return sh_moe_combine_launch(e, w.moe_y, w.moe_slot, w.moe_wts, k, m->d, nc, w.resid);
}

// Forward of 8 < nc <= SH_MAX_COLS columns when every matrix is Q4_K (and of
// any chunk of a qwen3 / qwen3moe model): each
// weight matrix is read once per chunk by sh_gemm_launch over ceil(nc / 8)
// operand groups. QKV, o, gate/up and down write split partials that the next
// step finishes (qkv_finish: RoPE + KV writes; residual prep; SwiGLU prep);
// attention runs per piece (FaSeg) of at most 8 columns of one sequence.
static int forward_chunk_mg(sh_model* m, const uint32_t* dev_tokens, uint32_t nc, const ColKv* cols,
                            const std::vector<FaSeg>& segs, bool want_logits, bool want_resid) {
  sh_engine* e = m->e;
  Workspace& w = m->ws;
  int rc;
  const uint32_t ncp = (nc + 7) / 8 * 8;  // columns per split in the partial buffer
  if ((rc = sh_embed_launch(e, m, dev_tokens, nc, w.resid))) return rc;
  // Operand the next GEMV reads: set 0 from the prep kernels and the attention
  // combine, set 1 from a residual prep fused into Wo / down (below).
  struct OpSet {
    uint16_t* bx;
    uint16_t* xs;
    float* cs;
    float* ssq;
  };
  const OpSet set0{w.bx, w.xs, w.cs, w.ssq}, set1{w.bx2, w.xs2, w.cs2, w.ssq2};
  OpSet cur = set0;
  // GEMVs whose input is RMS-normalized apply the norm factor to their outputs
  auto set_norm = [&](EpiArgs& ea) {
    ea.cs = cur.cs; ea.ssq = cur.ssq; ea.ssq_n = (m->d + 255) / 256; ea.norm_K = m->d; ea.eps = m->eps;
  };
  auto part_args = [&](const QMat& q) {
    EpiArgs pa;
    pa.out = w.gpart; pa.ldo = q.tiles * 16; pa.cs = w.cs;
    pa.part_stride = (size_t)ncp * pa.ldo;
    pa.part_cap = (uint32_t)(w.gpart_floats / pa.part_stride);
    return pa;
  };
  EpiArgs qkv;
  qkv.out = w.q; qkv.Dq = m->q_dim; qkv.Dkv = m->hd * m->n_kv; qkv.hd = m->hd; qkv.n_kv = m->n_kv; qkv.rope = m->rope;
  qkv.dbase = cols[0].kv->graph_base;  // graph capture: one cache per forward
  // The QKV finish takes its column table as a kernel argument, in pieces of at
  // most SH_MAX_COLS columns; a wider chunk of a non-NEOX model uploads the
  // table once (w.qtab, read by every layer) and finishes in one launch.
  const bool qtab = nc > SH_MAX_COLS && !m->neox;
  if (qtab) {
    std::vector<QkvColDev> t(nc);
    for (uint32_t j = 0; j < nc; ++j) {
      const ColKv& c = cols[j];
      t[j].pos = c.pos; t[j].slot = c.slot; t[j].mseq = c.kv->max_seq; t[j].pad = 0; t[j].kc = c.kv->k; t[j].vc = c.kv->v;
    }
    SH_HIP(hipMemcpyAsync(w.qtab, t.data(), (size_t)nc * sizeof(QkvColDev), hipMemcpyHostToDevice, e->stream));
  }
  auto qkv_finish = [&](const float* part, uint32_t np, size_t pstride, uint32_t ldp, const Layer& L,
                        const float* vpart, uint32_t vnp, uint32_t vldp, size_t vstride) {
    if (qtab) {
      QkvCols qc;
      qc.tab = w.qtab;
      if (vpart) { qc.vpart = vpart; qc.vnparts = vnp; qc.vldp = vldp; qc.vstride = vstride; }
      return sh_qkv_finish_launch(e, part, np, pstride, ldp, nc, qkv, qc);
    }
    for (uint32_t c0 = 0; c0 < nc; c0 += SH_MAX_COLS) {
      const uint32_t n = std::min<uint32_t>(SH_MAX_COLS, nc - c0);
      QkvCols qc;
      for (uint32_t j = 0; j < n; ++j) {
        const ColKv& c = cols[c0 + j];
        qc.pos[j] = c.pos; qc.slot[j] = c.slot; qc.mseq[j] = c.kv->max_seq; qc.kc[j] = c.kv->k; qc.vc[j] = c.kv->v;
      }
      if (vpart) { qc.vpart = vpart + (size_t)c0 * vldp; qc.vnparts = vnp; qc.vldp = vldp; qc.vstride = vstride; }
      EpiArgs q = qkv;
      q.out = qkv.out + (size_t)c0 * m->q_dim;
      const float* p0 = part + (size_t)c0 * ldp;
      const int rc = m->neox ? sh_qkv_finish_head_launch(e, p0, np, pstride, ldp, n, q, qc, L.q_norm, L.k_norm, m->eps,
                                                         true)
                             : sh_qkv_finish_launch(e, p0, np, pstride, ldp, n, q, qc);
      if (rc) return rc;
    }
    return (int)SH_OK;
  };
  // Wide calls (m->call16) stage f16 rows in w.bh and run every dense matmul
  // through sh_gemm16_launch; else the hi/lo operand groups and sh_gemm_launch.
  const bool f16 = m->call16;
  PrepArgs pr;
  pr.N = nc; pr.bx = w.bx; pr.xs = w.xs; pr.cs = w.cs; pr.part = w.gpart; pr.part_cols = ncp; pr.eps = m->eps;
  pr.ssq = w.ssq;
  if (f16) pr.bh = w.bh;
  uint32_t pending = 0, pending_ld = 0;
  auto resid_prep = [&](const float* norm_w) {
    pr.mode = PREP_RESID; pr.x = w.resid; pr.K = m->d; pr.norm_w = norm_w; pr.ldb = m->d;
    pr.nparts = pending; pr.part_ld = pending_ld;
    pending = 0;
    cur = set0;
    return sh_prep_launch(e, pr);
  };
  // At most 8 columns (one operand group), a Q4_K matrix takes the tuned GEMVs
  // of the fused path: the same split-partial layout and operand, and the
  // deep ring (one split) for the 8B-size gate/up. Mixed-type models
  // (Q4_K_M-style) and qwen3 chains keep this path for their structure and get
  // those kernels for their Q4_K matrices.
  static const bool tuned_small = [] {
    const char* s = getenv("SH_MG_TUNED");
    return !(s && atoi(s) == 0);
  }();
  auto gemm = [&](const QMat& q, const OpSet& op, EpiKind epi, const EpiArgs& ea, const char* tag, uint32_t* np) {
    if (f16) return sh_gemm16_launch(e, q, w.bh, q.K, nc, epi, ea, tag, np);
    if (tuned_small && nc <= 8 && q.type == GGML_Q4_K && (epi == EPI_PART || epi == EPI_STORE)) {
      if (epi == EPI_PART && sh_gemv_ring_t(q) && q.tiles % 7 == 0) {
        if (np) *np = 1;
        return sh_gemv_ring_launch(e, q, op.bx, op.xs, nc, EPI_PART, ea, tag, nullptr);
      }
      return sh_gemv_launch(e, q, op.bx, op.xs, nc, epi, ea, tag, np);
    }
    return sh_gemm_launch(e, q, op.bx, op.xs, op.cs, nc, epi, ea, tag, np);
  };
  // On those kernels a dense model's Wo and down finish the residual
  // themselves, as on the fused path: the last workgroup of each output
  // superblock adds the split partials, applies the next RMSNorm and writes
  // the operand into set 1, so no prep kernel runs between them and the next
  // GEMV (the arithmetic of the prep kernel, bit for bit).
  const bool pfuse = !f16 && tuned_small && nc <= 8 && !m->n_expert && fusion_enabled();
  auto prep_fusable = [&](const QMat& q) { return pfuse && q.type == GGML_Q4_K && sh_gemv_prep_fusable(q); };
  auto prep_fuse = [&](const float* norm_w) {
    PrepFuse pf;
    pf.resid = w.resid; pf.norm_w = norm_w; pf.bx = w.bx2; pf.xs = w.xs2; pf.cs = w.cs2; pf.ssq = w.ssq2;
    pf.cnt = w.sb_cnt; pf.K = m->d;
    return pf;
  };
  bool prepped = false;  // the operand of the next GEMV is built (set 1)
  // batched attention: one plan for the chunk's segments, one launch per layer
  // a causal single-sequence call (m->call_cm1): the chunk's columns as one
  // cm1 attention launch
  const bool cm1 = m->call_cm1;
  SH_CHECK(!cm1 || (segs.front().col0 == 0 && segs.back().col0 + segs.back().ncol == nc), SH_ERR_ARG,
           "cm1 attention: the segments must cover the chunk");
  FabGuard fab{e, FabLaunch{}};
  // one sequence's chain of at most 8 columns (the draft's forwards, graph
  // captures) takes the split attention with its masks as kernel arguments
  const bool single8 = segs.size() == 1 && segs[0].ncol <= 8;
  bool use_fab = !cm1 && fab_enabled() && !single8;
  for (const FaSeg& sg : segs) use_fab = use_fab && sg.hmasks;
  SH_CHECK(!qkv.dbase || cm1 || single8, SH_ERR_UNSUPPORTED, "graph capture: one chain of at most 8 columns");
  SH_CHECK(cm1 || use_fab || nc <= SH_MAX_COLS, SH_ERR_UNSUPPORTED,
           "chunks of more than %u columns need the batched attention (device masks)", SH_MAX_COLS);
  if (use_fab && (rc = plan_fab(m, segs, nc, &fab))) return rc;
  for (uint32_t l = 0; l < m->n_layer; ++l) {
    const Layer& L = m->layers[l];
    if (!prepped && (rc = resid_prep(L.attn_norm))) return rc;
    EpiArgs pq = part_args(L.wqkv);
    set_norm(pq);
    uint32_t nq = 0;
    if ((rc = gemm(L.wqkv, cur, EPI_PART, pq, "gemv_qkv", &nq))) return rc;
    const float* vpart = nullptr;
    uint32_t nv = 0, vldp = 0;
    size_t vstride = 0;
    if (L.wv.d) {  // v in a weight type of its own: its partials follow q / k's
      EpiArgs pv = part_args(L.wv);
      set_norm(pv);
      pv.out = w.gpart + nq * pq.part_stride;
      pv.part_cap = (uint32_t)((w.gpart_floats - nq * pq.part_stride) / pv.part_stride);
      if ((rc = gemm(L.wv, cur, EPI_PART, pv, "gemv_v", &nv))) return rc;
      vpart = pv.out; vldp = pv.ldo; vstride = pv.part_stride;
    }
    qkv.layer = l;
    prepped = false;
    cur = set0;  // the attention writes the Wo operand into set 0
    if ((rc = qkv_finish(w.gpart, nq, pq.part_stride, pq.ldo, L, vpart, nv, vldp, vstride))) return rc;
    if (cm1) {
      FaArgs fa;
      fa.layer = l; fa.N = nc; fa.col0 = 0; fa.kvlen = segs.back().kvlen; fa.mask_base = segs.front().mask_base;
      fa.dbase = segs.front().kv->graph_base;
      fa.kv_cap = segs.front().kv->max_seq;
      if ((rc = sh_fa16_launch(e, m, segs.front().kv, fa, w.q, w.attn, w.bx, w.xs, w.cs, f16 ? w.bh : nullptr)))
        return rc;
    } else if (use_fab) {
      if ((rc = sh_fab_launch(e, m, fab.fl, l, w.q, w.attn, w.bx, w.xs, w.cs, f16 ? w.bh : nullptr))) return rc;
    } else {
      for (const FaSeg& sg : segs) {
        FaArgs fa;
        fa.layer = l; fa.N = sg.ncol; fa.kvlen = sg.kvlen; fa.mask_base = sg.mask_base; fa.col0 = sg.col0;
        for (uint32_t j = 0; j < sg.ncol && j < 8; ++j) fa.colmask[j] = sg.colmask[j];
        fa.masks = sg.masks;
        fa.dbase = sg.kv->graph_base;
        fa.kv_cap = sg.kv->max_seq;
        if ((rc = sh_fa_launch(e, m, sg.kv, fa, w.q, w.fa_part, w.attn, w.bx, w.xs, w.cs))) return rc;
      }
      if (f16) {  // the attention rows as the Wo operand
        PrepArgs pa = pr;
        pa.mode = PREP_PLAIN; pa.x = w.attn; pa.K = m->q_dim; pa.ldb = m->q_dim; pa.norm_w = nullptr; pa.nparts = 0;
        if ((rc = sh_prep_launch(e, pa))) return rc;
      }
    }
    EpiArgs po = part_args(L.wo);
    if (prep_fusable(L.wo)) {
      const PrepFuse pf = prep_fuse(L.ffn_norm);
      if ((rc = sh_gemv_launch(e, L.wo, w.bx, w.xs, nc, EPI_PART, po, "gemv_o", nullptr, nullptr, &pf))) return rc;
      pending = 0;
      cur = set1;
      prepped = true;
    } else {
      if ((rc = gemm(L.wo, set0, EPI_PART, po, "gemv_o", &pending))) return rc;
      pending_ld = po.ldo;
    }
    if (m->n_expert && f16) {
      // the experts take the f32-level operand (the reference's expert matvec
      // is not its wide GEMM) and the router reads the residual, so one
      // f32-level prep adds Wo's partials and builds that operand (the f16
      // rows of a wide prep would go unread; same sums in the same order)
      PrepArgs px = pr;
      px.bh = nullptr; px.mode = PREP_RESID; px.x = w.resid; px.K = m->d; px.norm_w = L.ffn_norm;
      px.nparts = pending; px.part_ld = pending_ld;
      pending = 0;
      cur = set0;
      if ((rc = sh_prep_launch(e, px))) return rc;
    } else if (!prepped && (rc = resid_prep(L.ffn_norm))) {
      return rc;
    }
    if (m->n_expert) {  // routed experts add into the residual themselves
      // on a wide call the next operand's f16 rows come with the expert sum
      const float* next_norm =
          !f16 ? nullptr : (l + 1 < m->n_layer ? m->layers[l + 1].attn_norm : (want_logits ? m->out_norm : nullptr));
      if ((rc = moe_ffn(m, L, nc, next_norm))) return rc;
      prepped = next_norm != nullptr;
      cur = set0;
      continue;
    }
    EpiArgs pg = part_args(L.wgu);
    set_norm(pg);
    uint32_t ngu = 0;
    if ((rc = gemm(L.wgu, cur, EPI_PART, pg, "gemv_gate_up", &ngu))) return rc;
    prepped = false;
    cur = set0;
    pr.mode = PREP_SWIGLU; pr.x = nullptr; pr.nparts = ngu; pr.part_ld = pg.ldo; pr.K = m->ff; pr.norm_w = nullptr;
    pr.ldb = m->ff;
    if ((rc = sh_prep_launch(e, pr))) return rc;
    EpiArgs pd = part_args(L.wdown);
    const float* next_norm = l + 1 < m->n_layer ? m->layers[l + 1].attn_norm : (want_logits ? m->out_norm : nullptr);
    if (next_norm && prep_fusable(L.wdown)) {
      const PrepFuse pf = prep_fuse(next_norm);
      if ((rc = sh_gemv_launch(e, L.wdown, w.bx, w.xs, nc, EPI_PART, pd, "gemv_down", nullptr, nullptr, &pf)))
        return rc;
      pending = 0;
      cur = set1;
      prepped = true;
    } else {
      if ((rc = gemm(L.wdown, set0, EPI_PART, pd, "gemv_down", &pending))) return rc;
      pending_ld = pd.ldo;
    }
  }
  if (want_logits) {
    if (!prepped && (rc = resid_prep(m->out_norm))) return rc;
    EpiArgs st;
    st.out = w.logits; st.ldo = m->V; st.rows = m->V;
    set_norm(st);
    if ((rc = gemm(m->lm_head, cur, EPI_STORE, st, "gemv_lm_head", nullptr))) return rc;
  } else if (want_resid && pending) {
    if ((rc = sh_part_reduce_launch(e, w.gpart, pending, pending_ld, ncp, m->d, nc, w.resid, m->d, true))) return rc;
  }
  return SH_OK;
}

// Columns per forward chunk: SH_MAX_COLS when the multi-group path applies
// (all matrices K-quants) and takes the chunk (more than 8 columns, or a model
// the fused path cannot run), else 8.
static uint32_t chunk_cols(const sh_model* m, uint32_t n);

// Models whose forwards of up to 8 columns a HIP graph can capture: the fused
// path and the multi-group path (neither does host work between launches for
// such a chain).
static bool graph_model_ok(const sh_model* m) { return m->fused_ok || m->mg_ok; }

static uint32_t chunk_cols(const sh_model* m, uint32_t n) {
  static const bool forced8 = [] {
    const char* s = getenv("SH_CHUNK");
    return s && atoi(s) == 8;
  }();
  if (m->call16 && !forced8) return SH_MAX_COLS16;
  return (m->mg_ok && (n > 8 || !m->fused_ok) && !forced8) ? SH_MAX_COLS : 8;
}

// Longest attention segment on the multi-group path: SH_FA_MAX_ROWS query rows
// (gqa x columns) per kv head.
static uint32_t fa_seg_cols(const sh_model* m) {
  const uint32_t gqa = m->n_head / m->n_kv;
  return std::max<uint32_t>(8, std::min<uint32_t>(SH_MAX_COLS, (uint32_t)SH_FA_MAX_ROWS / gqa));
}

static int run_chunk(sh_model* m, const uint32_t* dev_tokens, uint32_t nc, const ColKv* cols,
                     const std::vector<FaSeg>& segs, bool want_logits, bool want_resid) {
  return (nc > 8 || !m->fused_ok || m->call16) ? forward_chunk_mg(m, dev_tokens, nc, cols, segs, want_logits, want_resid)
                                           : forward_chunk(m, dev_tokens, nc, cols, segs, want_logits, want_resid);
}

// Column geometry of a forward call: RoPE position, visibility mask and mask
// base per chunk. Causal chains: each chunk's columns see the cached prefix and
// earlier columns of the chunk (mask relative to the chunk start). Trees
// (L <= 64): positions = pos + depth, mask = ancestor-or-self relative to pos.
struct Plan {
  std::vector<int32_t> colpos;
  std::vector<uint64_t> mask;
  bool tree = false;
};

static int make_plan(uint32_t L, uint32_t pos, const int32_t* parents, Plan* p) {
  p->colpos.resize(L);
  p->mask.resize(L);
  p->tree = parents != nullptr;
  if (!parents) {
    for (uint32_t i = 0; i < L; ++i) {
      p->colpos[i] = (int32_t)(pos + i);
      const uint32_t j = i % 8;
      p->mask[i] = (j == 63) ? ~0ull : ((2ull << j) - 1ull);
    }
    return SH_OK;
  }
  SH_CHECK(L <= 64, SH_ERR_UNSUPPORTED, "tree verify supports at most 64 nodes (got %u)", L);
  for (uint32_t i = 0; i < L; ++i) {
    SH_CHECK(parents[i] < (int32_t)i, SH_ERR_ARG, "tree parent[%u]=%d must precede the node", i, parents[i]);
    uint64_t mk = 1ull << i;
    uint32_t depth = 0;
    if (parents[i] >= 0) {
      mk |= p->mask[parents[i]];
      depth = (uint32_t)(p->colpos[parents[i]] - (int32_t)pos) + 1;
    }
    p->mask[i] = mk;
    p->colpos[i] = (int32_t)(pos + depth);
  }
  return SH_OK;
}

// Grows the attention partial buffer for keys [0, max_kvlen).
static int ensure_fa_part(sh_model* m, uint32_t max_kvlen) {
  const uint32_t needed_splits = (max_kvlen + SH_FA_MIN_SPLIT_KEYS - 1) / SH_FA_MIN_SPLIT_KEYS;
  const size_t need = (size_t)m->n_kv * needed_splits * SH_FA_MAX_ROWS * sh_fa_part_stride(m->hd);
  if (need <= m->ws.fa_part_floats) return SH_OK;
  g_graph_gen.fetch_add(1);  // captured graphs may point into the old buffer
  SH_HIP(hipStreamSynchronize(m->e->stream));
  SH_HIP(hipFree(m->ws.fa_part));
  m->ws.fa_part = nullptr;
  SH_HIP(hipMalloc(&m->ws.fa_part, need * 4));
  m->ws.fa_part_floats = need;
  return SH_OK;
}

// Grows the cm1 attention buffers for chunks of up to ncol columns over keys
// [0, kv_cap). Captured graphs may point into the old buffers: they are
// dropped.
static int ensure_fa16(sh_model* m, uint32_t kv_cap, uint32_t ncol) {
  const uint32_t gqa = m->n_head / m->n_kv;
  Workspace& w = m->ws;
  const size_t pvh = sh_fa16_pv_halves(m->n_kv, m->hd, gqa, ncol, kv_cap);
  const size_t sw = sh_fa16_sync_words(m->n_kv, gqa, ncol, kv_cap);
  if (pvh <= w.fa16_pv_halves && sw <= w.fa16_sync_words) return SH_OK;
  const size_t P = std::max(pvh, w.fa16_pv_halves), W = std::max(sw, w.fa16_sync_words);
  g_graph_gen.fetch_add(1);
  SH_HIP(hipStreamSynchronize(m->e->stream));
  (void)hipFree(w.fa16_pv); (void)hipFree(w.fa16_ml); (void)hipFree(w.fa16_smax); (void)hipFree(w.fa16_flag);
  w.fa16_pv = nullptr; w.fa16_ml = nullptr; w.fa16_smax = nullptr; w.fa16_flag = nullptr;
  w.fa16_pv_halves = w.fa16_sync_words = 0;
  SH_HIP(hipMalloc(&w.fa16_pv, P * 2));
  SH_HIP(hipMalloc(&w.fa16_ml, P / m->hd * sizeof(float2)));
  SH_HIP(hipMalloc(&w.fa16_smax, W * 32 * sizeof(float)));
  SH_HIP(hipMalloc(&w.fa16_flag, (W + 1) * sizeof(uint32_t)));
  SH_HIP(hipMemsetAsync(w.fa16_flag, 0, (W + 1) * sizeof(uint32_t), m->e->stream));
  SH_HIP(hipMemsetAsync(w.fa16_smax, 0xFF, W * 32 * sizeof(float), m->e->stream));  // look-back words unset
  w.fa16_pv_halves = P;
  w.fa16_sync_words = W;
  return SH_OK;
}

// Runs the whole forward for L columns whose ids are at dev_tokens. If
// logits_dst != null, copies logits of the selected columns there (device).
static int forward_dev(sh_model* m, sh_kv* kv, const uint32_t* dev_tokens, uint32_t L, uint32_t pos,
                       const int32_t* parents, int logits_mode, float* logits_dev_out, float* resid_host,
                       float* logits_host) {
  sh_engine* e = m->e;
  SH_CHECK(L >= 1, SH_ERR_ARG, "empty prompt");
  const bool graph = kv->graph_base != nullptr;  // pos is an offset from *graph_base at replay
  SH_CHECK(graph || kv->pos == pos, SH_ERR_STATE,
           "cache.position %u doesn't match caller-supplied position_offset %u", kv->pos, pos);
  SH_CHECK(!graph || (L <= 8 && !parents && graph_model_ok(m)), SH_ERR_UNSUPPORTED,
           "graph capture: chains of at most 8 columns");
  SH_CHECK(kv->n_layer == m->n_layer && kv->n_kv == m->n_kv && kv->hd == m->hd, SH_ERR_ARG,
           "KV cache dims do not match the model");
  SH_CHECK((uint64_t)pos + L <= kv->max_seq, SH_ERR_CAPACITY, "positions [%u, %u) exceed KV capacity %u", pos,
           pos + L, kv->max_seq);
  Plan plan;
  int rc = make_plan(L, pos, parents, &plan);
  if (rc) return rc;
  uint32_t maxpos = 0;
  for (auto p : plan.colpos) maxpos = std::max<uint32_t>(maxpos, (uint32_t)p);
  if (!graph) {  // a capture sizes both for the cache capacity beforehand
    if ((rc = ensure_rope(m, maxpos + 1))) return rc;
    if ((rc = ensure_fa_part(m, pos + L))) return rc;
  }
  m->call16 = m->wide16 && L >= SH_WIDE16_COLS;  // one matmul of L columns in the reference
  // a masked forward of more than one token: the reference's cm1 attention
  // (models/llama.rs:216-222, ops/flash_attn.rs:442-471)
  m->call_cm1 = m->fa16 && L > 1 && !parents;
  const uint32_t CW = chunk_cols(m, L);
  if (m->call_cm1 && !graph && (rc = ensure_fa16(m, pos + L, std::min(L, CW)))) return rc;
  // Attention: one segment per chunk (device masks) on the multi-group path,
  // else pieces of <= 8 columns; a causal segment's masks are relative to its
  // first column.
  std::vector<uint64_t> hmask(L);
  std::vector<std::vector<FaSeg>> chunk_segs;
  for (uint32_t c0 = 0; c0 < L; c0 += CW) {
    const uint32_t nc = std::min<uint32_t>(CW, L - c0), piece = CW > 8 ? fa_seg_cols(m) : 8;
    std::vector<FaSeg> segs;
    for (uint32_t j0 = 0; j0 < nc; j0 += piece) {
      FaSeg sg;
      sg.kv = kv; sg.col0 = j0; sg.ncol = std::min<uint32_t>(piece, nc - j0); sg.kvlen = pos + c0 + j0 + sg.ncol;
      sg.mask_base = plan.tree ? pos : pos + c0 + j0;
      for (uint32_t t = 0; t < sg.ncol; ++t) {
        const uint64_t mk = plan.tree ? plan.mask[c0 + j0 + t] : (t == 63 ? ~0ull : (2ull << t) - 1ull);
        hmask[c0 + j0 + t] = mk;
        if (t < 8) sg.colmask[t] = mk;
      }
      sg.hmasks = hmask.data() + c0 + j0;
      segs.push_back(sg);
    }
    chunk_segs.push_back(segs);
  }
  uint64_t* dmask = nullptr;
  if (CW > 8 && !m->call_cm1 && L > 8) {  // <= 8 columns: one segment, masks as kernel arguments
    SH_HIP(hipMallocAsync((void**)&dmask, (size_t)L * 8, e->stream));
    SH_HIP(hipMemcpyAsync(dmask, hmask.data(), (size_t)L * 8, hipMemcpyHostToDevice, e->stream));
    for (size_t c = 0; c < chunk_segs.size(); ++c)
      for (FaSeg& sg : chunk_segs[c]) sg.masks = dmask + c * CW + sg.col0;
  }
  struct MaskFree {  // the masks stay allocated until every launch that reads them is queued
    sh_engine* e; uint64_t* p;
    ~MaskFree() { if (p) (void)hipFreeAsync(p, e->stream); }
  } mask_free{e, dmask};
  for (uint32_t c0 = 0; c0 < L; c0 += CW) {
    const uint32_t nc = std::min<uint32_t>(CW, L - c0);
    const bool last = c0 + nc == L;
    const bool want = logits_mode == 2 || (logits_mode == 1 && last);
    std::vector<ColKv> cols(nc);
    for (uint32_t j = 0; j < nc; ++j) {
      cols[j].kv = kv; cols[j].slot = pos + c0 + j; cols[j].pos = plan.colpos[c0 + j];
    }
    const std::vector<FaSeg>& segs = chunk_segs[c0 / CW];
    if ((rc = run_chunk(m, dev_tokens + c0, nc, cols.data(), segs, want, resid_host != nullptr))) return rc;
    if (resid_host)
      SH_HIP(hipMemcpyAsync(resid_host + (size_t)c0 * m->d, m->ws.resid, (size_t)nc * m->d * 4,
                            hipMemcpyDeviceToHost, e->stream));
    if (want) {
      const uint32_t j0 = logits_mode == 1 ? nc - 1 : 0;
      const uint32_t ncopy = nc - j0;
      const uint32_t dst_col = logits_mode == 1 ? 0 : c0;
      if (logits_dev_out)
        SH_HIP(hipMemcpyAsync(logits_dev_out + (size_t)dst_col * m->V, m->ws.logits + (size_t)j0 * m->V,
                              (size_t)ncopy * m->V * 4, hipMemcpyDeviceToDevice, e->stream));
      if (logits_host)
        SH_HIP(hipMemcpyAsync(logits_host + (size_t)dst_col * m->V, m->ws.logits + (size_t)j0 * m->V,
                              (size_t)ncopy * m->V * 4, hipMemcpyDeviceToHost, e->stream));
    }
    if (resid_host || logits_host) SH_HIP(hipStreamSynchronize(e->stream));
  }
  if (!graph) kv->pos = pos + L;
  return SH_OK;
}

static int upload_tokens(sh_model* m, const uint32_t* tokens, uint32_t L, uint32_t** dev) {
  uint32_t* d = nullptr;
  SH_CHECK(tokens, SH_ERR_ARG, "tokens is NULL");
  for (uint32_t i = 0; i < L; ++i)
    SH_CHECK(tokens[i] < m->V, SH_ERR_ARG, "token id %u out of range (vocab %u)", tokens[i], m->V);
  SH_HIP(hipMalloc(&d, (size_t)L * 4));
  SH_HIP(hipMemcpyAsync(d, tokens, (size_t)L * 4, hipMemcpyHostToDevice, m->e->stream));
  *dev = d;
  return SH_OK;
}

extern "C" int sh_forward_full(sh_engine* e, sh_model* m, sh_kv* kv, const uint32_t* tokens, uint32_t L,
                               uint32_t pos, const int32_t* parents, int logits_mode, float* logits_out,
                               float* residual_out) {
  SH_CHECK(e && m && kv, SH_ERR_ARG, "sh_forward_full: NULL handle");
  SH_CHECK(logits_mode >= 0 && logits_mode <= 2, SH_ERR_ARG, "logits_mode %d", logits_mode);
  SH_CHECK(L >= 1, SH_ERR_ARG, "empty prompt");
  uint32_t* dt = nullptr;
  int rc = upload_tokens(m, tokens, L, &dt);
  if (rc) return rc;
  rc = forward_dev(m, kv, dt, L, pos, parents, logits_mode, nullptr, residual_out,
                   logits_mode ? logits_out : nullptr);
  hipError_t se = hipStreamSynchronize(e->stream);
  (void)hipFree(dt);
  if (rc) return rc;
  SH_CHECK(se == hipSuccess, SH_ERR_HIP, "forward: %s", hipGetErrorString(se));
  kv->pending.clear();
  return sh_prof_flush(e);
}

static int spec_bufs(sh_engine* e, uint32_t V);
static bool graphs_enabled(const sh_engine* e);
static hipGraphExec_t graph_find(sh_engine* e, const std::vector<uintptr_t>& key);
static int graph_capture(sh_engine* e, const std::vector<uintptr_t>& key, const std::vector<sh_kv*>& kvs,
                         const std::vector<const uint32_t*>& bases, const std::function<int()>& body,
                         hipGraphExec_t* out);
static int graph_launch(sh_engine* e, hipGraphExec_t ex);

// Greedy verify of up to 8 tokens by graph replay: tokens staged at tok[32..],
// ids at samp[0..], base position at base[2].
static int verify_greedy_graph(sh_engine* e, sh_model* m, sh_kv* kv, const uint32_t* tokens, uint32_t L,
                               uint32_t pos, uint32_t* sampled_out) {
  int rc = spec_bufs(e, m->V);
  if (rc) return rc;
  uint32_t* hp = e->spec.pinned;
  for (uint32_t i = 0; i < L; ++i) hp[32 + i] = tokens[i];
  hp[66] = pos;
  const std::vector<uintptr_t> key = {2, (uintptr_t)m, (uintptr_t)kv, (uintptr_t)kv->k, kv->max_seq, L, m->fa16};
  hipGraphExec_t ex = graph_find(e, key);
  if (!ex) {
    if ((rc = ensure_rope(m, kv->max_seq)) || (rc = ensure_fa_part(m, kv->max_seq)) ||
        (rc = ensure_fa16(m, kv->max_seq, L)))
      return rc;
    rc = graph_capture(e, key, {kv}, {e->spec.base + 2}, [&] {
      int r = forward_dev(m, kv, e->spec.tok + 32, L, 0, nullptr, 2, nullptr, nullptr, nullptr);
      if (!r) r = sh_argmax_launch(e, m->ws.logits, m->V, L, m->ws.amax, e->spec.samp);
      if (!r && hipMemcpyAsync(e->spec.pinned + 48, e->spec.samp, (size_t)L * 4, hipMemcpyDeviceToHost,
                               e->stream) != hipSuccess) {
        sh_set_error("verify readback capture failed");
        r = SH_ERR_HIP;
      }
      return r;
    }, &ex);
    if (rc) return rc;
  }
  SH_HIP(hipMemcpyAsync(e->spec.tok + 32, hp + 32, (size_t)L * 4, hipMemcpyHostToDevice, e->stream));
  SH_HIP(hipMemcpyAsync(e->spec.base + 2, hp + 66, 4, hipMemcpyHostToDevice, e->stream));
  if ((rc = graph_launch(e, ex))) return rc;
  SH_HIP(hipStreamSynchronize(e->stream));
  for (uint32_t i = 0; i < L; ++i) sampled_out[i] = hp[48 + i];
  kv->pos = pos + L;
  kv->pending.clear();
  return SH_OK;
}

extern "C" int sh_verify_greedy(sh_engine* e, sh_model* m, sh_kv* kv, const uint32_t* tokens, uint32_t L,
                                uint32_t pos, uint32_t* sampled_out) {
  SH_CHECK(e && m && kv && sampled_out, SH_ERR_ARG, "sh_verify_greedy: NULL argument");
  SH_CHECK(L >= 1 && L <= 64, SH_ERR_ARG, "verify length %u outside [1, 64]", L);
  if (L <= 8 && graphs_enabled(e) && graph_model_ok(m)) {
    SH_CHECK(tokens, SH_ERR_ARG, "tokens is NULL");
    for (uint32_t i = 0; i < L; ++i)
      SH_CHECK(tokens[i] < m->V, SH_ERR_ARG, "token id %u out of range (vocab %u)", tokens[i], m->V);
    SH_CHECK(kv->pos == pos, SH_ERR_STATE, "cache.position %u doesn't match caller-supplied position_offset %u",
             kv->pos, pos);
    SH_CHECK((uint64_t)pos + L <= kv->max_seq, SH_ERR_CAPACITY, "positions [%u, %u) exceed KV capacity %u", pos,
             pos + L, kv->max_seq);
    SH_CHECK(kv->n_layer == m->n_layer && kv->n_kv == m->n_kv && kv->hd == m->hd, SH_ERR_ARG,
             "KV cache dims do not match the model");
    return verify_greedy_graph(e, m, kv, tokens, L, pos, sampled_out);
  }
  uint32_t* dt = nullptr;
  int rc = upload_tokens(m, tokens, L, &dt);
  if (rc) return rc;
  float* lg = nullptr;
  SH_HIP(hipMallocAsync((void**)&lg, (size_t)L * m->V * 4, e->stream));
  uint32_t* ids = nullptr;
  SH_HIP(hipMallocAsync((void**)&ids, 64 * 4, e->stream));
  rc = forward_dev(m, kv, dt, L, pos, nullptr, 2, lg, nullptr, nullptr);
  if (!rc) rc = sh_argmax_launch(e, lg, m->V, L, m->ws.amax, ids);
  if (!rc) {
    hipError_t ce = hipMemcpyAsync(sampled_out, ids, (size_t)L * 4, hipMemcpyDeviceToHost, e->stream);
    if (ce != hipSuccess) { sh_set_error("verify readback: %s", hipGetErrorString(ce)); rc = SH_ERR_HIP; }
  }
  hipError_t se = hipStreamSynchronize(e->stream);
  (void)hipFree(dt);
  (void)hipFreeAsync(lg, e->stream);
  (void)hipFreeAsync(ids, e->stream);
  if (rc) return rc;
  SH_CHECK(se == hipSuccess, SH_ERR_HIP, "verify: %s", hipGetErrorString(se));
  kv->pending.clear();
  return sh_prof_flush(e);
}

// Batched verify; logits go to the host (logits_out) and/or the device
// (logits_dev, [N_total][V]).
static int verify_unified_impl(sh_engine* e, sh_model* m, sh_kv* const* caches, uint32_t B, const uint32_t* tokens,
                               const uint32_t* seq_lens, const uint32_t* positions, const int32_t* parents,
                               float* logits_out, float* logits_dev, uint32_t* sampled_out, float* residual_out,
                               sh_sampling* samplers = nullptr) {
  SH_CHECK(e && m && caches && tokens && seq_lens, SH_ERR_ARG, "sh_verify_unified: NULL argument");
  SH_CHECK(B >= 1, SH_ERR_ARG, "verify_unified: empty batch");
  // per-sequence samplers: GREEDY (argmax) or COMPARE-style temperature
  // sampling of every column (REJECTION needs draft logits: sh_accept_sample)
  bool any_stoch = false;
  if (samplers)
    for (uint32_t s = 0; s < B; ++s) {
      const sh_sampling& sp = samplers[s];
      SH_CHECK(sp.mode == SH_SAMPLE_GREEDY || sp.mode == SH_SAMPLE_COMPARE, SH_ERR_ARG,
               "verify_unified: sequence %u sampler mode %u (GREEDY or COMPARE)", s, sp.mode);
      SH_CHECK(sp.mode == SH_SAMPLE_GREEDY || sp.temperature > 0.f, SH_ERR_ARG,
               "verify_unified: sequence %u temperature %g", s, (double)sp.temperature);
      if (sp.mode == SH_SAMPLE_COMPARE) {
        SampRow chk{};
        if (int frc = sh_samprow_filters(sp, m->V, chk)) return frc;
      }
      any_stoch = any_stoch || sp.mode == SH_SAMPLE_COMPARE;
    }
  SH_CHECK(!any_stoch || sampled_out, SH_ERR_ARG, "verify_unified: samplers without sampled_out");
  // prefix-sum column starts (q_starts) and per-sequence plans
  std::vector<uint32_t> q0(B + 1, 0);
  std::vector<Plan> plans(B);
  uint32_t max_kv = 0, maxpos = 0;
  int rc;
  for (uint32_t s = 0; s < B; ++s) {
    sh_kv* kv = caches[s];
    SH_CHECK(kv, SH_ERR_ARG, "verify_unified: cache %u is NULL", s);
    for (uint32_t t = 0; t < s; ++t)
      SH_CHECK(caches[t] != kv, SH_ERR_ARG, "verify_unified: sequences %u and %u share a cache", t, s);
    SH_CHECK(kv->n_layer == m->n_layer && kv->n_kv == m->n_kv && kv->hd == m->hd, SH_ERR_ARG,
             "verify_unified: cache %u dims do not match the model", s);
    const uint32_t L = seq_lens[s];
    SH_CHECK(L >= 1, SH_ERR_ARG, "verify_unified: sequence %u is empty", s);
    SH_CHECK((uint64_t)kv->pos + L <= kv->max_seq, SH_ERR_CAPACITY,
             "verify_unified: sequence %u positions [%u, %u) exceed KV capacity %u", s, kv->pos, kv->pos + L,
             kv->max_seq);
    q0[s + 1] = q0[s] + L;
    if ((rc = make_plan(L, kv->pos, parents ? parents + q0[s] : nullptr, &plans[s]))) return rc;
    if (positions)
      for (uint32_t i = 0; i < L; ++i)
        SH_CHECK(positions[q0[s] + i] == (uint32_t)plans[s].colpos[i], SH_ERR_ARG,
                 "verify_unified: positions[%u] = %u, expected %d", q0[s] + i, positions[q0[s] + i],
                 plans[s].colpos[i]);
    max_kv = std::max(max_kv, kv->pos + L);
    for (auto p : plans[s].colpos) maxpos = std::max<uint32_t>(maxpos, (uint32_t)p);
  }
  const uint32_t N = q0[B];
  if ((rc = ensure_rope(m, maxpos + 1))) return rc;
  if ((rc = ensure_fa_part(m, max_kv))) return rc;
  // flat columns: cache, slot, RoPE position, owning sequence, index within it
  std::vector<ColKv> cols(N);
  std::vector<uint32_t> cseq(N), cidx(N);
  for (uint32_t s = 0; s < B; ++s)
    for (uint32_t i = 0; i < seq_lens[s]; ++i) {
      const uint32_t j = q0[s] + i;
      cols[j].kv = caches[s]; cols[j].slot = caches[s]->pos + i; cols[j].pos = plans[s].colpos[i];
      cseq[j] = s; cidx[j] = i;
    }
  uint32_t* dt = nullptr;
  if ((rc = upload_tokens(m, tokens, N, &dt))) return rc;
  uint32_t* ids = nullptr;
  if (sampled_out) SH_HIP(hipMallocAsync((void**)&ids, SH_MAX_COLS16 * 4, e->stream));
  const bool want_logits = logits_out || logits_dev || sampled_out;
  m->call16 = m->wide16 && N >= SH_WIDE16_COLS;  // the reference's batch is one matmul of N columns
  m->call_cm1 = false;  // the batched attention is the reference's scalar kernel (ops/flash_attn.rs:819-1016)
  const uint32_t CW = chunk_cols(m, N);
  // attention segments: runs of one sequence's columns in a chunk (at most 8
  // each on the 8-column path; device masks on the multi-group path)
  std::vector<uint64_t> hmask(N);
  std::vector<std::vector<FaSeg>> chunk_segs;
  for (uint32_t c0 = 0; c0 < N; c0 += CW) {
    const uint32_t nc = std::min<uint32_t>(CW, N - c0), piece = CW > 8 ? fa_seg_cols(m) : 8;
    std::vector<FaSeg> segs;
    for (uint32_t j = 0; j < nc;) {
      const uint32_t s = cseq[c0 + j], i0 = cidx[c0 + j];
      uint32_t n = 1;
      while (j + n < nc && n < piece && cseq[c0 + j + n] == s) ++n;
      FaSeg sg;
      sg.kv = caches[s]; sg.col0 = j; sg.ncol = n;
      sg.kvlen = caches[s]->pos + i0 + n;
      sg.mask_base = plans[s].tree ? caches[s]->pos : caches[s]->pos + i0;
      for (uint32_t t = 0; t < n; ++t) {
        const uint64_t mk = plans[s].tree ? plans[s].mask[i0 + t] : (t == 63 ? ~0ull : (2ull << t) - 1ull);
        hmask[c0 + j + t] = mk;
        if (t < 8) sg.colmask[t] = mk;
      }
      sg.hmasks = hmask.data() + c0 + j;
      segs.push_back(sg);
      j += n;
    }
    chunk_segs.push_back(segs);
  }
  uint64_t* dmask = nullptr;
  if (CW > 8) {
    SH_HIP(hipMallocAsync((void**)&dmask, (size_t)N * 8, e->stream));
    SH_HIP(hipMemcpyAsync(dmask, hmask.data(), (size_t)N * 8, hipMemcpyHostToDevice, e->stream));
    for (size_t c = 0; c < chunk_segs.size(); ++c)
      for (FaSeg& sg : chunk_segs[c]) sg.masks = dmask + c * CW + sg.col0;
  }
  for (uint32_t c0 = 0; c0 < N && !rc; c0 += CW) {
    const uint32_t nc = std::min<uint32_t>(CW, N - c0);
    const std::vector<FaSeg>& segs = chunk_segs[c0 / CW];
    rc = run_chunk(m, dt + c0, nc, cols.data() + c0, segs, want_logits, residual_out != nullptr);
    if (rc) break;
    if (residual_out)
      SH_HIP(hipMemcpyAsync(residual_out + (size_t)c0 * m->d, m->ws.resid, (size_t)nc * m->d * 4,
                            hipMemcpyDeviceToHost, e->stream));
    if (logits_out)
      SH_HIP(hipMemcpyAsync(logits_out + (size_t)c0 * m->V, m->ws.logits, (size_t)nc * m->V * 4,
                            hipMemcpyDeviceToHost, e->stream));
    if (logits_dev)
      SH_HIP(hipMemcpyAsync(logits_dev + (size_t)c0 * m->V, m->ws.logits, (size_t)nc * m->V * 4,
                            hipMemcpyDeviceToDevice, e->stream));
    if (sampled_out) {
      if ((rc = sh_argmax_launch(e, m->ws.logits, m->V, nc, m->ws.amax, ids))) break;
      if (any_stoch) {
        // column c of sequence s (its j-th): uniform j of s's explicit array,
        // else Philox word counter + j of key (seed, 0x5EC)
        std::vector<SampRow> rows(nc);
        bool chunk_plain = false, chunk_filt = false;
        for (uint32_t c = 0; c < nc; ++c) {
          const uint32_t sq = cseq[c0 + c], j = cidx[c0 + c];
          const sh_sampling& sp = samplers[sq];
          SampRow& r = rows[c];
          r = SampRow{};
          r.greedy = sp.mode == SH_SAMPLE_GREEDY ? 1u : 0u;
          r.inv_t = r.greedy ? 1.0 : 1.0 / (double)sp.temperature;
          r.seed = sp.seed;
          r.word = sp.counter + j;
          r.explicit_u = sp.uniforms ? 1u : 0u;
          r.u = sp.uniforms ? sp.uniforms[j] : 0.f;
          if (!r.greedy) (void)sh_samprow_filters(sp, m->V, r);  // checked before the forward
          chunk_plain = chunk_plain || (!r.greedy && !r.top_k);
          chunk_filt = chunk_filt || (!r.greedy && r.top_k);
        }
        if (chunk_plain || chunk_filt) {
          SampRow* rdev = nullptr;
          double2* part = nullptr;
          SH_HIP(hipMallocAsync((void**)&rdev, nc * sizeof(SampRow), e->stream));
          SH_HIP(hipMallocAsync((void**)&part, sh_sample_rows_part_bytes(nc, m->V), e->stream));
          SH_HIP(hipMemcpyAsync(rdev, rows.data(), nc * sizeof(SampRow), hipMemcpyHostToDevice, e->stream));
          rc = sh_sample_rows_tab_launch(e, m->ws.logits, nc, m->V, rdev, part, ids, chunk_plain, chunk_filt);
          (void)hipFreeAsync(rdev, e->stream);
          (void)hipFreeAsync(part, e->stream);
          if (rc) break;
        }
      }
      SH_HIP(hipMemcpyAsync(sampled_out + c0, ids, (size_t)nc * 4, hipMemcpyDeviceToHost, e->stream));
    }
  }
  hipError_t se = hipStreamSynchronize(e->stream);
  (void)hipFree(dt);
  if (ids) (void)hipFree(ids);
  if (dmask) (void)hipFree(dmask);
  if (rc) return rc;
  SH_CHECK(se == hipSuccess, SH_ERR_HIP, "verify_unified: %s", hipGetErrorString(se));
  for (uint32_t s = 0; s < B; ++s) {
    caches[s]->pos += seq_lens[s];
    caches[s]->pending.clear();
    if (samplers && samplers[s].mode == SH_SAMPLE_COMPARE) samplers[s].counter += seq_lens[s];
  }
  return sh_prof_flush(e);
}

extern "C" int sh_verify_unified(sh_engine* e, sh_model* m, sh_kv* const* caches, uint32_t B,
                                 const uint32_t* tokens, const uint32_t* seq_lens, const uint32_t* positions,
                                 const int32_t* parents, float* logits_out, uint32_t* sampled_out,
                                 float* residual_out) {
  return verify_unified_impl(e, m, caches, B, tokens, seq_lens, positions, parents, logits_out, nullptr, sampled_out,
                             residual_out);
}

extern "C" int sh_verify_unified_sampled(sh_engine* e, sh_model* m, sh_kv* const* caches, uint32_t B,
                                         const uint32_t* tokens, const uint32_t* seq_lens, const uint32_t* positions,
                                         const int32_t* parents, sh_sampling* samplers, float* logits_out,
                                         uint32_t* sampled_out, float* residual_out) {
  return verify_unified_impl(e, m, caches, B, tokens, seq_lens, positions, parents, logits_out, nullptr, sampled_out,
                             residual_out, samplers);
}

extern "C" int sh_tree_verify_step(sh_engine* e, sh_model* target, sh_kv* const* caches, uint32_t B, uint32_t n,
                                   const uint32_t* tokens, const int32_t* parents, const float* q_logits_dev,
                                   const sh_sampling* s, uint32_t* path_out, uint32_t* path_len_out,
                                   uint32_t* next_tok_out) {
  SH_CHECK(e && target && caches && tokens && parents && s && path_out && path_len_out && next_tok_out, SH_ERR_ARG,
           "sh_tree_verify_step: NULL argument");
  SH_CHECK(B >= 1 && n >= 1 && n <= 64, SH_ERR_ARG, "tree_verify_step: B=%u n=%u (n <= 64)", B, n);
  const uint32_t V = target->V;
  std::vector<uint32_t> lens(B, n), base(B);
  for (uint32_t b = 0; b < B; ++b) {
    SH_CHECK(caches[b], SH_ERR_ARG, "tree_verify_step: cache %u is NULL", b);
    base[b] = caches[b]->pos;
  }
  float* lg = nullptr;
  uint32_t *dtok = nullptr, *dpath = nullptr, *dlen = nullptr, *dnext = nullptr;
  int32_t* dpar = nullptr;
  SH_HIP(hipMallocAsync((void**)&lg, (size_t)B * n * V * 4, e->stream));
  int rc = verify_unified_impl(e, target, caches, B, tokens, lens.data(), nullptr, parents, nullptr, lg, nullptr,
                               nullptr);
  if (!rc) {
    hipError_t me = hipMallocAsync((void**)&dtok, (size_t)B * n * 4, e->stream);
    if (me == hipSuccess) me = hipMallocAsync((void**)&dpar, (size_t)B * n * 4, e->stream);
    if (me == hipSuccess) me = hipMallocAsync((void**)&dpath, (size_t)B * n * 4, e->stream);
    if (me == hipSuccess) me = hipMallocAsync((void**)&dlen, (size_t)B * 4, e->stream);
    if (me == hipSuccess) me = hipMallocAsync((void**)&dnext, (size_t)B * 4, e->stream);
    if (me == hipSuccess) me = hipMemcpyAsync(dtok, tokens, (size_t)B * n * 4, hipMemcpyHostToDevice, e->stream);
    if (me == hipSuccess) me = hipMemcpyAsync(dpar, parents, (size_t)B * n * 4, hipMemcpyHostToDevice, e->stream);
    if (me != hipSuccess) { sh_set_error("tree_verify_step: %s", hipGetErrorString(me)); rc = SH_ERR_HIP; }
  }
  if (!rc) rc = sh_tree_accept(e, lg, q_logits_dev, dtok, dpar, B, n, V, s, dpath, dlen, dnext);
  if (!rc) {
    hipError_t me = hipMemcpyAsync(path_out, dpath, (size_t)B * n * 4, hipMemcpyDeviceToHost, e->stream);
    if (me == hipSuccess) me = hipMemcpyAsync(path_len_out, dlen, (size_t)B * 4, hipMemcpyDeviceToHost, e->stream);
    if (me == hipSuccess) me = hipMemcpyAsync(next_tok_out, dnext, (size_t)B * 4, hipMemcpyDeviceToHost, e->stream);
    if (me == hipSuccess) me = hipStreamSynchronize(e->stream);
    if (me != hipSuccess) { sh_set_error("tree_verify_step readback: %s", hipGetErrorString(me)); rc = SH_ERR_HIP; }
  }
  (void)hipFreeAsync(lg, e->stream);
  if (dtok) (void)hipFreeAsync(dtok, e->stream);
  if (dpar) (void)hipFreeAsync(dpar, e->stream);
  if (dpath) (void)hipFreeAsync(dpath, e->stream);
  if (dlen) (void)hipFreeAsync(dlen, e->stream);
  if (dnext) (void)hipFreeAsync(dnext, e->stream);
  if (rc) return rc;
  // keep the accepted path's K/V rows: node path[i] -> slot base + i
  for (uint32_t b = 0; b < B && !rc; ++b)
    rc = sh_kv_compact(caches[b], base[b], path_out + (size_t)b * n, path_len_out[b]);
  return rc;
}

// ------------------------------------------------------------------ spec step


static void free_spec_bufs(SpecBufs& sb) {
  (void)hipFree(sb.tok); (void)hipFree(sb.samp); (void)hipFree(sb.base); (void)hipFree(sb.dlogits);
  (void)hipFree(sb.tlogits); (void)hipFree(sb.udev); (void)hipFree(sb.rowstat); (void)hipHostFree(sb.pinned);
  sb = SpecBufs();
}

static int spec_bufs(sh_engine* e, uint32_t V) {
  SpecBufs& sb = e->spec;
  if (sb.tok && sb.vcap >= V) return SH_OK;
  SH_HIP(hipSetDevice(e->device));
  if (sb.tok) {
    g_graph_gen.fetch_add(1);  // captured graphs point into these buffers
    SH_HIP(hipStreamSynchronize(e->stream));
    free_spec_bufs(sb);
  }
  SH_HIP(hipMalloc(&sb.tok, 64 * 4));
  SH_HIP(hipMalloc(&sb.samp, 16 * 4));
  SH_HIP(hipMalloc(&sb.base, 8 * 4));
  sb.rng = reinterpret_cast<uint64_t*>(sb.base + 4);
  SH_HIP(hipMalloc(&sb.dlogits, (size_t)8 * V * 4));
  SH_HIP(hipMalloc(&sb.tlogits, (size_t)9 * V * 4));
  SH_HIP(hipMalloc(&sb.udev, 32 * 4));
  SH_HIP(hipMalloc(&sb.rowstat, SpecBufs::kRowstatBytes));
  SH_HIP(hipHostMalloc((void**)&sb.pinned, 128 * 4, hipHostMallocDefault));
  sb.vcap = V;
  return SH_OK;
}

// ------------------------------------------------------------------ graph replay

// Greedy spec steps and greedy verifies replay a captured HIP graph. While one
// is captured, each cache's sh_kv::graph_base points at a device base position and every
// position-dependent kernel argument (RoPE position, KV slot, live keys, mask
// base) is an offset from it, so one capture serves every position; the host
// writes the base values before each replay. A capture is keyed by its shape,
// models and caches, and all captures are dropped when a model or cache is
// destroyed. SH_GRAPH=0 turns replay off; profiling runs eagerly.

static bool graphs_enabled(const sh_engine* e) {
  static const bool on = [] {
    const char* s = getenv("SH_GRAPH");
    return !(s && std::string(s) == "0");
  }();
  return on && !e->profiling;
}

static hipGraphExec_t graph_find(sh_engine* e, const std::vector<uintptr_t>& key) {
  const uint64_t gen = g_graph_gen.load();
  std::vector<GraphEntry>& g = e->graphs;
  for (size_t i = 0; i < g.size();) {
    if (g[i].gen != gen) {  // a model or cache it used may be gone
      (void)hipGraphExecDestroy(g[i].exec);
      g.erase(g.begin() + i);
      continue;
    }
    if (g[i].key == key) return g[i].exec;
    ++i;
  }
  return nullptr;
}

// Captures body() on the engine stream (cache kvs[i] gets graph_base =
// bases[i] meanwhile) and caches the instantiated graph under key.
static int graph_capture(sh_engine* e, const std::vector<uintptr_t>& key, const std::vector<sh_kv*>& kvs,
                         const std::vector<const uint32_t*>& bases, const std::function<int()>& body,
                         hipGraphExec_t* out) {
  SH_HIP(hipStreamSynchronize(e->stream));
  SH_HIP(hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal));
  for (size_t i = 0; i < kvs.size(); ++i) kvs[i]->graph_base = bases[i];
  int rc = body();
  for (sh_kv* kv : kvs) kv->graph_base = nullptr;
  hipGraph_t g = nullptr;
  const hipError_t ce = hipStreamEndCapture(e->stream, &g);
  if (rc) {
    if (g) (void)hipGraphDestroy(g);
    return rc;
  }
  SH_CHECK(ce == hipSuccess && g, SH_ERR_HIP, "graph capture: %s", hipGetErrorString(ce));
  hipGraphExec_t ex = nullptr;
  const hipError_t ie = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  SH_CHECK(ie == hipSuccess, SH_ERR_HIP, "graph instantiate: %s", hipGetErrorString(ie));
  GraphEntry ge;
  ge.gen = g_graph_gen.load();
  ge.key = key;
  ge.exec = ex;
  e->graphs.push_back(ge);
  ++e->graph_captures;
  *out = ex;
  return SH_OK;
}

static int graph_launch(sh_engine* e, hipGraphExec_t ex) {
  SH_HIP(hipGraphLaunch(ex, e->stream));
  ++e->graph_launches;
  return SH_OK;
}

extern "C" int sh_engine_graph_stats(sh_engine* e, uint64_t* captures, uint64_t* launches) {
  SH_CHECK(e && captures && launches, SH_ERR_ARG, "sh_engine_graph_stats: NULL argument");
  *captures = e->graph_captures;
  *launches = e->graph_launches;
  return SH_OK;
}

// Greedy drafts (Engine::draft_tokens, inference/mod.rs:2062-2092): the
// catch-up forward of the np pending tokens and last at dpos, then n - 1
// single-token forwards at dpos + np + i, each argmax feeding the next
// embedding on the device (tok[np + 1 + i] = d_{i+1}); the ids are copied to
// the pinned staging buffer when copy_out is set. forced: the drafts are
// already staged in tok (the forced-acceptance diagnostic); the argmax ids go
// to tok[48 + i] instead and the work is the same.
static int enqueue_drafts(sh_engine* e, sh_model* dm, sh_kv* dkv, uint32_t n, uint32_t np, uint32_t dpos,
                          bool copy_out, bool forced = false) {
  uint32_t* ids = forced ? e->spec.tok + 48 : e->spec.tok + np + 1;
  int rc = forward_dev(dm, dkv, e->spec.tok, np + 1, dpos, nullptr, 1, nullptr, nullptr, nullptr);
  if (rc) return rc;
  // the chunk's logits are [np + 1][V]: the last column's row
  if ((rc = sh_argmax_launch(e, dm->ws.logits + (size_t)np * dm->V, dm->V, 1, dm->ws.amax, ids))) return rc;
  for (uint32_t i = 1; i < n; ++i) {
    if ((rc = forward_dev(dm, dkv, e->spec.tok + np + i, 1, dpos + np + i, nullptr, 1, nullptr, nullptr, nullptr)))
      return rc;
    if ((rc = sh_argmax_launch(e, dm->ws.logits, dm->V, 1, dm->ws.amax, ids + i))) return rc;
  }
  if (copy_out)
    SH_HIP(hipMemcpyAsync(e->spec.pinned, e->spec.tok + np + 1, n * 4, hipMemcpyDeviceToHost, e->stream));
  return SH_OK;
}

// Draft n tokens greedily and verify [last, d_1..d_n] (greedy): drafts at dpos,
// the verify at tpos; drafts and per-column argmax ids are copied to the pinned
// staging buffer.
static int enqueue_greedy_step(sh_engine* e, sh_model* tm, sh_model* dm, sh_kv* tkv, sh_kv* dkv, uint32_t n,
                               uint32_t np, uint32_t dpos, uint32_t tpos, bool forced) {
  int rc = enqueue_drafts(e, dm, dkv, n, np, dpos, true, forced);
  if (rc) return rc;
  // ws.logits holds the last chunk's logits only: a verify of more than 8
  // columns (k = 8) may take two chunks, whose logits are collected in tlogits
  float* lg = n + 1 > 8 ? e->spec.tlogits : nullptr;
  if ((rc = forward_dev(tm, tkv, e->spec.tok + np, n + 1, tpos, nullptr, 2, lg, nullptr, nullptr))) return rc;
  if ((rc = sh_argmax_launch(e, lg ? lg : tm->ws.logits, tm->V, n + 1, tm->ws.amax, e->spec.samp))) return rc;
  SH_HIP(hipMemcpyAsync(e->spec.pinned + 16, e->spec.samp, 11 * 4, hipMemcpyDeviceToHost, e->stream));
  return SH_OK;
}

// Stochastic step (COMPARE / REJECTION): draft ids stay on the device
// (tok[np+1+i] = d_{i+1}). COMPARE drafts greedily, as the reference does
// (mod.rs:2062-2092); REJECTION draws d_i ~ q_i = softmax(draft logits / T)
// (vocab-order inverse CDF), which its min(1, p/q) test and residual draw need
// to be lossless. Draft forwards at dpos (catch-up) and dpos + np + i, the
// verify [last, d_1..d_n] at tpos with all-position logits, then the
// per-column decision on the device. Uniform words per step: 2i / 2i+1 accept
// / (re)sample verify column i, 2(n+1) + i draw draft i (REJECTION); explicit
// uniforms (udev) are [3n + 2], else Philox words from ctr, or from the device
// words rng (graph replay: key and word base written before each replay).
static int enqueue_stoch_step(sh_engine* e, sh_model* tm, sh_model* dm, sh_kv* tkv, sh_kv* dkv, uint32_t n,
                              uint32_t np, uint32_t dpos, uint32_t tpos, const sh_sampling* s, const float* udev,
                              uint64_t ctr, const uint64_t* rng) {
  const bool rej = s->mode == SH_SAMPLE_REJECTION;
  const uint32_t V = tm->V;
  int rc;
  for (uint32_t i = 0; i < n; ++i) {
    float* q = e->spec.dlogits + (size_t)i * V;
    rc = i == 0 ? forward_dev(dm, dkv, e->spec.tok, np + 1, dpos, nullptr, 1, q, nullptr, nullptr)
                : forward_dev(dm, dkv, e->spec.tok + np + i, 1, dpos + np + i, nullptr, 1, q, nullptr, nullptr);
    if (rc) return rc;
    uint32_t* dst = e->spec.tok + np + 1 + i;
    rc = rej ? sh_sample_rows_launch(e, q, 1, V, s->temperature, udev, s->seed, ctr + 2ull * (n + 1) + i, 1,
                                     e->spec.rowstat, SpecBufs::kRowstatBytes, dst, rng)
             : sh_argmax_launch(e, q, V, 1, dm->ws.amax, dst);
    if (rc) return rc;
  }
  rc = forward_dev(tm, tkv, e->spec.tok + np, n + 1, tpos, nullptr, 2, e->spec.tlogits, nullptr, nullptr);
  if (rc) return rc;
  rc = sh_accept_launch(e, e->spec.tlogits, rej ? e->spec.dlogits : nullptr, e->spec.tok + np + 1, 1, n, V, s, ctr,
                        udev, e->spec.samp + 9, e->spec.samp + 10, nullptr, nullptr, rng);
  if (rc) return rc;
  uint32_t* hp = e->spec.pinned;
  SH_HIP(hipMemcpyAsync(hp, e->spec.tok + np + 1, n * 4, hipMemcpyDeviceToHost, e->stream));
  SH_HIP(hipMemcpyAsync(hp + 16, e->spec.samp, 11 * 4, hipMemcpyDeviceToHost, e->stream));
  return SH_OK;
}

static uint32_t f32_bits(float x) {
  uint32_t u;
  std::memcpy(&u, &x, 4);
  return u;
}

static int spec_step(sh_engine* e, sh_model* tm, sh_model* dm, sh_kv* tkv, sh_kv* dkv, uint32_t last_token,
                     uint32_t n_max, sh_sampling* s, const uint32_t* forced, uint32_t* emitted_out,
                     uint32_t* n_emitted, uint32_t* drafts_out) {
  SH_CHECK(e && tm && dm && tkv && dkv && emitted_out && n_emitted, SH_ERR_ARG, "sh_spec_step: NULL argument");
  SH_CHECK(tm->V == dm->V, SH_ERR_ARG, "draft vocab %u != target vocab %u", dm->V, tm->V);
  SH_CHECK(last_token < tm->V, SH_ERR_ARG, "last_token %u out of range", last_token);
  const uint32_t mode = s ? s->mode : SH_SAMPLE_GREEDY;
  SH_CHECK(mode <= SH_SAMPLE_REJECTION, SH_ERR_ARG, "sampling mode %u", mode);
  SampRow filt{};
  if (mode != SH_SAMPLE_GREEDY)
    if (int frc = sh_samprow_filters(*s, tm->V, filt)) return frc;
  SH_CHECK(mode != SH_SAMPLE_REJECTION || !filt.top_k, SH_ERR_UNSUPPORTED,
           "candidate filters (top_k / top_p / min_p) apply to COMPARE only");
  SH_CHECK(mode == SH_SAMPLE_GREEDY || (s && s->temperature > 0.f), SH_ERR_ARG,
           "stochastic modes need temperature > 0");
  const uint32_t n = std::min<uint32_t>(std::max<uint32_t>(n_max, 1), 8);  // mod.rs:2121
  const uint32_t P = tkv->pos;
  const uint32_t np = (uint32_t)dkv->pending.size();
  SH_CHECK(dkv->pos + np == P, SH_ERR_STATE, "draft cache position %u + %u pending != target position %u", dkv->pos,
           np, P);
  SH_CHECK((uint64_t)P + n + 1 <= tkv->max_seq && (uint64_t)P + n + 1 <= dkv->max_seq, SH_ERR_CAPACITY,
           "spec lookahead exceeds KV capacity (run.rs:270-283)");
  int rc = spec_bufs(e, tm->V);
  if (rc) return rc;
  uint32_t* hp = e->spec.pinned;
  for (uint32_t i = 0; i < np; ++i) hp[i] = dkv->pending[i];
  hp[np] = last_token;
  if (forced) {
    SH_CHECK(mode == SH_SAMPLE_GREEDY, SH_ERR_ARG, "forced drafts are greedy steps");
    for (uint32_t i = 0; i < n; ++i) {
      SH_CHECK(forced[i] < tm->V, SH_ERR_ARG, "forced draft %u out of range", forced[i]);
      hp[np + 1 + i] = forced[i];
    }
  }
  SH_HIP(hipMemcpyAsync(e->spec.tok, hp, (np + 1 + (forced ? n : 0)) * 4, hipMemcpyHostToDevice, e->stream));
  // The whole step replays one captured graph (the reference records a step as
  // one submit, inference/mod.rs:2181-2231): every position-dependent argument
  // is an offset from the device words base[0] (draft) / base[1] (target), and
  // the stochastic modes read their Philox key and word base from rng
  // (decode_dyn.rs:25-204 patches the same per-step values).
  const bool graph = n + 1 <= 8 && np + 1 <= 8 && graphs_enabled(e) && graph_model_ok(tm) && graph_model_ok(dm);
  const uint32_t d0 = dkv->pos, V = tm->V;
  const float* udev = nullptr;
  uint64_t ctr = mode == SH_SAMPLE_GREEDY ? 0 : s->counter;
  if (mode != SH_SAMPLE_GREEDY && s->uniforms) {
    SH_HIP(hipMemcpyAsync(e->spec.udev, s->uniforms, (size_t)(3 * n + 2) * 4, hipMemcpyHostToDevice, e->stream));
    udev = e->spec.udev;
    ctr = 0;
  }
  e->spec.last_n = 0;
  if (graph) {
    const std::vector<uintptr_t> key = {mode == SH_SAMPLE_GREEDY ? 1u : 3u, (uintptr_t)tm, (uintptr_t)dm,
                                        (uintptr_t)tkv, (uintptr_t)dkv, (uintptr_t)tkv->k, (uintptr_t)dkv->k,
                                        tkv->max_seq, dkv->max_seq, n, np, tm->fa16, dm->fa16, mode,
                                        mode == SH_SAMPLE_GREEDY ? 0u : f32_bits(s->temperature),
                                        mode == SH_SAMPLE_GREEDY ? 0u : s->top_k,
                                        mode == SH_SAMPLE_GREEDY ? 0u : f32_bits(s->top_p),
                                        mode == SH_SAMPLE_GREEDY ? 0u : f32_bits(s->min_p), udev ? 1u : 0u,
                                        forced ? 1u : 0u};
    hipGraphExec_t ex = graph_find(e, key);
    if (!ex) {
      // everything a capture reads is sized beforehand (nothing allocates while capturing)
      if ((rc = ensure_rope(tm, tkv->max_seq)) || (rc = ensure_rope(dm, dkv->max_seq)) ||
          (rc = ensure_fa_part(tm, tkv->max_seq)) || (rc = ensure_fa_part(dm, dkv->max_seq)) ||
          (rc = ensure_fa16(tm, tkv->max_seq, n + 1)) || (rc = ensure_fa16(dm, dkv->max_seq, np + 1)))
        return rc;
      if (mode != SH_SAMPLE_GREEDY) {
        void* sb = nullptr;
        if ((rc = sh_engine_scratch(e, SCR_ACCEPT, sh_accept_scratch_bytes(1, n, V, mode), &sb))) return rc;
      }
      rc = graph_capture(e, key, {dkv, tkv}, {e->spec.base, e->spec.base + 1}, [&] {
        return mode == SH_SAMPLE_GREEDY
                   ? enqueue_greedy_step(e, tm, dm, tkv, dkv, n, np, 0, 0, forced != nullptr)
                   : enqueue_stoch_step(e, tm, dm, tkv, dkv, n, np, 0, 0, s, udev, 0, udev ? nullptr : e->spec.rng);
      }, &ex);
      if (rc) return rc;
    }
    hp[64] = d0;
    hp[65] = P;
    uint64_t* hr = reinterpret_cast<uint64_t*>(hp + 68);
    hr[0] = mode == SH_SAMPLE_GREEDY ? 0 : s->seed;
    hr[1] = ctr;
    SH_HIP(hipMemcpyAsync(e->spec.base, hp + 64, 8 * 4, hipMemcpyHostToDevice, e->stream));
    if ((rc = graph_launch(e, ex))) return rc;
    dkv->pos = d0 + np + n;  // what the eager forwards leave
    tkv->pos = P + n + 1;
  } else {
    rc = mode == SH_SAMPLE_GREEDY ? enqueue_greedy_step(e, tm, dm, tkv, dkv, n, np, d0, P, forced != nullptr)
                                  : enqueue_stoch_step(e, tm, dm, tkv, dkv, n, np, d0, P, s, udev, ctr, nullptr);
    if (rc) return rc;
  }
  if (mode != SH_SAMPLE_GREEDY) {
    if (!udev) s->counter += 3 * n + 2;
    e->spec.last_n = n;
    e->spec.last_V = V;
  }
  SH_HIP(hipStreamSynchronize(e->stream));
  uint32_t drafts[8];
  for (uint32_t i = 0; i < n; ++i) drafts[i] = hp[i];
  uint32_t ne = 0;
  if (mode == SH_SAMPLE_GREEDY) {
    // host accept (inference/mod.rs:2168-2179)
    for (uint32_t i = 0; i <= n; ++i) {
      const uint32_t t = hp[16 + i];
      emitted_out[ne++] = t;
      if (i < n && t == drafts[i]) continue;
      break;
    }
  } else {
    const uint32_t acc = hp[16 + 9], nxt = hp[16 + 10];
    for (uint32_t i = 0; i < acc; ++i) emitted_out[ne++] = drafts[i];
    emitted_out[ne++] = nxt;
  }
  const uint32_t acc = ne - 1;
  tkv->pos = P + acc + 1;                               // truncate (mod.rs:2269-2270)
  dkv->pos = std::min(dkv->pos, P + acc + 1);
  dkv->pending.clear();
  if (acc == n) dkv->pending.push_back(drafts[n - 1]);  // d_n was never fed to the draft
  *n_emitted = ne;
  if (drafts_out) std::memcpy(drafts_out, drafts, n * 4);
  return sh_prof_flush(e);
}

extern "C" int sh_spec_step(sh_engine* e, sh_model* tm, sh_model* dm, sh_kv* tkv, sh_kv* dkv, uint32_t last_token,
                            uint32_t n_max, sh_sampling* s, uint32_t* emitted_out, uint32_t* n_emitted,
                            uint32_t* drafts_out) {
  return spec_step(e, tm, dm, tkv, dkv, last_token, n_max, s, nullptr, emitted_out, n_emitted, drafts_out);
}

extern "C" int sh_spec_step_forced(sh_engine* e, sh_model* tm, sh_model* dm, sh_kv* tkv, sh_kv* dkv,
                                   uint32_t last_token, uint32_t n_max, const uint32_t* forced_drafts,
                                   uint32_t* emitted_out, uint32_t* n_emitted) {
  SH_CHECK(forced_drafts, SH_ERR_ARG, "sh_spec_step_forced: forced_drafts is NULL");
  return spec_step(e, tm, dm, tkv, dkv, last_token, n_max, nullptr, forced_drafts, emitted_out, n_emitted, nullptr);
}

// Engine::draft_tokens (inference/mod.rs:2062-2092) with a separate draft
// model: the cache's pending tokens and last_token, then n - 1 single-token
// forwards, each argmax feeding the next embedding on the device; the ids come
// back at the end. The cache advances by its pending count + n (d_n is not
// fed). Replays a captured graph (positions from base[0]) where the model
// allows.
extern "C" int sh_draft_tokens(sh_engine* e, sh_model* dm, sh_kv* dkv, uint32_t last_token, uint32_t n_max,
                               uint32_t* drafts_out) {
  SH_CHECK(e && dm && dkv && drafts_out, SH_ERR_ARG, "sh_draft_tokens: NULL argument");
  SH_CHECK(last_token < dm->V, SH_ERR_ARG, "last_token %u out of range", last_token);
  const uint32_t n = std::min<uint32_t>(std::max<uint32_t>(n_max, 1), 8);  // mod.rs:2072
  const uint32_t np = (uint32_t)dkv->pending.size();
  SH_CHECK((uint64_t)dkv->pos + np + n <= dkv->max_seq, SH_ERR_CAPACITY, "draft lookahead exceeds KV capacity");
  int rc = spec_bufs(e, dm->V);
  if (rc) return rc;
  uint32_t* hp = e->spec.pinned;
  for (uint32_t i = 0; i < np; ++i) hp[i] = dkv->pending[i];
  hp[np] = last_token;
  SH_HIP(hipMemcpyAsync(e->spec.tok, hp, (np + 1) * 4, hipMemcpyHostToDevice, e->stream));
  const uint32_t d0 = dkv->pos;
  if (np + 1 <= 8 && graphs_enabled(e) && graph_model_ok(dm)) {
    const std::vector<uintptr_t> key = {4, (uintptr_t)dm, (uintptr_t)dkv, (uintptr_t)dkv->k, dkv->max_seq, n, np,
                                        dm->fa16};
    hipGraphExec_t ex = graph_find(e, key);
    if (!ex) {
      if ((rc = ensure_rope(dm, dkv->max_seq)) || (rc = ensure_fa_part(dm, dkv->max_seq)) ||
          (rc = ensure_fa16(dm, dkv->max_seq, np + 1)))
        return rc;
      rc = graph_capture(e, key, {dkv}, {e->spec.base}, [&] { return enqueue_drafts(e, dm, dkv, n, np, 0, true); },
                         &ex);
      if (rc) return rc;
    }
    hp[64] = d0;
    SH_HIP(hipMemcpyAsync(e->spec.base, hp + 64, 4, hipMemcpyHostToDevice, e->stream));
    if ((rc = graph_launch(e, ex))) return rc;
    dkv->pos = d0 + np + n;
  } else if ((rc = enqueue_drafts(e, dm, dkv, n, np, d0, true))) {
    return rc;
  }
  SH_HIP(hipStreamSynchronize(e->stream));
  std::memcpy(drafts_out, hp, n * 4);
  dkv->pending.clear();
  return sh_prof_flush(e);
}

// The batched speculative step of the reference's server (server/inference.rs:
// 2777-2924): drafts for every sequence, one verify_unified over all of them,
// per-sequence acceptance and rollback. The drafts of all sequences at one
// draft position go through the draft model as one batched forward (one
// column per sequence; a sequence's first position also carries its pending
// tokens), where the reference calls draft_tokens per sequence
// (server/inference.rs:2806-2812).
extern "C" int sh_spec_step_batch(sh_engine* e, sh_model* tm, sh_model* dm, sh_kv* const* tkv, sh_kv* const* dkv,
                                  uint32_t B, const uint32_t* last_tokens, uint32_t n_max, sh_sampling* samplers,
                                  uint32_t* emitted_out, uint32_t* n_emitted, uint32_t* drafts_out) {
  SH_CHECK(e && tm && dm && tkv && dkv && last_tokens && emitted_out && n_emitted, SH_ERR_ARG,
           "sh_spec_step_batch: NULL argument");
  SH_CHECK(B >= 1, SH_ERR_ARG, "spec_step_batch: empty batch");
  SH_CHECK(tm->V == dm->V, SH_ERR_ARG, "draft vocab %u != target vocab %u", dm->V, tm->V);
  const uint32_t n = std::min<uint32_t>(std::max<uint32_t>(n_max, 1), 8);
  std::vector<uint32_t> P(B), np(B);
  for (uint32_t s = 0; s < B; ++s) {
    SH_CHECK(tkv[s] && dkv[s], SH_ERR_ARG, "spec_step_batch: cache %u is NULL", s);
    SH_CHECK(last_tokens[s] < tm->V, SH_ERR_ARG, "spec_step_batch: last token %u of sequence %u", last_tokens[s], s);
    P[s] = tkv[s]->pos;
    np[s] = (uint32_t)dkv[s]->pending.size();
    SH_CHECK(dkv[s]->pos + np[s] == P[s], SH_ERR_STATE, "sequence %u: draft cache %u + %u pending != target %u", s,
             dkv[s]->pos, np[s], P[s]);
    SH_CHECK((uint64_t)P[s] + n + 1 <= tkv[s]->max_seq && (uint64_t)P[s] + n + 1 <= dkv[s]->max_seq,
             SH_ERR_CAPACITY, "sequence %u: spec lookahead exceeds KV capacity (run.rs:270-283)", s);
    if (samplers)
      SH_CHECK(samplers[s].mode == SH_SAMPLE_GREEDY || samplers[s].mode == SH_SAMPLE_COMPARE, SH_ERR_ARG,
               "spec_step_batch: sequence %u sampler mode %u (GREEDY or COMPARE)", s, samplers[s].mode);
  }
  // drafts: position 1 takes each sequence's pending tokens and last token,
  // positions 2..n its previous draft
  std::vector<uint32_t> drafts((size_t)B * n), toks, lens(B), ids;
  for (uint32_t i = 0; i < n; ++i) {
    toks.clear();
    for (uint32_t s = 0; s < B; ++s) {
      if (i == 0) {
        for (uint32_t t : dkv[s]->pending) toks.push_back(t);
        toks.push_back(last_tokens[s]);
        lens[s] = np[s] + 1;
      } else {
        toks.push_back(drafts[(size_t)s * n + i - 1]);
        lens[s] = 1;
      }
    }
    ids.assign(toks.size(), 0u);
    int rc = verify_unified_impl(e, dm, dkv, B, toks.data(), lens.data(), nullptr, nullptr, nullptr, nullptr,
                                 ids.data(), nullptr);
    if (rc) return rc;
    uint32_t q = 0;
    for (uint32_t s = 0; s < B; ++s) {
      q += lens[s];
      drafts[(size_t)s * n + i] = ids[q - 1];
    }
  }
  // verify [last, d_1..d_n] of every sequence in one batch
  toks.clear();
  for (uint32_t s = 0; s < B; ++s) {
    toks.push_back(last_tokens[s]);
    for (uint32_t i = 0; i < n; ++i) toks.push_back(drafts[(size_t)s * n + i]);
    lens[s] = n + 1;
  }
  ids.assign(toks.size(), 0u);
  int rc = verify_unified_impl(e, tm, tkv, B, toks.data(), lens.data(), nullptr, nullptr, nullptr, nullptr,
                               ids.data(), nullptr, samplers);
  if (rc) return rc;
  // per-sequence acceptance (server/inference.rs:2859-2883) and rollback
  for (uint32_t s = 0; s < B; ++s) {
    const uint32_t* col = ids.data() + (size_t)s * (n + 1);
    const uint32_t* d = drafts.data() + (size_t)s * n;
    uint32_t acc = 0;
    while (acc < n && col[acc] == d[acc]) ++acc;
    for (uint32_t i = 0; i <= acc; ++i) emitted_out[(size_t)s * (n + 1) + i] = col[i];
    n_emitted[s] = acc + 1;
    tkv[s]->pos = P[s] + acc + 1;
    dkv[s]->pos = std::min(dkv[s]->pos, P[s] + acc + 1);
    dkv[s]->pending.clear();
    if (acc == n) dkv[s]->pending.push_back(d[n - 1]);  // d_n was never fed to the draft
    if (drafts_out) std::memcpy(drafts_out + (size_t)s * n, d, n * 4);
  }
  return SH_OK;
}

extern "C" int sh_spec_step_logits(sh_engine* e, float* p_out, float* q_out, uint32_t* n_out, uint32_t* V_out) {
  SH_CHECK(e && n_out, SH_ERR_ARG, "sh_spec_step_logits: NULL argument");
  const uint32_t n = e->spec.last_n, V = e->spec.last_V;
  SH_CHECK(n > 0, SH_ERR_STATE, "no stochastic speculative step has run on this engine");
  SH_HIP(hipStreamSynchronize(e->stream));
  if (p_out) SH_HIP(hipMemcpy(p_out, e->spec.tlogits, (size_t)(n + 1) * V * 4, hipMemcpyDeviceToHost));
  if (q_out) SH_HIP(hipMemcpy(q_out, e->spec.dlogits, (size_t)n * V * 4, hipMemcpyDeviceToHost));
  *n_out = n;
  if (V_out) *V_out = V;
  return SH_OK;
}

// ------------------------------------------------------------------ kernel level

extern "C" int sh_qtensor_upload(sh_engine* e, int type, const void* host, uint32_t M, uint32_t K, sh_qtensor** out) {
  SH_CHECK(e && host && out, SH_ERR_ARG, "sh_qtensor_upload: NULL argument");
  SH_CHECK(M >= 1 && K >= 1, SH_ERR_ARG, "empty matrix");
  sh_qtensor* t = new sh_qtensor();
  t->e = e;
  int rc = sh_repack_upload(e, type, (const uint8_t*)host, M, K, &t->m);
  if (rc) { delete t; return rc; }
  *out = t;
  return SH_OK;
}

extern "C" void sh_qtensor_destroy(sh_qtensor* t) {
  if (!t) return;
  (void)hipStreamSynchronize(t->e->stream);
  sh_qmat_free(&t->m);
  delete t;
}

extern "C" int sh_gemv_quant(sh_engine* e, const sh_qtensor* w, const float* x_dev, uint32_t N, float* y_dev,
                             int accumulate) {
  SH_CHECK(e && w && x_dev && y_dev, SH_ERR_ARG, "sh_gemv_quant: NULL argument");
  SH_CHECK(N >= 1, SH_ERR_ARG, "N must be >= 1");
  const uint32_t K = w->m.K, M = w->m.M;
  uint16_t *bx = nullptr, *xs = nullptr;
  float *cs = nullptr, *part = nullptr;
  // Q4_K with more than 8 columns, and Q5_K / Q6_K at any width: the forward's
  // multi-group kernel, 64 columns per pass
  const bool mg = sh_is_kquant(w->m.type) && K % 256 == 0 && (N > 8 || w->m.type != GGML_Q4_K);
  const uint32_t CW = mg ? SH_MAX_COLS : 8, ngrp = CW / 8;
  const size_t bx_elems = ngrp * sh_grp_bx(K), xs_elems = ngrp * sh_grp_xs(K);
  const size_t part_floats = mg ? sh_gemm_part_floats(w->m) : sh_gemv_part_floats(w->m);
  SH_HIP(hipMallocAsync((void**)&bx, bx_elems * 2, e->stream));
  SH_HIP(hipMallocAsync((void**)&xs, xs_elems * 2, e->stream));
  SH_HIP(hipMallocAsync((void**)&cs, ngrp * sh_grp_cs(K) * sizeof(float), e->stream));
  SH_HIP(hipMallocAsync((void**)&part, std::max<size_t>(part_floats, 4) * sizeof(float), e->stream));
  SH_HIP(hipMemsetAsync(xs, 0, xs_elems * 2, e->stream));
  int rc = SH_OK;
  // The same kernels as the forward: split partials (finished here by a reduce)
  // where the forward would use them, else a direct store / accumulate.
  const bool split = w->m.type == GGML_Q4_K && part_floats > (size_t)8 * w->m.tiles * 16;
  for (uint32_t c0 = 0; c0 < N && !rc; c0 += CW) {
    const uint32_t nc = std::min<uint32_t>(CW, N - c0);
    PrepArgs pr;
    pr.mode = PREP_PLAIN; pr.x = const_cast<float*>(x_dev + (size_t)c0 * K); pr.K = K; pr.N = nc;
    pr.bx = bx; pr.xs = xs; pr.cs = cs;
    rc = sh_prep_launch(e, pr);
    if (rc) break;
    if (mg) {
      const uint32_t ncp = (nc + 7) / 8 * 8;
      EpiArgs pa;
      pa.out = part; pa.ldo = w->m.tiles * 16; pa.cs = cs;
      pa.part_stride = (size_t)ncp * pa.ldo;
      pa.part_cap = (uint32_t)(part_floats / pa.part_stride);
      uint32_t np = 0;
      rc = sh_gemm_launch(e, w->m, bx, xs, cs, nc, EPI_PART, pa, "gemm", &np);
      if (!rc)
        rc = sh_part_reduce_launch(e, part, np, pa.ldo, ncp, M, nc, y_dev + (size_t)c0 * M, M, accumulate != 0);
    } else if (split) {
      EpiArgs pa;
      pa.out = part; pa.ldo = w->m.tiles * 16; pa.cs = cs;
      pa.part_stride = (size_t)8 * pa.ldo;
      pa.part_cap = (uint32_t)(part_floats / pa.part_stride);
      uint32_t np = 0;
      rc = sh_gemv_launch(e, w->m, bx, xs, nc, EPI_PART, pa, "gemv", &np);
      if (!rc)
        rc = sh_part_reduce_launch(e, part, np, pa.ldo, 8, M, nc, y_dev + (size_t)c0 * M, M, accumulate != 0);
    } else {
      EpiArgs ea;
      ea.out = y_dev + (size_t)c0 * M;
      ea.ldo = M;
      ea.rows = M;
      ea.cs = cs;
      rc = sh_gemv_launch(e, w->m, bx, xs, nc, accumulate ? EPI_ADD : EPI_STORE, ea, "gemv");
    }
  }
  (void)hipFreeAsync(bx, e->stream);
  (void)hipFreeAsync(xs, e->stream);
  (void)hipFreeAsync(cs, e->stream);
  (void)hipFreeAsync(part, e->stream);
  if (rc) return rc;
  SH_HIP(hipStreamSynchronize(e->stream));
  return sh_prof_flush(e);
}

extern "C" int sh_gemm_wide16(sh_engine* e, const sh_qtensor* w, const float* x_dev, uint32_t N, float* y_dev,
                              int accumulate) {
  SH_CHECK(e && w && x_dev && y_dev, SH_ERR_ARG, "sh_gemm_wide16: NULL argument");
  SH_CHECK(N >= 1, SH_ERR_ARG, "N must be >= 1");
  SH_CHECK((w->m.type == GGML_Q4_K && w->m.K % 256 == 0) || sh_gemm16x_ok(w->m), SH_ERR_UNSUPPORTED,
           "sh_gemm_wide16: Q4_K, Q5_K, Q6_K (K a multiple of 256) or Q8_0 (of 32); type %d, K %u", w->m.type,
           w->m.K);
  const uint32_t K = w->m.K, M = w->m.M, CW = SH_MAX_COLS16;
  const size_t part_floats = sh_gemm16_part_floats(w->m);
  uint16_t* bh = nullptr;
  float* part = nullptr;
  SH_HIP(hipMallocAsync((void**)&bh, (size_t)CW * K * 2, e->stream));
  SH_HIP(hipMallocAsync((void**)&part, std::max<size_t>(part_floats, 4) * sizeof(float), e->stream));
  int rc = SH_OK;
  for (uint32_t c0 = 0; c0 < N && !rc; c0 += CW) {
    const uint32_t nc = std::min<uint32_t>(CW, N - c0), ncp = (nc + 7) / 8 * 8;
    PrepArgs pr;
    pr.mode = PREP_PLAIN; pr.x = const_cast<float*>(x_dev + (size_t)c0 * K); pr.K = K; pr.N = nc;
    pr.bh = bh; pr.ldb = K;
    if ((rc = sh_prep_launch(e, pr))) break;
    EpiArgs pa;
    pa.out = part; pa.ldo = w->m.tiles * 16;
    pa.part_stride = (size_t)ncp * pa.ldo;
    pa.part_cap = (uint32_t)(part_floats / pa.part_stride);
    uint32_t np = 0;
    rc = sh_gemm16_launch(e, w->m, bh, K, nc, EPI_PART, pa, "gemm16", &np);
    if (!rc) rc = sh_part_reduce_launch(e, part, np, pa.ldo, ncp, M, nc, y_dev + (size_t)c0 * M, M, accumulate != 0);
  }
  (void)hipFreeAsync(bh, e->stream);
  (void)hipFreeAsync(part, e->stream);
  if (rc) return rc;
  SH_HIP(hipStreamSynchronize(e->stream));
  return sh_prof_flush(e);
}
