// GGUF reader and model description (host-only; see gguf.h).
#include "gguf.h"

#include <algorithm>
#include <cmath>
#include <cstring>

bool sh_ggml_block(uint32_t type, uint32_t* elems, uint32_t* bytes) {
  switch (type) {
    case GGML_F32: *elems = 1; *bytes = 4; return true;
    case GGML_F16: *elems = 1; *bytes = 2; return true;
    case GGML_Q8_0: *elems = 32; *bytes = 34; return true;
    case GGML_Q4_K: *elems = 256; *bytes = 144; return true;
    case GGML_Q5_K: *elems = 256; *bytes = 176; return true;
    case GGML_Q6_K: *elems = 256; *bytes = 210; return true;
    default: return false;
  }
}

const GTensor* GFile::find(const std::string& n) const {
  for (auto& t : tensors)
    if (t.name == n) return &t;
  return nullptr;
}

namespace {

struct Rd {
  const uint8_t* p;
  const uint8_t* end;
  bool bad = false;
  uint64_t u(int n) {
    if (bad || (uint64_t)(end - p) < (uint64_t)n) { bad = true; return 0; }
    uint64_t v = 0;
    for (int i = 0; i < n; ++i) v |= (uint64_t)p[i] << (8 * i);
    p += n;
    return v;
  }
  std::string s() {
    const uint64_t n = u(8);
    if (bad || n > (uint64_t)(end - p)) { bad = true; return ""; }
    std::string r((const char*)p, n);
    p += n;
    return r;
  }
};

bool skip_value(Rd& r, uint32_t t, int depth = 0) {
  static const int sz[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
  if (depth > 4 || t > 12) return false;
  if (t == 8) { r.s(); return !r.bad; }
  if (t == 9) {
    const uint32_t et = (uint32_t)r.u(4);
    const uint64_t n = r.u(8);
    if (et > 12) return false;
    // fixed-size elements: one bounds check for the whole array
    if (et != 8 && et != 9) {
      const uint64_t left = (uint64_t)(r.end - r.p);
      if (r.bad || n > left / (uint64_t)sz[et]) return false;
      r.p += n * (uint64_t)sz[et];
      return true;
    }
    for (uint64_t i = 0; i < n && !r.bad; ++i)
      if (!skip_value(r, et, depth + 1)) return false;
    return !r.bad;
  }
  r.u(sz[t]);
  return !r.bad;
}

// a * b (+ c) without wrapping; false on overflow
bool mul_ok(uint64_t a, uint64_t b, uint64_t* out) { return !__builtin_mul_overflow(a, b, out); }

}  // namespace

int sh_gguf_parse(const uint8_t* img, uint64_t size, GFile* f) {
  SH_CHECK(img && f, SH_ERR_ARG, "gguf: NULL argument");
  SH_CHECK(size >= 24 && std::memcmp(img, "GGUF", 4) == 0, SH_ERR_FORMAT, "not a GGUF file (bad magic)");
  Rd r{img + 4, img + size};
  const uint32_t ver = (uint32_t)r.u(4);
  SH_CHECK(ver == 2 || ver == 3, SH_ERR_FORMAT, "unsupported GGUF version %u", ver);
  const uint64_t nt = r.u(8), nkv = r.u(8);
  SH_CHECK(nt < (1u << 24) && nkv < (1u << 24), SH_ERR_FORMAT, "implausible GGUF counts");
  uint32_t align = 32;
  for (uint64_t i = 0; i < nkv && !r.bad; ++i) {
    const std::string k = r.s();
    const uint32_t t = (uint32_t)r.u(4);
    if (r.bad) break;
    switch (t) {
      case 0: f->num[k] = (double)(uint8_t)r.u(1); break;
      case 1: f->num[k] = (double)(int8_t)r.u(1); break;
      case 2: f->num[k] = (double)(uint16_t)r.u(2); break;
      case 3: f->num[k] = (double)(int16_t)r.u(2); break;
      case 4: f->num[k] = (double)(uint32_t)r.u(4); break;
      case 5: f->num[k] = (double)(int32_t)r.u(4); break;
      case 6: { const uint32_t b = (uint32_t)r.u(4); float x; std::memcpy(&x, &b, 4); f->num[k] = x; break; }
      case 7: f->num[k] = (double)r.u(1); break;
      case 8: f->str[k] = r.s(); break;
      case 10: f->num[k] = (double)r.u(8); break;
      case 11: f->num[k] = (double)(int64_t)r.u(8); break;
      case 12: { const uint64_t b = r.u(8); double x; std::memcpy(&x, &b, 8); f->num[k] = x; break; }
      default:
        SH_CHECK(skip_value(r, t), SH_ERR_FORMAT, "bad GGUF metadata value type %u for %s", t, k.c_str());
    }
    if (k == "general.alignment" && t == 4 && !r.bad) align = (uint32_t)f->num[k];
  }
  SH_CHECK(!r.bad, SH_ERR_FORMAT, "truncated GGUF metadata");
  SH_CHECK(align && align <= (1u << 20) && (align & (align - 1)) == 0, SH_ERR_FORMAT, "bad alignment %u", align);
  for (uint64_t i = 0; i < nt && !r.bad; ++i) {
    GTensor t;
    t.name = r.s();
    t.nd = (uint32_t)r.u(4);
    if (r.bad) break;
    SH_CHECK(t.nd >= 1 && t.nd <= 4, SH_ERR_FORMAT, "tensor %s has %u dims", t.name.c_str(), t.nd);
    for (uint32_t j = 0; j < t.nd; ++j) t.ne[j] = r.u(8);
    t.type = (uint32_t)r.u(4);
    t.off = r.u(8);
    f->tensors.push_back(t);
  }
  SH_CHECK(!r.bad, SH_ERR_FORMAT, "truncated GGUF tensor table");
  const uint64_t pos = (uint64_t)(r.p - img);
  const uint64_t start = (pos + align - 1) / align * align;  // pos < size <= 2^64 - 2^20: no wrap
  SH_CHECK(start <= size, SH_ERR_FORMAT, "GGUF data section past end of file");
  f->base = img;
  f->size = size;
  f->data = img + start;
  const uint64_t avail = size - start;
  for (auto& t : f->tensors) {
    uint64_t n = 1;
    for (int j = 0; j < 4; ++j)
      SH_CHECK(mul_ok(n, t.ne[j], &n), SH_ERR_FORMAT, "tensor %s: element count overflows", t.name.c_str());
    uint32_t be = 0, bb = 0;
    if (!sh_ggml_block(t.type, &be, &bb)) { t.bytes = 0; continue; }  // rejected if the model uses it
    SH_CHECK(t.ne[0] % be == 0, SH_ERR_FORMAT, "tensor %s: row of %llu elements is not whole blocks of %u",
             t.name.c_str(), (unsigned long long)t.ne[0], be);
    SH_CHECK(mul_ok(n / be, bb, &t.bytes), SH_ERR_FORMAT, "tensor %s: byte size overflows", t.name.c_str());
    SH_CHECK(t.off <= avail && t.bytes <= avail - t.off, SH_ERR_FORMAT, "tensor %s extends past end of file",
             t.name.c_str());
  }
  return SH_OK;
}

namespace {

double num_or(const GFile& f, const std::string& k, double dflt, bool* found = nullptr) {
  auto it = f.num.find(k);
  if (found) *found = it != f.num.end();
  return it == f.num.end() ? dflt : it->second;
}

// A whole-number metadata value in [lo, hi], or the default when absent.
int u32_key(const GFile& f, const std::string& k, uint32_t* out, bool required, uint32_t dflt, uint32_t lo,
            uint32_t hi) {
  bool found = false;
  const double v = num_or(f, k, (double)dflt, &found);
  SH_CHECK(found || !required, SH_ERR_FORMAT, "missing required metadata %s", k.c_str());
  SH_CHECK(std::isfinite(v) && v == std::floor(v) && v >= (double)lo && v <= (double)hi, SH_ERR_FORMAT,
           "metadata %s = %g outside [%u, %u]", k.c_str(), v, lo, hi);
  *out = (uint32_t)v;
  return SH_OK;
}

bool matrix_type(uint32_t t) {
  return t == GGML_Q4_K || t == GGML_Q8_0 || t == GGML_Q5_K || t == GGML_Q6_K;
}
static bool sh_kquant_type(uint32_t t) { return t == GGML_Q4_K || t == GGML_Q5_K || t == GGML_Q6_K; }

// Looks up a tensor and checks it is a rows x cols matrix (n_mat slabs) of a
// known type; vectors (rows = 0) must be f32 [cols].
int get_tensor(const GFile& f, const std::string& name, uint64_t cols, uint64_t rows, uint64_t n_mat, bool required,
               TRef* out) {
  const GTensor* t = f.find(name);
  if (!t) {
    SH_CHECK(!required, SH_ERR_FORMAT, "missing tensor %s", name.c_str());
    *out = TRef();
    return SH_OK;
  }
  uint32_t be = 0, bb = 0;
  SH_CHECK(sh_ggml_block(t->type, &be, &bb), SH_ERR_UNSUPPORTED, "tensor %s: GGML type %u not supported",
           name.c_str(), t->type);
  if (rows == 0) {  // f32 vector
    SH_CHECK(t->type == GGML_F32 && t->ne[0] == cols && t->ne[1] == 1 && t->ne[2] == 1 && t->ne[3] == 1,
             SH_ERR_FORMAT, "tensor %s: f32 [%llu] expected", name.c_str(), (unsigned long long)cols);
  } else {
    SH_CHECK(t->ne[0] == cols && t->ne[1] == rows && t->ne[2] == n_mat && t->ne[3] == 1, SH_ERR_FORMAT,
             "tensor %s: shape [%llu, %llu, %llu, %llu], expected [%llu, %llu, %llu, 1]", name.c_str(),
             (unsigned long long)t->ne[0], (unsigned long long)t->ne[1], (unsigned long long)t->ne[2],
             (unsigned long long)t->ne[3], (unsigned long long)cols, (unsigned long long)rows,
             (unsigned long long)n_mat);
  }
  out->data = f.data + t->off;
  out->type = t->type;
  out->cols = cols;
  out->rows = rows ? rows : 1;
  out->n_mat = n_mat;
  out->row_bytes = cols / be * bb;
  return SH_OK;
}

}  // namespace

int sh_gguf_describe(const GFile& f, ModelDesc* m) {
  auto arch_it = f.str.find("general.architecture");
  SH_CHECK(arch_it != f.str.end(), SH_ERR_FORMAT, "missing general.architecture");
  const std::string& A = arch_it->second;
  if (A == "llama") m->arch = ARCH_LLAMA;
  else if (A == "qwen3") m->arch = ARCH_QWEN3;
  else if (A == "qwen3moe") m->arch = ARCH_QWEN3MOE;
  else SH_CHECK(false, SH_ERR_UNSUPPORTED, "architecture '%s' not supported (llama, qwen3, qwen3moe)", A.c_str());
  const bool qwen = m->arch != ARCH_LLAMA;
  const std::string p = A + ".";
  int rc;
  constexpr uint32_t kBig = 1u << 24;
  // keys / defaults: models/llama.rs:1038-1048, models/qwen3.rs:609-638
  if ((rc = u32_key(f, p + "block_count", &m->n_layer, true, 0, 1, 4096)) ||
      (rc = u32_key(f, p + "attention.head_count", &m->n_head, true, 0, 1, 1024)) ||
      (rc = u32_key(f, p + "attention.head_count_kv", &m->n_kv, false, m->n_head, 1, 1024)) ||
      (rc = u32_key(f, p + "embedding_length", &m->d, true, 0, 1, 65536)) ||
      (rc = u32_key(f, p + "context_length", &m->n_ctx, false, qwen ? 32768 : 0, 0, 0x7FFFFFFFu)))
    return rc;
  if (m->arch == ARCH_QWEN3MOE) {
    if ((rc = u32_key(f, p + "expert_count", &m->n_expert, true, 0, 1, 1024)) ||
        (rc = u32_key(f, p + "expert_used_count", &m->n_expert_used, true, 0, 1, 64)) ||
        (rc = u32_key(f, p + "expert_feed_forward_length", &m->expert_ff, true, 0, 1, kBig)))
      return rc;
    SH_CHECK(m->n_expert_used <= m->n_expert, SH_ERR_FORMAT, "expert_used_count %u > expert_count %u",
             m->n_expert_used, m->n_expert);
    m->ff = 0;
  } else if ((rc = u32_key(f, p + "feed_forward_length", &m->ff, true, 0, 1, kBig))) {
    return rc;
  }
  SH_CHECK(m->n_head % m->n_kv == 0, SH_ERR_FORMAT, "head_count %u is not a multiple of head_count_kv %u", m->n_head,
           m->n_kv);
  if (qwen) {
    if ((rc = u32_key(f, p + "attention.key_length", &m->hd, false, m->d / m->n_head, 1, 1024))) return rc;
  } else {
    SH_CHECK(m->d % m->n_head == 0, SH_ERR_FORMAT, "embedding_length %u not a multiple of head_count %u", m->d,
             m->n_head);
    m->hd = m->d / m->n_head;
  }
  uint32_t rope_dim = 0;
  if ((rc = u32_key(f, p + "rope.dimension_count", &rope_dim, false, m->hd, 1, 1024))) return rc;
  const double theta = num_or(f, p + "rope.freq_base", qwen ? 1e6 : 1e4);
  const double eps = num_or(f, p + "attention.layer_norm_rms_epsilon", qwen ? 1e-6 : 1e-5);
  SH_CHECK(std::isfinite(theta) && theta > 1.0, SH_ERR_FORMAT, "rope.freq_base %g", theta);
  SH_CHECK(std::isfinite(eps) && eps >= 0.0 && eps < 1.0, SH_ERR_FORMAT, "layer_norm_rms_epsilon %g", eps);
  m->theta = (float)theta;
  m->eps = (float)eps;
  m->neox = qwen;
  m->qk_norm = qwen;
  SH_CHECK(rope_dim == m->hd, SH_ERR_UNSUPPORTED, "partial RoPE (rope_dim %u != head_dim %u)", rope_dim, m->hd);
  SH_CHECK(m->hd == 64 || m->hd == 128, SH_ERR_UNSUPPORTED, "head_dim %u (64 or 128 supported)", m->hd);
  const GTensor* te = f.find("token_embd.weight");
  SH_CHECK(te, SH_ERR_FORMAT, "missing tensor token_embd.weight");
  if ((rc = u32_key(f, p + "vocab_size", &m->V, false, (uint32_t)std::min<uint64_t>(te->ne[1], 0xFFFFFFFFull), 1,
                    kBig)))
    return rc;
  if ((rc = get_tensor(f, "token_embd.weight", m->d, m->V, 1, true, &m->tok_embd))) return rc;
  if ((rc = get_tensor(f, "output_norm.weight", m->d, 0, 1, true, &m->out_norm))) return rc;
  // lm_head = output.unwrap_or(token_embd) (llama.rs:424, qwen3.rs:673)
  if ((rc = get_tensor(f, "output.weight", m->d, m->V, 1, false, &m->output))) return rc;
  if (!m->output.present()) m->output = m->tok_embd;
  SH_CHECK(matrix_type(m->output.type), SH_ERR_UNSUPPORTED, "lm_head type %u (K-quants and Q8_0 supported)",
           m->output.type);
  const uint32_t qd = m->q_dim(), kvd = m->kv_dim();
  m->layers.assign(m->n_layer, LayerDesc());
  for (uint32_t l = 0; l < m->n_layer; ++l) {
    LayerDesc& L = m->layers[l];
    const std::string b = "blk." + std::to_string(l) + ".";
    if ((rc = get_tensor(f, b + "attn_norm.weight", m->d, 0, 1, true, &L.attn_norm)) ||
        (rc = get_tensor(f, b + "ffn_norm.weight", m->d, 0, 1, true, &L.ffn_norm)) ||
        (rc = get_tensor(f, b + "attn_q.weight", m->d, qd, 1, true, &L.wq)) ||
        (rc = get_tensor(f, b + "attn_k.weight", m->d, kvd, 1, true, &L.wk)) ||
        (rc = get_tensor(f, b + "attn_v.weight", m->d, kvd, 1, true, &L.wv)) ||
        (rc = get_tensor(f, b + "attn_output.weight", qd, m->d, 1, true, &L.wo)))
      return rc;
    if (m->qk_norm &&
        ((rc = get_tensor(f, b + "attn_q_norm.weight", m->hd, 0, 1, true, &L.q_norm)) ||
         (rc = get_tensor(f, b + "attn_k_norm.weight", m->hd, 0, 1, true, &L.k_norm))))
      return rc;
    if (m->arch == ARCH_QWEN3MOE) {
      const uint32_t E = m->n_expert, ef = m->expert_ff;
      if ((rc = get_tensor(f, b + "ffn_gate_inp.weight", m->d, E, 1, true, &L.gate_inp)) ||
          (rc = get_tensor(f, b + "ffn_gate_exps.weight", m->d, ef, E, true, &L.gate_exps)) ||
          (rc = get_tensor(f, b + "ffn_up_exps.weight", m->d, ef, E, true, &L.up_exps)) ||
          (rc = get_tensor(f, b + "ffn_down_exps.weight", ef, m->d, E, true, &L.down_exps)))
        return rc;
      SH_CHECK(L.gate_inp.type == GGML_F32 || matrix_type(L.gate_inp.type), SH_ERR_UNSUPPORTED,
               "layer %u: router type %u", l, L.gate_inp.type);
      for (const TRef* t : {&L.gate_exps, &L.up_exps, &L.down_exps})
        SH_CHECK(sh_kquant_type(t->type), SH_ERR_UNSUPPORTED,
                 "layer %u: expert weights of type %u (Q4_K / Q5_K / Q6_K supported)", l, t->type);
      SH_CHECK(L.gate_exps.type == L.up_exps.type, SH_ERR_UNSUPPORTED, "layer %u: ffn_gate_exps / ffn_up_exps types differ",
               l);
    } else {
      if ((rc = get_tensor(f, b + "ffn_gate.weight", m->d, m->ff, 1, true, &L.gate)) ||
          (rc = get_tensor(f, b + "ffn_up.weight", m->d, m->ff, 1, true, &L.up)) ||
          (rc = get_tensor(f, b + "ffn_down.weight", m->ff, m->d, 1, true, &L.down)))
        return rc;
      SH_CHECK(L.gate.type == L.up.type, SH_ERR_UNSUPPORTED, "layer %u: ffn_gate type %u != ffn_up type %u", l,
               L.gate.type, L.up.type);
    }
    for (const TRef* t : {&L.wq, &L.wk, &L.wv, &L.wo, &L.gate, &L.up, &L.down})
      if (t->present())
        SH_CHECK(matrix_type(t->type), SH_ERR_UNSUPPORTED, "layer %u: matrix type %u (K-quants and Q8_0 supported)",
                 l, t->type);
    // attn_v may differ (Q4_K_M-style files keep it in Q6_K on some layers)
    SH_CHECK(L.wq.type == L.wk.type, SH_ERR_UNSUPPORTED, "layer %u: attn_q/k types %u/%u differ", l, L.wq.type,
             L.wk.type);
  }
  return SH_OK;
}

// What the device path runs: the fused 8-column path takes llama models whose
// layer matrices are uniformly Q4_K or uniformly Q8_0 (lm_head Q4_K or Q8_0);
// the multi-group path takes any mix of K-quants (Q4_K / Q5_K / Q6_K, the
// routed experts included) for every architecture. token_embd may be any type the reader
// knows (the gather dequantizes rows).
int sh_gguf_supported(const ModelDesc& m) {
  bool all_kq = sh_kquant_type(m.output.type), uniform = m.arch == ARCH_LLAMA;
  const uint32_t wt = m.layers.empty() ? (uint32_t)GGML_Q4_K : m.layers[0].wq.type;
  uniform = uniform && (wt == GGML_Q4_K || wt == GGML_Q8_0) &&
            (m.output.type == GGML_Q4_K || m.output.type == GGML_Q8_0);
  for (uint32_t l = 0; l < m.n_layer; ++l) {
    const LayerDesc& L = m.layers[l];
    for (const TRef* t : {&L.wq, &L.wk, &L.wv, &L.wo, &L.gate, &L.up, &L.down, &L.gate_exps, &L.up_exps, &L.down_exps})
      if (t->present()) {
        all_kq = all_kq && sh_kquant_type(t->type);
        uniform = uniform && t->type == wt;
      }
    if (L.gate_inp.present())
      SH_CHECK(L.gate_inp.type == GGML_F32, SH_ERR_UNSUPPORTED, "layer %u: router type %u (f32 only)", l,
               L.gate_inp.type);
  }
  SH_CHECK(all_kq || uniform, SH_ERR_UNSUPPORTED,
           "weight types: the matrices must all be K-quants (Q4_K / Q5_K / Q6_K), or llama layers uniformly Q4_K or "
           "Q8_0 (first layer type %u, lm_head %u)",
           wt, m.output.type);
  SH_CHECK(m.arch != ARCH_QWEN3MOE || (m.n_expert <= 1024 && m.d % 4 == 0 && (m.d + m.n_expert) * 4 <= 60 * 1024),
           SH_ERR_UNSUPPORTED, "moe: %u experts at n_embd %u", m.n_expert, m.d);
  return SH_OK;
}

extern "C" int sh_gguf_inspect(const void* data, uint64_t size, sh_model_dims* out) {
  SH_CHECK(data && out, SH_ERR_ARG, "sh_gguf_inspect: NULL argument");
  GFile f;
  ModelDesc m;
  int rc = sh_gguf_parse((const uint8_t*)data, size, &f);
  if (!rc) rc = sh_gguf_describe(f, &m);
  if (!rc) rc = sh_gguf_supported(m);
  if (rc) return rc;
  std::memset(out, 0, sizeof *out);
  out->n_layer = m.n_layer; out->n_embd = m.d; out->n_head = m.n_head; out->n_head_kv = m.n_kv;
  out->head_dim = m.hd; out->n_ff = m.ff; out->n_vocab = m.V; out->n_ctx_train = m.n_ctx;
  out->rms_eps = m.eps; out->rope_freq_base = m.theta;
  out->weight_type = m.layers.empty() ? -1 : (int32_t)m.layers[0].wo.type;
  double bytes = (double)m.output.rows * (double)m.output.row_bytes;
  for (const LayerDesc& L : m.layers)
    for (const TRef* t : {&L.wq, &L.wk, &L.wv, &L.wo, &L.gate, &L.up, &L.down, &L.gate_exps, &L.up_exps,
                          &L.down_exps})
      if (t->present()) bytes += (double)t->rows * (double)t->row_bytes * (double)t->n_mat;
  out->weight_bytes = bytes;
  return SH_OK;
}
