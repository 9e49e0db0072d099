// Synthetic GGUF model generator (host-only, OpenMP).
//
// Produces GGUF v3 byte images of Llama, Qwen3 and Qwen3-MoE architecture
// models whose weights are N(0, std) draws from a counter-based
// Philox4x64-10 stream, quantized to Q8_0 or Q4_K by the quantizer below. The reference never quantizes weights (it
// only reads GGUF files), so the quantizer is an input generator, not a parity
// target: the GPU path and the CPU oracle both read the SAME bytes.
//
// Format follows the reader in crates/seeker-core/src/gguf/mod.rs:161-230
// (magic "GGUF", version 3, u64 counts, metadata KV, tensor infos, data section
// aligned to `general.alignment` = 32) and block layouts from
// crates/seeker-core/src/gguf/types.rs:92-136 (Q8_0 = 32 elem / 34 B,
// Q4_K = 256 elem / 144 B). Metadata keys and tensor names follow
// crates/seeker-vulkan/src/models/llama.rs:1038-1048 and :1074-1090,
// models/qwen3.rs:591-698 and models/qwen35moe.rs:126-130, 4118-4131.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <functional>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "sh_f16.h"
#include "sh_philox.h"

namespace {

enum : uint32_t { GT_F32 = 0, GT_F16 = 1, GT_Q8_0 = 8, GT_Q4_K = 12, GT_Q5_K = 13, GT_Q6_K = 14 };
enum : uint32_t { MV_U32 = 4, MV_F32 = 6, MV_STRING = 8 };

struct Buf {
  std::vector<uint8_t> b;
  void u32(uint32_t v) { raw(&v, 4); }
  void u64(uint64_t v) { raw(&v, 8); }
  void f32(float v) { raw(&v, 4); }
  void str(const std::string& s) { u64(s.size()); raw(s.data(), s.size()); }
  void raw(const void* p, size_t n) {
    const uint8_t* c = (const uint8_t*)p;
    b.insert(b.end(), c, c + n);
  }
};

// Draw element e of the N(0,1) stream with key (seed, stream). Each Philox
// block yields 4 u64 words; words (0,1) and (2,3) are Box-Muller pairs.
// Counter convention matches numpy.random.Philox: block i uses counter i+1.
inline void normals4(uint64_t seed, uint64_t stream, uint64_t block, double out[4]) {
  uint64_t ctr[4] = {block + 1, 0, 0, 0};
  uint64_t key[2] = {seed, stream};
  uint64_t w[4];
  sh_philox4x64_10(ctr, key, w);
  for (int p = 0; p < 2; ++p) {
    double u1 = ((double)(w[2 * p] >> 11) + 0.5) * 0x1.0p-53;
    double u2 = ((double)(w[2 * p + 1] >> 11) + 0.5) * 0x1.0p-53;
    double r = std::sqrt(-2.0 * std::log(u1));
    double t = 6.283185307179586476925286766559 * u2;
    out[2 * p] = r * std::cos(t);
    out[2 * p + 1] = r * std::sin(t);
  }
}

inline int round_half_up(float v) { return (int)std::floor(v + 0.5f); }

// Q8_0: d = amax/127 (stored f16), q = clamp(round(x / d), -127, 127).
void quant_q8_0_block(const float* x, uint8_t* out) {
  float amax = 0.f;
  for (int i = 0; i < 32; ++i) amax = std::fmax(amax, std::fabs(x[i]));
  float d = amax / 127.f;
  uint16_t dh = sh_f32_to_f16(d);
  std::memcpy(out, &dh, 2);
  for (int i = 0; i < 32; ++i) {
    int q = d > 0.f ? round_half_up(x[i] / d) : 0;
    q = q < -127 ? -127 : (q > 127 ? 127 : q);
    out[2 + i] = (uint8_t)(int8_t)q;
  }
}

// Q4_K: per 32-element sub-block s, value ~= d*sc_s*q - dmin*m_s with 6-bit
// sc_s, m_s and 4-bit q. d = max(range_s/15)/63, dmin = max(-min_s)/63.
void quant_q4_k_block(const float* x, uint8_t* out) {
  float scr[8], mr[8];
  for (int s = 0; s < 8; ++s) {
    float mn = x[32 * s], mx = x[32 * s];
    for (int i = 1; i < 32; ++i) {
      mn = std::fmin(mn, x[32 * s + i]);
      mx = std::fmax(mx, x[32 * s + i]);
    }
    if (mn > 0.f) mn = 0.f;
    mr[s] = -mn;
    scr[s] = (mx - mn) / 15.f;
  }
  float dmax = 0.f, mmax = 0.f;
  for (int s = 0; s < 8; ++s) { dmax = std::fmax(dmax, scr[s]); mmax = std::fmax(mmax, mr[s]); }
  uint16_t dh = sh_f32_to_f16(dmax / 63.f), mh = sh_f32_to_f16(mmax / 63.f);
  float d = sh_f16_to_f32(dh), dmin = sh_f16_to_f32(mh);
  int sc[8], m[8];
  for (int s = 0; s < 8; ++s) {
    int a = d > 0.f ? round_half_up(scr[s] / d) : 0;
    int b = dmin > 0.f ? round_half_up(mr[s] / dmin) : 0;
    sc[s] = a < 0 ? 0 : (a > 63 ? 63 : a);
    m[s] = b < 0 ? 0 : (b > 63 ? 63 : b);
  }
  std::memcpy(out, &dh, 2);
  std::memcpy(out + 2, &mh, 2);
  uint8_t* scales = out + 4;
  for (int j = 0; j < 4; ++j) {
    scales[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
    scales[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
    scales[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4));
  }
  uint8_t q[256];
  for (int s = 0; s < 8; ++s) {
    float step = d * (float)sc[s];
    float off = dmin * (float)m[s];
    for (int i = 0; i < 32; ++i) {
      int v = step > 0.f ? round_half_up((x[32 * s + i] + off) / step) : 0;
      q[32 * s + i] = (uint8_t)(v < 0 ? 0 : (v > 15 ? 15 : v));
    }
  }
  uint8_t* qs = out + 16;
  for (int g = 0; g < 4; ++g)
    for (int l = 0; l < 32; ++l) qs[32 * g + l] = (uint8_t)(q[64 * g + l] | (q[64 * g + 32 + l] << 4));
}

// Q5_K (176 B / 256): d, dmin, the Q4_K 6-bit scale / min packing, qh[32],
// qs[128]; element e of sub-block s (l = e % 32) keeps its low nibble in
// qs[32 (s / 2) + l] (bits 4 (s % 2)) and its fifth bit as bit s of qh[l]
// (the dequant order of llama.cpp's dequantize_row_q5_K). A min/max quantizer
// per 32-element sub-block with 31 steps.
void quant_q5_k_block(const float* x, uint8_t* out) {
  float scr[8], mr[8];
  for (int s = 0; s < 8; ++s) {
    float mn = x[32 * s], mx = x[32 * s];
    for (int i = 1; i < 32; ++i) {
      mn = std::fmin(mn, x[32 * s + i]);
      mx = std::fmax(mx, x[32 * s + i]);
    }
    if (mn > 0.f) mn = 0.f;
    mr[s] = -mn;
    scr[s] = (mx - mn) / 31.f;
  }
  float dmax = 0.f, mmax = 0.f;
  for (int s = 0; s < 8; ++s) { dmax = std::fmax(dmax, scr[s]); mmax = std::fmax(mmax, mr[s]); }
  uint16_t dh = sh_f32_to_f16(dmax / 63.f), mh = sh_f32_to_f16(mmax / 63.f);
  float d = sh_f16_to_f32(dh), dmin = sh_f16_to_f32(mh);
  int sc[8], m[8];
  for (int s = 0; s < 8; ++s) {
    int a = d > 0.f ? round_half_up(scr[s] / d) : 0;
    int b = dmin > 0.f ? round_half_up(mr[s] / dmin) : 0;
    sc[s] = a < 0 ? 0 : (a > 63 ? 63 : a);
    m[s] = b < 0 ? 0 : (b > 63 ? 63 : b);
  }
  std::memset(out, 0, 176);
  std::memcpy(out, &dh, 2);
  std::memcpy(out + 2, &mh, 2);
  uint8_t* scales = out + 4;
  for (int j = 0; j < 4; ++j) {
    scales[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
    scales[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
    scales[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4));
  }
  uint8_t* qh = out + 16;
  uint8_t* qs = out + 48;
  for (int s = 0; s < 8; ++s) {
    float step = d * (float)sc[s], off = dmin * (float)m[s];
    for (int l = 0; l < 32; ++l) {
      int v = step > 0.f ? round_half_up((x[32 * s + l] + off) / step) : 0;
      v = v < 0 ? 0 : (v > 31 ? 31 : v);
      qs[32 * (s / 2) + l] |= (uint8_t)((v & 0xF) << (4 * (s % 2)));
      if (v & 16) qh[l] |= (uint8_t)(1u << s);
    }
  }
}

// Q6_K (210 B / 256): ql[128], qh[64], int8 scales[16], d; element e (n =
// e / 128, g = e % 128 / 32, l = e % 32) keeps its low nibble in ql[64 n + l +
// 32 (g % 2)] (bits 4 (g / 2)) and its top two bits in qh[32 n + l] (bits 2 g),
// value d * scales[e / 16] * (q - 32) (run.rs:4257-4291). Symmetric per
// 16-element sub-block, 31 steps each way.
void quant_q6_k_block(const float* x, uint8_t* out) {
  float ss[16], smax = 0.f;
  for (int s = 0; s < 16; ++s) {
    float a = 0.f;
    for (int i = 0; i < 16; ++i) a = std::fmax(a, std::fabs(x[16 * s + i]));
    ss[s] = a / 31.f;
    smax = std::fmax(smax, ss[s]);
  }
  const uint16_t dh = sh_f32_to_f16(smax / 127.f);
  const float d = sh_f16_to_f32(dh);
  std::memset(out, 0, 210);
  uint8_t* ql = out;
  uint8_t* qh = out + 128;
  int8_t* sc = (int8_t*)(out + 192);
  for (int s = 0; s < 16; ++s) {
    int v = d > 0.f ? round_half_up(ss[s] / d) : 0;
    sc[s] = (int8_t)(v < 0 ? 0 : (v > 127 ? 127 : v));
  }
  for (int e = 0; e < 256; ++e) {
    const float step = d * (float)sc[e / 16];
    int q = step > 0.f ? round_half_up(x[e] / step) + 32 : 32;
    q = q < 0 ? 0 : (q > 63 ? 63 : q);
    const int n = e / 128, g = e % 128 / 32, l = e % 32;
    ql[64 * n + l + 32 * (g % 2)] |= (uint8_t)((q & 0xF) << (4 * (g / 2)));
    qh[32 * n + l] |= (uint8_t)((q >> 4) << (2 * g));
  }
  std::memcpy(out + 208, &dh, 2);
}

struct TensorSpec {
  std::string name;
  uint64_t ne0, ne1, ne2;  // ne0 = contracting / innermost dim, ne1 = rows, ne2 = expert slabs
  uint32_t type;
  int kind;                // 0: N(0, weight_std) quantized; 1: norm weight 1 + jitter N(0, 1); 2: f32 N(0, router_std)
  uint64_t offset;         // within data section
  uint64_t bytes;
};

uint64_t tensor_bytes(uint32_t type, uint64_t n) {
  switch (type) {
    case GT_F32: return n * 4;
    case GT_F16: return n * 2;
    case GT_Q8_0: return n / 32 * 34;
    case GT_Q4_K: return n / 256 * 144;
    case GT_Q5_K: return n / 256 * 176;
    case GT_Q6_K: return n / 256 * 210;
  }
  return 0;
}

void fill_tensor(const TensorSpec& t, uint64_t seed, uint64_t stream, float stdv, float jitter, float router_std,
                 uint8_t* dst) {
  const uint64_t n = t.ne0 * t.ne1 * t.ne2;
  if (t.kind != 0) {  // f32: norm weights (1 + jitter z) or the router (router_std z)
    const int64_t nb = (int64_t)((n + 3) / 4);
#pragma omp parallel for schedule(static, 256)
    for (int64_t b = 0; b < nb; ++b) {
      double z[4];
      normals4(seed, stream, (uint64_t)b, z);
      for (int i = 0; i < 4; ++i) {
        const uint64_t e = (uint64_t)b * 4 + i;
        if (e >= n) break;
        const float v = t.kind == 1 ? (float)(1.0 + (double)jitter * z[i]) : (float)((double)router_std * z[i]);
        std::memcpy(dst + 4 * e, &v, 4);
      }
    }
    return;
  }
  const bool kq = t.type == GT_Q4_K || t.type == GT_Q5_K || t.type == GT_Q6_K;
  const uint64_t blk = kq ? 256 : 32;
  const uint64_t bbytes = tensor_bytes(t.type, blk);
  const int64_t nblk = (int64_t)(n / blk);
#pragma omp parallel for schedule(static, 256)
  for (int64_t b = 0; b < nblk; ++b) {
    float x[256];
    for (uint64_t e = 0; e < blk; e += 4) {
      double z[4];
      normals4(seed, stream, ((uint64_t)b * blk + e) / 4, z);
      for (int i = 0; i < 4; ++i) x[e + i] = (float)(z[i] * (double)stdv);
    }
    uint8_t* o = dst + (uint64_t)b * bbytes;
    if (t.type == GT_Q4_K) quant_q4_k_block(x, o);
    else if (t.type == GT_Q5_K) quant_q5_k_block(x, o);
    else if (t.type == GT_Q6_K) quant_q6_k_block(x, o);
    else quant_q8_0_block(x, o);
  }
}

}  // namespace

extern "C" {

// Configuration of a synthetic model. arch: 0 llama (models/llama.rs:1038-1090),
// 1 qwen3 (models/qwen3.rs:591-698: decoupled head_dim, attn_q_norm /
// attn_k_norm), 2 qwen3moe (qwen3 attention; ffn_gate_inp f32 [n_embd,
// n_expert] router and 3-D ffn_{gate,up,down}_exps slabs, the layout of
// models/qwen35moe.rs:126-130). wtype/etype are GGML type ids (8 = Q8_0,
// 12 = Q4_K) of the matrices and token_embd. head_dim 0 = n_embd / n_head.
typedef struct sh_synth_cfg {
  uint32_t arch;
  uint32_t n_layer, n_embd, n_head, n_head_kv, head_dim, n_ff, n_vocab, n_ctx;
  uint32_t n_expert, n_expert_used, expert_ff;
  float rms_eps, rope_base, weight_std, norm_jitter, router_std;
  uint32_t wtype, etype;
  uint32_t tied;  // 1: no output.weight (lm_head = token_embd)
  uint64_t seed;
  uint32_t out_type;  // output.weight type (0: wtype)
  uint32_t mix;       // 1: attn_v and ffn_down(_exps) of even layers in Q6_K (the Q4_K_M-style mix)
} sh_synth_cfg;

// Build a GGUF v3 image in host memory. *out is malloc'd; free with
// sh_synth_free. Returns 0 on success.
int sh_synth_gguf(const sh_synth_cfg* c, uint8_t** out, uint64_t* size) {
  if (!c || !out || !size || c->arch > 2) return 1;
  if (c->n_head == 0 || c->n_head % (c->n_head_kv ? c->n_head_kv : 1)) return 2;
  if (c->head_dim == 0 && c->n_embd % c->n_head) return 2;
  const bool qwen = c->arch != 0, moe = c->arch == 2;
  const uint32_t wt = c->wtype, et = c->etype;
  auto blk = [](uint32_t t) -> uint64_t { return (t == GT_Q4_K || t == GT_Q5_K || t == GT_Q6_K) ? 256 : 32; };
  const uint64_t qk_w = std::max(blk(wt), c->mix ? (uint64_t)256 : (uint64_t)1), qk_e = blk(et);
  const uint32_t ot = c->out_type ? c->out_type : wt;
  const uint64_t d = c->n_embd, ff = c->n_ff, hd = c->head_dim ? c->head_dim : d / c->n_head;
  const uint64_t qd = hd * c->n_head, dkv = hd * c->n_head_kv, E = c->n_expert, ef = c->expert_ff;
  if (d % qk_w || qd % qk_w || d % qk_e || (!moe && ff % qk_w) || (moe && (ef % qk_w || !E || !c->n_expert_used)))
    return 3;

  std::vector<TensorSpec> ts;
  ts.push_back({"token_embd.weight", d, c->n_vocab, 1, et, 0, 0, 0});
  for (uint32_t i = 0; i < c->n_layer; ++i) {
    std::string p = "blk." + std::to_string(i) + ".";
    ts.push_back({p + "attn_norm.weight", d, 1, 1, GT_F32, 1, 0, 0});
    ts.push_back({p + "attn_q.weight", d, qd, 1, wt, 0, 0, 0});
    ts.push_back({p + "attn_k.weight", d, dkv, 1, wt, 0, 0, 0});
    const uint32_t mt = (c->mix == 1 && i % 2 == 0) ? (uint32_t)GT_Q6_K : wt;  // attn_v / ffn_down
    ts.push_back({p + "attn_v.weight", d, dkv, 1, mt, 0, 0, 0});
    if (qwen) {
      ts.push_back({p + "attn_q_norm.weight", hd, 1, 1, GT_F32, 1, 0, 0});
      ts.push_back({p + "attn_k_norm.weight", hd, 1, 1, GT_F32, 1, 0, 0});
    }
    ts.push_back({p + "attn_output.weight", qd, d, 1, wt, 0, 0, 0});
    ts.push_back({p + "ffn_norm.weight", d, 1, 1, GT_F32, 1, 0, 0});
    if (moe) {
      ts.push_back({p + "ffn_gate_inp.weight", d, E, 1, GT_F32, 2, 0, 0});
      ts.push_back({p + "ffn_gate_exps.weight", d, ef, E, wt, 0, 0, 0});
      ts.push_back({p + "ffn_up_exps.weight", d, ef, E, wt, 0, 0, 0});
      ts.push_back({p + "ffn_down_exps.weight", ef, d, E, mt, 0, 0, 0});
    } else {
      ts.push_back({p + "ffn_gate.weight", d, ff, 1, wt, 0, 0, 0});
      ts.push_back({p + "ffn_up.weight", d, ff, 1, wt, 0, 0, 0});
      ts.push_back({p + "ffn_down.weight", ff, d, 1, mt, 0, 0, 0});
    }
  }
  ts.push_back({"output_norm.weight", d, 1, 1, GT_F32, 1, 0, 0});
  if (!c->tied) ts.push_back({"output.weight", d, c->n_vocab, 1, ot, 0, 0, 0});

  const std::string A = c->arch == 0 ? "llama" : (c->arch == 1 ? "qwen3" : "qwen3moe");
  Buf h;
  std::vector<std::function<void()>> kvs;
  auto kv_str = [&](std::string k, std::string v) { kvs.push_back([&h, k, v] { h.str(k); h.u32(MV_STRING); h.str(v); }); };
  auto kv_u32 = [&](std::string k, uint32_t v) { kvs.push_back([&h, k, v] { h.str(k); h.u32(MV_U32); h.u32(v); }); };
  auto kv_f32 = [&](std::string k, float v) { kvs.push_back([&h, k, v] { h.str(k); h.u32(MV_F32); h.f32(v); }); };
  kv_str("general.architecture", A);
  kv_u32("general.alignment", 32);
  kv_u32(A + ".block_count", c->n_layer);
  kv_u32(A + ".attention.head_count", c->n_head);
  kv_u32(A + ".attention.head_count_kv", c->n_head_kv);
  kv_u32(A + ".embedding_length", c->n_embd);
  if (!moe) kv_u32(A + ".feed_forward_length", c->n_ff);
  kv_u32(A + ".context_length", c->n_ctx);
  kv_u32(A + ".rope.dimension_count", (uint32_t)hd);
  kv_f32(A + ".rope.freq_base", c->rope_base);
  kv_f32(A + ".attention.layer_norm_rms_epsilon", c->rms_eps);
  kv_u32(A + ".vocab_size", c->n_vocab);
  if (qwen) {
    kv_u32(A + ".attention.key_length", (uint32_t)hd);
    kv_u32(A + ".attention.value_length", (uint32_t)hd);
  }
  if (moe) {
    kv_u32(A + ".expert_count", c->n_expert);
    kv_u32(A + ".expert_used_count", c->n_expert_used);
    kv_u32(A + ".expert_feed_forward_length", c->expert_ff);
  }
  h.raw("GGUF", 4);
  h.u32(3);
  h.u64(ts.size());
  h.u64(kvs.size());
  for (auto& f : kvs) f();

  uint64_t off = 0;
  for (auto& t : ts) {
    t.bytes = tensor_bytes(t.type, t.ne0 * t.ne1 * t.ne2);
    t.offset = off;
    off += (t.bytes + 31) / 32 * 32;
  }
  for (auto& t : ts) {
    h.str(t.name);
    if (t.ne2 > 1) { h.u32(3); h.u64(t.ne0); h.u64(t.ne1); h.u64(t.ne2); }
    else if (t.ne1 == 1) { h.u32(1); h.u64(t.ne0); }
    else { h.u32(2); h.u64(t.ne0); h.u64(t.ne1); }
    h.u32(t.type);
    h.u64(t.offset);
  }
  uint64_t data_start = (h.b.size() + 31) / 32 * 32;
  uint64_t total = data_start + off;
  uint8_t* img = (uint8_t*)std::calloc(total, 1);
  if (!img) return 4;
  std::memcpy(img, h.b.data(), h.b.size());
  for (size_t i = 0; i < ts.size(); ++i)
    fill_tensor(ts[i], c->seed, (uint64_t)i, c->weight_std, c->norm_jitter, c->router_std,
                img + data_start + ts[i].offset);
  *out = img;
  *size = total;
  return 0;
}

// The Llama subset of sh_synth_cfg (norm weights all 1).
typedef struct sh_synth_llama_cfg {
  uint32_t n_layer, n_embd, n_head, n_head_kv, n_ff, n_vocab, n_ctx;
  float rms_eps, rope_base, weight_std;
  uint32_t wtype, etype;
  uint32_t tied;
  uint64_t seed;
} sh_synth_llama_cfg;

int sh_synth_llama_gguf(const sh_synth_llama_cfg* c, uint8_t** out, uint64_t* size) {
  if (!c) return 1;
  sh_synth_cfg g{};
  g.arch = 0;
  g.n_layer = c->n_layer; g.n_embd = c->n_embd; g.n_head = c->n_head; g.n_head_kv = c->n_head_kv;
  g.n_ff = c->n_ff; g.n_vocab = c->n_vocab; g.n_ctx = c->n_ctx;
  g.rms_eps = c->rms_eps; g.rope_base = c->rope_base; g.weight_std = c->weight_std;
  g.wtype = c->wtype; g.etype = c->etype; g.tied = c->tied; g.seed = c->seed;
  return sh_synth_gguf(&g, out, size);
}

void sh_synth_free(void* p) { std::free(p); }

// Token ids uniform in [0, vocab): id = (w >> 32) * vocab >> 32 over the
// Philox stream (seed, 0xFFFF_FFFF) word i (numpy counter convention).
void sh_synth_tokens(uint64_t seed, uint32_t n, uint32_t vocab, uint32_t* out) {
  for (uint32_t i = 0; i < n; ++i) {
    uint64_t ctr[4] = {(uint64_t)(i / 4) + 1, 0, 0, 0};
    uint64_t key[2] = {seed, 0xFFFFFFFFull};
    uint64_t w[4];
    sh_philox4x64_10(ctr, key, w);
    out[i] = (uint32_t)(((w[i % 4] >> 32) * (uint64_t)vocab) >> 32);
  }
}

// Fill n f32 values with N(mean, std) draws (stream key (seed, stream)).
void sh_synth_normal_f32(uint64_t seed, uint64_t stream, float mean, float stdv, uint64_t n, float* out) {
  const int64_t nb = (int64_t)((n + 3) / 4);
#pragma omp parallel for schedule(static, 1024)
  for (int64_t b = 0; b < nb; ++b) {
    double z[4];
    normals4(seed, stream, (uint64_t)b, z);
    for (int i = 0; i < 4; ++i) {
      uint64_t e = (uint64_t)b * 4 + i;
      if (e < n) out[e] = (float)(mean + stdv * z[i]);
    }
  }
}

// Quantize rows of f32 values (n multiple of the block size) to Q8_0 / Q4_K.
int sh_synth_quantize(uint32_t type, const float* x, uint64_t n, uint8_t* out) {
  if (type == GT_Q5_K || type == GT_Q6_K) {
    if (n % 256) return 1;
    const uint64_t bb = tensor_bytes(type, 256);
#pragma omp parallel for schedule(static, 256)
    for (int64_t b = 0; b < (int64_t)(n / 256); ++b) {
      if (type == GT_Q5_K) quant_q5_k_block(x + 256 * b, out + bb * b);
      else quant_q6_k_block(x + 256 * b, out + bb * b);
    }
    return 0;
  }
  if (type == GT_Q8_0) {
    if (n % 32) return 1;
#pragma omp parallel for schedule(static, 1024)
    for (int64_t b = 0; b < (int64_t)(n / 32); ++b) quant_q8_0_block(x + 32 * b, out + 34 * b);
    return 0;
  }
  if (type == GT_Q4_K) {
    if (n % 256) return 1;
#pragma omp parallel for schedule(static, 256)
    for (int64_t b = 0; b < (int64_t)(n / 256); ++b) quant_q4_k_block(x + 256 * b, out + 144 * b);
    return 0;
  }
  return 2;
}

}  // extern "C"
