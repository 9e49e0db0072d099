// GGUF reader and model description (host-only C++; no HIP).
//
// parse + validate a GGUF v2/v3 image held in caller memory (semantics of
// crates/seeker-core/src/gguf/mod.rs:161-230: magic, version, u64 counts,
// typed metadata, tensor infos, data section aligned to general.alignment),
// then describe the model it holds for one of the architectures this library
// runs: "llama" (models/llama.rs:1038-1090), "qwen3" (models/qwen3.rs:591-698:
// decoupled head_dim, per-head Q/K RMSNorm, NEOX RoPE) and "qwen3moe" (the
// qwen3 attention block with the routed-expert FFN of
// models/qwen35moe.rs:3117-3182, no shared expert).
//
// Every size is computed overflow-safe and every tensor the model reads is
// checked to lie inside the image with the shape the model needs, so a
// malformed file is rejected before any byte of it is used.
#pragma once
#include <cstdint>
#include <map>
#include <string>
#include <vector>

#include "sh_error.h"

// GGML type ids used here (crates/seeker-core/src/gguf/types.rs:17-60).
enum : int { GGML_F32 = 0, GGML_F16 = 1, GGML_Q8_0 = 8, GGML_Q4_K = 12, GGML_Q5_K = 13, GGML_Q6_K = 14 };

// (elements, bytes) per block of a GGML type (gguf/types.rs:90-136); false for
// a type this reader does not know.
bool sh_ggml_block(uint32_t type, uint32_t* elems, uint32_t* bytes);

struct GTensor {
  std::string name;
  uint32_t type = 0;
  uint64_t ne[4] = {1, 1, 1, 1};
  uint32_t nd = 0;
  uint64_t off = 0;    // from the data section start
  uint64_t bytes = 0;  // whole tensor
};

struct GFile {
  const uint8_t* base = nullptr;
  uint64_t size = 0;
  std::map<std::string, double> num;
  std::map<std::string, std::string> str;
  std::vector<GTensor> tensors;
  const uint8_t* data = nullptr;
  const GTensor* find(const std::string& n) const;
};

// Parses the header and tensor table; every tensor of a known type is checked
// to lie inside the image. Unknown tensor types are kept (bytes = 0) and
// rejected only if the model uses them.
int sh_gguf_parse(const uint8_t* img, uint64_t size, GFile* f);

enum ModelArch { ARCH_LLAMA = 0, ARCH_QWEN3 = 1, ARCH_QWEN3MOE = 2 };

struct TRef {  // a tensor the model reads
  const uint8_t* data = nullptr;
  uint32_t type = 0;
  uint64_t rows = 0, cols = 0, n_mat = 1;  // n_mat: expert slabs
  uint64_t row_bytes = 0;
  bool present() const { return data != nullptr; }
};

struct LayerDesc {
  TRef attn_norm, ffn_norm, q_norm, k_norm;  // f32 vectors (q/k norms: qwen3 / qwen3moe, [head_dim])
  TRef wq, wk, wv, wo;                       // [rows = out][cols = in]
  TRef gate, up, down;                       // dense FFN
  TRef gate_inp, gate_exps, up_exps, down_exps;  // routed experts (qwen3moe)
};

struct ModelDesc {
  int arch = ARCH_LLAMA;
  uint32_t n_layer = 0, d = 0, n_head = 0, n_kv = 0, hd = 0, ff = 0, V = 0, n_ctx = 0;
  uint32_t n_expert = 0, n_expert_used = 0, expert_ff = 0;
  float eps = 1e-5f, theta = 10000.f;
  bool neox = false;     // NEOX RoPE (pairs i, i + hd/2) instead of NORM (pairs 2i, 2i+1)
  bool qk_norm = false;  // per-head RMSNorm of q and k before RoPE
  TRef tok_embd, out_norm, output;  // output = token_embd when tied
  std::vector<LayerDesc> layers;
  uint32_t q_dim() const { return n_head * hd; }
  uint32_t kv_dim() const { return n_kv * hd; }
};

// Describes a parsed file as a model this library can run: architecture keys
// and defaults, every tensor present with the expected shape and a type the
// GEMV kernels take. Returns SH_OK, SH_ERR_FORMAT (malformed / inconsistent)
// or SH_ERR_UNSUPPORTED (valid, but a feature this build does not implement).
int sh_gguf_describe(const GFile& f, ModelDesc* out);

// Whether this build's device path runs the described model (architecture,
// matrix types); SH_ERR_UNSUPPORTED with a message otherwise.
int sh_gguf_supported(const ModelDesc& m);
