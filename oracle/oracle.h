/* CPU oracle for the seeker speculative-decoding verify path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library; it is never part of
 * the shipped product path.
 *
 * This is a plain-C restatement of the reference's algorithm (rgcottrell/seeker,
 * Rust + Vulkan/Slang), which cannot be compiled here (no Rust toolchain, no
 * slangc, no Vulkan). Every function cites the reference file:line it follows.
 * Numerics: f32 storage between ops (as the reference), f64 accumulation
 * inside ops (the exact value the reference's f32 kernels approximate), K/V
 * stored as IEEE f16 with round-to-nearest-even.
 */
#ifndef SEEKER_ORACLE_H
#define SEEKER_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { OR_F32 = 0, OR_F16 = 1, OR_Q8_0 = 8, OR_Q4_K = 12, OR_Q5_K = 13, OR_Q6_K = 14 };

float or_f16_to_f32(uint16_t h);
uint16_t or_f32_to_f16(float f);
uint16_t or_f64_to_f16(double f);

/* Philox4x64-10 block (numpy.random.Philox raw block for the given counter). */
void or_philox4x64_10(const uint64_t ctr[4], const uint64_t key[2], uint64_t out[4]);
/* Word i of stream key=(k0,k1): block (i/4 + 1, 0, 0, 0), word i % 4. */
uint64_t or_philox_word(uint64_t k0, uint64_t k1, uint64_t i);
float or_unit_f32(uint64_t w);

/* Dequantize one row of K elements (apps/seeker-cli/src/commands/run.rs:4212-4303). */
int or_dequant_row(int type, const uint8_t* raw, uint64_t row, uint64_t k, float* out);
/* y[j*M + m] = sum_k deq(W)[m,k] * x[j*K + k]  (ggml layout, ops/matmul.rs:295-299). */
int or_gemv(int type, const uint8_t* w, uint64_t M, uint64_t K, const float* x, uint32_t N, float* y);

/* The reference's wide-GEMM arithmetic (mul_mm_cm.slang, N >= 32): f16(dequant)
 * times f16(x), accumulated (here in f64). */
int or_gemv16(int type, const uint8_t* w, uint64_t M, uint64_t K, const float* x, uint32_t N, float* y);

typedef struct or_model or_model;
typedef struct or_kv or_kv;

/* Parse a llama / qwen3 / qwen3moe GGUF image kept in caller memory (must
 * outlive the model). */
int or_model_open(const uint8_t* img, uint64_t size, or_model** out);
void or_model_free(or_model* m);
/* Dense matmuls of later or_forward calls through or_gemv16 (on != 0) or
 * or_gemv (the MoE router and experts always use or_gemv). */
/* 0: exact dense matmuls; 1: all as or_gemv16; 2: as or_gemv16 in forward
 * calls of >= 32 columns (the reference's wide-GEMM dispatch). */
void or_model_set_mm16(or_model* m, int mode);
/* on != 0: causal forward calls of more than one column compute attention with
 * the reference's cooperative-matrix flash attention arithmetic (or_attn_cm1,
 * flash_attn_cm1.slang via ops/flash_attn.rs:442-471); single-column calls and
 * trees keep the exact softmax. Default off. */
void or_model_set_attn_cm1(or_model* m, int on);
/* flash_attn_cm1.slang for one query row q [hd] (f32, staged to f16 as the
 * shader does) over keys [0, n_keys) of an f16 cache whose key t row starts at
 * k + t * kv_stride (v likewise); visible[t] != 0 marks visible keys (NULL: all).
 * out [hd] f32. or_attn_cm1_core takes the staged f16 q16 directly. */
void or_attn_cm1(const float* q, const uint16_t* k, const uint16_t* v, size_t kv_stride, uint32_t hd,
                 uint32_t n_keys, const uint8_t* visible, float* out);
void or_attn_cm1_core(const uint16_t* q16, const uint16_t* k, const uint16_t* v, size_t kv_stride, uint32_t hd,
                      uint32_t n_keys, const uint8_t* visible, float* out);
/* n_layer, n_embd, n_head, n_head_kv, head_dim, n_ff, n_vocab */
void or_model_dims(const or_model* m, uint32_t dims[7]);
/* architecture (0 llama, 1 qwen3, 2 qwen3moe), n_expert, n_expert_used, expert_ff */
void or_model_moe_dims(const or_model* m, uint32_t dims[4]);
/* MoE gating: softmax over E logits, top-k (descending, ties to the lower
 * index), weights renormalized to sum 1 (topk_moe.slang with_norm). */
void or_moe_route(const float* logits, uint32_t E, uint32_t k, uint32_t* ids, float* w);

int or_kv_create(const or_model* m, uint32_t max_seq, or_kv** out);
void or_kv_free(or_kv* kv);
uint32_t or_kv_position(const or_kv* kv);
void or_kv_truncate(or_kv* kv, uint32_t new_pos);
void or_kv_set_position(or_kv* kv, uint32_t pos);
/* Raw f16 K or V of one layer in the reference layout [max_seq][n_kv][hd]. */
uint16_t* or_kv_layer(or_kv* kv, uint32_t layer, int is_v);
/* Move the K/V rows at slots base+src[i] to base+i (i < n, src ascending),
 * then position = base + n. */
void or_kv_compact(or_kv* kv, uint32_t base, const uint32_t* src, uint32_t n);

/* Forward L tokens at cache position pos (llama.rs:196-441, all-position
 * epilogue qwen35moe.rs:975-989). parents: NULL for a causal chain, else a
 * tree (parent index within the chunk, -1 = attaches to the prefix).
 * logits_mode: 0 none, 1 last column, 2 all columns ([L][V]).
 * residual_out: pre-output_norm hidden state [L][d] or NULL. */
int or_forward(or_model* m, or_kv* kv, const uint32_t* tokens, uint32_t L, uint32_t pos,
               const int32_t* parents, int logits_mode, float* logits, float* residual_out);

uint32_t or_argmax(const float* x, uint32_t n);
void or_softmax(const float* x, uint32_t n, float* out);

typedef struct or_sampler_cfg {
  float temperature;
  uint32_t top_k;
  float top_p;
  float min_p;
} or_sampler_cfg;

/* Host chain sample with an explicit uniform (inference/sample.rs:369-474). */
uint32_t or_sample_one(const float* logits, uint32_t V, const or_sampler_cfg* cfg, float u);
/* GPU full-vocab categorical: inverse CDF in vocab-index order of softmax(l/T)
 * (inference/ops/sampler.rs:303-368). */
uint32_t or_sample_vocab_order(const float* logits, uint32_t V, float temperature, float u);
/* sample_and_compare (inference/sample.rs:347-361) with explicit uniforms;
 * mode 0: host chain (sorted order), 1: vocab-order GPU chain. Returns n emitted. */
uint32_t or_sample_and_compare(const float* logits, uint32_t V, const uint32_t* drafts, uint32_t n,
                               const or_sampler_cfg* cfg, const float* uniforms, int mode,
                               uint32_t* emitted);

/* Speculative rejection sampling (new: Leviathan et al. 2023). p_logits [(k+1)][V],
 * q_logits [k][V]; u_acc[k], u_res[k+1]. Returns acc_len, writes next token. */
uint32_t or_rejection(const float* p_logits, const float* q_logits, const uint32_t* drafts, uint32_t k,
                      uint32_t V, float temperature, const float* u_acc, const float* u_res,
                      uint32_t* next_tok);
/* Tree acceptance (new: recursive rejection sampling over a token tree, the
 * multi-candidate speculative sampling of SpecInfer, Miao et al. 2024, with
 * Chen et al. 2023's single-draft step). Node 0 is the root; parents[i] < i;
 * p_logits [n][V] target logits at each node, q_logits [n][V] the draft logits
 * each node's children were drawn from. u [n][2]: u[2c] accepts child c,
 * u[2v+1] draws at node v. temperature 0: greedy. Returns 0 and writes the
 * accepted path (root first), its length and the next token. */
int or_tree_accept(const float* p_logits, const float* q_logits, const uint32_t* tokens, const int32_t* parents,
                   uint32_t n, uint32_t V, float temperature, const float* u, uint32_t* path, uint32_t* path_len,
                   uint32_t* next_tok);
/* softmax(l/T) in f64, rounded to f32. */
void or_probs(const float* logits, uint32_t V, float temperature, float* out);

/* Greedy speculative step with a separate draft model (inference/mod.rs:2108-2297):
 * draft n tokens greedily, verify [last, d_1..d_n], accept longest matching prefix,
 * truncate both caches. *dpending holds the draft's uncommitted tokens. */
int or_spec_step_greedy(or_model* tgt, or_model* drf, or_kv* tkv, or_kv* dkv, uint32_t last_token,
                        uint32_t n_max, uint32_t* dpending, uint32_t* n_dpending, uint32_t* emitted,
                        uint32_t* n_emitted, uint32_t* drafts_out);

/* Sampling modes of the speculative step (the values of include/seeker_hip.h's sh_sample_mode). */
enum { OR_SPEC_GREEDY = 0, OR_SPEC_COMPARE = 1, OR_SPEC_REJECTION = 2 };

/* Draft token at one position: argmax (GREEDY, COMPARE) or a vocab-order draw
 * from softmax(q/T) with uniform u (REJECTION). */
uint32_t or_spec_draft_token(int mode, const float* q_logits, uint32_t V, float T, float u);
/* Acceptance of one verify: p_logits [(n+1)][V], q_logits [n][V] (REJECTION),
 * u [2(n+1)]: u[2i] accepts draft i, u[2i+1] samples / resamples column i.
 * Returns the number of emitted tokens. */
uint32_t or_spec_accept(int mode, const float* p_logits, const float* q_logits, const uint32_t* drafts, uint32_t n,
                        uint32_t V, float T, const float* u, uint32_t* emitted);
/* Speculative step in any mode (inference/mod.rs:2108-2297); u [2(n+1) + n]
 * (NULL for GREEDY): verify-column uniforms, then one per draft draw. */
int or_spec_step(or_model* tgt, or_model* drf, or_kv* tkv, or_kv* dkv, uint32_t last_token, uint32_t n_max,
                 int mode, float T, const float* u, uint32_t* dpending, uint32_t* n_dpending, uint32_t* emitted,
                 uint32_t* n_emitted, uint32_t* drafts_out, float* p_out, float* q_out);

#ifdef __cplusplus
}
#endif
#endif
