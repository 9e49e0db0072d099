/* seeker_hip.h - C ABI of the MI355X (gfx950) speculative-decoding verify path.
 *
 * Drop-in boundary for the spec-decode subset of seeker-vulkan's `inference` +
 * `models` module surface (rgcottrell/seeker binds its backend by module
 * re-export, apps/seeker-cli/src/main.rs:22-29). A Rust crate binds this header
 * with bindgen exactly as crates/seeker-npu/build.rs:36-50 binds npu_shim.h.
 *
 * Conventions (mirroring crates/seeker-npu/shim/npu_shim.h:2-18):
 *  - every fallible call returns an int status, 0 = SH_OK; on failure the
 *    calling thread's sh_last_error() holds a human-readable message
 *    (the Rust side's Result<_, Box<dyn Error>> message);
 *  - handles are opaque and owned by the caller, released with *_destroy;
 *  - an sh_engine is driven by one host thread and owns one HIP stream;
 *    calls that return host data are synchronous;
 *  - host arrays are caller-allocated with explicit lengths;
 *  - "_dev" pointers are device pointers obtained from sh_dev_alloc.
 * Nothing here allocates on the host on behalf of the caller.
 */
#ifndef SEEKER_HIP_H
#define SEEKER_HIP_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct sh_engine sh_engine;
typedef struct sh_model sh_model;
typedef struct sh_kv sh_kv;
typedef struct sh_qtensor sh_qtensor;

enum sh_status {
  SH_OK = 0,
  SH_ERR_ARG = 1,         /* invalid argument / precondition (mod.rs:2326-2360 style) */
  SH_ERR_HIP = 2,         /* HIP runtime failure */
  SH_ERR_FORMAT = 3,      /* malformed or unsupported GGUF */
  SH_ERR_UNSUPPORTED = 4, /* valid request this build does not implement */
  SH_ERR_CAPACITY = 5,    /* KV capacity / size limit exceeded */
  SH_ERR_STATE = 6        /* cache position mismatch (llama.rs:186-192) */
};

/* Sampling modes for verify / spec steps. */
enum sh_sample_mode {
  SH_SAMPLE_GREEDY = 0,    /* per-column argmax, lowest index on ties (sample.rs:504-514) */
  SH_SAMPLE_COMPARE = 1,   /* reference sample-and-compare: softmax(l/T) inverse CDF in
                              vocab-index order (ops/sampler.rs:303-368) with per-column
                              uniforms, accept while sample == draft (sample.rs:347-361) */
  SH_SAMPLE_REJECTION = 2  /* new: min(1, p/q) accept + residual max(0, p - q) resample */
};

typedef struct sh_sampling {
  uint32_t mode;          /* enum sh_sample_mode */
  float temperature;      /* > 0 for COMPARE / REJECTION */
  uint64_t seed;          /* Philox4x64-10 key word 0 */
  uint64_t counter;       /* Philox word offset; advanced by calls that consume uniforms */
  const float* uniforms;  /* optional explicit host uniforms (overrides Philox), or NULL */
  /* Candidate filters of the reference's chain (SamplerConfig, sample.rs:85;
   * order sample.rs:369-473 / ops/sampler.rs:41-132), COMPARE only; zero
   * disables each. top_k in 1..256 (or >= V when V <= 256): a column draws
   * among its top_k logits sorted descending (ties to the lower id) after
   * top_p (0 < p < 1: drop once the cumulative softmax before a candidate
   * exceeds p), min_p (> 0: drop logits below max + ln min_p) and 1/T, in
   * that order, first candidate whose cumulative probability reaches u.
   * top_p / min_p without top_k, and top_k above 256, are refused
   * (SH_ERR_UNSUPPORTED). */
  uint32_t top_k;
  float top_p;
  float min_p;
  uint32_t reserved;      /* zero */
} sh_sampling;

typedef struct sh_model_dims {
  uint32_t n_layer, n_embd, n_head, n_head_kv, head_dim, n_ff, n_vocab, n_ctx_train;
  float rms_eps, rope_freq_base;
  int32_t weight_type; /* GGML type id of the 2-D weights */
  double weight_bytes; /* bytes a full-logits forward reads from the weight matrices */
} sh_model_dims;

typedef struct sh_kernel_stat {
  char name[48];
  uint64_t launches;
  double total_ms;
  double alg_bytes; /* algorithmic bytes summed over launches */
} sh_kernel_stat;

/* ---------------------------------------------------------------- misc */
const char* sh_last_error(void);
const char* sh_version(void);

/* ------------------------------------------------------------- engine */
/* Engine::new (crates/seeker-vulkan/src/inference/mod.rs:198). */
int sh_engine_create(int hip_device, sh_engine** out);
void sh_engine_destroy(sh_engine* e);
int sh_engine_sync(sh_engine* e);
/* Per-kernel hipEvent timing of every launch (profile.rs:25-173 analog). */
int sh_engine_set_profiling(sh_engine* e, int on);
int sh_engine_profile(sh_engine* e, sh_kernel_stat* out, uint32_t cap, uint32_t* n_out);
int sh_engine_profile_reset(sh_engine* e);
/* Graph replay counters: graphs captured and graph launches so far (the
 * reference's replay cache, inference/mod.rs:88-103, 988-1180, has the same
 * record-once / replay-per-step split). Diagnostic; no compute. */
int sh_engine_graph_stats(sh_engine* e, uint64_t* captures, uint64_t* launches);

/* Device buffers (plain HBM allocations for kernel-level entry points). */
int sh_dev_alloc(sh_engine* e, uint64_t bytes, void** out_dev);
int sh_dev_free(sh_engine* e, void* dev);
int sh_memcpy_h2d(sh_engine* e, void* dst_dev, const void* src, uint64_t bytes);
int sh_memcpy_d2h(sh_engine* e, void* dst, const void* src_dev, uint64_t bytes);

/* -------------------------------------------------------------- model */
/* models::open + Engine::upload_weights (models/mod.rs:537, inference/mod.rs:304)
 * for architectures "llama" (models/llama.rs:1038-1090), "qwen3" and
 * "qwen3moe" (models/qwen3.rs). Weight types: every matrix a K-quant (Q4_K,
 * Q5_K, Q6_K in any mix, e.g. Q4_K_M / Q5_K_M files; routed experts Q4_K), or
 * llama layers uniformly Q4_K or Q8_0; token_embd any of these, F16 or F32.
 * SH_ERR_UNSUPPORTED otherwise. */
int sh_model_load_gguf(sh_engine* e, const char* path, sh_model** out);
int sh_model_load_gguf_memory(sh_engine* e, const void* data, uint64_t size, sh_model** out);
void sh_model_destroy(sh_model* m);
/* Model::{vocab_size, cache_dims} (models/mod.rs:35-37). */
int sh_model_info(const sh_model* m, sh_model_dims* out);
/* Wide-GEMM arithmetic (ops/matmul.rs:406-446): the reference computes every
 * dense matmul of N >= 32 columns with its cooperative-matrix GEMM
 * (mul_mm_cm.slang: weights dequantized in f32 and rounded to f16, activations
 * rounded to f16, f32 accumulation) unless SEEKER_MM_CM=0. Here forward calls
 * of >= 32 columns (a batched verify counts all of its columns) do the same
 * when the model allows it (no routed experts, every matrix Q4_K) and the
 * switch is on (default on; SH_WIDE_F16=0 in the environment at upload turns
 * it off); otherwise they keep the f32-level path of narrower calls.
 * sh_model_wide_f16: *on = 1 when wide calls take the f16 arithmetic.
 * sh_model_set_wide_f16: on = 0 / 1; SH_ERR_UNSUPPORTED for 1 on a model
 * that does not allow it. */
int sh_model_wide_f16(const sh_model* m, int* on);
int sh_model_set_wide_f16(sh_model* m, int on);
/* Masked attention (ops/flash_attn.rs:442-471): the reference computes the
 * attention of every forward of more than one token (the causal mask of
 * models/llama.rs:216-222) with flash_attn_cm1.slang: q * scale * log2(e)
 * staged as f16, keys in 64-key blocks, P rounded to f16, P V accumulated per
 * 16-key chunk in f16, the output held in f16 and rescaled in f16 per block,
 * 1/L in f32. Here sh_forward_full / sh_verify_greedy / the verify and
 * draft catch-up forwards of sh_spec_step do the same for calls of more than
 * one column without tree parents, when the switch is on (default on;
 * SH_FA_CM=0 in the environment at upload turns it off). Single-column calls,
 * trees and batched verifies keep the f32-level attention (the reference's
 * scalar flash_attn.slang, ops/flash_attn.rs:488-632, 819-1016). */
int sh_model_cm1_attention(const sh_model* m, int* on);
int sh_model_set_cm1_attention(sh_model* m, int on);
/* The validation half of models::open (models/mod.rs:537; parse_params +
 * collect_weights, models/llama.rs:1038-1090) without a device: parses a GGUF
 * image in caller memory, checks every tensor the model reads (shape, type,
 * extent inside the image) and fills out as sh_model_info would. Returns
 * SH_ERR_FORMAT for a malformed file, SH_ERR_UNSUPPORTED for a valid one this
 * build cannot run. Touches no GPU. */
int sh_gguf_inspect(const void* data, uint64_t size, sh_model_dims* out);

/* ----------------------------------------------------------------- KV */
/* Engine::allocate_kv_cache (inference/mod.rs:318); f16 K/V. */
int sh_kv_create(sh_engine* e, const sh_model* m, uint32_t max_seq_len, sh_kv** out);
void sh_kv_destroy(sh_kv* kv);
int sh_kv_position(const sh_kv* kv, uint32_t* pos);
/* KvCache::truncate: position = min(new_pos, position) (kv_cache.rs:587-602). */
int sh_kv_truncate(sh_kv* kv, uint32_t new_pos);
/* Export / import positions [0, n_pos) of one layer's K (is_v = 0) or V in the
 * reference layout [n_pos][n_head_kv][head_dim] f16 (kv_cache.rs:99-111). */
int sh_kv_read_layer(sh_kv* kv, uint32_t layer, int is_v, uint32_t n_pos, uint16_t* out);
int sh_kv_write_layer(sh_kv* kv, uint32_t layer, int is_v, uint32_t n_pos, const uint16_t* in);
int sh_kv_set_position(sh_kv* kv, uint32_t pos);
/* New (no reference counterpart): move K/V rows base+src[i] -> base+i for
 * i < n (tree-verify path compaction), then position = base + n. */
int sh_kv_compact(sh_kv* kv, uint32_t base, const uint32_t* src, uint32_t n);

/* ------------------------------------------------------------ forward */
/* Model::record_forward_full(tokens, pos, full_logits, ..) + readback
 * (models/mod.rs:314-336, Engine::forward_full_readback inference/mod.rs:2427).
 * Llama body models/llama.rs:196-441 with all-position logits
 * (qwen35moe.rs:975-989). parents: NULL = causal chain, else tree parent index
 * per token (-1 = attaches to the cached prefix; positions = pos + depth).
 * logits_mode 0: none, 1: last column, 2: all columns. logits_out is [cols][V],
 * residual_out [L][n_embd] (pre-output_norm), either may be NULL.
 * Advances the cache position by L. */
int sh_forward_full(sh_engine* e, sh_model* m, sh_kv* kv, const uint32_t* tokens, uint32_t L, uint32_t pos,
                    const int32_t* parents, int logits_mode, float* logits_out, float* residual_out);

/* Greedy verify: forward [tokens] with all-position logits and return the
 * per-column argmax ids (record_greedy per column, inference/mod.rs:2154-2167). */
int sh_verify_greedy(sh_engine* e, sh_model* m, sh_kv* kv, const uint32_t* tokens, uint32_t L, uint32_t pos,
                     uint32_t* sampled_out);

/* Batched verify of B sequences: Engine::verify_unified (inference/mod.rs:
 * 2316-2398) over Model::record_forward_unified_verify (models/mod.rs:212-230,
 * Llama body models/llama.rs:620-837). Sequence s contributes seq_lens[s]
 * columns, packed flat in tokens (column starts = prefix sums, q_starts). Its
 * cache is caches[s] (the reference's BatchKvCache slot slots[s]); with
 * pos_s = that cache's position, column i of s writes K/V slot pos_s + i and
 * attends to the cached prefix plus, within the sequence, causally (parents ==
 * NULL) or to its tree ancestors (parents, flat, = index within the sequence
 * of the column's parent, -1 for a child of the prefix; trees <= 64 nodes).
 * positions (flat, optional) are the RoPE positions and must equal pos_s + i
 * (chains) or pos_s + depth (trees). Outputs, each optional: logits_out
 * [N_total][V], sampled_out [N_total] greedy argmax per column, residual_out
 * [N_total][n_embd] (before the output norm). Each cache advances by its
 * seq_len; the caller truncates it to the accepted length. */
int sh_verify_unified(sh_engine* e, sh_model* m, sh_kv* const* caches, uint32_t B, const uint32_t* tokens,
                      const uint32_t* seq_lens, const uint32_t* positions, const int32_t* parents,
                      float* logits_out, uint32_t* sampled_out, float* residual_out);
/* sh_verify_unified with the owning sequence's sampler per column, as the
 * reference's verify_unified (samplers[col_seq[i]].record_chain,
 * inference/mod.rs:2375-2386): samplers[s] (B entries) is GREEDY (argmax) or
 * COMPARE (softmax(l / T) inverse CDF in vocab order, ops/sampler.rs:303-368);
 * the j-th column of sequence s takes uniforms[j] of its explicit array, else
 * Philox word counter + j of key (seed, 0x5EC); each COMPARE sampler's counter
 * advances by seq_lens[s]. REJECTION is refused (it needs draft logits:
 * sh_accept_sample). samplers NULL: sh_verify_unified. */
int sh_verify_unified_sampled(sh_engine* e, sh_model* m, sh_kv* const* caches, uint32_t B, const uint32_t* tokens,
                              const uint32_t* seq_lens, const uint32_t* positions, const int32_t* parents,
                              sh_sampling* samplers, float* logits_out, uint32_t* sampled_out,
                              float* residual_out);

/* Engine::decode_speculative (inference/mod.rs:2108-2297) with a separate draft
 * model: drafts n = clamp(n_max,1,8) tokens on the device, verifies [last,
 * d_1..d_n], accepts, truncates both caches to pos + acc + 1. emitted_out
 * holds n + 1 entries; *n_emitted = acc + 1. drafts_out (n) may be NULL.
 *  - GREEDY (s NULL or mode 0): greedy drafts (draft_tokens mod.rs:2062-2092),
 *    host accept of matching argmax ids (mod.rs:2168-2179).
 *  - COMPARE: greedy drafts; each verify column i sampled in vocab order with
 *    uniform word 2i+1, accepted while sample == draft (mod.rs:2181-2231,
 *    sample.rs:347-361).
 *  - REJECTION (new): draft i drawn from softmax(draft logits / T) with word
 *    2(n+1) + i, accepted iff u_{2i} q(d) < p(d), first rejection resampled
 *    from max(0, p - q) with word 2i+1 (bonus from p_n).
 * Stochastic uniform words come from Philox key (seed, 0x5EC) at s->counter +
 * word, and the step advances s->counter by 3n + 2; with s->uniforms they are
 * uniforms[word], an array of 3n + 2 floats.
 * Every mode replays one captured HIP graph per (models, caches, n, pending
 * count, sampling parameters): positions, the Philox key and the word base are
 * device words written before each replay (the reference's single-submit
 * step with DecodeDyn patching, inference/mod.rs:2181-2231, decode_dyn.rs). */
int sh_spec_step(sh_engine* e, sh_model* target, sh_model* draft, sh_kv* tkv, sh_kv* dkv,
                 uint32_t last_token, uint32_t n_max, sh_sampling* s, uint32_t* emitted_out,
                 uint32_t* n_emitted, uint32_t* drafts_out);
/* Measurement diagnostic, no counterpart in the reference: a greedy
 * sh_spec_step whose drafts are forced_drafts[0..n) instead of the draft
 * model's argmax ids. The draft forwards still run, over the forced ids, so a
 * step does the same work (and replays the same graph shape) as a real one.
 * For the forced-acceptance throughput: drafts that replay the target's greedy
 * continuation are all accepted. Caches and pending tokens as sh_spec_step. */
int sh_spec_step_forced(sh_engine* e, sh_model* target, sh_model* draft, sh_kv* tkv, sh_kv* dkv,
                        uint32_t last_token, uint32_t n_max, const uint32_t* forced_drafts,
                        uint32_t* emitted_out, uint32_t* n_emitted);
/* Engine::draft_tokens (inference/mod.rs:2062-2092) with a separate draft
 * model: n = clamp(n_max, 1, 8) greedy drafts after last_token, fed through
 * the draft cache dkv (its pending tokens first, as sh_spec_step leaves them),
 * each argmax feeding the next position on the device; drafts_out [n]. The
 * cache advances by its pending count + n (d_n is not fed) and its pending
 * tokens are cleared: truncate it to the accepted length afterwards. Replays
 * one captured HIP graph per (model, cache, n, pending count). */
int sh_draft_tokens(sh_engine* e, sh_model* draft, sh_kv* dkv, uint32_t last_token, uint32_t n_max,
                    uint32_t* drafts_out);
/* The reference server's batched speculative step (server/inference.rs:
 * 2777-2924) for B sequences with their own target caches tkv[s], draft caches
 * dkv[s] and last tokens: n = clamp(n_max, 1, 8) greedy drafts per sequence,
 * the drafts of all sequences at one position drafted in one batched forward
 * of the draft model (the reference drafts each sequence with draft_tokens,
 * :2806-2812); one sh_verify_unified of every sequence's [last, d_1..d_n] with
 * its sampler (samplers NULL: greedy; else GREEDY or COMPARE per sequence, as
 * sh_verify_unified_sampled); per sequence the longest prefix whose sampled
 * token equals the draft is accepted (:2859-2883) and both caches are truncated
 * to pos + acc + 1. emitted_out [B][n + 1] (row s holds n_emitted[s] tokens),
 * drafts_out [B][n] (may be NULL). Draft caches carry d_n as pending after a
 * fully accepted step, as in sh_spec_step. */
int sh_spec_step_batch(sh_engine* e, sh_model* target, sh_model* draft, sh_kv* const* tkv, sh_kv* const* dkv,
                       uint32_t B, const uint32_t* last_tokens, uint32_t n_max, sh_sampling* samplers,
                       uint32_t* emitted_out, uint32_t* n_emitted, uint32_t* drafts_out);
/* Readback of the last stochastic sh_spec_step of this engine, the analog of
 * the reference's tensor taps (inference/context.rs:136-160, 283): target
 * logits p_out [(n+1)][V] and draft logits q_out [n][V] (either may be NULL),
 * *n_out = n, *V_out = V. SH_ERR_STATE if no stochastic step has run. */
int sh_spec_step_logits(sh_engine* e, float* p_out, float* q_out, uint32_t* n_out, uint32_t* V_out);

/* ------------------------------------------------------ kernel level */
/* Upload a GGUF-layout quantized matrix [M rows][K] (Q8_0, Q4_K, Q5_K or Q6_K;
 * the reference's mul_mat_vec_q4_k / q5_k / q6_k / q8_0 shaders) and repack it
 * for the MFMA GEMV. */
int sh_qtensor_upload(sh_engine* e, int ggml_type, const void* host_blocks, uint32_t M, uint32_t K,
                      sh_qtensor** out);
void sh_qtensor_destroy(sh_qtensor* t);
/* y[j][m] (+)= sum_k deq(W)[m][k] * x[j][k], j < N (ops/matmul.rs:295-299 layout,
 * batched columns matmul.rs:473-487, ACCUMULATE mul_mat_vec_head.slang:173-188). */
int sh_gemv_quant(sh_engine* e, const sh_qtensor* w, const float* x_dev, uint32_t N, float* y_dev,
                  int accumulate);
/* The reference's wide GEMM for N >= 32 columns (ops/matmul.rs:433-446,
 * mul_mm_cm.slang): y[j][m] (+)= sum_k f16(deq(W)[m][k]) * f16(x[j][k]) with
 * f32 accumulation, W Q4_K; the kernels the forward uses for calls of >= 32
 * columns (sh_model_wide_f16). Any N >= 1 (192 columns per pass). */
int sh_gemm_wide16(sh_engine* e, const sh_qtensor* w, const float* x_dev, uint32_t N, float* y_dev,
                   int accumulate);

/* Acceptance kernel for a batch of B sequences with k draft positions.
 * p_logits_dev [B][k+1][V], q_logits_dev [B][k][V] (REJECTION only, else NULL),
 * drafts_dev [B][k] u32. GREEDY / COMPARE follow sample_and_compare
 * (sample.rs:347-361, batched accept server/inference.rs:2859-2883);
 * REJECTION is new. Uniforms: Philox4x64-10 key (seed, 0x5EC), word
 * counter + 2*(b*(k+1)+i) (accept) and +1 (residual), or explicit host uniforms
 * [B][k+1][2]. Outputs acc_len_dev [B], next_tok_dev [B] (u32), enqueued on
 * the engine stream: ready after sh_engine_sync or any later synchronizing
 * call (with explicit uniforms the call itself waits, since the caller may
 * reuse that host array). The scratch (row partials, draw state) is the
 * engine's own, grown on the first call of a size and reused by later calls. */
int sh_accept_sample(sh_engine* e, const float* p_logits_dev, const float* q_logits_dev,
                     const uint32_t* drafts_dev, uint32_t B, uint32_t k, uint32_t V, const sh_sampling* s,
                     uint32_t* acc_len_dev, uint32_t* next_tok_dev);

/* No reference counterpart: sh_accept_sample for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Same arguments, kernels and results; it
 * calls no allocator and does not synchronize: the kernels are enqueued on the
 * engine's stream and acc_len_dev / next_tok_dev are ready after
 * sh_engine_sync (or any later synchronizing call). Its scratch is one static
 * 2 MiB device array per GPU, set up by sh_engine_create, so sizes whose
 * scratch exceeds it are refused with SH_ERR_CAPACITY (configs[1], B = 32,
 * k = 8, V = 128256, needs 170 KiB; up to B = 64, k = 16, V = 262144 fits).
 * Uniforms must come from Philox (s->uniforms NULL). The array is shared by
 * every call on that GPU and keeps the last call's contents; calls from other
 * streams or engines on that GPU are ordered through one per-device event
 * (each call's stream waits for the previous call's kernels), so they take the
 * array in turn. A caller capturing the call into a HIP graph must not replay
 * that graph concurrently with other no-alloc calls on the same GPU: replays
 * do not pass through that event. */
int sh_accept_sample_noalloc(sh_engine* e, const float* p_logits_dev, const float* q_logits_dev,
                             const uint32_t* drafts_dev, uint32_t B, uint32_t k, uint32_t V, const sh_sampling* s,
                             uint32_t* acc_len_dev, uint32_t* next_tok_dev);

/* New (no reference counterpart): the probabilities behind REJECTION's accept
 * tests, computed as sh_accept_sample computes them (f64 softmax of logits / T
 * over the same row statistics): probs_dev [B][k][3] = (p_i(d_i), q_i(d_i),
 * min(1, p_i(d_i) / q_i(d_i))) with the layouts of sh_accept_sample. */
int sh_accept_probs(sh_engine* e, const float* p_logits_dev, const float* q_logits_dev, const uint32_t* drafts_dev,
                    uint32_t B, uint32_t k, uint32_t V, float temperature, double* probs_dev);

/* New (no reference counterpart): tree acceptance for B token trees of n <= 64
 * nodes, recursive rejection sampling (SpecInfer multi-candidate speculative
 * sampling; one candidate per step reduces to sh_accept_sample's REJECTION).
 * Node 0 is the root (the last emitted token); parents_dev [B][n], parents[0]
 * = -1, parents[i] < i; tokens_dev [B][n]. p_logits_dev [B][n][V] are the
 * target logits after each node, q_logits_dev [B][n][V] the draft logits each
 * node's children were drawn from (leaf rows unused; NULL for GREEDY). From the
 * root, children are tried in index order: child c is accepted iff
 * u * q(tok_c) < cur(tok_c), cur = softmax(p/T) at the node and, after each
 * rejection, the normalised residual max(0, cur - q); with none accepted the
 * next token is drawn from cur, after an accepted leaf from the leaf's p.
 * GREEDY (or temperature 0) accepts the first child whose token is argmax p.
 * Uniforms: word counter + 2(b n + c) accepts child c, + 2(b n + v) + 1 draws at
 * node v (Philox key (seed, 0x5EC)), or explicit host uniforms [B][n][2].
 * Outputs (device): path_dev [B][n] accepted node indices, root first;
 * path_len_dev [B]; next_tok_dev [B]. Compact the path with sh_kv_compact. */
int sh_tree_accept(sh_engine* e, const float* p_logits_dev, const float* q_logits_dev, const uint32_t* tokens_dev,
                   const int32_t* parents_dev, uint32_t B, uint32_t n, uint32_t V, const sh_sampling* s,
                   uint32_t* path_dev, uint32_t* path_len_dev, uint32_t* next_tok_dev);

/* New (no reference counterpart): one tree verification step for B sequences
 * (configs[3]): sh_verify_unified over B trees of n nodes each (tokens, parents
 * [B][n] host; node 0 = the sequence's last emitted token, parents[0] = -1),
 * target logits kept on the device, sh_tree_accept against q_logits_dev
 * [B][n][V] (NULL for GREEDY), then sh_kv_compact of each accepted path
 * (node path[i] -> slot pos + i; position = pos + path_len). Outputs (host):
 * path_out [B][n], path_len_out [B], next_tok_out [B]. */
int sh_tree_verify_step(sh_engine* e, sh_model* target, sh_kv* const* caches, uint32_t B, uint32_t n,
                        const uint32_t* tokens, const int32_t* parents, const float* q_logits_dev,
                        const sh_sampling* s, uint32_t* path_out, uint32_t* path_len_out, uint32_t* next_tok_out);

#ifdef __cplusplus
}
#endif
#endif
