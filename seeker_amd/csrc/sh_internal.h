// Internal declarations shared by the HIP translation units of libseeker_hip.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <map>
#include <string>
#include <vector>

#include "../../include/seeker_hip.h"
#include "gguf.h"
#include "sh_error.h"

// Orderable argmax key: a larger float gives a larger key, ties the lower
// index. NaN and -inf give 0 and never win, so a row with no value above -inf
// yields index 0: the host rule (the first x[i] > best, best starting at -inf;
// inference/sample.rs:504-514). One definition for every argmax on the device
// (k_argmax, the greedy tree walk), so their semantics cannot drift apart.
__device__ __forceinline__ unsigned long long sh_amax_key(float v, uint32_t idx) {
  if (!(v > -__builtin_inff())) return 0ull;
  uint32_t b = __builtin_bit_cast(uint32_t, v);
  b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((unsigned long long)b << 32) | (unsigned long long)(~idx);
}
// The index a reduced key stands for (0 for the key 0 of a row without a value
// above -inf).
__device__ __forceinline__ uint32_t sh_amax_index(unsigned long long k) {
  return k == 0ull ? 0u : ~(uint32_t)(k & 0xFFFFFFFFull);
}

// ---------------------------------------------------------------- errors

#define SH_HIP(call)                                                              \
  do {                                                                            \
    hipError_t e_ = (call);                                                       \
    if (e_ != hipSuccess) {                                                       \
      sh_set_error("%s failed: %s (%s:%d)", #call, hipGetErrorString(e_), __FILE__, \
                   __LINE__);                                                     \
      return SH_ERR_HIP;                                                          \
    }                                                                             \
  } while (0)


// ------------------------------------------------------------ constants
// Activation operand ("B") layout for the MFMA GEMV: for each 8-column chunk,
// [K/32 blocks][64 lanes][8 f16]; lane = 16*g + c, g = (k%32)/8, c < 8 holds the
// high f16 part of column c, c >= 8 the low part (x - f32(hi)) of column c-8.
// XS (Q4_K minimum term): [K/256][16][8] f16, per 32-element sub-block sums
// of each column (hi in c, lo in c+8).
constexpr int SH_TILE_ROWS = 16;
constexpr int SH_Q4K_TILE_BYTES = 2304;  // 16 rows x 144 B, repacked
constexpr int SH_Q8_TILE_BYTES = 544;    // 16 rows x 34 B, repacked
constexpr int SH_Q5K_TILE_BYTES = 2816;  // 16 rows x 176 B, repacked
constexpr int SH_Q6K_TILE_BYTES = 3360;  // 16 rows x 210 B, repacked
// K-quants (256-element superblocks) that the multi-group GEMM decodes.
__host__ __device__ constexpr bool sh_is_kquant(int type) {
  return type == GGML_Q4_K || type == GGML_Q5_K || type == GGML_Q6_K;
}
constexpr uint32_t SH_MAX_COLS = 64;     // columns per forward chunk (8 operand groups of 8)
// argmax workspace (64-bit words): SH_MAX_COLS keys, then one arrival counter
// per column, 64 bytes apart
constexpr uint32_t SH_AMAX_WORDS = SH_MAX_COLS + 8 * SH_MAX_COLS;
constexpr uint32_t SH_MAX_PREP_COLS = 512;  // operand columns one prep builds (the MoE down operand: pairs)
constexpr int SH_FA_MIN_SPLIT_KEYS = 64;  // smallest key split of any attention launch (sizes fa_part)
constexpr uint32_t SH_WIDE16_COLS = 32;  // the reference's wide-GEMM threshold (ops/matmul.rs:433-446)
constexpr uint32_t SH_MAX_COLS16 = 192;  // columns per forward chunk of a wide f16 call (12 MFMA groups of 16)
constexpr int SH_FA_MAX_ROWS = 256;       // padded query rows (gqa x columns) per kv head
// Split partial row: O[hd], m, l, 2 pad (keeps rows 16-byte aligned).
__host__ __device__ constexpr uint32_t sh_fa_part_stride(uint32_t hd) { return hd + 4; }

// -------------------------------------------------------------- structs
struct KStat {
  uint64_t launches = 0;
  double ms = 0.0;
  double bytes = 0.0;
};

// Device buffers of the speculative step, owned by the engine (its captured
// graphs point into them).
struct SpecBufs {
  uint32_t* tok = nullptr;     // [64]: pending..., last, d_1..d_n; verify tokens at [32..]
  uint32_t* samp = nullptr;    // [16]: per-column ids; acc_len at [9], next token at [10]
  uint32_t* base = nullptr;    // [8] graph base positions (device): draft, target, verify; [4..7] = rng
  float* dlogits = nullptr;    // draft logits [8][V] of the last stochastic step
  float* tlogits = nullptr;    // target logits [9][V] of the last stochastic step
  float* udev = nullptr;       // [32] explicit uniforms of a stochastic step
  static constexpr size_t kRowstatBytes = 16384;  // scratch of the device draft draws (one row)
  double2* rowstat = nullptr;  // the device draft draws' scratch (sh_sample_rows_launch)
  uint64_t* rng = nullptr;     // = base + 4: Philox key and word base of a replayed stochastic step
  uint32_t* pinned = nullptr;  // host staging [128]; [64..71] go to base[0..7]
  uint32_t vcap = 0;
  uint32_t last_n = 0, last_V = 0;  // drafts and vocab of the last stochastic step (0: none)
};

// A captured HIP graph, keyed by its shape, models and caches; gen is the
// model/cache generation it was captured under (see graph replay in runtime.hip).
struct GraphEntry {
  uint64_t gen = 0;
  std::vector<uintptr_t> key;
  hipGraphExec_t exec = nullptr;
};

struct sh_engine {
  int device = 0;
  hipStream_t stream = nullptr;
  bool profiling = false;
  std::map<std::string, KStat> stats;
  struct Pending {
    std::string name;
    double bytes;
    hipEvent_t a, b;
  };
  std::vector<Pending> pending;
  std::vector<hipEvent_t> event_pool;
  SpecBufs spec;
  std::vector<GraphEntry> graphs;
  // Device scratch kept by the engine and reused by later calls (the engine
  // stream orders them): grown on demand by sh_engine_scratch.
  void* scr[4] = {nullptr, nullptr, nullptr, nullptr};
  size_t scr_bytes[4] = {0, 0, 0, 0};
  uint64_t graph_captures = 0, graph_launches = 0;  // replay counters (sh_engine_graph_stats)
};
// Scratch slots of sh_engine_scratch.
enum ScratchSlot { SCR_ACCEPT = 0, SCR_UNIFORMS = 1, SCR_TREE = 2, SCR_SMALL = 3 };
// *out = the engine's scratch of slot, at least `bytes` long. Growing it
// waits for the stream (earlier launches may still read the old block).
int sh_engine_scratch(sh_engine* e, int slot, size_t bytes, void** out);

// A weight matrix on the device, repacked into MFMA tiles.
struct QMat {
  int type = -1;
  uint32_t M = 0, K = 0;  // logical rows, contracting dim
  uint32_t tiles = 0;     // ceil(M / 16)
  uint8_t* d = nullptr;
  size_t bytes = 0;       // packed bytes
  double alg_bytes = 0;   // GGUF bytes of the logical matrix
};

struct sh_qtensor {
  sh_engine* e;
  QMat m;
};

struct Layer {
  float* attn_norm = nullptr;
  float* ffn_norm = nullptr;
  float* q_norm = nullptr;  // qwen3 / qwen3moe: per-head RMSNorm weights [hd]
  float* k_norm = nullptr;
  QMat wqkv;  // rows [q | k | v], or [q | k] when v is in another weight type
  QMat wv;    // v rows of their own (empty when they sit in wqkv)
  QMat wo;
  QMat wgu;   // tiles interleaved: gate tile t at 2t, up tile t at 2t+1
  QMat wdown;
  // qwen3moe routed experts: router f32 [E][d]; gate/up slabs of all experts
  // stacked (expert e's tiles interleaved like wgu, contiguous per expert),
  // down slabs stacked ([E][d] rows)
  float* router = nullptr;
  QMat wgu_exps;
  QMat wdown_exps;
};

struct QkvColDev;
struct Workspace {
  uint32_t max_cols = 0;
  float* resid = nullptr;     // [cols][d]
  float* resid2 = nullptr;    // [cols][d], the other half of the fused-prep residual ping-pong
  uint16_t* bx = nullptr;     // B operand buffer sized for max(K) x max_cols
  uint16_t* xs = nullptr;     // XS buffer
  float* q = nullptr;         // [cols][d] roped queries
  float* attn = nullptr;      // [cols][d]
  float* h = nullptr;         // [cols][ff] SwiGLU output
  float* logits = nullptr;    // [cols][V]
  float* fa_part = nullptr;   // flash-attn split partials
  float* gpart = nullptr;     // GEMV split-K partials
  uint32_t* tokens = nullptr; // [cols + 16] device token ids
  unsigned long long* amax = nullptr;  // SH_AMAX_WORDS: packed argmax keys, then per-column arrival counters (zeroed)
  float* cs = nullptr;        // [max(K)/256][8] inverse activation scales of the current B operand
  float* ssq = nullptr;       // [max(K)/256][8] per-superblock sums of squares of the normalized input
  uint16_t* bh = nullptr;     // [cols][max(K)] f16 operand rows of the wide f16 GEMM
  QkvColDev* qtab = nullptr;  // [cols] the chunk's QKV finish column table
  size_t fa_part_floats = 0;
  float* fab_part = nullptr;  // batched attention partials of every segment of a chunk (grown on demand)
  size_t fab_part_floats = 0;
  // cm1 attention (sh_fa16_launch, grown on demand): per 64-key block and row
  // the f16 P V accumulator, (M, l); per split the row maxima and a look-back
  // flag (zero between launches), then one error word
  uint16_t* fa16_pv = nullptr;
  float2* fa16_ml = nullptr;
  float* fa16_smax = nullptr;
  uint32_t* fa16_flag = nullptr;
  size_t fa16_pv_halves = 0, fa16_sync_words = 0;
  size_t gpart_floats = 0;
  // Second operand set, written by residual preps fused into the o / down GEMVs
  // (other workgroups of the producing kernel may still be staging the first):
  // sized for K = d, 8 columns.
  uint16_t* bx2 = nullptr;
  uint16_t* xs2 = nullptr;
  float* cs2 = nullptr;
  float* ssq2 = nullptr;
  uint32_t* sb_cnt = nullptr;  // [SH_SB_CNT x SH_SB_CNT_STRIDE] arrival counters of the fused residual prep (zero between launches)
  // routed-expert FFN (qwen3moe), P = columns x n_used pairs: router output,
  // routing plan, gate/up rows per sorted pair, down operand over the pairs
  // (P / 8 groups of K = expert_ff), down rows per sorted pair
  float* moe_logits = nullptr;   // [cols][n_expert] router logits
  uint32_t* moe_ids = nullptr;   // [cols][n_used]
  float* moe_wts = nullptr;      // [cols][n_used]
  uint32_t* moe_info = nullptr;  // chunk table (count, then (expert, first pair, n) per chunk)
  uint32_t* moe_col = nullptr;   // [P] input column of sorted pair s
  uint32_t* moe_slot = nullptr;  // [P] sorted position of pair (col, j)
  float* moe_hgu = nullptr;      // [P][2 expert_ff]
  uint16_t* moe_bx = nullptr;
  uint16_t* moe_xs = nullptr;
  float* moe_cs = nullptr;
  float* moe_y = nullptr;        // [P][d]
};

struct sh_model {
  sh_engine* e = nullptr;
  int arch = ARCH_LLAMA;
  uint32_t n_layer = 0, d = 0, n_head = 0, n_kv = 0, hd = 0, ff = 0, V = 0, n_ctx = 0;
  uint32_t q_dim = 0;  // n_head * hd (= d for llama)
  uint32_t n_expert = 0, n_used = 0, eff = 0;  // qwen3moe routed experts
  bool neox = false;   // NEOX RoPE + per-head Q/K RMSNorm (qwen3 / qwen3moe)
  float eps = 1e-5f, theta = 10000.f;
  int embd_type = -1;
  uint8_t* embd_raw = nullptr;  // token_embd in GGUF row layout (gather)
  size_t embd_row_bytes = 0;
  QMat lm_head;
  float* out_norm = nullptr;
  std::vector<Layer> layers;
  float2* rope = nullptr;       // [rope_max][hd/2] (cos, sin)
  uint32_t rope_max = 0;
  Workspace ws;
  double alg_weight_bytes = 0;  // bytes of every matrix a full-logits forward reads
  bool mg_ok = false;     // every matrix a K-quant: the multi-group path can run any chunk
  bool fused_ok = false;  // llama with uniform Q4_K / Q8_0 layers: chunks of <= 8 columns take the fused path
  // Forward calls of at least SH_WIDE16_COLS columns compute every dense matmul
  // as the reference's wide GEMM does (f16 weights and activations, f32
  // accumulation; sh_gemm16_launch): wide16_ok when the model allows it (no
  // routed experts, every matrix Q4_K), wide16 the switch (default on where
  // allowed), call16 set for the forward call in progress.
  bool wide16_ok = false;
  bool wide16 = false;
  bool call16 = false;
  // Causal single-sequence forward calls of more than one column compute
  // their attention with the reference's cooperative-matrix flash attention
  // arithmetic (sh_fa16_launch): fa16 the switch (default on; SH_FA_CM=0 at
  // upload turns it off), call_cm1 set for the forward call in progress.
  bool fa16 = true;
  bool call_cm1 = false;
};

struct sh_kv {
  sh_engine* e = nullptr;
  uint32_t n_layer = 0, n_kv = 0, hd = 0, max_seq = 0, pos = 0;
  uint16_t* k = nullptr;  // [layer][n_kv][max_seq][hd] f16
  uint16_t* v = nullptr;  // [layer][n_kv][max_seq/32][hd][32] f16, slot-permuted
  std::vector<uint32_t> pending;  // committed tokens not yet in this cache
  // Set only while a graph is being captured: forward positions in this cache
  // are offsets from the device value *graph_base (read by the kernels at
  // replay), and the host neither checks nor advances the position.
  const uint32_t* graph_base = nullptr;
};

// ------------------------------------------------------------ launchers
// All launchers enqueue on e->stream and return 0 or an SH_ERR code.
int sh_repack_upload(sh_engine* e, int type, const uint8_t* host, uint32_t M, uint32_t K, QMat* out);
int sh_repack_upload_gu(sh_engine* e, int type, const uint8_t* gate, const uint8_t* up, uint32_t M,
                        uint32_t K, QMat* out);
int sh_repack_upload_cat(sh_engine* e, int type, const uint8_t* const* parts, const uint32_t* rows,
                         int nparts, uint32_t K, QMat* out);
void sh_qmat_free(QMat* m);

// GEMV epilogues. EPI_PART writes split-K partial sums in packed row order,
// out[ks * part_stride + col * ldo + row], finished by the consumer (the next
// prep kernel or sh_part_reduce_launch).
enum EpiKind { EPI_STORE = 0, EPI_ADD = 1, EPI_QKV = 2, EPI_SWIGLU = 3, EPI_PART = 4 };
struct EpiArgs {
  float* out = nullptr;   // STORE/ADD: [N][ldo]; QKV: roped q [N][Dq]; SWIGLU: h [N][ldo]; PART: partials
  uint32_t ldo = 0;
  uint32_t rows = 0xFFFFFFFFu;  // STORE/ADD: logical rows M (ragged last tile)
  const float* cs = nullptr;    // [K/256][8] inverse activation scale per superblock and column
  size_t part_stride = 0;       // PART: floats between splits
  uint32_t part_cap = 0;        // PART: splits the buffer holds
  // RMSNorm of the input, applied to the outputs: y *= rsqrt(sum_i ssq[i][col] / norm_K + eps)
  // over the prep's per-superblock sums of squares ssq [ssq_n][8] (null: no norm).
  const float* ssq = nullptr;
  uint32_t ssq_n = 0, norm_K = 0;
  float eps = 0.f;
  // QKV: column c is roped at colpos[c] and its K/V row goes to slot slot[c] of
  // the cache (kc[c], vc[c], capacity mseq[c]); columns may belong to different
  // sequences' caches.
  uint32_t Dq = 0, Dkv = 0, hd = 0, n_kv = 0, layer = 0;
  const float2* rope = nullptr;
  int32_t colpos[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  uint32_t slot[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  uint32_t mseq[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  uint16_t* kc[8] = {nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
  uint16_t* vc[8] = {nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
  // Graph replay: colpos and slot are offsets from the device value *dbase.
  const uint32_t* dbase = nullptr;
};
// Where a split-K GEMV takes its activation operand from: the staged operand
// (B/XS/cs, the default), f32 rows x [N][ldx] (the operand is built in LDS, as
// the prep would build it, without a norm), or attention split partials (the
// split combine is done in LDS, as k_fa_combine would do it).
enum OpndKind { OPND_STAGED = 0, OPND_ROWS = 1, OPND_FA = 2, OPND_RESID = 3 };
struct OpndSrc {
  int kind = OPND_STAGED;
  const float* x = nullptr;  // OPND_ROWS; OPND_RESID: residual in [N][K]
  uint32_t ldx = 0;
  // OPND_RESID (whole-K kernel, N <= 2): every workgroup builds the whole
  // operand of rmsnorm(x + sum of split partials) * norm_w in LDS, workgroup 0
  // writes x + partials to rout (another buffer: the others still read x).
  float* rout = nullptr;
  const float* part = nullptr;
  uint32_t nparts = 0, part_ld = 0;
  const float* norm_w = nullptr;
  float eps = 0.f;
  const float* fa_part = nullptr;  // OPND_FA: partial layout of sh_fa_launch
  uint32_t n_layout = 0, rows_pad = 0, n_head = 0, gqa = 0, hd = 0, split_keys = 0, kv_off = 0;
  const uint32_t* dbase = nullptr;  // graph replay: live splits from *dbase + kv_off
};
// Residual prep fused into a split-K GEMV (EPI_PART, 256-row output
// superblocks): the last workgroup to finish output superblock j (arrival
// counter cnt[j]) adds the split partials of its rows to resid in split order,
// writes resid, the per-superblock sums of squares and the operand of
// resid * norm_w for the next GEMV (bx, xs, cs), as the PREP_RESID prep kernel
// does, bit for bit. The partials travel through agent-coherent stores and
// loads. The last arriver resets cnt[j] to zero.
constexpr uint32_t SH_SB_CNT = 256;
constexpr uint32_t SH_SB_CNT_STRIDE = 64;  // counters 256 bytes apart: no two share a cache line
struct PrepFuse {
  float* resid = nullptr;  // [N][K]
  const float* norm_w = nullptr;
  uint16_t* bx = nullptr;
  uint16_t* xs = nullptr;
  float* cs = nullptr;
  float* ssq = nullptr;
  uint32_t* cnt = nullptr;
  uint32_t K = 0;          // rows of the producing GEMV = elements of the residual
};
// Launch y = W x for N <= 8 columns; with EPI_PART, *nparts receives the
// number of split partials written (1 for the other epilogues). A non-staged
// src needs the split-K kernel (sh_gemv_fusable).
int sh_gemv_launch(sh_engine* e, const QMat& w, const uint16_t* bx, const uint16_t* xs, uint32_t N,
                   EpiKind epi, const EpiArgs& ea, const char* tag, uint32_t* nparts = nullptr,
                   const OpndSrc* src = nullptr, const PrepFuse* pf = nullptr);
// Whether an EPI_PART launch of w can carry a PrepFuse (split-K kernel, staged
// operand, whole 256-row output superblocks per workgroup row group).
bool sh_gemv_prep_fusable(const QMat& w);
// Superblocks per split when the EPI_PART launch of w takes the split-K kernel
// (which accepts OPND_ROWS / OPND_FA), else 0.
uint32_t sh_gemv_fusable(const QMat& w);
// Whether w's whole-K launches (QKV, SwiGLU) accept OPND_RESID for N columns.
bool sh_gemv_resid_fusable(const QMat& w, uint32_t N);
// Floats of partial-sum buffer the EPI_PART launches of w need (all splits).
size_t sh_gemv_part_floats(const QMat& w);
// Tiles per workgroup of the deep-ring whole-K kernel for w, or 0 when w does
// not take it (Q4_K with enough row tiles to fill the chip; SH_RING=0 turns it
// off). sh_gemv_ring_launch: y = W x through that kernel, EPI_STORE or
// EPI_PART (one split, whole sums). With swiglu (EPI_PART of the packed
// gate / up matrix), the last workgroup of each 256-element superblock of h
// also builds the down GEMV's operand of silu(gate) * up there (swiglu->bx,
// xs, cs, cnt; K = the FFN width), as the PREP_SWIGLU prep kernel does.
uint32_t sh_gemv_ring_t(const QMat& w);
int sh_gemv_ring_launch(sh_engine* e, const QMat& w, const uint16_t* bx, const uint16_t* xs, uint32_t N,
                        EpiKind epi, const EpiArgs& ea, const char* tag, const PrepFuse* swiglu = nullptr);
// y = W x for N <= SH_MAX_COLS columns (operand groups of 8, Q4_K) in one pass
// over W: EPI_PART (partials [split][8 ceil(N/8)][ldo]; *nparts = splits) or
// EPI_STORE. The operand of group g starts at g times one group's size.
int sh_gemm_launch(sh_engine* e, const QMat& w, const uint16_t* bx, const uint16_t* xs, const float* cs, uint32_t N,
                   EpiKind epi, const EpiArgs& ea, const char* tag, uint32_t* nparts = nullptr);
size_t sh_gemm_part_floats(const QMat& w);  // for SH_MAX_COLS columns
// y = W x with the reference's wide-GEMM arithmetic (f16 weights and
// activations, f32 accumulation) for N <= SH_MAX_COLS16 columns of f16 rows
// bh[col * ldb + k] (k_prep16_*), W Q4_K, Q5_K, Q6_K or Q8_0: EPI_PART
// (partials as sh_gemm_launch's; *nparts = splits) or EPI_STORE (out[col][row]).
int sh_gemm16_launch(sh_engine* e, const QMat& w, const uint16_t* bh, uint32_t ldb, uint32_t N, EpiKind epi,
                     const EpiArgs& ea, const char* tag, uint32_t* nparts = nullptr);
// Partial floats sh_gemm16_launch's EPI_PART needs for up to SH_MAX_COLS16 columns.
size_t sh_gemm16_part_floats(const QMat& w);
// The same arithmetic for Q8_0, Q5_K and Q6_K weights (gemm16x.hip), which
// sh_gemm16_launch hands these types to: whether w takes it, its partial
// floats, the launch.
bool sh_gemm16x_ok(const QMat& w);
size_t sh_gemm16x_part_floats(const QMat& w);
int sh_gemm16x_launch(sh_engine* e, const QMat& w, const uint16_t* bh, uint32_t ldb, uint32_t N, EpiKind epi,
                      const EpiArgs& ea, const char* tag, uint32_t* nparts);
// Fused QKV rows from sh_gemm_launch partials: RoPE, q out, K/V into each
// column's cache slot.
struct QkvColDev {  // one column of a device-resident column table
  int32_t pos;
  uint32_t slot, mseq, pad;
  uint16_t* kc;
  uint16_t* vc;
};
struct QkvCols {  // per column: RoPE position, cache slot, capacity, K and V caches
  // With tab set, the columns come from that device table (up to
  // SH_MAX_COLS16 of them) and the arrays below are unused.
  const QkvColDev* tab = nullptr;
  int32_t pos[SH_MAX_COLS];
  uint32_t slot[SH_MAX_COLS];
  uint32_t mseq[SH_MAX_COLS];
  uint16_t* kc[SH_MAX_COLS];
  uint16_t* vc[SH_MAX_COLS];
  // V rows from a matrix of their own (attn_v in another weight type than
  // attn_q / attn_k): its split partials [split][col][row], row 0 = first v row
  const float* vpart = nullptr;
  uint32_t vnparts = 0, vldp = 0;
  size_t vstride = 0;
  // first row to finish (multiple of 4): Dq + Dkv finishes the V rows only
  // (k_qkv_finish; q and k rows came from elsewhere)
  uint32_t row0 = 0;
};
int sh_qkv_finish_launch(sh_engine* e, const float* part, uint32_t nparts, size_t part_stride, uint32_t ldp,
                         uint32_t N, const EpiArgs& ea, const QkvCols& qc);
// The same from partials for qwen3-style attention: per-head RMSNorm of q and
// k (weights q_norm / k_norm [hd], null: none) and NEOX or NORM RoPE.
int sh_qkv_finish_head_launch(sh_engine* e, const float* part, uint32_t nparts, size_t part_stride, uint32_t ldp,
                              uint32_t N, const EpiArgs& ea, const QkvCols& qc, const float* q_norm,
                              const float* k_norm, float eps, bool neox);
// Expert-indirect y = W_e x for routed MoE FFNs: w stacks n_expert slabs
// (rows M / n_expert each); chunk table info = (n_chunks, then (expert, p0, n)
// per chunk), pair p's operand column gcol[p] (null: p), outputs
// ea.out[p][row] for rows < ea.rows (EPI_STORE). One launch covers max_chunks.
int sh_moe_gemm_launch(sh_engine* e, const QMat& w, uint32_t n_expert, const uint16_t* bx, const uint16_t* xs,
                       const float* cs, uint32_t max_chunks, const uint32_t* info, const uint32_t* gcol,
                       const EpiArgs& ea, const char* tag, double alg_bytes);

// Activation prep: finishes the previous GEMV (residual add of its split
// partials, or SwiGLU of gate/up partials) and builds the next activation
// operand B + XS + cs (N <= 8), one wave per (superblock, column). RMSNorm is
// split: the prep multiplies by the norm weight and writes per-superblock sums
// of squares; the consuming GEMV applies rsqrt(mean + eps) to its outputs
// (EpiArgs::ssq). Each 256-element superblock of a column is scaled by a power
// of two s so its max|y*s| lies in [2^9, 2^10): the f16 low halves then stay
// normal (an f16 subnormal keeps only 2^-24 of absolute resolution) and the
// 32-element XS sums stay below 2^15.
enum PrepMode { PREP_PLAIN = 0, PREP_RESID = 1, PREP_SWIGLU = 2, PREP_MOE_COMBINE = 3 };
struct PrepArgs {
  int mode = PREP_PLAIN;
  float* ssq = nullptr;         // with norm_w: per-superblock sums of squares [K/256][8] out
  float* x = nullptr;           // PLAIN/RESID: [N][K] input; RESID writes x + partials back
  const float* part = nullptr;  // partials [nparts][part_cols][part_ld]
  uint32_t nparts = 0, part_ld = 0, part_cols = 8;
  uint32_t K = 0, N = 0;
  const float* norm_w = nullptr;
  float eps = 0.f;
  uint16_t* bx = nullptr;
  uint16_t* xs = nullptr;
  float* cs = nullptr;
  // With bh: the operand of the wide f16 GEMM instead, bh[col * ldb + k] =
  // f16(y) with the RMS norm applied (y = (v * rsqrt(mean v^2 + eps)) * w),
  // as the reference's wide GEMM stages its input; ssq, bx, xs, cs unused.
  uint16_t* bh = nullptr;
  uint32_t ldb = 0;
  // PREP_MOE_COMBINE (with bh only): x += sum_j wts[col k + j] y[slot_of[col k
  // + j]] first (the routed experts' weighted sum, k_moe_combine's
  // arithmetic), then the operand as PREP_RESID without partials.
  const float* moe_y = nullptr;
  const uint32_t* moe_slot = nullptr;
  const float* moe_wts = nullptr;
  uint32_t moe_k = 0;
};
// N <= SH_MAX_PREP_COLS; the operand buffers hold ceil(N / 8) groups.
int sh_prep_launch(sh_engine* e, const PrepArgs& a);
// y[col][m] (+)= sum of nparts split partials, m < M.
int sh_part_reduce_launch(sh_engine* e, const float* part, uint32_t nparts, uint32_t part_ld, uint32_t part_cols,
                          uint32_t M, uint32_t N, float* y, uint32_t ldy, bool accumulate);
int sh_embed_launch(sh_engine* e, const sh_model* m, const uint32_t* tokens, uint32_t N, float* resid);
struct FaArgs {
  uint32_t layer = 0, N = 0;
  uint32_t col0 = 0;       // first column of the chunk (q, attn and operand column offset)
  uint32_t kvlen = 0;      // keys [0, kvlen) exist
  uint32_t mask_base = 0;  // keys >= mask_base need their bit in colmask
  uint64_t colmask[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  const uint64_t* masks = nullptr;  // device masks per column (N up to SH_MAX_COLS); null: colmask (N <= 8)
  // Graph replay: kvlen and mask_base are offsets from the device value *dbase,
  // the split grid covers kv_cap keys and splits past the live keys exit.
  const uint32_t* dbase = nullptr;
  uint32_t kv_cap = 0;
};
// Attention for the chunk's columns, then the split combine, which writes
// attn_out [N][n_embd] f32 and the Wo activation operand (bx, xs, per-superblock cs).
int sh_fa_launch(sh_engine* e, const sh_model* m, const sh_kv* kv, const FaArgs& fa, const float* q, float* part,
                 float* attn_out, uint16_t* bx, uint16_t* xs, float* cs, OpndSrc* combine_out = nullptr);
// With combine_out, the combine kernel is skipped and *combine_out describes
// the partials for a consumer that combines them itself (OPND_FA).

// Attention of a single-sequence causal chunk (columns [col0, col0 + N) of the
// forward chunk, keys [0, kvlen), chunk keys from mask_base) with the
// reference's cooperative-matrix flash attention arithmetic (attn16.hip):
// writes attn_out [N][n_head * hd] and the Wo operand (hi/lo groups bx, xs,
// cs, or with bh the f16 rows of the wide f16 GEMM). Graph replay as
// sh_fa_launch (fa.dbase, fa.kv_cap).
struct Fa16Args {
  const float* q = nullptr;  // roped queries of the call's first column [N][n_head * hd]
  const uint16_t* kc = nullptr;
  const uint16_t* vc = nullptr;
  uint32_t max_seq = 0, n_head = 0, n_kv = 0, gqa = 0, ncol = 0, col0 = 0, kvlen = 0, mask_base = 0;
  const uint32_t* dbase = nullptr;
  uint32_t n_rg = 0, nbmax = 0, max_splits = 0;
  float qs = 0.f;  // f32(f32(1 / sqrt(hd)) * f32(log2 e))
  uint16_t* pv = nullptr;
  float2* ml = nullptr;
  float* smax = nullptr;   // look-back words [n_kv][n_rg][max_splits][32], unset between launches
  uint32_t* err = nullptr;  // set when a look-back wait gave up
};
int sh_fa16_launch(sh_engine* e, const sh_model* m, const sh_kv* kv, const FaArgs& fa, const float* q,
                   float* attn_out, uint16_t* bx, uint16_t* xs, float* cs, uint16_t* bh = nullptr);
// Buffer sizes sh_fa16_launch needs for N columns over keys [0, kv_cap).
size_t sh_fa16_pv_halves(uint32_t n_kv, uint32_t hd, uint32_t gqa, uint32_t ncol, uint32_t kv_cap);
size_t sh_fa16_sync_words(uint32_t n_kv, uint32_t gqa, uint32_t ncol, uint32_t kv_cap);

// Batched attention (attn_batch.hip): every segment of a forward chunk in one
// launch per layer, then one combine launch. A segment is a run of one
// sequence's columns with its own cache, key count and per-column masks.
struct FabSegIn {
  const sh_kv* kv = nullptr;
  uint32_t col0 = 0, ncol = 0;    // chunk columns [col0, col0 + ncol)
  uint32_t kvlen = 0;             // keys [0, kvlen) exist
  uint32_t mask_base = 0;         // keys >= mask_base need their bit in the column mask
  const uint64_t* hmasks = nullptr;  // host: ncol masks (bit i: key mask_base + i)
};
struct FabSeg {  // device descriptor of a segment
  const uint16_t* k;
  const uint16_t* v;
  const uint64_t* masks;  // ncol masks (device)
  uint64_t part_off;      // floats into the partial buffer: [n_kv][nsplit * kp][rows_pad][hd + 4]
  uint32_t max_seq, kvlen, mask_base, col0, ncol, rows_pad, nsplit;
};
struct FabLaunch {
  uint8_t* dev = nullptr;  // device tables (segments, work items, column -> segment, masks)
  const FabSeg* segs = nullptr;
  const uint32_t* work = nullptr;    // (segment << 16 | key split) per workgroup
  const uint32_t* colseg = nullptr;  // segment of each chunk column
  float* part = nullptr;
  uint32_t nseg = 0, nwork = 0, nc = 0, tps = 0, rgw = 1, kp = 1;
  uint32_t max_nsv = 0;  // most partials (key splits x kp) of one segment
};
int sh_fab_plan(sh_engine* e, sh_model* m, const FabSegIn* in, uint32_t nseg, uint32_t nc, FabLaunch* out);
int sh_fab_launch(sh_engine* e, const sh_model* m, const FabLaunch& fl, uint32_t layer, const float* q, float* attn_out,
                  uint16_t* bx, uint16_t* xs, float* cs, uint16_t* bh = nullptr);
void sh_fab_free(sh_engine* e, FabLaunch& fl);
int sh_argmax_launch(sh_engine* e, const float* logits, uint32_t V, uint32_t N, unsigned long long* keys,
                     uint32_t* out_ids);
// Draws one token per row from softmax(logits / T) by the vocab-order inverse
// CDF (the COMPARE column sampler): row r uses uniform word word0 + wstride * r
// (explicit u_dev[word] or Philox key (seed, 0x5EC)). part: nrows * ceil(V /
// 8192) row-statistics partials of scratch. rng_dev (graph replay): the key
// and a word base added to word0 are read from the device words rng_dev[0..1].
int sh_sample_rows_launch(sh_engine* e, const float* logits, uint32_t nrows, uint32_t V, float T, const float* u_dev,
                          uint64_t seed, uint64_t word0, uint64_t wstride, void* scratch, size_t scratch_bytes,
                          uint32_t* out, const uint64_t* rng_dev = nullptr);
// Device scratch sh_sample_rows_launch needs: row-statistics partials and, for
// rows of many logits, the chunked draw's sums and counters.
size_t sh_sample_rows_scratch_bytes(uint32_t nrows, uint32_t V);
// Per-row parameters of the batched verify's column sampling.
struct SampRow {
  double inv_t;       // 1 / temperature
  uint64_t seed;      // Philox key word 0
  uint64_t word;      // Philox word (uniform index)
  float u;            // explicit uniform (explicit_u)
  uint32_t greedy;    // keep the argmax already in out[row]
  uint32_t explicit_u;
  uint32_t top_k;     // > 0: the filtered chain (sh_sample_filters)
  float top_p, log_min_p, inv_t_f;
  uint32_t filt_flags;
  uint32_t pad;
};
// The candidate filters of s for vocabulary V into r (top_k, top_p,
// log_min_p, inv_t_f, filt_flags; top_k 0 = none); SH_ERR_UNSUPPORTED for
// combinations the GPU chain does not take.
int sh_samprow_filters(const sh_sampling& s, uint32_t V, SampRow& r);
// Draws row r of logits [nrows][V] by rows_dev[r] (greedy rows untouched):
// the temperature-only rows when plain, the filtered rows (top_k > 0) when
// filtered; part: sh_sample_rows_part_bytes(nrows, V) of scratch.
int sh_sample_rows_tab_launch(sh_engine* e, const float* logits, uint32_t nrows, uint32_t V, const SampRow* rows_dev,
                              double2* part, uint32_t* out, bool plain, bool filtered);
size_t sh_sample_rows_part_bytes(uint32_t nrows, uint32_t V);
// Routed-expert FFN pieces (moe.hip): router logits [N][E] of the RMS-normed
// columns, top-k per column (ids, wts [N][k]) with the routing plan over
// P = N k pairs, the weighted sum into resid.
uint32_t sh_moe_max_chunks(uint32_t P, uint32_t E);
int sh_moe_route_launch(sh_engine* e, const float* x, const float* norm_w, const float* router, uint32_t d, uint32_t E,
                        float eps, uint32_t N, float* logits);
int sh_moe_plan_launch(sh_engine* e, const float* logits, uint32_t N, uint32_t E, uint32_t k, uint32_t* ids,
                       float* wts, uint32_t* info, uint32_t* pair_col, uint32_t* slot_of);
int sh_moe_combine_launch(sh_engine* e, const float* y, const uint32_t* slot_of, const float* wts, uint32_t k,
                          uint32_t d, uint32_t N, float* resid);
// Acceptance of B sequences (COMPARE / REJECTION), see sh_accept_sample;
// uniforms_dev (explicit) or Philox words from counter. scratch: device
// memory of sh_accept_scratch_bytes(B, k, V, mode) bytes, or null to allocate
// it on the stream.
size_t sh_accept_scratch_bytes(uint32_t B, uint32_t k, uint32_t V, uint32_t mode);
// Takes the per-device address of sh_accept_sample_noalloc's static scratch
// (once per device; call with that device current).
int sh_static_scratch_init(int dev);
int sh_accept_launch(sh_engine* e, const float* p_logits, const float* q_logits, const uint32_t* drafts, uint32_t B,
                     uint32_t k, uint32_t V, const sh_sampling* s, uint64_t counter, const float* uniforms_dev,
                     uint32_t* acc_len, uint32_t* next_tok, void* scratch = nullptr, double* probs_out = nullptr,
                     const uint64_t* rng_dev = nullptr);
int sh_kv_compact_launch(sh_engine* e, sh_kv* kv, uint32_t base, const uint32_t* src_dev, uint32_t n);

// Profiling helpers (no-ops unless e->profiling).
void sh_prof_begin(sh_engine* e, hipEvent_t* a);
void sh_prof_end(sh_engine* e, const char* name, double bytes, hipEvent_t a);
int sh_prof_flush(sh_engine* e);
