// Masked attention of single-sequence forward calls of more than one column,
// with the reference's cooperative-matrix flash attention arithmetic.
//
// The reference sends every forward of L > 1 tokens over an f16 cache to
// flash_attn_cm1.slang (ops/flash_attn.rs:442-471), single pass up to 16384
// keys (:1393-1410). Per query row: q staged as f16(q * (scale * log2 e))
// (:155-171); keys in 64-key blocks from key 0 (Bc, :39); per block the row
// maximum M of its visible scores (running, from -1e30), the f16 output
// rescaled by f16(exp2(M_old - M)) (:314-320), P = exp2(S - M) rounded to f16
// (:322-334), P V summed per 16-key chunk into an f16 accumulator (the
// f16-accumulating MMA, :349-358) and added to the f16 output (:363-374);
// O = f32(O16) / L at the end (:398-411).
//
// The f16 output is a sequential chain over the blocks (each step rounds), so
// the work splits in two kernels:
//   k_fa16:       everything that does not depend on the chain, in parallel
//                 over (key split of kW blocks, group of 32 query rows, kv
//                 head): per block S (one v_mfma_f32_16x16x32_f16 per 32 of
//                 head_dim: K and the staged q are f16 already), the block
//                 maxima, the running maximum M_j of every block (the maxima
//                 of earlier splits arrive by a look-back over per-split
//                 words), P16, l_j = sum P and the block's f16 P V accumulator
//                 (v_mfma_f32_16x16x16_f16 per 16-key chunk, rounded to f16
//                 after each chunk); writes PV16_j, M_j and l_j per row.
//   k_fa16_chain: one workgroup per (column, 256 outputs): the rows' PV16_j
//                 and (M_j, l_j) staged in LDS with all loads in flight, then
//                 one output per thread: the chain O16 <- f16(f16(e_j) O16) +
//                 PV16_j (f16 multiply and add, each rounded once) and L <-
//                 e_j L + l_j over the row's blocks, then O = f32(O16) / L as
//                 the attention row and the Wo operand; it also resets the
//                 look-back words for the next launch.
//
// Look-back: the workgroup of split s publishes its 32 row maxima with
// agent-coherent stores (sh_coherent.h) into words that hold kUnset until
// then (the data is its own flag: a maximum is never that NaN pattern), and
// polls the words of splits 0 .. s-1 of its (row group, kv head) only. The
// split is the fastest grid index, so those workgroups were dispatched before
// it (workgroups are dispatched in order of their linear index) and none of
// them waits on it: every wait ends. A spin bound keeps even a broken dispatch
// order from hanging the GPU (the maxima then come out wrong, not stuck).
#include <cstdlib>

#include "sh_internal.h"
#include "sh_coherent.h"
#include "sh_operand.h"

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
struct alignas(16) u32x4a { uint32_t x, y, z, w; };

constexpr float kNegBig = -1.0e30f;  // the shader's running-maximum start (NEG_BIG)
constexpr int kW = 4;                // waves (64-key blocks) per split
constexpr int kNG = 2 * kW;          // groups of 32 threads (look-back rows)
constexpr uint32_t kSpinMax = 1u << 20;
constexpr uint32_t kUnset = 0xFFFFFFFFu;  // a look-back word not yet published (a NaN: never a maximum)

__device__ __forceinline__ h8 ld_h8(const uint16_t* p) { return __builtin_bit_cast(h8, *(const u32x4a*)p); }

// Whether key `key` is visible to chunk column `col`: the cached prefix below
// mbase always, the chunk's own keys causally (models/llama.rs:904-955).
// (bitwise, not short-circuit: no branches around the selects that use it)
__device__ __forceinline__ bool fa16_visible(uint32_t key, uint32_t kvlen, uint32_t mbase, uint32_t col) {
  return (key < kvlen) & ((key < mbase) | (key - mbase <= col));
}

template <int HD>
__global__ __launch_bounds__(64 * kW) void k_fa16(Fa16Args a) {
  constexpr int NC = HD / 32, DT = HD / 16;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4, r = lane & 15;
  const uint32_t split = blockIdx.x, rg = blockIdx.y, kh = blockIdx.z;
  const uint32_t kb0 = a.dbase ? *a.dbase : 0u;  // graph replay: positions from the device base
  const uint32_t kvlen = a.kvlen + kb0, mbase = a.mask_base + kb0;
  const uint32_t R = a.gqa * a.ncol, rho0 = 32 * rg;
  // blocks of this row group: up to its last column's last visible key
  const uint32_t cmax = min(a.ncol - 1, (rho0 + 31) / a.gqa);
  const uint32_t nb = (min(mbase + cmax, kvlen - 1)) / 64 + 1;
  const uint32_t nsplit = (nb + kW - 1) / kW;
  if (split >= nsplit) return;  // whole workgroup: no later split waits on it
  const uint32_t blk = split * kW + wave;
  const bool live = blk < nb;  // wave-uniform
  const uint32_t k0 = blk * 64;
  const uint32_t Dq = a.n_head * HD;

  // every load first, all in flight before any use: the queries of the two
  // 16-row tiles (first: loads complete in order, so their staging waits for
  // them only), then K and V of the block (clamped rows stay in bounds and are
  // masked)
  f4 qraw[2][NC][2];
  uint32_t col[2];
  bool rok[2];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const uint32_t rho = rho0 + 16 * rt + r;
    rok[rt] = rho < R;
    const uint32_t rr = rok[rt] ? rho : 0u;
    col[rt] = rr / a.gqa;
    const float* qp = a.q + (size_t)col[rt] * Dq + (size_t)(kh * a.gqa + rr % a.gqa) * HD + 8 * g;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      qraw[rt][c][0] = *(const f4*)(qp + 32 * c);
      qraw[rt][c][1] = *(const f4*)(qp + 32 * c + 4);
    }
  }
  asm volatile("" ::: "memory");  // the K / V loads stay behind the query loads
  const uint16_t* kbase = a.kc + (size_t)kh * a.max_seq * HD;
  const uint16_t* vbase = a.vc + (size_t)kh * (a.max_seq / 32) * HD * 32;
  h8 kop[4][NC], vop[2][DT];
#pragma unroll
  for (int kt = 0; kt < 4; ++kt) {
    const uint32_t key = min(k0 + 16 * kt + r, a.max_seq - 1);
#pragma unroll
    for (int c = 0; c < NC; ++c) kop[kt][c] = ld_h8(kbase + (size_t)key * HD + 32 * c + 8 * g);
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t vb = min(k0 / 32 + h, a.max_seq / 32 - 1);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) vop[h][dt] = ld_h8(vbase + ((size_t)vb * HD + 16 * dt + r) * 32 + 8 * g);
  }
  asm volatile("" ::: "memory");  // ... and are all issued before the first use:
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)  // the staging below cannot move above this point
#pragma unroll
    for (int c = 0; c < NC; ++c) asm volatile("" : "+v"(qraw[rt][c][0]), "+v"(qraw[rt][c][1]));
  // staged queries: f16(q * qs), the f32 product rounded once more to f16
  h8 qop[2][NC];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const float x[8] = {qraw[rt][c][0][0], qraw[rt][c][0][1], qraw[rt][c][0][2], qraw[rt][c][0][3],
                          qraw[rt][c][1][0], qraw[rt][c][1][1], qraw[rt][c][1][2], qraw[rt][c][1][3]};
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        float y = x[t] * a.qs;
        asm volatile("" : "+v"(y));  // the f32 product, not a fused multiply-convert
        qop[rt][c][t] = (_Float16)y;
      }
    }

  // S^T[key][row] per 16-key tile kt and 16-row tile rt: lane (g, r) holds
  // keys 16 kt + 4 g + t of row 16 rt + r
  f4 s[4][2];
#pragma unroll
  for (int kt = 0; kt < 4; ++kt)
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NC; ++c) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop[kt][c], qop[rt][c], acc, 0, 0, 0);
      s[kt][rt] = acc;
    }
  // visibility (masked scores are -inf, by selects into plain registers) and
  // the block maxima
  float sv[2][16];
  float bmx[2];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    float m = kNegBig;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const uint32_t key = k0 + 16 * kt + 4 * g + t;
        const bool vis = live & rok[rt] & fa16_visible(key, kvlen, mbase, col[rt]);
        const float v = vis ? s[kt][rt][t] : -INFINITY;
        sv[rt][4 * kt + t] = v;
        m = fmaxf(m, v);
      }
    m = fmaxf(m, __shfl_xor(m, 16));
    m = fmaxf(m, __shfl_xor(m, 32));
    bmx[rt] = m;
  }
  __shared__ float sbm[kW][32];
  __shared__ float sred[kNG][32];
  __shared__ float sinc[32];
  if (g == 0) {
    sbm[wave][r] = bmx[0];
    sbm[wave][16 + r] = bmx[1];
  }
  __syncthreads();
  // publish the split's row maxima
  const size_t sync0 = ((size_t)kh * a.n_rg + rg) * a.max_splits;
  if (wave == 0 && lane < 32) {
    float m = sbm[0][lane];
#pragma unroll
    for (int w = 1; w < kW; ++w) m = fmaxf(m, sbm[w][lane]);
    sh_st_coh4(a.smax + (sync0 + split) * 32 + lane, __builtin_bit_cast(uint32_t, m));
  }
  // look-back: the maxima of every earlier split, each word polled until set
  {
    const uint32_t row = threadIdx.x & 31, jj = threadIdx.x >> 5;  // group jj: splits jj mod kNG
    float m = kNegBig;
    for (uint32_t j0 = jj; j0 < split; j0 += kNG * 8) {
      uint32_t v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const uint32_t j = j0 + kNG * u;
        v[u] = j < split ? sh_ld_coh4(a.smax + (sync0 + j) * 32 + row) : __builtin_bit_cast(uint32_t, kNegBig);
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) sh_coh_wait(v[u]);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        uint32_t spins = 0;
        while (v[u] == kUnset) {  // only words of earlier splits start unset
          if (++spins > kSpinMax) {
            __hip_atomic_store(a.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            v[u] = __builtin_bit_cast(uint32_t, kNegBig);
            break;
          }
          __builtin_amdgcn_s_sleep(1);
          v[u] = sh_ld_coh4(a.smax + (sync0 + j0 + kNG * u) * 32 + row);
          sh_coh_wait(v[u]);
        }
        m = fmaxf(m, __builtin_bit_cast(float, v[u]));
      }
    }
    sred[jj][row] = m;
  }
  __syncthreads();
  if (threadIdx.x < 32) {
    float m = sred[0][threadIdx.x];
#pragma unroll
    for (int u = 1; u < kNG; ++u) m = fmaxf(m, sred[u][threadIdx.x]);
    sinc[threadIdx.x] = m;
  }
  __syncthreads();
  if (!live) return;

  // the running maximum at this block: earlier splits, earlier waves, this one
  float Mj[2];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    float m = sinc[16 * rt + r];
    for (int w = 0; w <= wave; ++w) m = fmaxf(m, sbm[w][16 * rt + r]);
    Mj[rt] = m;
  }
  // P = exp2(S - M) (0 where masked), l_j = sum P, P16 as the B operand of the
  // 16-key chunk kt (lane (g, r): keys 4 g + t of row r)
  h4 pk[4][2];
  float lsum[2];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    float ps = 0.f;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const float x = sv[rt][4 * kt + t];
        const float p = x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(x - Mj[rt]);
        ps += p;
        pk[kt][rt][t] = (_Float16)p;
      }
    ps += __shfl_xor(ps, 16);
    ps += __shfl_xor(ps, 32);
    lsum[rt] = ps;
  }
  // P V per 16-row tile and 16-d tile: the f16 accumulator through four
  // chunks (V^T operand of chunk kt: the 4 slots of keys 4 g + t in the
  // 32-key V block kt / 2, half kt % 2 of the lane's 16-byte load)
  const size_t out0 = (((size_t)kh * a.n_rg + rg) * a.nbmax + blk) * 32;
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const uint32_t row = 16 * rt + r;
    uint16_t* dst = a.pv + (out0 + row) * HD + 4 * g;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        const h8 v8 = vop[kt >> 1][dt];
        const h4 va = (kt & 1) ? h4{v8[4], v8[5], v8[6], v8[7]} : h4{v8[0], v8[1], v8[2], v8[3]};
        acc = __builtin_amdgcn_mfma_f32_16x16x16f16(va, pk[kt][rt], acc, 0, 0, 0);
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[t] = (float)(_Float16)acc[t];  // the f16 accumulator
      }
      const h4 o = {(_Float16)acc[0], (_Float16)acc[1], (_Float16)acc[2], (_Float16)acc[3]};
      if (rok[rt]) *(uint2*)(dst + 16 * dt) = __builtin_bit_cast(uint2, o);
    }
    if (g == 0 && rok[rt]) a.ml[out0 + row] = make_float2(Mj[rt], lsum[rt]);
  }
}

// The output chain of the rows' blocks, then attn [N][Dq] and the Wo operand
// (the hi/lo groups, or with bh the f16 rows of the wide f16 GEMM). The
// workgroup (sb, col) owns outputs 256 sb .. +255 of column col (NH heads of
// HD); thread t owns output 256 sb + t. Blocks go through LDS in chunks of CB:
// every thread first issues its 16 loads of the chunk's PV16 rows, then the
// chain reads LDS.
template <int HD>
__global__ __launch_bounds__(256) void k_fa16_chain(Fa16Args a, float* __restrict__ attn, uint16_t* __restrict__ bx,
                                                    uint16_t* __restrict__ xs, float* __restrict__ cs,
                                                    uint16_t* __restrict__ bh) {
  constexpr int NH = 256 / HD, CB = 128, PPB = NH * HD / 8;  // 16-byte pieces per block
  constexpr int NLD = CB * PPB / 256;                          // loads per thread per chunk
  static_assert(NLD == 16, "16 loads per thread");
  typedef uint32_t u4v __attribute__((ext_vector_type(4)));
  __shared__ u4v pvs[CB * PPB];  // [block][local head][d / 8]
  __shared__ float2 mls[CB][NH];
  __shared__ float outf[256];
  const uint32_t sb = blockIdx.x, c = blockIdx.y, t = threadIdx.x;
  {  // the look-back words start unset in the next launch
    const uint32_t nword = a.n_kv * a.n_rg * a.max_splits * 32;
    const uint32_t tid = (blockIdx.y * gridDim.x + blockIdx.x) * 256 + t, nthr = gridDim.x * gridDim.y * 256;
    for (uint32_t i = tid; i < nword; i += nthr) a.smax[i] = __builtin_bit_cast(float, kUnset);
  }
  const uint32_t kb0 = a.dbase ? *a.dbase : 0u;
  const uint32_t kvlen = a.kvlen + kb0, mbase = a.mask_base + kb0;
  const uint32_t Dq = a.n_head * HD, h0 = 256 * sb / HD;
  const uint32_t nb = (min(mbase + c, kvlen - 1)) / 64 + 1;
  // row of local head hh: kv head, row group and row of query row c * gqa + head % gqa
  auto rowbase = [&](uint32_t hh) {
    const uint32_t head = h0 + hh, kh = head / a.gqa, rho = c * a.gqa + head % a.gqa;
    return (((size_t)kh * a.n_rg + rho / 32) * a.nbmax) * 32 + rho % 32;  // + 32 j: block j's row
  };
  const uint32_t hl = t / HD, d = t % HD;
  const bool valid = 256 * sb + t < Dq;
  float Mp = kNegBig, L = 0.f;
  _Float16 o = (_Float16)0.f;
  for (uint32_t j0 = 0; j0 < nb; j0 += CB) {
    const uint32_t nbc = min((uint32_t)CB, nb - j0);
    u4v buf[NLD];
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      const uint32_t p = t + 256 * i, jb = p / PPB, hh = (p % PPB) / (HD / 8), d8 = p % (HD / 8);
      buf[i] = u4v{0u, 0u, 0u, 0u};
      if (jb < nbc && h0 + hh < a.n_head)
        buf[i] = *(const u4v*)(a.pv + (rowbase(hh) + 32 * (size_t)(j0 + jb)) * HD + 8 * d8);
    }
    for (uint32_t i = t; i < nbc * NH; i += 256) {
      const uint32_t jb = i / NH, hh = i % NH;
      if (h0 + hh < a.n_head) mls[jb][hh] = a.ml[rowbase(hh) + 32 * (size_t)(j0 + jb)];
    }
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      const uint32_t p = t + 256 * i, jb = p / PPB, hh = (p % PPB) / (HD / 8);
      if (jb < nbc && h0 + hh < a.n_head) pvs[p] = buf[i];
    }
    __syncthreads();
    if (valid) {
      const _Float16* pvh = reinterpret_cast<const _Float16*>(pvs) + hl * HD + d;
      for (uint32_t jb0 = 0; jb0 < nbc; jb0 += 8) {
        // 8 blocks' LDS reads in flight, then their steps
        float2 m[8];
        _Float16 p[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const uint32_t jb = min(jb0 + u, nbc - 1);
          m[u] = mls[jb][hl];
          p[u] = pvh[(size_t)jb * PPB * 8];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          if (jb0 + u >= nbc) break;
          const float e = __builtin_amdgcn_exp2f(Mp - m[u].x);
          L = e * L + m[u].y;
          o = o * (_Float16)e;  // f16(f16(e) O16)
          asm volatile("" : "+v"(o));  // two roundings, not a fused multiply-add
          o = o + p[u];  // f16(O16 + PV16)
          Mp = m[u].x;
        }
      }
    }
    __syncthreads();
  }
  const float il = L == 0.f ? 0.f : 1.0f / L;
  outf[t] = valid ? (float)o * il : 0.f;
  __syncthreads();
  if (t >= 64) return;
  const float4 v = make_float4(outf[4 * t], outf[4 * t + 1], outf[4 * t + 2], outf[4 * t + 3]);
  const uint32_t k = 256 * sb + 4 * t;
  if (k < Dq) *(float4*)(attn + (size_t)(a.col0 + c) * Dq + k) = v;
  if (bh) {
    const h4 h = {(_Float16)v.x, (_Float16)v.y, (_Float16)v.z, (_Float16)v.w};
    if (k < Dq) *(uint2*)(bh + (size_t)(a.col0 + c) * Dq + k) = __builtin_bit_cast(uint2, h);
  } else {
    sh_operand_store_sb(v, Dq, sb, a.col0 + c, bx, xs, cs);
  }
}

}  // namespace

size_t sh_fa16_pv_halves(uint32_t n_kv, uint32_t hd, uint32_t gqa, uint32_t ncol, uint32_t kv_cap) {
  const uint32_t n_rg = (gqa * ncol + 31) / 32, nbmax = (kv_cap + 63) / 64;
  return (size_t)n_kv * n_rg * nbmax * 32 * hd;
}

size_t sh_fa16_sync_words(uint32_t n_kv, uint32_t gqa, uint32_t ncol, uint32_t kv_cap) {
  const uint32_t n_rg = (gqa * ncol + 31) / 32, nbmax = (kv_cap + 63) / 64;
  return (size_t)n_kv * n_rg * ((nbmax + kW - 1) / kW);
}

int sh_fa16_launch(sh_engine* e, const sh_model* m, const sh_kv* kv, const FaArgs& fa, const float* q,
                   float* attn_out, uint16_t* bx, uint16_t* xs, float* cs, uint16_t* bh) {
  const Workspace& w = m->ws;
  const uint32_t gqa = m->n_head / m->n_kv;
  SH_CHECK(fa.N >= 1 && fa.col0 + fa.N <= w.max_cols, SH_ERR_ARG, "cm1 attention: columns [%u, %u)", fa.col0,
           fa.col0 + fa.N);
  SH_CHECK(fa.kvlen > 0 || fa.dbase, SH_ERR_ARG, "attention over zero keys");
  SH_CHECK(!fa.dbase || fa.kv_cap >= fa.kvlen, SH_ERR_ARG, "attention: graph key capacity below the offset");
  SH_CHECK(kv->max_seq % 32 == 0 && kv->max_seq >= 32, SH_ERR_ARG, "kv max_seq must be a positive multiple of 32");
  SH_CHECK(m->hd == 64 || m->hd == 128, SH_ERR_UNSUPPORTED, "head_dim %u not supported (64, 128)", m->hd);
  const uint32_t kv_grid = fa.dbase ? fa.kv_cap : fa.kvlen;
  SH_CHECK(kv_grid <= kv->max_seq, SH_ERR_ARG, "attention keys %u beyond the cache %u", kv_grid, kv->max_seq);
  Fa16Args a;
  a.kc = kv->k + (size_t)m->n_kv * kv->max_seq * m->hd * fa.layer;
  a.vc = kv->v + (size_t)m->n_kv * kv->max_seq * m->hd * fa.layer;
  a.q = q + (size_t)fa.col0 * m->n_head * m->hd;
  a.max_seq = kv->max_seq; a.n_head = m->n_head; a.n_kv = m->n_kv; a.gqa = gqa; a.ncol = fa.N; a.col0 = fa.col0;
  a.kvlen = fa.kvlen; a.mask_base = fa.mask_base; a.dbase = fa.dbase;
  a.n_rg = (gqa * fa.N + 31) / 32;
  a.nbmax = (kv_grid + 63) / 64;
  a.max_splits = (a.nbmax + kW - 1) / kW;
  // q * (scale * log2 e) with scale = 1 / sqrt(head_dim), each in f32 (models/llama.rs:237)
  const float scale = 1.0f / sqrtf((float)m->hd);
  a.qs = scale * 1.44269504088896340736f;
  SH_CHECK(sh_fa16_pv_halves(m->n_kv, m->hd, gqa, fa.N, kv_grid) <= w.fa16_pv_halves &&
               sh_fa16_sync_words(m->n_kv, gqa, fa.N, kv_grid) <= w.fa16_sync_words,
           SH_ERR_CAPACITY, "cm1 attention buffers too small");
  a.pv = w.fa16_pv; a.ml = w.fa16_ml; a.smax = w.fa16_smax; a.err = w.fa16_flag + w.fa16_sync_words;
  hipEvent_t ev = nullptr;
  sh_prof_begin(e, &ev);
  const dim3 grid(a.max_splits, a.n_rg, m->n_kv);
  if (m->hd == 128) hipLaunchKernelGGL(k_fa16<128>, grid, dim3(64 * kW), 0, e->stream, a);
  else hipLaunchKernelGGL(k_fa16<64>, grid, dim3(64 * kW), 0, e->stream, a);
  SH_HIP(hipGetLastError());
  sh_prof_end(e, "attention", 2.0 * m->n_kv * (double)kv_grid * m->hd * 2.0, ev);
  sh_prof_begin(e, &ev);
  const dim3 cgrid((m->n_head * m->hd + 255) / 256, fa.N);
  if (m->hd == 128)
    hipLaunchKernelGGL(k_fa16_chain<128>, cgrid, dim3(256), 0, e->stream, a, attn_out, bx, xs, cs, bh);
  else
    hipLaunchKernelGGL(k_fa16_chain<64>, cgrid, dim3(256), 0, e->stream, a, attn_out, bx, xs, cs, bh);
  SH_HIP(hipGetLastError());
  sh_prof_end(e, "attn_combine", 0.0, ev);
  return SH_OK;
}
