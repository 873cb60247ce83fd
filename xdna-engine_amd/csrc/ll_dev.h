// ll_dev.h -- the low-latency persistent decode step (device side).
//
// The reference runs a decode token as one fused ELF dispatch whose ops pass
// activations through on-chip buffers (route_b_kernels/decode_fused/
// gen_decode.py:391-420; driver FusedDecoder::step_token, rust/npu-engine/
// src/asr/whisper_decoder.rs:1278-1286).  On MI355X a token at batch <= 4 is
// ~5 dependent GEMV/attention phases per layer, each needing the whole output
// of the previous one, so the cost is the cross-CU hand-off, not HBM.  This
// executor runs whole tokens (many per launch) in one cooperative launch of one
// 512-thread workgroup per CU:
//
// Exchange ("LL" vectors).  A phase publishes each output element as one
// 8-byte {fp32 value, 32-bit epoch} pair with an agent-scope store; a consumer
// polls the pairs it needs with 16-byte sc1 loads until every epoch equals the
// current step's.  An 8-byte store is single-copy atomic, so value and epoch
// arrive together and no flag or fence is needed: one store-to-load latency
// per hand-off.  Every vector is written exactly once per step (one buffer per
// phase and layer), and every workgroup reads all argmax partials at the end
// of a step, so a buffer is never rewritten while a reader of the previous
// step can still be polling it (the argmax partials alternate by step parity).
//
// Roles.  Workgroups with blockIdx % 4 == 0 are the attention side (A: norm +
// QKV, attention partials, merge, O projection; Whisper also the cross
// attention); the others the FFN side (F: norm + FC1 / gate-up, FC2 / down).
// Each side walks its own phase list and keeps its own copy of the residual
// stream in LDS, applying every residual update (FOLD phases) in the same
// order with the same code, so both copies are bit-identical and the residual
// itself is never exchanged.  A side issues the weight loads of its next GEMV
// before waiting for that GEMV's input, so the F side's FFN weights stream in
// while the A side runs attention, and the other way round.
//
// End of step: every workgroup takes a slice of the tied lm-head rows (GEMV
// with the final norm) and publishes its (max, index) per stream; every
// workgroup reads all partials, takes the same argmax, embeds the next token
// into its residual copy and starts the next step.
//
// Waits are bounded: a poll that exceeds the time limit sets status[0], and
// every poll checks status[0], so one stuck wait ends the whole launch.
#pragma once

#include "step_dev.h"

namespace xe {
namespace ll {

constexpr int kT = 512;       // threads per workgroup
constexpr int kW = kT / 64;   // waves
constexpr int kMaxNB = 4;     // streams per step
constexpr int kDM = 16;       // output elements per merge block
constexpr int kMaxSplits = 64;
constexpr int kRoleStride = 4;  // blockIdx % 4 == 0: attention side

// An exchange vector: element (b, i) is pair p[b * ld + i]; ld is even and p
// 16-byte aligned, so pairs 2j, 2j+1 of a row are one 16-byte load.
struct Vec {
  uint64_t *p;
  int ld;
  int pad;
};

enum Kind { LK_FOLD = 0, LK_GEMV = 1, LK_ATTN = 2, LK_MERGE = 3 };

// residual += post(src): plain add, or Gemma's RMSNorm (1 + w) of src first.
struct FoldD {
  Vec src;
  const float *post_w;
  float eps;
};

struct GemvD {
  const void *w;
  const float *scale;
  const uint8_t *exps;
  const float *bias;
  int m, k;
  int lpr, rpl;
  int in_vec;  // 1: input = exchange vector `in` (k pairs); 0: norm(residual)
  Vec in;
  int norm;
  const float *gamma, *beta;
  float eps;
  int act;
  Vec out;  // m outputs (m / 2 with GeGLU)
  // residual updates applied (in order) after the weight loads are issued and
  // before the norm: the waits for earlier phases' outputs overlap the loads
  int nfold;
  FoldD folds[3];
};

struct AttnD {
  Vec q;           // rows hold q at q_off (head h at q_off + h*hd), new k / v at k_off / v_off
  int qn;          // pairs to read per row (covers q and, for self attention, k and v)
  int q_off, k_off, v_off;
  int append;      // self attention: append the new k/v at pos
  uint16_t *kc, *vc;
  size_t kv_bstride;
  int max_ctx;
  int hq, hkv, hd;
  float scale;
  int fixed_len;   // > 0: cross attention over fixed_len keys
  const float *q_norm_w, *k_norm_w;
  float norm_eps;
  const float *rope_cos, *rope_sin;
  int max_splits;
  Vec part;        // row b: [hq][max_splits][hd + 2] = (m, l, acc[hd])
};

struct MergeD {
  Vec part;
  Vec out;
  int hq, hd, max_splits, fixed_len, div_norm;
};

struct Phase {
  int kind;
  int pad[3];
  union {
    FoldD fold;
    GemvD gemv;
    AttnD attn;
    MergeD merge;
  } u;
};

struct StepParams {
  const Phase *ph_a;
  int n_a;
  const Phase *ph_f;
  int n_f;
  // token embedding (tied with the lm-head)
  const void *emb;
  const float *emb_scale;
  const uint8_t *emb_exps;
  const float *pos_emb;
  int pos_off, pos_rows;
  float emb_mul;
  int use_mul;
  int vocab, d, nb;
  // lm-head: final norm, tile
  int head_norm;
  const float *head_gamma, *head_beta;
  float head_eps;
  int head_lpr, head_rpl;
  float *logits;  // [nb][vocab] plain fp32 (read by the host after the launch); may be null
  Vec arg;        // [2][nb][grid * 2]: (max, index) pairs per workgroup, by step parity
  int last_max;
  // stream state (written by workgroup 0 at each step's end)
  int32_t *tokens, *pos, *next, *hist;
  int hist_stride;
  const int32_t *forced;  // [n_forced][nb] input tokens of the first steps, or null
  int n_forced;
  int n_steps;
  unsigned ep0;  // epoch of step 0 (>= 1; buffers start at epoch 0)
  unsigned *status;
  uint64_t limit;  // wall-clock ticks a single wait may take
  // LDS layout (floats): residual [nb][d] | input [nb][kin] | scratch
  int kin;
  int scratch;
  // optional wall-clock trace of step 0: [n_a + n_f + 4][grid] phase end
  // times (A phases, F phases, lm-head, argmax, embed, kernel start)
  uint64_t *trace;
};

// ---------------------------------------------------------------------------
// exchange primitives
// ---------------------------------------------------------------------------
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

template <typename V>
__device__ __forceinline__ void put(const V &v, int b, int i, float x, unsigned ep) {
  __hip_atomic_store(gptr_w(v.p) + static_cast<size_t>(b) * v.ld + i,
                     static_cast<uint64_t>(ep) << 32 | __float_as_uint(x), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

struct Ctl {
  unsigned *status;
  uint64_t limit;
  int *bad;  // LDS flag, WG-uniform after a barrier
};

__device__ __forceinline__ bool stop_now(const Ctl &c, uint64_t t0) {
  return wall_clock64() - t0 > c.limit ||
         __hip_atomic_load(gptr(c.status), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u;
}

__device__ __forceinline__ void raise_stop(const Ctl &c) {
  __hip_atomic_store(gptr_w(c.status), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  *lptr(c.bad) = 1;
}

// Byte offset past every buffer's range (num_records 0x7ffffff0): a buffer
// load there returns zeros without touching memory.
constexpr int kNoRecord = 0x7ffffff0;

// 16-byte coherent (sc1) load of pairs 2j, 2j+1 at byte offset off of base.
__device__ __forceinline__ u32x4 ld_pairs(__amdgpu_buffer_rsrc_t rs, int off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, gdev::kCoherentSc1));
}

// Read nb rows x n pairs (n even) of v into LDS dst[b * ldd + i], polling until
// every epoch is ep.  All kT threads; ends with a barrier; WG-uniform result.
template <typename V>
__device__ __forceinline__ bool get(const V &v, int nb, int n, float *dst, int ldd, unsigned ep,
                                    const Ctl &c) {
  constexpr int U = 4;
  const int half = n >> 1;
  const int total = nb * half;
  const __amdgpu_buffer_rsrc_t rs = gdev::coherent_rsrc(v.p);
  XE_LDS float *D = lptr(dst);
  bool bad = false;
  for (int base = 0; base < total && !bad; base += kT * U) {
    u32x4 val[U];
    int off[U], di[U];
    bool need[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int q = base + u * kT + static_cast<int>(threadIdx.x);
      need[u] = q < total;
      const int b = need[u] ? q / half : 0, j = need[u] ? q % half : 0;
      // an offset past the buffer range reads zeros: no divergent branch
      off[u] = need[u] ? (b * v.ld + 2 * j) * 8 : kNoRecord;
      di[u] = b * ldd + 2 * j;
      val[u] = ld_pairs(rs, off[u]);
    }
    const uint64_t t0 = wall_clock64();
    unsigned spins = 0;
    while (true) {
      bool all = true;
#pragma unroll
      for (int u = 0; u < U; u++)
        if (need[u]) {
          if (val[u].y == ep && val[u].w == ep) {
            D[di[u]] = __uint_as_float(val[u].x);
            D[di[u] + 1] = __uint_as_float(val[u].z);
            need[u] = false;
          } else {
            all = false;
          }
        }
      if (all) break;
      if ((++spins & 63) == 0 && stop_now(c, t0)) {
        bad = true;
        break;
      }
#pragma unroll
      for (int u = 0; u < U; u++) val[u] = ld_pairs(rs, need[u] ? off[u] : kNoRecord);
    }
  }
  if (bad) raise_stop(c);
  __syncthreads();
  return *lptr(c.bad) == 0;
}

// Poll single pairs base[idx[i]] (merge inputs): up to NI per thread.  The
// pairs not needed read past the buffer range (zeros, no branch).
template <int NI>
__device__ __forceinline__ bool get_scattered(const uint64_t *base, const int (&idx)[NI], const bool (&need_in)[NI],
                                              float (&out)[NI], unsigned ep, const Ctl &c) {
  typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
  const __amdgpu_buffer_rsrc_t rs = gdev::coherent_rsrc(base);
  bool need[NI];
  u32x2 val[NI];
#pragma unroll
  for (int i = 0; i < NI; i++) {
    need[i] = need_in[i];
    val[i] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs, need[i] ? idx[i] * 8 : kNoRecord, 0,
                                                                           gdev::kCoherentSc1));
  }
  const uint64_t t0 = wall_clock64();
  unsigned spins = 0;
  while (true) {
    bool all = true;
#pragma unroll
    for (int i = 0; i < NI; i++)
      if (need[i]) {
        if (val[i].y == ep) {
          out[i] = __uint_as_float(val[i].x);
          need[i] = false;
        } else {
          all = false;
        }
      }
    if (all) return true;
    if ((++spins & 63) == 0 && stop_now(c, t0)) return false;
#pragma unroll
    for (int i = 0; i < NI; i++)
      val[i] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs, need[i] ? idx[i] * 8 : kNoRecord, 0,
                                                                             gdev::kCoherentSc1));
  }
}

// ---------------------------------------------------------------------------
// block reductions (kW waves), residual update and norm
// ---------------------------------------------------------------------------
template <int N>
__device__ __forceinline__ void sums(float (&v)[N], float *red, int &slot) {
  gdev::block_sums<kW, N>(v, red, slot);
}

// residual[b] += post(src[b]) for b < nb.  tmp: LDS [nb][d].
template <typename FD>
__device__ __forceinline__ bool fold(const FD &f, int nb, int d, float *xr, float *tmp, float *red,
                                     unsigned ep, const Ctl &c) {
  if (!get(f.src, nb, d, tmp, d, ep, c)) return false;
  int slot = 0;
  const XE_GLOBAL float *pw = gptr(f.post_w);
  for (int b = 0; b < nb; b++) {
    XE_LDS float *x = lptr(xr) + static_cast<size_t>(b) * d;
    const XE_LDS float *s = lptr(tmp) + static_cast<size_t>(b) * d;
    if (f.post_w) {
      float ss[1] = {0.f};
      for (int i = threadIdx.x; i < d; i += kT) ss[0] = __builtin_fmaf(s[i], s[i], ss[0]);
      sums<1>(ss, red, slot);
      const float inv = 1.0f / sqrtf(ss[0] / static_cast<float>(d) + f.eps);
      for (int i = threadIdx.x; i < d; i += kT) x[i] = x[i] + s[i] * inv * (1.0f + pw[i]);
    } else {
      for (int i = threadIdx.x; i < d; i += kT) x[i] = x[i] + s[i];
    }
  }
  __syncthreads();
  return true;
}

// dst[b] = norm(x[b]) (LayerNorm two-pass / RMS / RMS (1 + w) / copy).
__device__ __forceinline__ void norm_rows(const float *xr, int nb, int d, int norm, const float *gamma,
                                          const float *beta, float eps, float *dst, float *red) {
  int slot = 0;
  const float fd = static_cast<float>(d);
  const XE_GLOBAL float *gam = gptr(gamma), *bet = gptr(beta);
  for (int b = 0; b < nb; b++) {
    const XE_LDS float *x = lptr(xr) + static_cast<size_t>(b) * d;
    XE_LDS float *h = lptr(dst) + static_cast<size_t>(b) * d;
    if (norm == XE_NORM_LN) {
      float v1[1] = {0.f};
      for (int i = threadIdx.x; i < d; i += kT) v1[0] += x[i];
      sums<1>(v1, red, slot);
      const float mean = v1[0] / fd;
      float v2[1] = {0.f};
      for (int i = threadIdx.x; i < d; i += kT) {
        const float cc = x[i] - mean;
        v2[0] = __builtin_fmaf(cc, cc, v2[0]);
      }
      sums<1>(v2, red, slot);
      const float inv = 1.0f / sqrtf(v2[0] / fd + eps);
      for (int i = threadIdx.x; i < d; i += kT) h[i] = (x[i] - mean) * inv * gam[i] + bet[i];
    } else if (norm == XE_NORM_RMS || norm == XE_NORM_RMS1P) {
      float v1[1] = {0.f};
      for (int i = threadIdx.x; i < d; i += kT) v1[0] = __builtin_fmaf(x[i], x[i], v1[0]);
      sums<1>(v1, red, slot);
      const float inv = 1.0f / sqrtf(v1[0] / fd + eps);
      if (norm == XE_NORM_RMS1P)
        for (int i = threadIdx.x; i < d; i += kT) h[i] = x[i] * inv * (1.0f + gam[i]);
      else
        for (int i = threadIdx.x; i < d; i += kT) h[i] = x[i] * inv * gam[i];
    } else {
      for (int i = threadIdx.x; i < d; i += kT) h[i] = x[i];
    }
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------
// GEMV over rows [r0, r1) with the input in LDS.  The first tile's weight
// loads are issued before `prep` (which fetches / normalises the input), so
// they overlap the wait.  HEAD: lm-head mode (logits + running argmax instead
// of an exchange vector).
// ---------------------------------------------------------------------------
struct ArgBest {
  float v[kMaxNB];
  int i[kMaxNB];
};

// One GEMV code path for every phase (code size: the whole step runs from the
// instruction cache, so each phase kind must stay small and shared).  Tile:
// lanes per row LPR (runtime: 8/16/32/64) x two rows per lane (a GeGLU
// (gate, up) pair, or two neighbouring rows).  A load round holds NIT chunk
// iterations per row: every load of a round is issued, unconditionally,
// before any result is used, and a round consumes all it loaded before the
// next (a load still pending at a later load into the same register makes
// the compiler serialise the stream).
template <int WT>
struct Round {
  static constexpr int NIT = WT == XE_BF16 ? 4 : 9;
};

// Weight chunk loads through buffer descriptors: a chunk that is not needed
// (past the row end, past the round's iterations, or a dropped row) reads
// past the buffer range and comes back as zeros.  Weight matrices stay below
// 2 GB (32-bit offsets).
struct WRsrc {
  __amdgpu_buffer_rsrc_t w, e;
};
constexpr int kNontemporal = 2;  // cache-policy operand: nt (streamed once per step)

template <int WT>
__device__ __forceinline__ void load_chunk_buf(const WRsrc &rs, int row, int K, int c, bool valid, gdev::Chunk<WT> &out) {
  typedef unsigned u4v __attribute__((ext_vector_type(4)));
  auto ld16 = [&](int off) {
    const u4v v = __builtin_bit_cast(u4v, __builtin_amdgcn_raw_buffer_load_b128(rs.w, off, 0, kNontemporal));
    return make_uint4(v.x, v.y, v.z, v.w);
  };
  if constexpr (WT == XE_BF16) {
    const int off = valid ? (row * K + c * 16) * 2 : kNoRecord;
    out.lo = ld16(off);
    out.hi = ld16(valid ? off + 16 : kNoRecord);
  } else {
    out.q = ld16(valid ? row * K + c * 16 : kNoRecord);
    if constexpr (WT == XE_BFP16)
      out.e = __builtin_amdgcn_raw_buffer_load_b16(rs.e, valid ? row * (K / 8) + c * 2 : kNoRecord, 0, 0);
  }
}

template <int WT, int NB, bool HEAD, typename GD, typename Prep, typename Sub>
__device__ __forceinline__ bool gemv_rows(const GD &g, int nb, int r0, int r1, const float *xs, unsigned ep,
                                          Prep prep, float *logits, int vocab, int last_max, ArgBest &best,
                                          Sub tsub) {
  using gdev::Chunk;
  using gdev::chunk_dot;
  constexpr int RPL = 2;
  constexpr int NIT = Round<WT>::NIT;
  const int lpr_log = __builtin_ctz(static_cast<unsigned>(g.lpr));
  const int LPR = 1 << lpr_log;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rg = lane >> lpr_log, kl = lane & (LPR - 1);
  const int rows_per_wave = (64 >> lpr_log) * RPL;
  const int rows_per_tile = kW * rows_per_wave;
  const int K = g.k, nch = K / 16;
  const int n_it = (nch + LPR - 1) >> lpr_log;
  const int ntiles = r1 > r0 ? (r1 - r0 + rows_per_tile - 1) / rows_per_tile : 0;
  WRsrc rs;
  rs.w = gdev::coherent_rsrc(g.w);
  rs.e = gdev::coherent_rsrc(WT == XE_BFP16 ? static_cast<const void *>(g.exps) : g.w);
  bool ok = true;
  if (ntiles == 0) return prep();
  for (int tile = 0; tile < ntiles && ok; tile++) {
    const int row0 = r0 + tile * rows_per_tile + wave * rows_per_wave + rg * RPL;
    bool row_ok[RPL];
    int row[RPL];
#pragma unroll
    for (int i = 0; i < RPL; i++) {
      row[i] = row0 + i;
      row_ok[i] = row[i] < r1;
    }
    float acc[NB][RPL];
    float rscale[RPL], rbias[RPL];
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
      for (int i = 0; i < RPL; i++) acc[b][i] = 0.f;
    for (int it0 = 0; it0 < n_it && ok; it0 += NIT) {
      Chunk<WT> w[NIT][RPL];
#pragma unroll
      for (int u = 0; u < NIT; u++) {
        const int cc = ((it0 + u) << lpr_log) + kl;
        const bool valid = it0 + u < n_it && cc < nch;
#pragma unroll
        for (int i = 0; i < RPL; i++) load_chunk_buf<WT>(rs, row[i], K, cc, valid && row_ok[i], w[u][i]);
      }
      if (it0 == 0) {  // epilogue constants travel with the first round's loads
#pragma unroll
        for (int i = 0; i < RPL; i++) {
          const int rr = row_ok[i] ? row[i] : r0;
          rscale[i] = WT == XE_I8 ? gptr(g.scale)[rr] : 1.0f;
          rbias[i] = g.bias ? gptr(g.bias)[rr] : 0.0f;
        }
      }
      if (tile == 0 && it0 == 0) ok = prep();
      if (!ok) break;
#pragma unroll
      for (int u = 0; u < NIT; u++) {
        if (it0 + u < n_it) {
          const int cx = min(((it0 + u) << lpr_log) + kl, nch - 1);  // past the row end: zero weights
#pragma unroll
          for (int b = 0; b < NB; b++) {
            if (b < nb) {
              typedef float f32x4 __attribute__((ext_vector_type(4)));
              float4 xv[4];
              const XE_LDS f32x4 *xr =
                  reinterpret_cast<const XE_LDS f32x4 *>(lptr(xs) + static_cast<size_t>(b) * K + cx * 16);
#pragma unroll
              for (int j = 0; j < 4; j++) {
                const f32x4 t = xr[j];
                xv[j] = make_float4(t.x, t.y, t.z, t.w);
              }
#pragma unroll
              for (int i = 0; i < RPL; i++) acc[b][i] = chunk_dot<WT>(w[u][i], xv, acc[b][i]);
            }
          }
        }
      }
    }
    if (!ok) break;
    if (tile == 0) tsub(1);
    for (int off = LPR >> 1; off >= 1; off >>= 1) {
#pragma unroll
      for (int b = 0; b < NB; b++)
#pragma unroll
        for (int i = 0; i < RPL; i++) acc[b][i] += __shfl_xor(acc[b][i], off, 64);
    }
    if (kl == 0) {
#pragma unroll
      for (int b = 0; b < NB; b++) {
        if (b >= nb) break;
        float v[RPL];
#pragma unroll
        for (int i = 0; i < RPL; i++) {
          float t = acc[b][i];
          if (WT == XE_I8) t = t * rscale[i];
          if (g.bias) t = t + rbias[i];
          v[i] = t;
        }
        if constexpr (HEAD) {
#pragma unroll
          for (int i = 0; i < RPL; i++) {
            if (!row_ok[i]) continue;
            if (logits) gptr_w(logits)[static_cast<size_t>(b) * vocab + row[i]] = v[i];
            if (sdev::better(v[i], row[i], best.v[b], best.i[b], last_max)) {
              best.v[b] = v[i];
              best.i[b] = row[i];
            }
          }
        } else if (g.act == ACT_GEGLU_TANH) {
          if (row_ok[0]) put(g.out, b, row[0] / 2, gdev::gelu_tanh(v[0]) * v[1], ep);
        } else {
#pragma unroll
          for (int i = 0; i < RPL; i++) {
            if (!row_ok[i]) continue;
            float t = v[i];
            if (g.act == ACT_RELU) t = t > 0.f ? t : 0.f;
            else if (g.act == ACT_GELU_ERF) t = gdev::gelu_erf(t);
            put(g.out, b, row[i], t, ep);
          }
        }
      }
    }
  }
  return ok;
}

template <int WT, int NB, bool HEAD, typename GD, typename Prep, typename Sub>
__device__ __forceinline__ bool gemv_any(const GD &g, int nb, int r0, int r1, const float *xs, unsigned ep,
                                         Prep prep, float *logits, int vocab, int last_max, ArgBest &best,
                                         const Ctl &c, Sub tsub) {
  (void)c;
  return gemv_rows<WT, NB, HEAD>(g, nb, r0, r1, xs, ep, prep, logits, vocab, last_max, best, tsub);
}
struct NoSub {
  __device__ void operator()(int) const {}
};

// Rows of rank r out of n ranks (balanced contiguous split).
__device__ __forceinline__ void rank_rows(int m, int r, int n, int &r0, int &r1) {
  r0 = static_cast<int>((static_cast<long long>(m) * r) / n);
  r1 = static_cast<int>((static_cast<long long>(m) * (r + 1)) / n);
}

// ---------------------------------------------------------------------------
// attention partials over the current length, and the merge
// ---------------------------------------------------------------------------
__device__ __forceinline__ u32x4 ld_kv(__amdgpu_buffer_rsrc_t rs, int byte_off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, byte_off, 0, gdev::kCoherentSc1));
}

__device__ __forceinline__ void st_bf16_coherent(uint16_t *p, uint16_t v) {
  __hip_atomic_store(gptr_w(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Per-lane constants of the head transform (norm weights, RoPE cos/sin at
// the position), loaded before the block waits for q.  Lane j owns elements
// (j, j + hd/2) for j = lane + 64 i.
template <int HD>
struct HeadConsts {
  static constexpr int HALF = HD / 2;
  static constexpr int PER = (HALF + 63) / 64;
  float qn0[PER], qn1[PER], kn0[PER], kn1[PER], cs[PER], sn[PER];
};

template <int HD, typename AD>
__device__ __forceinline__ void load_head_consts(const AD &a, int posi, HeadConsts<HD> &hc) {
  constexpr int HALF = HeadConsts<HD>::HALF, PER = HeadConsts<HD>::PER;
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < PER; i++) {
    const int j = min(lane + 64 * i, HALF - 1);
    hc.qn0[i] = a.q_norm_w ? gptr(a.q_norm_w)[j] : 0.f;
    hc.qn1[i] = a.q_norm_w ? gptr(a.q_norm_w)[j + HALF] : 0.f;
    hc.kn0[i] = a.k_norm_w ? gptr(a.k_norm_w)[j] : 0.f;
    hc.kn1[i] = a.k_norm_w ? gptr(a.k_norm_w)[j + HALF] : 0.f;
    hc.cs[i] = a.rope_cos ? gptr(a.rope_cos)[static_cast<size_t>(posi) * HALF + j] : 1.f;
    hc.sn[i] = a.rope_sin ? gptr(a.rope_sin)[static_cast<size_t>(posi) * HALF + j] : 0.f;
  }
}

// Per-head RMSNorm (1 + w) and RoPE of one head vector (LDS src -> LDS dst),
// one wave; rotate-half pairing (npu-asr-host/src/lib.rs:143-185).
template <int HD>
__device__ __forceinline__ void head_xform(const XE_LDS float *src, XE_LDS float *dst, bool norm, const float (&w0)[HeadConsts<HD>::PER],
                                           const float (&w1)[HeadConsts<HD>::PER], bool rope, const HeadConsts<HD> &hc,
                                           float eps) {
  constexpr int HALF = HeadConsts<HD>::HALF, PER = HeadConsts<HD>::PER;
  const int lane = threadIdx.x & 63;
  float x0[PER], x1[PER];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < PER; i++) {
    const int j = lane + 64 * i;
    x0[i] = j < HALF ? src[j] : 0.f;
    x1[i] = j < HALF ? src[j + HALF] : 0.f;
    ss = ss + x0[i] * x0[i];
    ss = ss + x1[i] * x1[i];
  }
  if (norm) {
    ss = gdev::wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / static_cast<float>(HD) + eps);
#pragma unroll
    for (int i = 0; i < PER; i++) {
      x0[i] = x0[i] * inv * (1.0f + w0[i]);
      x1[i] = x1[i] * inv * (1.0f + w1[i]);
    }
  }
#pragma unroll
  for (int i = 0; i < PER; i++) {
    const int j = lane + 64 * i;
    if (j >= HALF) continue;
    float y0 = x0[i], y1 = x1[i];
    if (rope) {
      const float t0 = y0 * hc.cs[i] - y1 * hc.sn[i];
      const float t1 = y1 * hc.cs[i] + y0 * hc.sn[i];
      y0 = t0;
      y1 = t1;
    }
    dst[j] = y0;
    dst[j + HALF] = y1;
  }
}

// Keys one wave round covers: kW waves x (64 / (hd / 8)) keys.  A split is a
// multiple of it, spread so that every attention-side workgroup gets a share.
__host__ __device__ constexpr int round_keys(int hd) { return kW * (64 / (hd / 8)); }

__host__ __device__ __forceinline__ void ll_split(int len, int max_splits, int hd, int &chunk, int &nsplits) {
  const int gran = round_keys(hd);
  int per = (len + max_splits - 1) / max_splits;
  per = (per + gran - 1) / gran * gran;
  chunk = per < gran ? gran : per;
  nsplits = (len + chunk - 1) / chunk;
}

__host__ __device__ __forceinline__ int attn_scratch_floats(int hd, int g) {
  return g * hd + kW * g * (hd + 2) + hd;
}

// One split block of (stream b, kv head kvh): keys [split*chunk, ...).
// The block's first K/V loads and its head-transform constants are issued
// before `prep` (which waits for the q rows: qin, LDS [nb][a.qn]); scr:
// attn_scratch_floats.  Returns prep's result.
template <int HD, int G, typename AD, typename Prep, typename Sub>
__device__ __forceinline__ bool attn_block(const AD &a, int split, int kvh, int b, int len, const float *qin,
                                           float *scr, unsigned ep, Prep prep, Sub tsub) {
  constexpr int EPL = 8;
  constexpr int L = HD / EPL;
  constexpr int KPW = 64 / L;
  constexpr int UK = 4;
  constexpr int STEP = kW * KPW;
  XE_LDS float *S = lptr(scr);
  XE_LDS float(*qs)[HD] = reinterpret_cast<XE_LDS float(*)[HD]>(S);
  XE_LDS float(*red)[G][HD + 2] = reinterpret_cast<XE_LDS float(*)[G][HD + 2]>(S + G * HD);
  XE_LDS float *kt = S + G * HD + kW * G * (HD + 2);
  int chunk, nsplits;
  ll_split(len, a.max_splits, HD, chunk, nsplits);
  const int s0 = split * chunk;
  const int s1 = min(len, s0 + chunk);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int posi = len - 1;
  const int kg = lane / L, kl = lane % L;

  uint16_t *kbase = a.kc + a.kv_bstride * b + static_cast<size_t>(kvh) * a.max_ctx * HD;
  uint16_t *vbase = a.vc + a.kv_bstride * b + static_cast<size_t>(kvh) * a.max_ctx * HD;
  const __amdgpu_buffer_rsrc_t krs = gdev::coherent_rsrc(kbase);
  const __amdgpu_buffer_rsrc_t vrs = gdev::coherent_rsrc(vbase);
  const bool appender = a.append && split == nsplits - 1;

  // ---- issue the first key block's loads and the transform constants ----
  // The new key at posi is not read back from the cache: the lane group that
  // holds it takes the bf16-rounded values from LDS (below), so the cache
  // stores can drain while the block computes.
  auto load_keys = [&](int base, u32x4 (&kv)[UK], u32x4 (&vv)[UK], bool (&okk)[UK]) {
#pragma unroll
    for (int u = 0; u < UK; u++) {
      const int key = base + u * STEP;
      okk[u] = key < s1;
      const int off = okk[u] ? (key * HD + kl * EPL) * 2 : kNoRecord;
      kv[u] = ld_kv(krs, off);
      vv[u] = ld_kv(vrs, off);
    }
  };
  const int base0 = s0 + wave * KPW + kg;
  u32x4 kv[UK], vv[UK];
  bool okk[UK];
  load_keys(base0, kv, vv, okk);
  HeadConsts<HD> hc;
  load_head_consts<HD>(a, a.fixed_len > 0 ? 0 : posi, hc);
  if (!prep()) return false;
  tsub(0);

  const XE_LDS float *qrow = lptr(qin) + static_cast<size_t>(b) * a.qn;
  const XE_LDS float *vsrc = qrow + a.v_off + kvh * HD;
  const bool qnorm = a.q_norm_w != nullptr, knorm = a.k_norm_w != nullptr, rope = a.rope_cos != nullptr;
  for (int gg = wave; gg < G; gg += kW)
    head_xform<HD>(qrow + a.q_off + (kvh * G + gg) * HD, qs[gg], qnorm, hc.qn0, hc.qn1, rope, hc, a.norm_eps);
  if (appender && wave == kW - 1) {
    head_xform<HD>(qrow + a.k_off + kvh * HD, kt, knorm, hc.kn0, hc.kn1, rope, hc, a.norm_eps);
    __builtin_amdgcn_wave_barrier();
    for (int j = lane; j < HD; j += 64) {
      st_bf16_coherent(kbase + static_cast<size_t>(posi) * HD + j, adev::f32_to_bf16_rne(kt[j]));
      st_bf16_coherent(vbase + static_cast<size_t>(posi) * HD + j, adev::f32_to_bf16_rne(vsrc[j]));
    }
  }
  __syncthreads();  // q heads and the new k staged in LDS
  // the new key/value as stored in the cache (bf16, packed pairs)
  auto pack8 = [&](const XE_LDS float *src) {
    u32x4 r;
    r.x = static_cast<uint32_t>(adev::f32_to_bf16_rne(src[0])) | static_cast<uint32_t>(adev::f32_to_bf16_rne(src[1])) << 16;
    r.y = static_cast<uint32_t>(adev::f32_to_bf16_rne(src[2])) | static_cast<uint32_t>(adev::f32_to_bf16_rne(src[3])) << 16;
    r.z = static_cast<uint32_t>(adev::f32_to_bf16_rne(src[4])) | static_cast<uint32_t>(adev::f32_to_bf16_rne(src[5])) << 16;
    r.w = static_cast<uint32_t>(adev::f32_to_bf16_rne(src[6])) | static_cast<uint32_t>(adev::f32_to_bf16_rne(src[7])) << 16;
    return r;
  };
  u32x4 knew = {0u, 0u, 0u, 0u}, vnew = {0u, 0u, 0u, 0u};
  if (appender) {
    knew = pack8(kt + kl * EPL);
    vnew = pack8(vsrc + kl * EPL);
  }
  auto substitute = [&](int base, u32x4 (&kv)[UK], u32x4 (&vv)[UK]) {
    if (!appender) return;
#pragma unroll
    for (int u = 0; u < UK; u++) {
      const bool is_new = base + u * STEP == posi;
      kv[u].x = is_new ? knew.x : kv[u].x;
      kv[u].y = is_new ? knew.y : kv[u].y;
      kv[u].z = is_new ? knew.z : kv[u].z;
      kv[u].w = is_new ? knew.w : kv[u].w;
      vv[u].x = is_new ? vnew.x : vv[u].x;
      vv[u].y = is_new ? vnew.y : vv[u].y;
      vv[u].z = is_new ? vnew.z : vv[u].z;
      vv[u].w = is_new ? vnew.w : vv[u].w;
    }
  };
  substitute(base0, kv, vv);
  tsub(1);

  float qr[G][EPL];
#pragma unroll
  for (int gg = 0; gg < G; gg++)
#pragma unroll
    for (int e = 0; e < EPL; e++) qr[gg][e] = qs[gg][kl * EPL + e];
  float m[G], l[G], acc[G][EPL];
#pragma unroll
  for (int gg = 0; gg < G; gg++) {
    m[gg] = -INFINITY;
    l[gg] = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; e++) acc[gg][e] = 0.f;
  }
  const float sc2 = a.scale * adev::kLog2e;
  for (int base = base0; base < s1; base += STEP * UK) {
    if (base != base0) {
      load_keys(base, kv, vv, okk);
      substitute(base, kv, vv);
    }
    float s[UK][G];
    // key slots the whole wave is past (short splits) are skipped: the wave's
    // first key of slot u is base - kg + u * STEP
    const int wave_first = base - kg;
#pragma unroll
    for (int u = 0; u < UK; u++) {
      if (wave_first + u * STEP >= s1) {
#pragma unroll
        for (int gg = 0; gg < G; gg++) s[u][gg] = -INFINITY;
        continue;
      }
      const uint32_t w[4] = {kv[u].x, kv[u].y, kv[u].z, kv[u].w};
      float kf[EPL];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        kf[2 * i] = __uint_as_float(w[i] << 16);
        kf[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
      }
#pragma unroll
      for (int gg = 0; gg < G; gg++) {
        float dd = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; e++) dd = __builtin_fmaf(qr[gg][e], kf[e], dd);
#pragma unroll
        for (int off = L / 2; off >= 1; off >>= 1) dd += __shfl_xor(dd, off, 64);
        s[u][gg] = dd * sc2;
      }
    }
#pragma unroll
    for (int gg = 0; gg < G; gg++) {
      float mb = m[gg];
#pragma unroll
      for (int u = 0; u < UK; u++)
        if (okk[u]) mb = fmaxf(mb, s[u][gg]);
      if (mb == -INFINITY) continue;
      const float corr = __builtin_amdgcn_exp2f(m[gg] - mb);
      float pu[UK];
      float psum = 0.f;
#pragma unroll
      for (int u = 0; u < UK; u++) {
        pu[u] = okk[u] ? __builtin_amdgcn_exp2f(s[u][gg] - mb) : 0.f;
        psum += pu[u];
      }
      l[gg] = l[gg] * corr + psum;
      m[gg] = mb;
#pragma unroll
      for (int e = 0; e < EPL; e++) acc[gg][e] *= corr;
#pragma unroll
      for (int u = 0; u < UK; u++) {
        if (wave_first + u * STEP >= s1) continue;
        const uint32_t w[4] = {vv[u].x, vv[u].y, vv[u].z, vv[u].w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
          acc[gg][2 * i] = __builtin_fmaf(pu[u], __uint_as_float(w[i] << 16), acc[gg][2 * i]);
          acc[gg][2 * i + 1] = __builtin_fmaf(pu[u], __uint_as_float(w[i] & 0xffff0000u), acc[gg][2 * i + 1]);
        }
      }
    }
  }
#pragma unroll
  for (int off = L; off < 64; off <<= 1) {
#pragma unroll
    for (int gg = 0; gg < G; gg++) {
      const float mo = __shfl_xor(m[gg], off, 64);
      const float lo = __shfl_xor(l[gg], off, 64);
      const float mx = fmaxf(m[gg], mo);
      const float fa = mx == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m[gg] - mx);
      const float fc = mx == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mo - mx);
      l[gg] = l[gg] * fa + lo * fc;
#pragma unroll
      for (int e = 0; e < EPL; e++) {
        const float ao = __shfl_xor(acc[gg][e], off, 64);
        acc[gg][e] = acc[gg][e] * fa + ao * fc;
      }
      m[gg] = mx;
    }
  }
  tsub(2);
  if (kg == 0) {
#pragma unroll
    for (int gg = 0; gg < G; gg++) {
#pragma unroll
      for (int e = 0; e < EPL; e++) red[wave][gg][2 + kl * EPL + e] = acc[gg][e];
      if (kl == 0) {
        red[wave][gg][0] = m[gg];
        red[wave][gg][1] = l[gg];
      }
    }
  }
  __syncthreads();
  for (int t = threadIdx.x; t < G * (HD + 2); t += kT) {
    const int gg = t / (HD + 2), e = t % (HD + 2);
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < kW; w++) mx = fmaxf(mx, red[w][gg][0]);
    float v = 0.f;
    if (e == 0) {
      v = mx;
    } else {
#pragma unroll
      for (int w = 0; w < kW; w++) {
        const float mw = red[w][gg][0];
        const float f = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - mx);
        v += red[w][gg][e] * f;
      }
    }
    put(a.part, b, ((kvh * G + gg) * a.max_splits + split) * (HD + 2) + e, v, ep);
  }
  __syncthreads();  // scratch is reused by the next block
  return true;
}

// Merge block: stream b, q head h, outputs [e0, e0 + kDM) of the head.
// tab: LDS scratch >= kMaxSplits * (kDM + 2) + kMaxSplits + 2 floats.
__device__ __noinline__ bool merge_block(const XE_CONST MergeD &mg, int b, int h, int e0, int len, float *tab_,
                                            unsigned ep, const Ctl c) {
  const int HD = mg.hd;
  XE_LDS float *tab = lptr(tab_);
  int chunk, nsplits;
  ll_split(len, mg.max_splits, HD, chunk, nsplits);
  constexpr int W = kDM + 2;
  constexpr int NI = (kMaxSplits * W + kT - 1) / kT;
  int idx[NI];
  bool need[NI];
  float got[NI];
  const uint64_t *row = mg.part.p + static_cast<size_t>(b) * mg.part.ld + static_cast<size_t>(h) * mg.max_splits * (HD + 2);
#pragma unroll
  for (int i = 0; i < NI; i++) {
    const int it = threadIdx.x + i * kT;
    const int s = it / W, col = it % W;
    need[i] = s < nsplits;
    const int e = col < 2 ? col : 2 + e0 + (col - 2);
    idx[i] = (need[i] ? s : 0) * (HD + 2) + e;
  }
  const bool okp = get_scattered<NI>(row, idx, need, got, ep, c);
  if (!okp) raise_stop(c);
#pragma unroll
  for (int i = 0; i < NI; i++) {
    const int it = threadIdx.x + i * kT;
    if (need[i]) tab[it] = got[i];  // tab[s * W + col]
  }
  __syncthreads();
  if (*lptr(c.bad)) return false;
  XE_LDS float *wts = tab + kMaxSplits * W;
  if (threadIdx.x < 64) {
    float mx = -INFINITY;
    for (int s = threadIdx.x; s < nsplits; s += 64) mx = fmaxf(mx, tab[s * W]);
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    for (int s = threadIdx.x; s < nsplits; s += 64) {
      const float ms = tab[s * W];
      wts[s] = ms == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ms - mx);
    }
  }
  __syncthreads();
  if (threadIdx.x < kDM) {
    const int e = threadIdx.x;
    float ls = 0.f, at = 0.f;
    for (int s = 0; s < nsplits; s++) {
      ls += tab[s * W + 1] * wts[s];
      at += tab[s * W + 2 + e] * wts[s];
    }
    const float o = mg.div_norm ? at / ls : at * (1.0f / ls);
    put(mg.out, b, h * HD + e0 + e, o, ep);
  }
  __syncthreads();
  return true;
}

// host side (ll_launch.hip)
bool step_supported(int wdtype, int nb_t, int hd, int g);
void launch(const StepParams &sp, int wdtype, int nb_t, int hd, int g, size_t lds_bytes, int grid, hipStream_t s);

}  // namespace ll
}  // namespace xe
