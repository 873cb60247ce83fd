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
constexpr int kSubSlots = 4;    // trace sub-stage marks per phase

// An exchange vector: element (b, i) is pair p[b * ld + i]; ld is even and p
// 16-byte aligned, so pairs 2j, 2j+1 of a row are one 16-byte load.
struct Vec {
  uint64_t *p;
  int ld;
  int pad;
};

enum Kind { LK_FOLD = 0, LK_GEMV = 1, LK_ATTN = 2, LK_MERGE = 3, LK_DPART = 4, LK_REDUCE = 5 };

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
  // 1: this rank's weight slice (and epilogue constants) sits in the LDS
  // stage area, copied there by an earlier phase (Phase::issue)
  int staged;
  // 1: one tile's row groups past the fourth are K-split over waves 4..7
  // (waves w and w + 4 share a SIMD; see gemv_rows)
  int tail_split;
  // > 0: the activations stay in this workgroup's LDS (its slice of the
  // FFN's hidden vector, read by the next phase, LK_DPART) instead of `out`,
  // at this float offset into each input row
  int out_lds;
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
  // keys of a block the LDS key/value stage holds (0: none): a block of at
  // most kv_cap keys has its rows and head constants copied into LDS by the
  // phase before (Phase::kv_issue)
  int kv_cap;
  // int8 K and V rows (Whisper's per-utterance cross K / V, both or neither):
  // channel scales [heads * hd]; kc / vc then hold int8 [head][key][hd]
  const float *k_scale, *v_scale;
};

struct MergeD {
  Vec part;
  Vec out;
  int hq, hd, max_splits, fixed_len, div_norm;
};

// FFN output, first half: this rank's slice of the hidden vector (the
// previous phase's activations, in LDS) times the matching rows of the
// output projection stored transposed, four hidden rows interleaved (wt:
// [k / 4][d][4], element (k, j) at (k / 4 * d + j) * 4 + k % 4), giving
// partial sums for all d outputs: part row b = [ranks][d].  Slices start
// on multiples of four hidden rows.
struct DpartD {
  const void *wt;  // [k / 4][d][4] int8 or bf16
  int d, k;        // outputs, hidden size
  int unit;        // projection rows per hidden element of the previous GEMV (2: GeGLU pairs)
  int m_prev;      // rows of the previous GEMV (its rank split fixes this rank's k slice)
  int act_off;     // float offset of the slice in each LDS input row (the previous GEMV's out_lds)
  Vec part;
};

// FFN output, second half: rows [r0, r1) of d (this rank's share) summed
// over the ranks' partials (in a fixed order), then scale (int8) and bias.
struct ReduceD {
  Vec part;        // [ranks][d] per row b
  int d, nparts;
  const float *scale, *bias;
  Vec out;
};

struct Phase {
  int kind;
  // >= 0: at this phase's start, copy the weight slice of GEMV phase `issue`
  // (same role, staged) into the LDS stage area; its loads then complete
  // while this phase waits for its input
  int issue;
  // >= 0: at this phase's start, copy the key/value rows and head constants
  // of attention phase `kv_issue` (this rank's first block) into the LDS
  // key/value stage
  int kv_issue;
  int pad;
  union {
    FoldD fold;
    GemvD gemv;
    AttnD attn;
    MergeD merge;
    DpartD dpart;
    ReduceD reduce;
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
  // stop rule (whisper.rs:618-668): a stream whose generated token is `stop`
  // is done (done[b], kept across launches) and is fed `stop` from then on;
  // the launch ends once every stream is done.  stop < 0: no rule.
  int stop;
  int32_t *done;
  int n_steps;
  unsigned ep0;  // epoch of step 0 (>= 1; buffers start at epoch 0)
  unsigned *status;
  uint64_t limit;  // wall-clock ticks a single wait may take
  // failure-path test hook: the end-of-step argmax wait expects an epoch this
  // many steps ahead, which never arrives, so every workgroup's wait runs
  // into its limit and the launch stops the bounded way (0: off)
  unsigned stall;
  // LDS layout (floats) of a role (A: attention side, F: FFN side):
  // residual [nb][d] | input [nb][kin] | scratch | weight stage [stage] |
  // key/value stage [kv_floats] (A) | trace marks
  int kin_a, kin_f;
  int scratch;
  int stage_a, stage_f;
  int kv_floats;
  // optional wall-clock trace of step 0: [trace_slots][grid] mark times
  // (phase ends, lm-head, argmax, embed, kernel start, phase input-ready,
  // phase sub-stages).  Marks go to LDS (after the scratch area) and are
  // copied out once at the end of the step, so tracing adds no global store
  // (whose completion a later poll would wait for) inside the step.
  uint64_t *trace;
  int trace_slots;
};

// ---------------------------------------------------------------------------
// exchange primitives
// ---------------------------------------------------------------------------
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

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

// A phase kind on a role whose step loop is not compiled with it (each
// role's loop holds only its own kinds): status 3; every other wait ends.
__device__ __forceinline__ void wrong_role(const Ctl &c) {
  __hip_atomic_store(gptr_w(c.status), 3u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  *lptr(c.bad) = 1;
}

// Byte offset past every buffer's range (num_records 0x7ffffff0): a buffer
// load there returns zeros without touching memory.
constexpr int kNoRecord = 0x7ffffff0;

// 16-byte coherent (sc1) load of pairs 2j, 2j+1 at byte offset off of base.
__device__ __forceinline__ u32x4 ld_pairs(__amdgpu_buffer_rsrc_t rs, int off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, gdev::kCoherentSc1));
}

// GEMV inputs in LDS: 16-element chunks at a 20-float stride, so the 16-byte
// reads of one chunk by consecutive lanes (80 B apart) fall in distinct
// banks; at the plain 64 B stride every fourth lane collides.
__host__ __device__ constexpr int xstride(int n) { return n / 16 * 20; }
__device__ __forceinline__ int xpad(int i) { return i + ((i >> 4) << 2); }

// Read nb rows x n pairs (n even) of v into LDS dst[b * ldd + i], polling until
// every epoch is ep.  All kT threads; ends with a barrier; WG-uniform result.
// A round holds U 16-byte loads a thread (kT * U * 2 values); the rounds run
// one after another.  pad: dst rows in the GEMV input layout (xpad).
template <int U = 4, typename V>
__device__ __forceinline__ bool get(const V &v, int nb, int n, float *dst, int ldd, unsigned ep,
                                    const Ctl &c, bool pad = false) {
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
      di[u] = b * ldd + (pad ? xpad(2 * j) : 2 * j);  // a pair never straddles a chunk
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

constexpr int kNontemporal = 2;  // cache-policy operand: nt (streamed once per step)

// A workgroup barrier for LDS hand-offs only: this wave's LDS accesses are
// complete, then s_barrier.  __syncthreads() also waits for the wave's
// global stores (its workgroup-scope fence), which after the exchange puts
// of a phase costs their write latency (~0.5 us) before anyone moves on;
// exchange data never needs that wait (readers poll epochs).
__device__ __forceinline__ void lds_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt, expcnt unconstrained
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// LDS-direct copies: kStageGran bytes a wave per load instruction.
constexpr int kStageGran = 1024;
__host__ __device__ inline int stage_pad(int bytes) { return (bytes + kStageGran - 1) / kStageGran * kStageGran; }

// bytes [0, n) of src -> LDS dst, 16 bytes a lane, kStageGran a wave per
// load; past n the loads return zeros (buffer range), so dst must hold
// stage_pad(n) bytes.
__device__ __forceinline__ void lds_copy(const void *src, int n, XE_LDS uint8_t *dst) {
  const uint64_t a = reinterpret_cast<uint64_t>(src);
  const uint64_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a)));
  const uint64_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a >> 32)));
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void *>(hi << 32 | lo), static_cast<short>(0), n, 0x00020000);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int off = wave * kStageGran; off < n; off += kW * kStageGran)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, reinterpret_cast<XE_LDS void *>(dst + off), 16, lane * 16 + off, 0,
                                             0, kNontemporal);
}

// Norm gains of a d-vector, copied into LDS (nw: stage_pad(4 d) bytes) by
// LDS-direct loads issued before the poll they follow.  The weight stream
// evicts them from the caches between layers, and values loaded into
// registers before a poll are reloaded after it by the compiler (one memory
// round trip each, on the hand-off's critical path); LDS copies are not.
// Read them after nw_ready().
__device__ __forceinline__ void pre_w(const float *w, int d, float *nw) {
  if (w != nullptr) lds_copy(w, 4 * d, reinterpret_cast<XE_LDS uint8_t *>(lptr(nw)));
}
// Every wave's copies have landed (its loads, then the barrier).
__device__ __forceinline__ void nw_ready() {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
}
// LDS floats one pre_w copy of a d-vector takes.
__host__ __device__ inline int nw_floats(int d) { return stage_pad(4 * d) / 4; }

// residual[b] += post(src[b]) for b < nb.  tmp: LDS [nb][d].
// nw: the post-norm gain as pre_w copied it (issued by the caller).
template <typename FD>
__device__ __forceinline__ bool fold(const FD &f, int nb, int d, float *xr, float *tmp, float *red,
                                     unsigned ep, const Ctl &c, const float *nw) {
  if (!get(f.src, nb, d, tmp, d, ep, c)) return false;
  if (f.post_w) nw_ready();
  const XE_LDS float *pw = lptr(nw);
  int slot = 0;
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

// The last residual fold of a GEMV's input and its RMS norm in one block
// reduction (Gemma: t = x + RMSNorm(src)(1 + post_w), then RMS(t)):
//   sum t^2 = sum x^2 + 2 inv_s sum x s' + inv_s^2 sum s'^2, s' = src (1 + post_w),
// so sum src^2, sum x^2, sum x s', sum s'^2 come out of one reduction (the
// same algebra as the phase kernels' prologue).  residual[b] = t,
// dst[b] = RMS(t) (1 + gamma) (rms1p) or RMS(t) gamma; src is read into dst.
// dst rows are GEMV inputs (xstride / xpad layout).
// nw: post_w then gamma as pre_w copied them (nw_floats(d) floats apart;
// issued by the caller).
__device__ __forceinline__ void fold_rms_rows(int nb, int d, float *xr, float *dst, float *red, float eps_s,
                                              float eps, bool rms1p, const float *nw);
template <typename FD>
__device__ __forceinline__ bool fold_rms(const FD &f, int nb, int d, float *xr, float *dst, float *red,
                                         float eps, bool rms1p, unsigned ep, const Ctl &c, const float *nw) {
  if (!get(f.src, nb, d, dst, xstride(d), ep, c, true)) return false;
  nw_ready();
  fold_rms_rows(nb, d, xr, dst, red, f.eps, eps, rms1p, nw);
  return true;
}
// The arithmetic of fold_rms once src sits in dst (eps_s: the post norm's).
__device__ __forceinline__ void fold_rms_rows(int nb, int d, float *xr, float *dst, float *red, float eps_s,
                                              float eps, bool rms1p, const float *nw) {
  const XE_LDS float *pw = lptr(nw), *gm = lptr(nw) + nw_floats(d);
  int slot = 0;
  const float fd = static_cast<float>(d);
  for (int b = 0; b < nb; b++) {
    XE_LDS float *x = lptr(xr) + static_cast<size_t>(b) * d;
    XE_LDS float *h = lptr(dst) + static_cast<size_t>(b) * xstride(d);
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int i = threadIdx.x; i < d; i += kT) {
      const float sv = h[xpad(i)], xv = x[i];
      const float spv = sv * (1.0f + pw[i]);
      acc[0] = __builtin_fmaf(sv, sv, acc[0]);
      acc[1] = __builtin_fmaf(xv, xv, acc[1]);
      acc[2] = __builtin_fmaf(xv, spv, acc[2]);
      acc[3] = __builtin_fmaf(spv, spv, acc[3]);
    }
    sums<4>(acc, red, slot);
    const float inv_s = 1.0f / sqrtf(acc[0] / fd + eps_s);
    const float st2 = acc[1] + 2.0f * inv_s * acc[2] + inv_s * inv_s * acc[3];
    const float inv_t = 1.0f / sqrtf(fmaxf(st2, 0.f) / fd + eps);
    for (int i = threadIdx.x; i < d; i += kT) {
      const float t = x[i] + h[xpad(i)] * inv_s * (1.0f + pw[i]);
      x[i] = t;
      h[xpad(i)] = rms1p ? t * inv_t * (1.0f + gm[i]) : t * inv_t * gm[i];
    }
  }
  __syncthreads();
}

// dst[b] = norm(x[b]) (LayerNorm two-pass / RMS / RMS (1 + w) / copy) as a
// GEMV input (xstride / xpad layout); nw: gamma and beta as pre_w copied
// them (2 nw_floats(d)), read after nw_ready().
__device__ __forceinline__ void norm_rows(const float *xr, int nb, int d, int norm, float eps, float *dst, float *red,
                                          const float *nw) {
  int slot = 0;
  const float fd = static_cast<float>(d);
  const XE_LDS float *gam = lptr(nw), *bet = lptr(nw) + nw_floats(d);
  for (int b = 0; b < nb; b++) {
    const XE_LDS float *x = lptr(xr) + static_cast<size_t>(b) * d;
    XE_LDS float *h = lptr(dst) + static_cast<size_t>(b) * xstride(d);
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
      for (int i = threadIdx.x; i < d; i += kT) h[xpad(i)] = (x[i] - mean) * inv * gam[i] + bet[i];
    } else if (norm == XE_NORM_RMS || norm == XE_NORM_RMS1P) {
      float v1[1] = {0.f};
      for (int i = threadIdx.x; i < d; i += kT) v1[0] = __builtin_fmaf(x[i], x[i], v1[0]);
      sums<1>(v1, red, slot);
      const float inv = 1.0f / sqrtf(v1[0] / fd + eps);
      const bool p1 = norm == XE_NORM_RMS1P;
      for (int i = threadIdx.x; i < d; i += kT) h[xpad(i)] = x[i] * inv * (p1 ? 1.0f + gam[i] : gam[i]);
    } else {
      for (int i = threadIdx.x; i < d; i += kT) h[xpad(i)] = x[i];
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

// (v, i) <- the better of (v, i) and (ov, oi).  Symmetric (NaN values and
// negative indices never win), so a butterfly leaves every lane the same pair.
__device__ __forceinline__ void arg_pick(float &v, int &i, float ov, int oi, int last_max) {
  const bool a = i >= 0 && v == v, b = oi >= 0 && ov == ov;
  if (b && (!a || sdev::better(ov, oi, v, i, last_max))) {
    v = ov;
    i = oi;
  }
}

// Wave-wide argmax of (v, i) pairs (tie rule of sdev::better); every lane
// ends with the winner, or with i < 0 when no lane holds a valid pair.
__device__ __forceinline__ void wave_argbest(float &v, int &i, int last_max) {
  if (!(i >= 0 && v == v)) i = -1;
  arg_pick(v, i, gdev::dpp_get<gdev::kDppXor1>(v), gdev::dpp_get_i<gdev::kDppXor1>(i), last_max);
  arg_pick(v, i, gdev::dpp_get<gdev::kDppXor2>(v), gdev::dpp_get_i<gdev::kDppXor2>(i), last_max);
  arg_pick(v, i, gdev::dpp_get<gdev::kDppHalfMirror>(v), gdev::dpp_get_i<gdev::kDppHalfMirror>(i), last_max);
  arg_pick(v, i, gdev::dpp_get<gdev::kDppMirror>(v), gdev::dpp_get_i<gdev::kDppMirror>(i), last_max);
  {
    const auto rv = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    const auto ri = __builtin_amdgcn_permlane16_swap(static_cast<unsigned>(i), static_cast<unsigned>(i), false, false);
    v = __uint_as_float(rv[0]);
    i = static_cast<int>(ri[0]);
    arg_pick(v, i, __uint_as_float(rv[1]), static_cast<int>(ri[1]), last_max);
  }
  {
    const auto rv = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    const auto ri = __builtin_amdgcn_permlane32_swap(static_cast<unsigned>(i), static_cast<unsigned>(i), false, false);
    v = __uint_as_float(rv[0]);
    i = static_cast<int>(ri[0]);
    arg_pick(v, i, __uint_as_float(rv[1]), static_cast<int>(ri[1]), last_max);
  }
}

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

// ---------------------------------------------------------------------------
// LDS weight stage.  A staged GEMV phase's slice (this rank's rows [r0, r1))
// is copied into LDS by LDS-direct buffer loads issued at the start of an
// earlier phase of the role, so the phase itself finds its weights on chip
// when its input arrives: its hand-off wait no longer includes a memory round
// trip for weights issued after the previous phase.  Layout (bytes, each
// part padded to kStageGran, the span one wave moves per load):
// zero slot [kStageZero] | weights [rows][row bytes] | bfp16 exponents
// [rows][k / 8] | scale [rows] | bias [rows].
// ---------------------------------------------------------------------------
constexpr int kStageZero = 64;  // zero slot at the stage's start (chunks not valid read it)

struct StageLayout {
  int w, e, s, b, total;  // byte offsets of the parts and the padded size
};


__host__ __device__ inline StageLayout stage_layout(int wt, int rows, int k, bool bias) {
  StageLayout L;
  const int rb = wt == XE_BF16 ? 2 * k : k;
  L.w = kStageZero;
  L.e = L.w + stage_pad(rows * rb);
  L.s = L.e + (wt == XE_BFP16 ? stage_pad(rows * (k / 8)) : 0);
  L.b = L.s + (wt == XE_I8 ? stage_pad(rows * 4) : 0);
  L.total = L.b + (bias ? stage_pad(rows * 4) : 0);
  return L;
}

// Issue the copies of GEMV g's rows [r0, r1) into the stage area.  The
// caller has passed a block barrier since the stage's last reader.
template <int WT, typename GD>
__device__ __forceinline__ void stage_issue(const GD &g, int r0, int r1, float *stage) {
  if (r1 <= r0) return;
  const int rows = r1 - r0;
  const StageLayout L = stage_layout(WT, rows, g.k, g.bias != nullptr);
  XE_LDS uint8_t *st = reinterpret_cast<XE_LDS uint8_t *>(lptr(stage));
  const int rb = WT == XE_BF16 ? 2 * g.k : g.k;
  lds_copy(static_cast<const uint8_t *>(g.w) + static_cast<size_t>(r0) * rb, rows * rb, st + L.w);
  if (WT == XE_BFP16) lds_copy(g.exps + static_cast<size_t>(r0) * (g.k / 8), rows * (g.k / 8), st + L.e);
  if (WT == XE_I8) lds_copy(g.scale + r0, rows * 4, st + L.s);
  if (g.bias) lds_copy(g.bias + r0, rows * 4, st + L.b);
}

// One weight chunk from the stage: rw = byte offset of the row's weights
// (and re = of its exponents) within their parts; a chunk that is not valid
// reads the stage's zero slot (a select on the address, so the data goes
// straight into the registers the dot products read).
template <int WT>
__device__ __forceinline__ void load_chunk_lds(const XE_LDS uint8_t *st, const StageLayout &L, int rw, int re, int c,
                                               bool valid, gdev::Chunk<WT> &out) {
  auto u4 = [](u32x4 v) { return make_uint4(v.x, v.y, v.z, v.w); };
  if constexpr (WT == XE_BF16) {
    const XE_LDS u32x4 *p = reinterpret_cast<const XE_LDS u32x4 *>(st + (valid ? L.w + rw + c * 32 : 0));
    out.lo = u4(p[0]);
    out.hi = u4(p[1]);
  } else {
    out.q = u4(*reinterpret_cast<const XE_LDS u32x4 *>(st + (valid ? L.w + rw + c * 16 : 0)));
    if constexpr (WT == XE_BFP16)
      out.e = *reinterpret_cast<const XE_LDS uint16_t *>(st + (valid ? L.e + re + c * 2 : 0));
  }
}

// a[j] += dot(chunk elements 4 j .. 4 j + 3, x): four independent chains
// (bfp16: one per exponent half), so consecutive FMAs do not wait on each
// other.
template <int WT>
__device__ __forceinline__ void chunk_dot4(const gdev::Chunk<WT> &ch, const float4 (&xv)[4], float (&a)[4]) {
  using gdev::sb;
  if constexpr (WT == XE_I8) {
    const uint32_t w4[4] = {ch.q.x, ch.q.y, ch.q.z, ch.q.w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      a[j] = __builtin_fmaf(xv[j].x, sb(w4[j], 0), a[j]);
      a[j] = __builtin_fmaf(xv[j].y, sb(w4[j], 1), a[j]);
      a[j] = __builtin_fmaf(xv[j].z, sb(w4[j], 2), a[j]);
      a[j] = __builtin_fmaf(xv[j].w, sb(w4[j], 3), a[j]);
    }
  } else if constexpr (WT == XE_BFP16) {
    const uint32_t w4[4] = {ch.q.x, ch.q.y, ch.q.z, ch.q.w};
#pragma unroll
    for (int h = 0; h < 2; h++) {
      float d = 0.f;
#pragma unroll
      for (int i = 2 * h; i < 2 * h + 2; i++) {
        d = __builtin_fmaf(xv[i].x, sb(w4[i], 0), d);
        d = __builtin_fmaf(xv[i].y, sb(w4[i], 1), d);
        d = __builtin_fmaf(xv[i].z, sb(w4[i], 2), d);
        d = __builtin_fmaf(xv[i].w, sb(w4[i], 3), d);
      }
      const int e = static_cast<int>((ch.e >> (8 * h)) & 0xff) - 133;  // e - 127 - 6
      a[h] += __builtin_ldexpf(d, e);
    }
  } else {
    const uint32_t w8[8] = {ch.lo.x, ch.lo.y, ch.lo.z, ch.lo.w, ch.hi.x, ch.hi.y, ch.hi.z, ch.hi.w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t p = w8[2 * j], q = w8[2 * j + 1];
      a[j] = __builtin_fmaf(xv[j].x, __uint_as_float(p << 16), a[j]);
      a[j] = __builtin_fmaf(xv[j].y, __uint_as_float(p & 0xffff0000u), a[j]);
      a[j] = __builtin_fmaf(xv[j].z, __uint_as_float(q << 16), a[j]);
      a[j] = __builtin_fmaf(xv[j].w, __uint_as_float(q & 0xffff0000u), a[j]);
    }
  }
}

// ST: 1 / 0 compiles only the staged / streamed weight path (-1: staged_rt
// decides at run time); TAIL: false compiles the tail K split out.
template <int WT, int NB, bool HEAD, typename GD, typename Prep, typename Sub, int ST = -1, bool TAIL = true>
__device__ __forceinline__ bool gemv_rows(const GD &g, int nb, int r0, int r1, const float *xs, unsigned ep,
                                          Prep prep, float *logits, int vocab, int last_max, ArgBest &best,
                                          Sub tsub, const float *stage, bool staged_rt, float *kred, float *lout,
                                          int lout_ld) {
  using gdev::Chunk;
  const bool staged = ST >= 0 ? ST != 0 : staged_rt;
  constexpr int RPL = 2;
  constexpr int NIT = Round<WT>::NIT;
  const int lpr_log = __builtin_ctz(static_cast<unsigned>(g.lpr));
  const int LPR = 1 << lpr_log;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rg = lane >> lpr_log, kl = lane & (LPR - 1);
  // K segments (the tail split below): wave w takes segment seg of the
  // chunks for the rows of its group wgrp
  int S = 1;
  int seg = 0, wgrp = wave;
  const int rows_per_wave = (64 >> lpr_log) * RPL;
  const int rows_per_tile = kW * rows_per_wave;
  // Tail split: waves w and w + 4 share SIMD w % 4 (the older wave issues
  // first), so in one tile of 5 or 6 row groups (one a wave) the waves past
  // the fourth finish last, with their SIMD's other wave's work on top.
  // Waves 0..3 keep groups 0..3; waves 4..7 share the rest, each taking a K
  // segment (one group: quarters, two: halves); the segment sums meet in LDS.
  const int rpw_log = 7 - lpr_log;  // log2(rows_per_wave): RPL = 2
  const int nrg = (r1 - r0 + rows_per_wave - 1) >> rpw_log;
  const int tail = (TAIL && !HEAD && g.tail_split && (nrg == 5 || nrg == 6)) ? nrg - 4 : 0;
  if (tail > 0 && wave >= 4) {
    S = tail == 1 ? 4 : 2;
    seg = (wave - 4) & (S - 1);
    wgrp = 4 + ((wave - 4) >> (tail == 1 ? 2 : 1));
  }
  const int K = g.k, nch = K / 16;
  const int s_log = S == 4 ? 2 : S == 2 ? 1 : 0;
  const int seg_ch = (nch + S - 1) >> s_log;
  const int c_lo = seg * seg_ch, c_hi = min(nch, c_lo + seg_ch);
  const int n_it = (seg_ch + LPR - 1) >> lpr_log;
  const int ntiles = r1 > r0 ? (r1 - r0 + rows_per_tile - 1) >> (rpw_log + 3) : 0;
  const bool ksum = tail > 0;  // some wave holds a K segment
  WRsrc rs;
  rs.w = gdev::coherent_rsrc(g.w);
  rs.e = gdev::coherent_rsrc(WT == XE_BFP16 ? static_cast<const void *>(g.exps) : g.w);
  const XE_LDS uint8_t *st = reinterpret_cast<const XE_LDS uint8_t *>(lptr(stage));
  const StageLayout L = stage_layout(WT, r1 - r0, K, g.bias != nullptr);
  bool ok = true;
  if (ntiles == 0) return prep();
  if (staged) {
    ok = prep();
    // every wave's stage copies have landed (its own loads, then the barrier)
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  for (int tile = 0; tile < ntiles && ok; tile++) {
    const int row0 = r0 + tile * rows_per_tile + wgrp * rows_per_wave + rg * RPL;
    bool row_ok[RPL];
    int row[RPL];
#pragma unroll
    for (int i = 0; i < RPL; i++) {
      row[i] = row0 + i;
      row_ok[i] = row[i] < r1;
    }
    // stage offsets of the rows (a row past the slice reads row 0, zeroed)
    int rw[RPL], re[RPL];
#pragma unroll
    for (int i = 0; i < RPL; i++) {
      const int lr = row_ok[i] ? row[i] - r0 : 0;
      rw[i] = lr * (WT == XE_BF16 ? 2 * K : K);
      re[i] = lr * (K / 8);
    }
    float acc4[NB][RPL][4];
    float rscale[RPL], rbias[RPL];
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
      for (int i = 0; i < RPL; i++)
#pragma unroll
        for (int q = 0; q < 4; q++) acc4[b][i][q] = 0.f;
    for (int it0 = 0; it0 < n_it && ok; it0 += NIT) {
      Chunk<WT> w[NIT][RPL];
      // one branch around the whole round: inside a branch per chunk the
      // compiler waits for each chunk's reads before the next
      if (staged) {
#pragma unroll
        for (int u = 0; u < NIT; u++) {
          const int cc = c_lo + ((it0 + u) << lpr_log) + kl;
          const bool valid = it0 + u < n_it && cc < c_hi;
#pragma unroll
          for (int i = 0; i < RPL; i++) load_chunk_lds<WT>(st, L, rw[i], re[i], cc, valid && row_ok[i], w[u][i]);
        }
      } else {
#pragma unroll
        for (int u = 0; u < NIT; u++) {
          const int cc = c_lo + ((it0 + u) << lpr_log) + kl;
          const bool valid = it0 + u < n_it && cc < c_hi;
#pragma unroll
          for (int i = 0; i < RPL; i++) load_chunk_buf<WT>(rs, row[i], K, cc, valid && row_ok[i], w[u][i]);
        }
      }
      if (it0 == 0) {  // epilogue constants travel with the first round's loads
#pragma unroll
        for (int i = 0; i < RPL; i++) {
          const int rr = row_ok[i] ? row[i] : r0;
          if (staged) {
            rscale[i] = WT == XE_I8 ? reinterpret_cast<const XE_LDS float *>(st + L.s)[rr - r0] : 1.0f;
            rbias[i] = g.bias ? reinterpret_cast<const XE_LDS float *>(st + L.b)[rr - r0] : 0.0f;
          } else {
            rscale[i] = WT == XE_I8 ? gptr(g.scale)[rr] : 1.0f;
            rbias[i] = g.bias ? gptr(g.bias)[rr] : 0.0f;
          }
        }
      }
      if (tile == 0 && it0 == 0 && !staged) ok = prep();
      if (!ok) break;
      // every row of the NB tile (rows past nb hold unused values): a
      // branch on nb per chunk costs more than the FMAs it would skip
#pragma unroll
      for (int u = 0; u < NIT; u++) {
        if (it0 + u < n_it) {
          const int cx = min(c_lo + ((it0 + u) << lpr_log) + kl, nch - 1);  // past the segment: zero weights
#pragma unroll
          for (int b = 0; b < NB; b++) {
            typedef float f32x4 __attribute__((ext_vector_type(4)));
            float4 xv[4];
            const XE_LDS f32x4 *xr =
                reinterpret_cast<const XE_LDS f32x4 *>(lptr(xs) + static_cast<size_t>(b) * xstride(K) + cx * 20);
#pragma unroll
            for (int j = 0; j < 4; j++) {
              const f32x4 t = xr[j];
              xv[j] = make_float4(t.x, t.y, t.z, t.w);
            }
#pragma unroll
            for (int i = 0; i < RPL; i++) chunk_dot4<WT>(w[u][i], xv, acc4[b][i]);
          }
        }
      }
    }
    if (!ok) break;
    if (tile == 0) tsub(1);
    float acc[NB][RPL];
    {
      float flat[NB * RPL];
#pragma unroll
      for (int b = 0; b < NB; b++)
#pragma unroll
        for (int i = 0; i < RPL; i++)
          flat[b * RPL + i] = (acc4[b][i][0] + acc4[b][i][1]) + (acc4[b][i][2] + acc4[b][i][3]);
      gdev::group_sums<NB * RPL>(flat, lpr_log);
#pragma unroll
      for (int b = 0; b < NB; b++)
#pragma unroll
        for (int i = 0; i < RPL; i++) acc[b][i] = flat[b * RPL + i];
    }
    if (ksum) {  // segment sums in LDS, added in segment order by the segment-0 waves
      XE_LDS float *kr = lptr(kred);
      const int slot = wgrp * rows_per_wave + rg * RPL;
      if (kl == 0)
#pragma unroll
        for (int i = 0; i < RPL; i++)
#pragma unroll
          for (int b = 0; b < NB; b++) kr[((seg * rows_per_tile) + slot + i) * NB + b] = acc[b][i];
      __syncthreads();
      if (seg == 0 && kl == 0)
#pragma unroll
        for (int i = 0; i < RPL; i++)
#pragma unroll
          for (int b = 0; b < NB; b++) {
            float t = kr[(slot + i) * NB + b];
            for (int sg = 1; sg < S; sg++) t += kr[((sg * rows_per_tile) + slot + i) * NB + b];
            acc[b][i] = t;
          }
      __syncthreads();  // the next tile's sums overwrite these
    }
    if (kl == 0 && seg == 0) {
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
          const float t = gdev::gelu_tanh(v[0]) * v[1];
          if (row_ok[0]) {
            if (g.out_lds) lptr(lout)[b * lout_ld + (row[0] - r0) / 2] = t;
            else put(g.out, b, row[0] / 2, t, ep);
          }
        } else {
#pragma unroll
          for (int i = 0; i < RPL; i++) {
            if (!row_ok[i]) continue;
            float t = v[i];
            if (g.act == ACT_RELU) t = t > 0.f ? t : 0.f;
            else if (g.act == ACT_GELU_ERF) t = gdev::gelu_erf(t);
            if (g.out_lds) lptr(lout)[b * lout_ld + row[i] - r0] = t;
            else put(g.out, b, row[i], t, ep);
          }
        }
      }
    }
    if (tile == 0) tsub(2);  // outputs issued
  }
  return ok;
}

template <int WT, int NB, bool HEAD, typename GD, typename Prep, typename Sub>
__device__ __forceinline__ bool gemv_any(const GD &g, int nb, int r0, int r1, const float *xs, unsigned ep,
                                         Prep prep, float *logits, int vocab, int last_max, ArgBest &best,
                                         const Ctl &c, Sub tsub, const float *stage = nullptr,
                                         bool staged = false, float *kred = nullptr, float *lout = nullptr,
                                         int lout_ld = 0) {
  (void)c;
  return gemv_rows<WT, NB, HEAD>(g, nb, r0, r1, xs, ep, prep, logits, vocab, last_max, best, tsub, stage, staged,
                                 kred, lout, lout_ld);
}

// The lm-head slice with its tiles pipelined: tile t + 1's weight chunks are
// requested before tile t's dot products, so the weight stream does not stop
// for a memory round trip at every tile (gemv_rows issues a tile's loads only
// after the previous tile is done).  For a head whose rows take one load
// round (n_it <= NIT chunk iterations a lane).  One row a lane group (gemv_rows
// takes two), so the two tiles in flight hold the registers of one of its
// tiles: more would raise the step kernel's spills around this call.  Each
// row's arithmetic is gemv_rows' HEAD path (same chunks in the same order,
// the same lane sums, scale and tie rule), so the logits and the argmax are
// bit-identical to it.  The tied head has no bias.  Tiles past the slice
// load zeros (rows past r1 read nothing).
template <int WT>
__host__ __device__ constexpr bool head_one_round(int k, int lpr) {
  return (k / 16 + lpr - 1) / lpr <= Round<WT>::NIT;
}

template <int WT, int NB, typename GD, typename Prep>
__device__ __forceinline__ bool head_rows(const GD &g, int nb, int r0, int r1, const float *xs, Prep prep,
                                          float *logits, int vocab, int last_max, ArgBest &best) {
  using gdev::Chunk;
  constexpr int RPL = 1;
  constexpr int NIT = Round<WT>::NIT;
  const int lpr_log = __builtin_ctz(static_cast<unsigned>(g.lpr));
  const int LPR = 1 << lpr_log;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rg = lane >> lpr_log, kl = lane & (LPR - 1);
  const int rows_per_wave = (64 >> lpr_log) * RPL;
  const int K = g.k, nch = K / 16;
  const int n_it = (nch + LPR - 1) >> lpr_log;
  // wave tiles: a wave's rows_per_wave rows at a time
  const int nwt = r1 > r0 ? (r1 - r0 + rows_per_wave - 1) >> (6 - lpr_log) : 0;
  if (nwt == 0) return prep();
  WRsrc rs;
  rs.w = gdev::coherent_rsrc(g.w);
  rs.e = gdev::coherent_rsrc(WT == XE_BFP16 ? static_cast<const void *>(g.exps) : g.w);
  struct TileW {
    Chunk<WT> w[NIT][RPL];
    float scale[RPL];
  };
  auto first_row = [&](int wt) { return r0 + wt * rows_per_wave + rg * RPL; };
  auto load_tile = [&](int tile, TileW &t) {
    const int row0 = first_row(tile);
#pragma unroll
    for (int u = 0; u < NIT; u++) {
      const int cc = (u << lpr_log) + kl;
      const bool valid = u < n_it && cc < nch;
#pragma unroll
      for (int i = 0; i < RPL; i++) load_chunk_buf<WT>(rs, row0 + i, K, cc, valid && row0 + i < r1, t.w[u][i]);
    }
#pragma unroll
    for (int i = 0; i < RPL; i++) t.scale[i] = WT == XE_I8 ? gptr(g.scale)[row0 + i < r1 ? row0 + i : r0] : 1.0f;
  };
  auto compute_tile = [&](int tile, const TileW &t) {
    const int row0 = first_row(tile);
    float acc4[NB][RPL][4];
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
      for (int i = 0; i < RPL; i++)
#pragma unroll
        for (int q = 0; q < 4; q++) acc4[b][i][q] = 0.f;
#pragma unroll
    for (int u = 0; u < NIT; u++) {
      if (u < n_it) {
        const int cx = min((u << lpr_log) + kl, nch - 1);
#pragma unroll
        for (int b = 0; b < NB; b++) {
          typedef float f32x4 __attribute__((ext_vector_type(4)));
          float4 xv[4];
          const XE_LDS f32x4 *xr =
              reinterpret_cast<const XE_LDS f32x4 *>(lptr(xs) + static_cast<size_t>(b) * xstride(K) + cx * 20);
#pragma unroll
          for (int j = 0; j < 4; j++) {
            const f32x4 v = xr[j];
            xv[j] = make_float4(v.x, v.y, v.z, v.w);
          }
#pragma unroll
          for (int i = 0; i < RPL; i++) chunk_dot4<WT>(t.w[u][i], xv, acc4[b][i]);
        }
      }
    }
    float flat[NB * RPL];
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
      for (int i = 0; i < RPL; i++)
        flat[b * RPL + i] = (acc4[b][i][0] + acc4[b][i][1]) + (acc4[b][i][2] + acc4[b][i][3]);
    gdev::group_sums<NB * RPL>(flat, lpr_log);
    if (kl == 0) {
#pragma unroll
      for (int b = 0; b < NB; b++) {
        if (b >= nb) break;
#pragma unroll
        for (int i = 0; i < RPL; i++) {
          const int row = row0 + i;
          if (row >= r1) continue;
          float v = flat[b * RPL + i];
          if (WT == XE_I8) v = v * t.scale[i];
          if (logits) gptr_w(logits)[static_cast<size_t>(b) * vocab + row] = v;
          if (sdev::better(v, row, best.v[b], best.i[b], last_max)) {
            best.v[b] = v;
            best.i[b] = row;
          }
        }
      }
    }
  };
  // Wave tiles are handed out one at a time from an LDS counter: each wave
  // starts with tile `wave`, then takes the next free one, so the waves of a
  // SIMD pair (the older one issues first) stream until the slice is done
  // instead of the younger ones finishing alone (with equal static shares
  // the last wave of a workgroup ended ~6 us after its first).  Every row is
  // computed as before; the argmax order is total, so neither the logits nor
  // the winner depend on which wave takes a row.
  __shared__ int s_next;
  auto grab = [&]() -> int {
    int v = 0;
    if (lane == 0) v = __hip_atomic_fetch_add(&s_next, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    return __builtin_amdgcn_readfirstlane(v);
  };
  if (threadIdx.x == 0) s_next = kW;
  TileW ta, tb;
  int cur = wave;
  load_tile(cur, ta);         // tiles past the slice read nothing
  if (!prep()) return false;  // the final norm overlaps the first tile's loads; its barrier orders s_next
  while (cur < nwt) {
    const int nxt = grab();
    load_tile(nxt, tb);
    compute_tile(cur, ta);
    if (nxt >= nwt) break;
    const int nn = grab();
    load_tile(nn, ta);
    compute_tile(nxt, tb);
    cur = nn;
  }
  return true;
}

struct NoSub {
  __device__ void operator()(int) const {}
};

// Rows of rank r out of n ranks (balanced contiguous split).  Every phase
// computes its rows after its input arrives: the 32-bit quotient where the
// products fit (every plan here) is a fraction of the 64-bit one's
// instructions.
__device__ __forceinline__ void rank_rows(int m, int r, int n, int &r0, int &r1) {
  if (static_cast<unsigned>(m) * static_cast<unsigned>(n) < (1u << 31)) {
    r0 = static_cast<int>(static_cast<unsigned>(m * r) / static_cast<unsigned>(n));
    r1 = static_cast<int>(static_cast<unsigned>(m * (r + 1)) / static_cast<unsigned>(n));
    return;
  }
  r0 = static_cast<int>((static_cast<long long>(m) * r) / n);
  r1 = static_cast<int>((static_cast<long long>(m) * (r + 1)) / n);
}

// ---------------------------------------------------------------------------
// FFN output in two phases (LK_DPART, LK_REDUCE): each rank multiplies its
// slice of the hidden vector, left in LDS by the GEMV before, by the
// matching rows of the transposed output projection, and puts partial sums
// for every output; the ranks then sum those partials for their own share of
// the outputs.  The exchange between the two carries one value per output
// and rank instead of the whole hidden vector to every rank.
// ---------------------------------------------------------------------------
// The hidden slice [k0, k1) of this rank (the previous GEMV's rows / unit).
template <typename DD>
__device__ __forceinline__ void dpart_slice(const DD &dp, int rank, int nranks, int &k0, int &k1) {
  rank_rows(dp.m_prev / (dp.unit * 4), rank, nranks, k0, k1);
  k0 *= 4;
  k1 *= 4;
}

// Copy rows [k0, k1) of wt into the stage (after kStageZero).
template <int WT, typename DD>
__device__ __forceinline__ void dpart_stage_issue(const DD &dp, int k0, int k1, float *stage) {
  if (k1 <= k0) return;
  const int rb = (WT == XE_BF16 ? 2 : 1) * dp.d;
  lds_copy(static_cast<const uint8_t *>(dp.wt) + static_cast<size_t>(k0) * rb, (k1 - k0) * rb,
           reinterpret_cast<XE_LDS uint8_t *>(lptr(stage)) + kStageZero);
}

// partial[b][r] = sum over k < kn of wt[k0 + k][r] act[b][k] (act: LDS,
// 16-byte aligned, row stride act_ld a multiple of 4; kn a multiple of 4).
// A lane takes four consecutive outputs, four k at a time: one 16-byte
// (int8) or 32-byte (bf16) read of the interleaved stage and one broadcast
// read of the activations, the next group's reads issued before this
// group's FMAs.  The results go through LDS (obuf) so the puts run
// consecutive lanes over consecutive outputs.
template <int WT>
struct DpW {
  u32x4 a, b;  // b: bf16 only
};
template <int WT>
__device__ __forceinline__ void dpart_ld(const XE_LDS uint8_t *w, int elem, DpW<WT> &o) {
  const XE_LDS u32x4 *p = reinterpret_cast<const XE_LDS u32x4 *>(w + elem * (WT == XE_BF16 ? 2 : 1));
  o.a = p[0];
  if constexpr (WT == XE_BF16) o.b = p[1];
}
// weight of output e (of the lane's four), hidden row kk (of the group's four)
template <int WT>
__device__ __forceinline__ float dpart_wv(const DpW<WT> &v, int e, int kk) {
  if constexpr (WT == XE_BF16) {
    const int idx = e * 4 + kk;
    const uint32_t d = idx < 8 ? v.a[idx / 2] : v.b[(idx - 8) / 2];
    return __uint_as_float(idx & 1 ? d & 0xffff0000u : d << 16);
  } else {
    return gdev::sb(v.a[e], kk);
  }
}

// Lanes per SIMD: waves w and w + 4 share SIMD w % 4, so work is balanced
// across SIMDs when threads [0, 256) and [256, 512) carry equal shares.  The
// first quads go 256 to a pass over all kn (threads t and t + 256 alike
// after an even number of passes); the remaining tq < 256 quads are split
// into S segments of the k groups over the threads with one pass fewer, each
// segment's partial summed in segment order before the put.
struct DpartMap {
  int hq, tq, tb, S;
};
__device__ __forceinline__ DpartMap dpart_map(int d, int kn) {
  DpartMap m;
  const int nq = d / 4, ng = kn / 4;
  m.hq = nq / 256 * 256;
  m.tq = nq - m.hq;
  const int L = (m.hq / 256) % 2 ? kT - 256 : kT;
  m.tb = kT - L;
  m.S = m.tq > 0 ? max(1, min(L / m.tq, ng)) : 1;
  return m;
}
__host__ __device__ inline int dpart_obuf_floats(int nb, int d) { return nb * (d + 4 * kT); }

// acc[b][e] += sum over groups [g0, g1) (quad q), two groups a step with
// the next group's reads in flight during each group's FMAs.  Every row of
// the NB tile is computed (rows past nb hold unused values): a branch on nb
// inside the loop costs more than the FMAs it would skip.
template <int WT, int NB>
__device__ __forceinline__ void dpart_groups(const XE_LDS uint8_t *w, const XE_LDS float *a, int act_ld, int D,
                                             int q, int g0, int g1, float (&acc)[NB][4]) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  auto ld = [&](int g, DpW<WT> &wv, f4 (&xv)[NB]) {
    dpart_ld<WT>(w, (g * D + 4 * q) * 4, wv);
#pragma unroll
    for (int b = 0; b < NB; b++) xv[b] = *reinterpret_cast<const XE_LDS f4 *>(a + b * act_ld + 4 * g);
  };
  auto comp = [&](const DpW<WT> &wv, const f4 (&xv)[NB]) {
#pragma unroll
    for (int kk = 0; kk < 4; kk++) {
      float wf[4];
#pragma unroll
      for (int e = 0; e < 4; e++) wf[e] = dpart_wv<WT>(wv, e, kk);
#pragma unroll
      for (int b = 0; b < NB; b++)
#pragma unroll
        for (int e = 0; e < 4; e++) acc[b][e] = __builtin_fmaf(wf[e], xv[b][kk], acc[b][e]);
    }
  };
  if (g1 <= g0) return;
  DpW<WT> wa, wb;
  f4 xa[NB], xb[NB];
  ld(g0, wa, xa);
  int g = g0;
  for (; g + 2 <= g1; g += 2) {
    ld(g + 1, wb, xb);
    comp(wa, xa);
    if (g + 2 < g1) ld(g + 2, wa, xa);
    comp(wb, xb);
  }
  if (g < g1) comp(wa, xa);
}

template <int WT, int NB, typename DD, typename TS>
__device__ __forceinline__ void dpart_block(const DD &dp, int nb, int kn, const float *act, int act_ld,
                                            const float *stage, float *obuf, int rank, unsigned ep, TS &&tsub) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  const XE_LDS uint8_t *w = reinterpret_cast<const XE_LDS uint8_t *>(lptr(stage)) + kStageZero;
  const XE_LDS float *a = lptr(act);
  XE_LDS float *o = lptr(obuf);
  const int D = dp.d, ng = kn / 4;
  const DpartMap m = dpart_map(D, kn);
  XE_LDS float *tp = o + nb * D;  // tail partials [S][nb][tq][4]
  for (int q = threadIdx.x; q < m.hq; q += kT) {
    float acc[NB][4];
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
      for (int e = 0; e < 4; e++) acc[b][e] = 0.f;
    dpart_groups<WT, NB>(w, a, act_ld, D, q, 0, ng, acc);
#pragma unroll
    for (int b = 0; b < NB; b++)
      if (b < nb) *reinterpret_cast<XE_LDS f4 *>(o + b * D + 4 * q) = f4{acc[b][0], acc[b][1], acc[b][2], acc[b][3]};
  }
  {
    const int it = static_cast<int>(threadIdx.x) - m.tb;
    if (it >= 0 && it < m.tq * m.S) {
      const int qi = it % m.tq, sg = it / m.tq;
      float acc[NB][4];
#pragma unroll
      for (int b = 0; b < NB; b++)
#pragma unroll
        for (int e = 0; e < 4; e++) acc[b][e] = 0.f;
      dpart_groups<WT, NB>(w, a, act_ld, D, m.hq + qi, sg * ng / m.S, (sg + 1) * ng / m.S, acc);
#pragma unroll
      for (int b = 0; b < NB; b++)
        if (b < nb)
          *reinterpret_cast<XE_LDS f4 *>(tp + ((sg * nb + b) * m.tq + qi) * 4) =
              f4{acc[b][0], acc[b][1], acc[b][2], acc[b][3]};
    }
  }
  tsub(1);
  __syncthreads();
  tsub(2);
  for (int t = threadIdx.x; t < nb * D; t += kT) {
    const int b = t / D, r = t - b * D;
    float v;
    if (r < 4 * m.hq) {
      v = o[t];
    } else {
      const int ri = r - 4 * m.hq;
      v = tp[(b * m.tq) * 4 + ri];
      for (int sg = 1; sg < m.S; sg++) v += tp[((sg * nb + b) * m.tq) * 4 + ri];
    }
    put(dp.part, b, rank * D + r, v, ep);
  }
}

// Rows [r0, r1) of the FFN output: the nparts ranks' partials summed, times
// scale (int8 weights), plus bias.  Lane t polls parts p = t / kRedRows + i
// * (kT / kRedRows) of row j = t % kRedRows and adds them in i order; the
// lanes of a row meet by lane swaps (fixed pattern), the waves in LDS (wave
// order).  tab: LDS >= kW * NB * kRedRows + 2 * 256 floats.
constexpr int kRedRows = 8;      // output rows a rank sums (at most)
constexpr int kRedParts = 256;   // partials per output (at most)
template <int NB, typename RD, typename TS>
__device__ __forceinline__ bool reduce_block(const RD &rd, int nb, int r0, int r1, float *tab_, unsigned ep,
                                             const Ctl &c, TS &&tsub) {
  XE_LDS float *wsum = lptr(tab_);                    // [kW][NB][kRedRows]
  XE_LDS float *sb_ = wsum + kW * NB * kRedRows;      // scale | bias (aligned blocks)
  const int nr = r1 - r0, np = rd.nparts;
  // scale / bias of the rows: the 16-byte blocks holding them, copied into
  // LDS ahead of the poll
  const int a0 = r0 & ~3;
  if (rd.scale != nullptr) lds_copy(rd.scale + a0, (r1 - a0) * 4, reinterpret_cast<XE_LDS uint8_t *>(sb_));
  if (rd.bias != nullptr) lds_copy(rd.bias + a0, (r1 - a0) * 4, reinterpret_cast<XE_LDS uint8_t *>(sb_ + 256));
  constexpr int PI = kRedParts * kRedRows / kT;  // polls per lane and batch row
  constexpr int NI = NB * PI;
  const int j = threadIdx.x & (kRedRows - 1), p0 = threadIdx.x / kRedRows;
  int idx[NI];
  bool need[NI];
  float got[NI];
#pragma unroll
  for (int b = 0; b < NB; b++)
#pragma unroll
    for (int i = 0; i < PI; i++) {
      const int p = p0 + i * (kT / kRedRows);
      need[b * PI + i] = j < nr && p < np && b < nb;
      idx[b * PI + i] = need[b * PI + i] ? b * rd.part.ld + p * rd.d + r0 + j : 0;
      got[b * PI + i] = 0.f;
    }
  const bool okp = get_scattered<NI>(rd.part.p, idx, need, got, ep, c);
  if (!okp) raise_stop(c);
  tsub(1);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int b = 0; b < NB; b++) {
    if (b >= nb) break;
    float v = got[b * PI];
#pragma unroll
    for (int i = 1; i < PI; i++) v += got[b * PI + i];
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, true));  // row_ror:8
    auto swap_add = [](float x, bool half32) {
      const auto r = half32 ? __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false)
                            : __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
      return __uint_as_float(r[0]) + __uint_as_float(r[1]);
    };
    v = swap_add(swap_add(v, false), true);
    if (lane < kRedRows) wsum[(wave * NB + b) * kRedRows + lane] = v;
  }
  __builtin_amdgcn_s_waitcnt(0);  // the scale / bias copies (and every wave's, after the barrier)
  __syncthreads();
  if (*lptr(c.bad)) return false;
  if (threadIdx.x < nb * kRedRows) {
    const int b = threadIdx.x / kRedRows, jj = threadIdx.x % kRedRows;
    if (jj < nr) {
      float ws[kW];  // every wave's read first, then the sum in wave order
#pragma unroll
      for (int w = 0; w < kW; w++) ws[w] = wsum[(w * NB + b) * kRedRows + jj];
      float t = 0.f;
#pragma unroll
      for (int w = 0; w < kW; w++) t += ws[w];
      if (rd.scale != nullptr) t *= sb_[r0 - a0 + jj];
      if (rd.bias != nullptr) t += sb_[256 + r0 - a0 + jj];
      put(rd.out, b, r0 + jj, t, ep);
    }
  }
  lds_barrier();
  return true;
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

// The same constants from the key/value stage (after its copies landed).
template <int HD, typename AD>
__device__ __forceinline__ void load_head_consts_lds(const AD &a, const float *kvs, HeadConsts<HD> &hc) {
  constexpr int HALF = HeadConsts<HD>::HALF, PER = HeadConsts<HD>::PER;
  constexpr int SLOT = kStageGran / 4;
  const XE_LDS float *k = lptr(kvs);
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < PER; i++) {
    const int j = min(lane + 64 * i, HALF - 1);
    hc.qn0[i] = a.q_norm_w ? k[j] : 0.f;
    hc.qn1[i] = a.q_norm_w ? k[j + HALF] : 0.f;
    hc.kn0[i] = a.k_norm_w ? k[SLOT + j] : 0.f;
    hc.kn1[i] = a.k_norm_w ? k[SLOT + j + HALF] : 0.f;
    hc.cs[i] = a.rope_cos ? k[2 * SLOT + j] : 1.f;
    hc.sn[i] = a.rope_sin ? k[3 * SLOT + j] : 0.f;
  }
}

// Per-head RMSNorm (1 + w) and RoPE of one head vector (LDS src; out(d, y)
// takes dim d's result), one wave; rotate-half pairing
// (npu-asr-host/src/lib.rs:143-185).
template <int HD, typename Out>
__device__ __forceinline__ void head_xform(const XE_LDS float *src, Out out, bool norm, const float (&w0)[HeadConsts<HD>::PER],
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
    out(j, y0);
    out(j + HALF, y1);
  }
}

// Attention split blocks.  Keys are taken in 16-key tiles: a split is a
// multiple of one tile, spread so that every attention-side workgroup gets a
// share.
constexpr int kKeyTile = 16;
__host__ __device__ constexpr int round_keys(int) { return kKeyTile; }

__host__ __device__ __forceinline__ void ll_split(int len, int max_splits, int hd, int &chunk, int &nsplits) {
  const int gran = round_keys(hd);
  int per = (len + max_splits - 1) / max_splits;
  per = (per + gran - 1) / gran * gran;
  chunk = per < gran ? gran : per;
  nsplits = (len + chunk - 1) / chunk;
}

// Keys one round of a block covers (one Q.K tile per wave).
constexpr int kRoundKeys = kW * kKeyTile;

// ---------------------------------------------------------------------------
// Key/value stage (attention side).  The phase before an attention phase
// copies this rank's block into LDS with LDS-direct loads: q and k norm
// gains, the RoPE cos / sin rows at the position (one kStageGran slot each),
// then the block's key rows and value rows, each row padded by 16 bytes so
// the 16 Q.K lanes of a fragment (16 keys at one offset) fall in distinct
// banks.  When the attention phase polls for q nothing else is in flight
// (vector memory completes in issue order, so loads issued at the phase's
// start would hold the poll back by their memory latency).
// ---------------------------------------------------------------------------
__host__ __device__ inline int kv_row_bytes(int hd) { return 2 * hd + 16; }
__host__ __device__ inline int kv_stage_floats(int hd, int cap) {
  return (4 * kStageGran + 2 * cap * kv_row_bytes(hd)) / 4;
}

// Whether block `split` at length len is one the key/value stage holds (the
// issuing phase and the attention phase decide alike).
template <typename AD>
__host__ __device__ inline bool kv_staged(const AD &a, int split, int len) {
  if (a.kv_cap <= 0) return false;
  int chunk, nsplits;
  ll_split(len, a.max_splits, a.hd, chunk, nsplits);
  return split < nsplits && chunk <= a.kv_cap;
}

// One row of hd bf16 (row r of src) into LDS dst: lanes below hd / 8 move
// 16 bytes each.  Wave-uniform row.
__device__ __forceinline__ void lds_copy_row(__amdgpu_buffer_rsrc_t rs, int src_off, int bytes, XE_LDS uint8_t *dst) {
  const int lane = threadIdx.x & 63;
  if (lane * 16 < bytes)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, reinterpret_cast<XE_LDS void *>(dst), 16, src_off + lane * 16, 0, 0,
                                             gdev::kCoherentSc1);
}

// Issue the copies of attention block (split, kvh, b) at length len into the
// key/value stage kvs.  The caller has passed a block barrier since the
// stage's last reader.  Rows past the cache's current end are copied too
// (the new row is patched in from LDS; later ones are masked).
template <int HD, typename AD>
__device__ __forceinline__ void kv_stage_issue(const AD &a, int split, int kvh, int b, int len, float *kvs) {
  constexpr int HALF = HD / 2;
  XE_LDS uint8_t *kb = reinterpret_cast<XE_LDS uint8_t *>(lptr(kvs));
  const int posi = a.fixed_len > 0 ? 0 : len - 1;
  if (a.q_norm_w != nullptr) lds_copy(a.q_norm_w, 4 * HD, kb);
  if (a.k_norm_w != nullptr) lds_copy(a.k_norm_w, 4 * HD, kb + kStageGran);
  if (a.rope_cos != nullptr) {
    lds_copy(a.rope_cos + static_cast<size_t>(posi) * HALF, 4 * HALF, kb + 2 * kStageGran);
    lds_copy(a.rope_sin + static_cast<size_t>(posi) * HALF, 4 * HALF, kb + 3 * kStageGran);
  }
  int chunk, nsplits;
  ll_split(len, a.max_splits, HD, chunk, nsplits);
  const int s0 = split * chunk, s1 = min(len, s0 + chunk);
  const uint16_t *kbase = a.kc + a.kv_bstride * b + static_cast<size_t>(kvh) * a.max_ctx * HD;
  const uint16_t *vbase = a.vc + a.kv_bstride * b + static_cast<size_t>(kvh) * a.max_ctx * HD;
  const __amdgpu_buffer_rsrc_t krs = gdev::coherent_rsrc(kbase);
  const __amdgpu_buffer_rsrc_t vrs = gdev::coherent_rsrc(vbase);
  XE_LDS uint8_t *kk = kb + 4 * kStageGran;
  XE_LDS uint8_t *vv = kk + a.kv_cap * kv_row_bytes(HD);
  for (int r = threadIdx.x >> 6; r < s1 - s0; r += kW) {
    lds_copy_row(krs, (s0 + r) * HD * 2, HD * 2, kk + r * kv_row_bytes(HD));
    lds_copy_row(vrs, (s0 + r) * HD * 2, HD * 2, vv + r * kv_row_bytes(HD));
  }
}


// LDS scratch of a block (floats): new key [hd] | new key and value as
// stored (bf16 pairs) [hd] | scores / probabilities [kRoundKeys][g] | running
// max, sum, correction [3][16] | Q.K B operands [hd / 32][64 lanes][8 bf16] |
// per-wave P.V sums [kW][g][hd].
__host__ __device__ __forceinline__ int attn_scratch_floats(int hd, int g) {
  return 2 * hd + kRoundKeys * g + 48 + (hd / 32) * 256 + kW * g * hd;
}

typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ u32x2 ld_kv8(__amdgpu_buffer_rsrc_t rs, int byte_off) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs, byte_off, 0, gdev::kCoherentSc1));
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return static_cast<uint32_t>(adev::f32_to_bf16_rne(lo)) | static_cast<uint32_t>(adev::f32_to_bf16_rne(hi)) << 16;
}

// Signed byte j of w as a float.
__device__ __forceinline__ float i8_at(uint32_t w, int j) {
  return static_cast<float>(static_cast<int>(static_cast<int8_t>(w >> (8 * j))));
}

// Eight int8 values (k order) as eight bf16, exactly (at most 8 significant
// bits): the upper halves of their fp32 values, paired.
__device__ __forceinline__ u32x4 i8x8_to_bf16x8(u32x2 w) {
  uint32_t p[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t word = i < 2 ? w.x : w.y;
    const int j = 2 * (i & 1);
    p[i] = __builtin_amdgcn_perm(__float_as_uint(i8_at(word, j + 1)), __float_as_uint(i8_at(word, j)), 0x07060302u);
  }
  return u32x4{p[0], p[1], p[2], p[3]};
}

// One split block of (stream b, kv head kvh): keys [split*chunk, ...), the G
// query heads of the group at once.
//   Q.K: per wave one 16-key tile as v_mfma_f32_16x16x32_bf16 steps, K rows
//   straight from the bf16 cache as the A operand; B columns n, G + n and
//   2 G + n hold the three bf16 parts of query head n (q = hi + mid + lo
//   exactly), so C[key][n] + C[key][G + n] + C[key][2 G + n] is the score
//   from exact products with fp32 accumulation.
//   softmax: scores of the round in LDS, one wave per head (max, exp2, sum),
//   running max / sum across rounds.
//   P.V: lanes own 4 dims of a value row (hd / 4 lanes per key), keys spread
//   over the waves; fp32 FMAs; the waves' sums are added in LDS.
// The first round's K/V loads and the head-transform constants are issued
// before `prep` (which waits for the q rows: qin, LDS [nb][a.qn]).  The new
// key at the last position is not read back from the cache: lanes that hold
// it take the bf16-rounded values from LDS.  Partial out: (m, l, acc[hd]) per
// query head, m in log2 units of the scaled score.
// KV8: int8 K and V rows (the per-utterance cross K / V,
// route_b_kernels/decode_fused/gen_decode.py:263-282): K bytes convert to
// bf16 exactly for the MFMA, q is multiplied by the K channel scales before
// its three-part split (scores = sum_d (q[d] s_k[d]) k8[d]), and the partial
// sums are multiplied by the V channel scales (out[d] = s_v[d] sum_t p_t
// v8[t][d]); no append, no K/V stage.
template <int HD, int G, bool KV8, typename AD, typename Prep, typename Sub>
__device__ __forceinline__ bool attn_block(const AD &a, int split, int kvh, int b, int len, const float *qin,
                                           float *scr, unsigned ep, Prep prep, Sub tsub, float *kvs,
                                           bool staged) {
  static_assert(HD % 32 == 0 && HD <= 256 && 3 * G <= 16, "attention tile shape");
  constexpr int NJ = HD / 32;                  // MFMA steps per tile
  constexpr int LPK = HD / 4;                  // P.V lanes per key
  constexpr int KPI = 64 / LPK;                // keys per P.V load
  constexpr int PVK = kRoundKeys / (kW * KPI); // P.V loads per wave per round
  XE_LDS float *S = lptr(scr);
  XE_LDS float *kt = S;
  XE_LDS uint32_t *kvb = reinterpret_cast<XE_LDS uint32_t *>(kt + HD);  // k | v, bf16 pairs
  XE_LDS float *sc = kt + 2 * HD;              // [kRoundKeys][G]
  XE_LDS float *st = sc + kRoundKeys * G;      // m [16] | l [16] | corr [16]
  XE_LDS bf16x8_t *bfr = reinterpret_cast<XE_LDS bf16x8_t *>(st + 48);  // [NJ][64]
  XE_LDS float *red = st + 48 + NJ * 256;      // [kW][G][HD]
  int chunk, nsplits;
  ll_split(len, a.max_splits, HD, chunk, nsplits);
  const int s0 = split * chunk;
  const int s1 = min(len, s0 + chunk);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int posi = len - 1;

  uint16_t *kbase = a.kc + a.kv_bstride * b + static_cast<size_t>(kvh) * a.max_ctx * HD;
  uint16_t *vbase = a.vc + a.kv_bstride * b + static_cast<size_t>(kvh) * a.max_ctx * HD;
  // int8 rows: the same element offsets, in bytes
  const size_t kvoff8 = a.kv_bstride * b + static_cast<size_t>(kvh) * a.max_ctx * HD;
  const __amdgpu_buffer_rsrc_t krs =
      gdev::coherent_rsrc(KV8 ? static_cast<const void *>(reinterpret_cast<const uint8_t *>(a.kc) + kvoff8) : kbase);
  const __amdgpu_buffer_rsrc_t vrs =
      gdev::coherent_rsrc(KV8 ? static_cast<const void *>(reinterpret_cast<const uint8_t *>(a.vc) + kvoff8) : vbase);
  const bool appender = !KV8 && a.append && split == nsplits - 1;

  // lane roles: Q.K row (key) lane & 15, dims 8 (lane >> 4) + 32 j;
  // P.V key slot lane / LPK, dims 4 (lane % LPK) .. + 4
  const int qk_row = lane & 15, qk_dim = 8 * (lane >> 4);
  const int pv_slot = lane / LPK, pv_dim = 4 * (lane % LPK);
  u32x4 kf[NJ];
  u32x2 vf[PVK];
  u32x2 kf8[NJ];     // KV8: 8 int8 of a key
  uint32_t vf8[PVK]; // KV8: 4 int8 of a value row
  auto load_round = [&](int rb) {
    const int kq = rb + wave * kKeyTile + qk_row;
    const bool kok = kq < s1;
    if constexpr (KV8) {
#pragma unroll
      for (int j = 0; j < NJ; j++) kf8[j] = ld_kv8(krs, kok ? kq * HD + 32 * j + qk_dim : kNoRecord);
#pragma unroll
      for (int i = 0; i < PVK; i++) {
        const int kv = rb + (i * kW + wave) * KPI + pv_slot;
        vf8[i] = __builtin_amdgcn_raw_buffer_load_b32(vrs, kv < s1 ? kv * HD + pv_dim : kNoRecord, 0,
                                                      gdev::kCoherentSc1);
      }
    } else {
#pragma unroll
      for (int j = 0; j < NJ; j++) kf[j] = ld_kv(krs, kok ? (kq * HD + 32 * j + qk_dim) * 2 : kNoRecord);
#pragma unroll
      for (int i = 0; i < PVK; i++) {
        const int kv = rb + (i * kW + wave) * KPI + pv_slot;
        vf[i] = ld_kv8(vrs, kv < s1 ? (kv * HD + pv_dim) * 2 : kNoRecord);
      }
    }
  };
  HeadConsts<HD> hc;
  if (!staged) {
    load_round(s0);
    load_head_consts<HD>(a, a.fixed_len > 0 ? 0 : posi, hc);
  }
  if (threadIdx.x < 16) {
    st[threadIdx.x] = -INFINITY;
    st[16 + threadIdx.x] = 0.f;
  }
  if (!prep()) return false;
  // staged block: keys / values are read from the stage where they are used
  // (rows past the block read its last row: K gives masked scores, V is
  // zeroed), so they hold no registers across the block
  XE_LDS uint8_t *kk = reinterpret_cast<XE_LDS uint8_t *>(lptr(kvs)) + 4 * kStageGran;
  XE_LDS uint8_t *vv = kk + a.kv_cap * kv_row_bytes(HD);
  const int last = s1 - s0 - 1;
  if (staged) {
    // the stage's copies have landed in every wave (its loads, the barrier)
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    load_head_consts_lds<HD>(a, kvs, hc);
  }

  const XE_LDS float *qrow = lptr(qin) + static_cast<size_t>(b) * a.qn;
  const XE_LDS float *vsrc = qrow + a.v_off + kvh * HD;
  const bool qnorm = a.q_norm_w != nullptr, knorm = a.k_norm_w != nullptr, rope = a.rope_cos != nullptr;
  // B operands of the Q.K steps, written by the q head transforms: step j
  // (dims 32 j ..) lane (kg, n) holds dims 32 j + 8 kg .. + 8 of column n;
  // column n + p G (p = 0, 1, 2) is part p of query head n, where q = hi +
  // mid + lo exactly (truncation: each part takes the next 8 significant
  // bits), so the three columns' sum is the fp32 score of the bf16 keys.
  // Columns from 3 G on are never written: their products land in C columns
  // that nothing reads.
  XE_LDS uint16_t *bfh = reinterpret_cast<XE_LDS uint16_t *>(bfr);
  const float *ksc = KV8 ? a.k_scale + kvh * HD : nullptr;
  for (int gg = wave; gg < G; gg += kW) {
    head_xform<HD>(qrow + a.q_off + (kvh * G + gg) * HD, [&](int d, float x) {
      if constexpr (KV8) x = x * ksc[d];  // the K channel scale rides on q
      const uint32_t hi = __float_as_uint(x) & 0xffff0000u;
      const float r = x - __uint_as_float(hi);
      const uint32_t mid = __float_as_uint(r) & 0xffff0000u;
      const uint32_t lo = __float_as_uint(r - __uint_as_float(mid));
      XE_LDS uint16_t *o = bfh + (((d >> 5) * 64 + ((d & 31) >> 3) * 16 + gg) * 8 + (d & 7));
      o[0] = static_cast<uint16_t>(hi >> 16);
      o[8 * G] = static_cast<uint16_t>(mid >> 16);
      o[16 * G] = static_cast<uint16_t>(lo >> 16);
    }, qnorm, hc.qn0, hc.qn1, rope, hc, a.norm_eps);
  }
  if (appender && wave == kW - 1) {
    head_xform<HD>(qrow + a.k_off + kvh * HD, [&](int d, float x) { kt[d] = x; }, knorm, hc.kn0, hc.kn1, rope, hc,
                   a.norm_eps);
    __builtin_amdgcn_wave_barrier();
    // the new row as the cache holds it: one packed copy serves the lanes
    // that patch it in below and the cache stores at the end
    for (int j = lane; j < HD / 2; j += 64) {
      const uint32_t kp = pack_bf16x2(kt[2 * j], kt[2 * j + 1]);
      const uint32_t vp = pack_bf16x2(vsrc[2 * j], vsrc[2 * j + 1]);
      kvb[j] = kp;
      kvb[HD / 2 + j] = vp;
      if (staged) {  // the staged row of the position (its copy predates this step) takes the new values
        reinterpret_cast<XE_LDS uint32_t *>(kk + (posi - s0) * kv_row_bytes(HD))[j] = kp;
        reinterpret_cast<XE_LDS uint32_t *>(vv + (posi - s0) * kv_row_bytes(HD))[j] = vp;
      }
    }
  }
  __syncthreads();  // Q.K B operands and the new k / v staged in LDS
  tsub(0);

  const int col = lane & 15;

  const float sc2 = a.scale * adev::kLog2e;
  float acc[G][4];
#pragma unroll
  for (int gg = 0; gg < G; gg++)
#pragma unroll
    for (int e = 0; e < 4; e++) acc[gg][e] = 0.f;
  for (int rb = s0; rb < s1; rb += kRoundKeys) {
    if (rb != s0) load_round(rb);
    // ---- Q.K: this wave's 16-key tile ----
    const int tile0 = rb + wave * kKeyTile;
    if constexpr (KV8) {
#pragma unroll
      for (int j = 0; j < NJ; j++) kf[j] = i8x8_to_bf16x8(kf8[j]);
    }
    if (!KV8 && staged && tile0 < s1) {
      const int kq = min(wave * kKeyTile + qk_row, last);
#pragma unroll
      for (int j = 0; j < NJ; j++)
        kf[j] = *reinterpret_cast<const XE_LDS u32x4 *>(kk + kq * kv_row_bytes(HD) + (32 * j + qk_dim) * 2);
    }
    if (!staged && appender && posi >= tile0 && posi < tile0 + kKeyTile && tile0 + qk_row == posi) {
#pragma unroll
      for (int j = 0; j < NJ; j++) kf[j] = *reinterpret_cast<const XE_LDS u32x4 *>(kvb + 16 * j + qk_dim / 2);
    }
    if (tile0 < s1) {
      f32x4_t cacc = {0.f, 0.f, 0.f, 0.f};
      bf16x8_t bq[NJ];  // every B operand read first (one LDS latency, not NJ)
#pragma unroll
      for (int j = 0; j < NJ; j++) bq[j] = bfr[j * 64 + lane];
      __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of the chain
#pragma unroll
      for (int j = 0; j < NJ; j++)
        cacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kf[j]), bq[j], cacc, 0, 0, 0);
      // lane (row group r, column n < G): keys tile0 + 4r + i, head n; the
      // mid and lo parts sit G and 2 G columns to the right (row_shl)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float mid = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(cacc[i]), 0x100 + G, 0xF, 0xF, true));
        const float lo = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(cacc[i]), 0x100 + 2 * G, 0xF, 0xF, true));
        const int key_l = wave * kKeyTile + 4 * (lane >> 4) + i;
        if (col < G) sc[key_l * G + col] = tile0 + 4 * (lane >> 4) + i < s1 ? (cacc[i] + mid + lo) * sc2 : -INFINITY;
      }
    } else if (col < G) {
#pragma unroll
      for (int i = 0; i < 4; i++) sc[(wave * kKeyTile + 4 * (lane >> 4) + i) * G + col] = -INFINITY;
    }
    __syncthreads();
    if (rb == s0) tsub(1);
    // ---- softmax statistics of the round: wave gg handles head gg ----
    if (wave < G) {
      const int gg = wave;
      float sv[kRoundKeys / 64];
      float mx = -INFINITY;
#pragma unroll
      for (int t = 0; t < kRoundKeys / 64; t++) {
        sv[t] = sc[(lane + 64 * t) * G + gg];
        mx = fmaxf(mx, sv[t]);
      }
      mx = gdev::wave_max(mx);
      const float m_old = st[gg];
      const float m_new = fmaxf(m_old, mx);
      const float corr = m_old == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_old - m_new);
      float ps = 0.f;
#pragma unroll
      for (int t = 0; t < kRoundKeys / 64; t++) {
        const float p = sv[t] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(sv[t] - m_new);
        sc[(lane + 64 * t) * G + gg] = p;
        ps += p;
      }
      ps = gdev::wave_sum(ps);
      if (lane == 0) {
        st[gg] = m_new;
        st[16 + gg] = st[16 + gg] * corr + ps;
        st[32 + gg] = corr;
      }
    }
    __syncthreads();
    if (rb == s0) tsub(2);
    // ---- P.V over this wave's keys of the round ----
    if (rb != s0) {
#pragma unroll
      for (int gg = 0; gg < G; gg++) {
        const float corr = st[32 + gg];
#pragma unroll
        for (int e = 0; e < 4; e++) acc[gg][e] *= corr;
      }
    }
    if (!KV8 && staged) {
      // this wave's key slots (slot i * kW + wave, KPI keys each) hold keys
      // up to the block's last; four slots' reads are issued together
      const int nact = wave * KPI <= last ? (last / KPI - wave) / kW + 1 : 0;
      for (int i0 = 0; i0 < nact; i0 += 4) {
        u32x2 vq[4];
        float pq[4][G];
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const int key_l = ((i0 + q) * kW + wave) * KPI + pv_slot;
          const int kr = min(key_l, last);
          vq[q] = *reinterpret_cast<const XE_LDS u32x2 *>(vv + kr * kv_row_bytes(HD) + pv_dim * 2);
#pragma unroll
          for (int gg = 0; gg < G; gg++) pq[q][gg] = sc[kr * G + gg];
        }
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const int key_l = ((i0 + q) * kW + wave) * KPI + pv_slot;
          const bool in = i0 + q < nact && key_l <= last;
          const float vv4[4] = {__uint_as_float(vq[q].x << 16), __uint_as_float(vq[q].x & 0xffff0000u),
                                __uint_as_float(vq[q].y << 16), __uint_as_float(vq[q].y & 0xffff0000u)};
#pragma unroll
          for (int gg = 0; gg < G; gg++) {
            const float p = in ? pq[q][gg] : 0.f;
#pragma unroll
            for (int e = 0; e < 4; e++) acc[gg][e] = __builtin_fmaf(p, vv4[e], acc[gg][e]);
          }
        }
      }
    } else {
  #pragma unroll
      for (int i = 0; i < PVK; i++) {
        if (rb + (i * kW + wave) * KPI >= s1) continue;  // wave-uniform: slots past the split
        const int key_l = (i * kW + wave) * KPI + pv_slot;
        float vv[4];
        if constexpr (KV8) {
#pragma unroll
          for (int e = 0; e < 4; e++) vv[e] = i8_at(vf8[i], e);
        } else {
          u32x2 v = vf[i];
          if (appender && rb + key_l == posi) v = *reinterpret_cast<const XE_LDS u32x2 *>(kvb + HD / 2 + pv_dim / 2);
          vv[0] = __uint_as_float(v.x << 16);
          vv[1] = __uint_as_float(v.x & 0xffff0000u);
          vv[2] = __uint_as_float(v.y << 16);
          vv[3] = __uint_as_float(v.y & 0xffff0000u);
        }
        float p[G];
        if constexpr (G == 4) {
          const f32x4_t p4 = *reinterpret_cast<const XE_LDS f32x4_t *>(sc + key_l * G);
          p[0] = p4.x;
          p[1] = p4.y;
          p[2] = p4.z;
          p[3] = p4.w;
        } else {
  #pragma unroll
          for (int gg = 0; gg < G; gg++) p[gg] = sc[key_l * G + gg];
        }
  #pragma unroll
        for (int gg = 0; gg < G; gg++)
  #pragma unroll
          for (int e = 0; e < 4; e++) acc[gg][e] = __builtin_fmaf(p[gg], vv[e], acc[gg][e]);
      }
    }
    if (rb + kRoundKeys < s1) __syncthreads();  // scores of the next round overwrite sc
  }
  tsub(3);
  // ---- key slots of a wave (KPI > 1), then the waves ----
  if constexpr (KPI > 1) {
    float flat[G * 4];
#pragma unroll
    for (int gg = 0; gg < G; gg++)
#pragma unroll
      for (int e = 0; e < 4; e++) flat[gg * 4 + e] = acc[gg][e];
    // slots are the 16-lane rows (LPK == 16) or row pairs (LPK == 32)
#pragma unroll
    for (int t = 0; t < G * 4; t++) {
      if constexpr (LPK == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(flat[t]), __float_as_uint(flat[t]), false, false);
        flat[t] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
      }
      const auto r2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(flat[t]), __float_as_uint(flat[t]), false, false);
      flat[t] = __uint_as_float(r2[0]) + __uint_as_float(r2[1]);
    }
#pragma unroll
    for (int gg = 0; gg < G; gg++)
#pragma unroll
      for (int e = 0; e < 4; e++) acc[gg][e] = flat[gg * 4 + e];
  }
  if (lane < LPK) {
#pragma unroll
    for (int gg = 0; gg < G; gg++) {
      f32x4_t v4 = {acc[gg][0], acc[gg][1], acc[gg][2], acc[gg][3]};
      *reinterpret_cast<XE_LDS f32x4_t *>(red + (wave * G + gg) * HD + pv_dim) = v4;
    }
  }
  __syncthreads();
  // the partials go out with consecutive lanes on consecutive pairs (a
  // store instruction covers whole lines); each acc value is the waves' sum
  // (wave order), read straight from the per-wave sums
  for (int t = threadIdx.x; t < G * (HD + 2); t += kT) {
    const int gg = t / (HD + 2), e = t % (HD + 2);
    float v;
    if (e < 2) {
      v = st[16 * e + gg];
    } else {
      // all the waves' reads first, then the sum in wave order
      float rv[kW];
#pragma unroll
      for (int w = 0; w < kW; w++) rv[w] = red[(w * G + gg) * HD + e - 2];
      v = rv[0];
#pragma unroll
      for (int w = 1; w < kW; w++) v += rv[w];
      if constexpr (KV8) v = v * a.v_scale[kvh * HD + e - 2];  // the V channel scale
    }
    put(a.part, b, ((kvh * G + gg) * a.max_splits + split) * (HD + 2) + e, v, ep);
  }
  // the new key / value into the cache: read from the next step on (the
  // step-end fence orders these stores before the argmax hand-off); stored
  // last so that no wait above includes their completion (the compiler
  // waits for every vector-memory operation before an LDS read that an
  // LDS-direct copy might still be writing)
  if (appender && wave == kW - 1) {
    uint32_t *krow = reinterpret_cast<uint32_t *>(kbase + static_cast<size_t>(posi) * HD);
    uint32_t *vrow = reinterpret_cast<uint32_t *>(vbase + static_cast<size_t>(posi) * HD);
    for (int j = lane; j < HD / 2; j += 64) {
      __hip_atomic_store(gptr_w(krow) + j, kvb[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(gptr_w(vrow) + j, kvb[HD / 2 + j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  lds_barrier();  // scratch is reused by the next block
  return true;
}

// Merge block: stream b, q head h, outputs [e0, e0 + kDM) of the head.
// tab: LDS scratch >= kMaxSplits * (kDM + 2) + kMaxSplits + kW * (kDM + 1)
// floats.
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
    mx = gdev::wave_max(mx);
    for (int s = threadIdx.x; s < nsplits; s += 64) {
      const float ms = tab[s * W];
      wts[s] = ms == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ms - mx);
    }
  }
  __syncthreads();
  // weighted sums over the splits: lane (group, e) of all kT threads takes
  // splits group, group + kT / kDM, ...; the 64 / kDM groups of a wave meet
  // by lane swaps, the waves' sums in LDS (fixed order throughout)
  static_assert(kDM == 16, "merge lanes: 16 outputs a block");
  XE_LDS float *wsum = wts + kMaxSplits;  // [kW][kDM + 1]
  {
    const int e = threadIdx.x & (kDM - 1), grp = threadIdx.x >> 4;
    float ls = 0.f, at = 0.f;
    for (int s = grp; s < nsplits; s += kT / kDM) {
      const float w = wts[s];
      ls = __builtin_fmaf(tab[s * W + 1], w, ls);
      at = __builtin_fmaf(tab[s * W + 2 + e], w, at);
    }
    auto swap_add = [](float v, bool half32) {
      const auto r = half32 ? __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false)
                            : __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
      return __uint_as_float(r[0]) + __uint_as_float(r[1]);
    };
    at = swap_add(swap_add(at, false), true);
    ls = swap_add(swap_add(ls, false), true);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane < kDM) {
      wsum[wave * (kDM + 1) + lane] = at;
      if (lane == 0) wsum[wave * (kDM + 1) + kDM] = ls;
    }
  }
  __syncthreads();
  if (threadIdx.x < kDM) {
    const int e = threadIdx.x;
    float ls = 0.f, at = 0.f, wa[kW], wl[kW];  // every wave's reads first, then the sums in wave order
#pragma unroll
    for (int w = 0; w < kW; w++) {
      wa[w] = wsum[w * (kDM + 1) + e];
      wl[w] = wsum[w * (kDM + 1) + kDM];
    }
#pragma unroll
    for (int w = 0; w < kW; w++) {
      at += wa[w];
      ls += wl[w];
    }
    const float o = mg.div_norm ? at / ls : at * (1.0f / ls);
    put(mg.out, b, h * HD + e0 + e, o, ep);
  }
  lds_barrier();
  return true;
}

// host side (ll_launch.hip)
bool step_supported(int wdtype, int nb_t, int hd, int g, bool kv8);
void launch(const StepParams &sp, int wdtype, int nb_t, int hd, int g, bool kv8, size_t lds_bytes, int grid,
            hipStream_t s);

}  // namespace ll
}  // namespace xe
