// step_dev.h -- one decode step as a list of phases for the phase-kernel
// executors: one standalone kernel launch per phase (phases.hip), captured in
// a HIP graph per batch size or launched eagerly.
//
// Phase kinds: token embedding, norm+GEMV (gemv_dev.h), attention split
// partials and merge (attn_dev.h), greedy argmax partials and final.
#pragma once

#include "attn_dev.h"
#include "gemv_dev.h"

namespace xe {
namespace sdev {

// PH_GEMM_PRO / PH_GEMM: a projection over more streams than the GEMV tile
// holds (gemm.hip): the norm / residual prologue into Phase::xn, then the
// MFMA GEMM.
enum PhaseKind {
  PH_EMBED = 0,
  PH_GEMV = 1,
  PH_ATTN = 2,
  PH_MERGE = 3,
  PH_ARGMAX_PART = 4,
  PH_ARGMAX_FINAL = 5,
  PH_GEMM_PRO = 6,
  PH_GEMM = 7
};

constexpr int kArgBlocks = 64;

// Embedding: x[b] = dequant(E[tok[b]]) (+ P[pos[b] + pos_off]) (* mul)
struct EmbedParams {
  const void *emb;
  const float *emb_scale;
  const uint8_t *emb_exps;
  int wdtype;
  const float *pos_emb;
  int pos_off, pos_rows;
  float mul;
  int use_mul;
  const int32_t *tokens;
  const int32_t *pos;
  int vocab, d, batch;
  float *x;
};

// Greedy argmax over logits [batch, vocab]; last_max selects the tie rule.
struct ArgmaxParams {
  const float *logits;
  int vocab, batch, last_max;
  float *part_v;
  int *part_i;
  int32_t *next, *tokens, *pos, *hist;
  int hist_stride;
  // stop rule (whisper.rs:618-668): stop[0] is the stop token (< 0: none);
  // done[b] marks a stream that has emitted it, which is then fed the stop
  // token.  done may be null (no rule).
  const int32_t *stop;
  int32_t *done;
};

struct Phase {
  int kind;
  int variant;  // GEMV: tile (lpr, rpl); ATTN/MERGE: head_dim and group
  int lpr, rpl;
  int hd, g;
  int nblocks;  // virtual blocks of the phase
  int pad;
  float *xn;    // PH_GEMM_PRO: normalised activations out [batch][k]
  float *ws;    // PH_GEMM: split-K partial tiles
  unsigned *cnt;  // PH_GEMM: split-K arrival counters (zero between launches)
  union {
    gdev::GemvParams gemv;
    adev::AttnParams attn;
    EmbedParams emb;
    ArgmaxParams arg;
  } u;
};

template <bool COH>
__device__ __forceinline__ void embed_block(const EmbedParams &p, int vb) {
  const int chunks = (p.d + 255) / 256;
  const int b = vb / chunks, c = vb % chunks;
  if (b >= p.batch) return;
  int tok = p.tokens[b];
  tok = tok < 0 ? 0 : (tok >= p.vocab ? p.vocab - 1 : tok);
  int prow = p.pos[b] + p.pos_off;
  prow = prow < 0 ? 0 : (prow >= p.pos_rows ? p.pos_rows - 1 : prow);
  const int j = c * 256 + threadIdx.x;
  if (j >= p.d) return;
  const size_t i = static_cast<size_t>(tok) * p.d + j;
  float v;
  if (p.wdtype == XE_I8)
    v = static_cast<float>(static_cast<const int8_t *>(p.emb)[i]) * p.emb_scale[tok];
  else if (p.wdtype == XE_BF16)
    v = __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t *>(p.emb)[i]) << 16);
  else
    v = ldexpf(static_cast<float>(static_cast<const int8_t *>(p.emb)[i]), static_cast<int>(p.emb_exps[i / 8]) - 133);
  if (p.pos_emb) v = v + p.pos_emb[static_cast<size_t>(prow) * p.d + j];
  if (p.use_mul) v = v * p.mul;
  gdev::act_st<COH>(p.x + static_cast<size_t>(b) * p.d + j, v);
}

__device__ __forceinline__ bool better(float v, int i, float bv, int bi, int last_max) {
  if (v != v) return false;  // NaN never wins
  if (bi < 0) return true;
  if (v > bv) return true;
  if (v == bv) return last_max ? i > bi : i < bi;
  return false;
}

// Block k of row b reduces its slice of the logits (Iterator::max_by keeps
// the LAST of equal maxima, opt125m_decode.rs:303; strict > keeps the first,
// whisper.rs:749-757).  `better` orders every (value, index) pair totally, so
// the winner does not depend on the order of the compares: a thread's loads
// go out together (up to kArgU of them, one memory round trip for a slice of
// 256 kArgU logits), then a 64-lane butterfly and the four waves' winners.
// lds: at least 8 floats.
constexpr int kArgU = 16;
template <bool COH>
__device__ __forceinline__ void argmax_part_block(const ArgmaxParams &p, int vb, float *lds) {
  const int b = vb / kArgBlocks, k = vb % kArgBlocks;
  if (b >= p.batch) return;
  const int per = (p.vocab + kArgBlocks - 1) / kArgBlocks;
  const int lo = k * per, hi = min(p.vocab, lo + per);
  const float *row = p.logits + static_cast<size_t>(b) * p.vocab;
  float bv = -INFINITY;
  int bi = -1;
  for (int i0 = lo + static_cast<int>(threadIdx.x); i0 < hi; i0 += 256 * kArgU) {
    float v[kArgU];
#pragma unroll
    for (int u = 0; u < kArgU; u++) v[u] = i0 + 256 * u < hi ? gdev::act_ld<COH>(row, i0 + 256 * u) : 0.f;
#pragma unroll
    for (int u = 0; u < kArgU; u++) {
      const int i = i0 + 256 * u;
      if (i < hi && better(v[u], i, bv, bi, p.last_max)) {
        bv = v[u];
        bi = i;
      }
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(bv, off, 64);
    const int oi = __shfl_xor(bi, off, 64);
    if (oi >= 0 && better(ov, oi, bv, bi, p.last_max)) {
      bv = ov;
      bi = oi;
    }
  }
  float *sv = lds;
  int *si = reinterpret_cast<int *>(lds + 4);
  if ((threadIdx.x & 63) == 0) {
    sv[threadIdx.x >> 6] = bv;
    si[threadIdx.x >> 6] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float v = sv[0];
    int idx = si[0];
    for (int w = 1; w < 4; w++)
      if (si[w] >= 0 && better(sv[w], si[w], v, idx, p.last_max)) {
        v = sv[w];
        idx = si[w];
      }
    gdev::act_st<COH>(p.part_v + b * kArgBlocks + k, v);
    gdev::act_st<COH>(reinterpret_cast<float *>(p.part_i) + b * kArgBlocks + k, __int_as_float(idx));
  }
  __syncthreads();
}

// Wave 0 of the block for stream b merges the partials; the winner becomes the
// next input token, pos advances, hist[b][pos] records it.
template <bool COH>
__device__ __forceinline__ void argmax_final_block(const ArgmaxParams &p, int b) {
  if (b >= p.batch || threadIdx.x >= 64) return;
  float v = -INFINITY;
  int idx = -1;
  for (int k = threadIdx.x; k < kArgBlocks; k += 64) {
    const float pv = gdev::act_ld<COH>(p.part_v, b * kArgBlocks + k);
    const int pi = __float_as_int(gdev::act_ld<COH>(reinterpret_cast<const float *>(p.part_i), b * kArgBlocks + k));
    if (pi >= 0 && better(pv, pi, v, idx, p.last_max)) {
      v = pv;
      idx = pi;
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(v, off, 64);
    const int oi = __shfl_xor(idx, off, 64);
    if (oi >= 0 && better(ov, oi, v, idx, p.last_max)) {
      v = ov;
      idx = oi;
    }
  }
  if (threadIdx.x != 0) return;
  if (idx < 0) idx = 0;
  int tok = idx;
  if (p.done) {
    const int st = p.stop[0];
    if (st >= 0 && (p.done[b] != 0 || idx == st)) {
      p.done[b] = 1;
      tok = st;
    }
  }
  p.next[b] = idx;
  p.tokens[b] = tok;
  const int ps = p.pos[b];
  if (ps >= 0 && ps < p.hist_stride) p.hist[static_cast<size_t>(b) * p.hist_stride + ps] = idx;
  p.pos[b] = ps + 1;
}

}  // namespace sdev

// Standalone execution of one phase (gemv.hip / attn.hip / decoder.hip).
void launch_phase(const sdev::Phase &ph, hipStream_t s);
// gemm.hip
bool gemm_needs_prologue(const gdev::GemvParams &p);
int gemm_defer_splits(int m, int k, int batch);
bool gemm_i8_preferred(int m, int k, int batch, int wdtype);
bool gemm_prologue_takes_digits(const gdev::GemvParams &p, const float *xn);
bool gemm_prologue_takes_parts(const gdev::GemvParams &p, const float *xn);
void launch_gemm_prologue(const gdev::GemvParams &p, float *xn, hipStream_t s);
void launch_gemm(const gdev::GemvParams &p, int wdtype, float *ws, unsigned *cnt, hipStream_t s);
size_t gemm_ws_floats();
size_t gemm_cnt_words();

}  // namespace xe
