// decoder.hip -- the decode backends on one GPU: OPT (opt125m_decode.rs
// Opt::step/generate :252-315), Whisper (whisper_decoder.rs HostDecoder::step
// :401-535 and the fused/batched backends' precompute_cross / reset / step
// contract :1143-1349, :1751-1796) and Gemma-3 (npu-gemma config + HF Gemma3
// layer).  The reference runs each token as one fused ELF dispatch
// (gen_decode.py:391-420); here a token is a short chain of fused kernels
// captured once in a HIP graph and replayed:
//
//   embed ->  per layer: [norm+QKV GEMV] -> [q/k norm, RoPE, KV append,
//             split-K attention, merge] -> [O GEMV] -> (Whisper: [norm+cross-q
//             GEMV] -> [cross attention] -> [cross-out GEMV]) -> [norm+FC1 /
//             gate-up GeGLU GEMV] -> [FC2 GEMV]
//          -> [final norm + tied lm-head GEMV] -> [argmax -> next token, pos+1]
//
// Residual adds (and Gemma's post-attention / post-FFN RMSNorms) are folded
// into the prologue of the next GEMV, which also writes the updated residual
// stream (ping-pong buffers), so no kernel exists only to add vectors.
// Token ids and positions live in device memory and the argmax kernel feeds
// the next step, so a generate loop replays the graph with no host traffic.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <map>
#include <memory>

#include "common.h"
#include "quant.h"

namespace xe {
namespace {

// --------------------------------------------------------------------------
// synthetic weights (bit-identical to the oracle's generator)
// --------------------------------------------------------------------------
constexpr float kIh4InvStd = 2.6428997e-05f;  // 1 / sqrt((65536^2 - 1) / 3)

__host__ __device__ inline uint64_t mix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

inline uint64_t synth_base(uint64_t seed, uint32_t tensor) {
  return mix64(seed * 0xD1B54A32D192ED03ull + static_cast<uint64_t>(tensor));
}

__device__ inline float synth_value(uint64_t base, uint64_t idx, float mean, float k) {
  const uint64_t h = mix64(base + idx);
  const int32_t sum = static_cast<int32_t>(h & 0xffff) + static_cast<int32_t>((h >> 16) & 0xffff) +
                      static_cast<int32_t>((h >> 32) & 0xffff) + static_cast<int32_t>(h >> 48);
  const float v = __fmul_rn(static_cast<float>(sum - 131070), k);
  return __fadd_rn(v, mean);
}

__device__ inline uint16_t bf16_bits_dev(float x) {
  uint32_t bits = __float_as_uint(x);
  if ((bits & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((bits >> 16) | 0x0040u);
  uint32_t bias = 0x00007fffu + ((bits >> 16) & 1u);
  return static_cast<uint16_t>((bits + bias) >> 16);
}

__device__ inline float bf16_round_dev(float x) {
  return __uint_as_float(static_cast<uint32_t>(bf16_bits_dev(x)) << 16);
}

// One workgroup per source row: generate, quantise (int8 per-row / bf16 /
// bfp16) and store at destination row (row_off + r * row_stride).
__global__ __launch_bounds__(256) void synth_rows_kernel(uint64_t base, float mean, float k,
                                                         int rows, int cols, int wdtype,
                                                         int row_off, int row_stride, void *dst,
                                                         float *scale, uint8_t *exps) {
  const int r = blockIdx.x;
  if (r >= rows) return;
  const int drow = row_off + r * row_stride;
  const uint64_t rb = static_cast<uint64_t>(r) * cols;
  __shared__ float red[4];
  if (wdtype == XE_I8) {
    float amax = 0.f;
    for (int j = threadIdx.x; j < cols; j += 256) amax = fmaxf(amax, fabsf(synth_value(base, rb + j, mean, k)));
    for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float sc = amax > 0.0f ? __fdiv_rn(amax, 127.0f) : 1.0f;
    if (threadIdx.x == 0) scale[drow] = sc;
    int8_t *q = static_cast<int8_t *>(dst) + static_cast<size_t>(drow) * cols;
    for (int j = threadIdx.x; j < cols; j += 256) {
      float v = roundf(__fdiv_rn(synth_value(base, rb + j, mean, k), sc));
      v = fminf(fmaxf(v, -127.0f), 127.0f);
      q[j] = static_cast<int8_t>(v);
    }
  } else if (wdtype == XE_BF16) {
    uint16_t *o = static_cast<uint16_t *>(dst) + static_cast<size_t>(drow) * cols;
    for (int j = threadIdx.x; j < cols; j += 256) o[j] = bf16_bits_dev(synth_value(base, rb + j, mean, k));
  } else {
    // bfp16: thread t encodes block t (8 values)
    int8_t *mant = static_cast<int8_t *>(dst) + static_cast<size_t>(drow) * cols;
    uint8_t *ex = exps + static_cast<size_t>(drow) * (cols / 8);
    for (int bk = threadIdx.x; bk < cols / 8; bk += 256) {
      float v[8];
      float maxabs = 0.f;
      for (int i = 0; i < 8; i++) {
        v[i] = bf16_round_dev(synth_value(base, rb + bk * 8 + i, mean, k));
        maxabs = fmaxf(maxabs, fabsf(v[i]));
      }
      if (maxabs == 0.0f) maxabs = 1.0f;
      int e = ilogbf(maxabs);  // floor(log2) for normal floats (exact)
      e = e < -127 ? -127 : (e > 127 ? 127 : e);
      const float quantum = ldexpf(1.0f, e - 6);
      for (int i = 0; i < 8; i++) {
        float qv = rintf(__fdiv_rn(v[i], quantum));
        qv = fminf(fmaxf(qv, -128.0f), 127.0f);
        mant[bk * 8 + i] = static_cast<int8_t>(qv);
      }
      ex[bk] = static_cast<uint8_t>(e + 127);
    }
  }
}

__global__ void synth_vec_kernel(uint64_t base, float mean, float k, size_t n, float *dst,
                                 int round_bf16) {
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x) {
    float v = synth_value(base, i, mean, k);
    dst[i] = round_bf16 ? bf16_round_dev(v) : v;
  }
}

// --------------------------------------------------------------------------
// step kernels
// --------------------------------------------------------------------------

// x[b] = dequant(E[tok[b]]) (+ P[pos[b] + pos_off]) (* emb_scale)
__global__ void embed_kernel(const void *emb, const float *emb_scale_rows, const uint8_t *emb_exps,
                             int wdtype, const float *pos_emb, int pos_off, int pos_rows,
                             float mul, int use_mul, const int32_t *tokens, const int32_t *pos,
                             int vocab, int d, float *x) {
  const int b = blockIdx.y;
  int tok = tokens[b];
  tok = tok < 0 ? 0 : (tok >= vocab ? vocab - 1 : tok);
  int prow = pos[b] + pos_off;
  prow = prow < 0 ? 0 : (prow >= pos_rows ? pos_rows - 1 : prow);
  for (int j = blockIdx.x * blockDim.x + threadIdx.x; j < d; j += gridDim.x * blockDim.x) {
    const size_t i = static_cast<size_t>(tok) * d + j;
    float v;
    if (wdtype == XE_I8)
      v = static_cast<float>(static_cast<const int8_t *>(emb)[i]) * emb_scale_rows[tok];
    else if (wdtype == XE_BF16)
      v = __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t *>(emb)[i]) << 16);
    else
      v = ldexpf(static_cast<float>(static_cast<const int8_t *>(emb)[i]),
                 static_cast<int>(emb_exps[i / 8]) - 133);
    if (pos_emb) v = v + pos_emb[static_cast<size_t>(prow) * d + j];
    if (use_mul) v = v * mul;
    x[static_cast<size_t>(b) * d + j] = v;
  }
}

// f32 [T, H*hd] rows -> bf16 head-major [H, T, hd]
__global__ void cross_pack_kernel(const float *src, int t_rows, int heads, int hd, uint16_t *dst) {
  const size_t n = static_cast<size_t>(t_rows) * heads * hd;
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const int j = static_cast<int>(i % hd);
    const size_t r = i / hd;
    const int h = static_cast<int>(r % heads);
    const int t = static_cast<int>(r / heads);
    dst[(static_cast<size_t>(h) * t_rows + t) * hd + j] = bf16_bits_dev(src[i]);
  }
}

// Greedy argmax over logits[b, :]: block partials, then a merge launch.
// last_max = 1: Iterator::max_by (opt125m_decode.rs:303) keeps the LAST of
// equal maxima; else strict > keeps the first (whisper.rs:749-757).
// The winner becomes the next input token; pos advances; hist[b][pos] gets it.
constexpr int kArgBlocks = 64;

__device__ inline bool better(float v, int i, float bv, int bi, int last_max) {
  if (v != v) return false;  // NaN never wins
  if (bi < 0) return true;
  if (v > bv) return true;
  if (v == bv) return last_max ? i > bi : i < bi;
  return false;
}

// Partials: block k of row b reduces its slice of the logits.
__global__ __launch_bounds__(256) void argmax_partial_kernel(const float *logits, int vocab,
                                                             int last_max, float *part_v,
                                                             int *part_i) {
  const int b = blockIdx.y;
  const int per = (vocab + kArgBlocks - 1) / kArgBlocks;
  const int lo = blockIdx.x * per, hi = min(vocab, lo + per);
  const float *row = logits + static_cast<size_t>(b) * vocab;
  float bv = -INFINITY;
  int bi = -1;
  for (int i = lo + threadIdx.x; i < hi; i += 256) {
    const float v = row[i];
    if (better(v, i, bv, bi, last_max)) {
      bv = v;
      bi = i;
    }
  }
  __shared__ float sv[256];
  __shared__ int si[256];
  sv[threadIdx.x] = bv;
  si[threadIdx.x] = bi;
  __syncthreads();
  for (int w = 128; w >= 1; w >>= 1) {
    if (threadIdx.x < w) {
      const float ov = sv[threadIdx.x + w];
      const int oi = si[threadIdx.x + w];
      if (oi >= 0 && better(ov, oi, sv[threadIdx.x], si[threadIdx.x], last_max)) {
        sv[threadIdx.x] = ov;
        si[threadIdx.x] = oi;
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    part_v[b * kArgBlocks + blockIdx.x] = sv[0];
    part_i[b * kArgBlocks + blockIdx.x] = si[0];
  }
}

// Final: one wave per stream merges the partials; the winner becomes the
// next input token, pos advances, hist[b][pos] records it.
__global__ __launch_bounds__(64) void argmax_final_kernel(const float *part_v, const int *part_i,
                                                          int last_max, int32_t *next,
                                                          int32_t *tokens, int32_t *pos,
                                                          int32_t *hist, int hist_stride) {
  const int b = blockIdx.x;
  float v = -INFINITY;
  int idx = -1;
  for (int k = threadIdx.x; k < kArgBlocks; k += 64) {
    const float pv = part_v[b * kArgBlocks + k];
    const int pi = part_i[b * kArgBlocks + k];
    if (pi >= 0 && better(pv, pi, v, idx, last_max)) {
      v = pv;
      idx = pi;
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(v, off, 64);
    const int oi = __shfl_xor(idx, off, 64);
    if (oi >= 0 && better(ov, oi, v, idx, last_max)) {
      v = ov;
      idx = oi;
    }
  }
  if (threadIdx.x != 0) return;
  if (idx < 0) idx = 0;
  next[b] = idx;
  tokens[b] = idx;
  const int p = pos[b];
  if (p >= 0 && p < hist_stride) hist[static_cast<size_t>(b) * hist_stride + p] = idx;
  pos[b] = p + 1;
}

// --------------------------------------------------------------------------
// tensor table (mirrors the oracle's xo_tensor_spec: same shapes and laws)
// --------------------------------------------------------------------------
struct Spec {
  int rows = 0, cols = 0;
  bool quant = false;
  float mean = 0.f, stdv = 0.02f;
};

bool tensor_spec(const xe_model_config &c, int kind, int layer, Spec &s) {
  const int D = c.d_model, hq = c.n_heads * c.head_dim, hk = c.n_kv_heads * c.head_dim;
  const int F = c.ffn;
  const bool gem = c.family == XE_GEMMA3, wh = c.family == XE_WHISPER, opt = c.family == XE_OPT;
  s = Spec{};
  if (layer < 0) {
    switch (kind) {
      case XE_T_TOK_EMB: s.rows = c.vocab; s.cols = D; s.quant = true; return true;
      case XE_T_POS_EMB:
        if (gem) return false;
        s.rows = opt ? c.max_pos + 2 : c.max_pos; s.cols = D; return true;
      case XE_T_LNF_W: s.rows = 1; s.cols = D; s.mean = gem ? 0.f : 1.f; return true;
      case XE_T_LNF_B: if (gem) return false; s.rows = 1; s.cols = D; return true;
      case XE_T_ENC_OUT:
        if (!wh) return false;
        s.rows = c.n_cross; s.cols = D; s.stdv = 1.0f; return true;
      default: return false;
    }
  }
  switch (kind) {
    case XE_T_LN1_W: case XE_T_LN2_W: s.rows = 1; s.cols = D; s.mean = gem ? 0.f : 1.f; return true;
    case XE_T_LN1_B: case XE_T_LN2_B: if (gem) return false; s.rows = 1; s.cols = D; return true;
    case XE_T_Q_W: s.rows = hq; s.cols = D; s.quant = true; return true;
    case XE_T_K_W: case XE_T_V_W: s.rows = hk; s.cols = D; s.quant = true; return true;
    case XE_T_Q_B: if (gem) return false; s.rows = 1; s.cols = hq; return true;
    case XE_T_K_B: if (!opt) return false; s.rows = 1; s.cols = hk; return true;
    case XE_T_V_B: if (gem) return false; s.rows = 1; s.cols = hk; return true;
    case XE_T_O_W: s.rows = D; s.cols = hq; s.quant = true; return true;
    case XE_T_O_B: if (gem) return false; s.rows = 1; s.cols = D; return true;
    case XE_T_FC1_W: s.rows = F; s.cols = D; s.quant = true; return true;
    case XE_T_FC1_B: if (gem) return false; s.rows = 1; s.cols = F; return true;
    case XE_T_UP_W: if (!gem) return false; s.rows = F; s.cols = D; s.quant = true; return true;
    case XE_T_FC2_W: s.rows = D; s.cols = F; s.quant = true; return true;
    case XE_T_FC2_B: if (gem) return false; s.rows = 1; s.cols = D; return true;
    case XE_T_QNORM_W: case XE_T_KNORM_W:
      if (!gem) return false;
      s.rows = 1; s.cols = c.head_dim; return true;
    case XE_T_POST_ATTN_W: case XE_T_POST_FFN_W: if (!gem) return false; s.rows = 1; s.cols = D; return true;
    case XE_T_LNX_W: if (!wh) return false; s.rows = 1; s.cols = D; s.mean = 1.f; return true;
    case XE_T_LNX_B: case XE_T_XQ_B: case XE_T_XV_B: case XE_T_XO_B:
      if (!wh) return false;
      s.rows = 1; s.cols = D; return true;
    case XE_T_XQ_W: case XE_T_XK_W: case XE_T_XV_W: case XE_T_XO_W:
      if (!wh) return false;
      s.rows = D; s.cols = D; s.quant = true; return true;
    default: return false;
  }
}

size_t wbytes(int wdtype, size_t n) {
  return wdtype == XE_BF16 ? 2 * n : wdtype == XE_BFP16 ? n + n / 8 : n;
}

// A device-resident weight matrix (rows x cols).
struct Mat {
  int rows = 0, cols = 0, wdtype = XE_I8;
  void *w = nullptr;
  float *scale = nullptr;
  uint8_t *exps = nullptr;
  void alloc(int r, int c, int dt) {
    rows = r;
    cols = c;
    wdtype = dt;
    const size_t n = static_cast<size_t>(r) * c;
    XE_HIP(hipMalloc(&w, wbytes(dt, n) - (dt == XE_BFP16 ? n / 8 : 0)));
    if (dt == XE_I8) XE_HIP(hipMalloc(&scale, r * sizeof(float)));
    if (dt == XE_BFP16) XE_HIP(hipMalloc(&exps, n / 8));
  }
  void release() {
    (void)hipFree(w);
    (void)hipFree(scale);
    (void)hipFree(exps);
    w = nullptr;
    scale = nullptr;
    exps = nullptr;
  }
  size_t bytes() const {
    const size_t n = static_cast<size_t>(rows) * cols;
    return wbytes(wdtype, n) + (wdtype == XE_I8 ? rows * sizeof(float) : 0);
  }
};

// Where a tensor lives: a matrix (with row offset / stride) or a vector.
struct Place {
  Mat *mat = nullptr;
  int row_off = 0, row_stride = 1;
  float *vec = nullptr;  // f32 destination (vectors, position table, encoder)
};

struct Layer {
  Mat qkv, o, fc1, fc2;               // fc1 = gate/up interleaved for Gemma
  Mat xq, xk, xv, xo;                 // Whisper cross attention
  float *qkv_b = nullptr, *o_b = nullptr, *fc1_b = nullptr, *fc2_b = nullptr;
  float *ln1_w = nullptr, *ln1_b = nullptr, *ln2_w = nullptr, *ln2_b = nullptr;
  float *qn = nullptr, *kn = nullptr, *post_attn = nullptr, *post_ffn = nullptr;
  float *lnx_w = nullptr, *lnx_b = nullptr, *xq_b = nullptr, *xv_b = nullptr, *xo_b = nullptr;
  uint16_t *ck = nullptr, *cv = nullptr;  // Whisper cross K/V bf16 [H, T, hd]
};

template <typename T>
T *dalloc(size_t n, hipStream_t s, bool zero = true) {
  T *p = nullptr;
  XE_HIP(hipMalloc(reinterpret_cast<void **>(&p), std::max<size_t>(n, 1) * sizeof(T)));
  if (zero) XE_HIP(hipMemsetAsync(p, 0, std::max<size_t>(n, 1) * sizeof(T), s));
  return p;
}

}  // namespace
}  // namespace xe

using namespace xe;

struct xe_decoder {
  xe_device *dev = nullptr;
  xe_model_config c{};
  int max_batch = 1;
  hipStream_t s = nullptr;
  // weights
  Mat emb;
  float *pos_emb = nullptr;
  float *lnf_w = nullptr, *lnf_b = nullptr;
  float *enc = nullptr;  // Whisper synthetic / uploaded encoder output [T, D]
  std::vector<Layer> L;
  // state
  float *xa = nullptr, *xb = nullptr, *qkv = nullptr, *att = nullptr, *sub = nullptr;
  float *ffn = nullptr, *qx = nullptr, *logits = nullptr, *tmp = nullptr;
  uint16_t *kc = nullptr, *vc = nullptr;  // [L][B][hkv][max_ctx][hd]
  float *rope_cos = nullptr, *rope_sin = nullptr;
  int32_t *tokens = nullptr, *pos = nullptr, *next = nullptr, *hist = nullptr;
  float *arg_v = nullptr;
  int *arg_i = nullptr;
  float *attn_work = nullptr;
  int attn_splits = 1;
  int32_t *host_tok = nullptr;  // pinned staging [max_ctx + 1][max_batch] x 2
  std::map<int, hipGraphExec_t> graphs;
  double last_step_us = 0.0;
  bool cross_ready = false;
  int fed = 0;      // prompt length of the current streams
  int decoded = 0;  // steps decoded after the prompt
  // per-launch profiling (xe_decoder_profile_step): an event after each
  // launch on the decoder stream, with the launch's algorithmic bytes
  struct ProfEntry {
    std::string label;
    double bytes;
    hipEvent_t ev;
  };
  std::vector<ProfEntry> *prof = nullptr;
  std::vector<int32_t> prof_pos;  // host copy of positions for the byte counts
  void mark(const std::string &label, double bytes) {
    if (!prof) return;
    hipEvent_t e;
    XE_HIP(hipEventCreate(&e));
    XE_HIP(hipEventRecord(e, s));
    prof->push_back({label, bytes, e});
  }

  size_t nqkv() const { return static_cast<size_t>(c.n_heads + 2 * c.n_kv_heads) * c.head_dim; }
  size_t kv_layer_elems() const {
    return static_cast<size_t>(max_batch) * c.n_kv_heads * c.max_ctx * c.head_dim;
  }

  Place place(int kind, int layer) {
    Place p;
    if (layer < 0) {
      switch (kind) {
        case XE_T_TOK_EMB: p.mat = &emb; break;
        case XE_T_POS_EMB: p.vec = pos_emb; break;
        case XE_T_LNF_W: p.vec = lnf_w; break;
        case XE_T_LNF_B: p.vec = lnf_b; break;
        case XE_T_ENC_OUT: p.vec = enc; break;
      }
      return p;
    }
    Layer &l = L[layer];
    const int hq = c.n_heads * c.head_dim, hk = c.n_kv_heads * c.head_dim;
    const bool gem = c.family == XE_GEMMA3;
    switch (kind) {
      case XE_T_Q_W: p.mat = &l.qkv; break;
      case XE_T_K_W: p.mat = &l.qkv; p.row_off = hq; break;
      case XE_T_V_W: p.mat = &l.qkv; p.row_off = hq + hk; break;
      case XE_T_Q_B: p.vec = l.qkv_b; break;
      case XE_T_K_B: p.vec = l.qkv_b + hq; break;
      case XE_T_V_B: p.vec = l.qkv_b + hq + hk; break;
      case XE_T_O_W: p.mat = &l.o; break;
      case XE_T_O_B: p.vec = l.o_b; break;
      case XE_T_FC1_W: p.mat = &l.fc1; if (gem) p.row_stride = 2; break;
      case XE_T_UP_W: p.mat = &l.fc1; p.row_off = 1; p.row_stride = 2; break;
      case XE_T_FC1_B: p.vec = l.fc1_b; break;
      case XE_T_FC2_W: p.mat = &l.fc2; break;
      case XE_T_FC2_B: p.vec = l.fc2_b; break;
      case XE_T_LN1_W: p.vec = l.ln1_w; break;
      case XE_T_LN1_B: p.vec = l.ln1_b; break;
      case XE_T_LN2_W: p.vec = l.ln2_w; break;
      case XE_T_LN2_B: p.vec = l.ln2_b; break;
      case XE_T_QNORM_W: p.vec = l.qn; break;
      case XE_T_KNORM_W: p.vec = l.kn; break;
      case XE_T_POST_ATTN_W: p.vec = l.post_attn; break;
      case XE_T_POST_FFN_W: p.vec = l.post_ffn; break;
      case XE_T_LNX_W: p.vec = l.lnx_w; break;
      case XE_T_LNX_B: p.vec = l.lnx_b; break;
      case XE_T_XQ_W: p.mat = &l.xq; break;
      case XE_T_XQ_B: p.vec = l.xq_b; break;
      case XE_T_XK_W: p.mat = &l.xk; break;
      case XE_T_XV_W: p.mat = &l.xv; break;
      case XE_T_XV_B: p.vec = l.xv_b; break;
      case XE_T_XO_W: p.mat = &l.xo; break;
      case XE_T_XO_B: p.vec = l.xo_b; break;
    }
    return p;
  }
};

namespace {

void validate_config(const xe_model_config &c, int max_batch) {
  XE_REQUIRE(c.family >= XE_OPT && c.family <= XE_GEMMA3, "unknown model family");
  XE_REQUIRE(c.n_layers >= 1 && c.n_layers <= 64, "n_layers must be 1..64");
  XE_REQUIRE(c.d_model > 0 && c.d_model % 16 == 0, "d_model must be a positive multiple of 16");
  XE_REQUIRE(c.n_heads > 0 && c.n_kv_heads > 0 && c.n_heads % c.n_kv_heads == 0, "bad head counts");
  const int g = c.n_heads / c.n_kv_heads;
  XE_REQUIRE(g == 1 || g == 2 || g == 4 || g == 8, "GQA group must be 1, 2, 4 or 8");
  XE_REQUIRE(c.head_dim == 64 || c.head_dim == 128 || c.head_dim == 256, "head_dim must be 64/128/256");
  XE_REQUIRE(c.ffn > 0 && c.ffn % 16 == 0, "ffn must be a positive multiple of 16");
  XE_REQUIRE(c.vocab > 0, "vocab must be positive");
  XE_REQUIRE(c.max_ctx > 0 && c.max_ctx <= (1 << 20), "max_ctx out of range");
  XE_REQUIRE(c.wdtype == XE_I8 || c.wdtype == XE_BF16 || c.wdtype == XE_BFP16, "bad weight dtype");
  XE_REQUIRE(max_batch >= 1 && max_batch <= 1024, "max_batch must be 1..1024");
  if (c.family != XE_GEMMA3) XE_REQUIRE(c.max_pos > 0, "learned positions need max_pos");
  if (c.family == XE_WHISPER) XE_REQUIRE(c.n_cross > 0, "Whisper needs n_cross");
  if (c.family == XE_GEMMA3) XE_REQUIRE(c.rope_theta > 0, "Gemma needs rope_theta");
  if (c.family != XE_GEMMA3) XE_REQUIRE(c.n_heads == c.n_kv_heads, "OPT/Whisper are MHA");
}

void alloc_decoder(xe_decoder *d) {
  const auto &c = d->c;
  hipStream_t s = d->s;
  const int D = c.d_model, F = c.ffn, B = d->max_batch;
  const int hq = c.n_heads * c.head_dim, hk = c.n_kv_heads * c.head_dim;
  const bool gem = c.family == XE_GEMMA3, wh = c.family == XE_WHISPER;
  d->emb.alloc(c.vocab, D, c.wdtype);
  Spec sp;
  if (tensor_spec(c, XE_T_POS_EMB, -1, sp)) d->pos_emb = dalloc<float>(static_cast<size_t>(sp.rows) * D, s);
  d->lnf_w = dalloc<float>(D, s);
  d->lnf_b = dalloc<float>(D, s);
  if (wh) d->enc = dalloc<float>(static_cast<size_t>(c.n_cross) * D, s);
  d->L.resize(c.n_layers);
  for (auto &l : d->L) {
    l.qkv.alloc(hq + 2 * hk, D, c.wdtype);
    l.o.alloc(D, hq, c.wdtype);
    l.fc1.alloc(gem ? 2 * F : F, D, c.wdtype);
    l.fc2.alloc(D, F, c.wdtype);
    l.qkv_b = dalloc<float>(hq + 2 * hk, s);
    l.o_b = dalloc<float>(D, s);
    l.fc1_b = dalloc<float>(F, s);
    l.fc2_b = dalloc<float>(D, s);
    l.ln1_w = dalloc<float>(D, s);
    l.ln1_b = dalloc<float>(D, s);
    l.ln2_w = dalloc<float>(D, s);
    l.ln2_b = dalloc<float>(D, s);
    if (gem) {
      l.qn = dalloc<float>(c.head_dim, s);
      l.kn = dalloc<float>(c.head_dim, s);
      l.post_attn = dalloc<float>(D, s);
      l.post_ffn = dalloc<float>(D, s);
    }
    if (wh) {
      l.xq.alloc(D, D, c.wdtype);
      l.xk.alloc(D, D, c.wdtype);
      l.xv.alloc(D, D, c.wdtype);
      l.xo.alloc(D, D, c.wdtype);
      l.lnx_w = dalloc<float>(D, s);
      l.lnx_b = dalloc<float>(D, s);
      l.xq_b = dalloc<float>(D, s);
      l.xv_b = dalloc<float>(D, s);
      l.xo_b = dalloc<float>(D, s);
      l.ck = dalloc<uint16_t>(static_cast<size_t>(c.n_cross) * D, s);
      l.cv = dalloc<uint16_t>(static_cast<size_t>(c.n_cross) * D, s);
    }
  }
  d->xa = dalloc<float>(static_cast<size_t>(B) * D, s);
  d->xb = dalloc<float>(static_cast<size_t>(B) * D, s);
  d->qkv = dalloc<float>(static_cast<size_t>(B) * d->nqkv(), s);
  d->att = dalloc<float>(static_cast<size_t>(B) * std::max(hq, D), s);
  d->sub = dalloc<float>(static_cast<size_t>(B) * D, s);
  d->ffn = dalloc<float>(static_cast<size_t>(B) * F, s);
  d->qx = dalloc<float>(static_cast<size_t>(B) * D, s);
  d->logits = dalloc<float>(static_cast<size_t>(B) * c.vocab, s);
  const size_t kvn = d->kv_layer_elems() * c.n_layers;
  d->kc = dalloc<uint16_t>(kvn, s);
  d->vc = dalloc<uint16_t>(kvn, s);
  d->tokens = dalloc<int32_t>(B, s);
  d->pos = dalloc<int32_t>(B, s);
  d->next = dalloc<int32_t>(B, s);
  d->hist = dalloc<int32_t>(static_cast<size_t>(B) * (c.max_ctx + 1), s);
  d->arg_v = dalloc<float>(static_cast<size_t>(B) * kArgBlocks, s);
  d->arg_i = dalloc<int>(static_cast<size_t>(B) * kArgBlocks, s);
  // split-K attention: ~4 workgroups per CU at the largest batch, chunks >= 32 keys
  const int hkv_max = std::max(c.n_kv_heads, wh ? c.n_heads : 0);
  int ms = (4 * d->dev->num_cus) / std::max(1, hkv_max);
  const int cap = (std::max(c.max_ctx, wh ? c.n_cross : 0) + 63) / 64;
  ms = std::max(1, std::min(std::min(ms, cap), 64));
  d->attn_splits = ms;
  d->attn_work = dalloc<float>(attn_work_floats(B, std::max(c.n_heads, 1), c.head_dim, ms), s, false);
  if (gem) {
    const int half = c.head_dim / 2;
    std::vector<float> cs(static_cast<size_t>(c.max_ctx) * half), sn(cs.size());
    // HF rotary embedding in f32: inv_freq = 1 / theta^(2i/d); angle = pos * inv_freq
    for (int p = 0; p < c.max_ctx; p++)
      for (int i = 0; i < half; i++) {
        const float e = static_cast<float>(2 * i) / static_cast<float>(c.head_dim);
        const float inv = 1.0f / powf(c.rope_theta, e);
        const float ang = static_cast<float>(p) * inv;
        cs[static_cast<size_t>(p) * half + i] = cosf(ang);
        sn[static_cast<size_t>(p) * half + i] = sinf(ang);
      }
    d->rope_cos = dalloc<float>(cs.size(), s, false);
    d->rope_sin = dalloc<float>(sn.size(), s, false);
    XE_HIP(hipMemcpyAsync(d->rope_cos, cs.data(), cs.size() * 4, hipMemcpyHostToDevice, s));
    XE_HIP(hipMemcpyAsync(d->rope_sin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice, s));
  }
  XE_HIP(hipHostMalloc(reinterpret_cast<void **>(&d->host_tok),
                       static_cast<size_t>(2) * (c.max_ctx + 2) * B * sizeof(int32_t),
                       hipHostMallocDefault));
  XE_HIP(hipStreamSynchronize(s));
}

void free_decoder(xe_decoder *d) {
  if (d->s) (void)hipStreamSynchronize(d->s);
  for (auto &kv : d->graphs) (void)hipGraphExecDestroy(kv.second);
  d->emb.release();
  for (auto &l : d->L) {
    for (Mat *m : {&l.qkv, &l.o, &l.fc1, &l.fc2, &l.xq, &l.xk, &l.xv, &l.xo}) m->release();
    for (void *p : {static_cast<void *>(l.qkv_b), static_cast<void *>(l.o_b),
                    static_cast<void *>(l.fc1_b), static_cast<void *>(l.fc2_b),
                    static_cast<void *>(l.ln1_w), static_cast<void *>(l.ln1_b),
                    static_cast<void *>(l.ln2_w), static_cast<void *>(l.ln2_b),
                    static_cast<void *>(l.qn), static_cast<void *>(l.kn),
                    static_cast<void *>(l.post_attn), static_cast<void *>(l.post_ffn),
                    static_cast<void *>(l.lnx_w), static_cast<void *>(l.lnx_b),
                    static_cast<void *>(l.xq_b), static_cast<void *>(l.xv_b),
                    static_cast<void *>(l.xo_b), static_cast<void *>(l.ck),
                    static_cast<void *>(l.cv)})
      if (p) (void)hipFree(p);
  }
  for (void *p : {static_cast<void *>(d->pos_emb), static_cast<void *>(d->lnf_w),
                  static_cast<void *>(d->lnf_b), static_cast<void *>(d->enc),
                  static_cast<void *>(d->xa), static_cast<void *>(d->xb),
                  static_cast<void *>(d->qkv), static_cast<void *>(d->att),
                  static_cast<void *>(d->sub), static_cast<void *>(d->ffn),
                  static_cast<void *>(d->qx), static_cast<void *>(d->logits),
                  static_cast<void *>(d->kc), static_cast<void *>(d->vc),
                  static_cast<void *>(d->rope_cos), static_cast<void *>(d->rope_sin),
                  static_cast<void *>(d->tokens), static_cast<void *>(d->pos),
                  static_cast<void *>(d->next), static_cast<void *>(d->hist),
                  static_cast<void *>(d->arg_v), static_cast<void *>(d->arg_i),
                  static_cast<void *>(d->attn_work)})
    if (p) (void)hipFree(p);
  if (d->host_tok) (void)hipHostFree(d->host_tok);
  if (d->s) (void)hipStreamDestroy(d->s);
}

// ---- one GEMV over `batch` rows, chunked by 8 (the GEMV kernel's limit) ----
struct GemvCall {
  const Mat *m = nullptr;
  const float *bias = nullptr;
  const float *x = nullptr;
  int ldx = 0;
  const float *sub = nullptr;
  const float *post_w = nullptr;
  float *res_out = nullptr;
  int norm = XE_NORM_NONE;
  const float *gamma = nullptr, *beta = nullptr;
  float eps = 1e-5f;
  int act = ACT_NONE;
  float *y = nullptr;
  int ldy = 0;
};

// Algorithmic bytes of one GEMV over `batch` rows: weights (+ int8 scales,
// bias), activations in, outputs out, and the residual prologue's traffic.
double gemv_bytes(const GemvCall &g, int batch) {
  const Mat &m = *g.m;
  double b = static_cast<double>(m.bytes());
  if (g.bias) b += 4.0 * m.rows;
  const int out_cols = g.act == ACT_GEGLU_TANH ? m.rows / 2 : m.rows;
  b += 4.0 * batch * (static_cast<double>(m.cols) + out_cols);
  if (g.sub) b += 4.0 * batch * m.cols * (g.res_out ? 2 : 1);
  return b;
}

void run_gemv(const GemvCall &g, int batch, hipStream_t s) {
  for (int b0 = 0; b0 < batch; b0 += 8) {
    const int nb = std::min(8, batch - b0);
    GemvLaunch p;
    p.wdtype = g.m->wdtype;
    p.w = g.m->w;
    p.scale = g.m->scale;
    p.exps = g.m->exps;
    p.bias = g.bias;
    p.m = g.m->rows;
    p.k = g.m->cols;
    p.x = g.x + static_cast<size_t>(b0) * g.ldx;
    p.x_dtype = XE_F32;
    p.ldx = g.ldx;
    p.batch = nb;
    p.sub = g.sub ? g.sub + static_cast<size_t>(b0) * g.m->cols : nullptr;
    p.post_w = g.post_w;
    p.res_out = g.res_out ? g.res_out + static_cast<size_t>(b0) * g.m->cols : nullptr;
    p.norm = g.norm;
    p.gamma = g.gamma;
    p.beta = g.beta;
    p.eps = g.eps;
    p.act = g.act;
    p.y = g.y + static_cast<size_t>(b0) * g.ldy;
    p.ldy = g.ldy;
    launch_gemv(p, s);
  }
}

// Enqueue one decode step for streams [0, B) (tokens/pos already on device).
void enqueue_step(xe_decoder *d, int B) {
  const auto &c = d->c;
  hipStream_t s = d->s;
  const int D = c.d_model, F = c.ffn, hd = c.head_dim;
  const int hq = c.n_heads * hd, hk = c.n_kv_heads * hd;
  const bool gem = c.family == XE_GEMMA3, wh = c.family == XE_WHISPER, opt = c.family == XE_OPT;
  const int nq = static_cast<int>(d->nqkv());
  const int norm = gem ? XE_NORM_RMS1P : XE_NORM_LN;

  // embedding
  {
    const int pos_off = opt ? 2 : 0;
    Spec sp;
    const int prow = tensor_spec(c, XE_T_POS_EMB, -1, sp) ? sp.rows : 1;
    dim3 grid((D + 255) / 256, B);
    hipLaunchKernelGGL(embed_kernel, grid, dim3(256), 0, s, d->emb.w, d->emb.scale, d->emb.exps,
                       c.wdtype, d->pos_emb, pos_off, prow, sqrtf(static_cast<float>(D)),
                       gem ? 1 : 0, d->tokens, d->pos, c.vocab, D, d->xa);
    XE_HIP(hipGetLastError());
    d->mark("embed", static_cast<double>(B) * D * (wbytes(c.wdtype, 1) + 4 + (d->pos_emb ? 4 : 0)));
  }
  float *xcur = d->xa, *xalt = d->xb;
  const float *pend = nullptr, *pend_post = nullptr;
  auto take_pending = [&](GemvCall &g) {
    g.x = xcur;
    g.ldx = D;
    if (pend) {
      g.sub = pend;
      g.post_w = pend_post;
      g.res_out = xalt;
    }
  };
  auto after_pending = [&]() {
    if (pend) std::swap(xcur, xalt);
    pend = nullptr;
    pend_post = nullptr;
  };

  for (int li = 0; li < c.n_layers; li++) {
    Layer &l = d->L[li];
    // ---- norm + QKV ----
    {
      GemvCall g;
      g.m = &l.qkv;
      g.bias = gem ? nullptr : l.qkv_b;
      take_pending(g);
      g.norm = norm;
      g.gamma = l.ln1_w;
      g.beta = gem ? nullptr : l.ln1_b;
      g.eps = c.eps;
      g.y = d->qkv;
      g.ldy = nq;
      run_gemv(g, B, s);
      d->mark("gemv_qkv", gemv_bytes(g, B));
      after_pending();
    }
    // ---- self attention (append k/v at pos) ----
    {
      AttnLaunch a;
      a.q = d->qkv;
      a.q_stride = nq;
      a.kc = d->kc + d->kv_layer_elems() * li;
      a.vc = d->vc + d->kv_layer_elems() * li;
      a.kv_batch_stride = static_cast<size_t>(c.n_kv_heads) * c.max_ctx * hd;
      a.max_ctx = c.max_ctx;
      a.batch = B;
      a.hq = c.n_heads;
      a.hkv = c.n_kv_heads;
      a.hd = hd;
      a.scale = opt ? powf(static_cast<float>(hd), -0.5f) : 1.0f / sqrtf(static_cast<float>(hd));
      a.pos = d->pos;
      a.k_new = d->qkv + hq;
      a.v_new = d->qkv + hq + hk;
      a.kv_new_stride = nq;
      if (gem) {
        a.q_norm_w = l.qn;
        a.k_norm_w = l.kn;
        a.norm_eps = c.eps;
        a.rope_cos = d->rope_cos;
        a.rope_sin = d->rope_sin;
      }
      a.div_norm = opt ? 1 : 0;
      a.out = d->att;
      a.out_stride = hq;
      a.work = d->attn_work;
      a.max_splits = d->attn_splits;
      launch_attn(a, s);
      if (d->prof) {
        double kv = 0;
        for (int b = 0; b < B; b++) kv += static_cast<double>(d->prof_pos[b] + 1) * hk * 2 * 2;
        d->mark("attn_self", kv + 4.0 * B * (nq + hq) + 4.0 * B * hk);
      }
    }
    // ---- O projection ----
    {
      GemvCall g;
      g.m = &l.o;
      g.bias = gem ? nullptr : l.o_b;
      g.x = d->att;
      g.ldx = hq;
      g.y = d->sub;
      g.ldy = D;
      run_gemv(g, B, s);
      d->mark("gemv_o", gemv_bytes(g, B));
      pend = d->sub;
      pend_post = gem ? l.post_attn : nullptr;
    }
    // ---- Whisper cross attention ----
    if (wh) {
      GemvCall g;
      g.m = &l.xq;
      g.bias = l.xq_b;
      take_pending(g);
      g.norm = XE_NORM_LN;
      g.gamma = l.lnx_w;
      g.beta = l.lnx_b;
      g.eps = c.eps;
      g.y = d->qx;
      g.ldy = D;
      run_gemv(g, B, s);
      d->mark("gemv_xq", gemv_bytes(g, B));
      after_pending();
      AttnLaunch a;
      a.q = d->qx;
      a.q_stride = D;
      a.kc = l.ck;
      a.vc = l.cv;
      a.kv_batch_stride = 0;  // one encoder output shared by every stream
      a.max_ctx = c.n_cross;
      a.batch = B;
      a.hq = c.n_heads;
      a.hkv = c.n_heads;
      a.hd = hd;
      a.scale = 1.0f / sqrtf(static_cast<float>(hd));
      a.fixed_len = c.n_cross;
      a.out = d->att;
      a.out_stride = D;
      a.work = d->attn_work;
      a.max_splits = d->attn_splits;
      launch_attn(a, s);
      d->mark("attn_cross", static_cast<double>(c.n_cross) * D * 2 * 2 + 8.0 * B * D);
      GemvCall o;
      o.m = &l.xo;
      o.bias = l.xo_b;
      o.x = d->att;
      o.ldx = D;
      o.y = d->sub;
      o.ldy = D;
      run_gemv(o, B, s);
      d->mark("gemv_xo", gemv_bytes(o, B));
      pend = d->sub;
      pend_post = nullptr;
    }
    // ---- FFN ----
    {
      GemvCall g;
      g.m = &l.fc1;
      g.bias = gem ? nullptr : l.fc1_b;
      take_pending(g);
      g.norm = norm;
      g.gamma = l.ln2_w;
      g.beta = gem ? nullptr : l.ln2_b;
      g.eps = c.eps;
      g.act = gem ? ACT_GEGLU_TANH : (opt ? ACT_RELU : ACT_GELU_ERF);
      g.y = d->ffn;
      g.ldy = F;
      run_gemv(g, B, s);
      d->mark(gem ? "gemv_gateup" : "gemv_fc1", gemv_bytes(g, B));
      after_pending();
      GemvCall o;
      o.m = &l.fc2;
      o.bias = gem ? nullptr : l.fc2_b;
      o.x = d->ffn;
      o.ldx = F;
      o.y = d->sub;
      o.ldy = D;
      run_gemv(o, B, s);
      d->mark(gem ? "gemv_down" : "gemv_fc2", gemv_bytes(o, B));
      pend = d->sub;
      pend_post = gem ? l.post_ffn : nullptr;
    }
  }
  // ---- final norm + tied lm-head ----
  {
    GemvCall g;
    g.m = &d->emb;
    take_pending(g);
    g.res_out = nullptr;  // the residual is not needed after the head
    g.norm = norm;
    g.gamma = d->lnf_w;
    g.beta = gem ? nullptr : d->lnf_b;
    g.eps = c.eps;
    g.y = d->logits;
    g.ldy = c.vocab;
    run_gemv(g, B, s);
    d->mark("gemv_lmhead", gemv_bytes(g, B));
  }
  // ---- greedy argmax -> next token, pos + 1 ----
  hipLaunchKernelGGL(argmax_partial_kernel, dim3(kArgBlocks, B), dim3(256), 0, s, d->logits,
                     c.vocab, opt ? 1 : 0, d->arg_v, d->arg_i);
  XE_HIP(hipGetLastError());
  hipLaunchKernelGGL(argmax_final_kernel, dim3(B), dim3(64), 0, s, d->arg_v, d->arg_i,
                     opt ? 1 : 0, d->next, d->tokens, d->pos, d->hist, c.max_ctx + 1);
  XE_HIP(hipGetLastError());
  d->mark("argmax", 4.0 * B * c.vocab);
}

hipGraphExec_t graph_for(xe_decoder *d, int B) {
  auto it = d->graphs.find(B);
  if (it != d->graphs.end()) return it->second;
  hipGraph_t g = nullptr;
  XE_HIP(hipStreamBeginCapture(d->s, hipStreamCaptureModeRelaxed));
  try {
    enqueue_step(d, B);
  } catch (...) {
    hipGraph_t junk = nullptr;
    (void)hipStreamEndCapture(d->s, &junk);
    if (junk) (void)hipGraphDestroy(junk);
    throw;
  }
  XE_HIP(hipStreamEndCapture(d->s, &g));
  hipGraphExec_t ex = nullptr;
  XE_HIP(hipGraphInstantiate(&ex, g, nullptr, nullptr, 0));
  (void)hipGraphDestroy(g);
  d->graphs[B] = ex;
  return ex;
}

void run_step(xe_decoder *d, int B) {
  if (getenv("XE_NO_GRAPH")) {
    enqueue_step(d, B);
    return;
  }
  XE_HIP(hipGraphLaunch(graph_for(d, B), d->s));
}

void synth_matrix(xe_decoder *d, uint64_t seed, int kind, int layer, const Spec &sp, const Place &p) {
  const uint64_t base = synth_base(seed, XE_SYNTH_ID(kind, layer));
  const float k = sp.stdv * kIh4InvStd;
  hipLaunchKernelGGL(synth_rows_kernel, dim3(sp.rows), dim3(256), 0, d->s, base, sp.mean, k,
                     sp.rows, sp.cols, p.mat->wdtype, p.row_off, p.row_stride, p.mat->w,
                     p.mat->scale, p.mat->exps);
  XE_HIP(hipGetLastError());
}

void synth_vector(xe_decoder *d, uint64_t seed, int kind, int layer, const Spec &sp, float *dst,
                  int round_bf16) {
  const uint64_t base = synth_base(seed, XE_SYNTH_ID(kind, layer));
  const float k = sp.stdv * kIh4InvStd;
  const size_t n = static_cast<size_t>(sp.rows) * sp.cols;
  const int blocks = static_cast<int>(std::min<size_t>((n + 255) / 256, 4096));
  hipLaunchKernelGGL(synth_vec_kernel, dim3(blocks), dim3(256), 0, d->s, base, sp.mean, k, n, dst,
                     round_bf16);
  XE_HIP(hipGetLastError());
}

void upload_matrix(xe_decoder *d, const Spec &sp, const Place &p, const float *w) {
  const Mat &m = *p.mat;
  const size_t n = static_cast<size_t>(sp.rows) * sp.cols;
  std::vector<int8_t> q;
  std::vector<float> sc;
  std::vector<uint16_t> bf;
  std::vector<uint8_t> ex;
  if (m.wdtype == XE_I8) {
    q.resize(n);
    sc.resize(sp.rows);
    quant_rows_i8(w, sp.rows, sp.cols, q.data(), sc.data());
  } else if (m.wdtype == XE_BF16) {
    bf.resize(n);
    for (size_t i = 0; i < n; i++) bf[i] = f32_to_bf16_bits(w[i]);
  } else {
    q.resize(n);
    ex.resize(n / 8);
    bfp16_encode(w, sp.rows, sp.cols, q.data(), ex.data());
  }
  const size_t rb = m.wdtype == XE_BF16 ? 2 * static_cast<size_t>(sp.cols) : sp.cols;
  for (int r = 0; r < sp.rows; r++) {
    const int dr = p.row_off + r * p.row_stride;
    char *dst = static_cast<char *>(m.w) + static_cast<size_t>(dr) * rb;
    const void *src = m.wdtype == XE_BF16 ? static_cast<const void *>(bf.data() + static_cast<size_t>(r) * sp.cols)
                                          : static_cast<const void *>(q.data() + static_cast<size_t>(r) * sp.cols);
    XE_HIP(hipMemcpyAsync(dst, src, rb, hipMemcpyHostToDevice, d->s));
    if (m.wdtype == XE_I8)
      XE_HIP(hipMemcpyAsync(m.scale + dr, sc.data() + r, 4, hipMemcpyHostToDevice, d->s));
    if (m.wdtype == XE_BFP16)
      XE_HIP(hipMemcpyAsync(m.exps + static_cast<size_t>(dr) * (sp.cols / 8),
                            ex.data() + static_cast<size_t>(r) * (sp.cols / 8), sp.cols / 8,
                            hipMemcpyHostToDevice, d->s));
  }
  XE_HIP(hipStreamSynchronize(d->s));
}

void precompute_cross(xe_decoder *d) {
  const auto &c = d->c;
  const int D = c.d_model, T = c.n_cross;
  float *tmp = dalloc<float>(static_cast<size_t>(T) * D, d->s, false);
  struct Free {
    float *p;
    ~Free() { (void)hipFree(p); }
  } fr{tmp};
  for (int li = 0; li < c.n_layers; li++) {
    Layer &l = d->L[li];
    for (int which = 0; which < 2; which++) {
      GemvCall g;
      g.m = which == 0 ? &l.xk : &l.xv;
      g.bias = which == 0 ? nullptr : l.xv_b;
      g.x = d->enc;
      g.ldx = D;
      g.y = tmp;
      g.ldy = D;
      run_gemv(g, T, d->s);
      hipLaunchKernelGGL(cross_pack_kernel, dim3(1024), dim3(256), 0, d->s, tmp, T, c.n_heads,
                         c.head_dim, which == 0 ? l.ck : l.cv);
      XE_HIP(hipGetLastError());
    }
  }
  XE_HIP(hipStreamSynchronize(d->s));
  d->cross_ready = true;
}

template <typename F>
auto guard_d(F &&f, decltype(f()) on_error) -> decltype(f()) {
  try {
    set_error("");
    return f();
  } catch (const std::exception &e) {
    set_error(e.what());
  } catch (...) {
    set_error("unknown C++ exception");
  }
  return on_error;
}

}  // namespace

extern "C" {

xe_decoder *xe_decoder_create(xe_device *dev, const xe_model_config *cfg, int max_batch) {
  return guard_d([&]() -> xe_decoder * {
    XE_REQUIRE(dev && cfg, "null argument");
    validate_config(*cfg, max_batch);
    DeviceGuard dg(dev->ordinal);
    auto *d = new xe_decoder;
    d->dev = dev;
    d->c = *cfg;
    d->max_batch = max_batch;
    try {
      XE_HIP(hipStreamCreateWithFlags(&d->s, hipStreamNonBlocking));
      alloc_decoder(d);
    } catch (...) {
      free_decoder(d);
      delete d;
      throw;
    }
    return d;
  }, nullptr);
}

void xe_decoder_destroy(xe_decoder *dec) {
  guard_d([&]() -> int {
    if (!dec) return 0;
    DeviceGuard dg(dec->dev->ordinal);
    free_decoder(dec);
    delete dec;
    return 0;
  }, -1);
}

int xe_decoder_init_synthetic(xe_decoder *d, uint64_t seed) {
  return guard_d([&]() -> int {
    XE_REQUIRE(d, "null decoder");
    DeviceGuard dg(d->dev->ordinal);
    for (int kind = 0; kind < XE_T_COUNT; kind++)
      for (int layer = -1; layer < d->c.n_layers; layer++) {
        Spec sp;
        if (!tensor_spec(d->c, kind, layer, sp)) continue;
        Place p = d->place(kind, layer);
        if (sp.quant) {
          XE_REQUIRE(p.mat, "internal: quantised tensor without a matrix");
          synth_matrix(d, seed, kind, layer, sp, p);
        } else {
          XE_REQUIRE(p.vec, "internal: vector tensor without storage");
          synth_vector(d, seed, kind, layer, sp, p.vec, kind == XE_T_ENC_OUT);
        }
      }
    XE_HIP(hipStreamSynchronize(d->s));
    d->cross_ready = false;
    if (d->c.family == XE_WHISPER) precompute_cross(d);
    return 0;
  }, -1);
}

int xe_decoder_set_tensor(xe_decoder *d, int kind, int layer, const float *data, size_t count) {
  return guard_d([&]() -> int {
    XE_REQUIRE(d && data, "null argument");
    XE_REQUIRE(kind >= 0 && kind < XE_T_COUNT, "unknown tensor kind");
    XE_REQUIRE(layer >= -1 && layer < d->c.n_layers, "layer out of range");
    Spec sp;
    XE_REQUIRE(tensor_spec(d->c, kind, layer, sp), "tensor kind not used by this model family");
    XE_REQUIRE(count == static_cast<size_t>(sp.rows) * sp.cols, "tensor element count mismatch");
    DeviceGuard dg(d->dev->ordinal);
    Place p = d->place(kind, layer);
    if (sp.quant) {
      upload_matrix(d, sp, p, data);
    } else {
      std::vector<float> tmp(data, data + count);
      if (kind == XE_T_ENC_OUT)
        for (auto &v : tmp) v = bf16_round(v);
      XE_HIP(hipMemcpyAsync(p.vec, tmp.data(), count * 4, hipMemcpyHostToDevice, d->s));
      XE_HIP(hipStreamSynchronize(d->s));
    }
    if (kind == XE_T_XK_W || kind == XE_T_XV_W || kind == XE_T_XV_B || kind == XE_T_ENC_OUT)
      d->cross_ready = false;
    return 0;
  }, -1);
}

int xe_decoder_get_tensor_q8(xe_decoder *d, int kind, int layer, int8_t *q, float *scales) {
  return guard_d([&]() -> int {
    XE_REQUIRE(d && q && scales, "null argument");
    XE_REQUIRE(d->c.wdtype == XE_I8, "model weights are not int8");
    Spec sp;
    XE_REQUIRE(kind >= 0 && kind < XE_T_COUNT && layer >= -1 && layer < d->c.n_layers &&
                   tensor_spec(d->c, kind, layer, sp) && sp.quant,
               "not a quantised tensor of this model");
    DeviceGuard dg(d->dev->ordinal);
    Place p = d->place(kind, layer);
    for (int r = 0; r < sp.rows; r++) {
      const int dr = p.row_off + r * p.row_stride;
      XE_HIP(hipMemcpyAsync(q + static_cast<size_t>(r) * sp.cols,
                            static_cast<int8_t *>(p.mat->w) + static_cast<size_t>(dr) * sp.cols,
                            sp.cols, hipMemcpyDeviceToHost, d->s));
      XE_HIP(hipMemcpyAsync(scales + r, p.mat->scale + dr, 4, hipMemcpyDeviceToHost, d->s));
    }
    XE_HIP(hipStreamSynchronize(d->s));
    return 0;
  }, -1);
}

int xe_decoder_reset(xe_decoder *d) {
  return guard_d([&]() -> int {
    XE_REQUIRE(d, "null decoder");
    DeviceGuard dg(d->dev->ordinal);
    const size_t kvn = d->kv_layer_elems() * d->c.n_layers;
    XE_HIP(hipMemsetAsync(d->kc, 0, kvn * 2, d->s));
    XE_HIP(hipMemsetAsync(d->vc, 0, kvn * 2, d->s));
    XE_HIP(hipStreamSynchronize(d->s));
    return 0;
  }, -1);
}

int xe_decoder_set_cross(xe_decoder *d, const float *enc) {
  return guard_d([&]() -> int {
    XE_REQUIRE(d, "null decoder");
    XE_REQUIRE(d->c.family == XE_WHISPER, "cross attention is Whisper-only");
    DeviceGuard dg(d->dev->ordinal);
    if (enc) {
      const size_t n = static_cast<size_t>(d->c.n_cross) * d->c.d_model;
      std::vector<float> tmp(enc, enc + n);
      for (auto &v : tmp) v = bf16_round(v);
      XE_HIP(hipMemcpyAsync(d->enc, tmp.data(), n * 4, hipMemcpyHostToDevice, d->s));
    }
    precompute_cross(d);
    return 0;
  }, -1);
}

int xe_decoder_step(xe_decoder *d, const int32_t *tokens, const int32_t *pos, int batch,
                    float *logits, int32_t *next) {
  return guard_d([&]() -> int {
    XE_REQUIRE(d && tokens && pos, "null argument");
    XE_REQUIRE(batch >= 1 && batch <= d->max_batch, "batch out of range");
    XE_REQUIRE(d->c.family != XE_WHISPER || d->cross_ready, "Whisper: set_cross first");
    for (int b = 0; b < batch; b++) {
      XE_REQUIRE(tokens[b] >= 0 && tokens[b] < d->c.vocab, "token id out of range");
      XE_REQUIRE(pos[b] >= 0 && pos[b] < d->c.max_ctx, "position out of range");
      if (d->c.family == XE_OPT) XE_REQUIRE(pos[b] < d->c.max_pos, "position beyond the table");
      if (d->c.family == XE_WHISPER) XE_REQUIRE(pos[b] < d->c.max_pos, "position beyond the table");
    }
    DeviceGuard dg(d->dev->ordinal);
    int32_t *h = d->host_tok;
    XE_HIP(hipStreamSynchronize(d->s));  // staging reuse
    std::memcpy(h, tokens, batch * 4);
    std::memcpy(h + batch, pos, batch * 4);
    XE_HIP(hipMemcpyAsync(d->tokens, h, batch * 4, hipMemcpyHostToDevice, d->s));
    XE_HIP(hipMemcpyAsync(d->pos, h + batch, batch * 4, hipMemcpyHostToDevice, d->s));
    run_step(d, batch);
    if (logits)
      XE_HIP(hipMemcpyAsync(logits, d->logits, static_cast<size_t>(batch) * d->c.vocab * 4,
                            hipMemcpyDeviceToHost, d->s));
    if (next) XE_HIP(hipMemcpyAsync(next, d->next, batch * 4, hipMemcpyDeviceToHost, d->s));
    XE_HIP(hipStreamSynchronize(d->s));
    return 0;
  }, -1);
}

}  // extern "C"

namespace {

void check_ready(xe_decoder *d, int batch) {
  XE_REQUIRE(batch >= 1 && batch <= d->max_batch, "batch out of range");
  XE_REQUIRE(d->c.family != XE_WHISPER || d->cross_ready, "Whisper: set_cross first");
}

// Positions start at 0; the prompt's tokens are fed one step at a time (the
// argmax kernel leaves the next token and pos + 1 on the device).
void feed(xe_decoder *d, const int32_t *prompt, int n_prompt, int batch) {
  check_ready(d, batch);
  XE_REQUIRE(prompt && n_prompt >= 1, "empty prompt");
  XE_REQUIRE(n_prompt <= d->c.max_ctx, "prompt exceeds max_ctx");
  if (d->c.family != XE_GEMMA3) XE_REQUIRE(n_prompt <= d->c.max_pos, "prompt exceeds the position table");
  for (size_t i = 0; i < static_cast<size_t>(batch) * n_prompt; i++)
    XE_REQUIRE(prompt[i] >= 0 && prompt[i] < d->c.vocab, "prompt token out of range");
  XE_HIP(hipStreamSynchronize(d->s));
  int32_t *h = d->host_tok;
  XE_REQUIRE(static_cast<size_t>(n_prompt + 1) * batch <= static_cast<size_t>(2) * (d->c.max_ctx + 2) * d->max_batch,
             "prompt too long for staging");
  for (int p = 0; p < n_prompt; p++)
    for (int b = 0; b < batch; b++) h[static_cast<size_t>(p) * batch + b] = prompt[static_cast<size_t>(b) * n_prompt + p];
  int32_t *zpos = h + static_cast<size_t>(n_prompt) * batch;
  for (int b = 0; b < batch; b++) zpos[b] = 0;
  XE_HIP(hipMemcpyAsync(d->pos, zpos, batch * 4, hipMemcpyHostToDevice, d->s));
  if (!getenv("XE_NO_GRAPH")) (void)graph_for(d, batch);
  for (int p = 0; p < n_prompt; p++) {
    XE_HIP(hipMemcpyAsync(d->tokens, h + static_cast<size_t>(p) * batch, batch * 4,
                          hipMemcpyHostToDevice, d->s));
    run_step(d, batch);
  }
  XE_HIP(hipStreamSynchronize(d->s));
  d->fed = n_prompt;
  d->decoded = 0;
}

// n_steps further greedy steps from the device state; out [batch, n_steps]
// receives the tokens those steps emit (may be NULL).
void decode(xe_decoder *d, int batch, int n_steps, int32_t *out, double *device_us) {
  check_ready(d, batch);
  XE_REQUIRE(d->fed > 0, "feed a prompt first");
  XE_REQUIRE(n_steps >= 0, "negative step count");
  const int first_pos = d->fed + d->decoded;  // position the next step processes
  XE_REQUIRE(first_pos + n_steps <= d->c.max_ctx, "decode would run past max_ctx");
  if (d->c.family != XE_GEMMA3)
    XE_REQUIRE(first_pos + n_steps <= d->c.max_pos, "decode would run past the position table");
  hipEvent_t e0, e1;
  XE_HIP(hipEventCreate(&e0));
  XE_HIP(hipEventCreate(&e1));
  XE_HIP(hipEventRecord(e0, d->s));
  for (int i = 0; i < n_steps; i++) run_step(d, batch);
  XE_HIP(hipEventRecord(e1, d->s));
  XE_HIP(hipEventSynchronize(e1));
  float ms = 0.f;
  XE_HIP(hipEventElapsedTime(&ms, e0, e1));
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  if (n_steps > 0) d->last_step_us = 1000.0 * ms / n_steps;
  if (device_us) *device_us = 1000.0 * ms;
  d->decoded += n_steps;
  if (out && n_steps > 0) {
    std::vector<int32_t> hist(static_cast<size_t>(batch) * (d->c.max_ctx + 1));
    XE_HIP(hipMemcpy(hist.data(), d->hist, hist.size() * 4, hipMemcpyDeviceToHost));
    for (int b = 0; b < batch; b++)
      for (int i = 0; i < n_steps; i++)
        out[static_cast<size_t>(b) * n_steps + i] =
            hist[static_cast<size_t>(b) * (d->c.max_ctx + 1) + first_pos + i];
  }
}

}  // namespace

extern "C" {

int xe_decoder_feed(xe_decoder *d, const int32_t *prompt, int n_prompt, int batch) {
  return guard_d([&]() -> int {
    XE_REQUIRE(d, "null decoder");
    DeviceGuard dg(d->dev->ordinal);
    feed(d, prompt, n_prompt, batch);
    return 0;
  }, -1);
}

int xe_decoder_decode(xe_decoder *d, int batch, int n_steps, int32_t *out, double *device_us) {
  return guard_d([&]() -> int {
    XE_REQUIRE(d, "null decoder");
    DeviceGuard dg(d->dev->ordinal);
    decode(d, batch, n_steps, out, device_us);
    return 0;
  }, -1);
}

int xe_decoder_generate(xe_decoder *d, const int32_t *prompt, int n_prompt, int batch, int n_new,
                        int32_t *out) {
  return guard_d([&]() -> int {
    XE_REQUIRE(d && prompt && out, "null argument");
    XE_REQUIRE(n_new >= 1, "need at least one new token");
    XE_REQUIRE(n_prompt + n_new - 1 <= d->c.max_ctx, "prompt + new tokens exceed max_ctx");
    DeviceGuard dg(d->dev->ordinal);
    feed(d, prompt, n_prompt, batch);
    // the first new token was emitted by the last prompt step (hist[pos n_prompt-1])
    std::vector<int32_t> first(batch);
    {
      std::vector<int32_t> hist(static_cast<size_t>(batch) * (d->c.max_ctx + 1));
      XE_HIP(hipMemcpy(hist.data(), d->hist, hist.size() * 4, hipMemcpyDeviceToHost));
      for (int b = 0; b < batch; b++) first[b] = hist[static_cast<size_t>(b) * (d->c.max_ctx + 1) + n_prompt - 1];
    }
    std::vector<int32_t> rest(static_cast<size_t>(batch) * std::max(0, n_new - 1));
    decode(d, batch, n_new - 1, rest.data(), nullptr);
    for (int b = 0; b < batch; b++) {
      out[static_cast<size_t>(b) * n_new] = first[b];
      for (int i = 0; i + 1 < n_new; i++)
        out[static_cast<size_t>(b) * n_new + 1 + i] = rest[static_cast<size_t>(b) * (n_new - 1) + i];
    }
    return 0;
  }, -1);
}

int xe_decoder_profile_step(xe_decoder *d, int batch, int max_entries, char *labels, double *us,
                            double *bytes) {
  return guard_d([&]() -> int {
    XE_REQUIRE(d && labels && us && bytes, "null argument");
    check_ready(d, batch);
    XE_REQUIRE(d->fed > 0, "feed a prompt first");
    XE_REQUIRE(d->fed + d->decoded < d->c.max_ctx, "no room for another step");
    DeviceGuard dg(d->dev->ordinal);
    XE_HIP(hipStreamSynchronize(d->s));
    d->prof_pos.assign(batch, 0);
    XE_HIP(hipMemcpy(d->prof_pos.data(), d->pos, batch * 4, hipMemcpyDeviceToHost));
    std::vector<xe_decoder::ProfEntry> entries;
    d->prof = &entries;
    try {
      d->mark("start", 0.0);
      enqueue_step(d, batch);  // eager, one event after each launch
    } catch (...) {
      d->prof = nullptr;
      for (auto &e : entries) (void)hipEventDestroy(e.ev);
      throw;
    }
    d->prof = nullptr;
    XE_HIP(hipStreamSynchronize(d->s));
    d->decoded += 1;
    int n = 0;
    for (size_t i = 1; i < entries.size() && n < max_entries; i++, n++) {
      float ms = 0.f;
      XE_HIP(hipEventElapsedTime(&ms, entries[i - 1].ev, entries[i].ev));
      us[n] = 1000.0 * ms;
      bytes[n] = entries[i].bytes;
      std::snprintf(labels + 32 * n, 32, "%s", entries[i].label.c_str());
    }
    for (auto &e : entries) (void)hipEventDestroy(e.ev);
    return n;
  }, -1);
}

double xe_decoder_last_step_us(xe_decoder *d) { return d ? d->last_step_us : 0.0; }

uint64_t xe_decoder_weight_bytes(xe_decoder *d) {
  if (!d) return 0;
  uint64_t b = d->emb.bytes();
  for (auto &l : d->L) b += l.qkv.bytes() + l.o.bytes() + l.fc1.bytes() + l.fc2.bytes() +
                            l.xq.bytes() + l.xo.bytes();
  return b;
}

}  // extern "C"
