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

#include "ll_dev.h"
#include "quant.h"
#include "step_dev.h"

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

// Elements [start, start + n) of a synthetic stream into dst[0, n): fp32,
// bf16 bits (RNE) or int8 (the Irwin-Hall integer sum scaled by k and
// rounded half away from zero, clamped to +-127: uniform-ish int8 codes).
__global__ void synth_fill_kernel(uint64_t base, float mean, float k, uint64_t start, size_t n,
                                  void *dst, int dtype) {
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const float v = synth_value(base, start + i, mean, k);
    if (dtype == XE_BF16)
      static_cast<uint16_t *>(dst)[i] = bf16_bits_dev(v);
    else if (dtype == XE_I8)
      static_cast<int8_t *>(dst)[i] = static_cast<int8_t>(fminf(fmaxf(roundf(v), -127.0f), 127.0f));
    else
      static_cast<float *>(dst)[i] = v;
  }
}

// dst[i] = src[i] over n 16-byte words (a plain streaming copy: one read and
// one write per byte).
__global__ void copy16_kernel(const uint4 *src, uint4 *dst, size_t n) {
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x)
    dst[i] = src[i];
}

// --------------------------------------------------------------------------
// step kernels
// --------------------------------------------------------------------------

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

// f32 [T, H*hd] rows -> int8 head-major [H, T, hd] with per-channel scales:
// the host quantisation of the reference's int8 cross K / V
// (rust/npu-engine/src/asr/whisper_decoder.rs:1186-1219, write_buf_i8
// :1110-1134): s[c] = max_t |x[t][c]| / 127 (1.0 for a zero channel),
// q = clamp(round(x * (1/s)), -127, 127), round half away from zero.
// One workgroup a head; thread (wave w, lane j) takes channel j + 64 i of
// rows w, w + 4, ...  (one 256-byte row segment a wave per load).
__global__ __launch_bounds__(256) void cross_quant_kernel(const float *src, int t_rows, int heads, int hd,
                                                          int8_t *dst, float *scale) {
  __shared__ float red[4][256];
  const int h = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int D = heads * hd;
  for (int j0 = 0; j0 < hd; j0 += 64) {
    const int j = j0 + lane;
    float mx = 0.f;
    if (j < hd)
      for (int t = wave; t < t_rows; t += 4) mx = fmaxf(mx, fabsf(src[static_cast<size_t>(t) * D + h * hd + j]));
    red[wave][lane] = mx;
    __syncthreads();
    const float m = fmaxf(fmaxf(red[0][lane], red[1][lane]), fmaxf(red[2][lane], red[3][lane]));
    const float s = m > 0.f ? m * 1.0f / 127.0f : 1.0f;
    const float inv = s != 0.f ? 1.0f / s : 0.f;
    if (j < hd) {
      if (wave == 0) scale[h * hd + j] = s;
      for (int t = wave; t < t_rows; t += 4) {
        float r = roundf(src[static_cast<size_t>(t) * D + h * hd + j] * inv);
        r = r != r ? 0.f : fminf(fmaxf(r, -127.f), 127.f);  // NaN -> 0 (Rust `as i8`)
        dst[(static_cast<size_t>(h) * t_rows + t) * hd + j] = static_cast<int8_t>(r);
      }
    }
    __syncthreads();  // red is reused by the next channel block
  }
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

// src [rows][cols] -> dst [cols / 4][rows][4]: element (r, c) at
// (c / 4 * rows + r) * 4 + c % 4 (cols a multiple of 4); 32 x 32 tiles
// through LDS.
template <typename T>
__global__ void transpose4_kernel(const T *src, T *dst, int rows, int cols) {
  __shared__ T tile[32][33];
  const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
  for (int i = threadIdx.y; i < 32; i += 8) {
    const int r = r0 + i, c = c0 + threadIdx.x;
    if (r < rows && c < cols) tile[i][threadIdx.x] = src[static_cast<size_t>(r) * cols + c];
  }
  __syncthreads();
  for (int i = threadIdx.y; i < 32; i += 8) {
    const int c = c0 + i, r = r0 + threadIdx.x;
    if (c < cols && r < rows) dst[(static_cast<size_t>(c / 4) * rows + r) * 4 + c % 4] = tile[threadIdx.x][i];
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
  uint16_t *ck = nullptr, *cv = nullptr;  // Whisper cross K/V bf16 [H, T, hd] (int8 [H, T, hd] when quantised)
  float *cks = nullptr, *cvs = nullptr;    // int8 cross K / V channel scales [H * hd]
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
  float *xn = nullptr;  // GEMM path: normalised activations [max_batch][max K]
  float *gemm_ws = nullptr;  // GEMM split-K partials
  unsigned *gemm_cnt = nullptr;  // GEMM split-K counters (zeroed once, self-resetting)
  int8_t *gemm_xd = nullptr;     // int8 digit planes of a prologue's rows (the int8-MFMA GEMM)
  int *gemm_xe = nullptr;        // their per-stream exponents
  uint16_t *kc = nullptr, *vc = nullptr;  // [L][B][hkv][max_ctx][hd]
  float *rope_cos = nullptr, *rope_sin = nullptr;
  int32_t *tokens = nullptr, *pos = nullptr, *next = nullptr, *hist = nullptr;
  // stop rule: stop_dev[0] = the stop token (-1: none), stop_dev[1 + b] =
  // stream b has emitted it (xe_decoder_set_stop)
  int32_t *stop_dev = nullptr;
  int stop_id = -1;
  float *arg_v = nullptr;
  int *arg_i = nullptr;
  float *attn_work = nullptr;
  unsigned *attn_cnt = nullptr;  // split-attention arrival counters [max_batch * hkv] (self-resetting)
  int attn_splits = 1;
  int32_t *host_tok = nullptr;  // pinned staging [max_ctx + 1][max_batch] x 2
  int last_exec = XE_EXEC_GRAPH;  // executor of the last step launched (status messages)
  // status word of the low-latency step kernel's bounded waits
  unsigned int *step_status = nullptr;
  // one execution plan per batch size: the phase list of a step
  struct Plan {
    std::vector<sdev::Phase> phases;
    std::vector<std::string> labels;
    std::vector<double> bytes;  // algorithmic bytes per phase
    hipGraphExec_t graph = nullptr;
  };
  std::map<int, Plan> plans;
  // low-latency executor (ll_dev.h): one plan per batch size
  struct LLPlan {
    bool ok = false;
    std::string why;  // reason it is unsupported
    std::vector<ll::Phase> a, f;
    std::vector<std::string> a_labels, f_labels;
    std::vector<double> a_bytes, f_bytes;  // algorithmic bytes per phase (KV added per step)
    ll::Phase *dev_a = nullptr, *dev_f = nullptr;
    uint64_t *arena = nullptr;  // every exchange vector of the step
    ll::Vec arg{};
    int kin_a = 0, kin_f = 0, scratch = 0, nb_t = 1, grid = 0, hd = 64, g = 1;
    bool kv8 = false;  // int8 cross K / V (its own kernel instantiation)
    int stage_a = 0, stage_f = 0;  // LDS weight stage bytes per role (ll::StageLayout), 0: none staged
    int kv_floats = 0;             // LDS key/value stage (attention side), 0: none
    size_t lds_bytes = 0;
    int head_lpr = 8, head_rpl = 2;
  };
  std::map<int, LLPlan> ll_plans;
  // FFN output projections transposed ([ffn / 4][d_model][4] per layer) for the
  // low-latency executor's split FFN output (ll::DpartD); empty until a plan
  // uses them, refreshed when a layer's projection is set
  std::vector<void *> ll_fc2t;
  unsigned ll_epoch = 1;           // epoch of the next step (exchange buffers start at 0)
  int32_t *ll_forced = nullptr;    // device [max_ctx + 1][max_batch] prompt tokens
  double last_step_us = 0.0;
  bool cross_ready = false;
  int cross_i8k = 0, cross_i8v = 0;  // per-utterance int8 cross K / V (xe_decoder_set_cross_int8)
  // Host copy of every stream's next position (the one the kernels append
  // the K/V row at and read the RoPE / position row of): feed() sets it to
  // the prompt length, step() to pos + 1, decode() and profile_step()
  // advance it.  live = streams whose device token / position state was set
  // by feed() or step() since the last reset; decode(batch) needs batch <= live.
  std::vector<int> hpos;
  int live = 0;
  // bound every position a run of n_steps from the host positions would
  // process: the K/V rows and position rows of streams b < batch
  void require_room(int batch, int n_steps) const {
    XE_REQUIRE(batch <= live, "decode batch exceeds the streams fed or stepped since the last reset");
    for (int b = 0; b < batch; b++) {
      XE_REQUIRE(static_cast<long>(hpos[b]) + n_steps <= c.max_ctx, "decode would run past max_ctx");
      if (c.family != XE_GEMMA3)
        XE_REQUIRE(static_cast<long>(hpos[b]) + n_steps <= c.max_pos, "decode would run past the position table");
    }
  }
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

// Splits per (stream, kv head) of the split-K attention phases of a batch:
// about one workgroup per CU over the batch's (stream, kv head) pairs, at
// most one per 64 cache rows and at most 64.  Gemma over ctx 512..4096, with
// the merge inside the split kernel: b = 64 at 4 splits 24.0k tok/s, 8: 22.9k,
// 16: 19.9k, 2: 20.0k; b = 16 at 16 splits 7.70k, 32: 7.40k, 8: 7.47k.  Each
// split block pays its q transform, its cross-wave merge and its partial
// stores, so fewer, longer splits win once the chip is covered.  (A stream's
// blocks past its filled length return at once; split_range sizes chunks
// from the length.)
int attn_splits_for(const xe_decoder *d, int batch, int hkv) {
  const auto &c = d->c;
  const int cus = d->dev->num_cus > 0 ? d->dev->num_cus : 256;
  int ms = cus / std::max(1, batch * hkv);
  const int cap = (std::max(c.max_ctx, c.family == XE_WHISPER ? c.n_cross : 0) + 63) / 64;
  return std::max(1, std::min(std::min(ms, cap), 64));
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
      l.cks = dalloc<float>(D, s);
      l.cvs = dalloc<float>(D, s);
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
  d->xn = dalloc<float>(static_cast<size_t>(B) * std::max(std::max(D, F), std::max(hq, static_cast<int>(d->nqkv()))), s);
  if (B >= 4 || F > 4096) {  // the GEMM path can run (see PlanBuilder::gemv)
    d->gemm_ws = dalloc<float>(gemm_ws_floats(), s);
    d->gemm_cnt = dalloc<unsigned>(gemm_cnt_words(), s);
    XE_HIP(hipMemsetAsync(d->gemm_cnt, 0, gemm_cnt_words() * sizeof(unsigned), s));
    d->gemm_xd = dalloc<int8_t>(static_cast<size_t>(4) * B * D, s);
    d->gemm_xe = dalloc<int>(B, s);
  }
  const size_t kvn = d->kv_layer_elems() * c.n_layers;
  d->kc = dalloc<uint16_t>(kvn, s);
  d->vc = dalloc<uint16_t>(kvn, s);
  d->tokens = dalloc<int32_t>(B, s);
  d->pos = dalloc<int32_t>(B, s);
  d->next = dalloc<int32_t>(B, s);
  d->hist = dalloc<int32_t>(static_cast<size_t>(B) * (c.max_ctx + 1), s);
  d->stop_dev = dalloc<int32_t>(static_cast<size_t>(B) + 1, s);
  XE_HIP(hipMemsetAsync(d->stop_dev, 0xff, 4, s));  // no stop token
  d->arg_v = dalloc<float>(static_cast<size_t>(B) * sdev::kArgBlocks, s);
  d->arg_i = dalloc<int>(static_cast<size_t>(B) * sdev::kArgBlocks, s);
  d->step_status = dalloc<unsigned int>(64, s);
  d->ll_forced = dalloc<int32_t>(static_cast<size_t>(c.max_ctx + 1) * B, s);
  // split-K attention: the phase plan of a batch takes attn_splits_for(); the
  // workspace holds the partials of the largest batch x splits product
  const int hkv_max = std::max(c.n_kv_heads, wh ? c.n_heads : 0);
  size_t part_rows = 0;
  for (int b = 1; b <= B; b++)
    part_rows = std::max(part_rows, static_cast<size_t>(b) * attn_splits_for(d, b, hkv_max));
  d->attn_splits = attn_splits_for(d, B, hkv_max);
  d->attn_work = dalloc<float>(attn_work_floats(static_cast<int>(part_rows), std::max(c.n_heads, 1), c.head_dim, 1),
                               s, false);
  d->attn_cnt = dalloc<unsigned>(static_cast<size_t>(B) * hkv_max, s);  // zeroed
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

// Every cached execution plan (graphs, device phase lists, exchange arenas).
void drop_plans(xe_decoder *d) {
  if (d->s) (void)hipStreamSynchronize(d->s);
  for (auto &kv : d->plans) {
    if (kv.second.graph) (void)hipGraphExecDestroy(kv.second.graph);
  }
  d->plans.clear();
  for (auto &kv : d->ll_plans) {
    if (kv.second.dev_a) (void)hipFree(kv.second.dev_a);
    if (kv.second.dev_f) (void)hipFree(kv.second.dev_f);
    if (kv.second.arena) (void)hipFree(kv.second.arena);
  }
  d->ll_plans.clear();
}

void free_decoder(xe_decoder *d) {
  drop_plans(d);
  for (void *p : d->ll_fc2t)
    if (p) (void)hipFree(p);
  if (d->ll_forced) (void)hipFree(d->ll_forced);
  if (d->step_status) (void)hipFree(d->step_status);
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
                    static_cast<void *>(l.cv), static_cast<void *>(l.cks),
                    static_cast<void *>(l.cvs)})
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
                  static_cast<void *>(d->stop_dev), static_cast<void *>(d->arg_v), static_cast<void *>(d->arg_i),
                  static_cast<void *>(d->attn_work), static_cast<void *>(d->xn),
                  static_cast<void *>(d->gemm_ws), static_cast<void *>(d->gemm_cnt),
                  static_cast<void *>(d->gemm_xd), static_cast<void *>(d->gemm_xe),
                  static_cast<void *>(d->attn_cnt)})
    if (p) (void)hipFree(p);
  if (d->host_tok) (void)hipHostFree(d->host_tok);
  if (d->s) (void)hipStreamDestroy(d->s);
}

// ---- host-side description of one GEMV over `batch` rows ----
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

struct PlanBuilder {
  xe_decoder::Plan &plan;
  float *xn = nullptr;  // GEMM path scratch (null: GEMV only)
  float *ws = nullptr;
  unsigned *cnt = nullptr;
  int8_t *xd = nullptr;  // digit planes (4 x batch x K bytes, K <= xd_k) and exponents
  int *xe = nullptr;
  int xd_k = 0;
  int last_gemm = -1;  // the last phase pushed, when it is a GEMM
  void push(const sdev::Phase &ph, const std::string &label, double bytes) {
    plan.phases.push_back(ph);
    plan.labels.push_back(label);
    plan.bytes.push_back(bytes);
    last_gemm = ph.kind == sdev::PH_GEMM ? static_cast<int>(plan.phases.size()) - 1 : -1;
  }
  // A prologue whose `sub` is the output of the GEMM pushed just before it,
  // when that GEMM splits K, adds the GEMM's split partials itself (in split
  // order, then the GEMM's own epilogue: the same values): the GEMM stores
  // each split's raw sums to the workspace and loses its arrival counter and
  // finishing workgroup, one memory round trip of its critical path.
  // XE_GEMM_DEFER=0 (read when a plan is built) keeps the GEMM's own finish.
  void adopt_parts(gdev::GemvParams &q) {
    const char *env = std::getenv("XE_GEMM_DEFER");
    if ((env && std::string(env) == "0") || !q.sub || last_gemm < 0 || !ws) return;
    sdev::Phase &pp = plan.phases[last_gemm];
    gdev::GemvParams &g = pp.u.gemv;
    if (g.y != q.sub || g.act != ACT_NONE || g.ldy != g.m || g.m != q.k || g.batch != q.batch || g.part) return;
    const int ks = gemm_defer_splits(g.m, g.k, g.batch);
    if (ks < 2 || static_cast<size_t>(ks) * g.batch * g.m > gemm_ws_floats()) return;
    gdev::GemvParams t = q;
    t.sub = nullptr;
    t.sub_part = ws;
    t.sub_ks = ks;
    t.sub_scale = (pp.variant == XE_I8 || pp.variant == XE_I4) ? g.scale : nullptr;
    t.sub_bias = g.bias;
    t.sub_out_scale = g.out_scale;
    if (!gemm_prologue_takes_parts(t, xn)) return;
    g.part = ws;
    q = t;
  }
  // One projection over `batch` streams.  Up to 8 streams whose activations
  // fit the GEMV's LDS staging: the GEMV, in chunks of 8.  Otherwise the MFMA
  // GEMM (gemm.hip) over all streams, after its prologue when the phase
  // normalises or adds a residual.
  void gemv(const GemvCall &g, int batch, const std::string &label) {
    const size_t stage = gdev::gemv_lds_floats(std::min(batch, 8), g.m->cols, g.sub != nullptr) * sizeof(float);
    if (xn && (gemm_preferred(g.m->rows, g.m->cols, batch) || stage > 160 * 1024 - 1024)) {
      gemm(g, batch, label);
      return;
    }
    for (int b0 = 0; b0 < batch; b0 += 8) {
      const int nb = std::min(8, batch - b0);
      GemvLaunch L;
      L.wdtype = g.m->wdtype;
      L.w = g.m->w;
      L.scale = g.m->scale;
      L.exps = g.m->exps;
      L.bias = g.bias;
      L.m = g.m->rows;
      L.k = g.m->cols;
      L.x = g.x + static_cast<size_t>(b0) * g.ldx;
      L.x_dtype = XE_F32;
      L.ldx = g.ldx;
      L.batch = nb;
      L.sub = g.sub ? g.sub + static_cast<size_t>(b0) * g.m->cols : nullptr;
      L.post_w = g.post_w;
      L.res_out = g.res_out ? g.res_out + static_cast<size_t>(b0) * g.m->cols : nullptr;
      L.norm = g.norm;
      L.gamma = g.gamma;
      L.beta = g.beta;
      L.eps = g.eps;
      L.act = g.act;
      L.y = g.y + static_cast<size_t>(b0) * g.ldy;
      L.ldy = g.ldy;
      XE_REQUIRE(L.k % 16 == 0, "gemv: K must be a multiple of 16");
      sdev::Phase ph{};
      ph.kind = sdev::PH_GEMV;
      ph.variant = L.wdtype;
      const gdev::Tile t = gdev::choose_tile(L.m, L.k, L.act);
      ph.lpr = t.lpr;
      ph.rpl = t.rpl;
      const int rows = 4 * (64 / t.lpr) * t.rpl;
      ph.nblocks = (L.m + rows - 1) / rows;
      ph.u.gemv = gdev::to_params(L);
      push(ph, label, gemv_bytes(g, nb));
    }
  }
  void gemm(const GemvCall &g, int batch, const std::string &label) {
    GemvLaunch L;
    L.wdtype = g.m->wdtype;
    L.w = g.m->w;
    L.scale = g.m->scale;
    L.exps = g.m->exps;
    L.bias = g.bias;
    L.m = g.m->rows;
    L.k = g.m->cols;
    L.x = g.x;
    L.x_dtype = XE_F32;
    L.ldx = g.ldx;
    L.batch = batch;
    L.sub = g.sub;
    L.post_w = g.post_w;
    L.res_out = g.res_out;
    L.norm = g.norm;
    L.gamma = g.gamma;
    L.beta = g.beta;
    L.eps = g.eps;
    L.act = g.act;
    L.y = g.y;
    L.ldy = g.ldy;
    XE_REQUIRE(L.k % 16 == 0, "gemm: K must be a multiple of 16");
    sdev::Phase ph{};
    ph.variant = L.wdtype;
    ph.u.gemv = gdev::to_params(L);
    if (gemm_needs_prologue(ph.u.gemv)) {
      ph.kind = sdev::PH_GEMM_PRO;
      ph.nblocks = batch;
      ph.xn = xn;
      adopt_parts(ph.u.gemv);
      // int8 weights too wide for the K-sliced kernel (the lm-head): the
      // prologue writes the rows' int8 digit planes for the int8 matrix cores
      if (xd && L.k <= xd_k && gemm_i8_preferred(L.m, L.k, batch, L.wdtype)) {
        gdev::GemvParams t = ph.u.gemv;
        t.xd = xd;
        t.xe = xe;
        if (gemm_prologue_takes_digits(t, xn)) ph.u.gemv = t;
      }
      const int sub_reads = ph.u.gemv.sub_part ? ph.u.gemv.sub_ks : (L.sub ? 1 : 0);
      push(ph, label + "_pro", 4.0 * batch * L.k * (2 + sub_reads + (L.res_out ? 1 : 0)));
      gdev::GemvParams &q = ph.u.gemv;
      q.x = xn;
      q.ldx = L.k;
      q.sub = nullptr;
      q.sub_part = nullptr;
      q.post_w = nullptr;
      q.res_out = nullptr;
      q.norm = XE_NORM_NONE;
      ph.xn = nullptr;
    }
    ph.kind = sdev::PH_GEMM;
    ph.nblocks = ((L.m + 63) / 64) * ((batch + 63) / 64);
    ph.ws = ws;
    ph.cnt = cnt;
    push(ph, label, gemv_bytes(g, batch));
  }
  void attn(const AttnLaunch &a, const std::string &label, double bytes) {
    sdev::Phase ph{};
    ph.kind = sdev::PH_ATTN;
    ph.hd = a.hd;
    ph.g = a.hq / a.hkv;
    ph.nblocks = a.max_splits * a.hkv * a.batch;
    ph.u.attn = adev::to_params(a);
    push(ph, label, bytes);
    if (a.max_splits > 1 && !a.cnt) {
      ph.kind = sdev::PH_MERGE;
      ph.nblocks = ((ph.g * ph.hd + 255) / 256) * a.hkv * a.batch;
      push(ph, label + "_merge",
           4.0 * a.batch * a.hq * (a.hd + 2) * std::min(a.max_splits, 64));
    }
  }
};

// The phase list of one decode step for streams [0, B) (tokens/pos on device).
void build_plan(xe_decoder *d, int B, xe_decoder::Plan &plan) {
  const auto &c = d->c;
  const int D = c.d_model, F = c.ffn, hd = c.head_dim;
  const int hq = c.n_heads * hd, hk = c.n_kv_heads * hd;
  const bool gem = c.family == XE_GEMMA3, wh = c.family == XE_WHISPER, opt = c.family == XE_OPT;
  const int nq = static_cast<int>(d->nqkv());
  const int norm = gem ? XE_NORM_RMS1P : XE_NORM_LN;
  PlanBuilder pb{plan, d->gemm_ws ? d->xn : nullptr, d->gemm_ws, d->gemm_cnt, d->gemm_xd, d->gemm_xe, c.d_model};
  // the split attention kernel merges in place (arrival counters)
  unsigned *attn_cnt = d->attn_cnt;

  // embedding
  {
    sdev::Phase ph{};
    ph.kind = sdev::PH_EMBED;
    Spec sp;
    sdev::EmbedParams &e = ph.u.emb;
    e.emb = d->emb.w;
    e.emb_scale = d->emb.scale;
    e.emb_exps = d->emb.exps;
    e.wdtype = c.wdtype;
    e.pos_emb = d->pos_emb;
    e.pos_off = opt ? 2 : 0;
    e.pos_rows = tensor_spec(c, XE_T_POS_EMB, -1, sp) ? sp.rows : 1;
    e.mul = sqrtf(static_cast<float>(D));
    e.use_mul = gem ? 1 : 0;
    e.tokens = d->tokens;
    e.pos = d->pos;
    e.vocab = c.vocab;
    e.d = D;
    e.batch = B;
    e.x = d->xa;
    ph.nblocks = B * ((D + 255) / 256);
    pb.push(ph, "embed", static_cast<double>(B) * D * (wbytes(c.wdtype, 1) + 4 + (d->pos_emb ? 4 : 0)));
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
      pb.gemv(g, B, "gemv_qkv");
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
      a.cnt = attn_cnt;
      a.max_splits = attn_splits_for(d, B, c.n_kv_heads);
      // KV bytes depend on the positions; profile_step fills them in
      pb.attn(a, "attn_self", 4.0 * B * (nq + hq) + 4.0 * B * hk);
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
      pb.gemv(g, B, "gemv_o");
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
      pb.gemv(g, B, "gemv_xq");
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
      a.cnt = attn_cnt;
      a.max_splits = attn_splits_for(d, B, c.n_heads);
      a.k_scale = d->cross_i8k ? l.cks : nullptr;
      a.v_scale = d->cross_i8v ? l.cvs : nullptr;
      pb.attn(a, "attn_cross",
              static_cast<double>(c.n_cross) * D * ((d->cross_i8k ? 1 : 2) + (d->cross_i8v ? 1 : 2)) + 8.0 * B * D);
      GemvCall o;
      o.m = &l.xo;
      o.bias = l.xo_b;
      o.x = d->att;
      o.ldx = D;
      o.y = d->sub;
      o.ldy = D;
      pb.gemv(o, B, "gemv_xo");
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
      pb.gemv(g, B, gem ? "gemv_gateup" : "gemv_fc1");
      after_pending();
      GemvCall o;
      o.m = &l.fc2;
      o.bias = gem ? nullptr : l.fc2_b;
      o.x = d->ffn;
      o.ldx = F;
      o.y = d->sub;
      o.ldy = D;
      pb.gemv(o, B, gem ? "gemv_down" : "gemv_fc2");
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
    pb.gemv(g, B, "gemv_lmhead");
  }
  // ---- greedy argmax -> next token, pos + 1 ----
  {
    sdev::Phase ph{};
    sdev::ArgmaxParams &ap = ph.u.arg;
    ap.logits = d->logits;
    ap.vocab = c.vocab;
    ap.batch = B;
    ap.last_max = opt ? 1 : 0;
    ap.part_v = d->arg_v;
    ap.part_i = d->arg_i;
    ap.next = d->next;
    ap.tokens = d->tokens;
    ap.pos = d->pos;
    ap.hist = d->hist;
    ap.hist_stride = c.max_ctx + 1;
    ap.stop = d->stop_dev;
    ap.done = d->stop_dev + 1;
    ph.kind = sdev::PH_ARGMAX_PART;
    ph.nblocks = B * sdev::kArgBlocks;
    pb.push(ph, "argmax", 4.0 * B * c.vocab);
    ph.kind = sdev::PH_ARGMAX_FINAL;
    ph.nblocks = B;
    pb.push(ph, "argmax_final", 8.0 * B * sdev::kArgBlocks);
  }
}

xe_decoder::Plan &plan_for(xe_decoder *d, int B) {
  auto it = d->plans.find(B);
  if (it != d->plans.end()) return it->second;
  xe_decoder::Plan &plan = d->plans[B];
  build_plan(d, B, plan);
  return plan;
}

// ---------------------------------------------------------------------------
// low-latency executor: phase lists per role (ll_dev.h)
// ---------------------------------------------------------------------------
// GEMV tile for `ranks` workgroups of kT threads sharing m rows: lanes per
// row LPR in {8, 16, 32, 64}, two rows per lane (ll_dev.h gemv_rows).  Each
// tile costs one memory round trip per load round (NIT chunk iterations per
// row: ll_dev.h Round); then fewer valid chunks per lane (serial FMA work).
void ll_tile(int m, int ranks, int k, bool geglu, int wdtype, int &lpr, int &rpl) {
  (void)geglu;
  const int rows = (m + ranks - 1) / ranks, nch = k / 16;
  const int nit = wdtype == XE_BF16 ? 4 : 9;
  long best = -1;
  rpl = 2;
  for (int cand : {8, 16, 32, 64}) {
    const int per_tile = ll::kW * (64 / cand) * 2;
    const long tiles = (rows + per_tile - 1) / per_tile;
    const long n_it = (nch + cand - 1) / cand;
    const long rounds = (n_it + nit - 1) / nit;
    const long cost = tiles * rounds * 1000 + tiles * std::min<long>(n_it, nit) * 20;
    if (best < 0 || cost < best) {
      best = cost;
      lpr = cand;
    }
  }
}


// Trace marks of one traced step: phase ends, 4 step marks, phase
// input-ready times, kSubSlots sub-stage marks per phase.
size_t ll_trace_slots(const xe_decoder::LLPlan &P) {
  const size_t n = P.a.size() + P.f.size();
  return 2 * n + 4 + ll::kSubSlots * n;
}

constexpr size_t kLLLds = 160 * 1024 - 2048;  // dynamic LDS of the step kernel (static LDS aside)

// Key/value staging (ll::kv_stage_issue): each attention phase's blocks of
// up to kv_cap keys (one round at most) are copied into LDS at the start of
// the phase before it, which on the attention side waits for its own input
// long enough for the copies to land.  kv_cap covers the longest block the
// cache allows, or the most keys budget (bytes, < 0: none) leaves room for
// (a multiple of the key tile); longer blocks load their keys as before.
// Returns the stage's floats.
int plan_kv_stage(std::vector<ll::Phase> &list, int hd, int max_ctx, long budget) {
  int floats = 0;
  for (int j = 1; j < static_cast<int>(list.size()); j++) {
    if (list[j].kind != ll::LK_ATTN) continue;
    ll::AttnD &a = list[j].u.attn;
    if (a.k_scale) {  // int8 rows are read where they are used, not staged
      a.kv_cap = 0;
      continue;
    }
    int chunk, nsplits;
    ll::ll_split(a.fixed_len > 0 ? a.fixed_len : max_ctx, a.max_splits, hd, chunk, nsplits);
    int cap = std::min(chunk, ll::kRoundKeys);
    while (cap > 0 && 4L * ll::kv_stage_floats(hd, cap) > budget) cap -= ll::kKeyTile;
    a.kv_cap = std::max(cap, 0);
    if (a.kv_cap == 0) continue;
    list[j - 1].kv_issue = j;
    floats = std::max(floats, ll::kv_stage_floats(hd, a.kv_cap));
  }
  return floats;
}

// LDS weight staging (ll::StageLayout).  A GEMV phase whose input is an
// exchange vector follows another phase of its role directly, so weights
// it loads at its own start arrive only a memory round trip after that
// phase: such a phase gets its slice copied into LDS at the start of an
// earlier phase, the one after the role's previous staged phase (the stage
// holds one slice at a time).  budget < 0: nothing staged.
// dpart_need: the stage bytes of a split FFN output phase (ll::LK_DPART),
// which is always staged, by the phase right before it.
void plan_stage(std::vector<ll::Phase> &list, int ranks, int wt, long budget, int &stage_bytes,
                int dpart_need = 0) {
  for (auto &ph : list) {
    ph.issue = -1;
    ph.kv_issue = -1;
    if (ph.kind == ll::LK_GEMV) ph.u.gemv.staged = 0;
    if (ph.kind == ll::LK_ATTN) ph.u.attn.kv_cap = 0;
  }
  int last = -1;  // the previous staged phase
  for (int j = 0; j < static_cast<int>(list.size()); j++) {
    if (list[j].kind == ll::LK_DPART && j > 0) {  // the GEMV before never reads the stage itself
      list[j - 1].issue = j;
      last = j;
      stage_bytes = std::max(stage_bytes, dpart_need);
      continue;
    }
    if (list[j].kind != ll::LK_GEMV) continue;
    ll::GemvD &g = list[j].u.gemv;
    const int at = last + 1;
    // input from the previous phase, no residual update (the kernel's staged
    // path waits for the input vector alone); an earlier phase to ride on
    if (!g.in_vec || g.nfold > 0 || at >= j) continue;
    // the kernel's row split (ll_kernel.h: GeGLU pairs, and activations kept
    // in LDS for the split FFN output on multiples of four of them)
    const int unit = (g.act == ACT_GEGLU_TANH ? 2 : 1) * (g.out_lds ? 4 : 1);
    const int rows = (g.m / unit + ranks - 1) / ranks * unit;
    const int need = ll::stage_layout(wt, rows, g.k, g.bias != nullptr).total;
    if (need > budget) continue;
    g.staged = 1;
    list[at].issue = j;
    last = j;
    stage_bytes = std::max(stage_bytes, need);
  }
}
// Transposed FFN output projection of one layer (int8 / bf16 weights):
// ll_fc2t[layer] = fc2.w^T with four hidden rows interleaved,
// [ffn / 4][d_model][4] (ll::DpartD), on the decoder's stream.
void ll_fc2t_layer(xe_decoder *d, int layer) {
  const Mat &m = d->L[layer].fc2;
  const dim3 grid((m.cols + 31) / 32, (m.rows + 31) / 32), block(32, 8);
  if (m.wdtype == XE_BF16)
    transpose4_kernel<uint16_t><<<grid, block, 0, d->s>>>(static_cast<const uint16_t *>(m.w),
                                                         static_cast<uint16_t *>(d->ll_fc2t[layer]), m.rows, m.cols);
  else
    transpose4_kernel<int8_t><<<grid, block, 0, d->s>>>(static_cast<const int8_t *>(m.w),
                                                       static_cast<int8_t *>(d->ll_fc2t[layer]), m.rows, m.cols);
  XE_HIP(hipGetLastError());
}

void ll_fc2t_ensure(xe_decoder *d) {
  if (!d->ll_fc2t.empty()) return;
  d->ll_fc2t.assign(d->c.n_layers, nullptr);
  for (int li = 0; li < d->c.n_layers; li++) {
    const Mat &m = d->L[li].fc2;
    XE_HIP(hipMalloc(&d->ll_fc2t[li], wbytes(m.wdtype, static_cast<size_t>(m.rows) * m.cols)));
    ll_fc2t_layer(d, li);
  }
}

void build_ll_plan(xe_decoder *d, int B, xe_decoder::LLPlan &P) {
  const auto &c = d->c;
  const int D = c.d_model, F = c.ffn, hd = c.head_dim;
  const int hq = c.n_heads * hd, hk = c.n_kv_heads * hd;
  const bool gem = c.family == XE_GEMMA3, wh = c.family == XE_WHISPER, opt = c.family == XE_OPT;
  const int nq = static_cast<int>(d->nqkv());
  const int norm = gem ? XE_NORM_RMS1P : XE_NORM_LN;
  const int g = c.n_heads / c.n_kv_heads;
  P.ok = false;
  if (B > ll::kMaxNB) { P.why = "batch > 4"; return; }
  if (d->cross_i8k != d->cross_i8v) { P.why = "int8 cross K or V alone runs on the phase kernels"; return; }
  P.nb_t = B <= 1 ? 1 : B <= 2 ? 2 : 4;
  P.hd = hd;
  P.g = g;
  P.kv8 = d->cross_i8k && d->cross_i8v;
  if (!ll::step_supported(c.wdtype, P.nb_t, hd, g, P.kv8)) {
    P.why = P.kv8 ? "int8 cross K/V with non-int8 weights runs on the phase kernels" : "head_dim / group not instantiated";
    return;
  }
  if (hd % ll::kDM != 0) { P.why = "head_dim not a multiple of 16"; return; }
  for (int k : {D, F, hq}) if (k % 16) { P.why = "K not a multiple of 16"; return; }
  P.grid = d->dev->num_cus > 0 ? d->dev->num_cus : 256;
  const int n_a = (P.grid + ll::kRoleStride - 1) / ll::kRoleStride, n_f = P.grid - n_a;
  const char *tail_env = std::getenv("XE_LL_TAIL");
  const int tail_mode = tail_env ? std::atoi(tail_env) : 1;

  // exchange arena: offsets first, one allocation after
  size_t pairs = 0;
  std::vector<std::pair<size_t, int>> vecs;  // (offset, ld)
  auto vec = [&](int n) -> int {  // returns index into vecs
    const int ld = (n + 1) / 2 * 2;
    vecs.push_back({pairs, ld});
    pairs += static_cast<size_t>(ld) * B;
    pairs = (pairs + 1) / 2 * 2;
    return static_cast<int>(vecs.size()) - 1;
  };
  // phases refer to vectors by index until the arena exists: (list, phase, field) -> vec
  enum Field { F_GEMV_IN, F_GEMV_OUT, F_FOLD_SRC, F_ATTN_Q, F_ATTN_PART, F_MERGE_PART, F_MERGE_OUT,
               F_GEMV_FOLD0, F_GEMV_FOLD1, F_GEMV_FOLD2, F_DPART_PART, F_REDUCE_PART, F_REDUCE_OUT };
  struct Fix {
    std::vector<ll::Phase> *list;
    size_t idx;
    Field field;
    int vec;
  };
  std::vector<Fix> fix;
  auto field_of = [](ll::Phase &ph, Field f) -> ll::Vec & {
    switch (f) {
      case F_GEMV_IN: return ph.u.gemv.in;
      case F_GEMV_OUT: return ph.u.gemv.out;
      case F_FOLD_SRC: return ph.u.fold.src;
      case F_ATTN_Q: return ph.u.attn.q;
      case F_ATTN_PART: return ph.u.attn.part;
      case F_MERGE_PART: return ph.u.merge.part;
      case F_GEMV_FOLD0: return ph.u.gemv.folds[0].src;
      case F_GEMV_FOLD1: return ph.u.gemv.folds[1].src;
      case F_GEMV_FOLD2: return ph.u.gemv.folds[2].src;
      case F_DPART_PART: return ph.u.dpart.part;
      case F_REDUCE_PART: return ph.u.reduce.part;
      case F_REDUCE_OUT: return ph.u.reduce.out;
      default: return ph.u.merge.out;
    }
  };
  auto splits_for = [&](int heads_kv, int len_cap) {
    int ms = n_a / std::max(1, heads_kv * B);
    const int gran = ll::round_keys(hd);
    const int cap = (len_cap + gran - 1) / gran;
    return std::max(1, std::min(std::min(ms, cap), ll::kMaxSplits));
  };
  const int ms_self = splits_for(c.n_kv_heads, c.max_ctx);
  const int ms_cross = wh ? splits_for(c.n_heads, c.n_cross) : 1;

  auto labels_of = [&](std::vector<ll::Phase> &list) -> std::vector<std::string> & {
    return &list == &P.a ? P.a_labels : P.f_labels;
  };
  auto bytes_of = [&](std::vector<ll::Phase> &list) -> std::vector<double> & {
    return &list == &P.a ? P.a_bytes : P.f_bytes;
  };
  struct PreFold {
    int vec;
    const float *post_w;
  };
  auto gemv = [&](std::vector<ll::Phase> &list, int ranks, const Mat &m, const float *bias, int in_vec,
                  int norm_kind, const float *gamma, const float *beta, int act, int out_vec, const char *label,
                  std::vector<PreFold> pre = {}, int out_lds = 0) {
    ll::Phase ph{};
    ph.kind = ll::LK_GEMV;
    ll::GemvD &gd = ph.u.gemv;
    gd.w = m.w;
    gd.scale = m.scale;
    gd.exps = m.exps;
    gd.bias = bias;
    gd.m = m.rows;
    gd.k = m.cols;
    ll_tile(m.rows, ranks, m.cols, act == ACT_GEGLU_TANH, m.wdtype, gd.lpr, gd.rpl);
    // the tail K split runs on the FFN side only (the attention side's step
    // loop is compiled without it; on every GEMV it measured -1.4 %)
    gd.tail_split = &list == &P.f && (tail_mode == 2 || (tail_mode == 1 && out_lds > 0)) ? 1 : 0;
    gd.in_vec = in_vec >= 0 ? 1 : 0;
    gd.norm = norm_kind;
    gd.gamma = gamma;
    gd.beta = beta;
    gd.eps = c.eps;
    gd.act = act;
    XE_REQUIRE(pre.size() <= 3, "internal: too many residual updates before one GEMV");
    gd.nfold = static_cast<int>(pre.size());
    for (size_t f = 0; f < pre.size(); f++) {
      gd.folds[f].post_w = pre[f].post_w;
      gd.folds[f].eps = c.eps;
    }
    list.push_back(ph);
    labels_of(list).push_back(label);
    bytes_of(list).push_back(static_cast<double>(m.bytes()) + (bias ? 4.0 * m.rows : 0.0) +
                             4.0 * B * (m.cols + (act == ACT_GEGLU_TANH ? m.rows / 2 : m.rows)));
    for (size_t f = 0; f < pre.size(); f++)
      fix.push_back({&list, list.size() - 1, static_cast<Field>(F_GEMV_FOLD0 + f), pre[f].vec});
    if (in_vec >= 0) fix.push_back({&list, list.size() - 1, F_GEMV_IN, in_vec});
    if (out_lds > 0) list.back().u.gemv.out_lds = out_lds;
    else fix.push_back({&list, list.size() - 1, F_GEMV_OUT, out_vec});
  };
  auto fold = [&](std::vector<ll::Phase> &list, int src, const float *post_w, const char *label) {
    ll::Phase ph{};
    ph.kind = ll::LK_FOLD;
    ph.u.fold.post_w = post_w;
    ph.u.fold.eps = c.eps;
    list.push_back(ph);
    labels_of(list).push_back(label);
    bytes_of(list).push_back(4.0 * B * D);
    fix.push_back({&list, list.size() - 1, F_FOLD_SRC, src});
  };
  auto attn = [&](int qv, int qn, int q_off, int k_off, int v_off, bool append, uint16_t *kc, uint16_t *vc,
                  size_t bstride, int max_ctx, int heads, int heads_kv, float scale, int fixed_len,
                  const float *qnw, const float *knw, bool rope, int ms, int part, int out, int div_norm,
                  const char *label) {
    ll::Phase ph{};
    ph.kind = ll::LK_ATTN;
    ll::AttnD &a = ph.u.attn;
    a.qn = qn;
    a.q_off = q_off;
    a.k_off = k_off;
    a.v_off = v_off;
    a.append = append ? 1 : 0;
    a.kc = kc;
    a.vc = vc;
    a.kv_bstride = bstride;
    a.max_ctx = max_ctx;
    a.hq = heads;
    a.hkv = heads_kv;
    XE_REQUIRE(heads / heads_kv == g, "internal: attention group differs from the kernel's");
    a.hd = hd;
    a.scale = scale;
    a.fixed_len = fixed_len;
    a.q_norm_w = qnw;
    a.k_norm_w = knw;
    a.norm_eps = c.eps;
    a.rope_cos = rope ? d->rope_cos : nullptr;
    a.rope_sin = rope ? d->rope_sin : nullptr;
    a.max_splits = ms;
    P.a.push_back(ph);
    P.a_labels.push_back(label);
    P.a_bytes.push_back(fixed_len > 0 ? 4.0 * fixed_len * heads_kv * hd * B : 0.0);
    fix.push_back({&P.a, P.a.size() - 1, F_ATTN_Q, qv});
    fix.push_back({&P.a, P.a.size() - 1, F_ATTN_PART, part});
    ll::Phase mp{};
    mp.kind = ll::LK_MERGE;
    mp.u.merge.hq = heads;
    mp.u.merge.hd = hd;
    mp.u.merge.max_splits = ms;
    mp.u.merge.fixed_len = fixed_len;
    mp.u.merge.div_norm = div_norm;
    P.a.push_back(mp);
    P.a_labels.push_back(std::string(label) + "_merge");
    P.a_bytes.push_back(4.0 * B * heads * hd);
    fix.push_back({&P.a, P.a.size() - 1, F_MERGE_PART, part});
    fix.push_back({&P.a, P.a.size() - 1, F_MERGE_OUT, out});
  };
  // FFN output split: int8 / bf16 weights, at most kRedRows outputs per
  // F rank to sum, kRedParts ranks (XE_LL_FFN_SPLIT=0: the plain GEMV pair)
  const char *fs_env = std::getenv("XE_LL_FFN_SPLIT");
  const bool ffn_split = !(fs_env && std::string(fs_env) == "0") &&
                         (c.wdtype == XE_I8 || c.wdtype == XE_BF16) && D % 4 == 0 &&
                         (D + n_f - 1) / n_f <= ll::kRedRows && n_f <= ll::kRedParts;
  const int ffn_kn = 4 * ((F / 4 + n_f - 1) / n_f);  // hidden slice of an F rank (at most; multiples of 4)
  if (ffn_split) ll_fc2t_ensure(d);
  P.a.clear();
  P.f.clear();
  P.a_labels.clear();
  P.f_labels.clear();
  P.a_bytes.clear();
  P.f_bytes.clear();

  // Residual updates ride in the prologue of the next GEMV that needs the
  // residual: A side QKV(L) folds o(L-1) [or xo(L-1)] and down(L-1), Whisper
  // XQ(L) folds o(L); F side FC1(L) folds down(L-1), o(L) [and xo(L)].  The
  // tails fold what is left before the lm-head.
  int p_o = -1, p_xo = -1, p_down = -1;  // previous layer's vectors
  const float *p_post_attn = nullptr, *p_post_ffn = nullptr;
  for (int li = 0; li < c.n_layers; li++) {
    Layer &l = d->L[li];
    const int v_qkv = vec(nq);
    const int v_part = vec(hq * ms_self * (hd + 2));
    const int v_att = vec(hq);
    const int v_o = vec(D);
    const int v_ffn = vec(F);
    const int v_down = vec(D);
    // ---- A side ----
    std::vector<PreFold> pre_a;
    if (li > 0) {
      if (wh) pre_a.push_back({p_xo, nullptr});
      else pre_a.push_back({p_o, p_post_attn});
      pre_a.push_back({p_down, p_post_ffn});
    }
    gemv(P.a, n_a, l.qkv, gem ? nullptr : l.qkv_b, -1, norm, l.ln1_w, gem ? nullptr : l.ln1_b, ACT_NONE, v_qkv,
         "gemv_qkv", pre_a);
    attn(v_qkv, nq, 0, hq, hq + hk, true, d->kc + d->kv_layer_elems() * li, d->vc + d->kv_layer_elems() * li,
         static_cast<size_t>(c.n_kv_heads) * c.max_ctx * hd, c.max_ctx, c.n_heads, c.n_kv_heads,
         opt ? powf(static_cast<float>(hd), -0.5f) : 1.0f / sqrtf(static_cast<float>(hd)), 0,
         gem ? l.qn : nullptr, gem ? l.kn : nullptr, gem, ms_self, v_part, v_att, opt ? 1 : 0, "attn_self");
    gemv(P.a, n_a, l.o, gem ? nullptr : l.o_b, v_att, XE_NORM_NONE, nullptr, nullptr, ACT_NONE, v_o, "gemv_o");
    int v_xo = -1;
    if (wh) {
      const int v_xq = vec(D);
      const int v_xpart = vec(c.n_heads * ms_cross * (hd + 2));
      const int v_xatt = vec(D);
      v_xo = vec(D);
      gemv(P.a, n_a, l.xq, l.xq_b, -1, XE_NORM_LN, l.lnx_w, l.lnx_b, ACT_NONE, v_xq, "gemv_xq", {{v_o, nullptr}});
      attn(v_xq, D, 0, 0, 0, false, l.ck, l.cv, 0, c.n_cross, c.n_heads, c.n_heads,
           1.0f / sqrtf(static_cast<float>(hd)), c.n_cross, nullptr, nullptr, false, ms_cross, v_xpart, v_xatt, 0,
           "attn_cross");
      if (d->cross_i8k && d->cross_i8v) {  // int8 cross K and V (the attention phase, before its merge)
        ll::AttnD &ca = P.a[P.a.size() - 2].u.attn;
        ca.k_scale = l.cks;
        ca.v_scale = l.cvs;
        P.a_bytes[P.a_bytes.size() - 2] = 2.0 * c.n_cross * c.n_heads * hd * B;
      }
      gemv(P.a, n_a, l.xo, l.xo_b, v_xatt, XE_NORM_NONE, nullptr, nullptr, ACT_NONE, v_xo, "gemv_xo");
    }
    // ---- F side ----
    std::vector<PreFold> pre_f;
    if (li > 0) pre_f.push_back({p_down, p_post_ffn});
    pre_f.push_back({v_o, gem ? l.post_attn : nullptr});
    if (wh) pre_f.push_back({v_xo, nullptr});
    const int act = gem ? ACT_GEGLU_TANH : (opt ? ACT_RELU : ACT_GELU_ERF);
    if (ffn_split) {
      // FFN output split (ll::DpartD / ReduceD): the hidden slice stays in
      // LDS, partials for every output cross over, each rank sums its share
      gemv(P.f, n_f, l.fc1, gem ? nullptr : l.fc1_b, -1, norm, l.ln2_w, gem ? nullptr : l.ln2_b, act, -1,
           gem ? "gemv_gateup" : "gemv_fc1", pre_f, ll::xstride(D));
      const int v_dpart = vec(n_f * D);
      ll::Phase dp{};
      dp.kind = ll::LK_DPART;
      dp.u.dpart.wt = d->ll_fc2t[li];
      dp.u.dpart.d = D;
      dp.u.dpart.k = F;
      dp.u.dpart.unit = gem ? 2 : 1;
      dp.u.dpart.m_prev = l.fc1.rows;
      dp.u.dpart.act_off = ll::xstride(D);
      P.f.push_back(dp);
      P.f_labels.push_back(gem ? "ffn_down_part" : "ffn_fc2_part");
      P.f_bytes.push_back(static_cast<double>(l.fc2.bytes()) + 8.0 * B * n_f * D);
      fix.push_back({&P.f, P.f.size() - 1, F_DPART_PART, v_dpart});
      ll::Phase rp{};
      rp.kind = ll::LK_REDUCE;
      rp.u.reduce.d = D;
      rp.u.reduce.nparts = n_f;
      rp.u.reduce.scale = l.fc2.scale;
      rp.u.reduce.bias = gem ? nullptr : l.fc2_b;
      P.f.push_back(rp);
      P.f_labels.push_back(gem ? "ffn_down_reduce" : "ffn_fc2_reduce");
      P.f_bytes.push_back(8.0 * B * n_f * D);
      fix.push_back({&P.f, P.f.size() - 1, F_REDUCE_PART, v_dpart});
      fix.push_back({&P.f, P.f.size() - 1, F_REDUCE_OUT, v_down});
    } else {
      gemv(P.f, n_f, l.fc1, gem ? nullptr : l.fc1_b, -1, norm, l.ln2_w, gem ? nullptr : l.ln2_b, act, v_ffn,
           gem ? "gemv_gateup" : "gemv_fc1", pre_f);
      gemv(P.f, n_f, l.fc2, gem ? nullptr : l.fc2_b, v_ffn, XE_NORM_NONE, nullptr, nullptr, ACT_NONE, v_down,
           gem ? "gemv_down" : "gemv_fc2");
    }
    p_o = v_o;
    p_xo = v_xo;
    p_down = v_down;
    p_post_attn = gem ? l.post_attn : nullptr;
    p_post_ffn = gem ? l.post_ffn : nullptr;
  }
  // tails: the last layer's updates before the lm-head
  if (wh) fold(P.a, p_xo, nullptr, "fold_xo");
  else fold(P.a, p_o, p_post_attn, "fold_o");
  fold(P.a, p_down, p_post_ffn, "fold_down");
  fold(P.f, p_down, p_post_ffn, "fold_down");
  // argmax partials: [2 parities][B rows][grid * 2]
  const size_t arg_off = pairs;
  const int arg_ld = 2 * P.grid;
  pairs += static_cast<size_t>(2) * B * arg_ld;

  XE_HIP(hipMalloc(reinterpret_cast<void **>(&P.arena), pairs * 8));
  XE_HIP(hipMemsetAsync(P.arena, 0, pairs * 8, d->s));
  for (auto &fx : fix) {
    ll::Vec &v = field_of((*fx.list)[fx.idx], fx.field);
    v.p = P.arena + vecs[fx.vec].first;
    v.ld = vecs[fx.vec].second;
  }
  P.arg.p = P.arena + arg_off;
  P.arg.ld = arg_ld;

  ll_tile(c.vocab, P.grid, D, false, c.wdtype, P.head_lpr, P.head_rpl);
  // inputs per role (GEMV inputs padded, ll::xstride; attention q rows and
  // fold sources plain): A holds QKV / O / cross-attention inputs and q rows,
  // F the FFN inputs
  P.kin_a = std::max(std::max(ll::xstride(D), ll::xstride(hq)), std::max(nq, D));
  // F: the GEMV inputs, or (split FFN output) the FFN input and the hidden slice
  P.kin_f = ffn_split ? ll::xstride(D) + (ffn_kn + 3) / 4 * 4 : std::max(ll::xstride(D), ll::xstride(F));
  // scratch: attention blocks, merge tables, argmax partials, and the norm
  // gains of a GEMV input (up to 3 folds, gamma, beta: 5 regions)
  P.scratch = std::max(std::max(ll::attn_scratch_floats(hd, g), ll::attn_scratch_floats(hd, 1)),
                       std::max(ll::kMaxSplits * (ll::kDM + 2) + ll::kMaxSplits + ll::kW * (ll::kDM + 1), P.nb_t * 2 * P.grid));
  P.scratch = std::max(P.scratch, 5 * ll::nw_floats(D));
  if (ffn_split)  // the partials' staging and the reduce tables
    P.scratch = std::max(P.scratch, std::max(ll::dpart_obuf_floats(P.nb_t, D), ll::kW * P.nb_t * ll::kRedRows + 512));
  P.scratch += 16;
  auto base = [&](int kin) {
    return static_cast<long>(sizeof(float)) *
           (static_cast<long>(P.nb_t) * D + static_cast<long>(P.nb_t) * kin + ((P.scratch + 3) & ~3));
  };
  const long base_a = base(P.kin_a), base_f = base(P.kin_f);
  const long trace_res = static_cast<long>(sizeof(uint64_t) * (ll_trace_slots(P) + 1));  // a traced launch's marks
  if (std::max(base_a, base_f) + trace_res > static_cast<long>(kLLLds)) { P.why = "LDS need too large"; return; }
  // the weight stages take what each role's LDS has left
  const char *st_env = std::getenv("XE_LL_STAGE");
  const bool stage_on = !(st_env && std::string(st_env) == "0");
  P.stage_a = P.stage_f = 0;
  plan_stage(P.a, n_a, c.wdtype, stage_on ? static_cast<long>(kLLLds) - base_a - trace_res : -1, P.stage_a);
  // the split FFN output's projection slice goes to the stage during the GEMV before it
  const int dpart_need = ffn_split ? ll::kStageZero + ll::stage_pad(ffn_kn * D * (c.wdtype == XE_BF16 ? 2 : 1)) : 0;
  if (dpart_need > static_cast<long>(kLLLds) - base_f - trace_res) { P.why = "LDS need too large (FFN split)"; return; }
  plan_stage(P.f, n_f, c.wdtype, stage_on ? static_cast<long>(kLLLds) - base_f - trace_res : -1, P.stage_f,
             dpart_need);
  // then the attention side's key/value stage
  const char *kv_env = std::getenv("XE_LL_KV");
  const bool kv_on = !(kv_env && std::string(kv_env) == "0");
  P.kv_floats = plan_kv_stage(P.a, hd, c.max_ctx,
                              kv_on ? static_cast<long>(kLLLds) - base_a - P.stage_a - trace_res : -1);
  P.lds_bytes = static_cast<size_t>(std::max(base_a + P.stage_a + 4L * P.kv_floats, base_f + P.stage_f));

  XE_HIP(hipMalloc(reinterpret_cast<void **>(&P.dev_a), std::max<size_t>(1, P.a.size()) * sizeof(ll::Phase)));
  XE_HIP(hipMalloc(reinterpret_cast<void **>(&P.dev_f), std::max<size_t>(1, P.f.size()) * sizeof(ll::Phase)));
  XE_HIP(hipMemcpyAsync(P.dev_a, P.a.data(), P.a.size() * sizeof(ll::Phase), hipMemcpyHostToDevice, d->s));
  XE_HIP(hipMemcpyAsync(P.dev_f, P.f.data(), P.f.size() * sizeof(ll::Phase), hipMemcpyHostToDevice, d->s));
  XE_HIP(hipStreamSynchronize(d->s));
  P.ok = true;
}

xe_decoder::LLPlan &ll_plan_for(xe_decoder *d, int B) {
  auto it = d->ll_plans.find(B);
  if (it != d->ll_plans.end()) return it->second;
  xe_decoder::LLPlan &P = d->ll_plans[B];
  build_ll_plan(d, B, P);
  return P;
}

constexpr int kLLChunk = 256;  // decode steps per low-latency launch
constexpr int kStopCheck = 8;  // phase-kernel steps between looks at the stop flags

// n_steps tokens in one launch.  forced: device [n_forced][B] input tokens of
// the first steps (prompt feeding); logits: written for every step (the last
// step's values remain).

void run_ll(xe_decoder *d, int B, int n_steps, const int32_t *forced, int n_forced, bool want_logits,
            uint64_t *trace = nullptr) {
  xe_decoder::LLPlan &P = ll_plan_for(d, B);
  XE_REQUIRE(P.ok, "low-latency executor unsupported here: " + P.why);
  d->last_exec = XE_EXEC_LL;
  const auto &c = d->c;
  const bool gem = c.family == XE_GEMMA3, opt = c.family == XE_OPT;
  ll::StepParams sp{};
  sp.ph_a = P.dev_a;
  sp.n_a = static_cast<int>(P.a.size());
  sp.ph_f = P.dev_f;
  sp.n_f = static_cast<int>(P.f.size());
  sp.emb = d->emb.w;
  sp.emb_scale = d->emb.scale;
  sp.emb_exps = d->emb.exps;
  sp.pos_emb = d->pos_emb;
  Spec ps;
  sp.pos_off = opt ? 2 : 0;
  sp.pos_rows = tensor_spec(c, XE_T_POS_EMB, -1, ps) ? ps.rows : 1;
  sp.emb_mul = sqrtf(static_cast<float>(c.d_model));
  sp.use_mul = gem ? 1 : 0;
  sp.vocab = c.vocab;
  sp.d = c.d_model;
  sp.nb = B;
  sp.head_norm = gem ? XE_NORM_RMS1P : XE_NORM_LN;
  sp.head_gamma = d->lnf_w;
  sp.head_beta = gem ? nullptr : d->lnf_b;
  sp.head_eps = c.eps;
  sp.head_lpr = P.head_lpr;
  sp.head_rpl = P.head_rpl;
  sp.logits = want_logits ? d->logits : nullptr;
  sp.arg = P.arg;
  sp.last_max = opt ? 1 : 0;
  sp.tokens = d->tokens;
  sp.pos = d->pos;
  sp.next = d->next;
  sp.hist = d->hist;
  sp.hist_stride = c.max_ctx + 1;
  sp.forced = forced;
  sp.n_forced = forced ? n_forced : 0;
  sp.stop = d->stop_id;
  sp.done = d->stop_dev + 1;
  sp.n_steps = n_steps;
  sp.ep0 = d->ll_epoch;
  sp.status = d->step_status;
  int khz = 0;
  XE_HIP(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, d->dev->ordinal));
  // 50 ms per wait; XE_WAIT_LIMIT_US overrides it and XE_LL_STALL_TEST=1
  // makes the end-of-step wait expect an epoch that never comes (both for
  // tests of the bounded-wait failure path)
  const char *lim = std::getenv("XE_WAIT_LIMIT_US");
  const double lim_us = lim ? std::max(1.0, std::atof(lim)) : 50000.0;
  sp.limit = static_cast<uint64_t>(static_cast<double>(khz > 0 ? khz : 100000) * lim_us / 1000.0);
  const char *stall = std::getenv("XE_LL_STALL_TEST");
  sp.stall = (stall && std::atoi(stall) > 0) ? 1u : 0u;
  sp.kin_a = P.kin_a;
  sp.kin_f = P.kin_f;
  sp.scratch = P.scratch;
  sp.stage_a = P.stage_a / 4;
  sp.stage_f = P.stage_f / 4;
  sp.kv_floats = P.kv_floats;
  sp.trace = trace;
  // a traced launch keeps its marks in LDS behind the scratch area
  sp.trace_slots = trace ? static_cast<int>(ll_trace_slots(P)) : 0;
  const size_t lds = P.lds_bytes + (trace ? sizeof(uint64_t) * (sp.trace_slots + 1) : 0);
  ll::launch(sp, c.wdtype, P.nb_t, P.hd, P.g, P.kv8, lds, P.grid, d->s);
  d->ll_epoch += static_cast<unsigned>(n_steps);
}

// Executor choice for the phase kernels: one HIP graph per token (the
// default); XE_STEP=eager launches the phases one by one (profiling).
enum class Exec { Graph, Eager };

Exec exec_for(const xe_decoder::Plan &plan) {
  const char *e = getenv("XE_STEP");
  if (getenv("XE_NO_GRAPH") || (e && std::string(e) == "eager")) return Exec::Eager;
  return Exec::Graph;
}

hipGraphExec_t graph_for(xe_decoder *d, xe_decoder::Plan &plan) {
  if (plan.graph) return plan.graph;
  hipGraph_t g = nullptr;
  XE_HIP(hipStreamBeginCapture(d->s, hipStreamCaptureModeRelaxed));
  try {
    for (const auto &ph : plan.phases) launch_phase(ph, d->s);
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
  plan.graph = ex;
  return ex;
}

// The low-latency executor (the default) where its plan supports the model
// and batch; otherwise, or when XE_STEP / XE_NO_GRAPH name a phase-kernel
// executor, the phase kernels.
bool use_ll(xe_decoder *d, int B) {
  const char *e = getenv("XE_STEP");
  if (getenv("XE_NO_GRAPH") || (e && *e && std::string(e) != "ll")) return false;
  return ll_plan_for(d, B).ok;
}

void run_step(xe_decoder *d, int B) {
  if (use_ll(d, B)) {
    run_ll(d, B, 1, nullptr, 0, true);
    return;
  }
  d->last_exec = XE_EXEC_GRAPH;
  xe_decoder::Plan &plan = plan_for(d, B);
  switch (exec_for(plan)) {
    case Exec::Graph:
      XE_HIP(hipGraphLaunch(graph_for(d, plan), d->s));
      return;
    case Exec::Eager:
      for (const auto &ph : plan.phases) launch_phase(ph, d->s);
      return;
  }
}

// Run one GEMV over `batch` rows now (standalone kernels; chunks of 8).
void run_gemv_now(const GemvCall &g, int batch, hipStream_t s) {
  xe_decoder::Plan tmp;
  PlanBuilder pb{tmp};
  pb.gemv(g, batch, "gemv");
  for (const auto &ph : tmp.phases) launch_phase(ph, s);
}

// After a run of low-latency launches: a wait that timed out (or a plan the
// kernel could not run) leaves the status word set; report it and clear it.
void check_step_status(xe_decoder *d) {
  unsigned st = 0;
  XE_HIP(hipMemcpy(&st, d->step_status, 4, hipMemcpyDeviceToHost));
  if (st) {
    XE_HIP(hipMemset(d->step_status, 0, 4));
    if (st == 2u)
      fail("low-latency step kernel: GEMV tile not compiled (host/device tile menus differ); results are invalid");
    if (st == 3u)
      fail("low-latency step kernel: a phase kind on a role not compiled for it (plan error); results are invalid");
    fail("low-latency step kernel: an exchange wait timed out (every workgroup stopped); results are invalid");
  }
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
      run_gemv_now(g, T, d->s);
      if (which == 0 ? d->cross_i8k : d->cross_i8v)
        hipLaunchKernelGGL(cross_quant_kernel, dim3(c.n_heads), dim3(256), 0, d->s, tmp, T, c.n_heads, c.head_dim,
                           reinterpret_cast<int8_t *>(which == 0 ? l.ck : l.cv), which == 0 ? l.cks : l.cvs);
      else
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

int xe_buf_fill_synthetic(xe_buf *buf, size_t offset, int dtype, uint64_t seed, uint32_t stream,
                          uint64_t start, float mean, float stdv, size_t count) {
  return guard_d([&]() -> int {
    XE_REQUIRE(buf && buf->ptr, "null buffer");
    XE_REQUIRE(dtype == XE_F32 || dtype == XE_BF16 || dtype == XE_I8, "dtype must be XE_F32, XE_BF16 or XE_I8");
    const size_t es = dtype == XE_F32 ? 4 : dtype == XE_BF16 ? 2 : 1;
    XE_REQUIRE(offset % es == 0, "offset not aligned to the element size");
    XE_REQUIRE(count <= (buf->size - std::min(offset, buf->size)) / es, "fill runs past the buffer");
    if (count == 0) return 0;
    DeviceGuard dg(buf->dev->ordinal);
    hipStream_t st = buf->dev->stream;
    const size_t blocks = std::min<size_t>((count + 255) / 256, 8192);
    synth_fill_kernel<<<static_cast<unsigned>(blocks), 256, 0, st>>>(
        synth_base(seed, stream), mean, stdv * kIh4InvStd, start, count,
        static_cast<char *>(buf->ptr) + offset, dtype);
    XE_HIP(hipGetLastError());
    XE_HIP(hipStreamSynchronize(st));
    return 0;
  }, -1);
}

int xe_buf_copy(xe_buf *dst, size_t dst_off, const xe_buf *src, size_t src_off, size_t nbytes) {
  return guard_d([&]() -> int {
    XE_REQUIRE(dst && src && dst->ptr && src->ptr, "null buffer");
    XE_REQUIRE(dst->dev == src->dev, "buffers on different devices");
    XE_REQUIRE(nbytes % 16 == 0 && dst_off % 16 == 0 && src_off % 16 == 0,
               "copy sizes and offsets must be multiples of 16 bytes");
    XE_REQUIRE(dst_off <= dst->size && nbytes <= dst->size - dst_off, "copy runs past the destination");
    XE_REQUIRE(src_off <= src->size && nbytes <= src->size - src_off, "copy runs past the source");
    if (nbytes == 0) return 0;
    DeviceGuard dg(dst->dev->ordinal);
    hipStream_t st = dst->dev->stream;
    const size_t n = nbytes / 16;
    const size_t blocks = std::min<size_t>((n + 255) / 256, 16384);
    copy16_kernel<<<static_cast<unsigned>(blocks), 256, 0, st>>>(
        reinterpret_cast<const uint4 *>(static_cast<const char *>(src->ptr) + src_off),
        reinterpret_cast<uint4 *>(static_cast<char *>(dst->ptr) + dst_off), n);
    XE_HIP(hipGetLastError());
    XE_HIP(hipStreamSynchronize(st));
    return 0;
  }, -1);
}

xe_decoder *xe_decoder_create(xe_device *dev, const xe_model_config *cfg, int max_batch) {
  return guard_d([&]() -> xe_decoder * {
    XE_REQUIRE(dev && cfg, "null argument");
    validate_config(*cfg, max_batch);
    DeviceGuard dg(dev->ordinal);
    auto *d = new xe_decoder;
    d->dev = dev;
    d->c = *cfg;
    d->max_batch = max_batch;
    d->hpos.assign(max_batch, 0);
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
    for (size_t li = 0; li < d->ll_fc2t.size(); li++) ll_fc2t_layer(d, static_cast<int>(li));
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
      if (kind == XE_T_FC2_W && !d->ll_fc2t.empty()) ll_fc2t_layer(d, layer);
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

int xe_model_tensor_shape(const xe_model_config *cfg, int kind, int layer, int *rows, int *cols) {
  try {
    XE_REQUIRE(cfg, "null config");
    XE_REQUIRE(layer >= -1 && layer < cfg->n_layers, "layer out of range");
    Spec sp;
    if (kind < 0 || kind >= XE_T_COUNT || !tensor_spec(*cfg, kind, layer, sp)) {
      set_error("tensor kind not used by this model family");
      return -1;
    }
    if (rows) *rows = sp.rows;
    if (cols) *cols = sp.cols;
    return 0;
  } catch (const std::exception &e) {
    set_error(e.what());
    return -1;
  }
}

int xe_decoder_config(xe_decoder *d, xe_model_config *out) {
  if (!d || !out) {
    set_error("null argument");
    return -1;
  }
  *out = d->c;
  return 0;
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
    d->hpos.assign(d->max_batch, 0);
    d->live = 0;
    return 0;
  }, -1);
}

int xe_decoder_prime_kv(xe_decoder *d, int stream, int n_pos, uint64_t seed) {
  return guard_d([&]() -> int {
    XE_REQUIRE(d, "null decoder");
    XE_REQUIRE(stream >= 0 && stream < d->max_batch, "stream out of range");
    XE_REQUIRE(n_pos >= 0 && n_pos < d->c.max_ctx, "n_pos must be in [0, max_ctx)");
    if (d->c.family != XE_GEMMA3) XE_REQUIRE(n_pos < d->c.max_pos, "n_pos beyond the position table");
    DeviceGuard dg(d->dev->ordinal);
    const auto &c = d->c;
    const int hk = c.n_kv_heads, hd = c.head_dim;
    const size_t count = static_cast<size_t>(n_pos) * hd;
    if (count > 0) {
      const unsigned blocks = static_cast<unsigned>(std::min<size_t>((count + 255) / 256, 4096));
      for (int l = 0; l < c.n_layers; l++)
        for (int h = 0; h < hk; h++) {
          // element (pos, e) of (layer, stream, head) sits at the same offset
          // as in the oracle's cache: [layer][stream][head][max_ctx][hd]
          const size_t off = d->kv_layer_elems() * l + ((static_cast<size_t>(stream) * hk + h) * c.max_ctx) * hd;
          const uint32_t id = static_cast<uint32_t>(2 * (l * hk + h));
          synth_fill_kernel<<<blocks, 256, 0, d->s>>>(synth_base(seed, id), 0.0f, kIh4InvStd, 0, count,
                                                      d->kc + off, XE_BF16);
          XE_HIP(hipGetLastError());
          synth_fill_kernel<<<blocks, 256, 0, d->s>>>(synth_base(seed, id + 1), 0.0f, kIh4InvStd, 0, count,
                                                      d->vc + off, XE_BF16);
          XE_HIP(hipGetLastError());
        }
    }
    XE_HIP(hipStreamSynchronize(d->s));
    int32_t *h = d->host_tok;
    h[0] = n_pos;
    XE_HIP(hipMemcpyAsync(d->pos + stream, h, 4, hipMemcpyHostToDevice, d->s));
    XE_HIP(hipStreamSynchronize(d->s));
    d->hpos[stream] = n_pos;
    d->live = std::max(d->live, stream + 1);
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

int xe_decoder_set_cross_int8(xe_decoder *d, int k_int8, int v_int8) {
  return guard_d([&]() -> int {
    XE_REQUIRE(d, "null decoder");
    XE_REQUIRE(d->c.family == XE_WHISPER, "cross attention is Whisper-only");
    DeviceGuard dg(d->dev->ordinal);
    const int k = k_int8 ? 1 : 0, v = v_int8 ? 1 : 0;
    if (k != d->cross_i8k || v != d->cross_i8v) {
      drop_plans(d);  // the cross-attention phase and the executor choice change
      d->cross_i8k = k;
      d->cross_i8v = v;
      d->cross_ready = false;
    }
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
    check_step_status(d);
    for (int b = 0; b < batch; b++) d->hpos[b] = pos[b] + 1;
    d->live = std::max(d->live, batch);
    return 0;
  }, -1);
}

// ---------------------------------------------------------------------------
// Resident decode step (the reference's ElfResident: a constant program bound
// once, per-token parameters written into a host-mapped scratchpad, then
// dispatch -- npu-xrt/src/lib.rs:591-629, xrt_shim.h:95-111).  Here the
// program is the decoder's step for one batch size (its HIP graph or the
// low-latency kernel, built on first use and kept), the scratchpad is pinned
// host memory holding tokens and positions, and dispatch copies them to the
// device, launches the step and (dispatch) waits or (dispatch_start) returns
// a run handle.
// ---------------------------------------------------------------------------
}  // extern "C"

struct xe_resident {
  xe_decoder *d = nullptr;
  int batch = 0;
  int32_t *stage = nullptr;  // pinned: tokens [batch] | positions [batch] | next [batch]
  bool written = false;
  bool in_flight = false;
  int n_done = 0;            // completed dispatches
};

namespace xe {
void resident_done(xe_resident *r) {
  if (!r || !r->in_flight) return;
  r->in_flight = false;
  r->n_done++;
  DeviceGuard dg(r->d->dev->ordinal);
  check_step_status(r->d);
}
}  // namespace xe

extern "C" {

xe_resident *xe_resident_open(xe_decoder *d, int batch) {
  return guard_d([&]() -> xe_resident * {
    XE_REQUIRE(d, "null decoder");
    XE_REQUIRE(batch >= 1 && batch <= d->max_batch, "batch out of range");
    DeviceGuard dg(d->dev->ordinal);
    auto *r = new xe_resident;
    r->d = d;
    r->batch = batch;
    const hipError_t e = hipHostMalloc(reinterpret_cast<void **>(&r->stage), 3 * batch * sizeof(int32_t),
                                       hipHostMallocDefault);
    if (e != hipSuccess) {
      delete r;
      XE_HIP(e);
    }
    if (!use_ll(d, batch)) {  // capture the step graph once, now
      xe_decoder::Plan &plan = plan_for(d, batch);
      if (exec_for(plan) == Exec::Graph) (void)graph_for(d, plan);
    }
    return r;
  }, nullptr);
}

void xe_resident_close(xe_resident *r) {
  guard_d([&]() -> int {
    if (!r) return 0;
    DeviceGuard dg(r->d->dev->ordinal);
    (void)hipStreamSynchronize(r->d->s);
    (void)hipHostFree(r->stage);
    delete r;
    return 0;
  }, -1);
}

int xe_resident_write(xe_resident *r, const int32_t *tokens, const int32_t *pos) {
  return guard_d([&]() -> int {
    XE_REQUIRE(r && tokens && pos, "null argument");
    XE_REQUIRE(!r->in_flight, "a dispatch is in flight: wait for it before writing new parameters");
    const auto &c = r->d->c;
    for (int b = 0; b < r->batch; b++) {
      XE_REQUIRE(tokens[b] >= 0 && tokens[b] < c.vocab, "token id out of range");
      XE_REQUIRE(pos[b] >= 0 && pos[b] < c.max_ctx, "position out of range");
      if (c.family != XE_GEMMA3) XE_REQUIRE(pos[b] < c.max_pos, "position beyond the table");
    }
    std::memcpy(r->stage, tokens, r->batch * 4);
    std::memcpy(r->stage + r->batch, pos, r->batch * 4);
    r->written = true;
    return 0;
  }, -1);
}

namespace {
void resident_submit(xe_resident *r) {
  XE_REQUIRE(r, "null resident step");
  XE_REQUIRE(r->written, "xe_resident_write first");
  XE_REQUIRE(!r->in_flight, "a dispatch is already in flight");
  xe_decoder *d = r->d;
  XE_REQUIRE(d->c.family != XE_WHISPER || d->cross_ready, "Whisper: set_cross first");
  const int B = r->batch;
  XE_HIP(hipMemcpyAsync(d->tokens, r->stage, B * 4, hipMemcpyHostToDevice, d->s));
  XE_HIP(hipMemcpyAsync(d->pos, r->stage + B, B * 4, hipMemcpyHostToDevice, d->s));
  run_step(d, B);
  XE_HIP(hipMemcpyAsync(r->stage + 2 * B, d->next, B * 4, hipMemcpyDeviceToHost, d->s));
  for (int b = 0; b < B; b++) d->hpos[b] = r->stage[B + b] + 1;
  d->live = std::max(d->live, B);
  r->in_flight = true;
}
}  // namespace

int xe_resident_dispatch(xe_resident *r) {
  return guard_d([&]() -> int {
    DeviceGuard dg(r ? r->d->dev->ordinal : 0);
    resident_submit(r);
    XE_HIP(hipStreamSynchronize(r->d->s));
    resident_done(r);
    return 0;
  }, -1);
}

xe_run *xe_resident_dispatch_start(xe_resident *r) {
  return guard_d([&]() -> xe_run * {
    DeviceGuard dg(r ? r->d->dev->ordinal : 0);
    resident_submit(r);
    auto *run = new xe_run;
    run->ordinal = r->d->dev->ordinal;
    run->res = r;
    hipError_t e = hipEventCreateWithFlags(&run->ev, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventRecord(run->ev, r->d->s);
    if (e != hipSuccess) {
      if (run->ev) (void)hipEventDestroy(run->ev);
      delete run;
      (void)hipStreamSynchronize(r->d->s);
      r->in_flight = false;
      XE_HIP(e);
    }
    return run;
  }, nullptr);
}

int xe_resident_read(xe_resident *r, int32_t *next, float *logits) {
  return guard_d([&]() -> int {
    XE_REQUIRE(r, "null resident step");
    XE_REQUIRE(!r->in_flight, "a dispatch is in flight: wait for its run first");
    XE_REQUIRE(r->n_done > 0, "no completed dispatch");
    if (next) std::memcpy(next, r->stage + 2 * r->batch, r->batch * 4);
    if (logits) {
      DeviceGuard dg(r->d->dev->ordinal);
      XE_HIP(hipMemcpy(logits, r->d->logits, static_cast<size_t>(r->batch) * r->d->c.vocab * 4,
                       hipMemcpyDeviceToHost));
    }
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
  XE_HIP(hipMemsetAsync(d->stop_dev + 1, 0, batch * 4, d->s));  // no stream has stopped
  if (use_ll(d, batch)) {  // the whole prompt in one launch, tokens forced
    XE_HIP(hipMemcpyAsync(d->ll_forced, h, static_cast<size_t>(n_prompt) * batch * 4, hipMemcpyHostToDevice, d->s));
    XE_HIP(hipMemcpyAsync(d->tokens, h, batch * 4, hipMemcpyHostToDevice, d->s));
    run_ll(d, batch, n_prompt, d->ll_forced, n_prompt, false);
    XE_HIP(hipStreamSynchronize(d->s));
    check_step_status(d);
    for (int b = 0; b < batch; b++) d->hpos[b] = n_prompt;
    d->live = batch;
    return;
  }
  {
    xe_decoder::Plan &plan = plan_for(d, batch);  // build (and capture) before timing
    if (exec_for(plan) == Exec::Graph) (void)graph_for(d, plan);
  }
  for (int p = 0; p < n_prompt; p++) {
    XE_HIP(hipMemcpyAsync(d->tokens, h + static_cast<size_t>(p) * batch, batch * 4,
                          hipMemcpyHostToDevice, d->s));
    // only the last prompt step's argmax is a generated token: earlier
    // steps' stop marks are cleared
    if (p == n_prompt - 1 && p > 0 && d->stop_id >= 0)
      XE_HIP(hipMemsetAsync(d->stop_dev + 1, 0, batch * 4, d->s));
    run_step(d, batch);
  }
  XE_HIP(hipStreamSynchronize(d->s));
  check_step_status(d);
  for (int b = 0; b < batch; b++) d->hpos[b] = n_prompt;
  d->live = batch;
}

// n_steps further greedy steps from the device state; out [batch, n_steps]
// receives the tokens those steps emit (may be NULL).  With a stop token set
// the run ends once every stream has emitted it (the stop token fills the
// rest of a stopped stream's row); returns the steps that ran.
int decode(xe_decoder *d, int batch, int n_steps, int32_t *out, double *device_us) {
  check_ready(d, batch);
  XE_REQUIRE(d->live > 0, "feed a prompt first");
  XE_REQUIRE(n_steps >= 0, "negative step count");
  d->require_room(batch, n_steps);
  const std::vector<int> first_pos(d->hpos.begin(), d->hpos.begin() + batch);  // positions the next step processes
  hipEvent_t e0, e1;
  XE_HIP(hipEventCreate(&e0));
  XE_HIP(hipEventCreate(&e1));
  const bool ll_exec = use_ll(d, batch);
  const bool stop = d->stop_id >= 0;
  // with a stop token the host looks at the done flags after every chunk of
  // steps (a low-latency launch also ends by itself once every stream is
  // done) and launches no more once all streams have stopped
  int32_t *hdone = d->host_tok;
  auto all_done = [&]() -> bool {
    XE_HIP(hipMemcpyAsync(hdone, d->stop_dev + 1, batch * 4, hipMemcpyDeviceToHost, d->s));
    XE_HIP(hipStreamSynchronize(d->s));
    for (int b = 0; b < batch; b++)
      if (!hdone[b]) return false;
    return true;
  };
  XE_HIP(hipStreamSynchronize(d->s));  // host_tok staging is free
  std::vector<int32_t> pre_done(batch, 0);  // streams stopped before this run
  if (stop) {
    (void)all_done();
    pre_done.assign(hdone, hdone + batch);
  }
  XE_HIP(hipEventRecord(e0, d->s));
  if (ll_exec) {
    for (int i = 0; i < n_steps; i += kLLChunk) {
      if (stop && all_done()) break;
      run_ll(d, batch, std::min(kLLChunk, n_steps - i), nullptr, 0, false);
    }
  } else {
    for (int i = 0; i < n_steps; i++) {
      if (stop && i % kStopCheck == 0 && all_done()) break;
      run_step(d, batch);
    }
  }
  XE_HIP(hipEventRecord(e1, d->s));
  XE_HIP(hipEventSynchronize(e1));
  float ms = 0.f;
  XE_HIP(hipEventElapsedTime(&ms, e0, e1));
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  check_step_status(d);
  // steps that ran (streams advance in lockstep)
  int ran = n_steps;
  if (stop && n_steps > 0) {
    XE_HIP(hipMemcpy(hdone, d->pos, 4, hipMemcpyDeviceToHost));
    ran = std::max(0, std::min(n_steps, hdone[0] - first_pos[0]));
  }
  if (ran > 0) d->last_step_us = 1000.0 * ms / ran;
  if (device_us) *device_us = 1000.0 * ms;
  for (int b = 0; b < batch; b++) d->hpos[b] += ran;
  if (out && n_steps > 0) {
    std::vector<int32_t> hist(static_cast<size_t>(batch) * (d->c.max_ctx + 1));
    XE_HIP(hipMemcpy(hist.data(), d->hist, hist.size() * 4, hipMemcpyDeviceToHost));
    for (int b = 0; b < batch; b++) {
      bool done = pre_done[b] != 0;  // a stream that had stopped emits nothing more
      for (int i = 0; i < n_steps; i++) {
        int32_t t = i < ran ? hist[static_cast<size_t>(b) * (d->c.max_ctx + 1) + first_pos[b] + i] : d->stop_id;
        if (done) t = d->stop_id;
        if (stop && t == d->stop_id) done = true;
        out[static_cast<size_t>(b) * n_steps + i] = t;
      }
    }
  }
  return ran;
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
    return decode(d, batch, n_steps, out, device_us);
  }, -1);
}

int xe_decoder_set_stop(xe_decoder *d, int32_t stop_id) {
  return guard_d([&]() -> int {
    XE_REQUIRE(d, "null decoder");
    XE_REQUIRE(stop_id >= -1 && stop_id < d->c.vocab, "stop token must be -1 (none) or a token id");
    DeviceGuard dg(d->dev->ordinal);
    XE_HIP(hipStreamSynchronize(d->s));  // host_tok staging is free
    d->host_tok[0] = stop_id;
    XE_HIP(hipMemcpyAsync(d->stop_dev, d->host_tok, 4, hipMemcpyHostToDevice, d->s));
    XE_HIP(hipStreamSynchronize(d->s));
    d->stop_id = stop_id;
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
      const bool done = d->stop_id >= 0 && first[b] == d->stop_id;
      for (int i = 0; i + 1 < n_new; i++)
        out[static_cast<size_t>(b) * n_new + 1 + i] =
            done ? d->stop_id : rest[static_cast<size_t>(b) * (n_new - 1) + i];
    }
    return 0;
  }, -1);
}

int xe_decoder_generate_until(xe_decoder *d, const int32_t *prompt, int n_prompt, int batch, int max_new,
                              int32_t stop_id, int32_t *out, int32_t *n_out) {
  const int prev = d ? d->stop_id : -1;
  if (xe_decoder_set_stop(d, stop_id) != 0) return -1;
  const int rc = xe_decoder_generate(d, prompt, n_prompt, batch, max_new, out);
  if (xe_decoder_set_stop(d, prev) != 0) return -1;
  if (rc != 0) return rc;
  if (n_out)
    for (int b = 0; b < batch; b++) {
      int n = 0;
      while (n < max_new && (stop_id < 0 || out[static_cast<size_t>(b) * max_new + n] != stop_id)) n++;
      n_out[b] = n;
    }
  return 0;
}

int xe_decoder_profile_step(xe_decoder *d, int batch, int max_entries, char *labels, double *us,
                            double *bytes) {
  return guard_d([&]() -> int {
    XE_REQUIRE(d && labels && us && bytes, "null argument");
    check_ready(d, batch);
    XE_REQUIRE(d->live > 0, "feed a prompt first");
    d->require_room(batch, 1);
    DeviceGuard dg(d->dev->ordinal);
    XE_HIP(hipStreamSynchronize(d->s));
    d->prof_pos.assign(batch, 0);
    XE_HIP(hipMemcpy(d->prof_pos.data(), d->pos, batch * 4, hipMemcpyDeviceToHost));
    std::vector<xe_decoder::ProfEntry> entries;
    d->prof = &entries;
    xe_decoder::Plan &plan = plan_for(d, batch);
    const double hk4 = static_cast<double>(d->c.n_kv_heads) * d->c.head_dim * 4;
    double kv_bytes = 0;
    for (int b = 0; b < batch; b++) kv_bytes += (d->prof_pos[b] + 1) * hk4;
    auto phase_bytes = [&](size_t i) {
      return plan.bytes[i] + (plan.labels[i] == "attn_self" ? kv_bytes : 0.0);
    };
    if (use_ll(d, batch)) {
      // One low-latency step with the wall-clock trace: per role, each phase's
      // time is the advance of that role's latest phase end (the A and F
      // sides overlap, so the two lists are separate timelines).
      xe_decoder::LLPlan &P = ll_plan_for(d, batch);
      const size_t na = P.a.size(), nf = P.f.size(), G = static_cast<size_t>(P.grid);
      const size_t slots = ll_trace_slots(P);
      uint64_t *tr = nullptr;
      XE_HIP(hipMalloc(reinterpret_cast<void **>(&tr), slots * G * sizeof(uint64_t)));
      std::vector<uint64_t> h(slots * G);
      try {
        XE_HIP(hipMemsetAsync(tr, 0, slots * G * sizeof(uint64_t), d->s));
        run_ll(d, batch, 1, nullptr, 0, true, tr);
        XE_HIP(hipStreamSynchronize(d->s));
        XE_HIP(hipMemcpy(h.data(), tr, h.size() * sizeof(uint64_t), hipMemcpyDeviceToHost));
      } catch (...) {
        (void)hipFree(tr);
        throw;
      }
      (void)hipFree(tr);
      check_step_status(d);
      for (int b = 0; b < batch; b++) d->hpos[b] += 1;
      if (const char *raw = getenv("XE_LL_TRACE_RAW")) {
        // diagnostic: the raw per-workgroup trace, [slots][grid] u64 ticks
        if (FILE *f = std::fopen(raw, "wb")) {
          const uint64_t dims[4] = {slots, G, na, nf};
          std::fwrite(dims, sizeof(dims), 1, f);
          std::fwrite(h.data(), sizeof(uint64_t), h.size(), f);
          std::fclose(f);
        }
      }
      int khz = 0;
      XE_HIP(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, d->dev->ordinal));
      XE_REQUIRE(khz > 0, "device wall clock rate unknown");
      const double us_per_tick = 1000.0 / khz;
      uint64_t t0 = ~0ull;
      for (size_t w = 0; w < G; w++) t0 = std::min(t0, h[(na + nf + 3) * G + w]);
      auto slot_max = [&](size_t sl) {
        uint64_t m = 0;
        for (size_t w = 0; w < G; w++) m = std::max(m, h[sl * G + w]);
        return m;
      };
      int n = 0;
      auto emit = [&](const std::string &label, uint64_t from, uint64_t to, double b) {
        if (n >= max_entries) return;
        us[n] = to > from ? (to - from) * us_per_tick : 0.0;
        bytes[n] = b;
        std::snprintf(labels + 32 * n, 32, "%s", label.c_str());
        n++;
      };
      // per phase: "wait" = previous end -> input ready (latest over the
      // role's workgroups), then ready -> end
      uint64_t prev = t0, a_end = t0, f_end = t0;
      for (size_t i = 0; i < na; i++) {
        const uint64_t r = slot_max(na + nf + 4 + i), e = slot_max(i);
        emit("A:wait:" + P.a_labels[i], prev, std::max(prev, r), 0.0);
        const bool is_attn = P.a[i].kind == ll::LK_ATTN;
        if (is_attn) {  // sub-stages: q staged, scores, softmax, P.V, partials out
          const size_t sb = 2 * (na + nf) + 4 + ll::kSubSlots * i;
          const uint64_t s0 = slot_max(sb), s1 = slot_max(sb + 1), s2 = slot_max(sb + 2), s3 = slot_max(sb + 3);
          emit("A:" + P.a_labels[i] + ".stage", std::max(prev, r), s0, 0.0);
          emit("A:" + P.a_labels[i] + ".qk", s0, s1, P.a_bytes[i] + (P.a_labels[i] == "attn_self" ? kv_bytes : 0.0));
          emit("A:" + P.a_labels[i] + ".softmax", s1, s2, 0.0);
          emit("A:" + P.a_labels[i] + ".pv", s2, s3, 0.0);
          emit("A:" + P.a_labels[i] + ".out", s3, e, 0.0);
        } else if (P.a[i].kind == ll::LK_GEMV) {  // compute / reduction + epilogue
          const uint64_t s1 = slot_max(2 * (na + nf) + 4 + ll::kSubSlots * i + 1);
          emit("A:" + P.a_labels[i] + ".mac", std::max(prev, r), s1, P.a_bytes[i]);
          emit("A:" + P.a_labels[i] + ".epi", s1, e, 0.0);
        } else {
          emit("A:" + P.a_labels[i], std::max(prev, r), e, P.a_bytes[i]);
        }
        prev = std::max(prev, e);
      }
      a_end = prev;
      prev = t0;
      for (size_t i = 0; i < nf; i++) {
        const uint64_t r = slot_max(2 * na + nf + 4 + i), e = slot_max(na + i);
        emit("F:wait:" + P.f_labels[i], prev, std::max(prev, r), 0.0);
        if (P.f[i].kind == ll::LK_GEMV) {
          const uint64_t s1 = slot_max(2 * (na + nf) + 4 + ll::kSubSlots * (na + i) + 1);
          emit("F:" + P.f_labels[i] + ".mac", std::max(prev, r), s1, P.f_bytes[i]);
          emit("F:" + P.f_labels[i] + ".epi", s1, e, 0.0);
        } else {
          emit("F:" + P.f_labels[i], std::max(prev, r), e, P.f_bytes[i]);
        }
        prev = std::max(prev, e);
      }
      f_end = prev;
      const uint64_t lm = slot_max(na + nf), am = slot_max(na + nf + 1), em = slot_max(na + nf + 2);
      emit("gemv_lmhead", std::max(a_end, f_end), lm, static_cast<double>(d->emb.bytes()));
      emit("argmax", lm, am, 16.0 * batch * G);
      emit("embed", am, em, static_cast<double>(batch) * d->c.d_model * 4);
      return n;
    }
    try {
      d->mark("start", 0.0);
      for (size_t i = 0; i < plan.phases.size(); i++) {  // eager, one event after each launch
        launch_phase(plan.phases[i], d->s);
        d->mark(plan.labels[i], phase_bytes(i));
      }
    } catch (...) {
      d->prof = nullptr;
      for (auto &e : entries) (void)hipEventDestroy(e.ev);
      throw;
    }
    d->prof = nullptr;
    XE_HIP(hipStreamSynchronize(d->s));
    for (int b = 0; b < batch; b++) d->hpos[b] += 1;
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

int xe_decoder_executor(xe_decoder *d, int batch) {
  return guard_d([&]() -> int {
    XE_REQUIRE(d, "null decoder");
    XE_REQUIRE(batch >= 1 && batch <= d->max_batch, "batch out of range");
    DeviceGuard dg(d->dev->ordinal);
    if (use_ll(d, batch)) return XE_EXEC_LL;
    switch (exec_for(plan_for(d, batch))) {
      case Exec::Eager: return XE_EXEC_EAGER;
      case Exec::Graph: break;
    }
    return XE_EXEC_GRAPH;
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
