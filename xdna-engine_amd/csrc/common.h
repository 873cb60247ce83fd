// common.h -- internals shared by the HIP sources of libxdna_engine.so.
//
// Error model (rust/npu-xrt/shim/xrt_shim.cpp:42-56): internal code throws
// xe::Error; every extern "C" entry point catches it (and anything else),
// stores the message in a thread-local string and returns NULL / -1.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/xdna_engine.h"

namespace xe {

struct Error : std::runtime_error {
  using std::runtime_error::runtime_error;
};

[[noreturn]] void fail(const std::string &msg);
void hip_check(hipError_t e, const char *what, const char *file, int line);
#define XE_HIP(call) ::xe::hip_check((call), #call, __FILE__, __LINE__)
#define XE_REQUIRE(cond, msg)                        \
  do {                                               \
    if (!(cond)) ::xe::fail(std::string(msg));       \
  } while (0)

void set_error(const std::string &msg);

// Scoped "make this device current" guard.
struct DeviceGuard {
  int prev = -1;
  explicit DeviceGuard(int ordinal);
  ~DeviceGuard();
};

}  // namespace xe

// ---------------------------------------------------------------------------
// Opaque handle bodies
// ---------------------------------------------------------------------------

struct xe_device {
  int ordinal = 0;
  hipStream_t stream = nullptr;  // default-priority stream owned by the device
  std::string arch;
  int num_cus = 0;
  size_t max_lds = 0;
};

struct xe_buf {
  xe_device *dev = nullptr;
  void *ptr = nullptr;
  size_t size = 0;
};

// A registered weight matrix [m, k] resident in HBM.
//   XE_I8    q int8 [m,k] row-major + scale fp32 [m]
//   XE_BF16  bits uint16 [m,k]
//   XE_BFP16 mant int8 [m,k] + exps uint8 [m, k/8] (biased exponent e+127)
struct xe_weight {
  xe_ctx *ctx = nullptr;
  int wdtype = XE_I8;
  int m = 0, k = 0;
  void *w = nullptr;       // device
  float *scale = nullptr;  // device, XE_I8 only
  uint8_t *exps = nullptr; // device, XE_BFP16 only
  float *bias = nullptr;   // device or null
  int norm = XE_NORM_NONE;
  float *gamma = nullptr;  // device, k
  float *beta = nullptr;   // device, k
  float eps = 1e-5f;
  bool owns = true;        // false for views into a decoder's arena
};

struct xe_ctx {
  xe_device *dev = nullptr;
  uint64_t dispatches = 0;
  // reusable staging for the host-pointer entry points
  void *scratch = nullptr;
  size_t scratch_size = 0;
  void *host_pinned = nullptr;
  size_t host_pinned_size = 0;
  // split-K attention workspace (partials) and the per-(stream, kv head)
  // arrival counters of the in-place merge (zeroed once, self-resetting)
  float *attn_work = nullptr;
  size_t attn_work_floats = 0;
  unsigned *attn_cnt = nullptr;
  size_t attn_cnt_words = 0;
  // batched GEMM (more than 8 rows): split-K partials, arrival counters
  // (zeroed once, self-resetting) and the prologue's normalised rows
  float *gemm_ws = nullptr;
  unsigned *gemm_cnt = nullptr;
  float *gemm_xn = nullptr;
  size_t gemm_xn_floats = 0;
  // W8A8: partial maxima, the device scale_a and the int8 activations
  char *w8a8_ws = nullptr;
  size_t w8a8_ws_size = 0;
  char *ensure_w8a8(size_t aq_bytes);
  void *ensure_scratch(size_t n);
  void ensure_gemm(size_t xn_floats);
  void *ensure_pinned(size_t n);
  void ensure_attn(size_t work_floats, size_t cnt_words = 0);
};

// A pending asynchronous submission: an event recorded on a stream after the
// work (shim_run_*_start / shim_run_wait, xrt_shim.h:47-54).  For a resident
// decode dispatch, `res` is checked once the event has completed.
struct xe_resident;
struct xe_run {
  int ordinal = 0;
  hipEvent_t ev = nullptr;
  xe_resident *res = nullptr;
  bool done = false;
};

namespace xe {

// Completion work of a resident dispatch (its status word; decoder.hip).
void resident_done(xe_resident *r);

// ---------------------------------------------------------------------------
// Kernel launch surfaces (implemented in gemv.hip / attn.hip)
// ---------------------------------------------------------------------------

enum Act { ACT_NONE = 0, ACT_RELU = 1, ACT_GELU_ERF = 2, ACT_GEGLU_TANH = 3 };

// One fused norm + GEMV launch.  y[b, m'] = epilogue(W . prologue(x)[b]).
struct GemvLaunch {
  // weights
  int wdtype = XE_I8;
  const void *w = nullptr;
  const float *scale = nullptr;
  const uint8_t *exps = nullptr;
  const float *bias = nullptr;
  int m = 0, k = 0;
  // activations: x [batch, k] (x_dtype XE_F32 / XE_BF16), row stride ldx
  const void *x = nullptr;
  int x_dtype = XE_F32;
  int ldx = 0;
  int batch = 1;
  // prologue: t = x (+ post(sub)); res_out <- t (block 0); h = norm(t)
  const float *sub = nullptr;      // optional sublayer output [batch, k]
  const float *post_w = nullptr;   // optional Gemma (1+w) RMSNorm on sub
  float *res_out = nullptr;        // optional: updated residual [batch, k]
  int norm = XE_NORM_NONE;
  const float *gamma = nullptr;
  const float *beta = nullptr;
  float eps = 1e-5f;
  // epilogue
  int act = ACT_NONE;              // GEGLU pairs rows (2r gate, 2r+1 up)
  float out_scale = 1.0f;          // multiplies (acc*scale + bias)
  float *y = nullptr;              // [batch, ldy]
  int ldy = 0;
};

void launch_gemv(const GemvLaunch &p, hipStream_t s);
// More than 8 rows: the MFMA GEMM (gemm.hip), after a prologue kernel into xn
// [batch, k] when the launch has a norm or residual prologue.  fp32 x only.
// ws / cnt: split-K workspace (gemm_op_ws_floats() floats) and per-tile
// arrival counters (gemm_op_cnt_words(), zeroed once; they re-arm).
void launch_gemm_op(const GemvLaunch &L, float *xn, float *ws, unsigned *cnt, hipStream_t s);
// Whether a projection of `batch` rows over an m x k weight runs on the MFMA
// GEMM (gemm.hip) instead of the GEMV.
bool gemm_preferred(int m, int k, int batch);
size_t gemm_op_ws_floats();
size_t gemm_op_cnt_words();
// Output of an int8 x int8 -> i32 product: the raw accumulator (acc set), or
// the W8A8 dequant of dequant_epi (rust/npu-asr/src/ctx2.rs:1386-1435):
// v = (acc * scale_a) * ws[c]; EPI_BIAS adds bias[c]; EPI_SILU_BIAS gives
// z * fast_sigmoid(z) of z = v + bias[c] (ctx2.rs:1338-1348).
enum Epi { EPI_NONE = 0, EPI_BIAS = 1, EPI_SILU_BIAS = 2 };
struct W8a8Epi {
  int32_t *acc = nullptr;          // [batch, m] raw, or null
  float *y = nullptr;              // [batch, m] dequantised
  const float *scale_a = nullptr;  // device scalar
  const float *ws = nullptr;       // [m] weight scales
  const float *bias = nullptr;     // [m]
  int epi = EPI_NONE;
};

// fast_exp_nonpos (rust/npu-asr-host/src/lib.rs:38-55): 2^floor + a degree-5
// polynomial of 2^frac, evaluated in the reference's order (no contraction).
__device__ __forceinline__ float fast_exp_nonpos(float x) {
  x = x < -87.0f ? -87.0f : x;
  const float y = x * 1.442695040888963f;
  const float yf = floorf(y);
  const float f = y - yf;
  const float p = 1.0f + f * (0.6931471805599453f +
                              f * (0.2402265069591007f +
                                   f * (0.05550410866482158f +
                                        f * (0.009618129107628477f + f * 0.0013333558146428443f))));
  const uint32_t e = static_cast<uint32_t>(static_cast<int>(yf) + 127);
  return p * __uint_as_float(e << 23);
}

__device__ __forceinline__ float fast_sigmoid(float x) {
  if (x >= 0.0f) return 1.0f / (1.0f + fast_exp_nonpos(-x));
  const float e = fast_exp_nonpos(x);
  return e / (1.0f + e);
}

__device__ __forceinline__ void w8a8_store(const W8a8Epi &e, int b, int r, int m, int32_t a) {
  const size_t o = static_cast<size_t>(b) * m + r;
  if (e.acc) {
    e.acc[o] = a;
    return;
  }
  float v = static_cast<float>(a) * e.scale_a[0] * e.ws[r];
  if (e.epi == EPI_BIAS) {
    v = v + e.bias[r];
  } else if (e.epi == EPI_SILU_BIAS) {
    const float z = v + e.bias[r];
    v = z * fast_sigmoid(z);
  }
  e.y[o] = v;
}

// int8 activations x int8 weights -> int32 (exact), with the output stage
// above.  <= 8 rows: an sdot4 GEMV; more (up to the reference's Mp = 512):
// launch_w8a8_mfma.
void launch_gemv_i8act(const int8_t *q, const int8_t *xq, int m, int k, int batch,
                       const W8a8Epi &e, hipStream_t s);
void launch_w8a8_mfma(const int8_t *wq, const int8_t *aq, int m, int k, int batch, const W8a8Epi &e,
                      hipStream_t s);
// Dynamic per-tensor activation quant (quant_scale + quant_i8, ctx2.rs:
// 1352-1377): partial maxima (w8a8_partial_floats() floats), then aq and the
// device scalar scale_out.
void launch_w8a8_quant(const float *a, size_t n, float *partial, int8_t *aq, float *scale_out,
                       hipStream_t s);
size_t w8a8_partial_floats();

struct AttnLaunch {
  // q fp32 [batch, q_stride] with the hq heads at q_off (head h at h*hd)
  const float *q = nullptr;
  int q_stride = 0;
  // KV cache bf16 [batch, hkv, max_ctx, hd] (kv_batch_stride 0 = shared)
  uint16_t *kc = nullptr;
  uint16_t *vc = nullptr;
  size_t kv_batch_stride = 0;  // elements between streams (0 = shared cache)
  int max_ctx = 0;
  int batch = 1, hq = 1, hkv = 1, hd = 64;
  float scale = 1.0f;
  // lengths: lens[b] if non-null, else (pos[b] + 1), else fixed_len
  const int32_t *lens = nullptr;
  const int32_t *pos = nullptr;
  int fixed_len = 0;
  // optional append of the new token's k/v (fp32 [batch, kv_stride]) at pos
  const float *k_new = nullptr;
  const float *v_new = nullptr;
  int kv_new_stride = 0;
  // optional Gemma per-head RMSNorm (1+w) + RoPE on q and the new k
  const float *q_norm_w = nullptr;
  const float *k_norm_w = nullptr;
  float norm_eps = 1e-6f;
  const float *rope_cos = nullptr;  // [max_ctx, hd/2]
  const float *rope_sin = nullptr;
  int div_norm = 0;                 // p = e / sum (OPT) instead of e * (1/sum)
  // output fp32 [batch, out_stride], head h at h*hd
  float *out = nullptr;
  int out_stride = 0;
  // workspace for the split partials
  float *work = nullptr;
  // arrival counters [batch * hkv], zero between launches: the split kernel
  // merges its partials in place (no merge launch); null: a merge follows
  unsigned *cnt = nullptr;
  int max_splits = 0;
  // int8 K / V instead of bf16 (kc / vc then hold int8 [batch, hkv, max_ctx,
  // hd]; no append): per-channel scales [hkv * hd], or null
  const float *k_scale = nullptr;
  const float *v_scale = nullptr;
};

size_t attn_work_floats(int batch, int hq, int hd, int max_splits);
// Device address (resolved once per device) and capacity in floats of the
// static split-partial workspace used by xe_attn_decode_dev_static.
void *attn_static_scratch(int ordinal);
size_t attn_static_floats();
void launch_attn(const AttnLaunch &p, hipStream_t s);

// ---------------------------------------------------------------------------
// Address-space views.  A pointer read from a descriptor in memory (rather
// than a kernel argument) is generic to the compiler, which then emits flat
// instructions: they count against both the vector-memory and the LDS wait
// counters, so every LDS wait would also wait for the weight stream.  These
// casts give global (1) and LDS (3) instructions.
// ---------------------------------------------------------------------------
#define XE_GLOBAL __attribute__((address_space(1)))
#define XE_LDS __attribute__((address_space(3)))
// Constant (4): read-only for the kernel's lifetime.  Loads through it at a
// uniform address become scalar loads, so descriptor fields (loop bounds,
// pointers) are known wave-uniform and branches on them stay scalar.
#define XE_CONST __attribute__((address_space(4)))

template <typename T>
__device__ __forceinline__ const XE_GLOBAL T *gptr(const T *p) {
  return (const XE_GLOBAL T *)p;
}
template <typename T>
__device__ __forceinline__ XE_GLOBAL T *gptr_w(T *p) {
  return (XE_GLOBAL T *)p;
}
template <typename T>
__device__ __forceinline__ const XE_CONST T *cptr(const T *p) {
  return (const XE_CONST T *)p;
}
template <typename T>
__device__ __forceinline__ XE_LDS T *lptr(T *p) {
  return (XE_LDS T *)p;
}
template <typename T>
__device__ __forceinline__ const XE_LDS T *lptr(const T *p) {
  return (const XE_LDS T *)p;
}

}  // namespace xe
