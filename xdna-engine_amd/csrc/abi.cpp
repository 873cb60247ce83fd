// abi.cpp -- extern "C" boundary of libxdna_engine.so: device layer (the
// XRT-shim analog, rust/npu-xrt/shim/xrt_shim.h:16-113) and op layer (the
// CtxDecode analog, rust/npu-asr/src/ctx_decode.rs:142-694).
//
// Every entry point runs its body inside guard(): C++ exceptions and HIP
// errors become a NULL / -1 return plus a thread-local message, the
// convention of xrt_shim.cpp:42-56 and npu-capi/src/lib.rs:11-41.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <mutex>

#include "common.h"
#include "quant.h"

namespace xe {

static thread_local std::string g_err;

void set_error(const std::string &msg) { g_err = msg; }

void fail(const std::string &msg) { throw Error(msg); }

void hip_check(hipError_t e, const char *what, const char *file, int line) {
  if (e != hipSuccess) {
    char buf[512];
    snprintf(buf, sizeof(buf), "%s failed: %s (%s:%d)", what, hipGetErrorString(e), file, line);
    throw Error(buf);
  }
}

DeviceGuard::DeviceGuard(int ordinal) {
  XE_HIP(hipGetDevice(&prev));
  if (prev != ordinal) XE_HIP(hipSetDevice(ordinal));
}
DeviceGuard::~DeviceGuard() {
  int cur = -1;
  if (hipGetDevice(&cur) == hipSuccess && prev >= 0 && cur != prev) (void)hipSetDevice(prev);
}

template <typename F>
static auto guard(F &&f, decltype(f()) on_error) -> decltype(f()) {
  try {
    g_err.clear();
    return f();
  } catch (const std::exception &e) {
    g_err = e.what();
  } catch (...) {
    g_err = "unknown C++ exception";
  }
  return on_error;
}

}  // namespace xe

using namespace xe;

// ---------------------------------------------------------------------------
// ctx staging helpers
// ---------------------------------------------------------------------------
void *xe_ctx::ensure_scratch(size_t n) {
  if (n > scratch_size) {
    if (scratch) XE_HIP(hipFree(scratch));
    scratch = nullptr;
    scratch_size = 0;
    XE_HIP(hipMalloc(&scratch, n));
    scratch_size = n;
  }
  return scratch;
}

void *xe_ctx::ensure_pinned(size_t n) {
  if (n > host_pinned_size) {
    if (host_pinned) XE_HIP(hipHostFree(host_pinned));
    host_pinned = nullptr;
    host_pinned_size = 0;
    XE_HIP(hipHostMalloc(&host_pinned, n, hipHostMallocDefault));
    host_pinned_size = n;
  }
  return host_pinned;
}

void xe_ctx::ensure_attn(size_t work_floats, size_t cnt_words) {
  if (work_floats > attn_work_floats) {
    if (attn_work) XE_HIP(hipFree(attn_work));
    attn_work = nullptr;
    attn_work_floats = 0;
    XE_HIP(hipMalloc(&attn_work, work_floats * sizeof(float)));
    attn_work_floats = work_floats;
  }
  if (cnt_words > attn_cnt_words) {
    if (attn_cnt) XE_HIP(hipFree(attn_cnt));
    attn_cnt = nullptr;
    attn_cnt_words = 0;
    XE_HIP(hipMalloc(&attn_cnt, cnt_words * sizeof(unsigned)));
    XE_HIP(hipMemsetAsync(attn_cnt, 0, cnt_words * sizeof(unsigned), dev->stream));
    attn_cnt_words = cnt_words;
  }
}

// Layout: [0, 256) partial maxima (w8a8_partial_floats() <= 64 floats),
// [256, 512) scale_a, then the int8 activations.
char *xe_ctx::ensure_w8a8(size_t aq_bytes) {
  const size_t n = 512 + aq_bytes;
  if (n > w8a8_ws_size) {
    if (w8a8_ws) XE_HIP(hipFree(w8a8_ws));
    w8a8_ws = nullptr;
    w8a8_ws_size = 0;
    XE_HIP(hipMalloc(&w8a8_ws, n));
    w8a8_ws_size = n;
  }
  return w8a8_ws;
}

void xe_ctx::ensure_gemm(size_t xn_floats) {
  if (!gemm_ws) {
    XE_HIP(hipMalloc(&gemm_ws, gemm_op_ws_floats() * sizeof(float)));
    XE_HIP(hipMalloc(&gemm_cnt, gemm_op_cnt_words() * sizeof(unsigned)));
    XE_HIP(hipMemsetAsync(gemm_cnt, 0, gemm_op_cnt_words() * sizeof(unsigned), dev->stream));
  }
  if (xn_floats > gemm_xn_floats) {
    if (gemm_xn) XE_HIP(hipFree(gemm_xn));
    gemm_xn = nullptr;
    gemm_xn_floats = 0;
    XE_HIP(hipMalloc(&gemm_xn, xn_floats * sizeof(float)));
    gemm_xn_floats = xn_floats;
  }
}

namespace {

template <typename T>
T *dev_upload(const T *src, size_t n, hipStream_t s) {
  T *d = nullptr;
  XE_HIP(hipMalloc(reinterpret_cast<void **>(&d), n * sizeof(T)));
  if (src) {
    XE_HIP(hipMemcpyAsync(d, src, n * sizeof(T), hipMemcpyHostToDevice, s));
    XE_HIP(hipStreamSynchronize(s));
  }
  return d;
}

// The matrix, scales, exponents and bias belong to the weight unless it is a
// view (xe_register_weight_view); a pre-norm's gamma / beta always do.
void free_weight(xe_weight *w) {
  if (!w) return;
  if (w->owns) {
    (void)hipFree(w->w);
    (void)hipFree(w->scale);
    (void)hipFree(w->exps);
    (void)hipFree(w->bias);
  }
  (void)hipFree(w->gamma);
  (void)hipFree(w->beta);
  delete w;
}

xe_weight *new_weight(xe_ctx *ctx, int wdtype, int m, int k) {
  XE_REQUIRE(ctx && ctx->dev, "null ctx");
  XE_REQUIRE(m > 0 && k > 0, "weight shape must be positive");
  XE_REQUIRE(k % 16 == 0, "weight K must be a multiple of 16");
  XE_REQUIRE(wdtype == XE_I8 || wdtype == XE_BF16 || wdtype == XE_BFP16 || wdtype == XE_I4,
             "unknown weight dtype");
  auto *w = new xe_weight;
  w->ctx = ctx;
  w->wdtype = wdtype;
  w->m = m;
  w->k = k;
  return w;
}

// Row-major [m,k] fp32 from either layout.
std::vector<float> to_mk(const float *w, int m, int k, int layout) {
  std::vector<float> out(static_cast<size_t>(m) * k);
  if (layout == XE_LAYOUT_MK) {
    std::memcpy(out.data(), w, out.size() * sizeof(float));
  } else {
    XE_REQUIRE(layout == XE_LAYOUT_KN, "unknown weight layout");
    for (int r = 0; r < k; r++)
      for (int c = 0; c < m; c++) out[static_cast<size_t>(c) * k + r] = w[static_cast<size_t>(r) * m + c];
  }
  return out;
}

void fill_weight_from_f32(xe_weight *wt, const float *w_mk, const float *bias) {
  const int m = wt->m, k = wt->k;
  hipStream_t s = wt->ctx->dev->stream;
  const size_t n = static_cast<size_t>(m) * k;
  if (wt->wdtype == XE_I8) {
    std::vector<int8_t> q(n);
    std::vector<float> sc(m);
    quant_rows_i8(w_mk, m, k, q.data(), sc.data());
    wt->w = dev_upload(q.data(), n, s);
    wt->scale = dev_upload(sc.data(), m, s);
  } else if (wt->wdtype == XE_I4) {
    std::vector<uint8_t> q(n / 2);
    std::vector<float> sc(m);
    quant_rows_i4(w_mk, m, k, q.data(), sc.data());
    wt->w = dev_upload(q.data(), n / 2, s);
    wt->scale = dev_upload(sc.data(), m, s);
  } else if (wt->wdtype == XE_BF16) {
    std::vector<uint16_t> b(n);
    for (size_t i = 0; i < n; i++) b[i] = f32_to_bf16_bits(w_mk[i]);
    wt->w = dev_upload(b.data(), n, s);
  } else {
    std::vector<int8_t> mant(n);
    std::vector<uint8_t> ex(n / 8);
    bfp16_encode(w_mk, m, k, mant.data(), ex.data());
    wt->w = dev_upload(mant.data(), n, s);
    wt->exps = dev_upload(ex.data(), n / 8, s);
  }
  if (bias) wt->bias = dev_upload(bias, m, s);
}

void set_norm(xe_weight *w, int norm, const float *gamma, const float *beta, float eps) {
  XE_REQUIRE(norm >= XE_NORM_NONE && norm <= XE_NORM_RMS1P, "unknown norm kind");
  hipStream_t s = w->ctx->dev->stream;
  (void)hipFree(w->gamma);
  (void)hipFree(w->beta);
  w->gamma = w->beta = nullptr;
  w->norm = norm;
  w->eps = eps;
  if (norm == XE_NORM_NONE) return;
  XE_REQUIRE(gamma, "norm needs gamma");
  w->gamma = dev_upload(gamma, w->k, s);
  if (norm == XE_NORM_LN) {
    XE_REQUIRE(beta, "LayerNorm needs beta");
    w->beta = dev_upload(beta, w->k, s);
  }
}

GemvLaunch gemv_args(const xe_weight *w, const void *x, int x_dtype, int batch, float *y) {
  GemvLaunch g;
  g.wdtype = w->wdtype;
  g.w = w->w;
  g.scale = w->scale;
  g.exps = w->exps;
  g.bias = w->bias;
  g.m = w->m;
  g.k = w->k;
  g.x = x;
  g.x_dtype = x_dtype;
  g.ldx = w->k;
  g.batch = batch;
  g.norm = w->norm;
  g.gamma = w->gamma;
  g.beta = w->beta;
  g.eps = w->eps;
  g.y = y;
  g.ldy = w->m;
  return g;
}

// Up to 8 rows: the GEMV kernels; 9..kMaxOpBatch: the MFMA GEMM (fp32 x).
constexpr int kMaxOpBatch = 512;  // the reference's largest batched tile (Mp <= 512, ctx2.rs)

void launch_linear(xe_ctx *ctx, const xe_weight *w, const void *x, int x_dtype, int batch,
                   float *y, hipStream_t s) {
  if (!gemm_preferred(w->m, w->k, batch)) {
    launch_gemv(gemv_args(w, x, x_dtype, batch, y), s);
  } else {
    // the prologue (norm, or bf16 x to fp32) writes batch x k floats
    ctx->ensure_gemm(w->norm != XE_NORM_NONE || x_dtype == XE_BF16 ? static_cast<size_t>(batch) * w->k : 0);
    launch_gemm_op(gemv_args(w, x, x_dtype, batch, y), ctx->gemm_xn, ctx->gemm_ws, ctx->gemm_cnt, s);
  }
  ctx->dispatches++;
}

// int8 x int8 -> i32 with an output stage: the sdot4 GEMV up to 8 rows, the
// int8 MFMA GEMM beyond.
void launch_i8act(xe_ctx *ctx, const xe_weight *w, const int8_t *xq_dev, int batch, const W8a8Epi &e,
                  hipStream_t s) {
  if (batch <= 8)
    launch_gemv_i8act(static_cast<const int8_t *>(w->w), xq_dev, w->m, w->k, batch, e, s);
  else
    launch_w8a8_mfma(static_cast<const int8_t *>(w->w), xq_dev, w->m, w->k, batch, e, s);
  ctx->dispatches++;
}

// forward_view_int8 on the device: quant (two kernels), product + dequant.
void run_w8a8(xe_ctx *ctx, const xe_weight *w, const float *x_dev, int batch, int epi, float *y_dev,
              float *scale_a_dev, hipStream_t s) {
  XE_REQUIRE(w->wdtype == XE_I8, "xe_w8a8_linear needs an XE_I8 weight");
  XE_REQUIRE(batch >= 1 && batch <= kMaxOpBatch, "batch must be 1..512");
  XE_REQUIRE(epi == XE_EPI_NONE || epi == XE_EPI_BIAS || epi == XE_EPI_SILU_BIAS, "unknown epilogue");
  XE_REQUIRE(epi == XE_EPI_NONE || w->bias, "a bias epilogue needs a weight with a bias");
  const size_t n = static_cast<size_t>(batch) * w->k;
  char *ws = ctx->ensure_w8a8(n);
  float *partial = reinterpret_cast<float *>(ws);
  float *sa = scale_a_dev ? scale_a_dev : reinterpret_cast<float *>(ws + 256);
  int8_t *aq = reinterpret_cast<int8_t *>(ws + 512);
  launch_w8a8_quant(x_dev, n, partial, aq, sa, s);
  ctx->dispatches += 2;
  W8a8Epi e;
  e.y = y_dev;
  e.scale_a = sa;
  e.ws = w->scale;
  e.bias = w->bias;
  e.epi = epi;
  launch_i8act(ctx, w, aq, batch, e, s);
}

int run_gemv_host(xe_ctx *ctx, const xe_weight *w, const void *x, int x_dtype, int batch,
                  float *y) {
  XE_REQUIRE(ctx && w && x && y, "null argument");
  XE_REQUIRE(x_dtype == XE_F32 || x_dtype == XE_BF16, "x dtype must be XE_F32 or XE_BF16");
  XE_REQUIRE(batch >= 1 && batch <= kMaxOpBatch, "gemv batch must be 1..512");
  DeviceGuard dg(ctx->dev->ordinal);
  hipStream_t s = ctx->dev->stream;
  // more than 8 rows run on the GEMM, which reads fp32: widen bf16 here
  std::vector<float> widened;
  if (batch > 8 && x_dtype == XE_BF16) {
    const uint16_t *xb = static_cast<const uint16_t *>(x);
    widened.resize(static_cast<size_t>(batch) * w->k);
    for (size_t i = 0; i < widened.size(); i++) {
      const uint32_t u = static_cast<uint32_t>(xb[i]) << 16;
      std::memcpy(&widened[i], &u, 4);
    }
    x = widened.data();
    x_dtype = XE_F32;
  }
  const size_t xbytes = static_cast<size_t>(batch) * w->k * (x_dtype == XE_F32 ? 4 : 2);
  const size_t ybytes = static_cast<size_t>(batch) * w->m * 4;
  char *d = static_cast<char *>(ctx->ensure_scratch(xbytes + ybytes + 256));
  void *dx = d;
  float *dy = reinterpret_cast<float *>(d + ((xbytes + 255) / 256) * 256);
  XE_HIP(hipMemcpyAsync(dx, x, xbytes, hipMemcpyHostToDevice, s));
  launch_linear(ctx, w, dx, x_dtype, batch, dy, s);
  XE_HIP(hipMemcpyAsync(y, dy, ybytes, hipMemcpyDeviceToHost, s));
  XE_HIP(hipStreamSynchronize(s));
  return 0;
}

}  // namespace

// ===========================================================================
// extern "C"
// ===========================================================================
extern "C" {

const char *xe_last_error(void) { return g_err.c_str(); }
int xe_abi_version(void) { return XE_ABI_VERSION; }

int xe_device_count(void) {
  return guard([&]() -> int {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
  }, -1);
}

xe_device *xe_device_open(int ordinal) {
  return guard([&]() -> xe_device * {
    int n = 0;
    XE_HIP(hipGetDeviceCount(&n));
    XE_REQUIRE(ordinal >= 0 && ordinal < n, "device ordinal out of range");
    XE_HIP(hipSetDevice(ordinal));
    auto *d = new xe_device;
    d->ordinal = ordinal;
    hipDeviceProp_t prop;
    XE_HIP(hipGetDeviceProperties(&prop, ordinal));
    d->arch = prop.gcnArchName;
    d->num_cus = prop.multiProcessorCount;
    d->max_lds = prop.sharedMemPerBlock;
    // default priority: other priorities have hung on this hardware pool
    XE_HIP(hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking));
    // the static attention workspace's device address, once per device
    (void)attn_static_scratch(ordinal);
    return d;
  }, nullptr);
}

void xe_device_close(xe_device *dev) {
  guard([&]() -> int {
    if (!dev) return 0;
    DeviceGuard dg(dev->ordinal);
    (void)hipStreamSynchronize(dev->stream);
    (void)hipStreamDestroy(dev->stream);
    delete dev;
    return 0;
  }, -1);
}

int xe_device_synchronize(xe_device *dev) {
  return guard([&]() -> int {
    XE_REQUIRE(dev, "null device");
    DeviceGuard dg(dev->ordinal);
    XE_HIP(hipStreamSynchronize(dev->stream));
    return 0;
  }, -1);
}

int xe_device_name(xe_device *dev, char *buf, int cap) {
  return guard([&]() -> int {
    XE_REQUIRE(dev && buf && cap > 0, "null argument");
    int n = snprintf(buf, cap, "%s", dev->arch.c_str());
    return n < cap ? n : cap - 1;
  }, -1);
}

xe_buf *xe_buf_alloc(xe_device *dev, size_t nbytes) {
  return guard([&]() -> xe_buf * {
    XE_REQUIRE(dev, "null device");
    XE_REQUIRE(nbytes > 0, "zero-size buffer");
    DeviceGuard dg(dev->ordinal);
    auto *b = new xe_buf;
    b->dev = dev;
    b->size = nbytes;
    if (hipMalloc(&b->ptr, nbytes) != hipSuccess) {
      delete b;
      fail("hipMalloc of " + std::to_string(nbytes) + " bytes failed");
    }
    return b;
  }, nullptr);
}

void xe_buf_free(xe_buf *buf) {
  guard([&]() -> int {
    if (!buf) return 0;
    DeviceGuard dg(buf->dev->ordinal);
    (void)hipStreamSynchronize(buf->dev->stream);
    (void)hipFree(buf->ptr);
    delete buf;
    return 0;
  }, -1);
}

int xe_buf_write(xe_buf *buf, const void *src, size_t nbytes, size_t offset) {
  return guard([&]() -> int {
    XE_REQUIRE(buf && src, "null argument");
    XE_REQUIRE(offset <= buf->size && nbytes <= buf->size - offset, "write out of bounds");
    DeviceGuard dg(buf->dev->ordinal);
    XE_HIP(hipMemcpyAsync(static_cast<char *>(buf->ptr) + offset, src, nbytes,
                          hipMemcpyHostToDevice, buf->dev->stream));
    XE_HIP(hipStreamSynchronize(buf->dev->stream));
    return 0;
  }, -1);
}

int xe_buf_read(xe_buf *buf, void *dst, size_t nbytes, size_t offset) {
  return guard([&]() -> int {
    XE_REQUIRE(buf && dst, "null argument");
    XE_REQUIRE(offset <= buf->size && nbytes <= buf->size - offset, "read out of bounds");
    DeviceGuard dg(buf->dev->ordinal);
    XE_HIP(hipMemcpyAsync(dst, static_cast<char *>(buf->ptr) + offset, nbytes,
                          hipMemcpyDeviceToHost, buf->dev->stream));
    XE_HIP(hipStreamSynchronize(buf->dev->stream));
    return 0;
  }, -1);
}

void *xe_buf_device_ptr(xe_buf *buf) { return buf ? buf->ptr : nullptr; }
size_t xe_buf_size(xe_buf *buf) { return buf ? buf->size : 0; }

// ---- op layer ------------------------------------------------------------

xe_ctx *xe_ctx_create(xe_device *dev) {
  return guard([&]() -> xe_ctx * {
    XE_REQUIRE(dev, "null device");
    auto *c = new xe_ctx;
    c->dev = dev;
    return c;
  }, nullptr);
}

void xe_ctx_destroy(xe_ctx *ctx) {
  guard([&]() -> int {
    if (!ctx) return 0;
    DeviceGuard dg(ctx->dev->ordinal);
    (void)hipStreamSynchronize(ctx->dev->stream);
    if (ctx->scratch) (void)hipFree(ctx->scratch);
    if (ctx->host_pinned) (void)hipHostFree(ctx->host_pinned);
    if (ctx->attn_work) (void)hipFree(ctx->attn_work);
    if (ctx->attn_cnt) (void)hipFree(ctx->attn_cnt);
    if (ctx->gemm_ws) (void)hipFree(ctx->gemm_ws);
    if (ctx->gemm_cnt) (void)hipFree(ctx->gemm_cnt);
    if (ctx->gemm_xn) (void)hipFree(ctx->gemm_xn);
    if (ctx->w8a8_ws) (void)hipFree(ctx->w8a8_ws);
    delete ctx;
    return 0;
  }, -1);
}

uint64_t xe_ctx_dispatches(xe_ctx *ctx) { return ctx ? ctx->dispatches : 0; }
void xe_ctx_reset_dispatches(xe_ctx *ctx) {
  if (ctx) ctx->dispatches = 0;
}

xe_run *xe_ctx_record(xe_ctx *ctx) {
  return guard([&]() -> xe_run * {
    XE_REQUIRE(ctx, "null ctx");
    DeviceGuard dg(ctx->dev->ordinal);
    auto *r = new xe_run;
    r->ordinal = ctx->dev->ordinal;
    const hipError_t e = hipEventCreateWithFlags(&r->ev, hipEventDisableTiming);
    if (e != hipSuccess) {
      delete r;
      XE_HIP(e);
    }
    const hipError_t e2 = hipEventRecord(r->ev, ctx->dev->stream);
    if (e2 != hipSuccess) {
      (void)hipEventDestroy(r->ev);
      delete r;
      XE_HIP(e2);
    }
    return r;
  }, nullptr);
}

int xe_run_query(xe_run *run) {
  return guard([&]() -> int {
    XE_REQUIRE(run, "null run");
    if (run->done) return 1;
    DeviceGuard dg(run->ordinal);
    const hipError_t e = hipEventQuery(run->ev);
    if (e == hipErrorNotReady) return 0;
    XE_HIP(e);
    run->done = true;
    if (run->res) resident_done(run->res);
    return 1;
  }, -1);
}

int xe_run_wait(xe_run *run) {
  return guard([&]() -> int {
    XE_REQUIRE(run, "null run");
    if (run->done) return 0;
    DeviceGuard dg(run->ordinal);
    XE_HIP(hipEventSynchronize(run->ev));
    run->done = true;
    if (run->res) resident_done(run->res);
    return 0;
  }, -1);
}

void xe_run_free(xe_run *run) {
  guard([&]() -> int {
    if (!run) return 0;
    DeviceGuard dg(run->ordinal);
    (void)hipEventSynchronize(run->ev);  // a handle freed early still lets the work finish
    (void)hipEventDestroy(run->ev);
    xe_resident *res = run->done ? nullptr : run->res;
    delete run;
    if (res) resident_done(res);  // its status is still checked (an error is reported here)
    return 0;
  }, -1);
}

int xe_ctx_synchronize(xe_ctx *ctx) {
  return guard([&]() -> int {
    XE_REQUIRE(ctx, "null ctx");
    DeviceGuard dg(ctx->dev->ordinal);
    XE_HIP(hipStreamSynchronize(ctx->dev->stream));
    return 0;
  }, -1);
}

xe_weight *xe_register_weight(xe_ctx *ctx, int wdtype, int m, int k, const float *w,
                              int layout, const float *bias) {
  return guard([&]() -> xe_weight * {
    XE_REQUIRE(w, "null weight");
    DeviceGuard dg(ctx ? ctx->dev->ordinal : 0);
    xe_weight *wt = new_weight(ctx, wdtype, m, k);
    try {
      std::vector<float> mk = to_mk(w, m, k, layout);
      fill_weight_from_f32(wt, mk.data(), bias);
    } catch (...) {
      free_weight(wt);
      throw;
    }
    return wt;
  }, nullptr);
}

xe_weight *xe_register_weight_q8(xe_ctx *ctx, int m, int k, const int8_t *q, const float *scales,
                                 const float *bias) {
  return guard([&]() -> xe_weight * {
    XE_REQUIRE(q && scales, "null weight or scales");
    DeviceGuard dg(ctx ? ctx->dev->ordinal : 0);
    xe_weight *wt = new_weight(ctx, XE_I8, m, k);
    hipStream_t s = ctx->dev->stream;
    wt->w = dev_upload(q, static_cast<size_t>(m) * k, s);
    wt->scale = dev_upload(scales, m, s);
    if (bias) wt->bias = dev_upload(bias, m, s);
    return wt;
  }, nullptr);
}

xe_weight *xe_register_weight_q8_rule(xe_ctx *ctx, int m, int k, const float *w, int layout,
                                      const float *bias, int rule) {
  return guard([&]() -> xe_weight * {
    XE_REQUIRE(w, "null weight");
    XE_REQUIRE(rule == XE_Q8_LIN || rule == XE_Q8_ELF, "unknown int8 quantisation rule");
    DeviceGuard dg(ctx ? ctx->dev->ordinal : 0);
    xe_weight *wt = new_weight(ctx, XE_I8, m, k);
    try {
      std::vector<float> mk = to_mk(w, m, k, layout);
      if (rule == XE_Q8_LIN) {
        fill_weight_from_f32(wt, mk.data(), bias);
      } else {
        hipStream_t s = ctx->dev->stream;
        std::vector<int8_t> q(mk.size());
        std::vector<float> sc(m);
        quant_rows_i8_elf(mk.data(), m, k, q.data(), sc.data());
        wt->w = dev_upload(q.data(), q.size(), s);
        wt->scale = dev_upload(sc.data(), m, s);
        if (bias) wt->bias = dev_upload(bias, m, s);
      }
    } catch (...) {
      free_weight(wt);
      throw;
    }
    return wt;
  }, nullptr);
}

xe_weight *xe_register_weight_q4(xe_ctx *ctx, int m, int k, const uint8_t *packed, const float *scales,
                                 const float *bias) {
  return guard([&]() -> xe_weight * {
    XE_REQUIRE(packed && scales, "null weight or scales");
    DeviceGuard dg(ctx ? ctx->dev->ordinal : 0);
    xe_weight *wt = new_weight(ctx, XE_I4, m, k);
    hipStream_t s = ctx->dev->stream;
    wt->w = dev_upload(packed, static_cast<size_t>(m) * k / 2, s);
    wt->scale = dev_upload(scales, m, s);
    if (bias) wt->bias = dev_upload(bias, m, s);
    return wt;
  }, nullptr);
}

xe_weight *xe_register_weight_q4_kn(xe_ctx *ctx, int m, int k, const uint8_t *packed_kn,
                                    const float *scales, const float *bias) {
  return guard([&]() -> xe_weight * {
    XE_REQUIRE(packed_kn && scales, "null weight or scales");
    XE_REQUIRE(m % 2 == 0, "int4 [K, N/2] layout needs an even N");
    DeviceGuard dg(ctx ? ctx->dev->ordinal : 0);
    xe_weight *wt = new_weight(ctx, XE_I4, m, k);
    // [k][m/2] (two output columns a byte) -> [m][k/2] (two k a byte)
    std::vector<uint8_t> mk(static_cast<size_t>(m) * k / 2, 0);
    for (int r = 0; r < k; r++)
      for (int c = 0; c < m; c++) {
        const uint8_t byte = packed_kn[static_cast<size_t>(r) * (m / 2) + c / 2];
        const uint8_t nib = (c & 1) ? static_cast<uint8_t>(byte >> 4) : static_cast<uint8_t>(byte & 0x0F);
        mk[static_cast<size_t>(c) * (k / 2) + r / 2] |= static_cast<uint8_t>((r & 1) ? nib << 4 : nib);
      }
    hipStream_t s = ctx->dev->stream;
    wt->w = dev_upload(mk.data(), mk.size(), s);
    wt->scale = dev_upload(scales, m, s);
    if (bias) wt->bias = dev_upload(bias, m, s);
    return wt;
  }, nullptr);
}

xe_weight *xe_register_weight_bfp16(xe_ctx *ctx, int m, int k, const int8_t *mant,
                                    const uint8_t *exps, const float *bias) {
  return guard([&]() -> xe_weight * {
    XE_REQUIRE(mant && exps, "null mantissas or exponents");
    DeviceGuard dg(ctx ? ctx->dev->ordinal : 0);
    xe_weight *wt = new_weight(ctx, XE_BFP16, m, k);
    hipStream_t s = ctx->dev->stream;
    wt->w = dev_upload(mant, static_cast<size_t>(m) * k, s);
    wt->exps = dev_upload(exps, static_cast<size_t>(m) * k / 8, s);
    if (bias) wt->bias = dev_upload(bias, m, s);
    return wt;
  }, nullptr);
}

xe_weight *xe_register_weight_bf16(xe_ctx *ctx, int m, int k, const uint16_t *bits,
                                   const float *bias) {
  return guard([&]() -> xe_weight * {
    XE_REQUIRE(bits, "null weight");
    DeviceGuard dg(ctx ? ctx->dev->ordinal : 0);
    xe_weight *wt = new_weight(ctx, XE_BF16, m, k);
    hipStream_t s = ctx->dev->stream;
    wt->w = dev_upload(bits, static_cast<size_t>(m) * k, s);
    if (bias) wt->bias = dev_upload(bias, m, s);
    return wt;
  }, nullptr);
}

xe_weight *xe_register_weight_view(xe_ctx *ctx, int wdtype, int m, int k, const void *w_dev,
                                   const float *scale_dev, const uint8_t *exps_dev,
                                   const float *bias_dev) {
  return guard([&]() -> xe_weight * {
    XE_REQUIRE(w_dev, "null weight pointer");
    XE_REQUIRE(wdtype == XE_I8 || wdtype == XE_BF16 || wdtype == XE_BFP16 || wdtype == XE_I4,
               "unknown weight dtype");
    XE_REQUIRE((wdtype != XE_I8 && wdtype != XE_I4) || scale_dev, "int8/int4 weight view needs scales");
    XE_REQUIRE(wdtype != XE_BFP16 || exps_dev, "bfp16 weight view needs exponents");
    DeviceGuard dg(ctx ? ctx->dev->ordinal : 0);
    xe_weight *wt = new_weight(ctx, wdtype, m, k);
    wt->owns = false;
    wt->w = const_cast<void *>(w_dev);
    wt->scale = const_cast<float *>(scale_dev);
    wt->exps = const_cast<uint8_t *>(exps_dev);
    wt->bias = const_cast<float *>(bias_dev);
    return wt;
  }, nullptr);
}

xe_weight *xe_register_fused(xe_ctx *ctx, int wdtype, int m, int k, const float *w, int layout,
                             int norm, const float *gamma, const float *beta, float eps,
                             const float *bias) {
  return guard([&]() -> xe_weight * {
    XE_REQUIRE(w, "null weight");
    DeviceGuard dg(ctx ? ctx->dev->ordinal : 0);
    xe_weight *wt = new_weight(ctx, wdtype, m, k);
    try {
      std::vector<float> mk = to_mk(w, m, k, layout);
      fill_weight_from_f32(wt, mk.data(), bias);
      set_norm(wt, norm, gamma, beta, eps);
    } catch (...) {
      free_weight(wt);
      throw;
    }
    return wt;
  }, nullptr);
}

int xe_weight_set_norm(xe_weight *w, int norm, const float *gamma, const float *beta, float eps) {
  return guard([&]() -> int {
    XE_REQUIRE(w, "null weight");
    DeviceGuard dg(w->ctx->dev->ordinal);
    set_norm(w, norm, gamma, beta, eps);
    return 0;
  }, -1);
}

void xe_weight_free(xe_weight *w) {
  guard([&]() -> int {
    if (!w) return 0;
    DeviceGuard dg(w->ctx->dev->ordinal);
    (void)hipStreamSynchronize(w->ctx->dev->stream);
    free_weight(w);
    return 0;
  }, -1);
}

int xe_weight_shape(const xe_weight *w, int *m, int *k, int *wdtype) {
  if (!w) {
    set_error("null weight");
    return -1;
  }
  if (m) *m = w->m;
  if (k) *k = w->k;
  if (wdtype) *wdtype = w->wdtype;
  return 0;
}

int xe_gemv(xe_ctx *ctx, const xe_weight *w, const void *x, int x_dtype, int batch, float *y) {
  return guard([&]() -> int {
    XE_REQUIRE(!w || w->norm == XE_NORM_NONE,
               "xe_gemv on a fused weight: use xe_fused_norm_gemv");
    return run_gemv_host(ctx, w, x, x_dtype, batch, y);
  }, -1);
}

int xe_fused_norm_gemv(xe_ctx *ctx, const xe_weight *w, const void *x, int x_dtype, int batch,
                       float *y) {
  return guard([&]() -> int { return run_gemv_host(ctx, w, x, x_dtype, batch, y); }, -1);
}

int xe_gemv_dev(xe_ctx *ctx, const xe_weight *w, const void *x_dev, int x_dtype, int batch,
                float *y_dev) {
  return guard([&]() -> int {
    XE_REQUIRE(ctx && w && x_dev && y_dev, "null argument");
    XE_REQUIRE(x_dtype == XE_F32 || x_dtype == XE_BF16, "x dtype must be XE_F32 or XE_BF16");
    XE_REQUIRE(batch >= 1 && batch <= kMaxOpBatch, "gemv batch must be 1..512");
    DeviceGuard dg(ctx->dev->ordinal);
    launch_linear(ctx, w, x_dev, x_dtype, batch, y_dev, ctx->dev->stream);
    return 0;
  }, -1);
}

int xe_gemv_i8act_dev(xe_ctx *ctx, const xe_weight *w, const int8_t *xq_dev, int batch,
                      int32_t *acc_dev) {
  return guard([&]() -> int {
    XE_REQUIRE(ctx && w && xq_dev && acc_dev, "null argument");
    XE_REQUIRE(w->wdtype == XE_I8, "xe_gemv_i8act needs an XE_I8 weight");
    XE_REQUIRE(batch >= 1 && batch <= kMaxOpBatch, "batch must be 1..512");
    DeviceGuard dg(ctx->dev->ordinal);
    W8a8Epi e;
    e.acc = acc_dev;
    launch_i8act(ctx, w, xq_dev, batch, e, ctx->dev->stream);
    return 0;
  }, -1);
}

int xe_gemv_i8act(xe_ctx *ctx, const xe_weight *w, const int8_t *xq, int batch, int32_t *acc) {
  return guard([&]() -> int {
    XE_REQUIRE(ctx && w && xq && acc, "null argument");
    XE_REQUIRE(w->wdtype == XE_I8, "xe_gemv_i8act needs an XE_I8 weight");
    XE_REQUIRE(batch >= 1 && batch <= kMaxOpBatch, "batch must be 1..512");
    DeviceGuard dg(ctx->dev->ordinal);
    hipStream_t s = ctx->dev->stream;
    const size_t xb = static_cast<size_t>(batch) * w->k;
    const size_t ab = static_cast<size_t>(batch) * w->m * 4;
    char *d = static_cast<char *>(ctx->ensure_scratch(xb + ab + 256));
    int32_t *da = reinterpret_cast<int32_t *>(d + ((xb + 255) / 256) * 256);
    XE_HIP(hipMemcpyAsync(d, xq, xb, hipMemcpyHostToDevice, s));
    W8a8Epi e;
    e.acc = da;
    launch_i8act(ctx, w, reinterpret_cast<int8_t *>(d), batch, e, s);
    XE_HIP(hipMemcpyAsync(acc, da, ab, hipMemcpyDeviceToHost, s));
    XE_HIP(hipStreamSynchronize(s));
    return 0;
  }, -1);
}

int xe_w8a8_linear_dev(xe_ctx *ctx, const xe_weight *w, const float *x_dev, int batch, int epi,
                       float *y_dev, float *scale_a_dev) {
  return guard([&]() -> int {
    XE_REQUIRE(ctx && w && x_dev && y_dev, "null argument");
    DeviceGuard dg(ctx->dev->ordinal);
    run_w8a8(ctx, w, x_dev, batch, epi, y_dev, scale_a_dev, ctx->dev->stream);
    return 0;
  }, -1);
}

int xe_w8a8_linear(xe_ctx *ctx, const xe_weight *w, const float *x, int batch, float *y,
                   float *scale_a_out) {
  return guard([&]() -> int {
    XE_REQUIRE(ctx && w && x && y, "null argument");
    XE_REQUIRE(batch >= 1 && batch <= kMaxOpBatch, "batch must be 1..512");
    DeviceGuard dg(ctx->dev->ordinal);
    hipStream_t s = ctx->dev->stream;
    // forward_view_int8 (ctx2.rs:771-830) with Epi::Bias when the op has a
    // bias, Epi::None otherwise; x in and y (and scale_a) out are the only
    // host transfers
    const size_t xb = static_cast<size_t>(batch) * w->k * 4;
    const size_t yb = static_cast<size_t>(batch) * w->m * 4;
    char *d = static_cast<char *>(ctx->ensure_scratch(xb + yb + 512));
    float *dx = reinterpret_cast<float *>(d);
    float *dy = reinterpret_cast<float *>(d + ((xb + 255) / 256) * 256);
    float *dsa = reinterpret_cast<float *>(d + ((xb + 255) / 256) * 256 + ((yb + 255) / 256) * 256);
    XE_HIP(hipMemcpyAsync(dx, x, xb, hipMemcpyHostToDevice, s));
    run_w8a8(ctx, w, dx, batch, w->bias ? XE_EPI_BIAS : XE_EPI_NONE, dy, dsa, s);
    XE_HIP(hipMemcpyAsync(y, dy, yb, hipMemcpyDeviceToHost, s));
    float sa = 0.f;
    XE_HIP(hipMemcpyAsync(&sa, dsa, 4, hipMemcpyDeviceToHost, s));
    XE_HIP(hipStreamSynchronize(s));
    if (scale_a_out) *scale_a_out = sa;
    return 0;
  }, -1);
}

// Splits per (stream, kv head): about XE_ATTN_WG_PER_CU (default 2)
// workgroups per CU in total, at most one per 64 cache rows and at most 64.
// With the merge inside the split kernel, 2 a CU against 4 (graph replays,
// config 3): GQA 4q/1kv x 256 b = 64 ctx 4096 52.3 / 58.3 us, b = 16 ctx
// 4096 33.0 / 47.1, b = 64 ctx 1024 26.2 / 37.2; ctx 32768 within 4 %.
static int attn_splits(const xe_ctx *ctx, int batch, int hkv, int max_ctx) {
  static const int per_cu = [] {
    const char *e = std::getenv("XE_ATTN_WG_PER_CU");
    return e && std::atoi(e) > 0 ? std::atoi(e) : 2;
  }();
  const int target = per_cu * ctx->dev->num_cus;
  int ms = target / (batch * hkv);
  const int cap = (max_ctx + 63) / 64;
  ms = ms < 1 ? 1 : ms;
  ms = ms > cap ? cap : ms;
  return ms > 64 ? 64 : ms;
}

// work: the split partials (attn_work_floats(batch, hq, hd, splits) floats);
// null = the ctx's own workspace, grown on demand, with the ctx's arrival
// counters: the split kernel merges in place (the last split block of a
// (stream, kv head) to arrive merges its partials, one launch).  A caller's
// workspace (the allocation-free entry point) takes the separate merge launch.
// XE_ATTN_MERGE=launch selects the merge launch for the ctx workspace too.
static bool attn_merge_in_place() {
  const char *e = std::getenv("XE_ATTN_MERGE");
  return !(e && std::string(e) == "launch");
}

static int attn_impl(xe_ctx *ctx, const float *q, const uint16_t *kc, const uint16_t *vc,
                     const int32_t *lens, int batch, int hq, int hkv, int hd, int max_ctx,
                     float scale, float *out, float *work = nullptr) {
  AttnLaunch a;
  a.q = q;
  a.kc = const_cast<uint16_t *>(kc);
  a.vc = const_cast<uint16_t *>(vc);
  a.kv_batch_stride = static_cast<size_t>(hkv) * max_ctx * hd;
  a.max_ctx = max_ctx;
  a.batch = batch;
  a.hq = hq;
  a.hkv = hkv;
  a.hd = hd;
  a.scale = scale;
  a.lens = lens;
  a.out = out;
  a.max_splits = attn_splits(ctx, batch, hkv, max_ctx);
  if (work) {
    a.work = work;
  } else {
    const bool in_place = attn_merge_in_place();
    ctx->ensure_attn(attn_work_floats(batch, hq, hd, a.max_splits),
                     in_place ? static_cast<size_t>(batch) * hkv : 0);
    a.work = ctx->attn_work;
    a.cnt = in_place ? ctx->attn_cnt : nullptr;
  }
  launch_attn(a, ctx->dev->stream);
  ctx->dispatches++;
  return 0;
}

int xe_attn_decode_dev(xe_ctx *ctx, const float *q_dev, const uint16_t *kc_dev,
                       const uint16_t *vc_dev, const int32_t *lens_dev, int batch, int hq, int hkv,
                       int hd, int max_ctx, float scale, float *out_dev) {
  return guard([&]() -> int {
    XE_REQUIRE(ctx && q_dev && kc_dev && vc_dev && lens_dev && out_dev, "null argument");
    XE_REQUIRE(batch > 0 && hq > 0 && hkv > 0 && hd > 0, "bad shape");
    DeviceGuard dg(ctx->dev->ordinal);
    return attn_impl(ctx, q_dev, kc_dev, vc_dev, lens_dev, batch, hq, hkv, hd, max_ctx, scale,
                     out_dev);
  }, -1);
}

int xe_attn_decode_dev_static(xe_ctx *ctx, const float *q_dev, const uint16_t *kc_dev,
                              const uint16_t *vc_dev, const int32_t *lens_dev, int batch, int hq,
                              int hkv, int hd, int max_ctx, float scale, float *out_dev) {
  return guard([&]() -> int {
    XE_REQUIRE(ctx && q_dev && kc_dev && vc_dev && lens_dev && out_dev, "null argument");
    XE_REQUIRE(batch > 0 && hq > 0 && hkv > 0 && hd > 0, "bad shape");
    DeviceGuard dg(ctx->dev->ordinal);
    const size_t need = attn_work_floats(batch, hq, hd, attn_splits(ctx, batch, hkv, max_ctx));
    XE_REQUIRE(need <= attn_static_floats(),
               "xe_attn_decode_dev_static: " + std::to_string(need) + " partial floats needed, the static "
               "workspace holds " + std::to_string(attn_static_floats()) +
               " (fewer streams or query heads per call)");
    float *work = static_cast<float *>(attn_static_scratch(ctx->dev->ordinal));
    return attn_impl(ctx, q_dev, kc_dev, vc_dev, lens_dev, batch, hq, hkv, hd, max_ctx, scale,
                     out_dev, work);
  }, -1);
}

int xe_attn_decode(xe_ctx *ctx, const float *q, const uint16_t *kc, const uint16_t *vc,
                   const int32_t *lens, int batch, int hq, int hkv, int hd, int max_ctx,
                   float scale, float *out) {
  return guard([&]() -> int {
    XE_REQUIRE(ctx && q && kc && vc && lens && out, "null argument");
    XE_REQUIRE(batch > 0 && hq > 0 && hkv > 0 && hd > 0 && max_ctx > 0, "bad shape");
    for (int b = 0; b < batch; b++)
      XE_REQUIRE(lens[b] >= 1 && lens[b] <= max_ctx, "lens[b] must be in [1, max_ctx]");
    DeviceGuard dg(ctx->dev->ordinal);
    hipStream_t s = ctx->dev->stream;
    const size_t qn = static_cast<size_t>(batch) * hq * hd;
    const size_t kvn = static_cast<size_t>(batch) * hkv * max_ctx * hd;
    float *dq = nullptr, *dout = nullptr;
    uint16_t *dk = nullptr, *dv = nullptr;
    int32_t *dl = nullptr;
    XE_HIP(hipMalloc(&dq, qn * 4));
    XE_HIP(hipMalloc(&dout, qn * 4));
    XE_HIP(hipMalloc(&dk, kvn * 2));
    XE_HIP(hipMalloc(&dv, kvn * 2));
    XE_HIP(hipMalloc(&dl, batch * 4));
    struct Free {
      void *p[5];
      ~Free() {
        for (void *x : p) (void)hipFree(x);
      }
    } fr{{dq, dout, dk, dv, dl}};
    XE_HIP(hipMemcpyAsync(dq, q, qn * 4, hipMemcpyHostToDevice, s));
    XE_HIP(hipMemcpyAsync(dk, kc, kvn * 2, hipMemcpyHostToDevice, s));
    XE_HIP(hipMemcpyAsync(dv, vc, kvn * 2, hipMemcpyHostToDevice, s));
    XE_HIP(hipMemcpyAsync(dl, lens, batch * 4, hipMemcpyHostToDevice, s));
    attn_impl(ctx, dq, dk, dv, dl, batch, hq, hkv, hd, max_ctx, scale, dout);
    XE_HIP(hipMemcpyAsync(out, dout, qn * 4, hipMemcpyDeviceToHost, s));
    XE_HIP(hipStreamSynchronize(s));
    return 0;
  }, -1);
}

}  // extern "C"

namespace {

// Device microseconds per repetition of `enqueue` (HIP events on the ctx
// stream around the repetitions).  XE_PROBE_EAGER: plain launches, so the
// time includes any host gaps between short kernels (a profiler's per-kernel
// trace then gives the kernel durations; graph launches under a kernel
// tracer have crashed in the HIP runtime on this image).  Otherwise the
// launches are captured once in a HIP graph and the graph is replayed.
template <typename F>
double time_eager(xe_ctx *ctx, int reps, F &&enqueue) {
  hipStream_t s = ctx->dev->stream;
  enqueue();  // warm-up
  hipEvent_t e0 = nullptr, e1 = nullptr;
  XE_HIP(hipEventCreate(&e0));
  const hipError_t ce = hipEventCreate(&e1);
  if (ce != hipSuccess) {
    (void)hipEventDestroy(e0);
    XE_HIP(ce);
  }
  double us = 0.0;
  try {
    XE_HIP(hipEventRecord(e0, s));
    for (int r = 0; r < reps; r++) enqueue();
    XE_HIP(hipEventRecord(e1, s));
    XE_HIP(hipEventSynchronize(e1));
    float ms = 0.f;
    XE_HIP(hipEventElapsedTime(&ms, e0, e1));
    us = 1000.0 * ms / reps;
  } catch (...) {
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    throw;
  }
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  return us;
}

template <typename F>
double time_captured(xe_ctx *ctx, int reps, int flags, F &&enqueue) {
  if (flags & XE_PROBE_EAGER) return time_eager(ctx, reps, enqueue);
  hipStream_t s = ctx->dev->stream;
  XE_HIP(hipStreamSynchronize(s));
  hipGraph_t g = nullptr;
  XE_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeRelaxed));
  try {
    enqueue();
  } catch (...) {
    hipGraph_t junk = nullptr;
    (void)hipStreamEndCapture(s, &junk);
    if (junk) (void)hipGraphDestroy(junk);
    throw;
  }
  XE_HIP(hipStreamEndCapture(s, &g));
  hipGraphExec_t ex = nullptr;
  const hipError_t ie = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  XE_HIP(ie);
  hipEvent_t e0 = nullptr, e1 = nullptr;
  double us = 0.0;
  try {
    XE_HIP(hipGraphLaunch(ex, s));  // warm-up replay
    XE_HIP(hipEventCreate(&e0));
    XE_HIP(hipEventCreate(&e1));
    XE_HIP(hipEventRecord(e0, s));
    for (int r = 0; r < reps; r++) XE_HIP(hipGraphLaunch(ex, s));
    XE_HIP(hipEventRecord(e1, s));
    XE_HIP(hipEventSynchronize(e1));
    float ms = 0.f;
    XE_HIP(hipEventElapsedTime(&ms, e0, e1));
    us = 1000.0 * ms / reps;
  } catch (...) {
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    (void)hipGraphExecDestroy(ex);
    throw;
  }
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  (void)hipGraphExecDestroy(ex);
  return us;
}

}  // namespace

extern "C" {

int xe_probe_gemv(xe_ctx *ctx, const xe_weight *const *ws, int n_weights, const void *x_dev,
                  int x_dtype, int batch, float *y_dev, int reps, int flags,
                  double *us_per_launch) {
  return guard([&]() -> int {
    XE_REQUIRE(ctx && ws && n_weights > 0 && x_dev && y_dev && us_per_launch, "null argument");
    XE_REQUIRE(reps > 0, "reps must be positive");
    XE_REQUIRE(batch >= 1 && batch <= kMaxOpBatch, "gemv batch must be 1..512");
    for (int i = 0; i < n_weights; i++) {
      XE_REQUIRE(ws[i], "null weight");
      XE_REQUIRE(ws[i]->m == ws[0]->m && ws[i]->k == ws[0]->k, "probe weights differ in shape");
    }
    DeviceGuard dg(ctx->dev->ordinal);
    if (gemm_preferred(ws[0]->m, ws[0]->k, batch))
      ctx->ensure_gemm(static_cast<size_t>(batch) * ws[0]->k);  // no allocation under capture
    const double us = time_captured(ctx, reps, flags, [&]() {
      for (int i = 0; i < n_weights; i++)
        launch_linear(ctx, ws[i], x_dev, x_dtype, batch, y_dev, ctx->dev->stream);
    });
    *us_per_launch = us / n_weights;
    return 0;
  }, -1);
}

int xe_probe_attn(xe_ctx *ctx, const float *q_dev, const uint16_t *kc_dev, const uint16_t *vc_dev,
                  const int32_t *lens_dev, int batch, int hq, int hkv, int hd, int max_ctx,
                  float scale, float *out_dev, int reps, int flags, double *us_per_call) {
  return guard([&]() -> int {
    XE_REQUIRE(ctx && q_dev && kc_dev && vc_dev && lens_dev && out_dev && us_per_call, "null argument");
    XE_REQUIRE(batch > 0 && hq > 0 && hkv > 0 && hd > 0 && reps > 0, "bad shape");
    DeviceGuard dg(ctx->dev->ordinal);
    ctx->ensure_attn(attn_work_floats(batch, hq, hd, attn_splits(ctx, batch, hkv, max_ctx)),
                     attn_merge_in_place() ? static_cast<size_t>(batch) * hkv : 0);  // no allocation under capture
    *us_per_call = time_captured(ctx, reps, flags, [&]() {
      attn_impl(ctx, q_dev, kc_dev, vc_dev, lens_dev, batch, hq, hkv, hd, max_ctx, scale, out_dev);
    });
    return 0;
  }, -1);
}

}  // extern "C"
