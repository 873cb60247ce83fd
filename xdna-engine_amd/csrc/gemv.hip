// gemv.hip -- decode GEMV kernels for gfx950 (device code in gemv_dev.h) and
// the int8-activation x int8-weight -> int32 GEMV of the W8A8 path.
#include <algorithm>

#include "step_dev.h"

namespace xe {
namespace gdev {

int cu_count() {
  static int n = 0;
  if (!n) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      n = 0;
    if (n <= 0) n = 256;
  }
  return n;
}

// Tile choice, from a graph-replay sweep on MI355X (weights rotated past the
// 256 MB Infinity Cache): 4-wave workgroups always win; with enough rows, a
// narrow lane split with 2 rows per lane keeps the most bytes in flight
// (lm-head 262144 x 1152: LPR 8, RPL 2 -> 6.1 TB/s); with few rows, a wide
// split gives the workgroup count (down 1152 x 6912: LPR 64).  Candidates in
// order of preference; the first with >= one workgroup per CU and >= 70% of
// lanes busy on K wins, else the one with the most workgroups.
// XE_GEMV_TILE="lpr,rpl[,4]" overrides (tuning).
Tile choose_tile(int m, int k, int act) {
  const char *env = getenv("XE_GEMV_TILE");
  if (env) {
    int a = 0, b = 0, c = 4;
    if (sscanf(env, "%d,%d,%d", &a, &b, &c) >= 2) {
      Tile t{a, b, 4};
      if (act == ACT_GEGLU_TANH && t.rpl < 2) t.rpl = 2;
      return t;
    }
  }
  const int nch = k / 16;
  const int cus = cu_count();
  static const Tile cands[] = {{8, 2, 4}, {16, 2, 4}, {16, 1, 4}, {32, 2, 4},
                               {32, 1, 4}, {64, 2, 4}, {64, 1, 4}};
  Tile best{32, 2, 4};
  int best_wgs = -1;
  for (const Tile &t : cands) {
    if (act == ACT_GEGLU_TANH && t.rpl < 2) continue;
    const int it = (nch + t.lpr - 1) / t.lpr;
    const bool eff = static_cast<double>(nch) / (it * t.lpr) >= 0.7;
    const int rows = t.wpb * (64 / t.lpr) * t.rpl;
    const int wgs = (m + rows - 1) / rows;
    if (eff && wgs >= cus) return t;
    if (eff && wgs > best_wgs) {
      best = t;
      best_wgs = wgs;
    }
  }
  return best;
}

GemvParams to_params(const GemvLaunch &L) {
  GemvParams p{};
  p.w = L.w;
  p.scale = L.scale;
  p.exps = L.exps;
  p.bias = L.bias;
  p.m = L.m;
  p.k = L.k;
  p.x = L.x;
  p.x_bf16 = L.x_dtype == XE_BF16;
  p.ldx = L.ldx ? L.ldx : L.k;
  p.batch = L.batch;
  p.sub = L.sub;
  p.post_w = L.post_w;
  p.res_out = L.res_out;
  p.norm = L.norm;
  p.gamma = L.gamma;
  p.beta = L.beta;
  p.eps = L.eps;
  p.act = L.act;
  p.out_scale = L.out_scale;
  p.y = L.y;
  p.ldy = L.ldy ? L.ldy : (L.act == ACT_GEGLU_TANH ? L.m / 2 : L.m);
  return p;
}

}  // namespace gdev

namespace {

using gdev::GemvParams;
using gdev::Tile;

template <int WT, int NB, int LPR, int RPL, int WPB>
__global__ __launch_bounds__(64 * WPB) void gemv_kernel(GemvParams p) {
  extern __shared__ float4 xs4[];
  __shared__ float red[2 * gdev::kRedN * gdev::kMaxWaves];
  gdev::gemv_tiles<WT, NB, LPR, RPL, WPB>(p, xs4, red, blockIdx.x, gridDim.x, blockIdx.x == 0);
}

// ---------------------------------------------------------------------------
// int8 x int8 -> int32 (W8A8 device part; exact)
// ---------------------------------------------------------------------------
constexpr int kThreads = 256;
constexpr int kWaves = 4;

template <int NB>
__global__ __launch_bounds__(kThreads) void gemv_i8act_kernel(const int8_t *__restrict__ q,
                                                             const int8_t *__restrict__ xq,
                                                             int m, int k, int batch,
                                                             W8a8Epi e) {
  extern __shared__ float4 xs4[];
  int8_t *xs = reinterpret_cast<int8_t *>(xs4);
  for (int i = threadIdx.x; i < batch * k; i += kThreads) xs[i] = xq[i];
  __syncthreads();
  constexpr int LPR = 16, RG = 64 / LPR;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rg = lane / LPR, kl = lane % LPR;
  const int r = (blockIdx.x * kWaves + wave) * RG + rg;
  const int nch = k / 16;
  const int rr = r < m ? r : m - 1;
  int32_t acc[NB];
#pragma unroll
  for (int b = 0; b < NB; b++) acc[b] = 0;
  const uint4 *wr = reinterpret_cast<const uint4 *>(q + static_cast<size_t>(rr) * k);
  for (int c = kl; c < nch; c += LPR) {
    const uint4 w = gdev::ld_nt16(wr + c);
#pragma unroll
    for (int b = 0; b < NB; b++) {
      if (b < batch) {
        const uint4 xv = *reinterpret_cast<const uint4 *>(xs + static_cast<size_t>(b) * k + c * 16);
        int32_t a = acc[b];
        a = __builtin_amdgcn_sdot4(static_cast<int>(w.x), static_cast<int>(xv.x), a, false);
        a = __builtin_amdgcn_sdot4(static_cast<int>(w.y), static_cast<int>(xv.y), a, false);
        a = __builtin_amdgcn_sdot4(static_cast<int>(w.z), static_cast<int>(xv.z), a, false);
        a = __builtin_amdgcn_sdot4(static_cast<int>(w.w), static_cast<int>(xv.w), a, false);
        acc[b] = a;
      }
    }
  }
#pragma unroll
  for (int b = 0; b < NB; b++) {
    int32_t v = acc[b];
#pragma unroll
    for (int off = LPR / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    acc[b] = v;
  }
  if (kl == 0 && r < m)
    for (int b = 0; b < batch && b < NB; b++) w8a8_store(e, b, r, m, acc[b]);
}

// ---------------------------------------------------------------------------
// host-side dispatch
// ---------------------------------------------------------------------------
using GemvFn = void (*)(GemvParams);

template <int WT, int NB>
GemvFn pick_lpr_rpl(int lpr, int rpl) {
#define XE_CASE(L, R) \
  if (lpr == L && rpl == R) return gemv_kernel<WT, NB, L, R, 4>;
  XE_CASE(8, 1) XE_CASE(8, 2) XE_CASE(16, 1) XE_CASE(16, 2)
  XE_CASE(32, 1) XE_CASE(32, 2) XE_CASE(64, 1) XE_CASE(64, 2)
#undef XE_CASE
  return nullptr;
}

template <int WT>
GemvFn pick_nb(int nb, int lpr, int rpl) {
  switch (nb) {
    case 1: return pick_lpr_rpl<WT, 1>(lpr, rpl);
    case 2: return pick_lpr_rpl<WT, 2>(lpr, rpl);
    case 4: return pick_lpr_rpl<WT, 4>(lpr, rpl);
    case 8: return pick_lpr_rpl<WT, 8>(lpr, rpl);
  }
  return nullptr;
}

GemvFn pick(int wt, int nb, int lpr, int rpl) {
  switch (wt) {
    case XE_I8: return pick_nb<XE_I8>(nb, lpr, rpl);
    case XE_BF16: return pick_nb<XE_BF16>(nb, lpr, rpl);
    case XE_BFP16: return pick_nb<XE_BFP16>(nb, lpr, rpl);
    case XE_I4: return pick_nb<XE_I4>(nb, lpr, rpl);
  }
  return nullptr;
}

}  // namespace

void launch_gemv(const GemvLaunch &L, hipStream_t s) {
  XE_REQUIRE(L.m > 0 && L.k > 0 && L.batch > 0, "gemv: empty shape");
  XE_REQUIRE(L.k % 16 == 0, "gemv: K must be a multiple of 16");
  XE_REQUIRE(L.batch <= 8, "gemv: batch > 8 must use the batched GEMM path");
  XE_REQUIRE(L.act != ACT_GEGLU_TANH || L.m % 2 == 0, "gemv: GeGLU needs paired rows");
  XE_REQUIRE(L.norm == XE_NORM_NONE || L.gamma, "gemv: norm without gamma");
  XE_REQUIRE(L.norm != XE_NORM_LN || L.beta, "gemv: LayerNorm without beta");
  XE_REQUIRE((L.wdtype != XE_I8 && L.wdtype != XE_I4) || L.scale, "gemv: int8/int4 weight without scales");
  XE_REQUIRE(L.wdtype != XE_BFP16 || L.exps, "gemv: bfp16 weight without exponents");
  XE_REQUIRE(!L.sub || L.x_dtype == XE_F32, "gemv: residual prologue needs fp32 x");
  const int nb = L.batch <= 1 ? 1 : L.batch <= 2 ? 2 : L.batch <= 4 ? 4 : 8;
  const Tile t = gdev::choose_tile(L.m, L.k, L.act);
  GemvFn fn = pick(L.wdtype, nb, t.lpr, t.rpl);
  XE_REQUIRE(fn, "gemv: no kernel for this dtype/tile");
  const GemvParams p = gdev::to_params(L);
  const size_t lds = gdev::gemv_lds_floats(nb, L.k, L.sub != nullptr) * sizeof(float);
  XE_REQUIRE(lds <= 160 * 1024 - 1024, "gemv: batch*K too large for LDS staging");
  if (lds > 64 * 1024)
    XE_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(fn),
                               hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
  const int rows_per_block = t.wpb * (64 / t.lpr) * t.rpl;
  const int tiles = (L.m + rows_per_block - 1) / rows_per_block;
  // at most 4 workgroups per CU: large GEMVs loop over tiles and stage x once
  const int grid = std::min(tiles, 4 * gdev::cu_count());
  hipLaunchKernelGGL(fn, dim3(grid), dim3(64 * t.wpb), lds, s, p);
  XE_HIP(hipGetLastError());
}

// One GEMV phase of a step (phase.variant = weight dtype; tile in phase).
void launch_gemv_phase(const sdev::Phase &ph, hipStream_t s) {
  const GemvParams &p = ph.u.gemv;
  const int nb = p.batch <= 1 ? 1 : p.batch <= 2 ? 2 : p.batch <= 4 ? 4 : 8;
  GemvFn fn = pick(ph.variant, nb, ph.lpr, ph.rpl);
  XE_REQUIRE(fn, "gemv phase: no kernel for this dtype/tile");
  const size_t lds = gdev::gemv_lds_floats(nb, p.k, p.sub != nullptr) * sizeof(float);
  XE_REQUIRE(lds <= 160 * 1024 - 1024, "gemv: batch*K too large for LDS staging");
  if (lds > 64 * 1024)
    XE_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(fn),
                               hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
  const int rows_per_block = 4 * (64 / ph.lpr) * ph.rpl;
  const int tiles = (p.m + rows_per_block - 1) / rows_per_block;
  const int grid = std::min(tiles, 4 * gdev::cu_count());
  hipLaunchKernelGGL(fn, dim3(grid), dim3(256), lds, s, p);
  XE_HIP(hipGetLastError());
}

void launch_gemv_i8act(const int8_t *q, const int8_t *xq, int m, int k, int batch,
                       const W8a8Epi &e, hipStream_t s) {
  XE_REQUIRE(m > 0 && k > 0 && batch > 0 && batch <= 8, "gemv_i8act: bad shape");
  XE_REQUIRE(k % 16 == 0, "gemv_i8act: K must be a multiple of 16");
  const size_t lds = static_cast<size_t>(batch) * k;
  XE_REQUIRE(lds <= 160 * 1024 - 1024, "gemv_i8act: batch*K too large");
  const int rows_per_block = kWaves * 4;
  const int grid = (m + rows_per_block - 1) / rows_per_block;
  auto fn = batch <= 1 ? gemv_i8act_kernel<1> : batch <= 4 ? gemv_i8act_kernel<4> : gemv_i8act_kernel<8>;
  if (lds > 64 * 1024)
    XE_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(fn),
                               hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
  hipLaunchKernelGGL(fn, dim3(grid), dim3(kThreads), lds, s, q, xq, m, k, batch, e);
  XE_HIP(hipGetLastError());
}

}  // namespace xe
