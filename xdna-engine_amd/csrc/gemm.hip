// gemm.hip -- decode projections for 16 or more streams on MFMA.
//
// At b >= 16 a decode projection Y[b, m] = act(scale[m] * sum_k W[m, k] X[b, k]
// + bias[m]) is a real GEMM (the reference's batched lockstep decoder,
// rust/npu-engine/src/asr/whisper_decoder.rs:1541-1831, runs it as an NPU
// GEMM with N = B).  Here it runs on v_mfma_f32_16x16x32_bf16:
//
//   A (weights): 16 rows x 32 k per step.  int8 and bfp16 weights convert to
//   bf16 exactly (at most 8 significant bits), bf16 weights are used as is.
//   B (activations): the fp32 activations split into three bf16 parts,
//   x = hi + mid + lo exactly (truncation: each part takes the next 8
//   significant bits), so the three MFMAs sum the exact fp32 products.
//   Accumulation is fp32.  Numerically this is the fp32 GEMV of the b <= 8
//   path up to summation order, so greedy streams stay the oracle's.
//
// Workgroup: 4 waves, 64 weight rows (16 per wave) x 64 streams (4 MFMA
// column blocks), K in steps of 64.  The activation tile of a step is staged
// in LDS as its three parts, the next step's weights and activations are
// loaded before the current step's MFMAs.  Within a lane's 16 contiguous k
// the two MFMAs of a step take k 0..7 and 8..15: the A and B operands use
// the same k permutation, so the dot products are unchanged.
//
// The norm / residual prologue of a GEMV phase (gemv_dev.h gemv_prologue)
// runs as its own kernel, one workgroup per stream row, writing the
// normalised activations that the GEMM reads.
#include "gemv_dev.h"

namespace xe {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 64, kBN = 64, kBK = 64;
constexpr int kGT = 256;             // threads
constexpr int kXS = kBK + 8;         // LDS row stride (bf16) of a staged part
constexpr int kNoRec = 0x7ffffff0;  // past every buffer: loads return zeros

// Upper 16 bits of two fp32 values (exact bf16 of values with <= 8
// significant bits) packed as a bf16 pair.
__device__ __forceinline__ uint32_t pack_hi16(float lo, float hi) {
  return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

__device__ __forceinline__ float trunc_bf16(float x) { return __uint_as_float(__float_as_uint(x) & 0xffff0000u); }

template <int WT>
struct WLoad {  // one lane's 16 weights of a step (raw)
  u32x4 q;      // int8 / bfp16 mantissas, or bf16 k 0..7
  u32x4 q2;     // bf16 k 8..15
  uint32_t e;   // bfp16: the two block exponents
};

template <int WT>
__device__ __forceinline__ void load_w(const __amdgpu_buffer_rsrc_t &rw, const __amdgpu_buffer_rsrc_t &re, int row,
                                       int k, bool ok, int K, WLoad<WT> &o) {
  if constexpr (WT == XE_BF16) {
    const int off = ok ? (row * K + k) * 2 : kNoRec;
    o.q = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, off, 0, 2));
    o.q2 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, ok ? off + 16 : kNoRec, 0, 2));
  } else {
    o.q = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, ok ? row * K + k : kNoRec, 0, 2));
    if constexpr (WT == XE_BFP16)
      o.e = __builtin_amdgcn_raw_buffer_load_b16(re, ok ? row * (K / 8) + k / 8 : kNoRec, 0, 2);
  }
}

// bf16 A operands of the two MFMAs of a step.
template <int WT>
__device__ __forceinline__ void to_bf16(const WLoad<WT> &w, bf16x8 &a0, bf16x8 &a1) {
  if constexpr (WT == XE_BF16) {
    a0 = __builtin_bit_cast(bf16x8, w.q);
    a1 = __builtin_bit_cast(bf16x8, w.q2);
  } else {
    const uint32_t d[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
    uint32_t p[8];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      float f[4];
#pragma unroll
      for (int j = 0; j < 4; j++) f[j] = static_cast<float>(static_cast<int>(static_cast<int8_t>(d[i] >> (8 * j))));
      if constexpr (WT == XE_BFP16) {
        // bytes 0..7 share exponent byte 0, bytes 8..15 exponent byte 1
        const int e = static_cast<int>((w.e >> (i < 2 ? 0 : 8)) & 0xffu) - 133;
#pragma unroll
        for (int j = 0; j < 4; j++) f[j] = __builtin_ldexpf(f[j], e);
      }
      p[2 * i] = pack_hi16(f[0], f[1]);
      p[2 * i + 1] = pack_hi16(f[2], f[3]);
    }
    a0 = __builtin_bit_cast(bf16x8, u32x4{p[0], p[1], p[2], p[3]});
    a1 = __builtin_bit_cast(bf16x8, u32x4{p[4], p[5], p[6], p[7]});
  }
}

template <int WT>
__global__ __launch_bounds__(kGT) void gemm_kernel(gdev::GemvParams p) {
  // three parts x [kBN][kXS] bf16
  __shared__ __attribute__((aligned(16))) uint16_t xs[3][kBN * kXS];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int m0 = blockIdx.x * kBM, b0 = blockIdx.y * kBN;
  const int K = p.k;
  const int nsteps = (K + kBK - 1) / kBK;
  const int nb = min(kBN, p.batch - b0);
  const __amdgpu_buffer_rsrc_t rw = gdev::coherent_rsrc(p.w);
  const __amdgpu_buffer_rsrc_t re = gdev::coherent_rsrc(WT == XE_BFP16 ? static_cast<const void *>(p.exps) : p.w);
  const __amdgpu_buffer_rsrc_t rx = gdev::coherent_rsrc(p.x);

  // this lane's weight row and k offset within a step
  const int wrow = m0 + wave * 16 + (lane & 15);
  const bool wrow_ok = wrow < p.m;
  const int wk = 16 * (lane >> 4);
  // activation staging: thread t stages row t / 4, k (t % 4) * 16 .. + 16
  const int srow = threadIdx.x >> 2, sk = (threadIdx.x & 3) * 16;
  const bool srow_ok = srow < nb;

  WLoad<WT> wcur, wnxt;
  f32x4 xcur[4], xnxt[4];
  auto load_x = [&](int step, f32x4 (&xv)[4]) {
    const int k = step * kBK + sk;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const bool ok = srow_ok && k + 4 * i < K;
      const int off = ok ? ((b0 + srow) * p.ldx + k + 4 * i) * 4 : kNoRec;
      xv[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0));
    }
  };
  auto load_wstep = [&](int step, WLoad<WT> &w) {
    const int k = step * kBK + wk;
    load_w<WT>(rw, re, wrow, k, wrow_ok && k < K, K, w);
  };
  load_wstep(0, wcur);
  load_x(0, xcur);

  f32x4 acc[4];
#pragma unroll
  for (int j = 0; j < 4; j++) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int step = 0; step < nsteps; step++) {
    // stage this step's activations as three bf16 parts
    {
      uint32_t hp[8], mp[8], lp[8];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float v[4] = {xcur[i].x, xcur[i].y, xcur[i].z, xcur[i].w};
        float h[4], m[4], l[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
          h[j] = trunc_bf16(v[j]);
          const float r = v[j] - h[j];
          m[j] = trunc_bf16(r);
          l[j] = trunc_bf16(r - m[j]);
        }
        hp[2 * i] = pack_hi16(h[0], h[1]);
        hp[2 * i + 1] = pack_hi16(h[2], h[3]);
        mp[2 * i] = pack_hi16(m[0], m[1]);
        mp[2 * i + 1] = pack_hi16(m[2], m[3]);
        lp[2 * i] = pack_hi16(l[0], l[1]);
        lp[2 * i + 1] = pack_hi16(l[2], l[3]);
      }
      if (step > 0) __syncthreads();  // the previous step's reads are done
      uint32_t *dh = reinterpret_cast<uint32_t *>(xs[0] + srow * kXS + sk);
      uint32_t *dm = reinterpret_cast<uint32_t *>(xs[1] + srow * kXS + sk);
      uint32_t *dl = reinterpret_cast<uint32_t *>(xs[2] + srow * kXS + sk);
      *reinterpret_cast<u32x4 *>(dh) = u32x4{hp[0], hp[1], hp[2], hp[3]};
      *reinterpret_cast<u32x4 *>(dh + 4) = u32x4{hp[4], hp[5], hp[6], hp[7]};
      *reinterpret_cast<u32x4 *>(dm) = u32x4{mp[0], mp[1], mp[2], mp[3]};
      *reinterpret_cast<u32x4 *>(dm + 4) = u32x4{mp[4], mp[5], mp[6], mp[7]};
      *reinterpret_cast<u32x4 *>(dl) = u32x4{lp[0], lp[1], lp[2], lp[3]};
      *reinterpret_cast<u32x4 *>(dl + 4) = u32x4{lp[4], lp[5], lp[6], lp[7]};
    }
    if (step + 1 < nsteps) {
      load_wstep(step + 1, wnxt);
      load_x(step + 1, xnxt);
    }
    __syncthreads();
    bf16x8 a0, a1;
    to_bf16<WT>(wcur, a0, a1);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      if (16 * j < nb) {  // column blocks past the batch are skipped (uniform)
        const int brow = 16 * j + (lane & 15);
#pragma unroll
        for (int part = 0; part < 3; part++) {
          const uint16_t *src = xs[part] + brow * kXS + wk;
          const bf16x8 x0 = *reinterpret_cast<const bf16x8 *>(src);
          const bf16x8 x1 = *reinterpret_cast<const bf16x8 *>(src + 8);
          acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, x0, acc[j], 0, 0, 0);
          acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, x1, acc[j], 0, 0, 0);
        }
      }
    }
    wcur = wnxt;
#pragma unroll
    for (int i = 0; i < 4; i++) xcur[i] = xnxt[i];
  }

  // epilogue: lane holds rows r0 + i (i = 0..3) of column block j's stream
  const int r0 = m0 + wave * 16 + 4 * (lane >> 4);
  float sc[4], bi[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int r = min(r0 + i, p.m - 1);
    sc[i] = WT == XE_I8 ? p.scale[r] : 1.0f;
    bi[i] = p.bias ? p.bias[r] : 0.0f;
  }
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int b = 16 * j + (lane & 15);
    if (b >= nb) continue;
    float *yrow = p.y + static_cast<size_t>(b0 + b) * p.ldy;
    float t[4];
#pragma unroll
    for (int i = 0; i < 4; i++) t[i] = acc[j][i] * sc[i] + bi[i];
    if (p.act == ACT_GEGLU_TANH) {
      // rows come in (gate, up) pairs: r0 + (0, 1) and r0 + (2, 3)
#pragma unroll
      for (int i = 0; i < 4; i += 2)
        if (r0 + i + 1 < p.m) yrow[(r0 + i) / 2] = gdev::gelu_tanh(t[i]) * t[i + 1] * p.out_scale;
    } else {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        if (r0 + i >= p.m) continue;
        float v = t[i];
        if (p.act == ACT_RELU) v = v > 0.f ? v : 0.f;
        else if (p.act == ACT_GELU_ERF) v = gdev::gelu_erf(v);
        yrow[r0 + i] = v * p.out_scale;
      }
    }
  }
}

// Norm / residual prologue of one stream row (blockIdx.x): p.x, p.sub and
// p.res_out point at row 0 and advance by ldx / k per row; the normalised
// row goes to xn [batch][k].
__global__ __launch_bounds__(256) void gemm_prologue_kernel(gdev::GemvParams p, float *xn) {
  extern __shared__ float4 xs4[];
  __shared__ float red[2 * 4 * gdev::kMaxWaves];
  const int b = blockIdx.x;
  gdev::GemvParams q = p;
  q.x = static_cast<const float *>(p.x) + static_cast<size_t>(b) * p.ldx;
  q.sub = p.sub ? p.sub + static_cast<size_t>(b) * p.k : nullptr;
  q.res_out = p.res_out ? p.res_out + static_cast<size_t>(b) * p.k : nullptr;
  q.batch = 1;
  gdev::gemv_prologue<1, 4, false>(q, xs4, red, true);
  const float *xs = reinterpret_cast<const float *>(xs4);
  for (int i = threadIdx.x; i < p.k; i += 256) xn[static_cast<size_t>(b) * p.k + i] = xs[i];
}

using GemmFn = void (*)(gdev::GemvParams);

GemmFn pick_gemm(int wdtype) {
  switch (wdtype) {
    case XE_I8: return gemm_kernel<XE_I8>;
    case XE_BF16: return gemm_kernel<XE_BF16>;
    case XE_BFP16: return gemm_kernel<XE_BFP16>;
  }
  return nullptr;
}

}  // namespace

bool gemm_needs_prologue(const gdev::GemvParams &p) { return p.sub != nullptr || p.norm != XE_NORM_NONE; }

// Prologue (when the phase has one) into xn, then the GEMM reading xn.
void launch_gemm_prologue(const gdev::GemvParams &p, float *xn, hipStream_t s) {
  XE_REQUIRE(!p.x_bf16, "gemm: fp32 activations only");
  const size_t lds = gdev::gemv_lds_floats(1, p.k, p.sub != nullptr) * sizeof(float);
  XE_REQUIRE(lds <= 160 * 1024 - 1024, "gemm prologue: K too large for LDS staging");
  if (lds > 64 * 1024)
    XE_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(gemm_prologue_kernel),
                               hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
  hipLaunchKernelGGL(gemm_prologue_kernel, dim3(p.batch), dim3(256), lds, s, p, xn);
  XE_HIP(hipGetLastError());
}

void launch_gemm(const gdev::GemvParams &p, int wdtype, hipStream_t s) {
  XE_REQUIRE(p.m > 0 && p.k > 0 && p.batch > 0, "gemm: empty shape");
  XE_REQUIRE(p.k % 16 == 0, "gemm: K must be a multiple of 16");
  XE_REQUIRE(!p.x_bf16, "gemm: fp32 activations only");
  XE_REQUIRE(p.act != ACT_GEGLU_TANH || p.m % 4 == 0, "gemm: GeGLU rows must pair within 4-row groups");
  XE_REQUIRE(wdtype != XE_I8 || p.scale, "gemm: int8 weight without scales");
  XE_REQUIRE(wdtype != XE_BFP16 || p.exps, "gemm: bfp16 weight without exponents");
  // buffer offsets are 32-bit: weights and activations below 2 GB
  const size_t wb = static_cast<size_t>(p.m) * p.k * (wdtype == XE_BF16 ? 2 : 1);
  XE_REQUIRE(wb < (size_t(1) << 31) && static_cast<size_t>(p.batch) * p.ldx * 4 < (size_t(1) << 31),
             "gemm: operand above 2 GB");
  GemmFn fn = pick_gemm(wdtype);
  XE_REQUIRE(fn, "gemm: unsupported weight dtype");
  hipLaunchKernelGGL(fn, dim3((p.m + kBM - 1) / kBM, (p.batch + kBN - 1) / kBN), dim3(kGT), 0, s, p);
  XE_HIP(hipGetLastError());
}

}  // namespace xe
