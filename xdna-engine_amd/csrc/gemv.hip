// gemv.hip -- decode GEMV for gfx950: y[b] = epilogue(W . prologue(x[b])).
//
// Replaces the reference's resident GEMV dispatch (CtxDecode::gemv,
// rust/npu-asr/src/ctx_decode.rs:325-366, and the whole-array design
// route_b_kernels/decode_norm_gemv/norm_gemv_iron.py:52-216) and its fused
// pre-norm (ctx_decode.rs:566-643, aie_kernels/norm_gemv_prologue.cc:31-75).
//
// Batch <= 8 decode is HBM-bound on the weight stream, so the kernel is built
// around the weight bytes:
//   * Each wave covers RG = 64/LPR row groups; a group's LPR lanes split K in
//     16-element chunks (16 B of int8 / bfp16 mantissas, 32 B of bf16), so one
//     load instruction of the wave reads RG rows x LPR*16 B contiguous runs:
//     whole 128-byte lines from HBM.
//   * RPL rows per lane share the x chunk held in registers.
//   * Weight loads for the first U chunks are issued before the prologue, so
//     the norm/residual prologue overlaps the HBM latency.
//   * x (after the prologue) lives in LDS as fp32 [b][K]; a lane reads its
//     16-element chunk as four 16 B words.
//   * The group reduction is an xor-butterfly over LPR lanes (DPP/swizzle).
//   * int8 -> fp32 dequant happens in registers; the per-row fp32 scale is
//     applied after the sum, as in Lin::fwd (opt125m_decode.rs:120-122).
#include <algorithm>

#include "common.h"

namespace xe {
namespace {

constexpr int kMaxWaves = 4;

struct GemvParams {
  const void *w;
  const float *scale;
  const uint8_t *exps;
  const float *bias;
  int m, k;
  const void *x;
  int x_bf16;
  int ldx;
  int batch;
  const float *sub;
  const float *post_w;
  float *res_out;
  int norm;
  const float *gamma;
  const float *beta;
  float eps;
  int act;
  float out_scale;
  float *y;
  int ldy;
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Block-wide sums of N values over WPB waves with one barrier; `slot`
// alternates so back-to-back reductions never overwrite a slot still being
// read.  red holds 2 * 4 * kMaxWaves floats.
template <int WPB, int N>
__device__ __forceinline__ void block_sums(float (&v)[N], float *red, int &slot) {
#pragma unroll
  for (int i = 0; i < N; i++) v[i] = wave_sum(v[i]);
  if constexpr (WPB == 1) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float *r = red + slot * 4 * kMaxWaves;
  slot ^= 1;
  if (lane == 0)
#pragma unroll
    for (int i = 0; i < N; i++) r[i * kMaxWaves + wave] = v[i];
  __syncthreads();
#pragma unroll
  for (int i = 0; i < N; i++) {
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < WPB; w++) t += r[i * kMaxWaves + w];
    v[i] = t;
  }
}

__device__ __forceinline__ float gelu_erf(float x) {
  // Abramowitz & Stegun 7.1.26 erf, the reference's host GELU
  // (rust/npu-asr-host/src/lib.rs:464-489).
  float z = x * 0.70710678118654752f;
  float sgn = z < 0.f ? -1.f : 1.f;
  float a = fabsf(z);
  float t = 1.0f / (1.0f + 0.3275911f * a);
  float y = 1.0f - (((((1.061405429f * t - 1.453152027f) * t) + 1.421413741f) * t -
                     0.284496736f) * t + 0.254829592f) * t * expf(-a * a);
  return 0.5f * x * (1.0f + sgn * y);
}

__device__ __forceinline__ float gelu_tanh(float x) {
  // gelu_pytorch_tanh (rust/npu-gemma/src/lib.rs:74-77).
  const float c = 0.79788456f;
  return 0.5f * x * (1.0f + tanhf(c * (x + 0.044715f * x * x * x)));
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// 16-byte streaming load (weights are read once per launch: nontemporal).
__device__ __forceinline__ uint4 ld_nt16(const void *ptr) {
  const u32x4 v = __builtin_nontemporal_load(static_cast<const u32x4 *>(ptr));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// One 16-element chunk of a weight row, raw.
template <int WT>
struct Chunk;
template <>
struct Chunk<XE_I8> {
  uint4 q;
};
template <>
struct Chunk<XE_BFP16> {
  uint4 q;
  uint32_t e;  // two biased exponents (low 16 bits)
};
template <>
struct Chunk<XE_BF16> {
  uint4 lo, hi;
};

template <int WT>
__device__ __forceinline__ void load_chunk(const GemvParams &p, int row, int c,
                                           Chunk<WT> &out) {
  if constexpr (WT == XE_I8) {
    const uint4 *base = reinterpret_cast<const uint4 *>(
        static_cast<const int8_t *>(p.w) + static_cast<size_t>(row) * p.k);
    out.q = ld_nt16(base + c);
  } else if constexpr (WT == XE_BFP16) {
    const uint4 *base = reinterpret_cast<const uint4 *>(
        static_cast<const int8_t *>(p.w) + static_cast<size_t>(row) * p.k);
    out.q = ld_nt16(base + c);
    const uint16_t *eb = reinterpret_cast<const uint16_t *>(
        p.exps + static_cast<size_t>(row) * (p.k / 8));
    out.e = eb[c];
  } else {
    const uint4 *base = reinterpret_cast<const uint4 *>(
        static_cast<const uint16_t *>(p.w) + static_cast<size_t>(row) * p.k);
    out.lo = ld_nt16(base + 2 * c);
    out.hi = ld_nt16(base + 2 * c + 1);
  }
}

__device__ __forceinline__ float sb(uint32_t w, int j) {
  return static_cast<float>(static_cast<int>(static_cast<int8_t>(w >> (8 * j))));
}

// acc += dot(chunk, x[16])
template <int WT>
__device__ __forceinline__ float chunk_dot(const Chunk<WT> &ch, const float4 (&xv)[4],
                                           float acc) {
  if constexpr (WT == XE_I8) {
    const uint32_t w4[4] = {ch.q.x, ch.q.y, ch.q.z, ch.q.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      acc = __builtin_fmaf(xv[i].x, sb(w4[i], 0), acc);
      acc = __builtin_fmaf(xv[i].y, sb(w4[i], 1), acc);
      acc = __builtin_fmaf(xv[i].z, sb(w4[i], 2), acc);
      acc = __builtin_fmaf(xv[i].w, sb(w4[i], 3), acc);
    }
    return acc;
  } else if constexpr (WT == XE_BFP16) {
    const uint32_t w4[4] = {ch.q.x, ch.q.y, ch.q.z, ch.q.w};
    float d[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
      float s = 0.f;
#pragma unroll
      for (int i = 2 * h; i < 2 * h + 2; i++) {
        s = __builtin_fmaf(xv[i].x, sb(w4[i], 0), s);
        s = __builtin_fmaf(xv[i].y, sb(w4[i], 1), s);
        s = __builtin_fmaf(xv[i].z, sb(w4[i], 2), s);
        s = __builtin_fmaf(xv[i].w, sb(w4[i], 3), s);
      }
      d[h] = s;
    }
    const int e0 = static_cast<int>(ch.e & 0xff) - 133;  // e - 127 - 6
    const int e1 = static_cast<int>((ch.e >> 8) & 0xff) - 133;
    acc += __builtin_ldexpf(d[0], e0);
    acc += __builtin_ldexpf(d[1], e1);
    return acc;
  } else {
    const uint32_t w8[8] = {ch.lo.x, ch.lo.y, ch.lo.z, ch.lo.w,
                            ch.hi.x, ch.hi.y, ch.hi.z, ch.hi.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t a = w8[2 * i], b = w8[2 * i + 1];
      acc = __builtin_fmaf(xv[i].x, __uint_as_float(a << 16), acc);
      acc = __builtin_fmaf(xv[i].y, __uint_as_float(a & 0xffff0000u), acc);
      acc = __builtin_fmaf(xv[i].z, __uint_as_float(b << 16), acc);
      acc = __builtin_fmaf(xv[i].w, __uint_as_float(b & 0xffff0000u), acc);
    }
    return acc;
  }
}

// Prologue: x (+ post(sub)) -> res_out (block 0) -> norm -> LDS (transposed).
// Prologue: x (+ post(sub)) -> res_out (block 0) -> norm -> LDS, fp32.
// Statistics are reduced once per row:
//   Gemma (sub + post_w, RMS1P): t = x + sub*inv_s*(1+w) and
//     sum t^2 = sum x^2 + 2 inv_s sum x*s' + inv_s^2 sum s'^2 (s' = sub*(1+w)),
//     so sum sub^2, sum x^2, sum x*s', sum s'^2 come out of one reduction.
//   LayerNorm: two passes (sum t, then sum (t - mean)^2) as the reference's
//     layer_norm (npu-asr-host/src/lib.rs:79-109); one-pass variance loses
//     everything on near-constant rows.
template <int NB, int WPB>
__device__ void gemv_prologue(const GemvParams &p, float4 *xs4, float *red) {
  constexpr int kThreads = 64 * WPB;
  constexpr int UNR = 4;  // float4 loads in flight per thread
  const int K = p.k, K4 = K / 4;
  const float fk = static_cast<float>(K);
  float *xs = reinterpret_cast<float *>(xs4);
  float *sb = xs + static_cast<size_t>(NB) * K;  // sub staging (one row)
  int slot = 0;
  for (int b = 0; b < p.batch && b < NB; b++) {
    float4 *xb4 = xs4 + static_cast<size_t>(b) * K4;
    float *xb = xs + static_cast<size_t>(b) * K;
    const float4 *sub4 = p.sub ? reinterpret_cast<const float4 *>(p.sub + static_cast<size_t>(b) * K) : nullptr;
    const bool fold = p.sub && p.post_w;  // Gemma post-norm + residual
    float acc[4] = {0.f, 0.f, 0.f, 0.f};  // fold: sum sub^2, x^2, x*s', s'^2
    for (int i0 = threadIdx.x; i0 < K4; i0 += kThreads * UNR) {
      float4 v[UNR], sv[UNR];
#pragma unroll
      for (int u = 0; u < UNR; u++) {
        const int i = i0 + u * kThreads;
        if (i < K4) {
          if (p.x_bf16) {
            const uint2 r = reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(p.x) +
                                                            static_cast<size_t>(b) * p.ldx)[i];
            v[u] = make_float4(__uint_as_float(r.x << 16), __uint_as_float(r.x & 0xffff0000u),
                               __uint_as_float(r.y << 16), __uint_as_float(r.y & 0xffff0000u));
          } else {
            v[u] = reinterpret_cast<const float4 *>(static_cast<const float *>(p.x) +
                                                    static_cast<size_t>(b) * p.ldx)[i];
          }
          if (sub4) sv[u] = sub4[i];
        }
      }
#pragma unroll
      for (int u = 0; u < UNR; u++) {
        const int i = i0 + u * kThreads;
        if (i >= K4) continue;
        xb4[i] = v[u];
        if (sub4) reinterpret_cast<float4 *>(sb)[i] = sv[u];
        if (fold) {
          const float4 w = reinterpret_cast<const float4 *>(p.post_w)[i];
          const float xv[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
          const float su[4] = {sv[u].x, sv[u].y, sv[u].z, sv[u].w};
          const float wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
          for (int j = 0; j < 4; j++) {
            const float sp = su[j] * (1.0f + wv[j]);
            acc[0] = __builtin_fmaf(su[j], su[j], acc[0]);
            acc[1] = __builtin_fmaf(xv[j], xv[j], acc[1]);
            acc[2] = __builtin_fmaf(xv[j], sp, acc[2]);
            acc[3] = __builtin_fmaf(sp, sp, acc[3]);
          }
        }
      }
    }
    if (fold) {
      block_sums<WPB, 4>(acc, red, slot);
      const float inv_s = 1.0f / sqrtf(acc[0] / fk + p.eps);
      const float st2 = acc[1] + 2.0f * inv_s * acc[2] + inv_s * inv_s * acc[3];
      const float inv_t = p.norm != XE_NORM_NONE ? 1.0f / sqrtf(fmaxf(st2, 0.f) / fk + p.eps) : 1.f;
      __syncthreads();  // staging complete (block_sums' barrier is skipped for WPB == 1)
      for (int i = threadIdx.x; i < K; i += kThreads) {
        const float t = xb[i] + sb[i] * inv_s * (1.0f + p.post_w[i]);
        if (p.res_out && blockIdx.x == 0) p.res_out[static_cast<size_t>(b) * K + i] = t;
        float h = t;
        if (p.norm == XE_NORM_RMS1P) h = t * inv_t * (1.0f + p.gamma[i]);
        else if (p.norm == XE_NORM_RMS) h = t * inv_t * p.gamma[i];
        xb[i] = h;
      }
      if (p.norm == XE_NORM_LN) {  // not a model combination; keep it exact anyway
        __syncthreads();
        float v1[1] = {0.f};
        for (int i = threadIdx.x; i < K; i += kThreads) v1[0] += xb[i];
        block_sums<WPB, 1>(v1, red, slot);
        const float mean = v1[0] / fk;
        float v2[1] = {0.f};
        for (int i = threadIdx.x; i < K; i += kThreads) {
          const float c = xb[i] - mean;
          v2[0] = __builtin_fmaf(c, c, v2[0]);
        }
        block_sums<WPB, 1>(v2, red, slot);
        const float inv = 1.0f / sqrtf(v2[0] / fk + p.eps);
        __syncthreads();
        for (int i = threadIdx.x; i < K; i += kThreads)
          xb[i] = (xb[i] - mean) * inv * p.gamma[i] + p.beta[i];
      }
    } else {
      __syncthreads();
      if (p.sub) {
        for (int i = threadIdx.x; i < K; i += kThreads) {
          const float t = xb[i] + sb[i];
          xb[i] = t;
          if (p.res_out && blockIdx.x == 0) p.res_out[static_cast<size_t>(b) * K + i] = t;
        }
        if (p.norm != XE_NORM_NONE) __syncthreads();
      }
      if (p.norm == XE_NORM_LN) {
        float v1[1] = {0.f};
        for (int i = threadIdx.x; i < K; i += kThreads) v1[0] += xb[i];
        block_sums<WPB, 1>(v1, red, slot);
        const float mean = v1[0] / fk;
        float v2[1] = {0.f};
        for (int i = threadIdx.x; i < K; i += kThreads) {
          const float c = xb[i] - mean;
          v2[0] = __builtin_fmaf(c, c, v2[0]);
        }
        block_sums<WPB, 1>(v2, red, slot);
        const float inv = 1.0f / sqrtf(v2[0] / fk + p.eps);
        for (int i = threadIdx.x; i < K; i += kThreads)
          xb[i] = (xb[i] - mean) * inv * p.gamma[i] + p.beta[i];
      } else if (p.norm != XE_NORM_NONE) {
        float v1[1] = {0.f};
        for (int i = threadIdx.x; i < K; i += kThreads) v1[0] = __builtin_fmaf(xb[i], xb[i], v1[0]);
        block_sums<WPB, 1>(v1, red, slot);
        const float inv = 1.0f / sqrtf(v1[0] / fk + p.eps);
        for (int i = threadIdx.x; i < K; i += kThreads)
          xb[i] = p.norm == XE_NORM_RMS1P ? xb[i] * inv * (1.0f + p.gamma[i]) : xb[i] * inv * p.gamma[i];
      }
    }
    if (p.sub && b + 1 < p.batch && b + 1 < NB) __syncthreads();  // sub staging is reused
  }
  __syncthreads();
}

template <int WT, int NB, int LPR, int RPL, int WPB>
__global__ __launch_bounds__(64 * WPB) void gemv_kernel(GemvParams p) {
  extern __shared__ float4 xs4[];
  __shared__ float red[2 * 4 * kMaxWaves];
  constexpr int RG = 64 / LPR;
  constexpr int U = (RPL >= 2) ? 2 : 4;  // chunks prefetched per row
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rg = lane / LPR, kl = lane % LPR;
  constexpr int rows_per_wave = RG * RPL;
  constexpr int rows_per_block = WPB * rows_per_wave;
  const int K = p.k, nch = K / 16;
  const int n_it = (nch + LPR - 1) / LPR;
  const int ntiles = (p.m + rows_per_block - 1) / rows_per_block;
  const float *xs = reinterpret_cast<const float *>(xs4);

  // The grid may be smaller than the tile count: each workgroup stages x once
  // (the prologue) and walks tiles blockIdx.x, + gridDim.x, ...
  for (int tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int row0 = tile * rows_per_block + wave * rows_per_wave + rg * RPL;
    bool row_ok[RPL];
    int row[RPL];
#pragma unroll
    for (int i = 0; i < RPL; i++) {
      row[i] = row0 + i;
      row_ok[i] = row[i] < p.m;
      if (!row_ok[i]) row[i] = p.m - 1;  // clamp: loads stay in bounds, result dropped
    }

    // Issue the first U chunks of this tile's weights (before the prologue
    // on the first tile, so it overlaps the HBM latency).
    Chunk<WT> pre[U][RPL];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int c = u * LPR + kl;
#pragma unroll
      for (int i = 0; i < RPL; i++)
        if (c < nch) load_chunk<WT>(p, row[i], c, pre[u][i]);
    }
    if (tile == static_cast<int>(blockIdx.x)) gemv_prologue<NB, WPB>(p, xs4, red);

    float acc[NB][RPL];
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
      for (int i = 0; i < RPL; i++) acc[b][i] = 0.f;

    auto compute = [&](const Chunk<WT>(&chs)[RPL], int c) {
#pragma unroll
      for (int b = 0; b < NB; b++) {
        if (b < p.batch) {
          float4 xv[4];
          const float4 *xr = reinterpret_cast<const float4 *>(xs + static_cast<size_t>(b) * K + c * 16);
#pragma unroll
          for (int j = 0; j < 4; j++) xv[j] = xr[j];
#pragma unroll
          for (int i = 0; i < RPL; i++) acc[b][i] = chunk_dot<WT>(chs[i], xv, acc[b][i]);
        }
      }
    };

#pragma unroll
    for (int u = 0; u < U; u++) {
      const int c = u * LPR + kl;
      if (c < nch) compute(pre[u], c);
    }
    for (int it = U; it < n_it; it += U) {
      Chunk<WT> cur[U][RPL];
#pragma unroll
      for (int u = 0; u < U; u++) {
        const int c = (it + u) * LPR + kl;
#pragma unroll
        for (int i = 0; i < RPL; i++)
          if (c < nch) load_chunk<WT>(p, row[i], c, cur[u][i]);
      }
#pragma unroll
      for (int u = 0; u < U; u++) {
        const int c = (it + u) * LPR + kl;
        if (c < nch) compute(cur[u], c);
      }
    }

    // ---- reduce over the LPR lanes of the group ----
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
      for (int i = 0; i < RPL; i++) {
        float v = acc[b][i];
#pragma unroll
        for (int off = LPR / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
        acc[b][i] = v;
      }

    // ---- epilogue (lane 0 of each group) ----
    if (kl == 0) {
#pragma unroll
      for (int b = 0; b < NB; b++) {
        if (b >= p.batch) break;
        float v[RPL];
#pragma unroll
        for (int i = 0; i < RPL; i++) {
          float t = acc[b][i];
          if (WT == XE_I8) t = t * p.scale[row[i]];
          if (p.bias) t = t + p.bias[row[i]];
          v[i] = t;
        }
        if (p.act == ACT_GEGLU_TANH) {
#pragma unroll
          for (int i = 0; i + 1 < RPL; i += 2)
            if (row_ok[i])
              p.y[static_cast<size_t>(b) * p.ldy + row[i] / 2] =
                  gelu_tanh(v[i]) * v[i + 1] * p.out_scale;
        } else {
#pragma unroll
          for (int i = 0; i < RPL; i++) {
            if (!row_ok[i]) continue;
            float t = v[i];
            if (p.act == ACT_RELU) t = t > 0.f ? t : 0.f;
            else if (p.act == ACT_GELU_ERF) t = gelu_erf(t);
            p.y[static_cast<size_t>(b) * p.ldy + row[i]] = t * p.out_scale;
          }
        }
      }
    }
  }
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
                                                             int32_t *__restrict__ acc_out) {
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
    const uint4 w = ld_nt16(wr + c);
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
    for (int b = 0; b < batch && b < NB; b++) acc_out[static_cast<size_t>(b) * m + r] = acc[b];
}

// ---------------------------------------------------------------------------
// host-side dispatch
// ---------------------------------------------------------------------------
using GemvFn = void (*)(GemvParams);

template <int WT, int NB, int WPB>
GemvFn pick_lpr_rpl(int lpr, int rpl) {
#define XE_CASE(L, R) \
  if (lpr == L && rpl == R) return gemv_kernel<WT, NB, L, R, WPB>;
  XE_CASE(8, 1) XE_CASE(8, 2) XE_CASE(16, 1) XE_CASE(16, 2)
  XE_CASE(32, 1) XE_CASE(32, 2) XE_CASE(64, 1) XE_CASE(64, 2)
#undef XE_CASE
  return nullptr;
}

template <int WT, int NB>
GemvFn pick_wpb(int wpb, int lpr, int rpl) {
  // 4-wave workgroups only: 1-wave ones lost every measured shape
  if (wpb == 4) return pick_lpr_rpl<WT, NB, 4>(lpr, rpl);
  return nullptr;
}

template <int WT>
GemvFn pick_nb(int nb, int wpb, int lpr, int rpl) {
  switch (nb) {
    case 1: return pick_wpb<WT, 1>(wpb, lpr, rpl);
    case 2: return pick_wpb<WT, 2>(wpb, lpr, rpl);
    case 4: return pick_wpb<WT, 4>(wpb, lpr, rpl);
    case 8: return pick_wpb<WT, 8>(wpb, lpr, rpl);
  }
  return nullptr;
}

GemvFn pick(int wt, int nb, int wpb, int lpr, int rpl) {
  switch (wt) {
    case XE_I8: return pick_nb<XE_I8>(nb, wpb, lpr, rpl);
    case XE_BF16: return pick_nb<XE_BF16>(nb, wpb, lpr, rpl);
    case XE_BFP16: return pick_nb<XE_BFP16>(nb, wpb, lpr, rpl);
  }
  return nullptr;
}

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

struct Tile {
  int lpr, rpl, wpb;
};

// Tile choice, from a graph-replay sweep on MI355X (weights rotated past the
// 256 MB Infinity Cache): 4-wave workgroups always win; with enough rows, a
// narrow lane split with 2 rows per lane keeps the most bytes in flight
// (lm-head 262144 x 1152: LPR 8, RPL 2 -> 6.1 TB/s); with few rows, a wide
// split gives the workgroup count (down 1152 x 6912: LPR 64).  Candidates in
// order of preference; the first with >= one workgroup per CU and >= 70% of
// lanes busy on K wins, else the one with the most workgroups.
// XE_GEMV_TILE="lpr,rpl,wpb" overrides (tuning).
Tile choose_tile(int m, int k, int act) {
  const char *env = getenv("XE_GEMV_TILE");
  if (env) {
    int a = 0, b = 0, c = 4;
    if (sscanf(env, "%d,%d,%d", &a, &b, &c) >= 2) {
      Tile t{a, b, c};
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

}  // namespace

void launch_gemv(const GemvLaunch &L, hipStream_t s) {
  XE_REQUIRE(L.m > 0 && L.k > 0 && L.batch > 0, "gemv: empty shape");
  XE_REQUIRE(L.k % 16 == 0, "gemv: K must be a multiple of 16");
  XE_REQUIRE(L.batch <= 8, "gemv: batch > 8 must use the batched GEMM path");
  XE_REQUIRE(L.act != ACT_GEGLU_TANH || L.m % 2 == 0, "gemv: GeGLU needs paired rows");
  XE_REQUIRE(L.norm == XE_NORM_NONE || L.gamma, "gemv: norm without gamma");
  XE_REQUIRE(L.norm != XE_NORM_LN || L.beta, "gemv: LayerNorm without beta");
  XE_REQUIRE(L.wdtype != XE_I8 || L.scale, "gemv: int8 weight without scales");
  XE_REQUIRE(L.wdtype != XE_BFP16 || L.exps, "gemv: bfp16 weight without exponents");
  const int nb = L.batch <= 1 ? 1 : L.batch <= 2 ? 2 : L.batch <= 4 ? 4 : 8;
  const Tile t = choose_tile(L.m, L.k, L.act);
  GemvFn fn = pick(L.wdtype, nb, t.wpb, t.lpr, t.rpl);
  XE_REQUIRE(fn, "gemv: no kernel for this dtype/tile");
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
  const size_t lds = static_cast<size_t>(nb + (L.sub ? 1 : 0)) * L.k * sizeof(float);
  XE_REQUIRE(lds <= 160 * 1024 - 1024, "gemv: batch*K too large for LDS staging");
  if (lds > 64 * 1024)
    XE_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(fn),
                               hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
  const int rows_per_block = t.wpb * (64 / t.lpr) * t.rpl;
  const int tiles = (L.m + rows_per_block - 1) / rows_per_block;
  // at most 4 workgroups per CU: large GEMVs loop over tiles and stage x once
  const int grid = std::min(tiles, 4 * cu_count());
  hipLaunchKernelGGL(fn, dim3(grid), dim3(64 * t.wpb), lds, s, p);
  XE_HIP(hipGetLastError());
}

void launch_gemv_i8act(const int8_t *q, const int8_t *xq, int m, int k, int batch,
                       int32_t *acc, hipStream_t s) {
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
  hipLaunchKernelGGL(fn, dim3(grid), dim3(kThreads), lds, s, q, xq, m, k, batch, acc);
  XE_HIP(hipGetLastError());
}

}  // namespace xe
