// gemv_dev.h -- device side of the decode GEMV: y[b] = epilogue(W . prologue(x[b])).
//
// Replaces the reference's resident GEMV dispatch (CtxDecode::gemv,
// rust/npu-asr/src/ctx_decode.rs:325-366, and the whole-array design
// route_b_kernels/decode_norm_gemv/norm_gemv_iron.py:52-216) and its fused
// pre-norm (ctx_decode.rs:566-643, aie_kernels/norm_gemv_prologue.cc:31-75).
//
// Batch <= 8 decode is HBM-bound on the weight stream, so the work is built
// around the weight bytes:
//   * Each wave covers RG = 64/LPR row groups; a group's LPR lanes split K in
//     16-element chunks (16 B of int8 / bfp16 mantissas, 32 B of bf16), so one
//     load instruction of the wave reads RG rows x LPR*16 B contiguous runs:
//     whole 128-byte lines from HBM.
//   * RPL rows per lane share the x chunk held in registers.
//   * Weight loads run as a ping-pong of two sets of U chunks per row; the
//     first two sets are issued before the prologue, so they overlap HBM
//     latency.
//   * x (after the prologue) lives in LDS as fp32 [b][K], each chunk's four
//     16 B words permuted (xs_word) so a wave's chunk reads are free of bank
//     conflicts; every row of the batch tile is computed (no branch on the
//     batch count), rows past the batch being zero.
//   * The group reduction is an xor-butterfly over LPR lanes.
//   * int8 -> fp32 dequant happens in registers; the per-row fp32 scale is
//     applied after the sum, as in Lin::fwd (opt125m_decode.rs:120-122).
//
// act_ld / act_st<COH>: plain loads and stores, or coherent ones (sc1 loads,
// agent-scope stores) for code that reads in one launch what another XCD
// wrote (the attention merge inside the split kernel, the low-latency step
// kernel), since the XCDs' L2s are not coherent with each other.  Weights
// are read-only and always use plain streaming loads.
#pragma once

#include "common.h"

namespace xe {
namespace gdev {

constexpr int kMaxWaves = 8;

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
  // The MFMA GEMM's split-K partials handed to the consumer: with part set
  // and K split over z, split z stores its raw sums (before scale, bias and
  // activation) to part[(z * batch + b) * m + r] and no epilogue runs.
  float *part;
  // `sub` of a GEMM prologue given as such partials (sub_ks splits): sub[b][i]
  // = ((sum over z in order of sub_part[(z * batch + b) * k + i]) * sub_scale[i]
  // + sub_bias[i]) * sub_out_scale, null scale / bias meaning 1 / 0: the
  // producer's own epilogue, so the values are the ones it would have stored.
  const float *sub_part;
  const float *sub_scale;
  const float *sub_bias;
  float sub_out_scale;
  int sub_ks;
  // int8 digit planes of the normalised activations (the int8-MFMA GEMM):
  // a GEMM prologue writes them when xd is set, the GEMM reads them instead
  // of x.  Stream b's row is x = 2^(xe[b] - 30) (d0 2^24 + d1 2^16 + d2 2^8
  // + d3), plane d at xd[(d * batch + b) * k + i], xe[b] the exponent with
  // every |x| < 2^xe[b].
  int8_t *xd;
  int *xe;
};

// ---- coherent (agent-scope) or plain activation access ----
// A coherent load is a buffer load with the sc1 cache-policy bit: the
// instruction an agent-scope relaxed atomic load compiles to on gfx950 (it
// misses the XCD's own L2), but issued as a plain load, so the compiler can
// keep many in flight under one wait and use the 16-byte form.  Ordering with
// the phase barrier comes from the barrier's workgroup fence (__syncthreads).
// `base` must be the same in every lane of the wave (it becomes the buffer
// descriptor); `idx` is the per-lane element index, < 2^29.
constexpr int kCoherentSc1 = 16;  // cache-policy operand: sc1

__device__ __forceinline__ __amdgpu_buffer_rsrc_t coherent_rsrc(const void *base) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  // readfirstlane returns int: widen through uint32_t, never sign-extend
  const uint64_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a)));
  const uint64_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a >> 32)));
  // 0x00020000: 32-bit data format (raw buffer, no swizzle, no stride)
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void *>(hi << 32 | lo), static_cast<short>(0),
                                           0x7ffffff0, 0x00020000);
}

template <bool COH>
__device__ __forceinline__ float act_ld(const float *base, int idx) {
  if constexpr (COH) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(coherent_rsrc(base), idx * 4, 0,
                                                                          kCoherentSc1));
  } else {
    return gptr(base)[idx];
  }
}

// idx is a multiple of 4 (16-byte aligned element)
template <bool COH>
__device__ __forceinline__ float4 act_ld4(const float *base, int idx) {
  if constexpr (COH) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    const f32x4 v = __builtin_bit_cast(
        f32x4, __builtin_amdgcn_raw_buffer_load_b128(coherent_rsrc(base), idx * 4, 0, kCoherentSc1));
    return make_float4(v.x, v.y, v.z, v.w);
  } else {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    const f32x4 v = *gptr(reinterpret_cast<const f32x4 *>(base + idx));
    return make_float4(v.x, v.y, v.z, v.w);
  }
}

template <bool COH>
__device__ __forceinline__ void act_st(float *p, float v) {
  if constexpr (COH) {
    __hip_atomic_store(gptr_w(reinterpret_cast<unsigned int *>(p)), __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  } else {
    *gptr_w(p) = v;
  }
}

// Cross-lane butterflies without the LDS crossbar: DPP inside 16-lane rows
// (quad permutes, then the half-row and row mirrors, which pair the lanes of
// neighbouring groups once each group is uniform) and gfx950's permlane swaps
// across rows (permlane16_swap(v, v) hands a lane its neighbouring row's
// value in one result half and its own in the other).  After the steps for
// 2^k lanes, every lane of each aligned 2^k group holds op over the group; op
// must be commutative, which also makes every lane's result bit-identical.
template <int CTRL>
__device__ __forceinline__ float dpp_get(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}
template <int CTRL>
__device__ __forceinline__ int dpp_get_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true);
}
constexpr int kDppXor1 = 0xB1;    // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;    // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;

// op over aligned groups of 2^log2g lanes (log2g wave-uniform, 0..6).
template <typename Op>
__device__ __forceinline__ float group_reduce(float v, int log2g, Op op) {
  if (log2g >= 1) v = op(v, dpp_get<kDppXor1>(v));
  if (log2g >= 2) v = op(v, dpp_get<kDppXor2>(v));
  if (log2g >= 3) v = op(v, dpp_get<kDppHalfMirror>(v));
  if (log2g >= 4) v = op(v, dpp_get<kDppMirror>(v));
  if (log2g >= 5) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = op(__uint_as_float(r[0]), __uint_as_float(r[1]));
  }
  if (log2g >= 6) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = op(__uint_as_float(r[0]), __uint_as_float(r[1]));
  }
  return v;
}
struct OpAdd {
  __device__ float operator()(float a, float b) const { return a + b; }
};
struct OpMax {
  __device__ float operator()(float a, float b) const { return fmaxf(a, b); }
};
__device__ __forceinline__ float group_sum(float v, int log2g) { return group_reduce(v, log2g, OpAdd{}); }
// N independent group sums, level by level (one uniform branch per level).
template <int N>
__device__ __forceinline__ void group_sums(float (&v)[N], int log2g) {
  if (log2g >= 1)
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = v[i] + dpp_get<kDppXor1>(v[i]);
  if (log2g >= 2)
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = v[i] + dpp_get<kDppXor2>(v[i]);
  if (log2g >= 3)
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = v[i] + dpp_get<kDppHalfMirror>(v[i]);
  if (log2g >= 4)
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = v[i] + dpp_get<kDppMirror>(v[i]);
  if (log2g >= 5)
#pragma unroll
    for (int i = 0; i < N; i++) {
      const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[i]), __float_as_uint(v[i]), false, false);
      v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
  if (log2g >= 6)
#pragma unroll
    for (int i = 0; i < N; i++) {
      const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[i]), __float_as_uint(v[i]), false, false);
      v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
}
__device__ __forceinline__ float wave_sum(float v) { return group_reduce(v, 6, OpAdd{}); }
__device__ __forceinline__ float wave_max(float v) { return group_reduce(v, 6, OpMax{}); }

// Block-wide sums of N values over WPB waves with one barrier; `slot`
// alternates so back-to-back reductions never overwrite a slot still being
// read.  red holds 2 * 4 * kMaxWaves floats.
template <int WPB, int N>
__device__ __forceinline__ void block_sums(float (&v)[N], float *red, int &slot) {
#pragma unroll
  for (int i = 0; i < N; i++) v[i] = wave_sum(v[i]);
  if constexpr (WPB == 1) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  XE_LDS float *r = lptr(red) + slot * 4 * kMaxWaves;
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

// 16-byte streaming load (weights are read once per step: nontemporal).
__device__ __forceinline__ uint4 ld_nt16(const void *ptr) {
  const u32x4 v = __builtin_nontemporal_load(gptr(static_cast<const u32x4 *>(ptr)));
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
struct Chunk<XE_I4> {
  uint2 q;  // 16 nibbles, k order (nibble i of the 64 bits = element i)
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

// Zero a chunk's weights unless `keep` (a select, not a branch: a divergent
// branch around a load or its use makes the compiler wait for every load in
// flight, which serialises the weight stream).
__device__ __forceinline__ void mask_u4(uint4 &v, bool keep) {
  // per component: a select of whole vector objects is lowered through memory
  v.x = keep ? v.x : 0u;
  v.y = keep ? v.y : 0u;
  v.z = keep ? v.z : 0u;
  v.w = keep ? v.w : 0u;
}

template <int WT>
__device__ __forceinline__ void mask_chunk(Chunk<WT> &c, bool keep) {
  if constexpr (WT == XE_BF16) {
    mask_u4(c.lo, keep);
    mask_u4(c.hi, keep);
  } else if constexpr (WT == XE_I4) {
    c.q.x = keep ? c.q.x : 0u;
    c.q.y = keep ? c.q.y : 0u;
  } else {
    mask_u4(c.q, keep);
  }
}

// 8-byte streaming load (int4 chunks).
__device__ __forceinline__ uint2 ld_nt8(const void *ptr) {
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 v = __builtin_nontemporal_load(gptr(static_cast<const u32x2 *>(ptr)));
  return make_uint2(v.x, v.y);
}

template <int WT>
__device__ __forceinline__ void load_chunk(const GemvParams &p, int row, int c, Chunk<WT> &out) {
  if constexpr (WT == XE_I4) {
    const uint2 *base = reinterpret_cast<const uint2 *>(static_cast<const uint8_t *>(p.w) +
                                                        static_cast<size_t>(row) * (p.k / 2));
    out.q = ld_nt8(base + c);
  } else if constexpr (WT == XE_I8) {
    const uint4 *base = reinterpret_cast<const uint4 *>(static_cast<const int8_t *>(p.w) +
                                                        static_cast<size_t>(row) * p.k);
    out.q = ld_nt16(base + c);
  } else if constexpr (WT == XE_BFP16) {
    const uint4 *base = reinterpret_cast<const uint4 *>(static_cast<const int8_t *>(p.w) +
                                                        static_cast<size_t>(row) * p.k);
    out.q = ld_nt16(base + c);
    const uint16_t *eb = reinterpret_cast<const uint16_t *>(p.exps + static_cast<size_t>(row) * (p.k / 8));
    out.e = gptr(eb)[c];
  } else {
    const uint4 *base = reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(p.w) +
                                                        static_cast<size_t>(row) * p.k);
    out.lo = ld_nt16(base + 2 * c);
    out.hi = ld_nt16(base + 2 * c + 1);
  }
}

__device__ __forceinline__ float sb(uint32_t w, int j) {
  return static_cast<float>(static_cast<int>(static_cast<int8_t>(w >> (8 * j))));
}
// Signed nibble j of w (bits 4j..4j+3), the reference's ((v ^ 8) - 8).
__device__ __forceinline__ float sn(uint32_t w, int j) {
  // the builtin is typed unsigned: convert its sign-extended bits as int
  return static_cast<float>(static_cast<int>(__builtin_amdgcn_sbfe(static_cast<int>(w), 4 * j, 4)));
}

// acc += dot(chunk, x[16])
template <int WT>
__device__ __forceinline__ float chunk_dot(const Chunk<WT> &ch, const float4 (&xv)[4], float acc) {
  if constexpr (WT == XE_I4) {
    const uint32_t w2[2] = {ch.q.x, ch.q.y};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t w = w2[i / 2];
      const int j0 = 4 * (i & 1);
      acc = __builtin_fmaf(xv[i].x, sn(w, j0), acc);
      acc = __builtin_fmaf(xv[i].y, sn(w, j0 + 1), acc);
      acc = __builtin_fmaf(xv[i].z, sn(w, j0 + 2), acc);
      acc = __builtin_fmaf(xv[i].w, sn(w, j0 + 3), acc);
    }
    return acc;
  } else if constexpr (WT == XE_I8) {
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
    const uint32_t w8[8] = {ch.lo.x, ch.lo.y, ch.lo.z, ch.lo.w, ch.hi.x, ch.hi.y, ch.hi.z, ch.hi.w};
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

// LDS the GEMV needs: x rows + one staged sub row per batch row (floats).
__host__ __device__ inline size_t gemv_lds_floats(int nb, int k, bool sub) {
  return static_cast<size_t>(nb) * k * (sub ? 2 : 1);
}

// x rows sit in LDS as fp32 [b][K].  With more than one row (NB > 1) the
// four float4 words of each 16-element chunk are permuted by the chunk index:
// word j of chunk c is stored at float4 slot 4c + (j ^ ((c >> 2) & 3)).  A
// wave reads word j of the 16 consecutive chunks of its LPR lanes in one
// ds_read_b128; unpermuted, chunks c and c + 4 are 256 B apart and hit the
// same banks (4-way conflicts); with the permutation the 16 lanes cover all
// 64 banks once.  One row is read once per chunk and stays unpermuted (the
// address arithmetic would cost more than the conflicts).
template <int NB>
__host__ __device__ __forceinline__ int xs_word(int i4) { return NB > 1 ? i4 ^ ((i4 >> 4) & 3) : i4; }
template <int NB>
__host__ __device__ __forceinline__ int xs_elem(int e) { return 4 * xs_word<NB>(e >> 2) + (e & 3); }

// Block-wide sums of N values over WPB waves with one barrier (red holds
// 2 * kRedN * kMaxWaves floats, N <= kRedN; `slot` alternates as in
// block_sums).  Each value: its wave's sum, then the waves' sums in wave
// order.
constexpr int kRedN = 32;
template <int WPB, int N>
__device__ __forceinline__ void block_sums_wide(float (&v)[N], float *red, int &slot) {
  static_assert(N <= kRedN, "too many sums");
#pragma unroll
  for (int i = 0; i < N; i++) v[i] = wave_sum(v[i]);
  if constexpr (WPB == 1) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  XE_LDS float *r = lptr(red) + slot * kRedN * kMaxWaves;
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

// Prologue: x (+ post(sub)) -> res_out (the writer workgroup) -> norm -> LDS,
// fp32, for every batch row at once (one load round, one reduction per
// statistic for all rows); rows past the batch are zero in LDS, so the main
// loop reads them without a branch.  Statistics:
//   Gemma (sub + post_w, RMS1P): t = x + sub*inv_s*(1+w) and
//     sum t^2 = sum x^2 + 2 inv_s sum x*s' + inv_s^2 sum s'^2 (s' = sub*(1+w)),
//     so sum sub^2, sum x^2, sum x*s', sum s'^2 come out of one reduction.
//   LayerNorm: two passes (sum t, then sum (t - mean)^2) as the reference's
//     layer_norm (npu-asr-host/src/lib.rs:79-109); one-pass variance loses
//     everything on near-constant rows.
// Per row, each thread accumulates its elements in the same order as the
// batched GEMM's prologue kernels (gemm.hip), so both give the same bits.
// red: 2 * kRedN * kMaxWaves floats.
template <int NB, int WPB>
__device__ __forceinline__ void gemv_prologue(const GemvParams &p, float4 *xs4, float *red, bool writer) {
  constexpr int kThreads = 64 * WPB;
  // float4 loads in flight per thread and row (the per-thread element order,
  // t, t + kThreads, ..., does not depend on it)
  constexpr int UNR = NB >= 4 ? 1 : NB == 2 ? 2 : 4;
  const int K = p.k, K4 = K / 4;
  const int nb = p.batch < NB ? p.batch : NB;
  const float fk = static_cast<float>(K);
  float *xs = reinterpret_cast<float *>(xs4);
  float *sb = xs + static_cast<size_t>(NB) * K;  // sub staging [NB][K] (unpermuted)
  const bool fold = p.sub && p.post_w;            // Gemma post-norm + residual
  int slot = 0;
  // ---- loads: raw x (and sub) to LDS; the fold's four sums per row ----
  float acc[NB][4];
#pragma unroll
  for (int b = 0; b < NB; b++)
#pragma unroll
    for (int q = 0; q < 4; q++) acc[b][q] = 0.f;
  for (int i0 = threadIdx.x; i0 < K4; i0 += kThreads * UNR) {
    float4 v[NB][UNR], sv[NB][UNR];
#pragma unroll
    for (int b = 0; b < NB; b++) {
      if (b >= nb) break;
      const float *xrow = static_cast<const float *>(p.x) + static_cast<size_t>(b) * p.ldx;
      const float *subr = p.sub ? p.sub + static_cast<size_t>(b) * K : nullptr;
#pragma unroll
      for (int u = 0; u < UNR; u++) {
        const int i = i0 + u * kThreads;
        if (i < K4) {
          if (p.x_bf16) {
            const uint2 r = reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(p.x) +
                                                            static_cast<size_t>(b) * p.ldx)[i];
            v[b][u] = make_float4(__uint_as_float(r.x << 16), __uint_as_float(r.x & 0xffff0000u),
                                  __uint_as_float(r.y << 16), __uint_as_float(r.y & 0xffff0000u));
          } else {
            v[b][u] = act_ld4<false>(xrow, 4 * i);
          }
          if (subr) sv[b][u] = act_ld4<false>(subr, 4 * i);
        }
      }
    }
#pragma unroll
    for (int b = 0; b < NB; b++) {
      if (b >= nb) break;
#pragma unroll
      for (int u = 0; u < UNR; u++) {
        const int i = i0 + u * kThreads;
        if (i >= K4) continue;
        xs4[static_cast<size_t>(b) * K4 + xs_word<NB>(i)] = v[b][u];
        if (p.sub) reinterpret_cast<float4 *>(sb)[static_cast<size_t>(b) * K4 + i] = sv[b][u];
        if (fold) {
          const float4 w = reinterpret_cast<const float4 *>(p.post_w)[i];
          const float xv[4] = {v[b][u].x, v[b][u].y, v[b][u].z, v[b][u].w};
          const float su[4] = {sv[b][u].x, sv[b][u].y, sv[b][u].z, sv[b][u].w};
          const float wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
          for (int j = 0; j < 4; j++) {
            const float sp = su[j] * (1.0f + wv[j]);
            acc[b][0] = __builtin_fmaf(su[j], su[j], acc[b][0]);
            acc[b][1] = __builtin_fmaf(xv[j], xv[j], acc[b][1]);
            acc[b][2] = __builtin_fmaf(xv[j], sp, acc[b][2]);
            acc[b][3] = __builtin_fmaf(sp, sp, acc[b][3]);
          }
        }
      }
    }
  }
  // rows past the batch: zeros (read by the branch-free main loop)
  for (int i = threadIdx.x; i < (NB - nb) * K4; i += kThreads)
    xs4[static_cast<size_t>(nb) * K4 + i] = make_float4(0.f, 0.f, 0.f, 0.f);
  float inv_t[NB];
  if (fold) {
    float sums[NB * 4];
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
      for (int q = 0; q < 4; q++) sums[4 * b + q] = acc[b][q];
    block_sums_wide<WPB, NB * 4>(sums, red, slot);
    float inv_s[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) {
      inv_s[b] = 1.0f / sqrtf(sums[4 * b] / fk + p.eps);
      const float st2 = sums[4 * b + 1] + 2.0f * inv_s[b] * sums[4 * b + 2] + inv_s[b] * inv_s[b] * sums[4 * b + 3];
      inv_t[b] = p.norm != XE_NORM_NONE ? 1.0f / sqrtf(fmaxf(st2, 0.f) / fk + p.eps) : 1.f;
    }
    __syncthreads();  // staging complete (block_sums_wide skips its barrier for one wave)
    for (int i = threadIdx.x; i < K; i += kThreads) {
      const int pi = xs_elem<NB>(i);
      const float pw = 1.0f + p.post_w[i];
      const float g = p.norm == XE_NORM_RMS1P ? 1.0f + p.gamma[i] : p.norm == XE_NORM_RMS ? p.gamma[i] : 0.f;
#pragma unroll
      for (int b = 0; b < NB; b++) {
        if (b >= nb) break;
        float *xb = xs + static_cast<size_t>(b) * K;
        const float t = xb[pi] + sb[static_cast<size_t>(b) * K + i] * inv_s[b] * pw;
        if (p.res_out && writer) act_st<false>(p.res_out + static_cast<size_t>(b) * K + i, t);
        float h = t;
        if (p.norm == XE_NORM_RMS1P || p.norm == XE_NORM_RMS) h = t * inv_t[b] * g;
        xb[pi] = h;
      }
    }
    if (p.norm == XE_NORM_LN) {  // not a model combination; kept exact anyway
      __syncthreads();
      float mean[NB], v1[NB];
#pragma unroll
      for (int b = 0; b < NB; b++) v1[b] = 0.f;
      for (int i = threadIdx.x; i < K; i += kThreads)
#pragma unroll
        for (int b = 0; b < NB; b++) v1[b] += xs[static_cast<size_t>(b) * K + xs_elem<NB>(i)];
      block_sums_wide<WPB, NB>(v1, red, slot);
#pragma unroll
      for (int b = 0; b < NB; b++) {
        mean[b] = v1[b] / fk;
        v1[b] = 0.f;
      }
      for (int i = threadIdx.x; i < K; i += kThreads)
#pragma unroll
        for (int b = 0; b < NB; b++) {
          const float c = xs[static_cast<size_t>(b) * K + xs_elem<NB>(i)] - mean[b];
          v1[b] = __builtin_fmaf(c, c, v1[b]);
        }
      block_sums_wide<WPB, NB>(v1, red, slot);
      __syncthreads();
      for (int i = threadIdx.x; i < K; i += kThreads) {
        const int pi = xs_elem<NB>(i);
#pragma unroll
        for (int b = 0; b < NB; b++) {
          if (b >= nb) break;
          float *xb = xs + static_cast<size_t>(b) * K;
          xb[pi] = (xb[pi] - mean[b]) * (1.0f / sqrtf(v1[b] / fk + p.eps)) * p.gamma[i] + p.beta[i];
        }
      }
    }
  } else {
    __syncthreads();
    if (p.sub) {
      for (int i = threadIdx.x; i < K; i += kThreads) {
        const int pi = xs_elem<NB>(i);
#pragma unroll
        for (int b = 0; b < NB; b++) {
          if (b >= nb) break;
          float *xb = xs + static_cast<size_t>(b) * K;
          const float t = xb[pi] + sb[static_cast<size_t>(b) * K + i];
          xb[pi] = t;
          if (p.res_out && writer) act_st<false>(p.res_out + static_cast<size_t>(b) * K + i, t);
        }
      }
      if (p.norm != XE_NORM_NONE) __syncthreads();
    }
    if (p.norm == XE_NORM_LN) {
      float mean[NB], v1[NB];
#pragma unroll
      for (int b = 0; b < NB; b++) v1[b] = 0.f;
      for (int i = threadIdx.x; i < K; i += kThreads)
#pragma unroll
        for (int b = 0; b < NB; b++) v1[b] += xs[static_cast<size_t>(b) * K + xs_elem<NB>(i)];
      block_sums_wide<WPB, NB>(v1, red, slot);
#pragma unroll
      for (int b = 0; b < NB; b++) {
        mean[b] = v1[b] / fk;
        v1[b] = 0.f;
      }
      for (int i = threadIdx.x; i < K; i += kThreads)
#pragma unroll
        for (int b = 0; b < NB; b++) {
          const float c = xs[static_cast<size_t>(b) * K + xs_elem<NB>(i)] - mean[b];
          v1[b] = __builtin_fmaf(c, c, v1[b]);
        }
      block_sums_wide<WPB, NB>(v1, red, slot);
      float inv[NB];
#pragma unroll
      for (int b = 0; b < NB; b++) inv[b] = 1.0f / sqrtf(v1[b] / fk + p.eps);
      for (int i = threadIdx.x; i < K; i += kThreads) {
        const int pi = xs_elem<NB>(i);
        const float g = p.gamma[i], be = p.beta[i];
#pragma unroll
        for (int b = 0; b < NB; b++) {
          if (b >= nb) break;
          float *xb = xs + static_cast<size_t>(b) * K;
          xb[pi] = (xb[pi] - mean[b]) * inv[b] * g + be;
        }
      }
    } else if (p.norm != XE_NORM_NONE) {
      float v1[NB];
#pragma unroll
      for (int b = 0; b < NB; b++) v1[b] = 0.f;
      for (int i = threadIdx.x; i < K; i += kThreads)
#pragma unroll
        for (int b = 0; b < NB; b++) {
          const float x = xs[static_cast<size_t>(b) * K + xs_elem<NB>(i)];
          v1[b] = __builtin_fmaf(x, x, v1[b]);
        }
      block_sums_wide<WPB, NB>(v1, red, slot);
      float inv[NB];
#pragma unroll
      for (int b = 0; b < NB; b++) inv[b] = 1.0f / sqrtf(v1[b] / fk + p.eps);
      for (int i = threadIdx.x; i < K; i += kThreads) {
        const int pi = xs_elem<NB>(i);
        const float g = p.norm == XE_NORM_RMS1P ? 1.0f + p.gamma[i] : p.gamma[i];
#pragma unroll
        for (int b = 0; b < NB; b++) {
          if (b >= nb) break;
          float *xb = xs + static_cast<size_t>(b) * K;
          xb[pi] = xb[pi] * inv[b] * g;
        }
      }
    }
  }
  __syncthreads();
}

// Row tiles first_tile, first_tile + stride, ... of one GEMV; the first
// tile's weight loads are issued before the prologue.
template <int WT, int NB, int LPR, int RPL, int WPB>
__device__ __forceinline__ void gemv_tiles(const GemvParams &p, float4 *xs4, float *red, int first_tile, int stride,
                           bool writer) {
  constexpr int RG = 64 / LPR;
  // Chunks per row in one load set.  Two sets are in flight (ping-pong).
  constexpr int U = (RPL >= 2) ? 2 : 4;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rg = lane / LPR, kl = lane % LPR;
  constexpr int rows_per_wave = RG * RPL;
  constexpr int rows_per_block = WPB * rows_per_wave;
  const int K = p.k, nch = K / 16;
  const int n_it = (nch + LPR - 1) / LPR;
  const int ntiles = (p.m + rows_per_block - 1) / rows_per_block;
  const int K4 = K / 4;

  if (first_tile >= ntiles) return;
  for (int tile = first_tile; tile < ntiles; tile += stride) {
    const int row0 = tile * rows_per_block + wave * rows_per_wave + rg * RPL;
    bool row_ok[RPL];
    int row[RPL];
#pragma unroll
    for (int i = 0; i < RPL; i++) {
      row[i] = row0 + i;
      row_ok[i] = row[i] < p.m;
      if (!row_ok[i]) row[i] = p.m - 1;  // clamp: loads stay in bounds, result dropped
    }

    // Load set s covers chunk iterations [s*U, s*U + U).
    Chunk<WT> ca[U][RPL], cb[U][RPL];
    // Chunk iterations past n_it are skipped (a uniform branch); lanes past
    // the row's last chunk load a clamped chunk and zero it at use.
    auto load_set = [&](Chunk<WT>(&dst)[U][RPL], int it0) {
#pragma unroll
      for (int u = 0; u < U; u++) {
        if (it0 + u < n_it) {
          const int c = min((it0 + u) * LPR + kl, nch - 1);
#pragma unroll
          for (int i = 0; i < RPL; i++) load_chunk<WT>(p, row[i], c, dst[u][i]);
        }
      }
    };
    load_set(ca, 0);
    if (U < n_it) load_set(cb, U);
    if (tile == first_tile) gemv_prologue<NB, WPB>(p, xs4, red, writer);

    float acc[NB][RPL];
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
      for (int i = 0; i < RPL; i++) acc[b][i] = 0.f;

    // every row of the batch tile, without a branch on the batch count:
    // LDS rows past the batch are zero and their sums are dropped
    auto compute = [&](const Chunk<WT>(&chs)[RPL], int c) {
      const int sw = NB > 1 ? (c >> 2) & 3 : 0;  // the chunk's word permutation (xs_word)
#pragma unroll
      for (int b = 0; b < NB; b++) {
        float4 xv[4];
        const float4 *xr = xs4 + static_cast<size_t>(b) * K4 + 4 * c;
#pragma unroll
        for (int j = 0; j < 4; j++) xv[j] = xr[j ^ sw];
#pragma unroll
        for (int i = 0; i < RPL; i++) acc[b][i] = chunk_dot<WT>(chs[i], xv, acc[b][i]);
      }
    };

    auto compute_set = [&](const Chunk<WT>(&src)[U][RPL], int it0) {
#pragma unroll
      for (int u = 0; u < U; u++) {
        if (it0 + u < n_it) {
          const int c = (it0 + u) * LPR + kl;
          Chunk<WT> ch[RPL];
#pragma unroll
          for (int i = 0; i < RPL; i++) {
            ch[i] = src[u][i];
            mask_chunk<WT>(ch[i], c < nch);
          }
          compute(ch, min(c, nch - 1));
        }
      }
    };
    // ping-pong: while one set is consumed the other is in flight
    for (int it = 0; it < n_it; it += 2 * U) {
      compute_set(ca, it);
      if (it + 2 * U < n_it) load_set(ca, it + 2 * U);
      if (it + U < n_it) {
        compute_set(cb, it + U);
        if (it + 3 * U < n_it) load_set(cb, it + 3 * U);
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
          if (WT == XE_I8 || WT == XE_I4) t = t * gptr(p.scale)[row[i]];
          if (p.bias) t = t + gptr(p.bias)[row[i]];
          v[i] = t;
        }
        if (p.act == ACT_GEGLU_TANH) {
#pragma unroll
          for (int i = 0; i + 1 < RPL; i += 2)
            if (row_ok[i])
              act_st<false>(p.y + static_cast<size_t>(b) * p.ldy + row[i] / 2,
                          gelu_tanh(v[i]) * v[i + 1] * p.out_scale);
        } else {
#pragma unroll
          for (int i = 0; i < RPL; i++) {
            if (!row_ok[i]) continue;
            float t = v[i];
            if (p.act == ACT_RELU) t = t > 0.f ? t : 0.f;
            else if (p.act == ACT_GELU_ERF) t = gelu_erf(t);
            act_st<false>(p.y + static_cast<size_t>(b) * p.ldy + row[i], t * p.out_scale);
          }
        }
      }
    }
  }
}

// ---- host: tile choice (shared by the standalone kernel and the step kernel) ----
struct Tile {
  int lpr, rpl, wpb;
};

int cu_count();
Tile choose_tile(int m, int k, int act);
GemvParams to_params(const GemvLaunch &L);

}  // namespace gdev
}  // namespace xe
