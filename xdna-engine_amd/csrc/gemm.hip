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
// Two kernels share these operand rules:
//   gemm_ks_kernel (the decoder's projections): a workgroup tile of 16, 32 or
//   64 weight rows x 64 streams whose four waves split every 128-k step; each
//   lane loads its own operands straight into registers, and the waves'
//   partial tiles meet in LDS once, after the K loop.
//   gemm_kernel (outputs too wide for one workgroup a CU: the lm-head): 4
//   waves, 64 * MB weight rows x 64 streams, K in steps of 64; the
//   activation tile of a step is staged in LDS as its three parts, the next
//   step's weights and activations are loaded before the current step's
//   MFMAs.  Within a lane's 16 contiguous k the two MFMAs of a step take k
//   0..7 and 8..15: the A and B operands use the same k permutation, so the
//   dot products are unchanged.
// Both split K across workgroups when the tiles leave most CUs idle.
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

constexpr int kBN = 64, kBK = 64;
constexpr int kGT = 256;             // threads
constexpr int kXS = kBK + 8;         // LDS row stride (bf16) of a staged part
constexpr int kNoRec = 0x7ffffff0;  // past every buffer: loads return zeros
constexpr size_t kGemmWsFloats = size_t(8) << 20;  // split-K partials (32 MB)
constexpr size_t kGemmMaxTiles = 8192;     // split-K output tiles (counters)
constexpr int kMaxSplitsK = 16;            // splits of one GEMM

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
  if constexpr (WT == XE_I4) {
    // 16 nibbles (8 bytes) of row `row` from element k (k a multiple of 16)
    typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 v = __builtin_bit_cast(
        u32x2, __builtin_amdgcn_raw_buffer_load_b64(rw, ok ? row * (K / 2) + k / 2 : kNoRec, 0, 2));
    o.q = u32x4{v.x, v.y, 0u, 0u};
  } else if constexpr (WT == XE_BF16) {
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
  } else if constexpr (WT == XE_I4) {
    // signed nibbles (at most 4 significant bits: exact in bf16), k order
    const uint32_t d[2] = {w.q.x, w.q.y};
    uint32_t p[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const uint32_t word = d[i / 4];
      const int j = 2 * (i & 3);
      const float f0 = static_cast<float>(static_cast<int>(__builtin_amdgcn_sbfe(static_cast<int>(word), 4 * j, 4)));
      const float f1 = static_cast<float>(static_cast<int>(__builtin_amdgcn_sbfe(static_cast<int>(word), 4 * j + 4, 4)));
      p[i] = pack_hi16(f0, f1);
    }
    a0 = __builtin_bit_cast(bf16x8, u32x4{p[0], p[1], p[2], p[3]});
    a1 = __builtin_bit_cast(bf16x8, u32x4{p[4], p[5], p[6], p[7]});
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

// Row scales and biases of rows r0 .. r0 + 3 (1 and 0 where absent).
struct RowQuad {
  float s[4], b[4];
};

__device__ __forceinline__ RowQuad load_quad(const gdev::GemvParams &p, int wdtype, int r0) {
  RowQuad q;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int r = min(r0 + i, p.m - 1);
    q.s[i] = (wdtype == XE_I8 || wdtype == XE_I4) ? p.scale[r] : 1.0f;
    q.b[i] = p.bias ? p.bias[r] : 0.0f;
  }
  return q;
}

// Epilogue of rows r0 .. r0 + 3 (a GeGLU pair each half) of stream b, with
// their scales and biases already loaded.
__device__ __forceinline__ void epilogue4(const gdev::GemvParams &p, const RowQuad &rq, int r0, int b,
                                          const float (&acc)[4]) {
  float t[4];
#pragma unroll
  for (int i = 0; i < 4; i++) t[i] = acc[i] * rq.s[i] + rq.b[i];
  float *yrow = p.y + static_cast<size_t>(b) * p.ldy;
  if (p.act == ACT_GEGLU_TANH) {
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

__device__ __forceinline__ void epilogue4(const gdev::GemvParams &p, int wdtype, int r0, int b, const float (&acc)[4]) {
  epilogue4(p, load_quad(p, wdtype, r0), r0, b, acc);
}

// This thread's 16 activations (row srow, k sk .. sk + 15 of the step) split
// into three bf16 parts by truncation, x = hi + mid + lo exactly, stored in
// the LDS tile of each part.
__device__ __forceinline__ void stage_parts(const f32x4 (&x)[4], uint16_t (*xs)[kBN * kXS], int srow, int sk) {
  uint32_t hp[8], mp[8], lp[8];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const float v[4] = {x[i].x, x[i].y, x[i].z, x[i].w};
    float h[4], m[4], l[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
      h[q] = trunc_bf16(v[q]);
      const float r = v[q] - h[q];
      m[q] = trunc_bf16(r);
      l[q] = trunc_bf16(r - m[q]);
    }
    hp[2 * i] = pack_hi16(h[0], h[1]);
    hp[2 * i + 1] = pack_hi16(h[2], h[3]);
    mp[2 * i] = pack_hi16(m[0], m[1]);
    mp[2 * i + 1] = pack_hi16(m[2], m[3]);
    lp[2 * i] = pack_hi16(l[0], l[1]);
    lp[2 * i + 1] = pack_hi16(l[2], l[3]);
  }
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

// Split-K tail, after every wave of the workgroup has stored its partial
// tile ws[tile][z][b][r] with agent-scope stores: the workgroup counts itself
// in cnt[tile]; the last one to arrive adds the partials in split order (the
// same order on every run), runs the epilogue and re-arms the counter.
template <int WT, int BM, int BN = kBN>
// rq: this thread's row quad, prefetched (its q is the same in every item
// the thread takes), or null.  BN: streams a tile.
__device__ __forceinline__ void splitk_finish(const gdev::GemvParams &p, float *ws, unsigned *cnt, int tile, int ks,
                                              int nb, int m0, int b0, int &last, const RowQuad *rq = nullptr) {
  __builtin_amdgcn_s_waitcnt(0);  // this wave's partial stores have completed
  __syncthreads();
  if (threadIdx.x == 0)
    last = __hip_atomic_fetch_add(cnt + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == static_cast<unsigned>(ks - 1);
  __syncthreads();
  if (!last) return;
  // the reduction: item = (stream bb, row quad q), two items a thread per
  // round; every split's partial of both items in flight at once (ks <=
  // kMaxSplitsK), then summed in split order
  const __amdgpu_buffer_rsrc_t rws = gdev::coherent_rsrc(ws + static_cast<size_t>(tile) * ks * (BM * BN));
  const int items = nb * (BM / 4);
  for (int it0 = threadIdx.x; it0 < items; it0 += 2 * kGT) {
    f32x4 v[2][kMaxSplitsK];
#pragma unroll
    for (int r = 0; r < 2; r++) {
      const int it = it0 + r * kGT;
      const int bb = it / (BM / 4), q = it % (BM / 4);
#pragma unroll
      for (int zz = 0; zz < kMaxSplitsK; zz++)
        v[r][zz] = __builtin_bit_cast(
            f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                       rws, zz < ks && it < items ? ((zz * BN + bb) * BM + 4 * q) * 4 : kNoRec, 0, gdev::kCoherentSc1));
    }
#pragma unroll
    for (int r = 0; r < 2; r++) {
      const int it = it0 + r * kGT;
      if (it >= items) continue;
      const int bb = it / (BM / 4), q = it % (BM / 4);
      float sum[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int zz = 0; zz < kMaxSplitsK; zz++) {
        if (zz < ks) {
          sum[0] += v[r][zz].x;
          sum[1] += v[r][zz].y;
          sum[2] += v[r][zz].z;
          sum[3] += v[r][zz].w;
        }
      }
      if (rq) epilogue4(p, *rq, m0 + 4 * q, b0 + bb, sum);
      else epilogue4(p, WT, m0 + 4 * q, b0 + bb, sum);
    }
  }
  if (threadIdx.x == 0) __hip_atomic_store(cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Split-K: blockIdx.z takes K steps [z * spk, (z + 1) * spk).  With more than
// one split, each workgroup stores its partial tile (agent-scope stores) in
// ws[tile][z][b][r] and counts itself in cnt[tile]; the last one to arrive
// adds the partials in split order (the same order on every run) and runs
// the epilogue, then re-arms the counter for the next launch.
// MB: MFMA row blocks per wave (the wave's 16 * MB weight rows share each
// activation fragment read from LDS); a workgroup covers 64 * MB rows.
template <int WT, int MB>
__global__ __launch_bounds__(kGT) __attribute__((amdgpu_waves_per_eu(2))) void gemm_kernel(gdev::GemvParams p, float *ws, unsigned *cnt, int spk) {
  constexpr int BM = 64 * MB;
  // two buffers (step parity) x three parts x [kBN][kXS] bf16
  __shared__ __attribute__((aligned(16))) uint16_t xs[2][3][kBN * kXS];
  __shared__ int last;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int m0 = blockIdx.x * BM, b0 = blockIdx.y * kBN;
  const int K = p.k;
  const int ks = gridDim.z, z = blockIdx.z;
  const int step0 = z * spk;
  const int nsteps = min((K + kBK - 1) / kBK, step0 + spk) - step0;
  const int nb = min(kBN, p.batch - b0);
  const __amdgpu_buffer_rsrc_t rw = gdev::coherent_rsrc(p.w);
  const __amdgpu_buffer_rsrc_t re = gdev::coherent_rsrc(WT == XE_BFP16 ? static_cast<const void *>(p.exps) : p.w);
  const __amdgpu_buffer_rsrc_t rx = gdev::coherent_rsrc(p.x);

  // this lane's weight rows (one per row block) and k offset within a step
  const int wbase = m0 + wave * 16 * MB + (lane & 15);
  const int wk = 16 * (lane >> 4);
  // activation staging: thread t stages row t / 4, k (t % 4) * 16 .. + 16
  const int srow = threadIdx.x >> 2, sk = (threadIdx.x & 3) * 16;

  // pipeline of NS stages: the weights and activations of the next NS - 1
  // steps are in flight while a step computes (b = 64 probe, QKV / O /
  // gate-up / down: 12.9 / 12.5 / 20.5 / 18.9 us at two stages, 13.3 / 13.0
  // / 21.2 / 19.5 at three, 13.5 / 13.2 / 21.6 / 20.1 at four: with two
  // waves per SIMD the other wave covers the latency the deeper stages would)
  constexpr int NS = 2;
  struct Stage {
    WLoad<WT> w[MB];
    f32x4 x[4];
  };
  // k at or past xlim reads zeros: one per-lane bound folds "row exists" and
  // "k inside this split" into one compare (a separate loop-invariant flag
  // gets the loads unswitched into branches that wait for every load in
  // flight)
  const int kend = min(K, (step0 + nsteps) * kBK);
  const int xlim = srow < nb ? kend : 0;
  const int xrow = (b0 + srow) * p.ldx;
  auto issue = [&](int step, Stage &st) {
    const int k = (step0 + step) * kBK + sk;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int off = k + 4 * i < xlim ? (xrow + k + 4 * i) * 4 : kNoRec;
      st.x[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0));
    }
    const int kw = (step0 + step) * kBK + wk;
#pragma unroll
    for (int mb = 0; mb < MB; mb++) {
      const int row = wbase + 16 * mb;
      load_w<WT>(rw, re, row, kw, row < p.m && kw < kend, K, st.w[mb]);
    }
  };

  f32x4 acc[MB][4];
#pragma unroll
  for (int mb = 0; mb < MB; mb++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[mb][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Step s stages into LDS buffer s & 1 and reads it after one barrier: a
  // wave writes buffer s & 1 only after the barrier of step s - 1, which
  // every wave reaches after its reads of step s - 2.  Column blocks past the
  // batch hold zeros (their rows load as zeros) and are computed anyway: a
  // uniform branch per block keeps the scheduler from hoisting the reads.
  auto compute = [&](int step, const Stage &st) {
    uint16_t(*xb)[kBN * kXS] = xs[step & 1];
    stage_parts(st.x, xb, srow, sk);
    __syncthreads();
    bf16x8 a0[MB], a1[MB];
#pragma unroll
    for (int mb = 0; mb < MB; mb++) to_bf16<WT>(st.w[mb], a0[mb], a1[mb]);
    // a part's eight fragments are read before its MFMAs (all reads in
    // flight at once); with one row block the next part's reads also go out
    // before the current part's MFMAs (more row blocks: the registers are
    // worth more than the overlap)
    constexpr int RA = MB == 1 ? 2 : 1;
    bf16x8 bx[RA][4][2];
    auto rd = [&](int part, bf16x8(&d)[4][2]) {
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint16_t *src = xb[part] + (16 * j + (lane & 15)) * kXS + wk;
        d[j][0] = *reinterpret_cast<const bf16x8 *>(src);
        d[j][1] = *reinterpret_cast<const bf16x8 *>(src + 8);
      }
    };
    if constexpr (RA == 2) rd(0, bx[0]);
#pragma unroll
    for (int part = 0; part < 3; part++) {
      if constexpr (RA == 2) {
        if (part < 2) rd(part + 1, bx[(part + 1) & 1]);
      } else {
        rd(part, bx[0]);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int h = 0; h < 2; h++)
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
          for (int mb = 0; mb < MB; mb++)
            acc[mb][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(h ? a1[mb] : a0[mb], bx[part % RA][j][h],
                                                                  acc[mb][j], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Whole groups of NS steps, then the remainder (its stages are already in
  // flight).  No step inside the loop is conditional: a conditional step
  // makes the compiler wait for every load in flight at the loop's head.
  Stage sg[NS];
#pragma unroll
  for (int j = 0; j < NS - 1; j++) issue(j, sg[j]);
  int s0 = 0;
  for (; s0 + NS <= nsteps; s0 += NS) {
#pragma unroll
    for (int j = 0; j < NS; j++) {
      issue(s0 + j + NS - 1, sg[(j + NS - 1) % NS]);
      compute(s0 + j, sg[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < NS - 1; j++)
    if (s0 + j < nsteps) compute(s0 + j, sg[j]);

  // lane holds rows rl(mb) + i (i = 0..3) of column block j's stream
  if (ks == 1) {
#pragma unroll
    for (int mb = 0; mb < MB; mb++) {
      const int rl = wave * 16 * MB + 16 * mb + 4 * (lane >> 4);
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int b = 16 * j + (lane & 15);
        if (b >= nb) continue;
        const float a4[4] = {acc[mb][j][0], acc[mb][j][1], acc[mb][j][2], acc[mb][j][3]};
        epilogue4(p, WT, m0 + rl, b0 + b, a4);
      }
    }
    return;
  }
  const int tile = blockIdx.y * gridDim.x + blockIdx.x;
  float *part = ws + (static_cast<size_t>(tile) * ks + z) * (BM * kBN);
#pragma unroll
  for (int mb = 0; mb < MB; mb++) {
    const int rl = wave * 16 * MB + 16 * mb + 4 * (lane >> 4);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int b = 16 * j + (lane & 15);
#pragma unroll
      for (int i = 0; i < 4; i++)
        __hip_atomic_store(part + b * BM + rl + i, acc[mb][j][i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  splitk_finish<WT, BM>(p, ws, cnt, tile, ks, nb, m0, b0, last);
}

// ---- int8 weights x int8 digit planes on v_mfma_i32_16x16x64_i8 ----
//
// For int8 weights whose activations come out of a GEMM prologue (the norm
// in front of the lm-head): the prologue writes each stream's row as four
// signed base-256 digit planes of rint(x 2^(30 - E)) (GemvParams::xd / xe),
// so that
//   sum_k W[m][k] x[k] = 2^(E - 30) (C0 2^24 + C1 2^16 + C2 2^8 + C3),
//   C_d = sum_k W[m][k] d_k[k]   (exact in int32: |W| <= 127, |d| <= 128).
// The int8 weights are the MFMA A operand as stored (no conversion) and each
// digit plane a B operand: 4 MFMAs a 16 x 16 x 64 block, against 6 for the
// three bf16 parts of the fp32 path.  The four sums combine exactly in fp64
// and round once to fp32: the exact dot product of x rounded to 2^(E - 31),
// i.e. to 2^-30 of the stream's largest |x| (fp32 itself keeps 2^-24 of each
// element).  Workgroup: 8 waves of 32 weight rows (two 16-row blocks) x 64
// streams, K in steps of 64 whose digit planes are staged in LDS
// (double-buffered, one barrier a step); the next step's weights and digits
// are loaded before the current step's MFMAs.
constexpr int kI8MB = 2;   // 16-row blocks a wave
constexpr int kI8W = 8;    // waves a workgroup
constexpr int kI8T = 64 * kI8W;
constexpr int kI8XS = 80;  // LDS row stride (bytes) of a staged 64-k digit row: conflict-free 16-byte reads

__global__ __launch_bounds__(kI8T) __attribute__((amdgpu_waves_per_eu(2))) void gemm_i8_kernel(gdev::GemvParams p) {
  typedef int i32x4 __attribute__((ext_vector_type(4)));
  typedef int i32x2 __attribute__((ext_vector_type(2)));
  constexpr int MB = kI8MB, BM = 16 * kI8W * MB;
  __shared__ __attribute__((aligned(16))) int8_t xs[2][4][kBN * kI8XS];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int m0 = blockIdx.x * BM, b0 = blockIdx.y * kBN;
  const int K = p.k;
  const int nsteps = (K + 63) / 64;
  const int nb = min(kBN, p.batch - b0);
  const __amdgpu_buffer_rsrc_t rw = gdev::coherent_rsrc(p.w);
  const __amdgpu_buffer_rsrc_t rx = gdev::coherent_rsrc(p.xd);
  // A operand: this lane's rows (one a row block), k 16 (lane / 16) .. + 16
  // of the step; B operand: stream lane % 16 of a block, the same k
  const int wbase = m0 + wave * 16 * MB + (lane & 15);
  const int wk = 16 * (lane >> 4);
  // staging: thread t -> stream t / 8, k 8 (t % 8) .. + 8, all four planes
  const int srow = threadIdx.x >> 3, sk = 8 * (threadIdx.x & 7);
  const int plane = p.batch * K;
  struct Stage {
    i32x4 w[MB];
    i32x2 x[4];
  };
  auto issue = [&](int step, Stage &st) {
    const int k0 = step * 64;
    const bool xok = srow < nb && k0 + sk < K;
#pragma unroll
    for (int d = 0; d < 4; d++)
      st.x[d] = __builtin_bit_cast(
          i32x2, __builtin_amdgcn_raw_buffer_load_b64(rx, xok ? d * plane + (b0 + srow) * K + k0 + sk : kNoRec, 0, 0));
#pragma unroll
    for (int mb = 0; mb < MB; mb++) {
      const int row = wbase + 16 * mb;
      st.w[mb] = __builtin_bit_cast(
          i32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, row < p.m && k0 + wk < K ? row * K + k0 + wk : kNoRec, 0, 2));
    }
  };
  i32x4 acc[MB][4][4];
#pragma unroll
  for (int mb = 0; mb < MB; mb++)
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int d = 0; d < 4; d++) acc[mb][j][d] = i32x4{0, 0, 0, 0};
  // step s stages into buffer s & 1 and reads it after one barrier (a wave
  // writes buffer s & 1 only after the barrier of step s - 1, which every
  // wave reaches after its reads of step s - 2)
  auto compute = [&](int step, const Stage &st) {
    int8_t(*xb)[kBN * kI8XS] = xs[step & 1];
#pragma unroll
    for (int d = 0; d < 4; d++) *reinterpret_cast<i32x2 *>(&xb[d][srow * kI8XS + sk]) = st.x[d];
    __syncthreads();
#pragma unroll
    for (int d = 0; d < 4; d++) {
      i32x4 bx[4];
#pragma unroll
      for (int j = 0; j < 4; j++) bx[j] = *reinterpret_cast<const i32x4 *>(&xb[d][(16 * j + (lane & 15)) * kI8XS + wk]);
#pragma unroll
      for (int j = 0; j < 4; j++)
#pragma unroll
        for (int mb = 0; mb < MB; mb++)
          acc[mb][j][d] = __builtin_amdgcn_mfma_i32_16x16x64_i8(st.w[mb], bx[j], acc[mb][j][d], 0, 0, 0);
    }
  };
  Stage s0, s1;
  issue(0, s0);
  int s = 0;
  for (; s + 2 <= nsteps; s += 2) {
    issue(s + 1, s1);
    compute(s, s0);
    issue(s + 2, s0);
    compute(s + 1, s1);
  }
  if (s < nsteps) compute(s, s0);
  // lane holds rows rl + i (i = 0..3) of stream 16 j + lane % 16
#pragma unroll
  for (int mb = 0; mb < MB; mb++) {
    const int rl = wave * 16 * MB + 16 * mb + 4 * (lane >> 4);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int b = 16 * j + (lane & 15);
      if (b >= nb) continue;
      const int E = p.xe[b0 + b];
      float a4[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const double sum = ((static_cast<double>(acc[mb][j][0][i]) * 256.0 + static_cast<double>(acc[mb][j][1][i])) * 256.0 +
                            static_cast<double>(acc[mb][j][2][i])) * 256.0 + static_cast<double>(acc[mb][j][3][i]);
        a4[i] = static_cast<float>(ldexp(sum, E - 30));
      }
      epilogue4(p, XE_I8, m0 + rl, b0 + b, a4);
    }
  }
}

// ---- K-sliced GEMM: no LDS staging inside the K loop ----
//
// Workgroup tile: 64 weight rows x 64 streams, K in steps of 128.  Wave w
// takes k 32 w .. 32 w + 31 of every step for the whole tile (4 row blocks x
// 4 stream blocks = 16 MFMA blocks, 48 MFMAs a step with the three activation
// planes), so no operand is shared between waves: a lane loads the 8
// activations and the 8 weights of each block it feeds straight into
// registers (k 8 * (lane / 16) .. + 7 of the wave's slice, the same k for the
// A and B operands), splits the activations into their bf16 planes and
// converts the weights in registers.  The four waves' partial tiles are added
// in LDS in wave order once, after the K loop.
constexpr int kKsBK = 128;  // k per step (32 per wave)

template <int WT>
struct WLoad8 {  // one lane's 8 weights of one row block (raw)
  uint32_t q[WT == XE_BF16 ? 4 : (WT == XE_I4 ? 1 : 2)];
  uint32_t e;  // bfp16: the block's exponent byte
};

template <int WT>
__device__ __forceinline__ void load_w8(const __amdgpu_buffer_rsrc_t &rw, const __amdgpu_buffer_rsrc_t &re, int row,
                                        int k, bool ok, int K, WLoad8<WT> &o) {
  typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
  if constexpr (WT == XE_I4) {
    o.q[0] = __builtin_amdgcn_raw_buffer_load_b32(rw, ok ? row * (K / 2) + k / 2 : kNoRec, 0, 2);
  } else if constexpr (WT == XE_BF16) {
    const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, ok ? (row * K + k) * 2 : kNoRec, 0, 2));
    o.q[0] = v.x;
    o.q[1] = v.y;
    o.q[2] = v.z;
    o.q[3] = v.w;
  } else {
    const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rw, ok ? row * K + k : kNoRec, 0, 2));
    o.q[0] = v.x;
    o.q[1] = v.y;
    if constexpr (WT == XE_BFP16)
      o.e = __builtin_amdgcn_raw_buffer_load_b8(re, ok ? row * (K / 8) + k / 8 : kNoRec, 0, 2);
  }
}

// bf16 A operand (8 k) of one row block.
template <int WT>
__device__ __forceinline__ bf16x8 to_bf16x8(const WLoad8<WT> &w) {
  if constexpr (WT == XE_BF16) {
    return __builtin_bit_cast(bf16x8, u32x4{w.q[0], w.q[1], w.q[2], w.q[3]});
  } else if constexpr (WT == XE_I4) {
    uint32_t p[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int word = static_cast<int>(w.q[0]);
      // (the builtin's result type is unsigned: convert through int)
      const float f0 = static_cast<float>(static_cast<int>(__builtin_amdgcn_sbfe(word, 8 * i, 4)));
      const float f1 = static_cast<float>(static_cast<int>(__builtin_amdgcn_sbfe(word, 8 * i + 4, 4)));
      p[i] = pack_hi16(f0, f1);
    }
    return __builtin_bit_cast(bf16x8, u32x4{p[0], p[1], p[2], p[3]});
  } else {
    uint32_t p[4];
    const int e = WT == XE_BFP16 ? static_cast<int>(w.e & 0xffu) - 133 : 0;
#pragma unroll
    for (int i = 0; i < 2; i++) {
      float f[4];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        f[j] = static_cast<float>(static_cast<int>(static_cast<int8_t>(w.q[i] >> (8 * j))));
        if constexpr (WT == XE_BFP16) f[j] = __builtin_ldexpf(f[j], e);
      }
      p[2 * i] = pack_hi16(f[0], f[1]);
      p[2 * i + 1] = pack_hi16(f[2], f[3]);
    }
    return __builtin_bit_cast(bf16x8, u32x4{p[0], p[1], p[2], p[3]});
  }
}

// Three bf16 planes of 8 fp32 activations, x = hi + mid + lo exactly (each
// plane takes the next 8 significant bits by truncation).
__device__ __forceinline__ void split3(const f32x4 &x0, const f32x4 &x1, bf16x8 (&o)[3]) {
  const float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
  float r[8], l[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    r[i] = v[i] - trunc_bf16(v[i]);
    l[i] = r[i] - trunc_bf16(r[i]);
  }
  uint32_t h[4], m[4], w[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    h[i] = pack_hi16(v[2 * i], v[2 * i + 1]);
    m[i] = pack_hi16(r[2 * i], r[2 * i + 1]);
    w[i] = pack_hi16(l[2 * i], l[2 * i + 1]);
  }
  o[0] = __builtin_bit_cast(bf16x8, u32x4{h[0], h[1], h[2], h[3]});
  o[1] = __builtin_bit_cast(bf16x8, u32x4{m[0], m[1], m[2], m[3]});
  o[2] = __builtin_bit_cast(bf16x8, u32x4{w[0], w[1], w[2], w[3]});
}

// Coalesced operand loads through a wave-private LDS slice.  An MFMA operand
// puts 16 different rows on consecutive lanes, so loading it straight from
// memory makes every quad of lanes touch four cache lines (four times the
// address-unit cycles of a contiguous quad: measured, this bound the kernel).
// Each wave therefore loads its k-slice of the step row by row (4 or 8
// consecutive lanes on one row), stores it to its own LDS area as is, and
// reads the operands back in MFMA layout.  LDS traffic of one wave is
// ordered, so no barrier is needed.
template <int WT>
constexpr int w_slice_dw() {  // dwords of one row's 32-k weight slice
  return WT == XE_BF16 ? 16 : (WT == XE_I4 ? 4 : 8);
}
constexpr int kXD = 36;  // LDS row stride (dwords) of a wave's 32-k activation slice

template <int WT, int MB, int NJ>
__host__ __device__ constexpr int ks_stage_dw() {  // LDS dwords of one wave's slices
  return 16 * NJ * kXD + 16 * MB * (w_slice_dw<WT>() + 4);
}

template <int WT, int MB, int NJ>
__host__ __device__ constexpr int ks_lds_dw() {
  return 4 * ks_stage_dw<WT, MB, NJ>() > 4 * 16 * NJ * (16 * MB + 4) ? 4 * ks_stage_dw<WT, MB, NJ>()
                                                                       : 4 * 16 * NJ * (16 * MB + 4);
}

// NJ: stream blocks of 16 a tile (BN = 16 NJ streams: 16, 32 or 64).  EC
// (bfp16): the exponent bytes read with plain (L2-cached) loads instead of
// streaming ones.  Each 128-byte line of a row's exponents serves several
// steps, and a streamed line was fetched again (14336 x 4096 at 4 / 8
// streams: 1.35x the algorithmic bytes, 47.0 / 49.2 us; cached 40.4 / 41.6
// us, 4096 x 4096: -2 / -4 %), but a small tile, bound by latency rather
// than bytes, loses with cached loads (3072 x 768 at 4 / 8 streams, 16 rows
// x 768 a tile: 7.9 / 8.2 against 8.9 / 9.0 us).  So cached from kEcElems
// weights a split tile.
constexpr int kEcElems = 65536;
template <int WT, int MB, int NJ, bool EC = false>
__global__ __launch_bounds__(kGT) void gemm_ks_kernel(gdev::GemvParams p, float *ws, unsigned *cnt, int spk) {
  constexpr int BM = 16 * MB, BN = 16 * NJ;
  constexpr int WD = w_slice_dw<WT>(), WDP = WD + 4;
  // the waves' operand slices during the K loop; afterwards the four waves'
  // partial tiles [wave][stream][row] (row stride padded)
  constexpr int kRS = BM + 4;
  __shared__ __attribute__((aligned(16))) uint32_t lds[ks_lds_dw<WT, MB, NJ>()];
  float(*red)[BN * kRS] = reinterpret_cast<float(*)[BN * kRS]>(lds);
  __shared__ int last;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint32_t *xst = lds + wave * ks_stage_dw<WT, MB, NJ>();  // [BN][kXD]
  uint32_t *wst = xst + BN * kXD;                           // [BM][WDP]
  const int m0 = blockIdx.x * BM, b0 = blockIdx.y * BN;
  const int K = p.k;
  const int ks = gridDim.z, z = blockIdx.z;
  const int step0 = z * spk;
  const int nsteps = min((K + kKsBK - 1) / kKsBK, step0 + spk) - step0;
  const int nb = min(BN, p.batch - b0);
  const __amdgpu_buffer_rsrc_t rw = gdev::coherent_rsrc(p.w);
  const __amdgpu_buffer_rsrc_t re = gdev::coherent_rsrc(WT == XE_BFP16 ? static_cast<const void *>(p.exps) : p.w);
  const __amdgpu_buffer_rsrc_t rx = gdev::coherent_rsrc(p.x);
  constexpr int XI = 2 * NJ;  // activation load instructions a step (8 stream rows each)

  // MFMA layout: lane feeds row / stream lane % 16 of a block with k
  // 8 * (lane / 16) .. + 7 of the wave's 32-k slice
  const int lr = lane & 15, lq = lane >> 4;
  const int kend = min(K, (step0 + nsteps) * kKsBK);
  // coalesced activation loads: instruction i, lane -> stream row 8 i +
  // lane / 8, 16 bytes at k 4 (lane % 8); rows past the batch read zeros
  const int xr = lane >> 3, xc = 4 * (lane & 7);
  int xoff[XI], xlim[XI];
#pragma unroll
  for (int i = 0; i < XI; i++) {
    const int b = 8 * i + xr;
    xoff[i] = (b0 + b) * p.ldx + xc;
    xlim[i] = b < nb ? kend : 0;
  }
  // coalesced weight loads: instruction mb, lane -> row 16 mb + lane / 4,
  // a quarter of its 32-k slice
  const int wr = lane >> 2, wq = lane & 3;

  struct Stage {
    uint32_t w[MB][WD / 4];
    uint32_t e[MB];  // bfp16: exponent byte (MFMA layout)
    f32x4 x[XI];
  };
  auto issue = [&](int step, Stage &st) {
    const int k0 = (step0 + step) * kKsBK + 32 * wave;
#pragma unroll
    for (int i = 0; i < XI; i++)
      st.x[i] = __builtin_bit_cast(
          f32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, k0 + xc < xlim[i] ? (xoff[i] + k0) * 4 : kNoRec, 0, 0));
#pragma unroll
    for (int mb = 0; mb < MB; mb++) {
      // per lane: with K % 32 == 16 the last step's slice ends inside a row
      const int row = m0 + 16 * mb + wr;
      const bool ok = row < p.m && k0 + 8 * wq < kend;
      if constexpr (WT == XE_BF16) {
        const u32x4 v = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, ok ? (row * K + k0 + 8 * wq) * 2 : kNoRec, 0, 2));
        st.w[mb][0] = v.x;
        st.w[mb][1] = v.y;
        st.w[mb][2] = v.z;
        st.w[mb][3] = v.w;
      } else if constexpr (WT == XE_I4) {
        st.w[mb][0] = __builtin_amdgcn_raw_buffer_load_b32(rw, ok ? row * (K / 2) + k0 / 2 + 4 * wq : kNoRec, 0, 2);
      } else {
        typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 v =
            __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rw, ok ? row * K + k0 + 8 * wq : kNoRec, 0, 2));
        st.w[mb][0] = v.x;
        st.w[mb][1] = v.y;
      }
      if constexpr (WT == XE_BFP16) {
        const int erow = m0 + 16 * mb + lr, ek = k0 + 8 * lq;
        st.e[mb] = __builtin_amdgcn_raw_buffer_load_b8(re, erow < p.m && ek < kend ? erow * (K / 8) + ek / 8 : kNoRec,
                                                      0, EC ? 0 : 2);
      }
    }
  };

  // the epilogue's row scales and biases, in flight during the K loop: a
  // thread's items all have row quad threadIdx.x % (BM / 4)
  const RowQuad rq = load_quad(p, WT, m0 + 4 * (static_cast<int>(threadIdx.x) % (BM / 4)));

  f32x4 acc[MB][NJ];
#pragma unroll
  for (int mb = 0; mb < MB; mb++)
#pragma unroll
    for (int j = 0; j < NJ; j++) acc[mb][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // the MFMAs of one stream block interleave the row blocks, and with fewer
  // than four row blocks the stream blocks too (at least four independent
  // accumulators between two MFMAs on the same one)
  auto compute = [&](const Stage &st) {
    // the step's slices into LDS as loaded
#pragma unroll
    for (int i = 0; i < XI; i++) *reinterpret_cast<f32x4 *>(xst + (8 * i + xr) * kXD + xc) = st.x[i];
#pragma unroll
    for (int mb = 0; mb < MB; mb++) {
      uint32_t *d = wst + (16 * mb + wr) * WDP + wq * (WD / 4);
      if constexpr (WD / 4 == 4) {
        *reinterpret_cast<u32x4 *>(d) = u32x4{st.w[mb][0], st.w[mb][1], st.w[mb][2], st.w[mb][3]};
      } else if constexpr (WD / 4 == 2) {
        typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
        *reinterpret_cast<u32x2 *>(d) = u32x2{st.w[mb][0], st.w[mb][1]};
      } else {
        d[0] = st.w[mb][0];
      }
    }
    // and back in MFMA layout
    bf16x8 a[MB];
#pragma unroll
    for (int mb = 0; mb < MB; mb++) {
      const uint32_t *src = wst + (16 * mb + lr) * WDP + lq * (WD / 4);
      WLoad8<WT> wl;
#pragma unroll
      for (int i = 0; i < WD / 4; i++) wl.q[i] = src[i];
      if constexpr (WT == XE_BFP16) wl.e = st.e[mb];
      a[mb] = to_bf16x8<WT>(wl);
    }
    constexpr int JG0 = MB >= 4 ? 1 : 4 / MB;
    constexpr int JG = JG0 < NJ ? JG0 : NJ;  // stream blocks a group
#pragma unroll
    for (int j0 = 0; j0 < NJ; j0 += JG) {
      bf16x8 bx[JG][3];
#pragma unroll
      for (int jj = 0; jj < JG; jj++) {
        const uint32_t *src = xst + (16 * (j0 + jj) + lr) * kXD + 8 * lq;
        split3(*reinterpret_cast<const f32x4 *>(src), *reinterpret_cast<const f32x4 *>(src + 4), bx[jj]);
      }
#pragma unroll
      for (int pl = 0; pl < 3; pl++)
#pragma unroll
        for (int jj = 0; jj < JG; jj++)
#pragma unroll
          for (int mb = 0; mb < MB; mb++)
            acc[mb][j0 + jj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[mb], bx[jj][pl], acc[mb][j0 + jj], 0, 0, 0);
    }
  };

  // two stages: the next step's loads are in flight while a step computes
  // (three or four stages measured no faster at b = 64)
  Stage s0, s1;
  issue(0, s0);
  int s = 0;
  for (; s + 2 <= nsteps; s += 2) {
    issue(s + 1, s1);
    // the loads go out before this step's arithmetic waits for its own
    __builtin_amdgcn_sched_barrier(0);
    compute(s0);
    issue(s + 2, s0);
    __builtin_amdgcn_sched_barrier(0);
    compute(s1);
  }
  if (s < nsteps) compute(s0);
  __syncthreads();  // every wave is done with its slices: the LDS becomes red

  // the waves' partial tiles into LDS: lane holds rows 16 mb + 4 (lane / 16)
  // + i of stream 16 j + lane % 16
#pragma unroll
  for (int mb = 0; mb < MB; mb++)
#pragma unroll
    for (int j = 0; j < NJ; j++)
      *reinterpret_cast<f32x4 *>(&red[wave][(16 * j + lr) * kRS + 16 * mb + 4 * (lane >> 4)]) = acc[mb][j];
  __syncthreads();
  // item = (stream bb, row quad q): BN x BM / 4 items, RI a thread (the
  // last round partly empty when there are fewer items than threads)
  constexpr int QN = BM / 4;
  constexpr int ITEMS = BN * QN;
  constexpr int RI = (ITEMS + kGT - 1) / kGT;
  float sum[RI][4];
#pragma unroll
  for (int r = 0; r < RI; r++) {
    const int it = threadIdx.x + r * kGT;
    const int bb = it < ITEMS ? it / QN : 0, q = it % QN;
    f32x4 t = *reinterpret_cast<const f32x4 *>(&red[0][bb * kRS + 4 * q]);
#pragma unroll
    for (int w = 1; w < 4; w++) t += *reinterpret_cast<const f32x4 *>(&red[w][bb * kRS + 4 * q]);
    sum[r][0] = t.x;
    sum[r][1] = t.y;
    sum[r][2] = t.z;
    sum[r][3] = t.w;
  }
  if (ks == 1) {
#pragma unroll
    for (int r = 0; r < RI; r++) {
      const int it = threadIdx.x + r * kGT;
      const int bb = it / QN, q = it % QN;
      if (it < ITEMS && bb < nb) epilogue4(p, rq, m0 + 4 * q, b0 + bb, sum[r]);
    }
    return;
  }
  if (p.part) {
    // the consumer adds the splits: this split's raw sums, no counter
    float *dst = p.part + (static_cast<size_t>(z) * p.batch + b0) * p.m;
#pragma unroll
    for (int r = 0; r < RI; r++) {
      const int it = threadIdx.x + r * kGT;
      const int bb = it / QN, q = it % QN;
      if (it >= ITEMS || bb >= nb) continue;
      const int r0 = m0 + 4 * q;
      float *d = dst + static_cast<size_t>(bb) * p.m + r0;
      if ((p.m & 3) == 0 && r0 < p.m) {
        *reinterpret_cast<float4 *>(d) = make_float4(sum[r][0], sum[r][1], sum[r][2], sum[r][3]);
      } else {
#pragma unroll
        for (int i = 0; i < 4; i++)
          if (r0 + i < p.m) d[i] = sum[r][i];
      }
    }
    return;
  }
  const int tile = blockIdx.y * gridDim.x + blockIdx.x;
  // the partial tile with 16-byte sc1 stores (what an agent-scope atomic
  // store compiles to, four dwords at a time)
  const __amdgpu_buffer_rsrc_t rp = gdev::coherent_rsrc(ws + (static_cast<size_t>(tile) * ks + z) * (BM * BN));
#pragma unroll
  for (int r = 0; r < RI; r++) {
    const int it = threadIdx.x + r * kGT;
    const int bb = it / QN, q = it % QN;
    if (it < ITEMS)
      __builtin_amdgcn_raw_buffer_store_b128(
          __builtin_bit_cast(u32x4, f32x4{sum[r][0], sum[r][1], sum[r][2], sum[r][3]}), rp, (bb * BM + 4 * q) * 4, 0,
          gdev::kCoherentSc1);
  }
  splitk_finish<WT, BM, BN>(p, ws, cnt, tile, ks, nb, m0, b0, last, &rq);
}

// Norm / residual prologue of one stream row (blockIdx.x): p.x, p.sub and
// p.res_out point at row 0 and advance by ldx / k per row; the normalised
// row goes to xn [batch][k].
__global__ __launch_bounds__(256) void gemm_prologue_kernel(gdev::GemvParams p, float *xn) {
  extern __shared__ float4 xs4[];
  __shared__ float red[2 * gdev::kRedN * gdev::kMaxWaves];
  const int b = blockIdx.x;
  gdev::GemvParams q = p;
  q.x = static_cast<const float *>(p.x) + static_cast<size_t>(b) * p.ldx;
  q.sub = p.sub ? p.sub + static_cast<size_t>(b) * p.k : nullptr;
  q.res_out = p.res_out ? p.res_out + static_cast<size_t>(b) * p.k : nullptr;
  q.batch = 1;
  gdev::gemv_prologue<1, 4>(q, xs4, red, true);
  const float *xs = reinterpret_cast<const float *>(xs4);
  for (int i = threadIdx.x; i < p.k; i += 256) xn[static_cast<size_t>(b) * p.k + i] = xs[gdev::xs_elem<1>(i)];
}

// `sub` from a GEMM's split partials (GemvParams::sub_part): every split's
// value in flight at once, added in split order from zero, then the
// producer's epilogue (scale, bias, output scale), as splitk_finish and
// epilogue4 would have stored it.
__device__ __forceinline__ float sub_finish(const gdev::GemvParams &p, int i, float s) {
  const float sc = p.sub_scale ? p.sub_scale[i] : 1.0f;
  const float bi = p.sub_bias ? p.sub_bias[i] : 0.0f;
  return (s * sc + bi) * p.sub_out_scale;
}

// float4 chunk i4 of stream b
__device__ __forceinline__ float4 sub_parts4(const gdev::GemvParams &p, int b, int i4) {
  float4 v[kMaxSplitsK];
#pragma unroll
  for (int z = 0; z < kMaxSplitsK; z++)
    if (z < p.sub_ks)
      v[z] = reinterpret_cast<const float4 *>(p.sub_part + (static_cast<size_t>(z) * p.batch + b) * p.k)[i4];
  float s[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int z = 0; z < kMaxSplitsK; z++) {
    if (z < p.sub_ks) {
      s[0] += v[z].x;
      s[1] += v[z].y;
      s[2] += v[z].z;
      s[3] += v[z].w;
    }
  }
  const int i = 4 * i4;
  return make_float4(sub_finish(p, i, s[0]), sub_finish(p, i + 1, s[1]), sub_finish(p, i + 2, s[2]),
                     sub_finish(p, i + 3, s[3]));
}

// element i of stream b
__device__ __forceinline__ float sub_parts1(const gdev::GemvParams &p, int b, int i) {
  float v[kMaxSplitsK];
#pragma unroll
  for (int z = 0; z < kMaxSplitsK; z++)
    if (z < p.sub_ks) v[z] = p.sub_part[(static_cast<size_t>(z) * p.batch + b) * p.k + i];
  float s = 0.f;
#pragma unroll
  for (int z = 0; z < kMaxSplitsK; z++)
    if (z < p.sub_ks) s += v[z];
  return sub_finish(p, i, s);
}

// ---- int8 digit planes of a normalised row (GemvParams::xd / xe) ----
// Block maximum over the prologue's 256 threads; mx: 4 floats of LDS.
__device__ __forceinline__ float block_max256(float v, float *mx) {
  v = gdev::wave_max(v);
  if ((threadIdx.x & 63) == 0) mx[threadIdx.x >> 6] = v;
  __syncthreads();
  return fmaxf(fmaxf(mx[0], mx[1]), fmaxf(mx[2], mx[3]));
}

// The exponent E with every |x| < 2^E given the row's largest |x| (0 for
// a zero row).
__device__ __forceinline__ int digit_exp(float amax) {
  int e = 0;
  if (amax > 0.f) (void)frexpf(amax, &e);
  return e;
}

// Four signed base-256 digits of rint(v 2^(30 - E)) (|v| < 2^E, so the
// integer is at most 2^30): d3 the low byte read as signed, then d2, d1 of
// what remains, and d0 (at most 64 in magnitude).
__device__ __forceinline__ void digits_of(float v, int E, int (&d)[4]) {
  const int xi = __float2int_rn(__builtin_ldexpf(v, 30 - E));
  d[3] = static_cast<int8_t>(xi & 0xff);
  int r = (xi - d[3]) >> 8;
  d[2] = static_cast<int8_t>(r & 0xff);
  r = (r - d[2]) >> 8;
  d[1] = static_cast<int8_t>(r & 0xff);
  d[0] = (r - d[1]) >> 8;
}

// Elements i .. i + 3 of stream b (i a multiple of 4): one 4-byte store a plane.
__device__ __forceinline__ void put_digits4(const gdev::GemvParams &p, int b, int i, const float (&v)[4], int E) {
  uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int c = 0; c < 4; c++) {
    int d[4];
    digits_of(v[c], E, d);
#pragma unroll
    for (int q = 0; q < 4; q++) w[q] |= (static_cast<uint32_t>(d[q]) & 0xffu) << (8 * c);
  }
  const size_t plane = static_cast<size_t>(p.batch) * p.k;
#pragma unroll
  for (int q = 0; q < 4; q++)
    *reinterpret_cast<uint32_t *>(p.xd + q * plane + static_cast<size_t>(b) * p.k + i) = w[q];
}

// The Gemma sandwich-norm prologue (x + post-norm(sub) -> res_out, then the
// pre-norm) with every operand in registers: x, sub, post_w and gamma arrive
// in one memory round trip, one block reduction gives both statistics, and
// res_out and xn are stored from registers.  The same arithmetic in the same
// order as gemv_prologue's fold path (bit-identical).  A thread takes float4
// chunks threadIdx.x + j * 256, j < NV (K <= 1024 * NV).
template <int NV>
__global__ __launch_bounds__(256) void gemm_prologue_fold_kernel(gdev::GemvParams p, float *xn) {
  __shared__ float red[2 * 4 * gdev::kMaxWaves];
  const int b = blockIdx.x;
  const int K = p.k, K4 = K / 4;
  const float fk = static_cast<float>(K);
  const float4 *x4 = reinterpret_cast<const float4 *>(static_cast<const float *>(p.x) + static_cast<size_t>(b) * p.ldx);
  const float4 *s4 = p.sub_part ? nullptr : reinterpret_cast<const float4 *>(p.sub + static_cast<size_t>(b) * K);
  const float4 *w4 = reinterpret_cast<const float4 *>(p.post_w);
  const float4 *g4 = reinterpret_cast<const float4 *>(p.gamma);
  float4 v[NV], sv[NV], w[NV], g[NV];
#pragma unroll
  for (int j = 0; j < NV; j++) {
    const int i = threadIdx.x + j * 256;
    if (i < K4) {
      v[j] = x4[i];
      sv[j] = p.sub_part ? sub_parts4(p, b, i) : s4[i];
      w[j] = w4[i];
      g[j] = g4[i];
    }
  }
  float acc[4] = {0.f, 0.f, 0.f, 0.f};  // sum sub^2, x^2, x*s', s'^2
#pragma unroll
  for (int j = 0; j < NV; j++) {
    if (threadIdx.x + j * 256 >= K4) continue;
    const float xv[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
    const float su[4] = {sv[j].x, sv[j].y, sv[j].z, sv[j].w};
    const float wv[4] = {w[j].x, w[j].y, w[j].z, w[j].w};
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const float sp = su[c] * (1.0f + wv[c]);
      acc[0] = __builtin_fmaf(su[c], su[c], acc[0]);
      acc[1] = __builtin_fmaf(xv[c], xv[c], acc[1]);
      acc[2] = __builtin_fmaf(xv[c], sp, acc[2]);
      acc[3] = __builtin_fmaf(sp, sp, acc[3]);
    }
  }
  int slot = 0;
  gdev::block_sums<4, 4>(acc, red, slot);
  const float inv_s = 1.0f / sqrtf(acc[0] / fk + p.eps);
  const float st2 = acc[1] + 2.0f * inv_s * acc[2] + inv_s * inv_s * acc[3];
  const float inv_t = 1.0f / sqrtf(fmaxf(st2, 0.f) / fk + p.eps);
  const bool one_p = p.norm == XE_NORM_RMS1P;
  float h[NV][4];
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < NV; j++) {
    const int i = threadIdx.x + j * 256;
    if (i >= K4) continue;
    const float xv[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
    const float su[4] = {sv[j].x, sv[j].y, sv[j].z, sv[j].w};
    const float wv[4] = {w[j].x, w[j].y, w[j].z, w[j].w};
    const float gv[4] = {g[j].x, g[j].y, g[j].z, g[j].w};
    float t[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
      t[c] = xv[c] + su[c] * inv_s * (1.0f + wv[c]);
      h[j][c] = one_p ? t[c] * inv_t * (1.0f + gv[c]) : t[c] * inv_t * gv[c];
      amax = fmaxf(amax, fabsf(h[j][c]));
    }
    if (p.res_out)
      reinterpret_cast<float4 *>(p.res_out + static_cast<size_t>(b) * K)[i] = make_float4(t[0], t[1], t[2], t[3]);
    if (!p.xd)
      reinterpret_cast<float4 *>(xn + static_cast<size_t>(b) * K)[i] = make_float4(h[j][0], h[j][1], h[j][2], h[j][3]);
  }
  if (p.xd) {
    __shared__ float mx[4];
    const int E = digit_exp(block_max256(amax, mx));
    if (threadIdx.x == 0) p.xe[b] = E;
#pragma unroll
    for (int j = 0; j < NV; j++) {
      const int i = threadIdx.x + j * 256;
      if (i < K4) put_digits4(p, b, 4 * i, h[j], E);
    }
  }
}

// The GEMM prologue without the Gemma fold (optional residual add -> res_out,
// then LayerNorm / RMSNorm / none) with every operand in registers: thread t
// takes elements t + j * 256, j < NS, the per-thread order of
// gemv_prologue's plain path, so the sums and outputs are bit-identical.
// K <= 256 * NS.
template <int NS>
__global__ __launch_bounds__(256) void gemm_prologue_reg_kernel(gdev::GemvParams p, float *xn) {
  __shared__ float red[2 * 4 * gdev::kMaxWaves];
  const int b = blockIdx.x, K = p.k;
  const float fk = static_cast<float>(K);
  const float *xr = static_cast<const float *>(p.x) + static_cast<size_t>(b) * p.ldx;
  const uint16_t *xh = static_cast<const uint16_t *>(p.x) + static_cast<size_t>(b) * p.ldx;  // bf16 x
  const float *sr = p.sub ? p.sub + static_cast<size_t>(b) * K : nullptr;
  const bool has_sub = sr || p.sub_part;
  const bool ln = p.norm == XE_NORM_LN;
  float t[NS], sv[NS], g[NS], be[NS];
#pragma unroll
  for (int j = 0; j < NS; j++) {
    const int i = threadIdx.x + j * 256;
    t[j] = sv[j] = g[j] = be[j] = 0.f;
    if (i < K) {
      t[j] = p.x_bf16 ? __uint_as_float(static_cast<uint32_t>(xh[i]) << 16) : xr[i];
      if (has_sub) sv[j] = p.sub_part ? sub_parts1(p, b, i) : sr[i];
      if (p.norm != XE_NORM_NONE) g[j] = p.gamma[i];
      if (ln) be[j] = p.beta[i];
    }
  }
  if (has_sub) {
#pragma unroll
    for (int j = 0; j < NS; j++) {
      const int i = threadIdx.x + j * 256;
      if (i >= K) continue;
      t[j] = t[j] + sv[j];
      if (p.res_out) p.res_out[static_cast<size_t>(b) * K + i] = t[j];
    }
  }
  int slot = 0;
  if (ln) {
    float v1[1] = {0.f};
#pragma unroll
    for (int j = 0; j < NS; j++)
      if (threadIdx.x + j * 256 < K) v1[0] += t[j];
    gdev::block_sums<4, 1>(v1, red, slot);
    const float mean = v1[0] / fk;
    float v2[1] = {0.f};
#pragma unroll
    for (int j = 0; j < NS; j++) {
      if (threadIdx.x + j * 256 >= K) continue;
      const float c = t[j] - mean;
      v2[0] = __builtin_fmaf(c, c, v2[0]);
    }
    gdev::block_sums<4, 1>(v2, red, slot);
    const float inv = 1.0f / sqrtf(v2[0] / fk + p.eps);
#pragma unroll
    for (int j = 0; j < NS; j++) t[j] = (t[j] - mean) * inv * g[j] + be[j];
  } else if (p.norm != XE_NORM_NONE) {
    float v1[1] = {0.f};
#pragma unroll
    for (int j = 0; j < NS; j++)
      if (threadIdx.x + j * 256 < K) v1[0] = __builtin_fmaf(t[j], t[j], v1[0]);
    gdev::block_sums<4, 1>(v1, red, slot);
    const float inv = 1.0f / sqrtf(v1[0] / fk + p.eps);
#pragma unroll
    for (int j = 0; j < NS; j++)
      t[j] = p.norm == XE_NORM_RMS1P ? t[j] * inv * (1.0f + g[j]) : t[j] * inv * g[j];
  }
  if (p.xd) {
    __shared__ float mx[4];
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < NS; j++)
      if (threadIdx.x + j * 256 < K) amax = fmaxf(amax, fabsf(t[j]));
    const int E = digit_exp(block_max256(amax, mx));
    if (threadIdx.x == 0) p.xe[b] = E;
    const size_t plane = static_cast<size_t>(p.batch) * K;
#pragma unroll
    for (int j = 0; j < NS; j++) {
      const int i = threadIdx.x + j * 256;
      if (i >= K) continue;
      int d[4];
      digits_of(t[j], E, d);
#pragma unroll
      for (int q = 0; q < 4; q++) p.xd[q * plane + static_cast<size_t>(b) * K + i] = static_cast<int8_t>(d[q]);
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < NS; j++) {
    const int i = threadIdx.x + j * 256;
    if (i < K) xn[static_cast<size_t>(b) * K + i] = t[j];
  }
}

using GemmFn = void (*)(gdev::GemvParams, float *, unsigned *, int);

template <int WT>
GemmFn pick_mb(int mb) {
  switch (mb) {
    case 1: return gemm_kernel<WT, 1>;
    case 2: return gemm_kernel<WT, 2>;
    case 4: return gemm_kernel<WT, 4>;
  }
  return nullptr;
}

template <int WT, int NJ, bool EC = false>
GemmFn pick_ks_mb(int mb) {
  switch (mb) {
    case 1: return gemm_ks_kernel<WT, 1, NJ, EC>;
    case 2: return gemm_ks_kernel<WT, 2, NJ, EC>;
    case 4: return gemm_ks_kernel<WT, 4, NJ, EC>;
  }
  return nullptr;
}

template <int WT, bool EC = false>
GemmFn pick_ks_nj(int mb, int nj) {
  switch (nj) {
    case 1: return pick_ks_mb<WT, 1, EC>(mb);
    case 2: return pick_ks_mb<WT, 2, EC>(mb);
    case 4: return pick_ks_mb<WT, 4, EC>(mb);
  }
  return nullptr;
}

// spk: steps a K split spans (bfp16 exponents cached from kEcElems weights a
// split tile: 16 mb rows x spk steps of kKsBK)
GemmFn pick_ks(int wdtype, int mb, int nj, int spk) {
  switch (wdtype) {
    case XE_I8: return pick_ks_nj<XE_I8>(mb, nj);
    case XE_BF16: return pick_ks_nj<XE_BF16>(mb, nj);
    case XE_BFP16:
      return 16 * mb * spk * kKsBK >= kEcElems ? pick_ks_nj<XE_BFP16, true>(mb, nj) : pick_ks_nj<XE_BFP16>(mb, nj);
    case XE_I4: return pick_ks_nj<XE_I4>(mb, nj);
  }
  return nullptr;
}

GemmFn pick_gemm(int wdtype, int mb) {
  switch (wdtype) {
    case XE_I8: return pick_mb<XE_I8>(mb);
    case XE_BF16: return pick_mb<XE_BF16>(mb);
    case XE_BFP16: return pick_mb<XE_BFP16>(mb);
    case XE_I4: return pick_mb<XE_I4>(mb);
  }
  return nullptr;
}

// Shape of one GEMM launch: row blocks per wave (MB), splits of K.  The
// largest MB that still gives every CU about two workgroups (the fewer
// activation-fragment reads per weight byte, the better), then splits for
// about four workgroups per CU: at most kMaxSplitsK, at least two K steps
// each, and a bounded partial workspace.
struct GemmShape {
  int mb, ks, spk, tm, tb, nj;
};

GemmShape gemm_shape(int m, int k, int batch) {
  const int steps = (k + kBK - 1) / kBK;
  const int tb = (batch + kBN - 1) / kBN;
  const int cus = gdev::cu_count();
  GemmShape g{1, 1, steps, 0, tb, 4};
  // wide outputs (the lm-head): four row blocks per wave; else one
  g.mb = static_cast<long long>(m) * tb >= 64LL * 4 * 4 * cus ? 4 : 1;
  g.tm = (m + 64 * g.mb - 1) / (64 * g.mb);
  // split K only when the tiles leave most CUs idle: every split's partial
  // tile costs a write and a read of 64 x 64 x mb floats, so at least two
  // steps (128 k) per split (b = 64 probe: QKV 15.6 -> 14.0 us, O 15.3 ->
  // 13.8 us against four steps)
  const int tiles = g.tm * g.tb;
  int ks = 1;
  if (2 * tiles < cus) {
    ks = std::min(kMaxSplitsK, (cus + tiles - 1) / tiles);
    ks = std::min(ks, std::max(1, steps / 2));
    while (ks > 1 && static_cast<size_t>(tiles) * ks * 64 * g.mb * kBN > kGemmWsFloats) ks--;
  }
  g.spk = (steps + ks - 1) / ks;
  g.ks = (steps + g.spk - 1) / g.spk;  // no empty split
  return g;
}

// Shape of a K-sliced launch, or mb = 0 where none fits the chip in one
// round (outputs wider than 64 rows a CU: the lm-head).  Stream tiles of 16,
// 32 or 64 (the fewest 16-stream blocks that hold the batch, 64 beyond).
// Candidates: 1, 2 or 4 row blocks a wave, each with the most splits of K
// that keep the grid within one workgroup per CU and at least two steps a
// split; the cheapest by a cost fitted to b = 64 probes wins (ties to more
// row blocks): a step costs half a unit per 16-stream block for the
// activation slice plus one a row block, and a split tile's reduction half a
// unit a row block a split.  (b = 64, us: QKV 1536 x
// 1152 8.7 / 9.0 / 12.2 at 1 / 2 / 4 row blocks, O 1152 x 1024 7.5 / 8.5 /
// 11.7, gate/up 13824 x 1152 - / - / 16.6, down 1152 x 6912 18.6 / 14.3 /
// 16.2; gemm_kernel: 12.8, 12.6, 20.5, 18.9.)
GemmShape gemm_ks_shape(int m, int k, int batch) {
  const int steps = (k + kKsBK - 1) / kKsBK;
  const int cus = gdev::cu_count();
  const int nj = batch <= 16 ? 1 : batch <= 32 ? 2 : 4;
  const int bn = 16 * nj;
  const int tb = (batch + bn - 1) / bn;
  // one workgroup a CU (two, with K splits, measured slower at 8 streams:
  // 14336 x 4096 int8 34.4 against 32.3 us)
  const int slots = cus;
  GemmShape best{0, 1, steps, 0, tb, nj};
  int best_work = 0;
  for (int mb = 4; mb >= 1; mb /= 2) {
    const int tm = (m + 16 * mb - 1) / (16 * mb);
    const int tiles = tm * tb;
    if (tiles > slots) continue;
    int ks = std::max(1, std::min(std::min(slots / tiles, steps / 2), kMaxSplitsK));
    while (ks > 1 && static_cast<size_t>(tiles) * ks * 16 * mb * bn > kGemmWsFloats) ks--;
    const int spk = (steps + ks - 1) / ks;
    const int kss = (steps + spk - 1) / spk;
    const int work = spk * (nj + 2 * mb) + (kss > 1 ? mb * kss : 0);
    if (best.mb == 0 || work < best_work) {
      best = GemmShape{mb, kss, spk, tm, tb, nj};
      best_work = work;
    }
  }
  return best;
}

}  // namespace

bool gemm_needs_prologue(const gdev::GemvParams &p) {
  return p.sub != nullptr || p.sub_part != nullptr || p.norm != XE_NORM_NONE || p.x_bf16;
}

// int8 weights on the int8 matrix cores (gemm_i8_kernel) for outputs too wide
// for the K-sliced kernel (the lm-head), when the activations come out of a
// prologue that can write the digit planes: with XE_GEMM_I8=1 only.  At the
// Gemma-3-1B lm-head (262144 x 1152, 64 streams) it measured 167 us against
// 160 us for the bf16 path (one box, A/B; 4 waves x 32 rows at one or two
// waves a SIMD: 197 / 168 us): neither kernel is bound by its matrix cores,
// and the per-step staging of four digit planes costs what the 1.5x fewer
// MFMAs save.
bool gemm_i8_preferred(int m, int k, int batch, int wdtype) {
  const char *e = std::getenv("XE_GEMM_I8");
  if (!(e && std::string(e) == "1")) return false;
  return wdtype == XE_I8 && k % 16 == 0 && gemm_ks_shape(m, k, batch).mb == 0 &&
         static_cast<long long>(batch) * k * 4 < (1LL << 31);
}

// Splits of K the K-sliced GEMM takes for this shape when it splits (the
// consumer may then add the partials itself: GemvParams::part), else 0.
int gemm_defer_splits(int m, int k, int batch) {
  const GemmShape g = gemm_ks_shape(m, k, batch);
  return g.mb > 0 && g.ks > 1 ? g.ks : 0;
}

// The matrix cores take a projection beyond 8 rows, and from
// XE_GEMM_MIN_BATCH rows (default 4) when the weight holds at least
// XE_GEMM_MIN_WEIGHTS elements (default 0: every config-2 shape was as fast
// or faster there at 4 rows): on the VALU every weight costs one FMA a row,
// which at 8 rows bounds the GEMV by instruction issue (rocprof: 16.9 M VALU
// instructions for 14336 x 4096, 0.64 TB/s), while the MFMA GEMM converts
// each weight once and issues 3 MFMAs per 16 x 32 block (14336 x 4096 int8
// at 8 rows: 92 -> 32 us).  At 2 rows the GEMV stays faster (23.6 against
// 29.5 us).
bool gemm_preferred(int m, int k, int batch) {
  if (batch > 8) return true;
  static const int min_batch = [] {
    const char *e = std::getenv("XE_GEMM_MIN_BATCH");
    return e ? std::atoi(e) : 4;
  }();
  static const long long min_w = [] {
    const char *e = std::getenv("XE_GEMM_MIN_WEIGHTS");
    return e ? std::atoll(e) : 0LL;
  }();
  return min_batch > 0 && batch >= min_batch && static_cast<long long>(m) * k >= min_w && k % 16 == 0;
}

namespace {
// The register prologues: the Gemma fold (x + post-norm(sub), then the
// norm), and the plain one (optional residual add, then LN / RMS / none).
// Only these two take `sub` as split partials.
bool fold_prologue(const gdev::GemvParams &p, const float *xn) {
  auto al16 = [](const void *q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
  const float *sub = p.sub_part ? p.sub_part : p.sub;
  return !p.x_bf16 && sub && p.post_w && p.gamma && (p.norm == XE_NORM_RMS1P || p.norm == XE_NORM_RMS) &&
         p.k % 4 == 0 && p.ldx % 4 == 0 && p.k <= 4096 && al16(p.x) && al16(sub) && al16(p.post_w) &&
         al16(p.gamma) && al16(p.res_out) && al16(xn);
}
bool reg_prologue(const gdev::GemvParams &p) {
  const bool has_sub = p.sub || p.sub_part;
  return !(has_sub && p.post_w) && p.k <= 4096 && (p.norm == XE_NORM_NONE || p.gamma) &&
         (p.norm != XE_NORM_LN || p.beta);
}
}  // namespace

bool gemm_prologue_takes_digits(const gdev::GemvParams &p, const float *xn) {
  return p.xd && p.xe && p.k % 4 == 0 && (fold_prologue(p, xn) || reg_prologue(p));
}

bool gemm_prologue_takes_parts(const gdev::GemvParams &p, const float *xn) {
  return p.sub_part && p.sub_ks >= 1 && p.sub_ks <= kMaxSplitsK && (fold_prologue(p, xn) || reg_prologue(p));
}

// Prologue (when the phase has one) into xn, then the GEMM reading xn.
void launch_gemm_prologue(const gdev::GemvParams &p, float *xn, hipStream_t s) {
  XE_REQUIRE(!p.sub_part || gemm_prologue_takes_parts(p, xn), "gemm prologue: split partials on an unsupported path");
  XE_REQUIRE(!p.xd || gemm_prologue_takes_digits(p, xn), "gemm prologue: digit planes on an unsupported path");
  if (fold_prologue(p, xn)) {
    const int nv = (p.k / 4 + 255) / 256;
    auto fn = nv <= 1 ? gemm_prologue_fold_kernel<1> : nv <= 2 ? gemm_prologue_fold_kernel<2>
                                                                : gemm_prologue_fold_kernel<4>;
    hipLaunchKernelGGL(fn, dim3(p.batch), dim3(256), 0, s, p, xn);
    XE_HIP(hipGetLastError());
    return;
  }
  if (reg_prologue(p)) {
    auto fn = p.k <= 1024 ? gemm_prologue_reg_kernel<4> : p.k <= 2048 ? gemm_prologue_reg_kernel<8>
                                                                       : gemm_prologue_reg_kernel<16>;
    hipLaunchKernelGGL(fn, dim3(p.batch), dim3(256), 0, s, p, xn);
    XE_HIP(hipGetLastError());
    return;
  }
  const size_t lds = gdev::gemv_lds_floats(1, p.k, p.sub != nullptr) * sizeof(float);
  XE_REQUIRE(lds <= 160 * 1024 - 1024, "gemm prologue: K too large for LDS staging");
  if (lds > 64 * 1024)
    XE_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(gemm_prologue_kernel),
                               hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
  hipLaunchKernelGGL(gemm_prologue_kernel, dim3(p.batch), dim3(256), lds, s, p, xn);
  XE_HIP(hipGetLastError());
}

size_t gemm_ws_floats() { return kGemmWsFloats; }
size_t gemm_cnt_words() { return kGemmMaxTiles; }

void launch_gemm(const gdev::GemvParams &p, int wdtype, float *ws, unsigned *cnt, hipStream_t s) {
  XE_REQUIRE(p.m > 0 && p.k > 0 && p.batch > 0, "gemm: empty shape");
  XE_REQUIRE(p.k % 16 == 0, "gemm: K must be a multiple of 16");
  XE_REQUIRE(!p.x_bf16, "gemm: fp32 activations only");
  XE_REQUIRE(p.act != ACT_GEGLU_TANH || p.m % 4 == 0, "gemm: GeGLU rows must pair within 4-row groups");
  XE_REQUIRE((wdtype != XE_I8 && wdtype != XE_I4) || p.scale, "gemm: int8/int4 weight without scales");
  XE_REQUIRE(wdtype != XE_BFP16 || p.exps, "gemm: bfp16 weight without exponents");
  // buffer offsets are 32-bit: weights and activations below 2 GB
  const size_t wb = static_cast<size_t>(p.m) * p.k * (wdtype == XE_BF16 ? 2 : 1);
  XE_REQUIRE(wb < (size_t(1) << 31) && static_cast<size_t>(p.batch) * p.ldx * 4 < (size_t(1) << 31),
             "gemm: operand above 2 GB");
  if (p.xd) {  // int8 digit planes of the activations: the int8 matrix cores
    XE_REQUIRE(wdtype == XE_I8 && p.xe && p.act != ACT_GEGLU_TANH && !p.part,
               "gemm: digit planes need int8 weights and a plain epilogue");
    XE_REQUIRE(static_cast<long long>(p.batch) * p.k * 4 < (1LL << 31), "gemm: digit planes above 2 GB");
    const int bm = 16 * kI8W * kI8MB;
    hipLaunchKernelGGL(gemm_i8_kernel, dim3((p.m + bm - 1) / bm, (p.batch + kBN - 1) / kBN), dim3(kI8T), 0, s, p);
    XE_HIP(hipGetLastError());
    return;
  }
  GemmShape g = gemm_shape(p.m, p.k, p.batch);
  GemmFn fn = nullptr;
  const GemmShape gk = gemm_ks_shape(p.m, p.k, p.batch);
  if (gk.mb > 0) {
    g = gk;
    fn = pick_ks(wdtype, g.mb, g.nj, g.spk);
  } else {
    fn = pick_gemm(wdtype, g.mb);
  }
  XE_REQUIRE(fn, "gemm: unsupported weight dtype");
  XE_REQUIRE(g.ks == 1 || (ws && cnt && static_cast<size_t>(g.tm) * g.tb <= kGemmMaxTiles),
             "gemm: split-K workspace missing or too many tiles");
  // partials for the consumer: the split count it was built for
  XE_REQUIRE(!p.part || (gk.mb > 0 && g.ks > 1 && g.ks == gemm_defer_splits(p.m, p.k, p.batch) &&
                         p.act == ACT_NONE),
             "gemm: split partials need the K-sliced kernel with a K split");
  hipLaunchKernelGGL(fn, dim3(g.tm, g.tb, g.ks), dim3(kGT), 0, s, p, ws, cnt, g.spk);
  XE_HIP(hipGetLastError());
}

size_t gemm_op_ws_floats() { return kGemmWsFloats; }
size_t gemm_op_cnt_words() { return kGemmMaxTiles; }

void launch_gemm_op(const GemvLaunch &L, float *xn, float *ws, unsigned *cnt, hipStream_t s) {
  XE_REQUIRE(L.x_dtype == XE_F32 || L.x_dtype == XE_BF16, "gemm: fp32 or bf16 activations");
  gdev::GemvParams p = gdev::to_params(L);
  if (gemm_needs_prologue(p)) {  // bf16 x: the prologue writes it as fp32
    XE_REQUIRE(xn, "gemm: prologue without a row buffer");
    launch_gemm_prologue(p, xn, s);
    p.x = xn;
    p.x_bf16 = 0;
    p.ldx = p.k;
    p.sub = nullptr;
    p.post_w = nullptr;
    p.res_out = nullptr;
    p.norm = XE_NORM_NONE;
  }
  launch_gemm(p, L.wdtype, ws, cnt, s);
}

}  // namespace xe
