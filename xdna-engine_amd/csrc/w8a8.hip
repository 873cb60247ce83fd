// w8a8.hip -- W8A8 dynamic linear, every step on the GPU.
//
// The reference's int8 CtxAOp path (forward_view_int8,
// rust/npu-asr/src/ctx2.rs:771-830) quantises the activations on the host
// (quant_scale / quant_i8, :1352-1377), runs int8 x int8 -> i32 on the NPU
// and dequantises on the host (dequant_epi, :1386-1435); the host dequant is
// the cost it names (":145-149, int8 lost to bf16 on host dequant").  Here
// the four steps are kernels on one stream:
//
//   1. amax_partial_kernel   max|a| of grid-stride slices (exact: max is
//                            associative and NaN-ignoring like f32::max)
//   2. quant_kernel          every workgroup folds the partial maxima into
//                            scale_a = amax / 127 (1.0 for an all-zero
//                            tensor), then a_i8 = round-half-away(a /
//                            scale_a) clamped to +-127 (NaN -> 0, Rust's
//                            saturating cast)
//   3. the i32 product       <= 8 rows: the sdot4 GEMV (gemv.hip); more rows
//                            (the reference's batched tiles, Mp <= 512): an
//                            int8 MFMA GEMM (v_mfma_i32_16x16x64_i8), exact
//                            integer accumulation
//   4. the epilogue          fused into the product: v = (acc * scale_a) *
//                            ws[c] (+ bias[c], or SiLU(v + bias[c]) with the
//                            reference's fast_sigmoid), in the reference's
//                            operation order; the build has no FMA
//                            contraction, so the result is the reference's
//                            bit for bit.
#include "gemv_dev.h"

namespace xe {
namespace {

constexpr int kT = 256;
constexpr int kAmaxBlocks = 64;
constexpr int kNoRec = 0x7ffffff0;  // past every buffer: loads return zeros

typedef int i32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float block_max(float v) {
  __shared__ float red[kT / 64];
  v = gdev::wave_max(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float m = red[0];
#pragma unroll
  for (int w = 1; w < kT / 64; w++) m = fmaxf(m, red[w]);
  return m;
}

__global__ __launch_bounds__(kT) void amax_partial_kernel(const float *__restrict__ a, size_t n,
                                                          float *__restrict__ partial) {
  float m = 0.f;
  for (size_t i = static_cast<size_t>(blockIdx.x) * kT + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * kT)
    m = fmaxf(m, fabsf(a[i]));
  m = block_max(m);
  if (threadIdx.x == 0) partial[blockIdx.x] = m;
}

__device__ __forceinline__ float scale_from_partials(const float *partial) {
  float amax = 0.f;
#pragma unroll 8
  for (int i = 0; i < kAmaxBlocks; i++) amax = fmaxf(amax, partial[i]);
  return amax > 0.0f ? amax / 127.0f : 1.0f;
}

__global__ __launch_bounds__(kT) void quant_kernel(const float *__restrict__ a, size_t n,
                                                   const float *__restrict__ partial,
                                                   int8_t *__restrict__ aq, float *__restrict__ scale_out) {
  const float sa = scale_from_partials(partial);
  if (blockIdx.x == 0 && threadIdx.x == 0) scale_out[0] = sa;
  for (size_t i = static_cast<size_t>(blockIdx.x) * kT + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * kT) {
    float v = roundf(a[i] / sa);
    if (v != v) v = 0.0f;
    v = v < -127.0f ? -127.0f : (v > 127.0f ? 127.0f : v);
    aq[i] = static_cast<int8_t>(v);
  }
}

// int8 MFMA GEMM: acc[b, r] = sum_k aq[b, k] * wq[r, k].  Workgroup: 4 waves
// x 16 weight rows, NJ blocks of 16 activation rows; K in steps of 64 (one
// v_mfma_i32_16x16x64_i8 per column block).  A lane loads 16 consecutive k of
// its weight row and of its activation row at the same k offset (both
// operands use the same k assignment, so the integer dot products are exact
// whatever order the instruction sums them in).  Rows past m / batch and k
// past K read zeros (buffer loads with an out-of-range offset).
template <int NJ>
__global__ __launch_bounds__(kT) void w8a8_mfma_kernel(const int8_t *__restrict__ wq, const int8_t *__restrict__ aq,
                                                       int m, int k, int batch, W8a8Epi e) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r0 = blockIdx.x * 64 + wave * 16;
  const int b0 = blockIdx.y * 16 * NJ;
  const __amdgpu_buffer_rsrc_t rw = gdev::coherent_rsrc(wq);
  const __amdgpu_buffer_rsrc_t ra = gdev::coherent_rsrc(aq);
  const int row = r0 + (lane & 15);
  const int kl = 16 * (lane >> 4);
  const bool row_ok = row < m;
  int brow[NJ];
  bool b_ok[NJ];
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    brow[j] = b0 + 16 * j + (lane & 15);
    b_ok[j] = brow[j] < batch;
  }
  i32x4 acc[NJ];
#pragma unroll
  for (int j = 0; j < NJ; j++) acc[j] = i32x4{0, 0, 0, 0};
  constexpr int U = 4;  // K steps whose loads are in flight together
  const int nsteps = (k + 63) / 64;
  for (int s0 = 0; s0 < nsteps; s0 += U) {
    i32x4 wa[U], xb[U][NJ];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int kk = (s0 + u) * 64 + kl;
      const bool k_ok = kk < k;
      wa[u] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                            rw, (row_ok && k_ok) ? row * k + kk : kNoRec, 0, 2));
#pragma unroll
      for (int j = 0; j < NJ; j++)
        xb[u][j] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                 ra, (b_ok[j] && k_ok) ? brow[j] * k + kk : kNoRec, 0, 0));
    }
#pragma unroll
    for (int u = 0; u < U; u++)
#pragma unroll
      for (int j = 0; j < NJ; j++)
        acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wa[u], xb[u][j], acc[j], 0, 0, 0);
  }
  // lane holds weight rows r0 + 4 * (lane / 16) + i of activation row
  // b0 + 16 j + lane % 16
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    const int b = brow[j];
    if (b >= batch) continue;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int r = r0 + 4 * (lane >> 4) + i;
      if (r < m) w8a8_store(e, b, r, m, acc[j][i]);
    }
  }
}

}  // namespace

void launch_w8a8_quant(const float *a, size_t n, float *partial, int8_t *aq, float *scale_out,
                       hipStream_t s) {
  XE_REQUIRE(n > 0, "w8a8: empty activation tensor");
  hipLaunchKernelGGL(amax_partial_kernel, dim3(kAmaxBlocks), dim3(kT), 0, s, a, n, partial);
  XE_HIP(hipGetLastError());
  const size_t blocks = std::min<size_t>((n + kT * 4 - 1) / (kT * 4), 4 * gdev::cu_count());
  hipLaunchKernelGGL(quant_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kT), 0, s, a, n, partial, aq,
                     scale_out);
  XE_HIP(hipGetLastError());
}

size_t w8a8_partial_floats() { return kAmaxBlocks; }

void launch_w8a8_mfma(const int8_t *wq, const int8_t *aq, int m, int k, int batch, const W8a8Epi &e,
                      hipStream_t s) {
  XE_REQUIRE(m > 0 && k > 0 && batch > 0, "w8a8 gemm: empty shape");
  XE_REQUIRE(k % 16 == 0, "w8a8 gemm: K must be a multiple of 16");
  XE_REQUIRE(static_cast<size_t>(m) * k < (size_t(1) << 31) && static_cast<size_t>(batch) * k < (size_t(1) << 31),
             "w8a8 gemm: operand above 2 GB");
  const int nj = batch <= 16 ? 1 : batch <= 32 ? 2 : 4;
  const dim3 grid((m + 63) / 64, (batch + 16 * nj - 1) / (16 * nj));
  if (nj == 1) hipLaunchKernelGGL(w8a8_mfma_kernel<1>, grid, dim3(kT), 0, s, wq, aq, m, k, batch, e);
  else if (nj == 2) hipLaunchKernelGGL(w8a8_mfma_kernel<2>, grid, dim3(kT), 0, s, wq, aq, m, k, batch, e);
  else hipLaunchKernelGGL(w8a8_mfma_kernel<4>, grid, dim3(kT), 0, s, wq, aq, m, k, batch, e);
  XE_HIP(hipGetLastError());
}

}  // namespace xe
