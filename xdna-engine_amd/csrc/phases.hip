// phases.hip -- standalone kernels of a decode step's phase list (step_dev.h):
// launch_phase runs one phase as its own kernel (the HIP-graph and eager
// executors); the GEMV, GEMM and attention phases launch the kernels of
// gemv.hip, gemm.hip and attn.hip.
#include "step_dev.h"

namespace xe {
namespace {

// ---- standalone kernels for the non-GEMV/attention phases ----
__global__ __launch_bounds__(256) void embed_kernel(sdev::EmbedParams p) {
  sdev::embed_block<false>(p, blockIdx.x);
}
__global__ __launch_bounds__(256) void argmax_part_kernel(sdev::ArgmaxParams p) {
  __shared__ float lds[512];
  sdev::argmax_part_block<false>(p, blockIdx.x, lds);
}
__global__ __launch_bounds__(64) void argmax_final_kernel(sdev::ArgmaxParams p) {
  sdev::argmax_final_block<false>(p, blockIdx.x);
}

}  // namespace

void launch_gemv_phase(const sdev::Phase &ph, hipStream_t s);
void launch_attn_phase(const sdev::Phase &ph, hipStream_t s);

void launch_phase(const sdev::Phase &ph, hipStream_t s) {
  switch (ph.kind) {
    case sdev::PH_GEMV: launch_gemv_phase(ph, s); return;
    case sdev::PH_GEMM_PRO: launch_gemm_prologue(ph.u.gemv, ph.xn, s); return;
    case sdev::PH_GEMM: launch_gemm(ph.u.gemv, ph.variant, ph.ws, ph.cnt, s); return;
    case sdev::PH_ATTN:
    case sdev::PH_MERGE: launch_attn_phase(ph, s); return;
    case sdev::PH_EMBED:
      hipLaunchKernelGGL(embed_kernel, dim3(ph.nblocks), dim3(256), 0, s, ph.u.emb);
      break;
    case sdev::PH_ARGMAX_PART:
      hipLaunchKernelGGL(argmax_part_kernel, dim3(ph.nblocks), dim3(256), 0, s, ph.u.arg);
      break;
    case sdev::PH_ARGMAX_FINAL:
      hipLaunchKernelGGL(argmax_final_kernel, dim3(ph.nblocks), dim3(64), 0, s, ph.u.arg);
      break;
    default: fail("unknown phase kind");
  }
  XE_HIP(hipGetLastError());
}

}  // namespace xe
