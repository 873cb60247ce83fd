// persist.hip -- executors of a decode step's phase list (step_dev.h).
//
// launch_phase: one standalone kernel per phase (the HIP-graph path).
// launch_step:  host side of the persistent step kernel (step_kernel.h), one
//   launch per token.
#include "step_kernel.h"

namespace xe {
namespace {

using skern::StepFn;
using namespace skern;

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

StepFn pick_step(int wdtype, int nb, int hd, int g) {
  switch (wdtype) {
    case XE_I8: return pick_step_i8(nb, hd, g);
    case XE_BF16: return pick_step_bf16(nb, hd, g);
    case XE_BFP16: return pick_step_bfp16(nb, hd, g);
  }
  return nullptr;
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

bool step_kernel_supported(int wdtype, int nb, int hd, int g) {
  return pick_step(wdtype, nb, hd, g) != nullptr;
}

void launch_step(const StepLaunch &L, hipStream_t s) {
  StepFn fn = pick_step(L.wdtype, L.nb, L.hd, L.g);
  XE_REQUIRE(fn, "step kernel: unsupported (weight dtype, batch, head_dim, group)");
  XE_REQUIRE(L.lds_bytes <= 160 * 1024 - 4096, "step kernel: LDS need too large");
  if (L.lds_bytes > 64 * 1024)
    XE_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(fn),
                               hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(L.lds_bytes)));
  // One workgroup per CU: the grid must be co-resident for the flag barrier.
  // Check that the kernel's resources allow it rather than assuming.
  int per_cu = 0;
  XE_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(fn),
                                                      kStepThreads, L.lds_bytes));
  XE_REQUIRE(per_cu >= 1, "step kernel: does not fit on a CU");
  hipLaunchKernelGGL(fn, dim3(L.grid), dim3(kStepThreads), L.lds_bytes, s, L.phases, L.nphases,
                     L.flags, L.status, L.trace);
  XE_HIP(hipGetLastError());
}

}  // namespace xe
