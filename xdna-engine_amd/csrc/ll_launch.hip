// ll_launch.hip -- host side of the low-latency step kernel: kernel choice
// and the cooperative launch (the exchange protocol needs every workgroup
// resident at once; a cooperative launch fails instead of running a grid that
// does not fit).
#include "ll_kernel.h"

namespace xe {
namespace ll {

namespace {
StepFn pick(int wdtype, int nb_t, int hd, int g, bool kv8) {
  switch (wdtype) {
    case XE_I8: return pick_ll_i8(nb_t, hd, g, kv8);
    case XE_BF16: return pick_ll_bf16(nb_t, hd, g, kv8);
    case XE_BFP16: return pick_ll_bfp16(nb_t, hd, g, kv8);
  }
  return nullptr;
}
}  // namespace

bool step_supported(int wdtype, int nb_t, int hd, int g, bool kv8) {
  return pick(wdtype, nb_t, hd, g, kv8) != nullptr;
}

void launch(const StepParams &sp, int wdtype, int nb_t, int hd, int g, bool kv8, size_t lds_bytes, int grid,
            hipStream_t s) {
  StepFn fn = pick(wdtype, nb_t, hd, g, kv8);
  XE_REQUIRE(fn, "low-latency step: unsupported (weight dtype, batch, head_dim, group)");
  XE_REQUIRE(lds_bytes <= 160 * 1024 - 2048, "low-latency step: LDS need too large");
  XE_REQUIRE(sp.nb >= 1 && sp.nb <= nb_t && nb_t <= kMaxNB, "low-latency step: bad stream count");
  const void *f = reinterpret_cast<const void *>(fn);
  if (lds_bytes > 64 * 1024)
    XE_HIP(hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds_bytes)));
  int per_cu = 0;
  XE_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, f, kT, lds_bytes));
  XE_REQUIRE(per_cu >= 1, "low-latency step: the kernel does not fit on a CU");
  StepParams arg = sp;
  void *args[] = {&arg};
  XE_HIP(hipLaunchCooperativeKernel(f, dim3(grid), dim3(kT), args, static_cast<unsigned>(lds_bytes), s));
}

}  // namespace ll
}  // namespace xe
