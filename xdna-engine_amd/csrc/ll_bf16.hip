// ll_bf16.hip -- bf16-weight instantiations of the low-latency step kernel.
#include "ll_kernel.h"

namespace xe {
namespace ll {
StepFn pick_ll_bf16(int nb, int hd, int g, bool kv8) { return pick_nb<XE_BF16>(nb, hd, g, kv8); }
}  // namespace ll
}  // namespace xe
