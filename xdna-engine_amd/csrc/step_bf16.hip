// step_bf16.hip -- persistent step kernels for bf16 weights.
#include "step_kernel.h"

namespace xe {
namespace skern {

StepFn pick_step_bf16(int nb, int hd, int g) { return pick_nb<XE_BF16>(nb, hd, g); }

}  // namespace skern
}  // namespace xe
