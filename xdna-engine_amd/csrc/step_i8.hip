// step_i8.hip -- persistent step kernels for i8 weights.
#include "step_kernel.h"

namespace xe {
namespace skern {

StepFn pick_step_i8(int nb, int hd, int g) { return pick_nb<XE_I8>(nb, hd, g); }

}  // namespace skern
}  // namespace xe
