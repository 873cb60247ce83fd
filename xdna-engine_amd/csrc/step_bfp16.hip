// step_bfp16.hip -- persistent step kernels for bfp16 weights.
#include "step_kernel.h"

namespace xe {
namespace skern {

StepFn pick_step_bfp16(int nb, int hd, int g) { return pick_nb<XE_BFP16>(nb, hd, g); }

}  // namespace skern
}  // namespace xe
