// Kernel instantiations for K/V element type OC_FP8_E4M3FN.
#include "oc_kernels.h"

namespace oc {
OC_DEFINE_LAUNCHERS(OC_FP8_E4M3FN)
}  // namespace oc
