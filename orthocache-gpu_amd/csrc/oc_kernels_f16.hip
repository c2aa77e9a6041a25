// Kernel instantiations for K/V element type OC_F16.
#include "oc_kernels.h"

namespace oc {
OC_DEFINE_LAUNCHERS(OC_F16)
}  // namespace oc
