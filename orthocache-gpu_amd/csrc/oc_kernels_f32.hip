// Kernel instantiations for K/V element type OC_F32.
#include "oc_kernels.h"

namespace oc {
OC_DEFINE_LAUNCHERS(OC_F32)
}  // namespace oc
