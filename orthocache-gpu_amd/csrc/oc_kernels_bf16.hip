// Kernel instantiations for K/V element type OC_BF16.
#include "oc_kernels.h"

namespace oc {
OC_DEFINE_LAUNCHERS(OC_BF16)
}  // namespace oc
