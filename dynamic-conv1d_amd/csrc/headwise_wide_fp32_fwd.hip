// Wide-W headwise kernels (headwise_wide.h), fp32 forward.
#include "headwise_wide.h"

namespace dc {
template hipError_t dispatch_wide<float, false>(const HwProblem&, const HwWideArgs&);
}  // namespace dc
