// Wide-W headwise kernels (headwise_wide.h), fp32 backward.
#include "headwise_wide.h"

namespace dc {
template hipError_t dispatch_wide<float, true>(const HwProblem&, const HwWideArgs&);
}  // namespace dc
