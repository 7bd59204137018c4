// Wide-W headwise kernels (headwise_wide.h), fp16 backward.
#include "headwise_wide.h"

namespace dc {
template hipError_t dispatch_wide<fp16, true>(const HwProblem&, const HwWideArgs&);
}  // namespace dc
