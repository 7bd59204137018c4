// Instantiates the vectorised headwise bwd kernels for fp32.
#include "headwise_fast.h"

namespace dc {
template hipError_t dispatch_fast<float, true>(const HwProblem&, const HwPlan&);
}  // namespace dc
