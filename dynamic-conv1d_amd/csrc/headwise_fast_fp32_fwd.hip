// Instantiates the vectorised headwise fwd kernels for fp32.
#include "headwise_fast.h"

namespace dc {
template hipError_t dispatch_fast<float, false>(const HwProblem&, const HwPlan&);
}  // namespace dc
