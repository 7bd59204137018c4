// Instantiates the vectorised headwise fwd kernels for fp16.
#include "headwise_fast.h"

namespace dc {
template hipError_t dispatch_fast<fp16, false>(const HwProblem&, const HwPlan&);
}  // namespace dc
