// Instantiates the vectorised headwise fwd kernels for bf16.
#include "headwise_fast.h"

namespace dc {
template hipError_t dispatch_fast<bf16, false>(const HwProblem&, const HwPlan&);
}  // namespace dc
