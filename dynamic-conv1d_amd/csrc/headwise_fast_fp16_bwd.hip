// Instantiates the vectorised headwise bwd kernels for fp16.
#include "headwise_fast.h"

namespace dc {
template hipError_t dispatch_fast<fp16, true>(const HwProblem&, const HwPlan&);
}  // namespace dc
