// Instantiates the vectorised headwise bwd kernels for bf16.
#include "headwise_fast.h"

namespace dc {
template hipError_t dispatch_fast<bf16, true>(const HwProblem&, const HwPlan&);
}  // namespace dc
