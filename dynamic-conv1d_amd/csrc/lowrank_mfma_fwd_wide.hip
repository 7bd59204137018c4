// The lowrank forward (lowrank_mfma_fwd_kernel.h) at 9 <= W <= 16 taps with one
// or two rank chunks, and the accumulating pass over the last 16 taps of wider
// problems: the same kernel in one pass over the taps, a lane's x
// rows 4q-W+1 .. 4q+3 loaded directly (up to 19 rows) and the U operands of
// W x RC chunks staged in LDS (up to 128 KiB at W 16 with two chunks).  Its own
// translation unit, so these instantiations build in parallel with the rest.
#include "lowrank_mfma_fwd_launch.h"

namespace dc {

template <typename T>
hipError_t lr_fwd_wide_dispatch(const LrProblem* pp, int G) {
  const LrProblem& p = pp[0];
  const int rc = (int)((p.R + (p.static_w ? 1 : 0) + 15) / 16);
  if (p.accy) {  // the last 16 taps of a problem above W 16
    if (p.W != 16) return hipErrorInvalidValue;
    return rc == 1 ? launch_fwd<T, 16, 1, true>(pp, G) : rc == 2 ? launch_fwd<T, 16, 2, true>(pp, G)
                                                                : hipErrorInvalidValue;
  }
#define DC_LR_CASE(WW, CC) \
  if (p.W == WW && rc == CC) return launch_fwd<T, WW, CC>(pp, G);
  DC_LR_CASE(9, 1) DC_LR_CASE(10, 1) DC_LR_CASE(11, 1) DC_LR_CASE(12, 1)
  DC_LR_CASE(13, 1) DC_LR_CASE(14, 1) DC_LR_CASE(15, 1) DC_LR_CASE(16, 1)
  DC_LR_CASE(9, 2) DC_LR_CASE(10, 2) DC_LR_CASE(11, 2) DC_LR_CASE(12, 2)
  DC_LR_CASE(13, 2) DC_LR_CASE(14, 2) DC_LR_CASE(15, 2) DC_LR_CASE(16, 2)
#undef DC_LR_CASE
  return hipErrorInvalidValue;
}

template hipError_t lr_fwd_wide_dispatch<bf16>(const LrProblem*, int);
template hipError_t lr_fwd_wide_dispatch<fp16>(const LrProblem*, int);

}  // namespace dc
