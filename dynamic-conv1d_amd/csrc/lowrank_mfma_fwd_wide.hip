// The lowrank forward (lowrank_mfma_fwd_kernel.h) at 9 <= W <= 16 taps with one
// or two rank chunks and 17 <= W <= 32 with one, and the accumulating pass over
// the last 16 taps of wider problems at two rank chunks: the same kernel in one
// pass over the taps, a lane's x rows 4q-W+1 .. 4q+3 loaded directly (up to 35
// rows) and the U operands of W x RC chunks staged in LDS (up to 128 KiB at W
// 16 with two chunks or W 32 with one, on 8-wavefront workgroups).  Its own
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
  DC_LR_CASE(17, 1) DC_LR_CASE(18, 1) DC_LR_CASE(19, 1) DC_LR_CASE(20, 1)
  DC_LR_CASE(21, 1) DC_LR_CASE(22, 1) DC_LR_CASE(23, 1) DC_LR_CASE(24, 1)
  DC_LR_CASE(25, 1) DC_LR_CASE(26, 1) DC_LR_CASE(27, 1) DC_LR_CASE(28, 1)
  DC_LR_CASE(29, 1) DC_LR_CASE(30, 1) DC_LR_CASE(31, 1) DC_LR_CASE(32, 1)
#undef DC_LR_CASE
  return hipErrorInvalidValue;
}

template hipError_t lr_fwd_wide_dispatch<bf16>(const LrProblem*, int);
template hipError_t lr_fwd_wide_dispatch<fp16>(const LrProblem*, int);

}  // namespace dc
