// The lowrank forward (lowrank_mfma_fwd_kernel.h) as an accumulating pass
// (ACC: the tile's y rows, as the earlier passes stored them, are added before
// the store) at W <= 8 and one to four rank chunks (up to eight at W <= 4):
// the passes of 8 taps of problems above W 8 at three or four rank chunks, and
// every pass after the first of a problem above fwd_rank_pass(W) kernel ranks
// (passes of 128 ranks up to W 4, of 64 above).  Its own translation unit, so
// these instantiations build in parallel with the rest.
#include "lowrank_mfma_fwd_launch.h"

namespace dc {

template <typename T>
hipError_t lr_fwd_acc_dispatch(const LrProblem* pp, int G) {
  const LrProblem& p = pp[0];
  const int rc = (int)((p.R + (p.static_w ? 1 : 0) + 15) / 16);
  if (!p.accy) return hipErrorInvalidValue;
#define DC_LR_CASE(WW, CC) \
  if (p.W == WW && rc == CC) return launch_fwd<T, WW, CC, true>(pp, G);
  DC_LR_CASE(1, 1) DC_LR_CASE(1, 2) DC_LR_CASE(1, 3) DC_LR_CASE(1, 4)
  DC_LR_CASE(2, 1) DC_LR_CASE(2, 2) DC_LR_CASE(2, 3) DC_LR_CASE(2, 4)
  DC_LR_CASE(3, 1) DC_LR_CASE(3, 2) DC_LR_CASE(3, 3) DC_LR_CASE(3, 4)
  DC_LR_CASE(4, 1) DC_LR_CASE(4, 2) DC_LR_CASE(4, 3) DC_LR_CASE(4, 4)
  DC_LR_CASE(5, 1) DC_LR_CASE(5, 2) DC_LR_CASE(5, 3) DC_LR_CASE(5, 4)
  DC_LR_CASE(6, 1) DC_LR_CASE(6, 2) DC_LR_CASE(6, 3) DC_LR_CASE(6, 4)
  DC_LR_CASE(7, 1) DC_LR_CASE(7, 2) DC_LR_CASE(7, 3) DC_LR_CASE(7, 4)
  DC_LR_CASE(8, 1) DC_LR_CASE(8, 2) DC_LR_CASE(8, 3) DC_LR_CASE(8, 4)
  DC_LR_CASE(1, 5) DC_LR_CASE(1, 6) DC_LR_CASE(1, 7) DC_LR_CASE(1, 8)
  DC_LR_CASE(2, 5) DC_LR_CASE(2, 6) DC_LR_CASE(2, 7) DC_LR_CASE(2, 8)
  DC_LR_CASE(3, 5) DC_LR_CASE(3, 6) DC_LR_CASE(3, 7) DC_LR_CASE(3, 8)
  DC_LR_CASE(4, 5) DC_LR_CASE(4, 6) DC_LR_CASE(4, 7) DC_LR_CASE(4, 8)
#undef DC_LR_CASE
  return hipErrorInvalidValue;
}

template hipError_t lr_fwd_acc_dispatch<bf16>(const LrProblem*, int);
template hipError_t lr_fwd_acc_dispatch<fp16>(const LrProblem*, int);

}  // namespace dc
