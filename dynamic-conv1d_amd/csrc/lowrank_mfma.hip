// Lowrank dynamic convolution on bf16/fp16 MFMA (gfx950).  Filled in below.
#include "dc_common.h"
#include "dc_launch.h"

namespace dc {

bool lr_mfma_ok_impl(const LrProblem&, bool) { return false; }
int64_t lr_mfma_ws_bytes(const LrProblem&) { return 0; }
hipError_t lr_mfma_fwd(const LrProblem&) { return hipErrorInvalidValue; }
hipError_t lr_mfma_bwd(const LrProblem&) { return hipErrorInvalidValue; }

}  // namespace dc
