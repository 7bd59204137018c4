// hw_bwd_mma and hw_fwd_mma (headwise_mma.h) for bf16, without the static filter: one
// translation unit per dtype and static filter, so the instantiations build in parallel.
#include "headwise_mma.h"

namespace dc {

template <>
hipError_t hw_bwd_mma_launch<bf16, false>(const HwProblem& p, const HwMmaArgs& a, int hs) {
  const bf16* x = (const bf16*)p.x;
  const bf16* w = (const bf16*)p.weight;
  const bf16* sw = (const bf16*)p.static_w;
  const bf16* dy = (const bf16*)p.dy;
  bf16* dx = (bf16*)p.dx;
  bf16* dw = (bf16*)p.dweight;
#define DC_MMA(HS, WW)                                                                                   \
  if (hs == HS && p.W == WW) {                                                                           \
    hw_bwd_mma<bf16, WW, HS, false><<<a.nblk, 64, 0, p.stream>>>(x, w, sw, dy, dx, dw, p.ws, a);       \
    return hipGetLastError();                                                                            \
  }
  DC_MMA(16, 10) DC_MMA(16, 12) DC_MMA(16, 14) DC_MMA(16, 16) DC_MMA(16, 18) DC_MMA(16, 20)
  DC_MMA(16, 22) DC_MMA(16, 24) DC_MMA(16, 26) DC_MMA(16, 28) DC_MMA(16, 30) DC_MMA(16, 32)
  DC_MMA(32, 12) DC_MMA(32, 16) DC_MMA(32, 20) DC_MMA(32, 24) DC_MMA(32, 28) DC_MMA(32, 32)
  DC_MMA(64, 16) DC_MMA(64, 24) DC_MMA(64, 32)
  DC_MMA(8, 9) DC_MMA(8, 10) DC_MMA(8, 11) DC_MMA(8, 12) DC_MMA(8, 13) DC_MMA(8, 14) DC_MMA(8, 15) DC_MMA(8, 16) DC_MMA(8, 17) DC_MMA(8, 18) DC_MMA(8, 19) DC_MMA(8, 20)
  DC_MMA(8, 21) DC_MMA(8, 22) DC_MMA(8, 23) DC_MMA(8, 24) DC_MMA(8, 25) DC_MMA(8, 26) DC_MMA(8, 27) DC_MMA(8, 28) DC_MMA(8, 29) DC_MMA(8, 30) DC_MMA(8, 31) DC_MMA(8, 32)
#undef DC_MMA
  return hipErrorInvalidValue;
}

template <>
hipError_t hw_fwd_mma_launch<bf16, false>(const HwProblem& p, const HwMmaArgs& a, int hs) {
  const bf16* x = (const bf16*)p.x;
  const bf16* w = (const bf16*)p.weight;
  const bf16* sw = (const bf16*)p.static_w;
  bf16* y = (bf16*)p.y;
#define DC_MMA(HS, WW)                                                                  \
  if (hs == HS && p.W == WW) {                                                          \
    hw_fwd_mma<bf16, WW, HS, false><<<a.nblk, 64, 0, p.stream>>>(x, w, sw, y, a);      \
    return hipGetLastError();                                                           \
  }
  DC_MMA(16, 10) DC_MMA(16, 12) DC_MMA(16, 14) DC_MMA(16, 16) DC_MMA(16, 18) DC_MMA(16, 20)
  DC_MMA(16, 22) DC_MMA(16, 24) DC_MMA(16, 26) DC_MMA(16, 28) DC_MMA(16, 30) DC_MMA(16, 32)
  DC_MMA(32, 12) DC_MMA(32, 16) DC_MMA(32, 20) DC_MMA(32, 24) DC_MMA(32, 28) DC_MMA(32, 32)
  DC_MMA(64, 16) DC_MMA(64, 24) DC_MMA(64, 32)
  DC_MMA(8, 9) DC_MMA(8, 10) DC_MMA(8, 11) DC_MMA(8, 12) DC_MMA(8, 13) DC_MMA(8, 14) DC_MMA(8, 15) DC_MMA(8, 16) DC_MMA(8, 17) DC_MMA(8, 18) DC_MMA(8, 19) DC_MMA(8, 20)
  DC_MMA(8, 21) DC_MMA(8, 22) DC_MMA(8, 23) DC_MMA(8, 24) DC_MMA(8, 25) DC_MMA(8, 26) DC_MMA(8, 27) DC_MMA(8, 28) DC_MMA(8, 29) DC_MMA(8, 30) DC_MMA(8, 31) DC_MMA(8, 32)
#undef DC_MMA
  return hipErrorInvalidValue;
}

}  // namespace dc
