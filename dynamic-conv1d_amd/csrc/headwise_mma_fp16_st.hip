// hw_bwd_mma and hw_fwd_mma (headwise_mma.h) for fp16, with the static filter: one
// translation unit per dtype and static filter, so the instantiations build in parallel.
#include "headwise_mma.h"

namespace dc {

template <>
hipError_t hw_bwd_mma_launch<fp16, true>(const HwProblem& p, const HwMmaArgs& a, int hs) {
  const fp16* x = (const fp16*)p.x;
  const fp16* w = (const fp16*)p.weight;
  const fp16* sw = (const fp16*)p.static_w;
  const fp16* dy = (const fp16*)p.dy;
  fp16* dx = (fp16*)p.dx;
  fp16* dw = (fp16*)p.dweight;
#define DC_MMA(HS, WW)                                                                                   \
  if (hs == HS && p.W == WW) {                                                                           \
    hw_bwd_mma<fp16, WW, HS, true><<<a.nblk, 64, 0, p.stream>>>(x, w, sw, dy, dx, dw, p.ws, a);       \
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
hipError_t hw_fwd_mma_launch<fp16, true>(const HwProblem& p, const HwMmaArgs& a, int hs) {
  const fp16* x = (const fp16*)p.x;
  const fp16* w = (const fp16*)p.weight;
  const fp16* sw = (const fp16*)p.static_w;
  fp16* y = (fp16*)p.y;
#define DC_MMA(HS, WW)                                                                  \
  if (hs == HS && p.W == WW) {                                                          \
    hw_fwd_mma<fp16, WW, HS, true><<<a.nblk, 64, 0, p.stream>>>(x, w, sw, y, a);      \
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
