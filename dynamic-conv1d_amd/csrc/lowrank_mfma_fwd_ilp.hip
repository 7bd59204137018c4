// The lowrank forward kernel (lowrank_mfma_fwd_kernel.h) for one rank chunk
// without the z_eff writer, built with the scheduler's ILP strategy
// (`-mllvm -amdgpu-sched-strategy=max-ilp`, build.py): it interleaves each
// tap's eight MFMAs with the FMAs of the previous results and batches the
// operand reads, where the default schedule pairs each MFMA with its own uses
// and pads with s_nop.  B4 T4096 D2048 R16 W4 forward 29.0 -> 27.8 us, W8
// 38.6 -> 36.0 us; W1-3 and W5 unchanged.  It takes up to 149 VGPRs (three
// wavefronts per SIMD), so launches above kFwdIlpMaxWaves wavefronts keep the
// default build; the launch plan gives this build at most two wavefronts per
// SIMD (B2 T8192 D4096 R16: 50.7 us at 2048 wavefronts, 59.7 us at 3072, 54.3 us
// for the default build at 4096).
#include "lowrank_mfma_fwd_kernel.h"

namespace dc {

template <typename T, int W>
hipError_t lr_fwd_ilp_launch(const LrArgs& a, hipStream_t stream) {
  if (a.zvec)
    lr_fwd_mfma<T, W, 1, true, false, true><<<a.nblk, 256, 0, stream>>>(a);
  else
    lr_fwd_mfma<T, W, 1, false, false, true><<<a.nblk, 256, 0, stream>>>(a);
  return hipGetLastError();
}

#define DC_FWD_ILP(TT, WW) template hipError_t lr_fwd_ilp_launch<TT, WW>(const LrArgs&, hipStream_t);
DC_FWD_ILP(bf16, 1) DC_FWD_ILP(bf16, 2) DC_FWD_ILP(bf16, 3) DC_FWD_ILP(bf16, 4)
DC_FWD_ILP(bf16, 5) DC_FWD_ILP(bf16, 6) DC_FWD_ILP(bf16, 7) DC_FWD_ILP(bf16, 8)
DC_FWD_ILP(fp16, 1) DC_FWD_ILP(fp16, 2) DC_FWD_ILP(fp16, 3) DC_FWD_ILP(fp16, 4)
DC_FWD_ILP(fp16, 5) DC_FWD_ILP(fp16, 6) DC_FWD_ILP(fp16, 7) DC_FWD_ILP(fp16, 8)
#undef DC_FWD_ILP

}  // namespace dc
