// Lowrank forward on gfx950 matrix cores (bf16 / fp16): y from x, z, U (and static_w).
// Host side: launch plans and dispatch; the kernel is in lowrank_mfma_fwd_kernel.h.
#include "lowrank_mfma_fwd_launch.h"

namespace dc {

// ------------------------------------------------------------------- host
// Longest forward run (tiles) whose resources fit (see run_rsrc): rows of x, y,
// z and z_eff; with head-major y a wavefront's resource also spans the blocks
// of the heads its 128 channels touch (up to 127 / hd + 1 more, T rows each).
int64_t lr_fwd_max_run_tiles(const LrProblem& p) {
  const int64_t hd = p.yhd();
  int64_t rowb = p.xld() * 2;
  rowb = rowb > hd * 2 ? rowb : hd * 2;
  rowb = rowb > p.R * 2 ? rowb : p.R * 2;
  const int64_t zrp = p.zeff ? lr_bwd_zrow(p.R, p.static_w != nullptr) : 0;
  rowb = rowb > zrp * 2 ? rowb : zrp * 2;
  int64_t tiles = run_tiles_cap(rowb);
  if (hd != p.D) {
    // head-major y: rows of the other heads' blocks come first in its offsets
    const int64_t extra = (127 / hd + 1) * p.T * hd * 2;
    const int64_t rows = (kMaxSeqBytes - extra) / (hd * 2) - kSeqSlackRows - kRunHaloRows - 32;
    const int64_t yt = rows > 0 ? rows / 16 : 0;
    tiles = tiles < yt ? tiles : yt;
  }
  return tiles;
}

namespace {

template <typename T>
hipError_t dispatch_fwd(const LrProblem* pp, int G);

// Taps per forward pass: what one launch stages (W x RC operand chunks in LDS).
constexpr int fwd_pass_taps(int rc) { return rc <= 2 ? 16 : 8; }

// Wider problems (above W 16 at one or two rank chunks, above W 8 at three or
// four) as passes of taps: taps 0 .. W0-1 as a W0-tap problem (residual and
// z_eff included), then passes of P = fwd_pass_taps taps, each on x read kofs
// rows earlier and added to the stored y (accy).  U keeps its row stride W * D;
// a later pass's U and static_w start at its tap kofs.  y is rounded to the
// output type after each pass (two passes at W <= 32 and one or two rank
// chunks, up to four at W 32 and three or four).
template <typename T>
hipError_t dispatch_fwd_passes(const LrProblem* pp, int G, int P) {
  const int W = (int)pp[0].W, np = (W + P - 1) / P, w0 = W - (np - 1) * P;
  LrProblem a[kMaxGroups];
  for (int g = 0; g < G; ++g) {
    a[g] = pp[g];
    a[g].W = w0;
    a[g].u_ld = pp[g].uld();
  }
  hipError_t e = dispatch_fwd<T>(a, G);
  for (int ps = 1; ps < np && e == hipSuccess; ++ps) {
    const int kofs = w0 + (ps - 1) * P;
    for (int g = 0; g < G; ++g) {
      const LrProblem& p = pp[g];
      a[g] = p;
      a[g].W = P;
      a[g].u_ld = p.uld();
      a[g].kofs = kofs;
      a[g].accy = 1;
      a[g].U = static_cast<const T*>(p.U) + (int64_t)kofs * p.D;
      a[g].static_w = p.static_w ? static_cast<const T*>(p.static_w) + (int64_t)kofs * p.D : nullptr;
      a[g].residual = 0;
      a[g].zeff = nullptr;
    }
    e = dispatch_fwd<T>(a, G);
  }
  return e;
}

template <typename T>
hipError_t dispatch_fwd(const LrProblem* pp, int G) {
  const LrProblem& p = pp[0];
  const int rc = (int)((p.R + (p.static_w ? 1 : 0) + 15) / 16);
  if (p.accy) {  // a later pass: the accumulating kernels of fwd_pass_taps(rc) taps
    if (rc <= 2) return lr_fwd_wide_dispatch<T>(pp, G);
    if (p.W != 8) return hipErrorInvalidValue;
    return rc == 3 ? launch_fwd<T, 8, 3, true>(pp, G) : launch_fwd<T, 8, 4, true>(pp, G);
  }
  if (p.W > fwd_pass_taps(rc)) return dispatch_fwd_passes<T>(pp, G, fwd_pass_taps(rc));
#define DC_LR_CASE(WW, CC) \
  if (p.W == WW && rc == CC) return launch_fwd<T, WW, CC>(pp, G);
  DC_LR_CASE(1, 1) DC_LR_CASE(1, 2) DC_LR_CASE(1, 3) DC_LR_CASE(1, 4)
  DC_LR_CASE(2, 1) DC_LR_CASE(2, 2) DC_LR_CASE(2, 3) DC_LR_CASE(2, 4)
  DC_LR_CASE(3, 1) DC_LR_CASE(3, 2) DC_LR_CASE(3, 3) DC_LR_CASE(3, 4)
  DC_LR_CASE(4, 1) DC_LR_CASE(4, 2) DC_LR_CASE(4, 3) DC_LR_CASE(4, 4)
  DC_LR_CASE(5, 1) DC_LR_CASE(5, 2) DC_LR_CASE(5, 3) DC_LR_CASE(5, 4)
  DC_LR_CASE(6, 1) DC_LR_CASE(6, 2) DC_LR_CASE(6, 3) DC_LR_CASE(6, 4)
  DC_LR_CASE(7, 1) DC_LR_CASE(7, 2) DC_LR_CASE(7, 3) DC_LR_CASE(7, 4)
  DC_LR_CASE(8, 1) DC_LR_CASE(8, 2) DC_LR_CASE(8, 3) DC_LR_CASE(8, 4)
#undef DC_LR_CASE
  if (p.W > 8) return lr_fwd_wide_dispatch<T>(pp, G);
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t lr_mfma_fwd(const LrProblem* p, int G) {
  return p[0].dtype == kBF16 ? dispatch_fwd<bf16>(p, G) : dispatch_fwd<fp16>(p, G);
}

}  // namespace dc
