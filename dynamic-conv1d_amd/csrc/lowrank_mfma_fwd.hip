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
  rowb = rowb > p.zld() * 2 ? rowb : p.zld() * 2;  // z rows (a pass of ranks: the whole problem's)
  const int64_t zrp = p.zeff ? lr_zeff_rows(p) : 0;
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

// Taps per forward pass: what one launch stages (W x RC operand chunks in LDS,
// up to 128 KiB on 8-wavefront workgroups): one rank chunk up to W 32 in one
// pass, two up to 16, three or four up to 8.
constexpr int fwd_pass_taps(int rc) { return rc == 1 ? 32 : rc == 2 ? 16 : 8; }

// The passes of a forward launch sequence (fwd_plan).  Up to kernel rank 64
// one pass of ranks; wider problems (above W 32 at one rank chunk, above
// W 16 at two, above W 8 at three or four) run as passes of taps: taps 0 .. W0-1 as a
// W0-tap problem (residual and z_eff included), then passes of P =
// fwd_pass_taps taps, each on x read kofs rows earlier and added to the stored
// y (accy).  Above fwd_rank_pass(W) kernel ranks, passes of that many (z
// columns rofs .. of its rows, U rows rofs .., the static rank in the pass that
// holds index R), each split into passes of at most 8 taps, every pass after
// the first adding to the stored y.  y is rounded to the output type after
// each pass; lr_mfma_ok admits at most kFwdMaxPasses of them.
int fwd_plan(const LrProblem& p, FwdPass* out) {
  const int RK = (int)(p.R + (p.static_w ? 1 : 0)), W = (int)p.W, RP = fwd_rank_pass(W);
  const bool ranks = RK > RP;
  int n = 0;
  for (int rofs = 0; rofs < RK; rofs += RP) {
    const int rk = RK - rofs < RP ? RK - rofs : RP;  // kernel ranks of the pass
    const int rd = (int)p.R - rofs < 0 ? 0 : ((int)p.R - rofs < rk ? (int)p.R - rofs : rk);  // dynamic ones
    const int P = ranks ? 8 : fwd_pass_taps((rk + 15) / 16);
    const int nt = W <= P ? 1 : (W + P - 1) / P, w0 = W - (nt - 1) * P;
    for (int i = 0; i < nt; ++i) {
      if (n == kFwdMaxPlan) return -1;
      FwdPass& f = out[n++];
      f.rofs = rofs;
      f.R = rd;
      f.RK = rk;
      f.kofs = i == 0 ? 0 : w0 + (i - 1) * P;
      f.W = i == 0 ? w0 : P;
      f.accy = rofs > 0 || i > 0;
    }
  }
  return n;
}

int lr_fwd_npasses(const LrProblem& p) {
  FwdPass ps[kFwdMaxPlan];
  return fwd_plan(p, ps);
}

namespace {

// The kernel of one pass: the plain kernels up to W 8 (this unit) and at
// 9 <= W <= 32 (lowrank_mfma_fwd_wide.hip, which also holds the 16-tap
// accumulating pass above W 16), the accumulating ones up to W 8
// (lowrank_mfma_fwd_acc.hip).
template <typename T>
hipError_t dispatch_pass(const LrProblem* pp, int G) {
  const LrProblem& p = pp[0];
  const int rc = (int)((p.R + (p.static_w ? 1 : 0) + 15) / 16);
  if (p.accy) return p.W <= 8 ? lr_fwd_acc_dispatch<T>(pp, G) : lr_fwd_wide_dispatch<T>(pp, G);
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
  // kernel ranks 65-128 in one pass up to W 4 (fwd_rank_pass)
  DC_LR_CASE(1, 5) DC_LR_CASE(1, 6) DC_LR_CASE(1, 7) DC_LR_CASE(1, 8)
  DC_LR_CASE(2, 5) DC_LR_CASE(2, 6) DC_LR_CASE(2, 7) DC_LR_CASE(2, 8)
  DC_LR_CASE(3, 5) DC_LR_CASE(3, 6) DC_LR_CASE(3, 7) DC_LR_CASE(3, 8)
  DC_LR_CASE(4, 5) DC_LR_CASE(4, 6) DC_LR_CASE(4, 7) DC_LR_CASE(4, 8)
#undef DC_LR_CASE
  if (p.W > 8) return lr_fwd_wide_dispatch<T>(pp, G);
  return hipErrorInvalidValue;
}

// Every pass of fwd_plan in order: pass f of group g is pp[g] restricted to
// kernel ranks f.rofs .. f.rofs+f.RK-1 (z from column rofs of its rows, U from
// row rofs, static_w in the pass that holds rank R) and taps f.kofs ..
// f.kofs+f.W-1 (U and static_w from tap kofs), the residual in the first pass
// only, z_eff written by the first pass (one pass of ranks: the only kind that
// keeps a z_eff).
template <typename T>
hipError_t dispatch_fwd(const LrProblem* pp, int G) {
  FwdPass ps[kFwdMaxPlan];
  const int np = fwd_plan(pp[0], ps);
  if (np < 1) return hipErrorInvalidValue;
  hipError_t e = hipSuccess;
  for (int i = 0; i < np && e == hipSuccess; ++i) {
    const FwdPass& f = ps[i];
    LrProblem a[kMaxGroups];
    for (int g = 0; g < G; ++g) {
      const LrProblem& p = pp[g];
      a[g] = p;
      a[g].R = f.R;
      a[g].W = f.W;
      a[g].z = static_cast<const T*>(p.z) + f.rofs;
      a[g].z_ld = p.zld();
      a[g].U = static_cast<const T*>(p.U) + (int64_t)f.rofs * p.uld() + (int64_t)f.kofs * p.D;
      a[g].u_ld = p.uld();
      a[g].static_w = p.static_w && f.RK > f.R ? static_cast<const T*>(p.static_w) + (int64_t)f.kofs * p.D : nullptr;
      a[g].kofs = f.kofs;
      a[g].accy = f.accy;
      a[g].residual = i == 0 ? p.residual : 0;
      a[g].zeff = i == 0 ? p.zeff : nullptr;  // null above kernel rank 64 (lr_zeff_bytes is 0)
      a[g].zeff_rp = lr_zeff_rows(p);          // the whole problem's rows (its W decides)
    }
    e = dispatch_pass<T>(a, G);
  }
  return e;
}

}  // namespace

hipError_t lr_mfma_fwd(const LrProblem* p, int G) {
  return p[0].dtype == kBF16 ? dispatch_fwd<bf16>(p, G) : dispatch_fwd<fp16>(p, G);
}

}  // namespace dc
