// Launch plans of the lowrank forward (lowrank_mfma_fwd_kernel.h), shared by
// the host units that instantiate it: lowrank_mfma_fwd.hip (W <= 8) and
// lowrank_mfma_fwd_wide.hip (9 <= W <= 16, and the last 16 taps above W 16).
#pragma once

#include "lowrank_mfma_fwd_kernel.h"

namespace dc {
namespace {

// Wavefronts per problem: runs of about 8 tiles, at most 4096 wavefronts
// (4 per SIMD).  B4 T4096 D2048: 2048 wavefronts (31.4 us, 31.9 at 4096);
// B2 T8192 D4096: 4096 (61.8 us, 64.0 at 2048).
inline int fwd_target_waves(const LrProblem& p) {
  const int64_t tiles = p.B * ((p.T + 15) / 16) * ((p.D + 127) / 128);
  const int64_t w = tiles / 8;
  return (int)(w < 1 ? 1 : w > 4096 ? 4096 : w);
}

// One rank chunk without the z_eff writer: at most two wavefronts per SIMD, on
// the ILP build (longer runs where the problem is larger).  B2 T8192 D4096 R16:
// 54.5 us at 4096 wavefronts of the default build, 59.6 us at 3072 of the ILP
// build, 50.7 us at 2048; B4 T16384 D4096 R16: 240.4 -> 200.2 us (5.37 TB/s).
// Kernels with two or more rank chunks or the z_eff writer keep the wider
// launches (B2 T8192 D4096 R31 + static: 61.5 us at 4096, 72 us at 2048).
constexpr int kFwdIlpWaves = 2 * 4 * 256;

inline LrArgs make_args(const LrProblem& p, int target_waves, int wg_waves) {
  LrArgs a;
  a.Tn = (int)p.T;
  a.D = (int)p.D;
  a.R = (int)p.R;
  a.RK = (int)p.R + (p.static_w ? 1 : 0);
  a.has_static = p.static_w != nullptr;
  a.residual = p.residual;
  a.nch = (int)((p.D + 127) / 128);
  a.ncg = 0;
  a.zld = (int)p.zld();
  // 8-byte z loads: four ranks at a time from 8-byte aligned rows
  a.zvec = p.R % 4 == 0 && p.zld() % 4 == 0 && aligned_to(p.z, 8);
  const int64_t ntile = (p.T + 15) / 16;
  int64_t seg = (p.B * ntile * a.nch + target_waves - 1) / target_waves;
  if (seg < 1) seg = 1;
  if (seg > ntile) seg = ntile;
  const int64_t cap = lr_fwd_max_run_tiles(p);  // >= 1 (lr_mfma_ok)
  if (seg > cap) seg = cap;
  a.seg = (int)seg;
  a.nspb = (int)((ntile + seg - 1) / seg);
  a.nseg = (int)(p.B * a.nspb);
  a.nblk = ((a.nseg + wg_waves - 1) / wg_waves) * a.nch;
  a.uld = p.uld();
  a.kofs = p.kofs;
  return a;
}

template <typename T, int W, int RC, bool ACC = false>
hipError_t launch_fwd(const LrProblem* p, int G) {
  constexpr int NWV = fwd_wg_waves(W, RC), NT = 64 * NWV;
  int waves = fwd_target_waves(p[0]);
  if (RC == 1 && W <= 8 && !p[0].zeff && waves > kFwdIlpWaves) waves = kFwdIlpWaves;
  LrArgs a = make_args(p[0], waves, NWV);
  a.nblk1 = a.nblk;
  a.nblk = G * a.nblk1;
  a.xld = (int)p[0].xld();
  a.yhd = (int)p[0].yhd();
  a.zrp = p[0].zeff ? (int)lr_zeff_rows(p[0]) : 0;
  for (int g = 0; g < G; ++g) {
    a.grp[g] = LrFwdGroup{p[g].x, p[g].z, p[g].U, p[g].static_w, p[g].y, p[g].zeff};
    a.zvec = a.zvec && aligned_to(p[g].z, 8);
  }
  if (auditing()) {
    // the run resources of the longest run (from row 0): x, z, z_eff, and y
    // over the head blocks of the widest 128-channel chunk (U is staged through
    // plain pointers)
    const int64_t rows[3] = {(int64_t)a.xld * 2, (int64_t)a.zld * 2, (int64_t)a.zrp * 2};
    for (int64_t rowb : rows) audit_range(run_rsrc_bytes(a.Tn, rowb), kOobTile - 15 * rowb);
    int heads = 0;
    for (int c = 0; c < a.nch; ++c) {
      const int yh0 = c * 128 / a.yhd, yhl = (c * 128 + 127 < a.D - 1 ? c * 128 + 127 : a.D - 1) / a.yhd;
      heads = yhl - yh0 > heads ? yhl - yh0 : heads;
    }
    audit_range(run_rsrc_bytes((int64_t)heads * a.Tn + a.Tn, (int64_t)a.yhd * 2), kOobTile - 15 * (int64_t)a.yhd * 2);
    return hipSuccess;
  }
  if constexpr (ACC) {  // a later pass of taps (no z_eff writer)
    if (a.zvec)
      lr_fwd_mfma<T, W, RC, true, false, false, true><<<a.nblk, NT, 0, p[0].stream>>>(a);
    else
      lr_fwd_mfma<T, W, RC, false, false, false, true><<<a.nblk, NT, 0, p[0].stream>>>(a);
    return hipGetLastError();
  }
  if constexpr (RC == 1 && W <= 8) {
    // all wavefronts resident at the ILP build's three per SIMD (see lowrank_mfma_fwd_ilp.hip);
    // more only where the run length cap forces them
    static_assert(NWV == 4, "the ILP build launches 4-wavefront workgroups");
    if (a.zrp == 0 && a.nblk * 4 <= kFwdIlpMaxWaves) return lr_fwd_ilp_launch<T, W>(a, p[0].stream);
  }
  if constexpr (RC <= 4) {  // z_eff writer: kernel ranks up to 64 (above, lr_zeff_bytes is 0)
    if (a.zrp > 0) {
      if (a.zvec)
        lr_fwd_mfma<T, W, RC, true, true><<<a.nblk, NT, 0, p[0].stream>>>(a);
      else
        lr_fwd_mfma<T, W, RC, false, true><<<a.nblk, NT, 0, p[0].stream>>>(a);
      return hipGetLastError();
    }
  }
  if (a.zrp > 0) return hipErrorInvalidValue;
  if (a.zvec)
    lr_fwd_mfma<T, W, RC, true, false><<<a.nblk, NT, 0, p[0].stream>>>(a);
  else
    lr_fwd_mfma<T, W, RC, false, false><<<a.nblk, NT, 0, p[0].stream>>>(a);
  return hipGetLastError();
}

}  // namespace

// The forward at 9 <= W <= 16 with one or two rank chunks, and (accy) the
// second pass of taps above W 16 (lowrank_mfma_fwd_wide.hip).
template <typename T>
hipError_t lr_fwd_wide_dispatch(const LrProblem* pp, int G);

// The accumulating passes (accy) up to W 8 at every rank chunk count
// (lowrank_mfma_fwd_acc.hip): passes of 8 taps above W 8 at three or four rank
// chunks, and the passes of ranks above kernel rank 64.
template <typename T>
hipError_t lr_fwd_acc_dispatch(const LrProblem* pp, int G);

}  // namespace dc
