// dx of the lowrank backward over all kernel ranks in one launch, for the
// problems whose backward runs as passes of 32 ranks (lr_bwd_rank_split) at
// W <= 4: those passes then form dz and dU only (lr_bwd_mfma's DXM 3), and dx
// is rounded once, where passes that each added their ranks' share rounded it
// after every pass (or went through an fp32 accumulator).
//
// dx[t] = sum_k dy[t+k] * K[t+k, k] (+ dy[t] with the residual), K = z_eff U_eff
// (lowrank.py:143-205; the reference forms K over all R ranks in one product).
// The kernel has the forward's shape (lowrank_mfma_fwd_kernel.h): a workgroup
// of NWV wavefronts on one 128-channel chunk, the chunk's W x RC packed U
// operands staged once in LDS (stage_u), each wavefront one run of 16-row
// tiles, lane (q, n) rows 4q..4q+3 and channels 8n..8n+7 of the chunk; the tap
// weights of the lane's own rows come from the same MFMAs.  dx is formed in
// scatter form: dy[s] * K[s, k] goes to row s - k, which for k > s - 4q is a
// row of the group above; those sums pass up one group over ds_bpermute, and
// group 0's go to group 3 of the tile before, whose open rows wait one tile in
// registers (carry).  The tile after a run closes the run's last rows.
#include "lowrank_mfma_fwd_launch.h"

namespace dc {

namespace {

template <typename T, int W, int RC, bool ZV>
__global__ __launch_bounds__(64 * fwd_wg_waves(W, RC)) void lr_dx_mfma(LrArgs a) {
  static_assert(W >= 1 && W <= 4, "scatter sums reach one group up: W <= 4");
  constexpr int NWV = fwd_wg_waves(W, RC);
  constexpr int kFirstOpen = 5 - W;         // rows kFirstOpen..3 of a group take the group below's sums
  constexpr int NSC = W > 1 ? W - 1 : 1;    // open rows per group
  typedef ZRaw<T, RC, ZV> ZR;
  __shared__ u32x2 ub[W * RC * 8 * 64];

  const int lane = threadIdx.x & 63, wave = wave_id();
  const int q = lane >> 4, n = lane & 15;
  const int lb0 = xcd_remap(blockIdx.x, a.nblk);
  const int g = __builtin_amdgcn_readfirstlane(lb0 / a.nblk1);
  const int lb = lb0 - g * a.nblk1;
  const uint16_t* __restrict__ dy = reinterpret_cast<const uint16_t*>(pick(a.grp, g, &LrFwdGroup::x));
  const uint16_t* __restrict__ z = reinterpret_cast<const uint16_t*>(pick(a.grp, g, &LrFwdGroup::z));
  const uint16_t* __restrict__ U = reinterpret_cast<const uint16_t*>(pick(a.grp, g, &LrFwdGroup::U));
  const uint16_t* __restrict__ sw = reinterpret_cast<const uint16_t*>(pick(a.grp, g, &LrFwdGroup::sw));
  uint16_t* __restrict__ dx = reinterpret_cast<uint16_t*>(pick(a.grp, g, &LrFwdGroup::y));
  const int chunk = lb % a.nch, sgp = lb / a.nch;
  const int D = a.D, Tn = a.Tn, R = a.R, RK = a.RK;
  const int dl = chunk * 128 + 8 * n;  // first channel of the lane's octet
  const bool chv = dl < D;             // D % 8 == 0: octets are whole
  stage_u<W, RC>(ub, U, sw, R, RK, D, a.uld, dl, chv, q, lane, wave);
  __syncthreads();

  const int sg = sgp * NWV + wave;
  if (sg >= a.nseg) return;
  const int b = sg / a.nspb;
  const int ntile = (Tn + 15) >> 4;
  const int tile0 = (sg - b * a.nspb) * a.seg;
  const int tile1 = min(tile0 + a.seg, ntile);
  const int64_t row0 = (int64_t)b * Tn;
  const int rb = run_base_row(tile0);  // the run's resources start at row rb
  const int64_t rrow = row0 + rb;
  const int dyrowb = a.xld * 2, dxrowb = a.yhd * 2;  // dy rows xld apart, dx rows yhd (its dxld) apart
  const rsrc_t rdy = run_rsrc(dy + rrow * a.xld, Tn - rb, dyrowb);
  const rsrc_t rdx = run_rsrc(dx + rrow * a.yhd, Tn - rb, dxrowb);
  const int zld = a.zld;
  const rsrc_t rz = run_rsrc(z + rrow * zld, Tn - rb, zld * 2);
  const int dylane = chv ? (4 * q * a.xld + dl) * 2 : kOobLane;
  const int dxlane = chv ? (4 * q * a.yhd + dl) * 2 : kOobLane;
  const int src = ((lane + 16) & 63) << 2;  // ds_bpermute byte index of the group below
  const float res = a.residual ? 1.f : 0.f;

  float carry[NSC][8];  // group 3's open rows of the tile before (the run's first tile stores none)
#pragma unroll
  for (int m = 0; m < NSC; ++m)
#pragma unroll
    for (int j = 0; j < 8; ++j) carry[m][j] = 0.f;

  for (int tile = tile0; tile <= tile1; ++tile) {
    const bool live = tile < ntile;
    const int toff = live ? (tile * 16 - rb) * dyrowb : kOobTile;
    u32x4 dyr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) dyr[i] = bload128(rdy, dylane + toff + i * dyrowb);
    ZR zr;
    zr.load(rz, live ? (tile * 16 + n - rb) * zld * 2 : kOobTile, R, q);
    u32x2 zc[RC];
    zr.finish(zc, tile * 16 + n, R, RK, Tn, q);

    float own[4][8], S[NSC][8];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) own[i][j] = res * Mma16<T>::to_f(elem16(dyr[i], j));
#pragma unroll
    for (int m = 0; m < NSC; ++m)
#pragma unroll
      for (int j = 0; j < 8; ++j) S[m][j] = 0.f;
#pragma unroll
    for (int k = 0; k < W; ++k) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        f32x4 wk = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < RC; ++c) wk = Mma16<T>::run(zc[c], ub[((k * RC + c) * 8 + j) * 64 + lane], wk);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float v = wk[i] * Mma16<T>::to_f(elem16(dyr[i], j));
          if (i >= k)
            own[i - k][j] += v;               // row 4q+i-k of the lane's group
          else
            S[4 + i - k - kFirstOpen][j] += v;  // row 4+i-k of the group above
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }

    // Close the rows: group q's open rows add group q+1's sums (group 3: group
    // 0's of this tile, for the open rows of the tile before, held in carry).
    float recv[NSC][8];
#pragma unroll
    for (int m = 0; m < NSC; ++m)
#pragma unroll
      for (int j = 0; j < 8; ++j)
        recv[m][j] = W > 1 ? __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(S[m][j]))) : 0.f;
    const bool top = q == 3;
    const bool cur_live = tile < tile1, prev_live = tile > tile0;
    const int cur_off = cur_live ? dxlane + (tile * 16 - rb) * dxrowb : kOobTile;
    const int prev_off = prev_live ? dxlane + ((tile - 1) * 16 - rb) * dxrowb : kOobTile;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool open = W > 1 && i >= kFirstOpen;
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float s = own[i][j];
        if (open) s = (top ? carry[i - kFirstOpen][j] : s) + recv[i - kFirstOpen][j];
        v[j] = s;
      }
      u32x4 o;
#pragma unroll
      for (int h = 0; h < 4; ++h) o[h] = pack2<T>(v[2 * h], v[2 * h + 1]);
      bstore128<true>(o, rdx, (top && open ? prev_off : cur_off) + i * dxrowb);
    }
    if constexpr (W > 1) {
#pragma unroll
      for (int m = 0; m < NSC; ++m)
#pragma unroll
        for (int j = 0; j < 8; ++j) carry[m][j] = own[kFirstOpen + m][j];
    }
  }
}

template <typename T, int W, int RC>
hipError_t launch_dx(const LrProblem* p, int G) {
  constexpr int NWV = fwd_wg_waves(W, RC), NT = 64 * NWV;
  const LrProblem& p0 = p[0];
  LrArgs a{};
  a.Tn = (int)p0.T;
  a.D = (int)p0.D;
  a.R = (int)p0.R;
  a.RK = (int)p0.R + (p0.static_w ? 1 : 0);
  a.has_static = p0.static_w != nullptr;
  a.residual = p0.residual;
  a.nch = (int)((p0.D + 127) / 128);
  a.zld = (int)p0.zld();
  a.xld = (int)p0.D;      // dy: [B, T, D]
  a.yhd = (int)p0.dxld();  // dx rows
  a.uld = p0.uld();
  // runs as the forward's, capped so that the rows of dy, dx and z a run
  // touches (its tiles, the halo, the tile after it) stay inside the resources
  const int64_t ntile = (p0.T + 15) / 16;
  int64_t seg = (p0.B * ntile * a.nch + fwd_target_waves(p0) - 1) / fwd_target_waves(p0);
  int64_t rowb = p0.D > p0.dxld() ? p0.D : p0.dxld();
  rowb = 2 * (rowb > p0.zld() ? rowb : p0.zld());
  const int64_t cap = run_tiles_cap(rowb);
  if (seg > cap) seg = cap;
  if (seg < 1) seg = 1;
  if (seg > ntile) seg = ntile;
  a.seg = (int)seg;
  a.nspb = (int)((ntile + seg - 1) / seg);
  a.nseg = (int)(p0.B * a.nspb);
  a.nblk1 = ((a.nseg + NWV - 1) / NWV) * a.nch;
  a.nblk = G * a.nblk1;
  bool zvec = p0.R % 4 == 0 && p0.zld() % 4 == 0;
  for (int g = 0; g < G; ++g) {
    a.grp[g] = LrFwdGroup{p[g].dy, p[g].z, p[g].U, p[g].static_w, p[g].dx, nullptr};
    zvec = zvec && aligned_to(p[g].z, 8);
  }
  if (auditing()) {
    const int64_t rows[3] = {(int64_t)a.xld * 2, (int64_t)a.yhd * 2, (int64_t)a.zld * 2};
    for (int64_t rb : rows) audit_range(run_rsrc_bytes(a.Tn, rb), kOobTile - 15 * rb);
    return hipSuccess;
  }
  if (zvec)
    lr_dx_mfma<T, W, RC, true><<<a.nblk, NT, 0, p0.stream>>>(a);
  else
    lr_dx_mfma<T, W, RC, false><<<a.nblk, NT, 0, p0.stream>>>(a);
  return hipGetLastError();
}

}  // namespace

// W 1-4 at three to eight rank chunks (kernel ranks 33-128), the shapes
// lr_bwd_dx_split admits.
template <typename T>
hipError_t lr_dx_mfma_launch(const LrProblem* p, int G) {
  const int W = (int)p[0].W, rc = (int)((p[0].R + (p[0].static_w ? 1 : 0) + 15) / 16);
#define DC_DX_CASE(WW, CC) \
  if (W == WW && rc == CC) return launch_dx<T, WW, CC>(p, G);
  DC_DX_CASE(1, 3) DC_DX_CASE(1, 4) DC_DX_CASE(1, 5) DC_DX_CASE(1, 6) DC_DX_CASE(1, 7) DC_DX_CASE(1, 8)
  DC_DX_CASE(2, 3) DC_DX_CASE(2, 4) DC_DX_CASE(2, 5) DC_DX_CASE(2, 6) DC_DX_CASE(2, 7) DC_DX_CASE(2, 8)
  DC_DX_CASE(3, 3) DC_DX_CASE(3, 4) DC_DX_CASE(3, 5) DC_DX_CASE(3, 6) DC_DX_CASE(3, 7) DC_DX_CASE(3, 8)
  DC_DX_CASE(4, 3) DC_DX_CASE(4, 4) DC_DX_CASE(4, 5) DC_DX_CASE(4, 6) DC_DX_CASE(4, 7) DC_DX_CASE(4, 8)
#undef DC_DX_CASE
  return hipErrorInvalidValue;
}

template hipError_t lr_dx_mfma_launch<bf16>(const LrProblem*, int);
template hipError_t lr_dx_mfma_launch<fp16>(const LrProblem*, int);

}  // namespace dc
