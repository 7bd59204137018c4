// Lowrank forward in fp32 on gfx950 matrix cores (v_mfma_f32_16x16x4_f32).
//
// The reference's fp32 branch computes the tap weights with tl.dot(...,
// "ieee") (lowrank.py:60-61): true fp32 products, which the bf16 MFMA path
// cannot give.  v_mfma_f32_16x16x4_f32 can: fp32 operands, fp32 accumulation.
//
// Tile: a wavefront owns 16 rows x 64 channels.  Lane l = 16q + n owns rows
// 4q..4q+3 and channels 4n..4n+3 (one 16-byte piece per row).  For tap k and
// channel jj of the lane's four, the tap weights of the tile are
//   Kw[16 rows x 16 columns] = sum over rank steps kb of
//     A (16 x 4: z_eff rows t0..t0+15, ranks 4kb..4kb+3) x
//     B (4 x 16: U_eff ranks 4kb..4kb+3, channels 4n'+jj for n' = 0..15)
// with lane (q, n) supplying A[n][q] = z_eff[t0+n, 4kb+q] and B[q][n] =
// U_eff[4kb+q, k*D + 4n+jj]; the result lands as rows 4q..4q+3 of column n,
// i.e. exactly the lane's own rows and channel 4n+jj.  y = sum_k Kw_k x[t-k]
// (+ x) then needs only the lane's x rows 4q-W+1 .. 4q+3.
//
// z_eff / U_eff extend z / U by the static filter as rank R (z == 1) and by
// zero ranks up to a multiple of 4 (lowrank.py:223-225); neither is built.
// The B operands of a 64-channel chunk are staged once per workgroup in LDS;
// the 4 wavefronts of a workgroup take 4 consecutive runs of rows of that
// chunk.  Rows outside the sequence, ranks >= R and lanes past D use buffer
// range checks, as the other fast paths do.  y may be head-major (attention
// layout, [B, D/hd, T, hd]); stores then check the row against T.
//
// Both kernels give each run of tiles buffer resources that start at the run's
// base row (run_base_row: its first tile less a 32-row halo) and the host caps
// a run's length (lr_f32m_{fwd,bwd}_max_run_tiles), so offsets stay in int32
// and sequences of any length take these kernels, as in the 16-bit ones.
#include "lowrank_mfma.h"

namespace dc {

struct LrF32mArgs {
  int Tn, D, R, RK, residual;
  int nch;   // ceil(D / 64) channel chunks
  int seg;   // 16-row tiles per run
  int nspb;  // runs per sequence
  int nseg;  // B * nspb
  int nblk;  // ceil(nseg / 4) * nch
  int xld;   // row stride of x (elements)
  int yhd;   // y layout: D ([B, T, D]) or the head dim of [B, D/yhd, T, yhd] (yhd % 4 == 0)
  int uld;   // row stride of U (elements): the problem's W * D, all taps
  int kofs;  // ACC pass: its first tap (x read kofs rows earlier)
  int zld;   // row stride of z (elements): R, or the whole problem's for a pass of ranks
};

constexpr int kF32mMaxKb = 8;  // kernel rank <= 32
constexpr int kF32mFwdPassTaps = 8;  // above W 8 the forward runs as passes of taps

// ACC: a later pass of taps kofs .. kofs+W-1 of a wider problem (the host runs
// taps 0 .. W0-1 first, then passes of 8): x is read kofs rows earlier, U and
// static_w start at tap kofs, and the tile's y rows, as the earlier passes
// stored them, are added before the store (each lane its own rows).
template <int W, int NKB, bool ACC = false>
__global__ __launch_bounds__(256) void lr_fwd_f32m(const float* __restrict__ x, const float* __restrict__ z,
                                                   const float* __restrict__ U, const float* __restrict__ sw,
                                                   float* __restrict__ y, LrF32mArgs a) {
  constexpr int NR = W + 3;  // x rows 4q-W+1 .. 4q+3 of a lane
  // B operands: ub[(k * NKB + kb) * 64 + lane] = U_eff[4kb+q, k*D + d0 + 4n .. +3]
  __shared__ f32x4 ub[W * NKB * 64];

  const int lane = threadIdx.x & 63, wave = wave_id();
  const int q = lane >> 4, n = lane & 15;
  const int lb = xcd_remap(blockIdx.x, a.nblk);
  const int chunk = lb % a.nch, sgp = lb / a.nch;  // 4 wavefronts: one chunk, 4 consecutive runs
  const int D = a.D, Tn = a.Tn, R = a.R, RK = a.RK;
  const int dl = chunk * 64 + 4 * n;  // first channel of the lane's piece
  const bool chv = dl < D;            // D % 4 == 0: pieces are whole

  // ---- stage the chunk's B operands (every rank row r < RK, zero beyond)
  {
    // U rows uld elements apart; U may start at a later pass's tap kofs.  A pass
    // of ranks may hold no dynamic rank (R == 0: the static rank alone), whose
    // range is empty: R * uld - kofs * D would be negative there, and a negative
    // record count wraps to a range that takes kOobLane in
    const rsrc_t ru = make_rsrc(U, lr_u_bytes(R, a.uld, ACC ? a.kofs : 0, D, 4));
    const rsrc_t rs = make_rsrc(sw, lr_sw_bytes(sw != nullptr, W, D, 4));
    for (int kk = wave; kk < W * NKB; kk += 4) {
      const int k = kk / NKB, kb = kk - k * NKB;
      const int r = 4 * kb + q;
      const int col = (k * D + dl) * 4;
      const u32x4 vu = bload128(ru, chv && r < R ? r * a.uld * 4 + col : kOobLane);
      const u32x4 vs = bload128(rs, chv && r == R && r < RK ? col : kOobLane);
      f32x4 v;
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = __uint_as_float(vu[i]) + __uint_as_float(vs[i]);
      ub[kk * 64 + lane] = v;
    }
  }
  __syncthreads();

  const int sg = sgp * 4 + wave;
  if (sg >= a.nseg) return;
  const int b = sg / a.nspb;
  const int ntile = (Tn + 15) >> 4;
  const int tile0 = (sg - b * a.nspb) * a.seg;
  const int tile1 = min(tile0 + a.seg, ntile);
  const int64_t row0 = (int64_t)b * Tn;
  const int rb = run_base_row(tile0);  // offsets below are relative to the run's base row
  const int64_t rrow = row0 + rb;
  const int xrowb = a.xld * 4;
  const int yhd = a.yhd, yh = dl / yhd;
  const int yrowb = yhd * 4;
  // y is [B, T, D] (yhd == D) or head-major: the resource starts at row rb of
  // head yh0, the head of the chunk's first channel, and spans its heads up to
  // yhl (rows past T would land in the next head's block: stores check the row)
  const int yh0 = chunk * 64 / yhd, yhl = min(chunk * 64 + 63, D - 1) / yhd;
  const rsrc_t rx = run_rsrc(x + rrow * a.xld, Tn - rb, xrowb);
  const rsrc_t ry = run_rsrc(y + row0 * D + ((int64_t)yh0 * Tn + rb) * yhd, (int64_t)(yhl - yh0) * Tn + Tn - rb, yrowb);
  const rsrc_t rz = run_rsrc(z + rrow * a.zld, Tn - rb, a.zld * 4);
  const int xlane_off = chv ? (4 * q * a.xld + dl) * 4 : kOobLane;
  // y: the lane's piece lies in head yh (yhd % 4 == 0), rows yhd elements apart
  const int ylane_off = chv ? (((yh - yh0) * Tn + 4 * q) * yhd + dl - yh * yhd) * 4 : kOobLane;

  for (int tile = tile0; tile < tile1; ++tile) {
    const int t0 = tile * 16;
    u32x4 xr[NR];
#pragma unroll
    for (int m = 0; m < NR; ++m)
      xr[m] = bload128(rx, xlane_off + (t0 - rb - (ACC ? a.kofs : 0)) * xrowb + (m - (W - 1)) * xrowb);
    // A operands: z_eff[t0+n, 4kb+q]; the static rank R is 1 inside the sequence
    float za[NKB];
    const int zrow = (t0 + n - rb) * a.zld * 4;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      const int r = 4 * kb + q;
      za[kb] = __uint_as_float(bload32(rz, r < R ? zrow + r * 4 : kOobTile));
    }
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      const int r = 4 * kb + q;
      if (r == R && R < RK) za[kb] = t0 + n < Tn ? 1.f : 0.f;
    }

    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) acc[i][jj] = 0.f;
#pragma unroll
    for (int k = 0; k < W; ++k) {
      f32x4 kw[4];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) kw[jj] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        const f32x4 bu = ub[(k * NKB + kb) * 64 + lane];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) kw[jj] = __builtin_amdgcn_mfma_f32_16x16x4f32(za[kb], bu[jj], kw[jj], 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
          acc[i][jj] = fmaf(kw[jj][i], __uint_as_float(xr[i - k + W - 1][jj]), acc[i][jj]);
      // Consume tap k's weights before issuing tap k+1's products: 16 live
      // accumulators instead of 16 W (occupancy).
      __builtin_amdgcn_sched_barrier(0);
    }
    if (a.residual) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) acc[i][jj] += __uint_as_float(xr[i + W - 1][jj]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = t0 + 4 * q + i;
      const int yoff = row < Tn ? ylane_off + (t0 - rb + i) * yrowb : kOobTile;
      if constexpr (ACC) {  // the earlier passes' y of the lane's row
        const u32x4 p = bload128(ry, yoff);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) acc[i][jj] += __uint_as_float(p[jj]);
      }
      u32x4 o;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) o[jj] = __float_as_uint(acc[i][jj]);
      bstore128<true>(o, ry, yoff);
    }
  }
}

// ----------------------------------------------------------------- backward
//
// One pass over x and dy gives dx, dz, dU and dstatic_w in fp32 (reference:
// lowrank.py:87-140 and 159-205, fp32 branch 130-132, 196-198).
//
// Tile: 16 rows x 32 channels per wavefront; lane (q, n) owns rows 4q..4q+3
// and channels 2n, 2n+1 (8 bytes per row, 128 contiguous bytes across the 16
// lanes of a row group).  A workgroup is 8 wavefronts on 8 adjacent channel
// chunks (256 channels) of one run of rows.  With G_k[t, d] = dy[t, d] x[t-k, d]:
//   * dx, in scatter form as in the bf16 kernel: tap weights of the lane's own
//     rows (A = z_eff rows, B = U_eff), dy[s] K_w[s, k] added to dx row s-k;
//     the sums for rows of the group above go there by ds_bpermute, and group
//     3's last W-1 rows wait one tile (carry).
//   * dU[r, kD+d] += sum_t z_eff[t, r] G_k[t, d]: K = rows, 4 per MFMA.  In
//     step i lane group q supplies row 4q+i: A = z_eff[t0+4q+i, n] (rank n),
//     B = G_k[4q+i, 2n+jj], the lane's own value.
//   * dz[t, r] += sum_{k,d} G_k[t, d] U_eff[r, kD+d]: K = (tap, channel), 4 per
//     MFMA.  A needs G by row (lane (q,n): row n, channels 8q..8q+7), so each
//     tap's G tile goes through the wavefront's LDS slot (row-major, read back
//     by row); B = U_eff[n, kD + d0+8q .. +7], staged once per run in LDS.
// dz is summed over the 8 chunk wavefronts in LDS, in wave order, every DZB
// tiles (one barrier) and written as one fp32 partial per 256 channels; dU
// accumulates in registers over the run and is written as one partial per
// run.  reduce_partials adds both in a fixed order (deterministic).
//
// Passes: a launch covers the 16 kernel ranks rofs .. rofs+15 (kernel ranks
// 17-32 run as two rank passes) and the W taps kofs .. kofs+W-1 of the
// problem's (W 5-8 run as two tap passes of 2-4 taps each, as the scatter
// form needs).  A rank pass's tap weights, dU rows and dz columns are its
// ranks' (disjoint outputs).  A tap pass is the W-tap problem on x shifted
// down by kofs rows: x rows t-kofs-k, dx rows s-kofs (rows before 0, the
// causal padding, are out of range), U / static_w / dU columns from tap kofs
// (rows uld elements apart), and dz partials in slots of its own.  Every pass
// after the first adds its dx to what the earlier ones stored (ACC, a separate
// instantiation); only the first adds the residual.
struct LrF32mBwdArgs {
  int Tn, D, R, RK, residual;
  int nch;   // ceil(D / 32) chunks
  int ncg;   // ceil(nch / 8): workgroup columns (256 channels)
  int seg;   // 16-row tiles per run
  int nspb;  // runs per sequence
  int nseg;  // B * nspb
  int nblk;  // ncg * nseg
  int xld, dxld;  // row strides of x and dx (elements)
  int yhd;        // dy layout: D ([B, T, D]) or the head dim of [B, D/yhd, T, yhd] (yhd % 32 == 0)
  int rofs;       // first kernel rank of this pass (0, or 16 for the second of two)
  int kofs;       // first tap of this pass
  int uld;        // row stride of U and of the dU partials: the problem's W * D (all taps)
  int64_t BT;
};

template <int W, int NKB, bool ACC>
__global__ __launch_bounds__(512) void lr_bwd_f32m(const float* __restrict__ x, const float* __restrict__ z,
                                                   const float* __restrict__ U, const float* __restrict__ sw,
                                                   const float* __restrict__ dy, float* __restrict__ dx,
                                                   float* __restrict__ part_dz, float* __restrict__ part_du,
                                                   LrF32mBwdArgs a) {
  static_assert(W >= 2 && W <= 4, "scatter form: 2 <= W <= 4");
  static_assert(NKB >= 1 && NKB <= 4, "kernel rank <= 16");
  constexpr int NR = W + 3;   // x rows 4q-W+1 .. 4q+3 per lane
  constexpr int NCW = 8;      // chunk wavefronts per workgroup
  constexpr int NSC = W - 1;  // scatter partial sums per channel
  constexpr int DZB = 2;      // tiles per dz batch
  constexpr int GP = 36;      // G tile row pitch (floats): 32 channels + 4 pad
  __shared__ f32x4 uz_lds[NCW][W * 2 * 64];  // dz B operands of each wavefront
  __shared__ __attribute__((aligned(16))) float gt[NCW][16 * GP];
  __shared__ float dzred[2][NCW][DZB][256];

  const int lane = threadIdx.x & 63, wave = wave_id();
  const int q = lane >> 4, n = lane & 15;
  const int lb = xcd_remap(blockIdx.x, a.nblk);
  const int cg = lb % a.ncg, s = lb / a.ncg;
  const int chunk = cg * NCW + wave;
  const int D = a.D, Tn = a.Tn, R = a.R, RK = a.RK, rofs = ACC ? a.rofs : 0, kofs = ACC ? a.kofs : 0;
  const int uld = a.uld;
  const int d0 = chunk * 32;
  const int col = d0 + 2 * n;
  const bool chv = col < D;  // D % 4 == 0: a lane's 2 channels are both inside or both outside
  const int b = s / a.nspb;
  const int ntile = (Tn + 15) >> 4;
  const int tile0 = (s - b * a.nspb) * a.seg;
  const int tile1 = min(tile0 + a.seg, ntile);
  const int nit = tile1 - tile0;  // the same for every wavefront of the workgroup
  const int64_t row0 = (int64_t)b * Tn;
  const int yhd = a.yhd, head = d0 / yhd;  // yhd % 32 == 0: the chunk lies in one head
  const int xrowb = a.xld * 4, yrowb = yhd * 4, dxrowb = a.dxld * 4;
  // resources of the run's rows from its base row rb (offsets below are relative to it)
  const int rb = run_base_row(tile0);
  const int64_t rrow = row0 + rb;
  const rsrc_t rx = run_rsrc(x + rrow * a.xld, Tn - rb, xrowb);
  const rsrc_t rdy = run_rsrc(dy + row0 * D + ((int64_t)head * Tn + rb) * yhd, Tn - rb, yrowb);
  const rsrc_t rdx = run_rsrc(dx + rrow * a.dxld, Tn - rb, dxrowb);
  const rsrc_t rz = run_rsrc(z + rrow * R, Tn - rb, R * 4);
  const int xlo = chv ? (4 * q * a.xld + col) * 4 : kOobLane;
  const int ylo = chv ? (4 * q * yhd + col - head * yhd) * 4 : kOobLane;
  const int dxlo = chv ? (4 * q * a.dxld + col) * 4 : kOobLane;

  // ---- U_eff operands of the chunk (rank rows r < RK, zero beyond)
  const rsrc_t ru = make_rsrc(U, lr_u_bytes(R, uld, kofs, D, 4));
  const rsrc_t rs = make_rsrc(sw, lr_sw_bytes(sw != nullptr, W, D, 4));
  float uw[W][NKB][2];  // tap-weight B: U_eff[4kb+q, k*D + col + jj]
#pragma unroll
  for (int k = 0; k < W; ++k)
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      const int r = rofs + 4 * kb + q;  // kernel rank
      const int c4 = (k * D + col) * 4;
      const u32x2 vu = bload64(ru, chv && r < R ? r * uld * 4 + c4 : kOobLane);
      const u32x2 vs = bload64(rs, chv && r == R && r < RK ? c4 : kOobLane);
      uw[k][kb][0] = __uint_as_float(vu[0]) + __uint_as_float(vs[0]);
      uw[k][kb][1] = __uint_as_float(vu[1]) + __uint_as_float(vs[1]);
    }
  f32x4* __restrict__ my_uz = uz_lds[wave];
#pragma unroll
  for (int k = 0; k < W; ++k)
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      // dz B: U_eff[n, k*D + d0 + 8q + 4p .. +3]
      const int dd = d0 + 8 * q + 4 * p;
      const int c4 = (k * D + dd) * 4;
      const bool in = dd < D;
      const int rn = rofs + n;  // kernel rank of the lane's dz column
      const u32x4 vu = bload128(ru, in && rn < R ? rn * uld * 4 + c4 : kOobLane);
      const u32x4 vs = bload128(rs, in && rn == R && rn < RK ? c4 : kOobLane);
      f32x4 v;
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = __uint_as_float(vu[i]) + __uint_as_float(vs[i]);
      my_uz[(k * 2 + p) * 64 + lane] = v;  // read back by this lane only
    }
  float* __restrict__ my_g = gt[wave];

  f32x4 du[W][2];
#pragma unroll
  for (int k = 0; k < W; ++k)
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) du[k][jj] = f32x4{0.f, 0.f, 0.f, 0.f};
  float carry[NSC][2];
#pragma unroll
  for (int i = 0; i < NSC; ++i) carry[i][0] = carry[i][1] = 0.f;

  struct TileIn {
    u32x2 xr[NR], dyr[4];
    float za[NKB];  // z_eff[t0+n, 4kb+q]: tap-weight A
    float zt[4];    // z_eff[t0+4q+i, n]: dU A
  };
  auto load_tile = [&](int tile, TileIn& in) {
    const bool live = tile < tile1;
    const bool ylive = tile <= tile1;  // the tile after the run closes its last dx rows
    const int t0 = tile * 16;
    const int xt = live ? (t0 - kofs - rb) * xrowb : kOobTile;  // rows before 0 fall out of range
    const int yt = ylive ? (t0 - rb) * yrowb : kOobTile;
#pragma unroll
    for (int m = 0; m < NR; ++m) in.xr[m] = bload64(rx, xlo + xt + (m - (W - 1)) * xrowb);
#pragma unroll
    for (int m = 0; m < 4; ++m) in.dyr[m] = bload64(rdy, ylo + yt + m * yrowb);
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      const int r = rofs + 4 * kb + q;
      in.za[kb] = __uint_as_float(bload32(rz, ylive && r < R ? ((t0 + n - rb) * R + r) * 4 : kOobTile));
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
      in.zt[i] =
          __uint_as_float(bload32(rz, ylive && rofs + n < R ? ((t0 + 4 * q + i - rb) * R + rofs + n) * 4 : kOobTile));
  };

  // Scatter form (as lowrank_mfma_bwd.hip): S[m] holds the lane's sums for row
  // 4q-1-m; groups take the group below's for rows 4q+3-m; group 3 stores this
  // tile's rows 12 .. 15-NSC and the tile before's last NSC rows (carry).
  auto close_rows = [&](const float(&own)[4][2], const float(&S)[NSC][2], int tile) {
    const int src = ((lane + 16) & 63) << 2;
    float recv[NSC][2];
#pragma unroll
    for (int m = 0; m < NSC; ++m)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj)
        recv[m][jj] = __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(S[m][jj])));
    const bool top = q == 3;
    const int cur_off = tile < tile1 ? dxlo + (tile * 16 - kofs - rb) * dxrowb : kOobTile;
    const int prev_off = tile > tile0 && tile <= tile1 ? dxlo + ((tile - 1) * 16 - kofs - rb) * dxrowb : kOobTile;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      constexpr int kFirstOpen = 4 - NSC;
      const bool open = i >= kFirstOpen;
      u32x2 v;
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        float bv = own[i][jj];
        if (open) bv = (top ? carry[i - kFirstOpen][jj] : bv) + recv[3 - i][jj];
        v[jj] = __float_as_uint(bv);
      }
      const int off = (top && open ? prev_off : cur_off) + i * dxrowb;
      if constexpr (ACC) {  // the earlier rank pass's dx of this row (0 out of range: nothing stored there)
        const u32x2 o = bload64(rdx, off);
        v[0] = __float_as_uint(__uint_as_float(v[0]) + __uint_as_float(o[0]));
        v[1] = __float_as_uint(__uint_as_float(v[1]) + __uint_as_float(o[1]));
      }
      bstore64<true>(v, rdx, off);
    }
#pragma unroll
    for (int i = 0; i < NSC; ++i)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) carry[i][jj] = own[4 - NSC + i][jj];
  };
  // Tap weights of the lane's rows (K = ranks) times dy, into own / S.
  auto scatter_taps = [&](const float(&za)[NKB], const float(&dyf)[4][2], int k, float(&own)[4][2],
                          float(&S)[NSC][2]) {
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      f32x4 kw = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) kw = __builtin_amdgcn_mfma_f32_16x16x4f32(za[kb], uw[k][kb][jj], kw, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = i - k;
        if (r >= 0)
          own[r][jj] = fmaf(dyf[i][jj], kw[i], own[r][jj]);
        else
          S[-r - 1][jj] = fmaf(dyf[i][jj], kw[i], S[-r - 1][jj]);
      }
    }
  };
  // z_eff: the static rank R is 1 inside the sequence (the loads read 0 there)
  auto finish_z = [&](float(&za)[NKB], float(&zt)[4], int t0) {
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
      if (rofs + 4 * kb + q == R && R < RK) za[kb] = t0 + n < Tn ? 1.f : 0.f;
    if (rofs + n == R && R < RK) {
#pragma unroll
      for (int i = 0; i < 4; ++i) zt[i] = t0 + 4 * q + i < Tn ? 1.f : 0.f;
    }
  };

  auto compute_tile = [&](int it, const TileIn& in) {
    const int tile = tile0 + it;
    const int t0 = tile * 16;
    float za[NKB], zt[4];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) za[kb] = in.za[kb];
#pragma unroll
    for (int i = 0; i < 4; ++i) zt[i] = in.zt[i];
    finish_z(za, zt, t0);
    float dyf[4][2], xf[NR][2];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      dyf[m][0] = __uint_as_float(in.dyr[m][0]);
      dyf[m][1] = __uint_as_float(in.dyr[m][1]);
    }
#pragma unroll
    for (int m = 0; m < NR; ++m) {
      xf[m][0] = __uint_as_float(in.xr[m][0]);
      xf[m][1] = __uint_as_float(in.xr[m][1]);
    }
    float own[4][2], S[NSC][2];
#pragma unroll
    for (int i = 0; i < 4; ++i) own[i][0] = own[i][1] = 0.f;
#pragma unroll
    for (int i = 0; i < NSC; ++i) S[i][0] = S[i][1] = 0.f;
    f32x4 dz = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < W; ++k) {
      scatter_taps(za, dyf, k, own, S);
      float g[4][2];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) g[i][jj] = dyf[i][jj] * xf[i - k + W - 1][jj];
      // dU (K = rows): step i takes row 4q+i of every lane group
#pragma unroll
      for (int jj = 0; jj < 2; ++jj)
#pragma unroll
        for (int i = 0; i < 4; ++i) du[k][jj] = __builtin_amdgcn_mfma_f32_16x16x4f32(zt[i], g[i][jj], du[k][jj], 0, 0, 0);
      // dz (K = channels): the G tile by row through this wavefront's LDS slot.
      // The wave barriers keep the compiler from moving a write above a read
      // of another lane's slot (the hardware keeps a wavefront's LDS order).
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f32x2 gw = {g[i][0], g[i][1]};
        *reinterpret_cast<f32x2*>(my_g + (4 * q + i) * GP + 2 * n) = gw;
      }
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const f32x4 ga = *reinterpret_cast<const f32x4*>(my_g + n * GP + 8 * q + 4 * p);
        const f32x4 ub = my_uz[(k * 2 + p) * 64 + lane];
#pragma unroll
        for (int e = 0; e < 4; ++e) dz = __builtin_amdgcn_mfma_f32_16x16x4f32(ga[e], ub[e], dz, 0, 0, 0);
      }
    }
    if (a.residual && !ACC) {  // the first rank pass adds the residual
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) own[i][jj] += dyf[i][jj];
    }
    close_rows(own, S, tile);
    // dz rows 4q..4q+3, rank n: batch over DZB tiles, then the 8 wavefronts' sums in wave order
    const int slot = it % DZB, buf = (it / DZB) & 1;
#pragma unroll
    for (int i = 0; i < 4; ++i) dzred[buf][wave][slot][(4 * q + i) * 16 + n] = dz[i];
    if (slot == DZB - 1 || it == nit - 1) {
      __syncthreads();
      float* __restrict__ out = part_dz + ((int64_t)cg * a.BT + row0) * R;
      const int tb = tile - slot;
      for (int e = threadIdx.x; e < (slot + 1) * 256; e += 64 * NCW) {
        const int sl = e >> 8, rem = e & 255, rr = rem >> 4, nn = rem & 15;
        float v = dzred[buf][0][sl][rem];
#pragma unroll
        for (int w2 = 1; w2 < NCW; ++w2) v += dzred[buf][w2][sl][rem];
        const int t = (tb + sl) * 16 + rr;
        if (rofs + nn < R && nn < 16 && t < Tn) out[(int64_t)t * R + rofs + nn] = v;
      }
    }
  };

  TileIn ta, tb;
  load_tile(tile0, ta);
  for (int it = 0; it < nit; it += 2) {
    load_tile(tile0 + it + 1, tb);
    __builtin_amdgcn_sched_barrier(0);
    compute_tile(it, ta);
    load_tile(tile0 + it + 2, ta);
    __builtin_amdgcn_sched_barrier(0);
    if (it + 1 < nit) compute_tile(it + 1, tb);
  }
  // the tile after the run closes its last rows
  auto flush = [&](const TileIn& in) {
    const int tile = tile0 + nit;
    float za[NKB], zt[4];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) za[kb] = in.za[kb];
#pragma unroll
    for (int i = 0; i < 4; ++i) zt[i] = 0.f;
    finish_z(za, zt, tile * 16);
    float dyf[4][2], own[4][2], S[NSC][2];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      dyf[m][0] = __uint_as_float(in.dyr[m][0]);
      dyf[m][1] = __uint_as_float(in.dyr[m][1]);
      own[m][0] = own[m][1] = 0.f;
    }
#pragma unroll
    for (int i = 0; i < NSC; ++i) S[i][0] = S[i][1] = 0.f;
#pragma unroll
    for (int k = 1; k < W; ++k) scatter_taps(za, dyf, k, own, S);
    close_rows(own, S, tile);
  };
  if (nit & 1)
    flush(tb);
  else
    flush(ta);

  // ---- dU (and dstatic_w as rank R) partial of this run: ranks 4q+r, channels col, col+1
#pragma unroll
  for (int k = 0; k < W; ++k)
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int rk = rofs + 4 * q + r;  // kernel rank (this pass's 16)
        if (rk < RK && chv) part_du[((int64_t)s * RK + rk) * uld + (int64_t)k * D + col + jj] = du[k][jj][r];
      }
}

// ------------------------------------------------------------------- host
namespace {

// Longest forward run (tiles) whose resources fit (run_rsrc): rows of x, y and
// z; head-major y spans the head blocks of a wavefront's 64 channels, which
// adds up to (63 / hd + 1) * T * hd * 4 bytes to its offsets.
int64_t f32m_fwd_max_run_tiles(const LrProblem& p) {
  const int64_t hd = p.yhd();
  int64_t rowb = p.xld() * 4;
  if (hd * 4 > rowb) rowb = hd * 4;
  if (p.zld() * 4 > rowb) rowb = p.zld() * 4;  // z rows (a pass of ranks: the whole problem's)
  int64_t tiles = run_tiles_cap(rowb);
  if (hd != p.D) {
    const int64_t extra = (63 / hd + 1) * p.T * hd * 4;
    const int64_t rows = (kMaxSeqBytes - extra) / (hd * 4) - kSeqSlackRows - kRunHaloRows - 32;
    const int64_t yt = rows > 0 ? rows / 16 : 0;
    tiles = tiles < yt ? tiles : yt;
  }
  return tiles;
}

// Longest backward run: rows of x, dx, dy (one head's block of head-major dy)
// and z.
int64_t f32m_bwd_max_run_tiles(const LrProblem& p) {
  int64_t rowb = p.xld() * 4;
  const int64_t others[3] = {p.dxld() * 4, p.yhd() * 4, p.R * 4};
  for (int64_t v : others) rowb = rowb > v ? rowb : v;
  return run_tiles_cap(rowb);
}

LrF32mArgs make_f32m_args(const LrProblem& p) {
  LrF32mArgs a;
  a.Tn = (int)p.T;
  a.D = (int)p.D;
  a.R = (int)p.R;
  a.RK = (int)p.R + (p.static_w ? 1 : 0);
  a.residual = p.residual;
  a.nch = (int)((p.D + 63) / 64);
  // runs of about 8 tiles, at most 4096 wavefronts
  const int64_t ntile = (p.T + 15) / 16;
  const int64_t tiles = p.B * ntile * a.nch;
  int64_t waves = tiles / 8;
  if (waves < 1) waves = 1;
  if (waves > 4096) waves = 4096;
  int64_t seg = (tiles + waves - 1) / waves;
  if (seg < 1) seg = 1;
  if (seg > ntile) seg = ntile;
  const int64_t cap = f32m_fwd_max_run_tiles(p);  // >= 1 (lr_f32m_fwd_ok)
  if (seg > cap) seg = cap;
  a.seg = (int)seg;
  a.nspb = (int)((ntile + seg - 1) / seg);
  a.nseg = (int)(p.B * a.nspb);
  a.nblk = ((a.nseg + 3) / 4) * a.nch;
  a.xld = (int)p.xld();
  a.yhd = (int)p.yhd();
  a.uld = (int)p.uld();
  a.kofs = p.kofs;
  a.zld = (int)p.zld();
  return a;
}

template <int W, int NKB, bool ACC = false>
hipError_t launch_f32m(const LrProblem& p) {
  const LrF32mArgs a = make_f32m_args(p);
  if (auditing()) {
    // U and static_w of the pass; x, z and y (the head blocks of the widest
    // 64-channel chunk) for the longest run
    audit_range(lr_u_bytes(a.R, a.uld, ACC ? a.kofs : 0, a.D, 4), kOobLane);
    audit_range(lr_sw_bytes(p.static_w != nullptr, W, a.D, 4), kOobLane);
    const int64_t rows[2] = {(int64_t)a.xld * 4, (int64_t)a.zld * 4};
    for (int64_t rowb : rows) audit_range(run_rsrc_bytes(a.Tn, rowb), kOobTile - 15 * rowb);
    int heads = 0;
    for (int c = 0; c < a.nch; ++c) {
      const int yh0 = c * 64 / a.yhd, yhl = (c * 64 + 63 < a.D - 1 ? c * 64 + 63 : a.D - 1) / a.yhd;
      heads = yhl - yh0 > heads ? yhl - yh0 : heads;
    }
    audit_range(run_rsrc_bytes((int64_t)heads * a.Tn + a.Tn, (int64_t)a.yhd * 4), kOobTile - 15 * (int64_t)a.yhd * 4);
    return hipSuccess;
  }
  lr_fwd_f32m<W, NKB, ACC><<<a.nblk, 256, 0, p.stream>>>((const float*)p.x, (const float*)p.z, (const float*)p.U,
                                                           (const float*)p.static_w, (float*)p.y, a);
  return hipGetLastError();
}

hipError_t lr_f32m_fwd_one(const LrProblem& p);

}  // namespace

// fp32, W <= 32 (above 8 as passes of taps), kernel rank <= 64 (above 32 as
// passes of ranks), 16-byte pieces
// of x / y / U / static_w at every row (D, x row stride and head dim multiples
// of 4, pointers 16-byte aligned); sequences of any length (runs capped by
// f32m_fwd_max_run_tiles).
bool lr_f32m_fwd_ok(const LrProblem& p) {
  if (p.dtype != kFP32) return false;
  if (p.W < 1 || p.W > 32) return false;
  const int64_t rk = p.R + (p.static_w ? 1 : 0);
  if (rk > 2 * 4 * kF32mMaxKb) return false;
  if (p.D % 4 != 0 || p.xld() % 4 != 0 || p.yhd() % 4 != 0) return false;
  if (!aligned_to(p.x, 16) || !aligned_to(p.y, 16) || !aligned_to(p.U, 16) || !aligned_to(p.static_w, 16))
    return false;
  if (p.R * p.W * p.D * 4 >= kOobLane) return false;  // U offsets
  return f32m_fwd_max_run_tiles(p) >= 1;              // at least one tile per run fits
}

namespace {

// One launch of at most kF32mFwdPassTaps taps and 32 kernel ranks (accy: a
// later pass of taps or ranks, added to the stored y).
hipError_t lr_f32m_fwd_one(const LrProblem& p) {
  const int nkb = (int)((p.R + (p.static_w ? 1 : 0) + 3) / 4);
  const int kb = nkb <= 2 ? 2 : nkb <= 4 ? 4 : 8;  // rank steps, rounded up (zero steps add nothing)
#define DC_F32M_CASE(WW, KB) \
  if (p.W == WW && kb == KB) return p.accy ? launch_f32m<WW, KB, true>(p) : launch_f32m<WW, KB>(p);
  DC_F32M_CASE(1, 2) DC_F32M_CASE(1, 4) DC_F32M_CASE(1, 8)
  DC_F32M_CASE(2, 2) DC_F32M_CASE(2, 4) DC_F32M_CASE(2, 8)
  DC_F32M_CASE(3, 2) DC_F32M_CASE(3, 4) DC_F32M_CASE(3, 8)
  DC_F32M_CASE(4, 2) DC_F32M_CASE(4, 4) DC_F32M_CASE(4, 8)
  DC_F32M_CASE(5, 2) DC_F32M_CASE(5, 4) DC_F32M_CASE(5, 8)
  DC_F32M_CASE(6, 2) DC_F32M_CASE(6, 4) DC_F32M_CASE(6, 8)
  DC_F32M_CASE(7, 2) DC_F32M_CASE(7, 4) DC_F32M_CASE(7, 8)
  DC_F32M_CASE(8, 2) DC_F32M_CASE(8, 4) DC_F32M_CASE(8, 8)
#undef DC_F32M_CASE
  return hipErrorInvalidValue;
}

}  // namespace

namespace {

// Above W 8: taps 0 .. W0-1 (W0 = W - 8(n-1)) as a W0-tap problem (residual
// included), then passes of 8 taps added to the stored y; U keeps its row
// stride W * D, a later pass's U and static_w start at its tap.  p.accy: the
// first pass adds to y as well (a later pass of ranks).
hipError_t lr_f32m_fwd_taps(const LrProblem& p) {
  constexpr int P = kF32mFwdPassTaps;
  if (p.W <= P) return lr_f32m_fwd_one(p);
  const int W = (int)p.W, np = (W + P - 1) / P, w0 = W - (np - 1) * P;
  LrProblem a = p;
  a.W = w0;
  a.u_ld = p.uld();
  hipError_t e = lr_f32m_fwd_one(a);
  for (int ps = 1; ps < np && e == hipSuccess; ++ps) {
    const int kofs = w0 + (ps - 1) * P;
    a = p;
    a.W = P;
    a.u_ld = p.uld();
    a.kofs = kofs;
    a.accy = 1;
    a.U = (const float*)p.U + (int64_t)kofs * p.D;
    a.static_w = p.static_w ? (const float*)p.static_w + (int64_t)kofs * p.D : nullptr;
    a.residual = 0;
    e = lr_f32m_fwd_one(a);
  }
  return e;
}

}  // namespace

// Above kernel rank 32: passes of 32 kernel ranks (z columns rofs .. of rows
// R apart, U rows rofs .., the static rank in the pass that holds index R),
// each later one added to the stored y; each runs its passes of taps.
hipError_t lr_f32m_fwd(const LrProblem& p) {
  const int64_t RK = p.R + (p.static_w ? 1 : 0);
  if (RK <= 32) return lr_f32m_fwd_taps(p);
  hipError_t e = hipSuccess;
  for (int64_t rofs = 0; rofs < RK && e == hipSuccess; rofs += 32) {
    LrProblem a = p;
    const int64_t rd = p.R - rofs;  // dynamic ranks from rofs on
    a.R = rd < 0 ? 0 : rd > 32 ? 32 : rd;
    a.static_w = p.static_w && rd < 32 ? p.static_w : nullptr;  // kernel rank R falls in this pass
    a.z = (const float*)p.z + rofs;
    a.z_ld = p.R;
    a.U = (const float*)p.U + rofs * p.uld();
    a.u_ld = p.uld();
    if (rofs > 0) {
      a.accy = 1;
      a.residual = 0;
    }
    e = lr_f32m_fwd_taps(a);
  }
  return e;
}

namespace {

LrF32mBwdArgs make_f32m_bwd_args(const LrProblem& p) {
  LrF32mBwdArgs a;
  a.Tn = (int)p.T;
  a.D = (int)p.D;
  a.R = (int)p.R;
  a.RK = (int)p.R + (p.static_w ? 1 : 0);
  a.residual = p.residual;
  a.nch = (int)((p.D + 31) / 32);
  a.ncg = (a.nch + 7) / 8;
  // 2048 wavefronts (2 per SIMD): runs of ceil(tiles * 8 chunks / 2048) tiles
  const int64_t ntile = (p.T + 15) / 16;
  int64_t seg = (p.B * ntile * a.ncg * 8 + 2047) / 2048;
  if (seg < 2) seg = 2;
  if (seg > ntile) seg = ntile;
  const int64_t cap = f32m_bwd_max_run_tiles(p);  // >= 1 (lr_f32m_bwd_ok)
  if (seg > cap) seg = cap;
  a.seg = (int)seg;
  a.nspb = (int)((ntile + seg - 1) / seg);
  a.nseg = (int)(p.B * a.nspb);
  a.nblk = a.nseg * a.ncg;
  a.xld = (int)p.xld();
  a.dxld = (int)p.dxld();
  a.yhd = (int)p.yhd();
  a.rofs = 0;
  a.kofs = 0;
  a.uld = (int)(p.W * p.D);
  a.BT = p.B * p.T;
  return a;
}

struct F32mWs {
  int64_t dz_off, du_off, total;
};
// Tap passes of a W-tap problem: one for W <= 4, else ceil(W / 4) of 2-4 taps
// (the scatter form needs at least 2), the larger ones first: W 5 = 3 + 2,
// 8 = 4 + 4, 9 = 3 + 3 + 3, 17 = 4 + 4 + 3 + 3 + 3, 32 = 8 x 4.
inline int f32m_tap_passes(int W) { return W <= 4 ? 1 : (W + 3) / 4; }
inline int f32m_pass_taps(int W, int tp) {
  const int n = f32m_tap_passes(W), base = W / n;
  return tp < W % n ? base + 1 : base;
}

F32mWs f32m_ws(const LrProblem& p, const LrF32mBwdArgs& a) {
  F32mWs w;
  w.dz_off = 0;
  w.du_off = ((int64_t)f32m_tap_passes((int)p.W) * a.ncg * a.BT * a.R * 4 + 255) / 256 * 256;
  w.total = w.du_off + (int64_t)a.nseg * a.RK * p.W * p.D * 4;
  return w;
}

// One pass: W taps from kofs, NKB rank steps of 4 (ranks rofs .. rofs+4*NKB-1);
// U, static_w, the dz and dU partials already start at the pass's tap / slot.
template <int W, int NKB>
hipError_t launch_f32m_pass(const LrProblem& p, LrF32mBwdArgs a, const float* U, const float* sw, float* pdz,
                            float* pdu) {
  const bool first = a.rofs == 0 && a.kofs == 0;
  if (auditing()) {
    // U and static_w of the pass (kofs is the kernel's for every pass but the
    // first, which starts at tap 0); x, dy, dx and z for the longest run
    audit_range(lr_u_bytes(a.R, a.uld, first ? 0 : a.kofs, a.D, 4), kOobLane);
    audit_range(lr_sw_bytes(sw != nullptr, W, a.D, 4), kOobLane);
    const int64_t rows[4] = {(int64_t)a.xld * 4, (int64_t)a.yhd * 4, (int64_t)a.dxld * 4, (int64_t)a.R * 4};
    for (int64_t rowb : rows) audit_range(run_rsrc_bytes(a.Tn, rowb), kOobTile - 15 * rowb);
    return hipSuccess;
  }
  if (!first)
    lr_bwd_f32m<W, NKB, true><<<a.nblk, 512, 0, p.stream>>>((const float*)p.x, (const float*)p.z, U, sw,
                                                             (const float*)p.dy, (float*)p.dx, pdz, pdu, a);
  else
    lr_bwd_f32m<W, NKB, false><<<a.nblk, 512, 0, p.stream>>>((const float*)p.x, (const float*)p.z, U, sw,
                                                              (const float*)p.dy, (float*)p.dx, pdz, pdu, a);
  return hipGetLastError();
}

template <int W>
hipError_t launch_f32m_taps(const LrProblem& p, const LrF32mBwdArgs& a, const float* U, const float* sw, float* pdz,
                            float* pdu) {
  // kernel ranks 1-16: one pass; above: passes of 16 ranks (0-15, 16-31, ...)
  for (int rofs = 0; rofs < a.RK; rofs += 16) {
    const int nr = a.RK - rofs < 16 ? a.RK - rofs : 16;  // ranks of this pass
    const int nkb = (nr + 3) / 4;
    LrF32mBwdArgs b = a;
    b.rofs = rofs;
    const hipError_t e = nkb <= 2 ? launch_f32m_pass<W, 2>(p, b, U, sw, pdz, pdu)
                                  : launch_f32m_pass<W, 4>(p, b, U, sw, pdz, pdu);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_f32m_bwd(const LrProblem& p) {
  const LrF32mBwdArgs a = make_f32m_bwd_args(p);
  const F32mWs w = f32m_ws(p, a);
  float* pdz = (float*)((char*)p.ws + w.dz_off);
  float* pdu = (float*)((char*)p.ws + w.du_off);
  const int ntp = f32m_tap_passes((int)p.W);
  const int64_t dz_slot = (int64_t)a.ncg * a.BT * a.R;  // one tap pass's dz partials
  hipError_t e;
  for (int tp = 0, kofs = 0; tp < ntp; kofs += f32m_pass_taps((int)p.W, tp), ++tp) {
    const int wq = f32m_pass_taps((int)p.W, tp);
    LrF32mBwdArgs b = a;
    b.kofs = kofs;
    const float* U = (const float*)p.U + (int64_t)kofs * p.D;
    const float* sw = p.static_w ? (const float*)p.static_w + (int64_t)kofs * p.D : nullptr;
    float* dz_t = pdz + tp * dz_slot;
    float* du_t = pdu + (int64_t)kofs * p.D;
    switch (wq) {
      case 2: e = launch_f32m_taps<2>(p, b, U, sw, dz_t, du_t); break;
      case 3: e = launch_f32m_taps<3>(p, b, U, sw, dz_t, du_t); break;
      case 4: e = launch_f32m_taps<4>(p, b, U, sw, dz_t, du_t); break;
      default: e = hipErrorInvalidValue; break;
    }
    if (e != hipSuccess) return e;
  }
  const int64_t WD = p.W * p.D, RKWD = (int64_t)a.RK * WD;
  const PartialReduce jobs[3] = {
      {pdu, RKWD, a.nseg, p.R * WD, p.dU},
      {pdu + p.R * WD, RKWD, a.nseg, p.static_w ? WD : 0, p.dstatic_w},
      {pdz, a.BT * a.R, ntp * a.ncg, a.BT * a.R, p.dz},
  };
  return reduce_partials_multi(jobs, 3, p.dtype, p.stream);
}

}  // namespace

// fp32, 2 <= W <= 32 (above 4 as passes of 2-4 taps), kernel rank <= 64 (above
// 16 as rank passes of 16); D, x / dx row strides multiples of 4
// (8-byte lane pieces, 16-byte operand pieces); dy's head dim a multiple of 32
// (a chunk inside one head); 16-byte aligned x, dy, dx, U, static_w; sequences
// of any length (runs capped by f32m_bwd_max_run_tiles).
bool lr_f32m_bwd_ok(const LrProblem& p) {
  if (p.dtype != kFP32) return false;
  if (p.W < 2 || p.W > 32) return false;
  if (p.R + (p.static_w ? 1 : 0) > 64) return false;
  if (p.D % 4 != 0 || p.xld() % 4 != 0 || p.dxld() % 4 != 0) return false;
  if (p.yhd() != p.D && p.yhd() % 32 != 0) return false;
  if (!aligned_to(p.x, 16) || !aligned_to(p.dy, 16) || !aligned_to(p.dx, 16) || !aligned_to(p.U, 16) ||
      !aligned_to(p.static_w, 16))
    return false;
  if (p.R * p.W * p.D * 4 >= kOobLane) return false;
  return f32m_bwd_max_run_tiles(p) >= 1;
}

int64_t lr_f32m_ws_bytes(const LrProblem& p) { return f32m_ws(p, make_f32m_bwd_args(p)).total; }

hipError_t lr_f32m_bwd(const LrProblem& p) { return launch_f32m_bwd(p); }

}  // namespace dc
