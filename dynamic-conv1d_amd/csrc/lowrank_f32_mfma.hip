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
#include "lowrank_mfma.h"

namespace dc {

struct LrF32mArgs {
  int Tn, D, R, RK, residual;
  int nkb;   // rank steps of 4: ceil(RK / 4)
  int nch;   // ceil(D / 64) channel chunks
  int seg;   // 16-row tiles per run
  int nspb;  // runs per sequence
  int nseg;  // B * nspb
  int nblk;  // ceil(nseg / 4) * nch
  int xld;   // row stride of x (elements)
  int yhd;   // y layout: D ([B, T, D]) or the head dim of [B, D/yhd, T, yhd] (yhd % 4 == 0)
};

constexpr int kF32mMaxKb = 8;  // kernel rank <= 32

template <int W, int NKB>
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
    const rsrc_t ru = make_rsrc(U, (int64_t)R * W * D * 4);
    const rsrc_t rs = make_rsrc(sw, sw ? (int64_t)W * D * 4 : 0);
    for (int kk = wave; kk < W * NKB; kk += 4) {
      const int k = kk / NKB, kb = kk - k * NKB;
      const int r = 4 * kb + q;
      const int col = (k * D + dl) * 4;
      const u32x4 vu = bload128(ru, chv && r < R ? r * W * D * 4 + col : kOobLane);
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
  const int xrowb = a.xld * 4;
  const int yhd = a.yhd, yh = dl / yhd;
  const int yrowb = yhd * 4;
  const rsrc_t rx = make_rsrc(x + row0 * a.xld, (int64_t)Tn * xrowb);
  const rsrc_t ry = make_rsrc(y + row0 * D, (int64_t)Tn * D * 4);
  const rsrc_t rz = make_rsrc(z + row0 * R, (int64_t)Tn * R * 4);
  const int xlane_off = chv ? (4 * q * a.xld + dl) * 4 : kOobLane;
  // y: the lane's piece lies in head yh (yhd % 4 == 0), rows yhd elements apart
  const int ylane_off = chv ? ((yh * Tn + 4 * q) * yhd + dl - yh * yhd) * 4 : kOobLane;

  for (int tile = tile0; tile < tile1; ++tile) {
    const int t0 = tile * 16;
    u32x4 xr[NR];
#pragma unroll
    for (int m = 0; m < NR; ++m) xr[m] = bload128(rx, xlane_off + t0 * xrowb + (m - (W - 1)) * xrowb);
    // A operands: z_eff[t0+n, 4kb+q]; the static rank R is 1 inside the sequence
    float za[NKB];
    const int zrow = (t0 + n) * R * 4;
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
      u32x4 o;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) o[jj] = __float_as_uint(acc[i][jj]);
      const int row = t0 + 4 * q + i;
      bstore128<true>(o, ry, row < Tn ? ylane_off + (t0 + i) * yrowb : kOobTile);
    }
  }
}

// ------------------------------------------------------------------- host
namespace {

LrF32mArgs make_f32m_args(const LrProblem& p) {
  LrF32mArgs a;
  a.Tn = (int)p.T;
  a.D = (int)p.D;
  a.R = (int)p.R;
  a.RK = (int)p.R + (p.static_w ? 1 : 0);
  a.residual = p.residual;
  a.nkb = (a.RK + 3) / 4;
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
  a.seg = (int)seg;
  a.nspb = (int)((ntile + seg - 1) / seg);
  a.nseg = (int)(p.B * a.nspb);
  a.nblk = ((a.nseg + 3) / 4) * a.nch;
  a.xld = (int)p.xld();
  a.yhd = (int)p.yhd();
  return a;
}

template <int W, int NKB>
hipError_t launch_f32m(const LrProblem& p) {
  const LrF32mArgs a = make_f32m_args(p);
  lr_fwd_f32m<W, NKB><<<a.nblk, 256, 0, p.stream>>>((const float*)p.x, (const float*)p.z, (const float*)p.U,
                                                      (const float*)p.static_w, (float*)p.y, a);
  return hipGetLastError();
}

}  // namespace

// fp32, W <= 4, kernel rank <= 32, 16-byte pieces of x / y / U / static_w at
// every row (D, x row stride and head dim multiples of 4, pointers 16-byte
// aligned), sequences within the buffer range.
bool lr_f32m_fwd_ok(const LrProblem& p) {
  if (p.dtype != kFP32) return false;
  if (p.W < 1 || p.W > 4) return false;
  const int64_t rk = p.R + (p.static_w ? 1 : 0);
  if (rk > 4 * kF32mMaxKb) return false;
  if (p.D % 4 != 0 || p.xld() % 4 != 0 || p.yhd() % 4 != 0) return false;
  if (!aligned_to(p.x, 16) || !aligned_to(p.y, 16) || !aligned_to(p.U, 16) || !aligned_to(p.static_w, 16))
    return false;
  if (p.R * p.W * p.D * 4 >= kOobLane) return false;                    // U offsets
  if ((p.T + kSeqSlackRows) * p.xld() * 4 > kMaxSeqBytes) return false;  // x rows
  if ((p.T + kSeqSlackRows) * p.D * 4 > kMaxSeqBytes) return false;      // y rows
  return (p.T + kSeqSlackRows) * p.R * 4 <= kMaxSeqBytes;                // z rows
}

hipError_t lr_f32m_fwd(const LrProblem& p) {
  const int nkb = (int)((p.R + (p.static_w ? 1 : 0) + 3) / 4);
  const int kb = nkb <= 2 ? 2 : nkb <= 4 ? 4 : 8;  // rank steps, rounded up (zero steps add nothing)
#define DC_F32M_CASE(WW, KB) \
  if (p.W == WW && kb == KB) return launch_f32m<WW, KB>(p);
  DC_F32M_CASE(1, 2) DC_F32M_CASE(1, 4) DC_F32M_CASE(1, 8)
  DC_F32M_CASE(2, 2) DC_F32M_CASE(2, 4) DC_F32M_CASE(2, 8)
  DC_F32M_CASE(3, 2) DC_F32M_CASE(3, 4) DC_F32M_CASE(3, 8)
  DC_F32M_CASE(4, 2) DC_F32M_CASE(4, 4) DC_F32M_CASE(4, 8)
#undef DC_F32M_CASE
  return hipErrorInvalidValue;
}

}  // namespace dc
