// Lowrank forward kernel on gfx950 matrix cores (bf16 / fp16), shared by the
// default build (lowrank_mfma_fwd.hip) and the ILP-scheduled one
// (lowrank_mfma_fwd_ilp.hip).
//
// Forward tile (lr_fwd_mfma).  A wavefront owns 16 rows x 128 channels.
// Lane l = 16*q + n owns rows 4q..4q+3 and the channel octet 8n..8n+7.
// For each tap k the per-token weights come from eight
// v_mfma_f32_16x16x16 (bf16|f16) products, one per j = 0..7, whose 16
// output columns are the channels 8*col + j: the accumulator layout of the
// 16x16 MFMA (lane l holds rows 4q..4q+3 of column n) then leaves every lane
// holding exactly its own 8 channels for its own 4 rows, so the weights
// multiply 128-bit rows of x in registers and are never written anywhere.
// The B operands (U_eff, 16 ranks x 8 columns per lane) are loaded once per
// run as 128-bit row pieces and repacked; the A operand is the lane's row
// of z_eff.  Reference: lowrank.py:24-67 (Triton forward kernel).
//
// x rows: a lane needs rows 4q-W+1 .. 4q+3.  For 2 <= W <= 4 it loads only
// its own 4 rows; the W-1 rows above them are own rows of the lane group
// above (lane - 16), and group 0's are those of group 3 in the tile before,
// so they come over ds_bpermute (12 per tile at W = 4) instead of 3 more
// 128-bit loads per lane whose lines the L1 / L2 had to serve again
// (B4 T4096 D2048 R16: 31.3 -> 29.3 us).
//
// Groups: up to kMaxGroups independent problems of one shape share a launch
// (block index -> group); x may have a row stride xld > D, so the q / k / v
// inputs are read straight out of a fused [B, T, 3D] projection.
#pragma once

#include "lowrank_mfma.h"

namespace dc {

struct LrFwdGroup {
  const void* x;  // this group's first channel; rows xld elements apart
  const void* z;
  const void* U;
  const void* sw;
  void* y;
  void* zeff;     // padded z_eff for the backward (rows of zrp ranks), when zrp > 0
};

struct LrArgs {
  int Tn;          // sequence length
  int D;           // channels
  int R;           // dynamic rank (z.shape[-1])
  int RK;          // kernel rank = R + has_static
  int has_static;
  int residual;
  int nch;         // ceil(D / 128): 128-channel chunks, one per wavefront
  int ncg;         // unused
  int seg;         // 16-row tiles per run
  int nspb;        // runs per sequence
  int nseg;        // B * nspb
  int nblk;        // grid size (all groups)
  int nblk1;       // blocks per group
  int xld;         // row stride of x (elements)
  int zvec;        // R % 4 == 0 and z 8-byte aligned: 8-byte z loads (host dispatch)
  int yhd;         // y layout: D ([B, T, D]) or the head dim of [B, D/yhd, T, yhd] (yhd % 8 == 0)
  int zrp;         // > 0: the 128-channel chunk 0 wavefronts write z_eff rows of zrp ranks
  int64_t uld;     // row stride of U (elements): the problem's W * D, all taps
  int kofs;        // ACC pass: its first tap (x read kofs rows earlier)
  int zld;         // row stride of z (elements): R, or a wider problem's for a pass of ranks
  LrFwdGroup grp[kMaxGroups];
};

// Wavefronts per forward workgroup: 4, or 8 where the staged operands (W x RC
// x 4 KiB) exceed 80 KiB, so that the one workgroup a CU then holds still
// keeps two wavefronts per SIMD (four would leave one).  Each wavefront runs
// its own row run on the workgroup's 128-channel chunk.
constexpr int fwd_wg_waves(int W, int RC) { return W * RC > 20 ? 8 : 4; }

// Packed B operands of one 128-channel chunk, staged once per workgroup:
// ub[(k*RC + c)*8 + j][lane] = U_eff[16c + 4q + kk, k*D + dl + j], kk = 0..3.
template <int W, int RC>
__device__ __forceinline__ void stage_u(u32x2* __restrict__ lds, const uint16_t* __restrict__ U,
                                        const uint16_t* __restrict__ sw, int R, int RK, int D, int64_t WD, int dl,
                                        bool chv, int q, int lane, int wave) {
  for (int kc = wave; kc < W * RC; kc += fwd_wg_waves(W, RC)) {
    const int k = kc / RC, c = kc - k * RC;
    u32x4 rows[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int r = 16 * c + 4 * q + kk;
      const uint16_t* src = nullptr;
      if (chv && r < R) src = U + (int64_t)r * WD + (int64_t)k * D + dl;
      else if (chv && r < RK) src = sw + (int64_t)k * D + dl;
      rows[kk] = src ? *reinterpret_cast<const u32x4*>(src) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      u32x2 v;
      v[0] = elem16(rows[0], j) | (elem16(rows[1], j) << 16);
      v[1] = elem16(rows[2], j) | (elem16(rows[3], j) << 16);
      lds[(kc * 8 + j) * 64 + lane] = v;
    }
  }
}

// ZE: also write the padded z_eff for the backward (a separate instantiation,
// so calls without it run the kernel unchanged).  With it the compiler is held
// to 4 wavefronts per SIMD (<= 128 VGPRs) where the operands allow it: left
// alone it took 138 VGPRs at W 4 with two rank chunks, and the launches of 4096
// wavefronts (B2 T8192 D4096) need all four resident (forward 61.5 -> 68.9 us).
//
// ILP: the same kernel from the translation unit built with the scheduler's
// ILP strategy (lowrank_mfma_fwd_ilp.hip); a template argument of its own, so
// the two builds are distinct kernels.
//
// ACC: a later pass of a wider problem, whose y rows, as the earlier passes
// stored them, are added before the store (each lane loads and stores only its
// own rows): a pass of taps kofs .. kofs+W-1 (above W 16 at two rank chunks
// the host runs taps 0 .. W-17 first, then the last 16), whose x is read kofs
// rows earlier, or a pass of kernel ranks (above 64: z columns and U rows from
// the pass's first rank, kofs 0 unless taps are split as well).
//
// Up to W 4 with one or two rank chunks the kernels are held to 4 wavefronts
// per SIMD (128 VGPRs): the z_eff writer, and the unaligned z loads of two
// rank chunks (ZRaw), would otherwise take 138-140.
template <typename T, int W, int RC, bool ZV, bool ZE, bool ILP = false, bool ACC = false>
__global__ __launch_bounds__(64 * fwd_wg_waves(W, RC))
__attribute__((amdgpu_waves_per_eu((ZE || !ZV) && W <= 4 && RC <= 2 ? 4 : 1, 8)))
void lr_fwd_mfma(LrArgs a) {
  constexpr int NR = W + 3;  // x rows 4q-W+1 .. 4q+3 of a lane
  constexpr int NWV = fwd_wg_waves(W, RC);
  typedef ZRaw<T, RC, ZV> ZR;
  __shared__ u32x2 ub[W * RC * 8 * 64];

  const int lane = threadIdx.x & 63, wave = wave_id();
  const int q = lane >> 4, n = lane & 15;
  const int lb0 = xcd_remap(blockIdx.x, a.nblk);
  const int g = __builtin_amdgcn_readfirstlane(lb0 / a.nblk1);
  const int lb = lb0 - g * a.nblk1;
  const uint16_t* __restrict__ x = reinterpret_cast<const uint16_t*>(pick(a.grp, g, &LrFwdGroup::x));
  const uint16_t* __restrict__ z = reinterpret_cast<const uint16_t*>(pick(a.grp, g, &LrFwdGroup::z));
  const uint16_t* __restrict__ U = reinterpret_cast<const uint16_t*>(pick(a.grp, g, &LrFwdGroup::U));
  const uint16_t* __restrict__ sw = reinterpret_cast<const uint16_t*>(pick(a.grp, g, &LrFwdGroup::sw));
  uint16_t* __restrict__ y = reinterpret_cast<uint16_t*>(pick(a.grp, g, &LrFwdGroup::y));
  const int chunk = lb % a.nch, sgp = lb / a.nch;  // NWV wavefronts: one chunk, NWV consecutive runs
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
  // The run's resources start at row rb (run_base_row): offsets are relative to it.
  const int rb = run_base_row(tile0);
  const int64_t rrow = row0 + rb;
  // y is [B, T, D] (yhd == D) or head-major [B, D/yhd, T, yhd]: the lane's
  // octet lies in head yh, whose rows are yhd elements apart.  The y resource
  // starts at row rb of head yh0, the head of the wavefront's first channel,
  // and spans its heads up to yhl.  Rows past T would land in the next head's
  // block there, so stores check the row.
  const int yhd = a.yhd, yh = dl / yhd;
  const int yh0 = chunk * 128 / yhd, yhl = min(chunk * 128 + 127, D - 1) / yhd;
  const int rowb = yhd * 2, xrowb = a.xld * 2;
  const rsrc_t rx = run_rsrc(x + rrow * a.xld, Tn - rb, xrowb);
  const rsrc_t ry = run_rsrc(y + row0 * D + ((int64_t)yh0 * Tn + rb) * yhd, (int64_t)(yhl - yh0) * Tn + Tn - rb, rowb);
  const int zld = a.zld;  // z rows: R, or the whole problem's ranks for a pass of ranks (z then starts at its first)
  const rsrc_t rz = run_rsrc(z + rrow * zld, Tn - rb, zld * 2);
  const int zrp = ZE ? a.zrp : 0;
  const bool zrow_mine = ZE && n % a.nch == chunk;  // this wavefront writes row n of each tile's z_eff
  const rsrc_t rze = ZE ? run_rsrc((const uint16_t*)pick(a.grp, g, &LrFwdGroup::zeff) + rrow * zrp, Tn - rb, zrp * 2)
                        : make_rsrc(z, 0);
  // y: the lane's row-4q octet (head yh, relative to head yh0's row rb)
  const int lane_off = chv ? (((yh - yh0) * Tn + 4 * q) * yhd + dl - yh * yhd) * 2 : kOobLane;
  const int xlane_off = chv ? (4 * q * a.xld + dl) * 2 : kOobLane;   // the same in x
  // HX (2 <= W <= 4): a lane loads only its own rows 4q..4q+3; the W-1 rows
  // above them are the own rows of the lane group above (lane - 16), or for
  // group 0 those of group 3 in the tile before, passed with ds_bpermute.
  constexpr bool HX = W >= 2 && W <= 4;
  static_assert(!(ACC && ZE), "passes: z_eff from the first pass only");
  const int kofs = ACC ? a.kofs : 0;
  const int above = ((lane + 48) & 63) << 2;  // ds_bpermute byte address of lane - 16
  u32x4 prev[HX ? W - 1 : 1];                 // rows 16-W+1 .. 15 of the tile before (group 3 sends them)

  // Tile inputs (rows out of the sequence read as 0).  The loads are
  // unconditional (a tile past the run reads the out-of-range offset
  // kOobTile, which returns 0 and touches no memory).
  auto load_tile = [&](int tile, u32x4(&xr)[NR], ZR& zr) {
    const bool live = tile < tile1;
    const int toff = live ? (tile * 16 - rb - kofs) * xrowb : kOobTile;
#pragma unroll
    // with the halo from the lane group above (HX) every x row is loaded once: nontemporal
    // (B4 T4096 D2048 R16 forward 30.0 -> 29.2 us; R15 + static 31.8 -> 30.4 us)
    for (int m = HX ? W - 1 : 0; m < NR; ++m) xr[m] = bload128<HX ? kNt : 0>(rx, xlane_off + toff + (m - (W - 1)) * xrowb);
    zr.load(rz, live ? (tile * 16 + n - rb) * zld * 2 : kOobTile, R, q);
  };
  auto compute_tile = [&](int tile, u32x4(&xc)[NR], const ZR& zr) {
    u32x2 zc[RC];
    zr.finish(zc, tile * 16 + n, R, RK, Tn, q);
    if constexpr (ZE) {
      // z_eff for the backward: lane (q, n) holds ranks 16c+4q .. +3 of row n,
      // static rank included (finish), as the backward's padded rows need them.
      // Row n of a tile is written by the chunk n % nch, so every wavefront
      // takes an equal share (one writer per row).
#pragma unroll
      for (int c = 0; c < RC; ++c) {
        const int r0 = 16 * c + 4 * q;
        bstore64<false>(zc[c], rze,
                        zrow_mine && tile * 16 + n < Tn && r0 < zrp ? ((tile * 16 + n - rb) * zrp + r0) * 2 : kOobTile);
      }
      if constexpr (RC == 3) {
        // rows of 64 ranks for the backward's passes of 32 (lr_bwd_zrow): ranks 48-63 are zeros
        const int r0 = 48 + 4 * q;
        bstore64<false>(u32x2{0u, 0u}, rze,
                        zrow_mine && tile * 16 + n < Tn && r0 < zrp ? ((tile * 16 + n - rb) * zrp + r0) * 2 : kOobTile);
      }
    }
    if constexpr (HX) {
      // row 4q-W+1+m is own row 5-W+m (slot m+4) of the group above
#pragma unroll
      for (int m = 0; m < W - 1; ++m) {
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const uint32_t s = q == 3 ? prev[m][h] : xc[m + 4][h];
          xc[m][h] = (uint32_t)__builtin_amdgcn_ds_bpermute(above, (int)s);
        }
        prev[m] = xc[m + 4];
      }
    }
    float acc[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[i][j] = 0.f;
#pragma unroll
    for (int k = 0; k < W; ++k) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        f32x4 wk = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < RC; ++c) wk = Mma16<T>::run(zc[c], ub[((k * RC + c) * 8 + j) * 64 + lane], wk);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          acc[i][j] = fmaf(wk[i], Mma16<T>::to_f(elem16(xc[i - k + W - 1], j)), acc[i][j]);
      }
      // Consume tap k's weights before issuing tap k+1's products: keeps the
      // live accumulators at 8 x 4 instead of W x 8 x 4 (occupancy).
      __builtin_amdgcn_sched_barrier(0);
    }
    if (a.residual) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] += Mma16<T>::to_f(elem16(xc[i + W - 1], j));
    }
    const int toff = (tile * 16 - rb) * rowb;
    if constexpr (ACC) {  // the first pass's y of the lane's rows (rows past T read 0)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const u32x4 o = bload128(ry, tile * 16 + 4 * q + i < Tn ? lane_off + toff + i * rowb : kOobTile);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] += Mma16<T>::to_f(elem16(o, j));
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      u32x4 o;
#pragma unroll
      for (int h = 0; h < 4; ++h) o[h] = pack2<T>(acc[i][2 * h], acc[i][2 * h + 1]);
      bstore128<true>(o, ry, tile * 16 + 4 * q + i < Tn ? lane_off + toff + i * rowb : kOobTile);
    }
  };

  // One tile in flight per wavefront: at 114-125 VGPRs the kernel runs 4
  // wavefronts per SIMD, which hide the loads better than a second tile
  // buffer at 3 wavefronts (B4 T4096 D2048 R16: 32.3 -> 31.4 us).
  if constexpr (HX) {
    // the run's first tile: rows 16*tile0-W+1 .. 16*tile0-1 (before the sequence: 0), as group 3 would send them
    // (a later pass of taps reads x kofs rows earlier, its halo rows as well)
    const int xcol = chv ? dl * 2 : kOobLane;
#pragma unroll
    for (int m = 0; m < W - 1; ++m) prev[m] = bload128(rx, xcol + (tile0 * 16 - kofs + m + 1 - W - rb) * xrowb);
  }
  for (int tile = tile0; tile < tile1; ++tile) {
    u32x4 xr[NR];
    ZR zr;
    load_tile(tile, xr, zr);
    compute_tile(tile, xr, zr);
  }
}


// The ILP-scheduled build of the one-rank-chunk kernels without the z_eff
// writer (lowrank_mfma_fwd_ilp.hip, instantiated for bf16 / fp16 and W 1-8).
// At up to 149 VGPRs (bf16, W 3-8) it holds three wavefronts per SIMD where the
// default build holds four, so it serves launches of at most kFwdIlpMaxWaves
// wavefronts (all resident).
template <typename T, int W>
hipError_t lr_fwd_ilp_launch(const LrArgs& a, hipStream_t stream);
constexpr int kFwdIlpMaxWaves = 3 * 4 * 256;

}  // namespace dc
