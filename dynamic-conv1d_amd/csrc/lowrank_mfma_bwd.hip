// Lowrank backward on gfx950 matrix cores (bf16 / fp16): dx, dz, dU, dstatic_w.
#include "lowrank_mfma.h"

namespace dc {

// ---------------------------------------------------------------- backward
//
// One pass over x and dy produces dx, dz, dU and dstatic_w (reference:
// lowrank.py:87-140 and 159-205, two kernels that both read dy).
//
// Tile: a wavefront owns 16 rows x CPW channels (CPW = 64, or 32 for two rank
// chunks); lane l = 16q + n owns rows 4q..4q+3 and the NJ = CPW/16 channels
// NJ*n .. NJ*n+NJ-1 (one 8- or 4-byte load per row, 128 or 64 contiguous bytes
// per row across the 16 lanes of a row group).  With
// G_k[t, d] = bf16(dy[t, d] * x[t-k, d]) (the reference also rounds this
// product to bf16 before its dot products, lowrank.py:128):
//   * dU[r, kD+d] += sum_t z_eff[t, r] G_k[t, d]: MFMA with K = the 16 rows.
//     For each j the lane's four G values of column NJ*n+j are exactly the
//     B operand (rows 4q..4q+3 of column n); A is z_eff transposed.
//   * dz[t, r] += sum_d G_k[t, d] U_eff[r, kD+d]: needs K = channels.  Each
//     wavefront writes the packed dU operands (G transposed: channel-major,
//     4 rows per 8 bytes) into its own LDS slot, and two transposing reads
//     (ds_read_b64_tr_b16) return one row, 8 channels per lane: the A operand
//     of a 16x16x32 MFMA.  All values are bf16-exact, so this is exact.
//   * The residual's dy term rides on tap 0: its MFMA accumulator starts at 1.
//   * Tap weights Kw[t, k, :] = z_eff[t, :] U_eff[:, k]: one 16x16x16 MFMA per
//     rank chunk, or with two rank chunks one 16x16x32 over K = 32 ranks (z
//     rows of 32 ranks, 16-byte aligned).  z is read 8 or 16 bytes per lane
//     and row: z itself when its rows allow that, else a padded z_eff copy
//     (static column included) that lr_zpad writes into the workspace first.
//   * dx[t, d] = sum_k dy[t+k, d] Kw[t+k, k, d] (+ dy).  For 2 <= W <= 4 in
//     scatter form: a lane takes the tap weights of its own rows 4q..4q+3
//     (one MFMA row block) and adds dy[s] Kw[s, k] to dx row s-k; the sums
//     for rows of the group above (s-k < 4q) go to that group with one
//     ds_bpermute each, and group 3's rows wait one tile for group 0's sums
//     of the next tile.  Otherwise in gather form: the tap weights of rows
//     4q..4q+3+W-1 come from NB = ceil((W+3)/4) row blocks (A rows shifted by
//     4) and dy rows 4q..4q+W+2 are read from L1.
// A workgroup is NRW row runs x NCW = 256/CPW wavefronts on NCW adjacent
// channel chunks of the same rows.  dz partial sums over the 256 channels are
// added in LDS in wave order, once per batch of tiles, and written as one fp32
// partial per 256-channel group; dU accumulates in registers over the wavefront's run of
// tiles, the NRW runs of a chunk are added in LDS at the end (run order), and
// one fp32 partial per workgroup is written.  reduce_partials sums both
// deterministically.  NRW = 2 (8 wavefronts, 2 per SIMD at 255 VGPRs) halves
// the dU partials that are written and read back; it needs one rank chunk and
// W <= 4 (registers for the tap operands, LDS for the run exchange).  Two rank
// chunks use CPW = 32: the dU accumulators (RC x W x NJ MFMA tiles) then fit
// two wavefronts per SIMD where 64-channel tiles allowed one, and with the
// same wavefront count the runs are twice as long (half the dU partials).
//
// Passes of taps: a launch holds the tap-weight and dz operands and the dU
// accumulators of at most pass_taps(W, RC) taps (host code below), so wider
// problems run as consecutive launches over taps kofs .. kofs+W'-1: the W'-tap
// problem on x shifted down by kofs rows, whose dx rows land kofs rows earlier
// and are added to what the earlier passes stored (ACC), with U, static_w and
// the dU partial columns from tap kofs and dz partials in slots of their own.
//
// Groups: up to kMaxGroups independent problems of one shape share a launch
// (block index -> group); x and dx may have row strides xld, dxld > D, so the
// q / k / v convolutions read x out of a fused [B, T, 3D] projection and write
// dx into its gradient.

struct LrBwdGroup {
  const void* x;   // this group's first channel; rows xld elements apart
  const void* z;
  const void* U;
  const void* sw;
  const void* dy;
  void* dx;        // this group's first channel; rows dxld elements apart
  float* part_dz;
  float* part_du;
  void* dxs;       // the last pass over the fp32 accumulator (DXM 2): dx itself, rows dxsld apart
};

struct LrBwdArgs {
  int Tn, D, R, RK, residual;
  int nch;    // ceil(D / CPW) channel chunks
  int ncg;    // ceil(nch / NCW) chunk groups of 256 channels: one workgroup column
  int seg;    // tiles per run
  int nspb;   // runs per sequence
  int nseg;   // B * nspb
  int npair;  // ceil(nseg / NRW) workgroup rows: one dU partial each
  int nblk;   // ncg * npair * groups
  int nblk1;  // ncg * npair: blocks per group
  int xld;    // row stride of x (elements)
  int dxld;   // row stride of dx (elements; the fp32 accumulator's D past four passes)
  int dxsld;  // row stride of dx for the last pass over the accumulator (DXM 2)
  int nodx;   // dz and dU only (DXM 3): a separate launch (lr_dx_mfma) forms dx over all ranks
  // z rows: zld elements apart, ranks < zr loaded, ranks zr .. zrk-1 of z_eff
  // added as the static rank (ZRaw).  z itself (zld = zr = R, zrk = RK) when
  // R % 4 == 0 and z is 8-byte aligned, else the padded z_eff copy in the
  // workspace (zld = zr = zrk = RP, the static column included).
  int zld, zr, zrk;
  int yhd;    // dy layout: D ([B, T, D]) or the head dim of [B, D/yhd, T, yhd]
  int uld;    // row stride of U and of the dU partials: the problem's W * D (all taps)
  int kofs;   // first tap of this pass (0 without a tap split)
  int accdx;  // add dx to what an earlier pass stored
  // A pass of ranks writes its dz and dU partial entries into the whole
  // problem's layout: dz partial rows dzld (its R) floats apart (part_dz starts
  // at the pass's first rank), dU partials of dupr (its kernel rank) rows each
  // (part_du starts at the pass's first rank row).  Without rank passes dzld = R
  // and dupr = RK.
  int dzld, dupr;
  int64_t BT;
  LrBwdGroup grp[kMaxGroups];
};


// NJ (4 or 2) 16-bit channels of one row held by a lane: one 8- or 4-byte unit.
template <int NJ> struct LaneVec;
template <> struct LaneVec<4> {
  typedef u32x2 type;
  __device__ static __forceinline__ type load(rsrc_t r, int off) { return bload64(r, off); }
  __device__ static __forceinline__ type load_nt(rsrc_t r, int off) { return bload64<kNt>(r, off); }
  __device__ static __forceinline__ void store(type v, rsrc_t r, int off) { bstore64<true>(v, r, off); }
  __device__ static __forceinline__ uint32_t elem(const type& v, int j) { return elem16x2(v, j); }
  template <typename T>
  __device__ static __forceinline__ type pack(const float* f) {
    return type{pack2<T>(f[0], f[1]), pack2<T>(f[2], f[3])};
  }
};
template <> struct LaneVec<2> {
  typedef uint32_t type;
  __device__ static __forceinline__ type load(rsrc_t r, int off) { return bload32(r, off); }
  __device__ static __forceinline__ type load_nt(rsrc_t r, int off) { return bload32<kNt>(r, off); }
  __device__ static __forceinline__ void store(type v, rsrc_t r, int off) {
    __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, kNt);
  }
  __device__ static __forceinline__ uint32_t elem(const type& v, int j) { return j ? (v >> 16) : (v & 0xFFFFu); }
  template <typename T>
  __device__ static __forceinline__ type pack(const float* f) {
    return pack2<T>(f[0], f[1]);
  }
};

// U_eff operands of one wavefront's CPW-channel chunk, staged once per run (the
// chunk never changes across it): the dz operands always in LDS, the tap-weight
// operands in registers when W*RC <= 8 (UWREG) and in LDS otherwise.  For tap k
// and rank chunk c, lane (q, n) reads
//   uw[j] (j < NJ): ranks 16c+4q..16c+4q+3 of channel NJ*n+j, packed (B operand
//                   of the 16x16x16 tap-weight MFMA);
//   uz[s] (s < NS = CPW/32): rank 16c+n, channels 32s+8q..32s+8q+7 as they lie
//                   in U (B operand of the 16x16x32 dz MFMA).
template <int W, int RC, bool UWREG, int NJ, int NS, bool STAGE_UW = true>
__device__ __forceinline__ void stage_uops(u32x2* __restrict__ uw_lds,
                                           u32x2 (&uw_reg)[UWREG && STAGE_UW ? W * RC * NJ : 1],
                                           u32x4* __restrict__ uz_lds, const uint16_t* __restrict__ U,
                                           const uint16_t* __restrict__ sw, int R, int RK, int D, int uld, int kofs,
                                           int d0, int q, int n, int lane) {
  typedef LaneVec<NJ> LV;
  // U rows are uld elements apart (the whole problem's W*D: a pass of taps
  // starts U at its first tap's columns, so R rows end kofs * D elements
  // before R * uld); below kOobLane (host check).  sw starts at the pass's first tap too.
  const int WD = uld;
  // Buffer loads, all issued before the first use: rows r >= R of U and lanes
  // outside D read 0; the static row (r == R < RK) is read from sw and OR-ed in.
  const rsrc_t ru = make_rsrc(U, lr_u_bytes(R, WD, kofs, D, 2));
  const rsrc_t rs = make_rsrc(sw, lr_sw_bytes(RK > R, W, D, 2));
  const int cw = d0 + NJ * n < D ? (d0 + NJ * n) * 2 : kOobLane;  // the lane's tap-weight channels
  typename LV::type rows[W][RC][4];
  u32x4 zr[W][RC][NS];
#pragma unroll
  for (int k = 0; k < W; ++k)
#pragma unroll
    for (int c = 0; c < RC; ++c) {
      const bool has_static = RK > R && R >= 16 * c && R < 16 * c + 16;  // chunk c holds the static row
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int r = 16 * c + 4 * q + kk;
        if constexpr (STAGE_UW)
          rows[k][c][kk] = LV::load(ru, r < R ? cw + (r * WD + k * D) * 2 : kOobLane) |
                           LV::load(rs, has_static && r == R ? cw + k * D * 2 : kOobLane);
      }
      const int r = 16 * c + n;
#pragma unroll
      for (int s2 = 0; s2 < NS; ++s2) {
        const int dd = d0 + 32 * s2 + 8 * q;  // multiple of 8; D % 8 == 0, so dd < D means dd + 8 <= D
        const int cz = dd < D ? dd * 2 : kOobLane;
        zr[k][c][s2] = bload128(ru, r < R ? cz + (r * WD + k * D) * 2 : kOobLane) |
                       bload128(rs, has_static && r == R ? cz + k * D * 2 : kOobLane);
      }
    }
#pragma unroll
  for (int k = 0; k < W; ++k)
#pragma unroll
    for (int c = 0; c < RC; ++c) {
#pragma unroll
      for (int j = 0; j < (STAGE_UW ? NJ : 0); ++j) {
        const typename LV::type(&rw)[4] = rows[k][c];
        u32x2 uw;
        uw[0] = LV::elem(rw[0], j) | (LV::elem(rw[1], j) << 16);
        uw[1] = LV::elem(rw[2], j) | (LV::elem(rw[3], j) << 16);
        if constexpr (UWREG)
          uw_reg[(k * RC + c) * NJ + j] = uw;
        else
          uw_lds[((k * RC + c) * NJ + j) * 64 + lane] = uw;
      }
#pragma unroll
      for (int s2 = 0; s2 < NS; ++s2) uz_lds[((k * RC + c) * NS + s2) * 64 + lane] = zr[k][c][s2];
    }
}

// Tap-weight operands for K = 32 ranks (two rank chunks): lane (q, n) gives
// ranks 8q..8q+7 of channel NJ*n+j, packed (B operand of the 16x16x32 MFMA
// whose A is z_eff row n, ranks 8q..8q+7).  Row R (< RK) is static_w.
template <int W, int NJ>
__device__ __forceinline__ void stage_uw32(u32x4 (&uw)[W * NJ], const uint16_t* __restrict__ U,
                                           const uint16_t* __restrict__ sw, int R, int RK, int D, int uld, int kofs,
                                           int d0, int q, int n) {
  typedef LaneVec<NJ> LV;
  const int WD = uld;  // U row stride (see stage_uops)
  const rsrc_t ru = make_rsrc(U, lr_u_bytes(R, WD, kofs, D, 2));
  const rsrc_t rs = make_rsrc(sw, lr_sw_bytes(RK > R, W, D, 2));
  const int cw = d0 + NJ * n < D ? (d0 + NJ * n) * 2 : kOobLane;
  typename LV::type rows[W][8];
#pragma unroll
  for (int k = 0; k < W; ++k)
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      const int r = 8 * q + kk;
      rows[k][kk] = LV::load(ru, r < R ? cw + (r * WD + k * D) * 2 : kOobLane) |
                    LV::load(rs, RK > R && r == R ? cw + k * D * 2 : kOobLane);
    }
#pragma unroll
  for (int k = 0; k < W; ++k)
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      u32x4 v;
#pragma unroll
      for (int h = 0; h < 4; ++h) v[h] = LV::elem(rows[k][2 * h], j) | (LV::elem(rows[k][2 * h + 1], j) << 16);
      uw[k * NJ + j] = v;
    }
}

// A lane's NJ channels of one dx row as the passes keep them: the output type
// (DxVec<T, NJ, false>), or past four passes (two that split the ranks) an
// fp32 accumulator in the workspace (DxVec<T, NJ, true>), which the last pass
// rounds to dx once (more passes rounded in 16 bits each drift past the
// north-star bar).
template <typename T, int NJ, bool F32> struct DxVec {
  typedef LaneVec<NJ> LV;
  typedef typename LV::type type;
  static constexpr int ES = 2;
  __device__ static __forceinline__ type load(rsrc_t r, int off) { return LV::load(r, off); }
  __device__ static __forceinline__ void store(type v, rsrc_t r, int off) { LV::store(v, r, off); }
  __device__ static __forceinline__ float get(const type& v, int j) { return Mma16<T>::to_f(LV::elem(v, j)); }
  __device__ static __forceinline__ type make(const float* f) { return LV::template pack<T>(f); }
};
template <typename T> struct DxVec<T, 2, true> {
  typedef u32x2 type;
  static constexpr int ES = 4;
  __device__ static __forceinline__ type load(rsrc_t r, int off) { return bload64(r, off); }
  __device__ static __forceinline__ void store(type v, rsrc_t r, int off) { bstore64<true>(v, r, off); }
  __device__ static __forceinline__ float get(const type& v, int j) { return __uint_as_float(v[j]); }
  __device__ static __forceinline__ type make(const float* f) {
    return type{__float_as_uint(f[0]), __float_as_uint(f[1])};
  }
};
template <typename T> struct DxVec<T, 4, true> {
  typedef u32x4 type;
  static constexpr int ES = 4;
  __device__ static __forceinline__ type load(rsrc_t r, int off) { return bload128(r, off); }
  __device__ static __forceinline__ void store(type v, rsrc_t r, int off) { bstore128<true>(v, r, off); }
  __device__ static __forceinline__ float get(const type& v, int j) { return __uint_as_float(v[j]); }
  __device__ static __forceinline__ type make(const float* f) {
    return type{__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]), __float_as_uint(f[3])};
  }
};

// A operands of the tap-weight MFMA for one row block: four ranks per rank
// chunk (16x16x16, K = 16) or, with two rank chunks, eight ranks (16x16x32).
template <int RC, bool K32> struct ZOp { u32x2 c[RC]; };
template <int RC> struct ZOp<RC, true> { u32x4 v; };

// ACC: a later pass of taps (the host splits wide W), which adds its dx to
// what the earlier passes stored; a separate instantiation, so single-pass
// launches carry none of it.  DXM 1: dx rows are the fp32 accumulator (the
// group's dx pointer and dxld then address it), past four passes (or two that
// split the ranks); DXM 2: the last such pass, which adds to the accumulator's
// rows and stores dx itself (dxs, dxsld) rounded once; DXM 3: no dx at all
// (the passes of ranks when lr_dx_mfma forms dx in one launch over all ranks).
template <typename T, int W, int RC, int NRW, int CPW, bool ACC, int DXM = 0>
__global__ __launch_bounds__(64 * (256 / CPW) * NRW)
__attribute__((amdgpu_waves_per_eu((W <= 4 && (RC == 1 || CPW == 32)) || (RC == 1 && CPW == 32) ? 2 : 1, 8))) void
lr_bwd_mfma(LrBwdArgs a) {
  constexpr int NJ = CPW / 16;     // channels per lane
  constexpr int NS = CPW / 32;     // 32-channel K blocks of the dz MFMA
  constexpr int NCW = 256 / CPW;   // channel-chunk wavefronts per run: 256 channels per workgroup
  constexpr int NW = NCW * NRW;    // wavefronts per workgroup
  static_assert(CPW == 64 || CPW == 32, "64- or 32-channel tiles");
  static_assert(NRW == 1 || (RC == 1 && W <= 4 && CPW == 64), "two runs per workgroup: one rank chunk, W <= 4");
  typedef LaneVec<NJ> LV;
  // dx rows: loaded as DV, stored as DVS (DXM 0: the output type; 1: the fp32
  // accumulator; 2: the last pass, which adds to the accumulator's rows and
  // stores dx itself, rounded once)
  constexpr bool NODX = DXM == 3;
  typedef DxVec<T, NJ, DXM == 1 || DXM == 2> DV;
  typedef DxVec<T, NJ, DXM == 1> DVS;
  // dx in scatter form for 2 <= W <= 4 (SC): tap weights of the lane's own rows
  // only, partial sums for the rows of the group above passed across lanes.
  // Otherwise (gather form) NB row blocks of tap weights cover the look-ahead.
  constexpr bool SC = W >= 2 && W <= 4;
  constexpr int NB = SC ? 1 : (W + 6) / 4;  // MFMA row blocks of tap weights
  constexpr int NR = W + 3;                 // x rows 4q-W+1 .. 4q+3 per lane
  constexpr int NDY = SC ? 4 : W + 3;       // dy rows 4q .. 4q+NDY-1 per lane
  constexpr int NSC = SC ? W - 1 : 1;       // scatter partial sums per channel
  constexpr bool UWREG = W * RC <= 8;   // tap-weight operands in registers
  // Two rank chunks: the tap weights take K = 32 ranks in one 16x16x32 MFMA
  // (z rows of exactly 32 ranks: z itself or the padded z_eff copy).
  constexpr bool K32 = RC == 2;
  static_assert(!K32 || UWREG, "two rank chunks keep their tap-weight operands in registers");
  typedef ZOp<RC, K32> ZO;
  constexpr int NUW = W * RC * NJ;  // packed tap-weight operands per lane
  constexpr int NUZ = W * RC * NS;  // dz operands per lane
  // G tile in LDS, transposed: channel c's rows 4p..4p+3 (8 bytes) at byte
  // p*GPL + 8c + 8(c/16).  Written from the dU operands as they are packed;
  // read back with ds_read_b64_tr_b16 as the dz operand.  The pad of 8 bytes
  // per 16 channels keeps both access patterns within two-way bank conflicts.
  constexpr int GPL = 8 * CPW + CPW / 2;  // bytes per 4-row plane
  __shared__ u32x2 uw_lds[NW][UWREG ? 1 : NUW * 64];
  __shared__ u32x4 uz_lds[NW][NUZ * 64];
  __shared__ __attribute__((aligned(16))) uint8_t gtile[NW][4 * GPL];
  // dz partial sums of the workgroup's chunks, gathered for DZB tiles and
  // reduced once per batch (double-buffered: one barrier per batch).  Two
  // rank chunks batch too once registers already hold occupancy at one
  // wavefront per SIMD (W >= 2); at W = 1 the smaller LDS keeps two.  Row r,
  // rank n of a tile sits at (16r + n) ^ ((r / 4) << 4): the XOR puts the
  // four row groups a lane quarter writes at once in different banks.
  constexpr int DZB = !UWREG ? 1 : RC == 1 ? 4 : (RC == 2 && W >= 2) ? (CPW == 32 ? 2 : 4) : 1;
  __shared__ float dzred[2][NRW][NCW][DZB][RC * 256];

  const int lane = threadIdx.x & 63, wave = wave_id();
  const int cw = wave % NCW, rw = wave / NCW;  // chunk and run of this wavefront in the workgroup
  const int q = lane >> 4, n = lane & 15;
  const int lb0 = xcd_remap(blockIdx.x, a.nblk);
  const int g = __builtin_amdgcn_readfirstlane(lb0 / a.nblk1);
  const int lb = lb0 - g * a.nblk1;
  const uint16_t* __restrict__ x = reinterpret_cast<const uint16_t*>(pick(a.grp, g, &LrBwdGroup::x));
  const uint16_t* __restrict__ z = reinterpret_cast<const uint16_t*>(pick(a.grp, g, &LrBwdGroup::z));
  const uint16_t* __restrict__ U = reinterpret_cast<const uint16_t*>(pick(a.grp, g, &LrBwdGroup::U));
  const uint16_t* __restrict__ sw = reinterpret_cast<const uint16_t*>(pick(a.grp, g, &LrBwdGroup::sw));
  const uint16_t* __restrict__ dy = reinterpret_cast<const uint16_t*>(pick(a.grp, g, &LrBwdGroup::dy));
  char* __restrict__ dx = reinterpret_cast<char*>(pick(a.grp, g, &LrBwdGroup::dx));
  float* __restrict__ part_dz = pick(a.grp, g, &LrBwdGroup::part_dz);
  float* __restrict__ part_du = pick(a.grp, g, &LrBwdGroup::part_du);
  const int cg = lb % a.ncg, sp = lb / a.ncg;
  const int chunk = cg * NCW + cw;
  const int D = a.D, Tn = a.Tn;
  const int d0 = chunk * CPW;
  const int col = d0 + NJ * n;
  const bool chv = col < D;  // the lane's NJ channels inside D (D % 8 == 0: all or none)
  const int ntile = (Tn + 15) >> 4;
  // Run s of the grid: tiles [tile0, tile1) of sequence b, whose buffer
  // resources start at row rb (run_base_row).  A workgroup's last run can lie
  // past nseg (odd nseg): it has no tiles.
  struct Run {
    int tile0, tile1, rb;
    int64_t row0;
  };
  auto run_of = [&](int s) {
    Run r{0, 0, 0, 0};
    if (s < a.nseg) {
      const int b = s / a.nspb;
      r.tile0 = (s - b * a.nspb) * a.seg;
      r.tile1 = min(r.tile0 + a.seg, ntile);
      r.rb = run_base_row(r.tile0);
      r.row0 = (int64_t)b * Tn;
    }
    return r;
  };
  Run runs[NRW];
  int nit = 0;  // iterations of every wavefront: the longest run of the workgroup
#pragma unroll
  for (int i = 0; i < NRW; ++i) {
    runs[i] = run_of(sp * NRW + i);
    nit = max(nit, runs[i].tile1 - runs[i].tile0);
  }
  const Run me = rw == 0 ? runs[0] : runs[NRW - 1];
  const int tile0 = me.tile0, tile1 = me.tile1, rb = me.rb;
  const int64_t row0 = me.row0, rrow = row0 + rb;
  const int R = a.R, RK = a.RK;
  typedef ZRaw<T, RC, true> ZR;  // 8-byte z loads: rows of zld % 4 == 0 elements
  u32x2* __restrict__ my_uw = uw_lds[wave];
  u32x4* __restrict__ my_uz = uz_lds[wave];
  // G^T write position of the lane's channel NJ*n (plus 8j for channel NJ*n+j,
  // j < NJ), and the transposed-read position that returns row n, channels
  // 8q..8q+3 (plus 32 for 8q+4..8q+7, plus 8*32+16 per 32-channel block): the
  // instruction hands lane 4a+e of a 16-lane group element e of the 8 bytes
  // addressed by lane a+4i, as its element i.
  uint8_t* const my_g = gtile[wave];
  const int gw_lane = q * GPL + NJ * 8 * n + (n / (16 / NJ)) * 8;
  const int gr_lane = (n & 3) * GPL + (8 * q + (n >> 2)) * 8 + (q >> 1) * 8;
  const float res = a.residual && a.kofs == 0 ? 1.f : 0.f;  // tap 0's weight + 1: the residual term dy
  // A pass of taps kofs .. kofs+W-1 (the host splits W when the tap-weight
  // operands of all taps do not fit): it is the W-tap problem on x shifted
  // down by kofs rows, so x rows are read kofs rows earlier and its dx rows
  // land kofs rows earlier (rows before 0 are the causal padding: dropped),
  // added to what the previous passes stored (accdx).
  const int kofs = ACC ? a.kofs : 0;  // the first pass (or the only one) starts at tap 0: a constant
                                       // keeps the single-pass kernels' offsets as lean as before
  // dy is [B, T, D] (yhd == D) or head-major [B, D/yhd, T, yhd]; the host takes
  // this path only when yhd % CPW == 0, so a wavefront's channels lie in one
  // head and its dy resource covers that head's [T, yhd] block (rows past T
  // stay out of range either way).
  const int yhd = a.yhd, head = d0 / yhd;
  const int rowb = yhd * 2, xrowb = a.xld * 2, dxrowb = a.dxld * DV::ES;
  const int dxsld = DXM == 2 ? a.dxsld : a.dxld, dxsrowb = dxsld * DVS::ES;
  // resources of the run's rows from rb (offsets below are relative to row rb)
  const rsrc_t rx = run_rsrc(x + rrow * a.xld, Tn - rb, xrowb);
  const rsrc_t rdy = run_rsrc(dy + row0 * D + ((int64_t)head * Tn + rb) * yhd, Tn - rb, rowb);
  const rsrc_t rdx = run_rsrc(dx + rrow * a.dxld * DV::ES, Tn - rb, dxrowb);
  char* __restrict__ dxs = DXM == 2 ? reinterpret_cast<char*>(pick(a.grp, g, &LrBwdGroup::dxs)) : dx;
  const rsrc_t rdxs = DXM == 2 ? run_rsrc(dxs + rrow * dxsld * DVS::ES, Tn - rb, dxsrowb) : rdx;
  const int zld = a.zld, zr = a.zr, zrk = a.zrk;
  const rsrc_t rz = run_rsrc(z + rrow * zld, Tn - rb, zld * 2);
  // byte offsets of the lane's row-4q channels in dy, x and dx
  const int lane_off = chv ? (4 * q * yhd + col - head * yhd) * 2 : kOobLane;
  const int xlane_off = chv ? (4 * q * a.xld + col) * 2 : kOobLane;
  const int dxlane_off = chv ? (4 * q * a.dxld + col) * DV::ES : kOobLane;
  const int dxslane_off = chv ? (4 * q * dxsld + col) * DVS::ES : kOobLane;  // the stores

  u32x2 uw_reg[UWREG && !K32 ? NUW : 1];  // staged below, after the first tile's loads are issued
  u32x4 uw32[K32 ? W * NJ : 1];

  // Identity as the B operand: lane (q, n) gives rows 4q..4q+3 of column n.
  u32x2 ident;
  {
    const uint32_t one = Mma16<T>::kOne;
    uint32_t e[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) e[kk] = (4 * q + kk == n) ? one : 0u;
    ident[0] = e[0] | (e[1] << 16);
    ident[1] = e[2] | (e[3] << 16);
  }
  // K32: selection matrices as the B operand (ranks 8q..8q+7 of column n):
  // sel[c] picks rank 16c+n, so z_eff x sel[c] is z_eff's rank chunk c.
  u32x4 sel[K32 ? 2 : 1];
  if constexpr (K32) {
    const uint32_t one = Mma16<T>::kOne;
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const uint32_t lo = (8 * q + 2 * h == 16 * c + n) ? one : 0u;
        const uint32_t hi = (8 * q + 2 * h + 1 == 16 * c + n) ? one : 0u;
        sel[c][h] = lo | (hi << 16);
      }
  }

  f32x4 du[W][RC][NJ];
#pragma unroll
  for (int k = 0; k < W; ++k)
#pragma unroll
    for (int c = 0; c < RC; ++c)
#pragma unroll
      for (int j = 0; j < NJ; ++j) du[k][c][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Tile inputs (buffer loads: out-of-range rows / channels read as 0).  Two
  // buffers, A and B, alternate: while one tile is computed the next one's
  // loads are in flight.  The loads are unconditional (a tile past the run
  // reads the out-of-range offset kOobTile: 0, no memory traffic) and no
  // register is copied, so the compiler's waits stay partial (vmcnt(N)).
  struct TileIn {
    typename LV::type xr[NR], dyr[NDY];
    ZR zr[K32 ? 1 : NB];   // z_eff rows t0+4bb+n, ranks 16c+4q..+3: A operand of the tap-weight MFMA
    u32x4 z32[K32 ? NB : 1];  // K32: z_eff rows t0+4bb+n, ranks 8q..8q+7
    // ACC: the earlier passes' dx of the tile's rows 4q..4q+3 (shifted by kofs),
    // loaded with the tile's inputs so that the adds before the stores do not wait
    typename DV::type dxo[ACC ? 4 : 1];
  };
  auto load_tile = [&](int tile, TileIn& in) {
    const bool live = tile < tile1;
    // The scatter form also reads dy and z of the tile after the run: its
    // first rows close the run's last dx rows.
    const bool ylive = SC ? tile <= tile1 : live;
    const int xtoff = live ? (tile * 16 - rb - kofs) * xrowb : kOobTile;
    const int toff = ylive ? (tile * 16 - rb) * rowb : kOobTile;
#pragma unroll
    for (int m = 0; m < NR; ++m) in.xr[m] = LV::load(rx, xlane_off + xtoff + (m - (W - 1)) * xrowb);
    // In scatter form each dy row is read once: nontemporal (B4 T4096 D2048 R16 backward
    // 60.0 -> 58.8 us).  x rows, and the gather form's dy rows, are read again by the lane
    // group below and keep the default policy.
#pragma unroll
    for (int m = 0; m < NDY; ++m)
      in.dyr[m] = SC ? LV::load_nt(rdy, lane_off + toff + m * rowb) : LV::load(rdy, lane_off + toff + m * rowb);
#pragma unroll
    for (int bb = 0; bb < NB; ++bb) {
      if constexpr (K32)
        in.z32[bb] = bload128(rz, ylive ? ((tile * 16 + 4 * bb + n - rb) * zld + 8 * q) * 2 : kOobTile);
      else
        in.zr[bb].load(rz, ylive ? (tile * 16 + 4 * bb + n - rb) * zld * 2 : kOobTile, zr, q);
    }
    if constexpr (ACC) {
      const int dxo_off = live ? dxlane_off + (tile * 16 - rb - kofs) * dxrowb : kOobTile;
#pragma unroll
      for (int i = 0; i < 4; ++i) in.dxo[i] = DV::load(rdx, dxo_off + i * dxrowb);
    }
  };

  // Scatter form: S[m] holds the lane's contributions to row 4q-1-m (the group
  // above).  Each group passes S to the group above (lane - 16) and takes the
  // group below's for its rows 4q+3-m; group 3 takes group 0's, which belong
  // to rows 15-m of the tile before.  Groups 0-2 then store this tile's rows
  // 4q..4q+3.  Group 3 stores this tile's rows 12 .. 15-NSC (complete) and the
  // tile before's rows 16-NSC .. 15, held in `carry`, and carries this tile's.
  // Rows outside [tile0, tile1) are not stored.
  constexpr int NOPEN = NSC;  // rows of group 3 that wait for the next tile
  float carry[NOPEN][NJ];
#pragma unroll
  for (int i = 0; i < NOPEN; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) carry[i][j] = 0.f;
  // ACC: group 3's open rows are stored one tile late; their earlier-pass dx
  // (loaded with the tile before) waits here
  typename DV::type dxo_carry[ACC ? NOPEN : 1] = {};  // the first tile's open rows store nothing
  auto close_rows = [&](const float(&own)[4][NJ], const float(&S)[NSC][NJ], int tile,
                        const typename DV::type(&dxo)[ACC ? 4 : 1]) {
    const int src = ((lane + 16) & 63) << 2;  // ds_bpermute byte index of the group below
    float recv[NSC][NJ];
#pragma unroll
    for (int m = 0; m < NSC; ++m)
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        recv[m][j] = __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(S[m][j])));
    const bool top = q == 3;
    const bool cur_live = tile < tile1;
    const bool prev_live = tile > tile0 && tile <= tile1;
    const int cur_off = cur_live ? dxslane_off + (tile * 16 - rb - kofs) * dxsrowb : kOobTile;
    const int prev_off = prev_live ? dxslane_off + ((tile - 1) * 16 - rb - kofs) * dxsrowb : kOobTile;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      constexpr int kFirstOpen = 4 - NOPEN;
      const bool open = i >= kFirstOpen;  // rows that take the group below's sums
      float v[NJ];
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        float b = own[i][j];
        if (open) b = (top ? carry[i - kFirstOpen][j] : b) + recv[3 - i][j];
        v[j] = b;
      }
      const int off = (top && open ? prev_off : cur_off) + i * dxsrowb;
      if constexpr (ACC) {  // a later pass of taps adds to the stored rows
        typename DV::type o = dxo[ACC ? i : 0];
        if (open) o = top ? dxo_carry[ACC ? i - kFirstOpen : 0] : o;
#pragma unroll
        for (int j = 0; j < NJ; ++j) v[j] += DV::get(o, j);
      }
      DVS::store(DVS::make(v), rdxs, off);
    }
#pragma unroll
    for (int i = 0; i < NOPEN; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) carry[i][j] = own[4 - NOPEN + i][j];
    if constexpr (ACC) {
#pragma unroll
      for (int i = 0; i < NOPEN; ++i) dxo_carry[i] = dxo[4 - NOPEN + i];
    }
  };
  // Tap weights of the lane's rows 4q..4q+3 (row block 0) times dy: into
  // `own` for rows of the lane, into S for rows of the group above.
  // Tap k's weights of the operand's rows for channel NJ*n+j, accumulator started at w0.
  auto tap_w = [&](const ZO& za, int k, int j, float w0) {
    f32x4 wk = {w0, w0, w0, w0};
    if constexpr (K32) {
      wk = Mma32<T>::run(za.v, uw32[k * NJ + j], wk);
    } else {
#pragma unroll
      for (int c = 0; c < RC; ++c)
        wk = Mma16<T>::run(za.c[c], UWREG ? uw_reg[UWREG ? (k * RC + c) * NJ + j : 0]
                                          : my_uw[((k * RC + c) * NJ + j) * 64 + lane], wk);
    }
    return wk;
  };
  auto scatter_taps = [&](const ZO& zA0, const float(&dyf)[NDY][NJ], int k, int j, float(&own)[4][NJ],
                          float(&S)[NSC][NJ]) {
    const f32x4 wk = tap_w(zA0, k, j, k == 0 ? res : 0.f);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = i - k;  // dx row of this contribution, relative to 4q
      if (r >= 0)
        own[r][j] = fmaf(dyf[i][j], wk[i], own[r][j]);
      else
        S[-r - 1][j] = fmaf(dyf[i][j], wk[i], S[-r - 1][j]);
    }
  };
  auto compute_tile = [&](int it, const TileIn& in) {
    const int tile = tile0 + it;
    const bool live = tile < tile1;
    const int t0 = tile * 16;
    const int dxtoff = live ? (t0 - rb - kofs) * dxsrowb : kOobTile;  // tiles past the run store nothing
    const typename LV::type(&xr)[NR] = in.xr;
    const typename LV::type(&dyr)[NDY] = in.dyr;
    ZO zA[NB];
#pragma unroll
    for (int bb = 0; bb < NB; ++bb) {
      if constexpr (K32)
        zA[bb].v = in.z32[bb];
      else
        in.zr[bb].finish(zA[bb].c, t0 + 4 * bb + n, zr, zrk, Tn, q);
    }
    // z_eff transposed (rank n, rows 4q..4q+3), the A operand of the dU MFMA,
    // from row block 0 through an exact identity (K32: selection) product.
    u32x2 zT[RC];
#pragma unroll
    for (int c = 0; c < RC; ++c) {
      f32x4 tz;
      if constexpr (K32)
        tz = Mma32<T>::run(zA[0].v, sel[c], f32x4{0.f, 0.f, 0.f, 0.f});
      else
        tz = Mma16<T>::run(zA[0].c[c], ident, f32x4{0.f, 0.f, 0.f, 0.f});
      zT[c][0] = pack2<T>(tz[0], tz[1]);
      zT[c][1] = pack2<T>(tz[2], tz[3]);
    }

    float dyf[NDY][NJ];
#pragma unroll
    for (int m = 0; m < NDY; ++m)
#pragma unroll
      for (int j = 0; j < NJ; ++j) dyf[m][j] = Mma16<T>::to_f(LV::elem(dyr[m], j));

    float dxa[4][NJ], S[NSC][NJ];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) dxa[i][j] = 0.f;
#pragma unroll
    for (int m = 0; m < NSC; ++m)
#pragma unroll
      for (int j = 0; j < NJ; ++j) S[m][j] = 0.f;
    f32x4 dz[RC];
#pragma unroll
    for (int c = 0; c < RC; ++c) dz[c] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int k = 0; k < W; ++k) {
      // G_k = bf16(dy * x_shift) for rows 4q..4q+3, the lane's NJ channels (fp32 products).
      // The G tile passes between lanes through the wavefront's LDS slot: the
      // wave barriers keep the compiler from moving a write above a read of
      // another lane's bytes (the hardware keeps a wavefront's LDS order).
      __builtin_amdgcn_wave_barrier();
      float gf[4][NJ];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) gf[i][j] = dyf[i][j] * Mma16<T>::to_f(LV::elem(xr[i - k + W - 1], j));
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        if constexpr (SC && !NODX) scatter_taps(zA[0], dyf, k, j, dxa, S);
        // Gather form: dx += dy[4q+i+k] * Kw[4q+i+k, k] from the row blocks that hold rows k..k+3.
#pragma unroll
        for (int bb = 0; bb < (SC || NODX ? 0 : NB); ++bb) {
          if (4 * bb > 3 + k || 4 * bb + 3 < k) continue;
          const f32x4 wk = tap_w(zA[bb], k, j, k == 0 ? res : 0.f);  // k = 0 uses block 0 only
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int tr = i + k;  // row offset of dy / Kw in the lane window
            if (tr >= 4 * bb && tr < 4 * bb + 4) dxa[i][j] = fmaf(dyf[tr][j], wk[tr - 4 * bb], dxa[i][j]);
          }
        }
        // dU (K = rows): column j of G, rows 4q..4q+3, is the B operand as it
        // lies; the same 8 bytes go to the transposed G tile.
        u32x2 g;
        g[0] = pack2<T>(gf[0][j], gf[1][j]);
        g[1] = pack2<T>(gf[2][j], gf[3][j]);
        *reinterpret_cast<u32x2*>(my_g + gw_lane + 8 * j) = g;
#pragma unroll
        for (int c = 0; c < RC; ++c) du[k][c][j] = Mma16<T>::run(zT[c], g, du[k][c][j]);
      }
      // dz (K = 32 channels): A = G row n (this lane: row = lane % 16), channels 32s+8q..+7.
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int s2 = 0; s2 < NS; ++s2) {
        const u32x2 lo = lds_read_tr16(my_g + gr_lane + s2 * (8 * 32 + 16));
        const u32x2 hi = lds_read_tr16(my_g + gr_lane + s2 * (8 * 32 + 16) + 32);
        const u32x4 ga = {lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
        for (int c = 0; c < RC; ++c) dz[c] = Mma32<T>::run(ga, my_uz[((k * RC + c) * NS + s2) * 64 + lane], dz[c]);
      }
    }

    // ---- dx rows (the residual dy rides on tap 0's weight); out-of-range stores are dropped
    if constexpr (NODX) {
    } else if constexpr (SC) {
      close_rows(dxa, S, tile, in.dxo);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int off = dxslane_off + dxtoff + i * dxsrowb;
        if constexpr (ACC) {  // a later pass of taps adds to the stored rows (loaded with the tile)
#pragma unroll
          for (int j = 0; j < NJ; ++j) dxa[i][j] += DV::get(in.dxo[ACC ? i : 0], j);
        }
        DVS::store(DVS::make(dxa[i]), rdxs, off);
      }
    }
    // ---- dz: gather this wavefront's tile sums; every DZB iterations (and at the
    // last one) add each run's NCW chunk wavefronts in wave order, one partial per group.
    const int slot = it % DZB;
    const int buf = (it / DZB) & 1;
#pragma unroll
    for (int c = 0; c < RC; ++c)
#pragma unroll
      for (int i = 0; i < 4; ++i) dzred[buf][rw][cw][slot][c * 256 + (((4 * q + i) * 16 + n) ^ (q << 4))] = dz[c][i];
    if (slot == DZB - 1 || it == nit - 1) {
      __syncthreads();
      // The batch's sums go out at raised wave priority: every wavefront of the
      // workgroup waits at the next batch's barrier for the slowest one here
      // (configs[4] backward 156 -> 149 us, grouped 397 -> 383 us, W 8 285 ->
      // 276 us; one rank chunk unchanged).
      __builtin_amdgcn_s_setprio(1);
      constexpr int PER_RUN = RC * 256;
      constexpr int NTH = 64 * NW;
      static_assert(DZB * PER_RUN % NTH == 0, "whole passes over a full batch");
#pragma unroll
      for (int ri = 0; ri < NRW; ++ri) {
        const Run& ru = ri == 0 ? runs[0] : runs[NRW - 1];
        // rows of run ri from its base row; t >= T falls outside the resource
        const rsrc_t rout = run_rsrc(part_dz + ((int64_t)cg * a.BT + ru.row0 + ru.rb) * a.dzld, Tn - ru.rb, a.dzld * 4);
        const int tb = ru.tile0 + it - slot;  // run ri's tile of slot 0
#pragma unroll
        for (int m = 0; m < DZB * PER_RUN / NTH; ++m) {
          const int e2 = (int)threadIdx.x + m * NTH;
          const int sl = e2 / PER_RUN, rem = e2 - sl * PER_RUN;
          const int c = rem >> 8, rr = (rem >> 4) & 15, nn = rem & 15;
          const int r = 16 * c + nn;
          const int ti = tb + sl;  // the slot's tile of run ri
          const int t = ti * 16 + rr;
          const int pos = rem ^ (((rem >> 6) & 3) << 4);  // as written: row group (rr / 4) XOR-ed into bits 4-5
          float v = dzred[buf][ri][0][sl][pos];
#pragma unroll
          for (int w2 = 1; w2 < NCW; ++w2) v += dzred[buf][ri][w2][sl][pos];
          // slots past this batch (a short last batch), tiles past the run and ranks >= R store nothing
          const bool ok = sl <= slot && ti < ru.tile1 && r < R;
          __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), rout, ok ? ((t - ru.rb) * a.dzld + r) * 4 : kOobLane,
                                                0, 0);
        }
      }
      __builtin_amdgcn_s_setprio(0);
    }
  };

  // Every wavefront of the workgroup runs nit iterations (the barriers of the
  // dz batches are shared); tiles past its own run load and store nothing.
  TileIn ta, tb;
  load_tile(tile0, ta);
  __builtin_amdgcn_sched_barrier(0);  // the first tile's loads go out before the U staging waits
  stage_uops<W, RC, UWREG, NJ, NS, !K32>(my_uw, uw_reg, my_uz, U, sw, R, RK, D, a.uld, a.kofs, d0, q, n, lane);
  if constexpr (K32) stage_uw32<W, NJ>(uw32, U, sw, R, RK, D, a.uld, a.kofs, d0, q, n);
  for (int it = 0; it < nit; it += 2) {
    load_tile(tile0 + it + 1, tb);
    __builtin_amdgcn_sched_barrier(0);  // issue the next tile's loads before this tile's waits
    compute_tile(it, ta);
    load_tile(tile0 + it + 2, ta);
    __builtin_amdgcn_sched_barrier(0);
    if (it + 1 < nit) compute_tile(it + 1, tb);
  }
  if constexpr (SC && !NODX) {
    // The tile after the longest run (loaded into the buffer that is next in
    // turn) closes that run's last rows; in shorter runs it lies past tile1
    // and stores nothing.
    auto flush = [&](const TileIn& in) {
      const int tile = tile0 + nit;
      ZO zA0;
      if constexpr (K32)
        zA0.v = in.z32[0];
      else
        in.zr[0].finish(zA0.c, tile * 16 + n, zr, zrk, Tn, q);
      float dyf[NDY][NJ], own[4][NJ], S[NSC][NJ];
#pragma unroll
      for (int m = 0; m < NDY; ++m)
#pragma unroll
        for (int j = 0; j < NJ; ++j) dyf[m][j] = Mma16<T>::to_f(LV::elem(in.dyr[m], j));
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) own[i][j] = 0.f;
#pragma unroll
      for (int m = 0; m < NSC; ++m)
#pragma unroll
        for (int j = 0; j < NJ; ++j) S[m][j] = 0.f;
#pragma unroll
      for (int k = 1; k < W; ++k)
#pragma unroll
        for (int j = 0; j < NJ; ++j) scatter_taps(zA0, dyf, k, j, own, S);
      close_rows(own, S, tile, in.dxo);
    };
    if (nit & 1)
      flush(tb);
    else
      flush(ta);
  }

  if constexpr (NRW == 2) {
    // The second run's wavefronts hand their dU sums to the first run's
    // wavefronts of the same chunk through LDS (the dz buffers, now free).
    float* xch = &dzred[0][0][0][0][0];
    constexpr int NDU = W * RC * NJ * 4;  // dU floats per lane
    static_assert(4 * NDU * 64 <= 2 * NRW * 4 * DZB * RC * 256, "dU exchange fits the dz buffers");
    __syncthreads();
    if (rw == 1) {
#pragma unroll
      for (int k = 0; k < W; ++k)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int i = 0; i < 4; ++i) xch[((cw * W + k) * 16 + j * 4 + i) * 64 + lane] = du[k][0][j][i];
    }
    __syncthreads();
    if (rw == 1) return;
#pragma unroll
    for (int k = 0; k < W; ++k)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) du[k][0][j][i] += xch[((cw * W + k) * 16 + j * 4 + i) * 64 + lane];
  }

  // ---- dU partial of this workgroup row: rows r < RK of U_eff, the wavefront's
  // CPW columns per tap.  The resource spans this row's RK x W*D partial, so
  // rows r >= RK fall outside it (the host keeps (RK + 16) * W * D * 4 bytes
  // below kOobLane, so no offset wraps).
  // The partial's rows are uld (all taps' W*D) floats apart; a pass of taps
  // writes its own taps' columns (part_du starts at its first tap's).
  const int UL = a.uld;
  const rsrc_t rdu = make_rsrc(part_du + (int64_t)sp * a.dupr * UL, lr_dupart_bytes(RK, UL, a.kofs, D));
  const int du_lane = chv ? (4 * q * UL + col) * 4 : kOobLane;
#pragma unroll
  for (int k = 0; k < W; ++k)
#pragma unroll
    for (int c = 0; c < RC; ++c)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // the lane's NJ consecutive columns in one store (16- or 8-byte aligned: col % NJ == 0,
        // UL and D multiples of 8 floats, the partial 256-byte aligned plus a pass's kofs * D floats)
        const int off = du_lane + ((16 * c + i) * UL + k * D) * 4;
        if constexpr (NJ == 4)
          bstore128<false>(u32x4{__float_as_uint(du[k][c][0][i]), __float_as_uint(du[k][c][1][i]),
                                 __float_as_uint(du[k][c][2][i]), __float_as_uint(du[k][c][3][i])},
                           rdu, off);
        else
          __builtin_amdgcn_raw_buffer_store_b64(u32x2{__float_as_uint(du[k][c][0][i]), __float_as_uint(du[k][c][1][i])},
                                                rdu, off, 0, 0);
      }
}

// ------------------------------------------------------------------- host
namespace {

// Tile width and row runs per workgroup of a backward launch (see the kernel):
// 32-channel tiles for two rank chunks at W <= 4, two row runs per workgroup
// for one rank chunk at W <= 4, else 64-channel tiles and one run.  WIDE: the
// passes of a one-rank-chunk problem above W 8 take 32-channel tiles and one
// run (their later passes hold the earlier passes' dx as well, which 64-channel
// tiles at two runs per workgroup spill: W 16 at B4 T4096 D2048 R16 backward
// 440 us).
struct BwdShape {
  int cpw, nrw;
};
constexpr BwdShape bwd_shape(int W, int RC, bool wide = false) {
  return wide ? BwdShape{32, 1} : BwdShape{(RC == 2 && W <= 4) ? 32 : 64, (RC == 1 && W <= 4) ? 2 : 1};
}

// Taps per backward pass: what one pass's tap-weight and dz operands (registers
// and LDS) and dU accumulators hold for RC rank chunks.  Wider problems run as
// consecutive passes of taps kofs .. kofs+taps-1 (see the kernel's kofs),
// reading x and dy once per pass.  Every pass of a problem takes the same
// launch shape (bwd_shape: the dU partial rows of all passes line up); one rank
// chunk above W 4 runs passes of at most 8 taps on 32-channel tiles (bwd_shape's
// WIDE: 240-250 VGPRs at 8 taps, two wavefronts per SIMD; B4 T4096 D2048 R16
// W16 backward 271 -> 207 us against passes of 4 taps, W32 670 -> 377 us; W 5-8
// in one such pass 90-148 -> 66-103 us against one pass on 64-channel tiles at
// one wavefront per SIMD).
constexpr int pass_taps(int W, int RC) {
  return RC == 1 ? (W <= 8 ? W : 8) : RC == 2 ? (W < 4 ? W : 4) : RC == 3 ? (W < 2 ? W : 2) : 1;
}
constexpr int npasses(int W, int RC) { return (W + pass_taps(W, RC) - 1) / pass_taps(W, RC); }

// Rank chunks of a problem's launch shape: its own (one to four), or passes of
// kBwdRankPass ranks on the two-chunk kernels where lr_bwd_rank_split holds.
constexpr int kBwdRankPass = 32;
inline bool bwd_rank_split(const LrProblem& p) { return lr_bwd_rank_split(p.R + (p.static_w ? 1 : 0), p.W); }
inline int bwd_rc(const LrProblem& p) {
  const int rk = (int)(p.R + (p.static_w ? 1 : 0));
  return bwd_rank_split(p) ? 2 : (rk + 15) / 16;
}
inline int bwd_rank_passes(const LrProblem& p) {
  const int rk = (int)(p.R + (p.static_w ? 1 : 0));
  return bwd_rank_split(p) ? (rk + kBwdRankPass - 1) / kBwdRankPass : 1;
}

// More than four passes (ranks x taps) add dx into an fp32 accumulator in the
// workspace, whose last pass stores dx itself, rounded once (DXM 2; a launch
// that rounded the whole accumulator after the passes took 55 us more at B4
// T4096 D2048 R127 + static W4: 456 -> 400 us) (above W 16 at two rank chunks,
// above W 8 at three, above W 4 at four; one rank chunk takes at most four
// passes of 8 taps up to W 32), and so do more than two where the passes split
// the ranks: each rank pass adds a partial tap weight whose terms can cancel
// (dx near zero from partials of several units), and three or four roundings
// of such partials left single entries past the elementwise bar in a random
// sweep (|dx - dx_oracle| 0.0217 at R104 + static W1, 4 passes, and 0.0219 at
// R73 + static W2, 3 passes, against 0.02 + 2%).
constexpr int kBwdMaxBf16DxPasses = 4;
constexpr int kBwdMaxBf16DxRankPasses = 2;
// Passes of ranks at W <= 4 up to kernel rank 128 with dy in [B, T, D]: the
// passes form dz and dU only (DXM 3) and lr_dx_mfma forms dx over all ranks in
// one launch, rounded once (no fp32 accumulator).
inline bool bwd_dx_split(const LrProblem& p) {
  const int64_t rk = p.R + (p.static_w ? 1 : 0);
  return bwd_rank_split(p) && p.W <= 4 && rk <= 128 && p.yhd() == p.D;
}
// The workspace keeps room for the accumulator whether or not dx is split off:
// the size queries do not see dy's layout, on which the split depends.
inline bool bwd_f32dx_room(const LrProblem& p) {
  const int np = bwd_rank_passes(p) * npasses((int)p.W, bwd_rc(p));
  return np > kBwdMaxBf16DxPasses || (bwd_rank_passes(p) > 1 && np > kBwdMaxBf16DxRankPasses);
}
inline bool bwd_f32dx(const LrProblem& p) { return !bwd_dx_split(p) && bwd_f32dx_room(p); }

}  // namespace

// The passes of a backward launch sequence: kernel ranks rofs .. rofs+RK-1 (R
// of them dynamic) and taps kofs .. kofs+W-1; slot: the pass's dz partial slot
// (its pass of taps: the passes of ranks write disjoint columns of the same
// slots).  Every pass takes the same launch shape (bwd_rc), so the dU partial
// rows of all passes line up.
int bwd_plan(const LrProblem& p, BwdPass* out) {
  const int RK = (int)(p.R + (p.static_w ? 1 : 0)), W = (int)p.W, rc = bwd_rc(p);
  const int nrp = bwd_rank_passes(p), step = nrp > 1 ? kBwdRankPass : RK;
  const int ntp = npasses(W, rc);
  if (nrp * ntp > kBwdMaxPlan) return -1;
  int n = 0;
  for (int i = 0; i < nrp; ++i) {
    const int rofs = i * step, rk = RK - rofs < step ? RK - rofs : step;
    const int rd = (int)p.R - rofs < 0 ? 0 : ((int)p.R - rofs < rk ? (int)p.R - rofs : rk);
    // taps split as evenly as the pass count allows, the longer passes first
    // (each at most wp): a pass costs about one sweep of x, dy and dx plus its
    // taps' products, so W 9 as 5 + 4 beats 8 + 1
    for (int t = 0, kofs = 0; t < ntp; ++t) {
      BwdPass& b = out[n++];
      b.rofs = rofs;
      b.R = rd;
      b.RK = rk;
      b.kofs = kofs;
      b.W = W / ntp + (t < W % ntp ? 1 : 0);
      b.slot = t;
      kofs += b.W;
    }
  }
  return n;
}

// Longest backward run (tiles) whose resources fit (see run_rsrc): rows of x,
// dx, dy (one head's block of head-major dy), the z rows the kernel reads (z
// itself or the padded copy) and the fp32 dz partials.
int64_t lr_bwd_max_run_tiles(const LrProblem& p) {
  int64_t rowb = p.xld() * 2;
  // past four passes of taps the passes' dx rows are the fp32 accumulator (D floats each)
  const int64_t dxb = bwd_f32dx_room(p) ? p.D * 4 : p.dxld() * 2;
  // (the last pass over the accumulator also stores dx rows of dxld elements)
  const int64_t others[5] = {dxb, p.dxld() * 2, p.yhd() * 2, lr_bwd_zrow(p.R, p.static_w != nullptr, p.W) * 2,
                             p.R * 4};
  for (int64_t v : others) rowb = rowb > v ? rowb : v;
  return run_tiles_cap(rowb);
}

namespace {

LrBwdArgs make_bwd_args(const LrProblem& p, int target_waves) {
  LrBwdArgs a;
  const int rc = bwd_rc(p);
  const BwdShape sh = bwd_shape(pass_taps((int)p.W, rc), rc, rc == 1 && p.W > 4);  // every pass has the same shape
  const int ncw = 256 / sh.cpw;
  a.Tn = (int)p.T;
  a.D = (int)p.D;
  a.R = (int)p.R;
  a.RK = (int)p.R + (p.static_w ? 1 : 0);
  a.residual = p.residual;
  a.nch = (int)((p.D + sh.cpw - 1) / sh.cpw);
  a.ncg = (a.nch + ncw - 1) / ncw;
  const int64_t ntile = (p.T + 15) / 16;
  int64_t seg = (p.B * ntile * a.ncg * ncw + target_waves - 1) / target_waves;
  if (seg < 1) seg = 1;
  if (seg > ntile) seg = ntile;
  const int64_t cap = lr_bwd_max_run_tiles(p);  // >= 1 (lr_mfma_ok)
  if (seg > cap) seg = cap;
  a.seg = (int)seg;
  a.nspb = (int)((ntile + seg - 1) / seg);
  a.nseg = (int)(p.B * a.nspb);
  a.npair = (a.nseg + sh.nrw - 1) / sh.nrw;
  a.nblk = a.npair * a.ncg;
  a.BT = p.B * p.T;
  a.zld = a.zr = (int)p.R;
  a.zrk = a.RK;
  a.uld = (int)(p.W * p.D);
  a.kofs = 0;
  a.accdx = 0;
  a.dxsld = 0;
  a.nodx = 0;
  a.dzld = a.R;
  a.dupr = a.RK;
  return a;
}

// Ranks of the padded z_eff copy: RK rounded up to a multiple of 4, or 32 for
// two rank chunks (their 16x16x32 operands read ranks 8q..8q+7 of every row).
inline int64_t zpad_ranks(const LrProblem& p) { return lr_bwd_zrow(p.R, p.static_w != nullptr, p.W); }

// z_eff[t, r] = z[t, r] (r < R), 1 (r == R, static_w given), 0 up to RP: the
// backward's z operand when z cannot be read 8 bytes at a time.
struct ZpadArgs {
  const uint16_t* z[kMaxGroups];
  uint16_t* zp[kMaxGroups];
  int64_t n;  // BT * RP / 4: 4-rank pieces per group
  int R, RP, stat, one;
};
// One thread per 4 ranks of a padded row (RP % 4 == 0): four 2-byte reads of
// z (its rows need not be 4-byte aligned), one 8-byte store.  A grid-stride
// loop: the grid is capped (launch_zpad).
__global__ __launch_bounds__(256) void lr_zpad(ZpadArgs a) {
  const int g = blockIdx.y;
  const uint16_t* __restrict__ z = g == 0 ? a.z[0] : g == 1 ? a.z[1] : g == 2 ? a.z[2] : a.z[3];
  uint16_t* __restrict__ zp = g == 0 ? a.zp[0] : g == 1 ? a.zp[1] : g == 2 ? a.zp[2] : a.zp[3];
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < a.n; i += (int64_t)gridDim.x * 256) {
    const int64_t e = 4 * i;  // first element of the piece
    const int64_t t = e / a.RP;
    const int r0 = (int)(e - t * a.RP);
    uint32_t v[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int r = r0 + kk;
      v[kk] = r < a.R ? z[t * a.R + r] : (r == a.R && a.stat ? (uint32_t)a.one : 0u);
    }
    *reinterpret_cast<u32x2*>(zp + e) = u32x2{v[0] | (v[1] << 16), v[2] | (v[3] << 16)};
  }
}

// lr_zpad over G problems: z_eff of group g into dst[g].
template <typename T>
hipError_t launch_zpad(const LrProblem* p, int G, void* const* dst) {
  if (auditing()) return hipSuccess;  // plain pointers
  ZpadArgs za;
  const int64_t RP = zpad_ranks(p[0]);
  za.n = p[0].B * p[0].T * RP / 4;
  za.R = (int)p[0].R;
  za.RP = (int)RP;
  za.stat = p[0].static_w != nullptr;
  za.one = Mma16<T>::kOne;
  for (int g = 0; g < kMaxGroups; ++g) {
    za.z[g] = (const uint16_t*)p[g < G ? g : 0].z;
    za.zp[g] = (uint16_t*)dst[g < G ? g : 0];
  }
  const int64_t blocks = (za.n + 255) / 256;
  lr_zpad<<<dim3((unsigned)(blocks < 65536 ? blocks : 65536), G), 256, 0, p[0].stream>>>(za);
  return hipGetLastError();
}

constexpr int kBwdTargetWaves = 2048;

// The byte counts lr_bwd_mfma gives its buffer resources for pass b of wq taps
// (the range audit; see the kernel): U, static_w and the dU partial per pass;
// x, dy, dx, z and the dz partials for the longest run (from row 0).
void audit_bwd_pass(const LrBwdArgs& b, int wq, bool f32) {
  const int64_t D = b.D;
  audit_range(lr_u_bytes(b.R, b.uld, b.kofs, D, 2), kOobLane);
  audit_range(lr_sw_bytes(b.RK > b.R, wq, D, 2), kOobLane);
  audit_range(lr_dupart_bytes(b.RK, b.uld, b.kofs, D), kOobLane);
  const int64_t rows[6] = {(int64_t)b.xld * 2, (int64_t)b.yhd * 2, (int64_t)b.dxld * (f32 ? 4 : 2),
                           (int64_t)b.zld * 2, (int64_t)b.dzld * 4, (int64_t)b.dxsld * 2};
  for (int64_t rowb : rows) audit_range(run_rsrc_bytes(b.Tn, rowb), kOobTile - 15 * rowb);
}

// dx rows T-kt .. T-1 of every sequence from the passes' fp32 accumulator
// (rows of D floats), rounded to the output type into dx rows dxld elements
// apart: the rows that the last pass over the accumulator, whose taps start at
// kt, does not store.
struct DxRoundGroup {
  const float* src;
  uint16_t* dst;
};
struct DxRoundArgs {
  int64_t n4;   // B * kt * D / 4 quads per group
  int dq;       // D / 4 quads per row
  int kt;       // rows per sequence
  int Tn;
  int64_t dld;  // row stride of dx (elements, a multiple of 4)
  DxRoundGroup grp[kMaxGroups];
};

template <typename T>
__global__ __launch_bounds__(256) void lr_dx_round_tail(DxRoundArgs a) {
  const int g = blockIdx.y;
  const float* __restrict__ src = pick(a.grp, g, &DxRoundGroup::src);
  uint16_t* __restrict__ dst = pick(a.grp, g, &DxRoundGroup::dst);
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < a.n4; e += (int64_t)gridDim.x * 256) {
    const int64_t rl = e / a.dq;  // the tail row of the sequences, in order
    const int c = (int)(e - rl * a.dq) * 4;
    const int64_t b = rl / a.kt;
    const int64_t row = b * a.Tn + a.Tn - a.kt + (rl - b * a.kt);
    const float4 v = *reinterpret_cast<const float4*>(src + row * a.dq * 4 + c);
    u32x2 o;
    o[0] = pack2<T>(v.x, v.y);
    o[1] = pack2<T>(v.z, v.w);
    *reinterpret_cast<u32x2*>(dst + row * a.dld + c) = o;
  }
}

template <typename T>
hipError_t launch_dx_round_tail(const LrProblem* p, int G, int64_t dxf_off, int kofs) {
  if (auditing()) return hipSuccess;  // plain pointers
  DxRoundArgs a;
  a.kt = (int)(kofs < p[0].T ? kofs : p[0].T);
  a.Tn = (int)p[0].T;
  a.dq = (int)(p[0].D / 4);
  a.n4 = p[0].B * a.kt * a.dq;
  a.dld = p[0].dxld();
  for (int g = 0; g < kMaxGroups; ++g) {
    const LrProblem& q = p[g < G ? g : 0];
    a.grp[g] = DxRoundGroup{(const float*)((const char*)q.ws + dxf_off), (uint16_t*)q.dx};
  }
  const int64_t blocks = (a.n4 + 255) / 256;
  lr_dx_round_tail<T><<<dim3((unsigned)(blocks < 8192 ? blocks : 8192), G), 256, 0, p[0].stream>>>(a);
  return hipGetLastError();
}

// Workspace: [dz partials: passes x ncg x BT x R fp32][dU partials: npair x RK
// x W*D fp32][padded z_eff: BT x RP of z's type][past four passes, or two
// that split the ranks: the fp32 dx accumulator, BT x D], each 256-byte aligned.  The z_eff part is reserved
// whatever the pointers' alignment (the size query has none).
struct BwdWs {
  int64_t dz_off, du_off, zp_off, dxf_off, total;
};
BwdWs bwd_ws(const LrProblem& p, const LrBwdArgs& a) {
  BwdWs w;
  // one dz partial slot per pass of taps (the passes of ranks fill disjoint columns)
  const int64_t dz = (int64_t)npasses((int)p.W, bwd_rc(p)) * a.ncg * a.BT * a.R * 4;
  w.dz_off = 0;
  w.du_off = (dz + 255) / 256 * 256;
  w.zp_off = (w.du_off + (int64_t)a.npair * a.RK * p.W * p.D * 4 + 255) / 256 * 256;
  w.dxf_off = (w.zp_off + a.BT * zpad_ranks(p) * 2 + 255) / 256 * 256;
  w.total = w.dxf_off + (bwd_f32dx_room(p) ? a.BT * p.D * 4 : 0);
  return w;
}

template <typename T, int W, int RC, bool WIDE = false, bool F32 = false>
hipError_t launch_bwd_kernel(const LrBwdArgs& a, hipStream_t stream) {
  constexpr BwdShape SH = bwd_shape(W, RC, WIDE);  // as make_bwd_args
  constexpr int NRW = SH.nrw, CPW = SH.cpw, NT = 64 * (256 / CPW) * NRW;
  if constexpr (F32) {  // every pass on the fp32 dx accumulator; the last one stores dx itself
    if (a.accdx && a.dxsld > 0)
      lr_bwd_mfma<T, W, RC, NRW, CPW, true, 2><<<a.nblk, NT, 0, stream>>>(a);
    else if (a.accdx)
      lr_bwd_mfma<T, W, RC, NRW, CPW, true, 1><<<a.nblk, NT, 0, stream>>>(a);
    else
      lr_bwd_mfma<T, W, RC, NRW, CPW, false, 1><<<a.nblk, NT, 0, stream>>>(a);
    return hipGetLastError();
  }
  // later passes of taps: problems of 2+ rank chunks, and one rank chunk above W 8
  // (WIDE: passes of at most 8 taps)
  if constexpr (RC == 2 && !WIDE) {  // passes of ranks without dx (lr_dx_mfma forms it)
    if (a.nodx) {
      lr_bwd_mfma<T, W, RC, NRW, CPW, false, 3><<<a.nblk, NT, 0, stream>>>(a);
      return hipGetLastError();
    }
  }
  if constexpr (RC >= 2 || WIDE) {
    if (a.accdx) {
      lr_bwd_mfma<T, W, RC, NRW, CPW, true><<<a.nblk, NT, 0, stream>>>(a);
      return hipGetLastError();
    }
  }
  lr_bwd_mfma<T, W, RC, NRW, CPW, false><<<a.nblk, NT, 0, stream>>>(a);
  return hipGetLastError();
}

// One pass's kernel for wq taps and rc rank chunks (the instantiated pairs: up
// to pass_taps(W, RC) taps, as bwd_plan splits them); wide: a one-rank-chunk
// problem above W 4.
template <typename T>
hipError_t dispatch_bwd_kernel(const LrBwdArgs& a, int wq, int rc, bool wide, bool f32, hipStream_t stream) {
  if (f32) {  // more than four passes: two rank chunks above W 16, three or four above W 8 / 4
    switch (wq * 4 + rc) {  // (one rank chunk never takes more than four passes)
      case 6: return launch_bwd_kernel<T, 1, 2, false, true>(a, stream);
      case 10: return launch_bwd_kernel<T, 2, 2, false, true>(a, stream);
      case 14: return launch_bwd_kernel<T, 3, 2, false, true>(a, stream);
      case 18: return launch_bwd_kernel<T, 4, 2, false, true>(a, stream);
      case 7: return launch_bwd_kernel<T, 1, 3, false, true>(a, stream);
      case 11: return launch_bwd_kernel<T, 2, 3, false, true>(a, stream);
      case 8: return launch_bwd_kernel<T, 1, 4, false, true>(a, stream);
      default: return hipErrorInvalidValue;
    }
  }
  if (wide && rc == 1) {
    switch (wq) {
      case 1: return launch_bwd_kernel<T, 1, 1, true>(a, stream);
      case 2: return launch_bwd_kernel<T, 2, 1, true>(a, stream);
      case 3: return launch_bwd_kernel<T, 3, 1, true>(a, stream);
      case 4: return launch_bwd_kernel<T, 4, 1, true>(a, stream);
      case 5: return launch_bwd_kernel<T, 5, 1, true>(a, stream);
      case 6: return launch_bwd_kernel<T, 6, 1, true>(a, stream);
      case 7: return launch_bwd_kernel<T, 7, 1, true>(a, stream);
      case 8: return launch_bwd_kernel<T, 8, 1, true>(a, stream);
      default: return hipErrorInvalidValue;
    }
  }
#define DC_LR_CASE(WW, CC) \
  if (wq == WW && rc == CC) return launch_bwd_kernel<T, WW, CC>(a, stream);
  DC_LR_CASE(1, 1) DC_LR_CASE(2, 1) DC_LR_CASE(3, 1) DC_LR_CASE(4, 1)
  DC_LR_CASE(1, 2) DC_LR_CASE(2, 2) DC_LR_CASE(3, 2) DC_LR_CASE(4, 2)
  DC_LR_CASE(1, 3) DC_LR_CASE(2, 3)
  DC_LR_CASE(1, 4)
#undef DC_LR_CASE
  return hipErrorInvalidValue;
}

template <typename T>
hipError_t launch_bwd(const LrProblem* p, int G) {
  const int rc = bwd_rc(p[0]);
  BwdPass ps[kBwdMaxPlan];
  const int np = bwd_plan(p[0], ps);
  if (np < 1) return hipErrorInvalidValue;
  LrBwdArgs a = make_bwd_args(p[0], kBwdTargetWaves);
  const BwdWs w = bwd_ws(p[0], a);
  a.nblk1 = a.nblk;
  a.nblk = G * a.nblk1;
  a.xld = (int)p[0].xld();
  a.dxld = (int)p[0].dxld();
  a.yhd = (int)p[0].yhd();
  // z itself when its rows are what the kernel reads: R % 4 == 0 and 8-byte
  // aligned, or (two rank chunks, and passes of 32 ranks) rows of a multiple
  // of 32 dynamic ranks without the static one, 16-byte aligned.
  const bool K32 = rc == 2;
  bool zvec = K32 ? (p[0].R % 32 == 0 && p[0].static_w == nullptr) : p[0].R % 4 == 0;
  for (int g = 0; g < G; ++g) {
    float* pdz = (float*)((char*)p[g].ws + w.dz_off);
    float* pdu = (float*)((char*)p[g].ws + w.du_off);
    a.grp[g] = LrBwdGroup{p[g].x, p[g].z, p[g].U, p[g].static_w, p[g].dy, p[g].dx, pdz, pdu};
    zvec = zvec && aligned_to(p[g].z, K32 ? 16 : 8);
  }
  hipError_t e;
  if (!zvec) {
    // padded z_eff rows: the forward's copy when the caller kept it, else
    // written into the workspace first
    bool saved = true;
    for (int g = 0; g < G; ++g) saved = saved && p[g].zeff != nullptr;
    void* zp[kMaxGroups];
    for (int g = 0; g < G; ++g) zp[g] = saved ? p[g].zeff : (char*)p[g].ws + w.zp_off;
    if (!saved && (e = launch_zpad<T>(p, G, zp)) != hipSuccess) return e;
    for (int g = 0; g < G; ++g) a.grp[g].z = zp[g];
    a.zld = a.zr = a.zrk = (int)zpad_ranks(p[0]);
  }
  const int64_t D = p[0].D, WD = p[0].W * D, RKWD = (int64_t)a.RK * WD, R = p[0].R;
  const int64_t dz_slot = (int64_t)a.ncg * a.BT * R;  // one pass of taps' dz partials
  // past four passes every pass works on the fp32 accumulator (rows of D floats)
  const bool f32 = bwd_f32dx(p[0]), dxs = bwd_dx_split(p[0]);
  a.nodx = dxs ? 1 : 0;
  if (f32) {
    a.dxld = (int)D;
    for (int g = 0; g < G; ++g) a.grp[g].dx = (char*)p[g].ws + w.dxf_off;
  }
  a.dxsld = 0;
  for (int i = 0; i < np; ++i) {
    // pass i: ranks rofs .. (z from column rofs, U and the dU partial rows from
    // row rofs, dz partial columns from rofs, static_w in the pass that holds
    // rank R), taps kofs .. (U, static_w and the dU partial columns from tap
    // kofs; dz partials in the slot of its pass of taps); the residual in the
    // first pass only
    const BwdPass& f = ps[i];
    LrBwdArgs b = a;
    b.R = f.R;
    b.RK = f.RK;
    b.kofs = f.kofs;
    b.accdx = i > 0;
    b.residual = a.residual && i == 0;
    if (f32 && i == np - 1) {  // the last pass adds to the accumulator and stores dx, rounded once
      b.dxsld = (int)p[0].dxld();
      for (int g = 0; g < G; ++g) b.grp[g].dxs = p[g].dx;
    }
    for (int g = 0; g < G; ++g) {
      b.grp[g].z = static_cast<const T*>(a.grp[g].z) + f.rofs;
      b.grp[g].U = (const T*)p[g].U + f.rofs * WD + f.kofs * D;
      b.grp[g].sw = p[g].static_w && f.RK > f.R ? (const void*)((const T*)p[g].static_w + f.kofs * D) : nullptr;
      b.grp[g].part_dz = a.grp[g].part_dz + f.slot * dz_slot + f.rofs;
      b.grp[g].part_du = a.grp[g].part_du + f.rofs * WD + f.kofs * D;
    }
    if (auditing()) {
      audit_bwd_pass(b, f.W, f32);
      continue;
    }
    if ((e = dispatch_bwd_kernel<T>(b, f.W, rc, rc == 1 && p[0].W > 4, f32, p[0].stream)) != hipSuccess) return e;
  }
  if (dxs && (e = lr_dx_mfma_launch<T>(p, G)) != hipSuccess) return e;
  // The last pass stores dx rows 0 .. T-1-kofs of its taps kofs ..; the rows
  // after those (no terms of its taps) are rounded from the accumulator here
  // (passes that split only the ranks have kofs 0: nothing left).
  if (f32 && ps[np - 1].kofs > 0 && (e = launch_dx_round_tail<T>(p, G, w.dxf_off, ps[np - 1].kofs)) != hipSuccess)
    return e;
  PartialReduce jobs[kMaxReduceJobs];
  int nj = 0;
  const int nslot = npasses((int)p[0].W, rc);
  for (int g = 0; g < G; ++g) {
    const float* pdz = a.grp[g].part_dz;
    const float* pdu = a.grp[g].part_du;
    jobs[nj++] = {pdu, RKWD, a.npair, R * WD, p[g].dU};
    jobs[nj++] = {pdu + R * WD, RKWD, a.npair, p[g].static_w ? WD : 0, p[g].dstatic_w};
    jobs[nj++] = {pdz, a.BT * R, nslot * a.ncg, a.BT * R, p[g].dz};
  }
  return reduce_partials_multi(jobs, nj, p[0].dtype, p[0].stream);
}

}  // namespace

int64_t lr_mfma_ws_bytes(const LrProblem& p) { return bwd_ws(p, make_bwd_args(p, kBwdTargetWaves)).total; }

hipError_t lr_zeff_fill(const LrProblem* p, int G) {
  void* dst[kMaxGroups];
  for (int g = 0; g < G; ++g) dst[g] = p[g].zeff;
  return p[0].dtype == kBF16 ? launch_zpad<bf16>(p, G, dst) : launch_zpad<fp16>(p, G, dst);
}

hipError_t lr_mfma_bwd(const LrProblem* p, int G) {
  return p[0].dtype == kBF16 ? launch_bwd<bf16>(p, G) : launch_bwd<fp16>(p, G);
}

}  // namespace dc
