// Lowrank dynamic convolution in fp32 (the reference's tl.dot "ieee" branch,
// lowrank.py:60-61, 130-132, 196-198): forward and backward on the VALU.
//
// A lane owns one channel d of a 64-channel chunk and walks a run of rows of
// one sequence.  Its column of U_eff (U[:, k*D + d], plus static_w[k, d] as
// rank R, lowrank.py:223-225) sits in registers: RKP x W floats, RKP the kernel
// rank rounded up to 8, 16 or 32 (zero ranks beyond).  The z_eff row of the
// current step is the same for every lane of the wavefront: it is loaded once
// per chunk of rows across the lanes and broadcast from there.
//
//   forward   Kw_k = sum_r z[t, r] U[r, k, d];  y = sum_k Kw_k x[t-k] (+ x[t])
//   backward  dx by the scatter form (row s adds dy[s] Kw_k[s] into the open
//             accumulator of row s-k), G_k = dy[s] x[s-k] in fp32,
//             dU[r, k, d] += z[s, r] G_k (registers, one partial per run),
//             dz[s, r] = sum over channels of sum_k G_k U[r, k, d]: summed
//             across the wavefront's 64 lanes by a reduce-scatter butterfly
//             (lane l ends with rank l / (64/RKP)), then across the
//             workgroup's 4 chunks in LDS in wave order (one partial per
//             256 channels).
//
// Everything is fp32 with fp32 accumulation, in a fixed order (deterministic).
// Rows before 0 or past the run and lanes past D use buffer range checks
// (loads read 0, stores are dropped), as the other fast paths do.
#include "lowrank_mfma.h"

namespace dc {

struct LrF32Args {
  int Tn, D, R, RK, residual;
  int xld, dxld;  // row strides of x and dx (elements)
  int yhd;        // y / dy layout: D ([B, T, D]) or the head dim of [B, D/yhd, T, yhd] (yhd % 64 == 0)
  int nch;        // ceil(D / 64) chunks
  int ncg;        // ceil(nch / 4): workgroup columns (256 channels)
  int seg;        // rows per run
  int nspb;       // runs per sequence
  int nseg;       // B * nspb
  int nblk;       // ncg * nseg
  int64_t BT;
};

// Rows per chunk: a multiple of W, at least 4 (ring slots are compile-time).
template <int W> struct F32Unroll { static constexpr int value = (W >= 4) ? W : W * (4 / W); };

template <int W>
__device__ __forceinline__ constexpr int f32ring(int u, int k) {
  return ((u - k) % W + W) % W;
}

// z_eff of the UC rows of a chunk, spread over the wavefront: entry
// e = uu * RKP + r (row tc + uu, rank r) sits in register e / 64 of lane
// e % 64.  One coalesced load per register; ranks r >= R and rows past T read 0
// (buffer range), and finish() adds the static rank's 1.  row() hands a row to
// the VALU as wave-uniform values (v_readlane into SGPRs).
template <int UC, int RKP>
struct ZChunk {
  static constexpr int N = (UC * RKP + 63) / 64;
  float v[N];

  __device__ __forceinline__ void load(rsrc_t rz, int tc, int R, int lane) {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int e = j * 64 + lane, uu = e / RKP, r = e % RKP;
      v[j] = __uint_as_float(bload32(rz, (uu < UC && r < R) ? ((tc + uu) * R + r) * 4 : kOobTile));
    }
  }
  __device__ __forceinline__ void finish(const float (&fill)[N]) {
#pragma unroll
    for (int j = 0; j < N; ++j) v[j] += fill[j];
  }
  __device__ __forceinline__ void row(float (&zv)[RKP], int uu) const {
#pragma unroll
    for (int r = 0; r < RKP; ++r) {
      const int e = uu * RKP + r;
      zv[r] = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v[e / 64]), e % 64));
    }
  }
  // 1 in the static rank's entries (R < RK), 0 elsewhere
  __device__ static __forceinline__ void fill_of(float (&fill)[N], int R, int RK, int lane) {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int r = (j * 64 + lane) % RKP;
      fill[j] = (r >= R && r < RK) ? 1.f : 0.f;
    }
  }
};

// The lane's U_eff column: U[r, k*D + d] for r < R, static_w[k, d] as rank R,
// 0 beyond and for lanes past D (buffer loads at out-of-range offsets).
template <int W, int RKP>
__device__ __forceinline__ void load_ucol(float (&u)[RKP][W], const float* __restrict__ U,
                                          const float* __restrict__ sw, int R, int RK, int D, int d, bool dv) {
  const rsrc_t ru = make_rsrc(U, lr_u_bytes(R, (int64_t)W * D, 0, D, 4));
  const rsrc_t rs = make_rsrc(sw, lr_sw_bytes(sw != nullptr, W, D, 4));
#pragma unroll
  for (int r = 0; r < RKP; ++r)
#pragma unroll
    for (int k = 0; k < W; ++k) {
      const int col = (k * D + d) * 4;
      const float vu = __uint_as_float(bload32(ru, dv && r < R ? r * W * D * 4 + col : kOobLane));
      const float vs = __uint_as_float(bload32(rs, dv && r == R && r < RK ? col : kOobLane));
      u[r][k] = vu + vs;
    }
}

// ------------------------------------------------------------------ forward
template <int W, int RKP>
__global__ __launch_bounds__(256) void lr_fwd_f32(const float* __restrict__ x, const float* __restrict__ z,
                                                  const float* __restrict__ U, const float* __restrict__ sw,
                                                  float* __restrict__ y, LrF32Args a) {
  constexpr int UC = F32Unroll<W>::value;
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int lb = xcd_remap(blockIdx.x, a.nblk);
  const int cg = lb % a.ncg, s = lb / a.ncg;  // 4 wavefronts: 4 adjacent chunks, one run
  const int d = (cg * 4 + wave) * 64 + lane;
  const int D = a.D, Tn = a.Tn, R = a.R, RK = a.RK;
  const bool dv = d < D;
  const int b = s / a.nspb;
  const int t0 = (s - b * a.nspb) * a.seg;
  const int t1 = min(t0 + a.seg, Tn);
  const int64_t row0 = (int64_t)b * Tn;
  // y: the wavefront's 64 channels lie in one head (yhd % 64 == 0), whose
  // [T, yhd] block the resource covers (the whole [T, D] row block when yhd == D).
  const int yhd = a.yhd, head = ((cg * 4 + wave) * 64) / yhd;
  const int xrowb = a.xld * 4, yrowb = yhd * 4;
  const rsrc_t rx = make_rsrc(x + row0 * a.xld, (int64_t)Tn * xrowb);
  const rsrc_t ry = make_rsrc(y + row0 * D + (int64_t)head * Tn * yhd, (int64_t)Tn * yrowb);
  const int lo = dv ? d * 4 : kOobLane;
  const int ylo = dv ? (d - head * yhd) * 4 : kOobLane;
  const rsrc_t rz = make_rsrc(z + row0 * R, (int64_t)Tn * R * 4);
  typedef ZChunk<UC, RKP> ZC;
  float zfill[ZC::N];
  ZC::fill_of(zfill, R, RK, lane);

  float u[RKP][W];
  load_ucol<W, RKP>(u, U, sw, R, RK, D, d, dv);
  float xf[W];  // ring: row t in slot (t - t0) mod W; rows before 0 read 0
  xf[0] = 0.f;
#pragma unroll
  for (int i = 1; i < W; ++i) xf[W - i] = __uint_as_float(bload32(rx, lo + (t0 - i) * xrowb));

  struct Chunk {
    float x[UC];
    ZC z;
  };
  auto load_chunk = [&](int tc, Chunk& c) {
#pragma unroll
    for (int uu = 0; uu < UC; ++uu) {
      const int t = tc + uu;
      c.x[uu] = __uint_as_float(bload32(rx, lo + (t < t1 ? t * xrowb : kOobTile)));
    }
    c.z.load(rz, tc, R, lane);
  };
  auto compute_chunk = [&](int tc, Chunk& c) {
    c.z.finish(zfill);
#pragma unroll
    for (int uu = 0; uu < UC; ++uu) {
      const int t = tc + uu;
      const int p = uu % W;
      xf[p] = c.x[uu];
      float zv[RKP];
      c.z.row(zv, uu);
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < W; ++k) {
        float kw = 0.f;
#pragma unroll
        for (int r = 0; r < RKP; ++r) kw = fmaf(zv[r], u[r][k], kw);
        acc = fmaf(kw, xf[f32ring<W>(uu, k)], acc);
      }
      if (a.residual) acc += xf[p];
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc), ry, ylo + (t < t1 ? t * yrowb : kOobTile), 0, kNt);
    }
  };
  Chunk ca, cb;
  load_chunk(t0, ca);
  for (int tc = t0; tc < t1; tc += 2 * UC) {
    load_chunk(tc + UC, cb);
    __builtin_amdgcn_sched_barrier(0);
    compute_chunk(tc, ca);
    load_chunk(tc + 2 * UC, ca);
    __builtin_amdgcn_sched_barrier(0);
    if (tc + UC < t1) compute_chunk(tc + UC, cb);
  }
}

// ----------------------------------------------------------------- backward
// Sum over the 64 lanes of v[0 .. RKP), reduce-scattered: each step pairs every
// lane with a partner that differs in one lane bit (and agrees in the bits of
// the steps before), keeps the half of its entries that bit selects (upper half
// when set) and adds the partner's copy of that half, halving the entries.
// Bits 5 and 4 pair lanes through v_permlane32_swap / v_permlane16_swap (one
// swap exchanges both halves, so their sums need no selects); bits 3, 2, 1, 0
// through DPP within a row of 16 lanes: row_ror:8 (lane ^ 8), row_half_mirror
// (lane ^ 7: flips bit 2), quad_perm [3,2,1,0] (lane ^ 3: flips bit 1) and
// quad_perm [1,0,3,2] (lane ^ 1).  Lane l ends with rank l / (64 / RKP),
// summed over all 64 lanes (every lane of its group of 64 / RKP holds it).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppRor8 = 0x128, kDppHalfMirror = 0x141, kDppQuadRev = 0x1B, kDppQuadSwap1 = 0xB1;

template <int RKP, int N, int SWAP>
__device__ __forceinline__ void rs_swap(float (&v)[RKP]) {
#pragma unroll
  for (int i = 0; i < N / 2; ++i) {
    const auto p = SWAP == 32 ? __builtin_amdgcn_permlane32_swap(__float_as_uint(v[i]), __float_as_uint(v[N / 2 + i]),
                                                                 false, false)
                              : __builtin_amdgcn_permlane16_swap(__float_as_uint(v[i]), __float_as_uint(v[N / 2 + i]),
                                                                 false, false);
    v[i] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
  }
}

template <int RKP, int N, int BIT, int CTRL>
__device__ __forceinline__ void rs_dpp(float (&v)[RKP], int lane) {
  const bool hi = (lane & BIT) != 0;
#pragma unroll
  for (int i = 0; i < N / 2; ++i) {
    const float send = hi ? v[i] : v[N / 2 + i];
    const float keep = hi ? v[N / 2 + i] : v[i];
    v[i] = keep + dpp_mov<CTRL>(send);
  }
}

template <int RKP>
__device__ __forceinline__ float lane_reduce(float (&v)[RKP], int lane) {
  static_assert(RKP == 8 || RKP == 16 || RKP == 32, "rank padding");
  rs_swap<RKP, RKP, 32>(v);
  rs_swap<RKP, RKP / 2, 16>(v);
  rs_dpp<RKP, RKP / 4, 8, kDppRor8>(v, lane);
  if constexpr (RKP >= 16) rs_dpp<RKP, RKP / 8, 4, kDppHalfMirror>(v, lane);
  if constexpr (RKP >= 32) rs_dpp<RKP, RKP / 16, 2, kDppQuadRev>(v, lane);
  float s = v[0];
  if constexpr (RKP <= 8) s += dpp_mov<kDppHalfMirror>(s);
  if constexpr (RKP <= 16) s += dpp_mov<kDppQuadRev>(s);
  s += dpp_mov<kDppQuadSwap1>(s);
  return s;
}

template <int W, int RKP>
__global__ __launch_bounds__(256) void lr_bwd_f32(const float* __restrict__ x, const float* __restrict__ z,
                                                  const float* __restrict__ U, const float* __restrict__ sw,
                                                  const float* __restrict__ dy, float* __restrict__ dx,
                                                  float* __restrict__ part_dz, float* __restrict__ part_du,
                                                  LrF32Args a) {
  constexpr int UC = F32Unroll<W>::value;
  constexpr int DZB = 16;  // rows per dz batch (one barrier per batch)
  constexpr int LPR = 64 / RKP;  // lanes per rank after the butterfly
  __shared__ float dzs[2][4][DZB][RKP];
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int lb = xcd_remap(blockIdx.x, a.nblk);
  const int cg = lb % a.ncg, s = lb / a.ncg;  // 4 wavefronts: 4 adjacent chunks, one run
  const int d = (cg * 4 + wave) * 64 + lane;
  const int D = a.D, Tn = a.Tn, R = a.R, RK = a.RK;
  const bool dv = d < D;
  const int b = s / a.nspb;
  const int t0 = (s - b * a.nspb) * a.seg;
  const int t1 = min(t0 + a.seg, Tn);
  const int tend = t1 + W - 1;  // steps t0 .. tend-1: dx of row t needs dy, z of rows t .. t+W-1
  const int64_t row0 = (int64_t)b * Tn;
  // dy: [B, T, D] or head-major, as y in the forward
  const int yhd = a.yhd, head = ((cg * 4 + wave) * 64) / yhd;
  const int xrowb = a.xld * 4, rowb = yhd * 4, dxrowb = a.dxld * 4;
  const rsrc_t rx = make_rsrc(x + row0 * a.xld, (int64_t)Tn * xrowb);
  const rsrc_t rdy = make_rsrc(dy + row0 * D + (int64_t)head * Tn * yhd, (int64_t)Tn * rowb);
  const rsrc_t rdx = make_rsrc(dx + row0 * a.dxld, (int64_t)Tn * dxrowb);
  const int lo = dv ? d * 4 : kOobLane;
  const int ylo = dv ? (d - head * yhd) * 4 : kOobLane;
  const rsrc_t rz = make_rsrc(z + row0 * R, (int64_t)Tn * R * 4);
  typedef ZChunk<UC, RKP> ZC;
  float zfill[ZC::N];
  ZC::fill_of(zfill, R, RK, lane);
  const int64_t WD = (int64_t)W * D;

  float u[RKP][W], du[RKP][W];
  load_ucol<W, RKP>(u, U, sw, R, RK, D, d, dv);
#pragma unroll
  for (int r = 0; r < RKP; ++r)
#pragma unroll
    for (int k = 0; k < W; ++k) du[r][k] = 0.f;
  float xf[W], dxa[W];
  xf[0] = 0.f;
#pragma unroll
  for (int i = 1; i < W; ++i) xf[W - i] = __uint_as_float(bload32(rx, lo + (t0 - i) * xrowb));
#pragma unroll
  for (int k = 0; k < W; ++k) dxa[k] = 0.f;

  struct Chunk {
    float dy[UC], x[UC];
    ZC z;
  };
  auto load_chunk = [&](int tc, Chunk& c) {
#pragma unroll
    for (int uu = 0; uu < UC; ++uu) {
      const int t = tc + uu;
      c.dy[uu] = __uint_as_float(bload32(rdy, ylo + (t < tend ? t * rowb : kOobTile)));  // rows past T read 0
      c.x[uu] = __uint_as_float(bload32(rx, lo + (t < t1 ? t * xrowb : kOobTile)));
    }
    c.z.load(rz, tc, R, lane);
  };
  auto compute_chunk = [&](int tc, Chunk& c) {
    c.z.finish(zfill);
#pragma unroll
    for (int uu = 0; uu < UC; ++uu) {
      const int t = tc + uu;
      const int p = uu % W;
      const float dyv = c.dy[uu];
      float zv[RKP];
      c.z.row(zv, uu);
      // dx[t-k] += dy[t] Kw_k[t]; row t opens with its k = 0 term (+ residual).
#pragma unroll
      for (int k = 0; k < W; ++k) {
        float kw = 0.f;
#pragma unroll
        for (int r = 0; r < RKP; ++r) kw = fmaf(zv[r], u[r][k], kw);
        const int q = f32ring<W>(uu, k);
        if (k == 0)
          dxa[q] = a.residual ? fmaf(dyv, kw, dyv) : dyv * kw;
        else
          dxa[q] = fmaf(dyv, kw, dxa[q]);
      }
      // Rows past the run (t >= t1) only close dx: their G_k is 0 (dy taken
      // as 0), so dU and dz gain nothing, and their dz rows are not stored.
      const bool live = t < t1;  // wave-uniform (the 4 wavefronts share the run)
      xf[p] = c.x[uu];
      const float dyg = live ? dyv : 0.f;
      float g[W];
#pragma unroll
      for (int k = 0; k < W; ++k) g[k] = dyg * xf[f32ring<W>(uu, k)];
      float dzv[RKP];
#pragma unroll
      for (int r = 0; r < RKP; ++r) {
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < W; ++k) {
          du[r][k] = fmaf(zv[r], g[k], du[r][k]);
          acc = fmaf(g[k], u[r][k], acc);
        }
        dzv[r] = acc;
      }
      const float tot = lane_reduce<RKP>(dzv, lane);
      const int it = t - t0, slot = it % DZB, buf = (it / DZB) & 1;
      if (live && (lane & (LPR - 1)) == 0) dzs[buf][wave][slot][lane / LPR] = tot;
      if (live && (slot == DZB - 1 || t == t1 - 1)) {
        __syncthreads();
        const int tb = t - slot;  // first row of the batch
        for (int e = threadIdx.x; e < (slot + 1) * RKP; e += 256) {
          const int sl = e / RKP, r = e - sl * RKP;
          const float v = ((dzs[buf][0][sl][r] + dzs[buf][1][sl][r]) + dzs[buf][2][sl][r]) + dzs[buf][3][sl][r];
          if (r < R) part_dz[((int64_t)cg * a.BT + row0 + tb + sl) * R + r] = v;
        }
      }
      const int tdone = t - (W - 1);
      __builtin_amdgcn_raw_buffer_store_b32(
          __float_as_uint(dxa[(uu + 1) % W]), rdx,
          lo + (tdone >= t0 && tdone < t1 ? tdone * dxrowb : kOobTile), 0, kNt);
      __builtin_amdgcn_sched_barrier(0);  // one row's z_eff in SGPRs at a time
    }
  };
  Chunk ca, cb;
  load_chunk(t0, ca);
  for (int tc = t0; tc < tend; tc += 2 * UC) {
    load_chunk(tc + UC, cb);
    __builtin_amdgcn_sched_barrier(0);
    compute_chunk(tc, ca);
    load_chunk(tc + 2 * UC, ca);
    __builtin_amdgcn_sched_barrier(0);
    if (tc + UC < tend) compute_chunk(tc + UC, cb);
  }

  // dU (and dstatic_w as rank R) partial of this run
  if (dv) {
#pragma unroll
    for (int r = 0; r < RKP; ++r)
#pragma unroll
      for (int k = 0; k < W; ++k)
        if (r < RK) part_du[((int64_t)s * RK + r) * WD + (int64_t)k * D + d] = du[r][k];
  }
}

// ------------------------------------------------------------------- host
namespace {

int rank_pad(int64_t RK) { return RK <= 8 ? 8 : RK <= 16 ? 16 : 32; }

LrF32Args make_f32_args(const LrProblem& p, int target_waves) {
  LrF32Args a;
  a.Tn = (int)p.T;
  a.D = (int)p.D;
  a.R = (int)p.R;
  a.RK = (int)p.R + (p.static_w ? 1 : 0);
  a.residual = p.residual;
  a.xld = (int)p.xld();
  a.dxld = (int)p.dxld();
  a.yhd = (int)p.yhd();
  a.nch = (int)((p.D + 63) / 64);
  a.ncg = (a.nch + 3) / 4;
  int64_t seg = (p.B * p.T * a.ncg * 4 + target_waves - 1) / target_waves;
  if (seg < 16) seg = 16;
  if (seg > p.T) seg = p.T;
  a.seg = (int)seg;
  a.nspb = (int)((p.T + seg - 1) / seg);
  a.nseg = (int)(p.B * a.nspb);
  a.nblk = a.nseg * a.ncg;
  a.BT = p.B * p.T;
  return a;
}

constexpr int kF32TargetWaves = 2048;

struct F32Ws {
  int64_t dz_off, du_off, total;
};
F32Ws f32_ws(const LrProblem& p, const LrF32Args& a) {
  F32Ws w;
  w.dz_off = 0;
  w.du_off = ((int64_t)a.ncg * a.BT * a.R * 4 + 255) / 256 * 256;
  w.total = w.du_off + (int64_t)a.nseg * a.RK * p.W * p.D * 4;
  return w;
}

template <int W, int RKP>
hipError_t launch_f32(const LrProblem& p, bool bwd) {
  const LrF32Args a = make_f32_args(p, kF32TargetWaves);
  if (auditing()) {
    // U and static_w; one sequence of x, y or dy (one head's block) and dx, z
    audit_range(lr_u_bytes(a.R, (int64_t)W * a.D, 0, a.D, 4), kOobLane);
    audit_range(lr_sw_bytes(p.static_w != nullptr, W, a.D, 4), kOobLane);
    const int64_t rows[4] = {(int64_t)a.xld * 4, (int64_t)a.yhd * 4, (int64_t)p.dxld() * 4, (int64_t)a.R * 4};
    for (int64_t rowb : rows) audit_range((int64_t)a.Tn * rowb, kMaxSeqBytes - kSeqSlackRows * rowb);
    return hipSuccess;
  }
  if (!bwd) {
    lr_fwd_f32<W, RKP><<<a.nblk, 256, 0, p.stream>>>((const float*)p.x, (const float*)p.z, (const float*)p.U,
                                                      (const float*)p.static_w, (float*)p.y, a);
    return hipGetLastError();
  }
  const F32Ws w = f32_ws(p, a);
  float* pdz = (float*)((char*)p.ws + w.dz_off);
  float* pdu = (float*)((char*)p.ws + w.du_off);
  lr_bwd_f32<W, RKP><<<a.nblk, 256, 0, p.stream>>>((const float*)p.x, (const float*)p.z, (const float*)p.U,
                                                    (const float*)p.static_w, (const float*)p.dy, (float*)p.dx,
                                                    pdz, pdu, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t WD = p.W * p.D, RKWD = (int64_t)a.RK * WD;
  const PartialReduce jobs[3] = {
      {pdu, RKWD, a.nseg, p.R * WD, p.dU},
      {pdu + p.R * WD, RKWD, a.nseg, p.static_w ? WD : 0, p.dstatic_w},
      {pdz, a.BT * a.R, a.ncg, a.BT * a.R, p.dz},
  };
  return reduce_partials_multi(jobs, 3, p.dtype, p.stream);
}

}  // namespace

// fp32, W <= 4, kernel rank <= 32 (the lane's U column and dU in registers),
// sequences within the buffer range.
bool lr_f32_ok(const LrProblem& p) {
  if (p.dtype != kFP32) return false;
  if (p.W < 1 || p.W > 4) return false;
  if (p.R + (p.static_w ? 1 : 0) > 32) return false;
  if (p.R * p.W * p.D * 4 >= kOobLane) return false;  // U column offsets
  if (!aligned_to(p.x, 4) || !aligned_to(p.dy, 4) || !aligned_to(p.dx, 4)) return false;  // 4-byte buffer accesses
  if (p.yhd() != p.D && p.yhd() % 64 != 0) return false;  // a wavefront's 64 channels in one head
  const int64_t ld = p.xld() > p.dxld() ? p.xld() : p.dxld();
  if ((p.T + kSeqSlackRows) * ld * 4 > kMaxSeqBytes) return false;
  if ((p.T + kSeqSlackRows) * p.R * 4 > kMaxSeqBytes) return false;  // z rows
  return (p.T + kSeqSlackRows) * p.D * 4 <= kMaxSeqBytes;            // y / dy rows
}

int64_t lr_f32_ws_bytes(const LrProblem& p) { return f32_ws(p, make_f32_args(p, kF32TargetWaves)).total; }

hipError_t lr_f32(const LrProblem& p, bool bwd) {
  const int rkp = rank_pad(p.R + (p.static_w ? 1 : 0));
#define DC_F32_CASE(WW, RR) \
  if (p.W == WW && rkp == RR) return launch_f32<WW, RR>(p, bwd);
  DC_F32_CASE(1, 8) DC_F32_CASE(1, 16) DC_F32_CASE(1, 32)
  DC_F32_CASE(2, 8) DC_F32_CASE(2, 16) DC_F32_CASE(2, 32)
  DC_F32_CASE(3, 8) DC_F32_CASE(3, 16) DC_F32_CASE(3, 32)
  DC_F32_CASE(4, 8) DC_F32_CASE(4, 16) DC_F32_CASE(4, 32)
#undef DC_F32_CASE
  return hipErrorInvalidValue;
}

}  // namespace dc
