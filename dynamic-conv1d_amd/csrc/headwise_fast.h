// Headwise dynamic causal short convolution, forward and backward, for gfx950.
//
//   y[b,t,d] = sum_{k<W} (w[b,t,d/hs,k] + sw[k,d]) * x[b,t-k,d]  (+ x[b,t,d])
//
// Reference kernels: headwise.py:24-91 (causal_conv1d_fwd_kernel) and
// headwise.py:105-215 (causal_conv1d_bwd_kernel).
//
// Design (fast path).  The convolution is depthwise: a channel's window never
// mixes with another channel's, so the W-1 row halo of a channel lives in the
// registers of the lane that owns it.  A lane owns VEC = 16/sizeof(T)
// channels (one 128-bit load per row) and walks a run of `seg` consecutive
// rows of one sequence, keeping the last W rows of x (forward) or the W open
// dx accumulators (backward) in a register ring whose slot for row t is
// (t - t0) mod W.  Rows are processed in chunks of U (a multiple of W), so
// every ring index is a compile-time constant.  Each row costs exactly one
// 128-bit load of x (and dy), one contiguous load of the lane's NHL*W
// weights, and one 128-bit store: the HBM traffic is the algorithmic traffic
// plus a W-1 row halo per run.  64 lanes of a wavefront cover 64*VEC
// consecutive channels (a 1 KiB contiguous row segment per load instruction);
// a 256-thread workgroup stacks 4 wavefronts on 4 consecutive runs of the same
// channels, so a run's halo rows were just read by the wavefront above it.
//
// Memory pipeline.  All row traffic goes through buffer resources that cover
// the run's rows (rows before 0 or past T, and lanes past D, read 0 and drop
// stores), so no load sits under a branch.  Two chunk buffers, A and B,
// alternate: the next chunk's loads are issued before the current chunk is
// computed and no register is copied between them, so the compiler's waits
// stay partial (vmcnt counts in order: a load under a branch or a copy of a
// just-loaded register would make it wait for every load in flight).  x and
// dy rows are whole 1 KiB wavefront rows read once: nontemporal loads (B4
// T4096 D2048 W4 bf16: head size 32 forward 29.5 -> 27.6 us, backward
// 50.6 -> 47.2 us; head size 1 75.6 -> 72.7 and 150.9 -> 146.4 us).  Per-lane
// weight loads keep the default policy: at head size 1 a lane's 64-byte piece
// takes 4 instructions, and nontemporal lines are fetched again between them
// (forward 75 -> 98 us).  In whole wavefronts such pieces are loaded as
// contiguous 1 KiB instructions and handed to their lanes through LDS
// instead (TdwOf below), and those loads are nontemporal.
//
// Backward.  dx uses the scatter form: the row-t terms dy[t]*(w[t,k]+sw[k])
// are added into the open accumulator of row t-k; row t-W+1 is complete
// after step t and is stored.  dweight sums dy[t]*x[t-k] over the head's
// channels: in-lane when head_size <= VEC, then a butterfly over the
// head_size/VEC lanes of the head.  When a lane's dweight row piece is more
// than 16 bytes (head_size < VEC, e.g. 64 bytes at head_size 1, W 4, bf16),
// stores of it straight from the lanes write each 128-byte line in several
// partial pieces, which measured ~30% below contiguous stores; the wavefront
// then passes its dweight row through LDS and stores it as 16-byte lane
// pieces that are contiguous across the wavefront (TDW).  dstatic_w partial
// sums stay in registers for the whole run, are added across the 4 wavefronts
// of the workgroup in LDS in a fixed order, and one fp32 partial per workgroup
// is summed by reduce_partials (no atomics: bitwise deterministic).
#pragma once

#include "dc_common.h"
#include "dc_launch.h"

namespace dc {

template <typename T> struct VecOf { static constexpr int value = 16 / (int)sizeof(T); };

struct HwArgs {
  int Tn;        // sequence length
  int D;         // channels
  int H;         // heads
  int hs_shift;  // log2(head_size)
  int nvc;       // D / VEC lane columns
  int nvg;       // ceil(nvc / 64) wavefront column groups
  int seg;       // rows per run
  int nspb;      // runs per sequence = ceil(T / seg)
  int nseg;      // B * nspb
  int nblk;      // grid size
  int lph;       // lanes per head (head_size / VEC when > 1, else 1)
  int residual;
  int has_static;
};

// Rows per chunk: a multiple of W, at least 4.
template <int W> struct Unroll { static constexpr int value = (W >= 4) ? W : W * (4 / W); };

template <int W>
__device__ __forceinline__ constexpr int ring(int u, int k) {
  return ((u - k) % W + W) % W;
}

// Buffer geometry of one run.  The resources start at row `base` = the run's
// first halo row (max(t0 - (W-1), 0)) and end at T (capped at kHwRunBytes);
// the host keeps (seg + kHwSlackRows) rows of x and of weight within
// kHwRunBytes, so every in-range offset is below it, kHwRowOob (a row offset)
// and kHwLaneOob (a lane offset) are out of range alone or together, and no
// sum of offsets leaves int32.
constexpr int kHwRunBytes = 1 << 29;
constexpr int kHwRowOob = 1 << 29;
constexpr int kHwLaneOob = 1 << 30;
constexpr int kHwSlackRows = 40;

struct HwRun {
  int t0, t1;   // rows [t0, t1) of sequence b
  int base;     // first row covered by the resources
  int rowb;     // bytes per row of x / y / dy / dx
  int wrowb;    // bytes per row of weight / dweight
  int64_t xrow0, wrow0;  // element offsets of row `base` of sequence b
  int xrec, wrec;        // resource ranges (bytes)
  __device__ __forceinline__ HwRun(const HwArgs& a, int s, int W, int es) {
    const int b = s / a.nspb;
    t0 = (s - b * a.nspb) * a.seg;
    t1 = min(t0 + a.seg, a.Tn);
    base = max(t0 - (W - 1), 0);
    rowb = a.D * es;
    wrowb = a.H * W * es;
    xrow0 = ((int64_t)b * a.Tn + base) * a.D;
    wrow0 = ((int64_t)b * a.Tn + base) * a.H * W;
    xrec = (int)min((int64_t)(a.Tn - base) * rowb, (int64_t)kHwRunBytes);
    wrec = (int)min((int64_t)(a.Tn - base) * wrowb, (int64_t)kHwRunBytes);
  }
  // byte offset of row t, or the out-of-range row offset when !live
  __device__ __forceinline__ int xrow(int t, bool live = true) const { return live ? (t - base) * rowb : kHwRowOob; }
  __device__ __forceinline__ int wrow(int t, bool live = true) const { return live ? (t - base) * wrowb : kHwRowOob; }
};

// acc + a.lo * b.lo + a.hi * b.hi for packed 16-bit pairs (v_dot2c_f32_bf16 /
// v_dot2c_f32_f16): the products of two 16-bit values are exact in fp32.
template <typename T> struct Dot2;
template <> struct Dot2<bf16> {
  typedef __bf16 v2 __attribute__((ext_vector_type(2)));
  __device__ static __forceinline__ float run(uint32_t a, uint32_t b, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b), acc, false);
  }
};
template <> struct Dot2<fp16> {
  typedef _Float16 v2 __attribute__((ext_vector_type(2)));
  __device__ static __forceinline__ float run(uint32_t a, uint32_t b, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b), acc, false);
  }
};

// Sum over aligned groups of N lanes (N a power of two, 1..64), leaving the
// group sum in every lane of the group: DPP butterflies (quad_perm xor 1,
// xor 2, row_half_mirror, row_mirror: each pairs a lane with one of the other
// half of its group, and fuses into the add) up to 16 lanes, ds_bpermute
// beyond.
template <int N>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (N >= 2) v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
  if constexpr (N >= 4) v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
  if constexpr (N >= 8) v += dpp_f<0x141>(v);  // row_half_mirror
  if constexpr (N >= 16) v += dpp_f<0x140>(v); // row_mirror
  if constexpr (N >= 32) v += __shfl_xor(v, 16);
  if constexpr (N >= 64) v += __shfl_xor(v, 32);
  return v;
}

// The same for a group size n known only at run time (wave-uniform): the DPP
// steps run always and are selected by n (no branch); 32- and 64-lane groups
// add two ds_bpermute steps under one wave-uniform branch.
__device__ __forceinline__ float group_sum_sel(float v, int n) {
  float d = dpp_f<0xB1>(v);  // quad_perm [1,0,3,2]
  v = n >= 2 ? v + d : v;
  d = dpp_f<0x4E>(v);        // quad_perm [2,3,0,1]
  v = n >= 4 ? v + d : v;
  d = dpp_f<0x141>(v);       // row_half_mirror
  v = n >= 8 ? v + d : v;
  d = dpp_f<0x140>(v);       // row_mirror
  v = n >= 16 ? v + d : v;
  if (n >= 32) {
    v += __shfl_xor(v, 16);
    if (n >= 64) v += __shfl_xor(v, 32);
  }
  return v;
}

// A lane that owns whole heads (head_size <= VEC, one lane per head group)
// holds a weight / dweight row piece of NP 16-byte units.  With NP > 1,
// instruction i of a per-lane access would touch every lane's i-th unit, 64
// partial cache lines.  In whole wavefronts (nvc % 64 == 0) these pieces move
// through LDS instead: the wavefront loads / stores its NP KiB of the row
// as NP contiguous 1 KiB instructions (slot i*64 + l), and lane l's piece j is
// slot l*NP + j.  Weight loads then take the nontemporal policy (head size 1,
// B4 T4096 D2048 W4 bf16: forward 72.6 -> 72.0 us, backward 146.8 -> 143.7 us);
// dweight stores would otherwise write each line in several partial pieces.
template <typename T, int W, int HSV> struct TdwOf {
  static constexpr int BYTES = (VecOf<T>::value / HSV) * W * (int)sizeof(T);
  static constexpr bool value = BYTES % 16 == 0 && BYTES > 16;
  static constexpr int NP = BYTES / 16;  // pieces per lane
};

// Exchanges between the lanes of one wavefront through its own LDS slots.  The
// hardware runs a wavefront's LDS instructions in order, so no s_barrier is
// needed, but the compiler sees only this lane's addresses: it may move a
// later write above an earlier read that this lane provably does not alias
// (another lane's does).  __builtin_amdgcn_wave_barrier() keeps the phases in
// program order.
//
// Slots of the wavefront's contiguous 1 KiB loads -> the lane's own NP units.
template <int NP>
__device__ __forceinline__ void own_pieces(u32x4* my, const u32x4 (&in)[NP], u32x4 (&out)[NP], int lane) {
  __builtin_amdgcn_wave_barrier();  // the previous exchange's reads are done
#pragma unroll
  for (int i = 0; i < NP; ++i) my[i * 64 + lane] = in[i];
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int j = 0; j < NP; ++j) out[j] = my[lane * NP + j];
}

// ------------------------------------------------------------------ forward
template <typename T, int W, int HSV, bool TWL>
__global__ __launch_bounds__(256) void hw_fwd_fast(const T* __restrict__ x, const T* __restrict__ wt,
                                                   const T* __restrict__ sw, T* __restrict__ y, HwArgs a) {
  constexpr int VEC = VecOf<T>::value;
  constexpr int NWE = (VEC / HSV) * W;
  constexpr int U = Unroll<W>::value;
  constexpr int ES = (int)sizeof(T);
  typedef Raw<T, VEC> XR;
  typedef Raw<T, NWE> WR;
  // per-lane weight loads: nontemporal when a lane's piece is one unit of whole
  // heads, so an instruction reads the lanes' pieces as one contiguous run
  // (head size 4: forward 39.1 -> 37.5 us); several units per lane take the
  // transposed loads below in whole wavefronts, and heads over several lanes
  // (a shared piece per head) measured faster with the default policy
  constexpr int WPOL = (HSV < VEC && WR::NU == 1) ? kNt : 0;
  const int lb = xcd_remap(blockIdx.x, a.nblk);
  const int vg = lb % a.nvg, sgp = lb / a.nvg;
  const int wave = wave_id(), lane = threadIdx.x & 63;
  const int vc = vg * 64 + lane;
  const int s = sgp * 4 + wave;
  if (s >= a.nseg) return;
  const HwRun run(a, s, W, ES);
  const int t0 = run.t0, t1 = run.t1;
  const bool lv = vc < a.nvc;
  const int d0 = vc * VEC;
  const int xlo = lv ? d0 * ES : kHwLaneOob;
  const int wlo = lv ? (d0 >> a.hs_shift) * W * ES : kHwLaneOob;
  const rsrc_t rx = make_rsrc(x + run.xrow0, run.xrec);
  const rsrc_t ry = make_rsrc(y + run.xrow0, run.xrec);
  const rsrc_t rw = make_rsrc(wt + run.wrow0, run.wrec);
  const int64_t D = a.D;
  // TWL: transposed weight loads (TdwOf; the host takes them only in whole
  // wavefronts whose lanes own whole heads)
  constexpr int NPW = TWL ? TdwOf<T, W, HSV>::NP : 1;
  __shared__ u32x4 wlt[4][TWL ? NPW * 64 : 1];
  const int wlo0 = (((vc - lane) * VEC) >> a.hs_shift) * W * ES;  // weight byte offset of the wavefront's lane 0

  XR swr[W];
#pragma unroll
  for (int k = 0; k < W; ++k) {
    if (a.has_static && lv)
      swr[k].load(sw + (int64_t)k * D + d0);
    else
      swr[k].zero();
  }
  // x ring (fp32, each row converted once): row t lives in slot (t - t0) mod W;
  // rows before 0 read 0.
  float xf[W][VEC];
  zero_vals<VEC>(xf[0]);
#pragma unroll
  for (int i = 1; i < W; ++i) {
    XR h;
    bload_raw<kNt>(h, rx, xlo + run.xrow(t0 - i));
    h.to_float(xf[W - i]);
  }

  auto load_chunk = [&](int tc, XR(&xc)[U], WR(&wc)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = tc + u;
      bload_raw<kNt>(xc[u], rx, xlo + run.xrow(t, t < t1));
      if constexpr (TWL) {
#pragma unroll
        for (int i = 0; i < NPW; ++i) wc[u].u[i] = bload128<kNt>(rw, wlo0 + run.wrow(t, t < t1) + (i * 64 + lane) * 16);
      } else {
        bload_raw<WPOL>(wc[u], rw, wlo + run.wrow(t, t < t1));
      }
    }
  };
  auto compute_chunk = [&](int tc, const XR(&xc)[U], const WR(&wc)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = tc + u;
      const int p = u % W;
      xc[u].to_float(xf[p]);
      WR wr;
      if constexpr (TWL)
        own_pieces<NPW>(wlt[wave], wc[u].u, wr.u, lane);
      else
        wr = wc[u];
      float acc[VEC];
      zero_vals<VEC>(acc);
#pragma unroll
      for (int k = 0; k < W; ++k) {
        const int q = ring<W>(u, k);
#pragma unroll
        for (int j = 0; j < VEC; ++j) acc[j] = fmaf(wr.get((j / HSV) * W + k) + swr[k].get(j), xf[q][j], acc[j]);
      }
      if (a.residual) {
#pragma unroll
        for (int j = 0; j < VEC; ++j) acc[j] += xf[p][j];
      }
      bstore_vals<T, VEC, true>(ry, xlo + run.xrow(t, t < t1), acc);  // rows past the run: dropped
    }
  };

  if constexpr (HSV == 1) {
    // Head size 1: a second chunk in flight (W weights per channel) would cost
    // the third wavefront per SIMD; one chunk each, three wavefronts, hides
    // the loads better (hs1 forward 77 -> 76 us).
    for (int tc = t0; tc < t1; tc += U) {
      XR xa[U];
      WR wa[U];
      load_chunk(tc, xa, wa);
      compute_chunk(tc, xa, wa);
    }
    return;
  }
  XR xa[U], xb[U];
  WR wa[U], wb[U];
  load_chunk(t0, xa, wa);
  for (int tc = t0; tc < t1; tc += 2 * U) {
    load_chunk(tc + U, xb, wb);
    __builtin_amdgcn_sched_barrier(0);  // the next chunk's loads go out before this chunk's waits
    compute_chunk(tc, xa, wa);
    load_chunk(tc + 2 * U, xa, wa);
    __builtin_amdgcn_sched_barrier(0);
    if (tc + U < t1) compute_chunk(tc + U, xb, wb);
  }
}

// ----------------------------------------------------------------- backward

// LPH: lanes per head when known at compile time (1, 2, 4, 8), or 0 for the
// run-time group size a.lph (head sizes of 16 lanes and more).
template <typename T, int W, int HSV, bool HAS_STATIC, bool TDW, int LPH>
__global__ __launch_bounds__(256) void hw_bwd_fast(const T* __restrict__ x, const T* __restrict__ wt,
                                                   const T* __restrict__ sw, const T* __restrict__ dy,
                                                   T* __restrict__ dx, T* __restrict__ dwt_,
                                                   float* __restrict__ part, HwArgs a) {
  constexpr int VEC = VecOf<T>::value;
  constexpr int NHL = VEC / HSV;
  constexpr int NWE = NHL * W;
  constexpr int U = Unroll<W>::value;
  constexpr int ES = (int)sizeof(T);
  // 16-bit types with heads of 2+ channels in a lane: dweight's head sums by
  // dot2 on packed pairs; the fp32 x ring then only serves dstatic_w.
  constexpr bool DOT = ES == 2 && HSV >= 2;
  constexpr bool XF = !DOT || HAS_STATIC;
  constexpr int NPW = VEC * ES / 4;  // 32-bit words of a lane's row piece
  typedef Raw<T, VEC> XR;
  typedef Raw<T, NWE> WR;
  // per-lane weight loads: nontemporal when a lane's piece is one unit of whole
  // heads, so an instruction reads the lanes' pieces as one contiguous run
  // (head size 4: forward 39.1 -> 37.5 us); several units per lane take the
  // transposed loads below in whole wavefronts, and heads over several lanes
  // (a shared piece per head) measured faster with the default policy
  constexpr int WPOL = (HSV < VEC && WR::NU == 1) ? kNt : 0;
  const int lb = xcd_remap(blockIdx.x, a.nblk);
  const int vg = lb % a.nvg, sgp = lb / a.nvg;
  const int wave = wave_id(), lane = threadIdx.x & 63;
  const int vc = vg * 64 + lane;
  const int s = sgp * 4 + wave;
  // TDW: the host guarantees nvc % 64 == 0, so every lane is inside D.
  constexpr int NP = TDW ? TdwOf<T, W, HSV>::NP : 1;
  __shared__ u32x4 dwt[4][TDW ? NP * 64 : 1];  // dweight stores
  __shared__ u32x4 wlt[4][TDW ? NP * 64 : 1];  // weight loads

  float dsw[W][VEC];
#pragma unroll
  for (int k = 0; k < W; ++k) zero_vals<VEC>(dsw[k]);

  // Lanes of a head are aligned groups of `lph` consecutive columns and D is a
  // whole number of heads, so lanes past D form whole groups of their own.
  if (s < a.nseg) {
    const HwRun run(a, s, W, ES);
    const int t0 = run.t0, t1 = run.t1;
    const int tend = t1 + W - 1;  // steps t0 .. tend-1: dx of row t needs dy, w of rows t .. t+W-1
    const bool lv = vc < a.nvc;
    const int d0 = vc * VEC;
    const int xlo = lv ? d0 * ES : kHwLaneOob;
    const int wlo = lv ? (d0 >> a.hs_shift) * W * ES : kHwLaneOob;
    const int lph = LPH > 0 ? LPH : a.lph;
    const bool leader = (vc & (lph - 1)) == 0;
    const int dwlo = leader ? wlo : kHwLaneOob;  // one lane of a head stores its dweight
    // weight / dweight byte offset of the wavefront's lane 0 (TDW: lanes own consecutive heads)
    const int wlo0 = (((vc - lane) * VEC) >> a.hs_shift) * W * ES;
    const rsrc_t rx = make_rsrc(x + run.xrow0, run.xrec);
    const rsrc_t rdy = make_rsrc(dy + run.xrow0, run.xrec);
    const rsrc_t rdx = make_rsrc(dx + run.xrow0, run.xrec);
    const rsrc_t rw = make_rsrc(wt + run.wrow0, run.wrec);
    const rsrc_t rdw = make_rsrc(dwt_ + run.wrow0, run.wrec);
    const int residual = a.residual;
    const int64_t D = a.D;

    XR swr[W];
#pragma unroll
    for (int k = 0; k < W; ++k) {
      if (HAS_STATIC && lv)
        swr[k].load(sw + (int64_t)k * D + d0);
      else
        swr[k].zero();
    }
    // x rings, row t in slot (t - t0) mod W: fp32 (each row converted once)
    // for the per-channel products, packed 16-bit pairs for the head sums.
    float xf[XF ? W : 1][VEC];
    uint32_t xw[DOT ? W : 1][NPW];
    float dxa[W][VEC];
#pragma unroll
    for (int k = 0; k < W; ++k) zero_vals<VEC>(dxa[k]);
    if constexpr (XF) zero_vals<VEC>(xf[0]);
    if constexpr (DOT) __builtin_memset(xw[0], 0, sizeof(xw[0]));
#pragma unroll
    for (int i = 1; i < W; ++i) {
      XR h;
      bload_raw<kNt>(h, rx, xlo + run.xrow(t0 - i));
      if constexpr (XF) h.to_float(xf[W - i]);
      if constexpr (DOT) __builtin_memcpy(xw[W - i], h.u, sizeof(xw[0]));
    }

    struct Chunk {
      XR dy[U], x[U];
      WR w[U];
    };
    auto load_chunk = [&](int tc, Chunk& c) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int t = tc + u;
        bload_raw<kNt>(c.dy[u], rdy, xlo + run.xrow(t, t < tend));  // rows past T read 0
        if constexpr (TDW) {
#pragma unroll
          for (int i = 0; i < NP; ++i) c.w[u].u[i] = bload128<kNt>(rw, wlo0 + run.wrow(t, t < tend) + (i * 64 + lane) * 16);
        } else {
          bload_raw<WPOL>(c.w[u], rw, wlo + run.wrow(t, t < tend));
        }
        bload_raw<kNt>(c.x[u], rx, xlo + run.xrow(t, t < t1));
      }
    };
    auto compute_chunk = [&](int tc, const Chunk& c) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int t = tc + u;
        const int p = u % W;
        float dyv[VEC];
        c.dy[u].to_float(dyv);
        WR wr;
        if constexpr (TDW)
          own_pieces<NP>(wlt[wave], c.w[u].u, wr.u, lane);
        else
          wr = c.w[u];
        // dx[t-k] += dy[t] * (w[t, h, k] + sw[k]); row t opens with its k = 0 term.
        // Steps past tend read dy = w = 0 and add nothing.
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
          const float v = dyv[j] * (wr.get((j / HSV) * W) + swr[0].get(j));
          dxa[p][j] = residual ? v + dyv[j] : v;
        }
#pragma unroll
        for (int k = 1; k < W; ++k) {
          const int q = ring<W>(u, k);
#pragma unroll
          for (int j = 0; j < VEC; ++j)
            dxa[q][j] = fmaf(dyv[j], wr.get((j / HSV) * W + k) + swr[k].get(j), dxa[q][j]);
        }
        if (t < t1) {  // wave-uniform; no loads below
          if constexpr (XF) c.x[u].to_float(xf[p]);
          float dwv[NWE];
          if constexpr (DOT) {
            // dstatic_w per channel (fused products); dweight's head sums from
            // the packed pairs of dy and x, HSV / 2 dot2 steps per head and tap.
            __builtin_memcpy(xw[p], c.x[u].u, sizeof(xw[0]));
            uint32_t dyw[NPW];
            __builtin_memcpy(dyw, c.dy[u].u, sizeof(dyw));
#pragma unroll
            for (int k = 0; k < W; ++k) {
              const int q = ring<W>(u, k);
              if (HAS_STATIC) {
#pragma unroll
                for (int j = 0; j < VEC; ++j) dsw[k][j] = fmaf(dyv[j], xf[q][j], dsw[k][j]);
              }
#pragma unroll
              for (int hh = 0; hh < NHL; ++hh) {
                float sacc = 0.f;
#pragma unroll
                for (int j = 0; j < HSV / 2; ++j) sacc = Dot2<T>::run(dyw[hh * HSV / 2 + j], xw[q][hh * HSV / 2 + j], sacc);
                dwv[hh * W + k] = sacc;
              }
            }
          } else {
#pragma unroll
            for (int k = 0; k < W; ++k) {
              const int q = ring<W>(u, k);
              float pr[VEC];
#pragma unroll
              for (int j = 0; j < VEC; ++j) pr[j] = dyv[j] * xf[q][j];
              if (HAS_STATIC) {
#pragma unroll
                for (int j = 0; j < VEC; ++j) dsw[k][j] += pr[j];
              }
#pragma unroll
              for (int hh = 0; hh < NHL; ++hh) {
                float sacc = 0.f;
#pragma unroll
                for (int j = 0; j < HSV; ++j) sacc += pr[hh * HSV + j];
                dwv[hh * W + k] = sacc;
              }
            }
          }
          if constexpr (LPH == 0) {
#pragma unroll
            for (int k = 0; k < NWE; ++k) dwv[k] = group_sum_sel(dwv[k], lph);
          } else if constexpr (LPH > 1) {
#pragma unroll
            for (int k = 0; k < NWE; ++k) dwv[k] = group_sum<LPH>(dwv[k]);
          }
          if constexpr (TDW) {
            // Lane l's piece j goes to slot l*NP + j; slot i*64 + l is then
            // the wavefront's i-th contiguous 1 KiB (an exchange within the
            // wavefront, as own_pieces).
            T e[NWE];
#pragma unroll
            for (int i = 0; i < NWE; ++i) e[i] = (T)dwv[i];
            u32x4 pc[NP];
            __builtin_memcpy(pc, e, sizeof(pc));
            u32x4* my = dwt[wave];
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int j = 0; j < NP; ++j) my[lane * NP + j] = pc[j];
            __builtin_amdgcn_wave_barrier();
            const int o = wlo0 + run.wrow(t);
#pragma unroll
            for (int i = 0; i < NP; ++i) bstore128<true>(my[i * 64 + lane], rdw, o + (i * 64 + lane) * 16);
          } else {
            bstore_vals<T, NWE>(rdw, dwlo + run.wrow(t), dwv);
          }
        }
        const int tdone = t - (W - 1);
        bstore_vals<T, VEC, true>(rdx, xlo + run.xrow(tdone, tdone >= t0 && tdone < t1), dxa[(u + 1) % W]);
      }
    };

    if constexpr (HSV == 1) {
      // Head size 1 carries W weights per channel: one chunk in flight per
      // wavefront.  The launch has one wavefront per SIMD either way; the two
      // alternating chunk buffers of larger heads take 256 VGPRs + 128 AGPRs
      // here and measured slower (B4 T4096 D2048 W4 bf16 backward, static and
      // residual: 143 -> 149.5 us; without both: 137.6 -> 142.2 us).
      for (int tc = t0; tc < tend; tc += U) {
        Chunk c;
        load_chunk(tc, c);
        compute_chunk(tc, c);
      }
    } else {
      Chunk ca, cb;
      load_chunk(t0, ca);
      for (int tc = t0; tc < tend; tc += 2 * U) {
        load_chunk(tc + U, cb);
        __builtin_amdgcn_sched_barrier(0);  // the next chunk's loads go out before this chunk's waits
        compute_chunk(tc, ca);
        load_chunk(tc + 2 * U, ca);
        __builtin_amdgcn_sched_barrier(0);
        if (tc + U < tend) compute_chunk(tc + U, cb);
      }
    }
  }

  if (HAS_STATIC) {
    // Workgroup sum of the 4 wavefronts' dstatic partials, in wave order.
    constexpr int COLS = 64 * VEC;
    __shared__ float red[4][W][COLS];
#pragma unroll
    for (int k = 0; k < W; ++k)
#pragma unroll
      for (int j = 0; j < VEC; ++j) red[wave][k][lane * VEC + j] = dsw[k][j];
    __syncthreads();
    const int64_t D = a.D;
    for (int e = threadIdx.x; e < W * COLS; e += 256) {
      const int k = e / COLS, c = e - k * COLS;
      const int64_t d = (int64_t)vg * COLS + c;
      if (d < D) {
        const float v = ((red[0][k][c] + red[1][k][c]) + red[2][k][c]) + red[3][k][c];
        part[((int64_t)sgp * W + k) * D + d] = v;
      }
    }
  }
}

// Launch geometry shared by the host planner and the dispatchers.
struct HwPlan {
  HwArgs a;
  int nblk;
  int P;     // partial count (bwd)
  bool tdw;  // whole wavefronts (nvc % 64 == 0): transposed dweight stores allowed
};

template <typename T, int W, int HSV>
hipError_t launch_fwd_fast(const HwProblem& p, const HwPlan& pl) {
  if constexpr (TdwOf<T, W, HSV>::value) {
    // lanes that own whole heads (one or more), in whole wavefronts
    if (pl.tdw && pl.a.lph == 1) {
      hw_fwd_fast<T, W, HSV, true><<<pl.nblk, 256, 0, p.stream>>>((const T*)p.x, (const T*)p.weight,
                                                                  (const T*)p.static_w, (T*)p.y, pl.a);
      return hipGetLastError();
    }
  }
  hw_fwd_fast<T, W, HSV, false><<<pl.nblk, 256, 0, p.stream>>>((const T*)p.x, (const T*)p.weight,
                                                               (const T*)p.static_w, (T*)p.y, pl.a);
  return hipGetLastError();
}

template <typename T, int W, int HSV, bool TDW, int LPH>
void launch_bwd_kernel(const HwProblem& p, const HwPlan& pl) {
  if (p.static_w) {
    hw_bwd_fast<T, W, HSV, true, TDW, LPH><<<pl.nblk, 256, 0, p.stream>>>(
        (const T*)p.x, (const T*)p.weight, (const T*)p.static_w, (const T*)p.dy, (T*)p.dx, (T*)p.dweight, p.ws,
        pl.a);
  } else {
    hw_bwd_fast<T, W, HSV, false, TDW, LPH><<<pl.nblk, 256, 0, p.stream>>>(
        (const T*)p.x, (const T*)p.weight, nullptr, (const T*)p.dy, (T*)p.dx, (T*)p.dweight, nullptr, pl.a);
  }
}

template <typename T, int W, int HSV>
hipError_t launch_bwd_fast(const HwProblem& p, const HwPlan& pl) {
  bool launched = false;
  if constexpr (TdwOf<T, W, HSV>::value) {
    // The transposed dweight store needs lanes that own whole heads (one lane
    // per head or several heads per lane); heads over several lanes sum across
    // them first (below).
    if (pl.a.lph == 1) {
      if (pl.tdw)
        launch_bwd_kernel<T, W, HSV, true, 1>(p, pl);
      else
        launch_bwd_kernel<T, W, HSV, false, 1>(p, pl);
      launched = true;
    }
  }
  if (!launched) {
    if constexpr (HSV == VecOf<T>::value) {
      // head_size >= VEC: lanes per head from the plan
      switch (pl.a.lph) {
        case 1: launch_bwd_kernel<T, W, HSV, false, 1>(p, pl); break;
        case 2: launch_bwd_kernel<T, W, HSV, false, 2>(p, pl); break;
        case 4: launch_bwd_kernel<T, W, HSV, false, 4>(p, pl); break;
        case 8: launch_bwd_kernel<T, W, HSV, false, 8>(p, pl); break;
        default: launch_bwd_kernel<T, W, HSV, false, 0>(p, pl); break;
      }
    } else {
      launch_bwd_kernel<T, W, HSV, false, 1>(p, pl);
    }
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !p.static_w) return e;
  return reduce_partials(p.ws, p.W * p.D, pl.P, p.W * p.D, p.dstatic_w, p.dtype, p.stream);
}

// Dispatch on (W, HSV) for one element type.
template <typename T, bool BWD>
hipError_t dispatch_fast(const HwProblem& p, const HwPlan& pl) {
  constexpr int VEC = 16 / (int)sizeof(T);
  const int64_t hs = p.D / p.H;
  const int hsv = (int)(hs < VEC ? hs : VEC);
#define DC_HW_CASE(WW, HH)                                                                  \
  if (p.W == WW && hsv == HH) {                                                             \
    if constexpr (BWD) return launch_bwd_fast<T, WW, HH>(p, pl);                         \
    else return launch_fwd_fast<T, WW, HH>(p, pl);                                          \
  }
#define DC_HW_W(WW)                        \
  DC_HW_CASE(WW, 1)                        \
  DC_HW_CASE(WW, 2)                        \
  DC_HW_CASE(WW, 4)                        \
  if constexpr (VEC == 8) { DC_HW_CASE(WW, 8) }
  DC_HW_W(1)
  DC_HW_W(2)
  DC_HW_W(3)
  DC_HW_W(4)
  DC_HW_W(5)
  DC_HW_W(6)
  DC_HW_W(7)
  DC_HW_W(8)
#undef DC_HW_W
#undef DC_HW_CASE
  return hipErrorInvalidValue;
}

}  // namespace dc
