// Headwise dynamic convolution for 9 <= W <= 32 (the vectorised kernels of
// headwise_fast.h stop at W 8: their register rings grow with W x chunk rows).
//
//   y[b,t,d] = sum_{k<W} (w[b,t,d/hs,k] + sw[k,d]) * x[b,t-k,d]  (+ x[b,t,d])
//
// Reference kernels: headwise.py:24-91 (forward) and headwise.py:105-215
// (backward); any W (headwise.py:226).
//
// Layout.  A lane owns CPL channels (2 up to W 16, 1 above), a wavefront
// 64 * CPL consecutive channels (D a multiple of that), and walks a run of
// rows of one sequence one row at a time, keeping the last W rows of x (and in
// the backward the W open dx accumulators) in fp32 register rings whose slot
// for row t is (t - t0) mod M.  The rows of the next NB steps are in flight
// while a row is computed (NB raw buffers, the loads of row t+NB issued once
// row t's raw values are consumed): NB = 2 where a lane's weight piece is large
// (two heads per lane, or one channel per lane), 4 otherwise, whose rows are
// mostly x (and dy).  The rings have M slots,
// W rounded up to a multiple of NB, and rows are processed in unrolled blocks
// of M rows, so every ring and buffer index is a compile-time constant.
//
// Weight rows.  A wavefront's channels cover 64 * CPL / hs heads, whose
// weights are one contiguous segment of (64 * CPL / hs) * W elements of the row
// (16-byte multiple, checked on the host).  The wavefront loads it with
// 16-byte lane pieces that are contiguous across the wavefront, passes it
// through its own LDS slot, and each lane reads its head's W weights (head
// size 1: the two heads of its channels).  The backward's dweight row goes the
// same way in reverse: the lanes' channel sums are added over the head's lanes
// (DPP butterflies, ds_bpermute steps beyond 16 lanes; above W 16 over a
// run-time group size), written to the slot, and stored as contiguous 16-byte
// pieces.
//
// Backward.  dx in scatter form: row s adds dy[s] * (w[s,k] + sw[k] (+1 at
// k = 0: the residual)) to the open accumulator of row s-k; row s-W+1 is then
// complete and stored.  A run reads dy and w for W-1 rows past its end (their
// dx terms), which add nothing to dweight (stores dropped) or dstatic_w (dy
// masked).  dstatic_w partial sums stay in the wavefront's LDS slot (in
// registers at head size 1 up to W 12) over the run, are added across the
// workgroup's 4 wavefronts in LDS in a fixed order and written as one fp32
// partial per workgroup, summed by reduce_partials (deterministic).
#pragma once

#include "headwise_fast.h"

namespace dc {

constexpr int kHwWideMinW = 9, kHwWideMaxW = 32;
// Channels per lane: 2 up to W 16, 1 above (the x and dx rings hold W rows of
// a lane's channels); a wavefront covers 64 * CPL channels.
constexpr int kWideCplMaxW = 16;
constexpr int wide_cpl(int W) { return W <= kWideCplMaxW ? 2 : 1; }

// Row buffers in flight per wavefront: 2 where a lane's weight piece of a row
// is large (two heads per lane, or one channel per lane up to 64 heads of W
// taps per wavefront), else 4.  h1: two heads per lane (CPL 2, head size 1).
constexpr int wide_nb(bool h1, int cpl) { return h1 || cpl == 1 ? 2 : 4; }

struct HwWideArgs {
  int Tn;        // sequence length
  int D;         // channels (a multiple of 64 * CPL)
  int H;         // heads
  int hs_shift;  // log2(head size), 0 .. 7
  int lph;       // lanes per head (head size / CPL, at least 1): the one-channel kernels' head sums
  int nwc;       // D / (64 * CPL) wavefront columns
  int seg;       // rows per run (a multiple of the kernel's row block)
  int nspb;      // runs per sequence
  int nseg;      // B * nspb
  int nblk;      // grid size
  int sbytes;    // bytes of a wavefront's weight-row segment (a 16-byte multiple)
  int residual;
};

// 16-byte pieces per lane of a wavefront's weight-row segment, at most: 128
// heads with two heads per lane, else at most 64.
template <typename T, int W, bool H1>
struct WideSeg {
  static constexpr int BYTES = (H1 ? 128 : 64) * W * (int)sizeof(T);
  static constexpr int NP = (BYTES + 1023) / 1024;
};

// Rows [t0, t1) of sequence b.
struct WideRun {
  int b, t0, t1;
  __device__ __forceinline__ WideRun(const HwWideArgs& a, int s) {
    b = s / a.nspb;
    t0 = (s - b * a.nspb) * a.seg;
    t1 = min(t0 + a.seg, a.Tn);
  }
};

// A buffer resource over row t of a sequence whose rows of rowb bytes start at
// p0, or an empty one (every access out of range) when !live.  Built per row
// in scalar registers: the lanes' offsets within a row stay the same for every
// row, so the unrolled row blocks hold no per-row offsets in vector registers.
template <typename P>
__device__ __forceinline__ rsrc_t row_rsrc(P* p0, int64_t row_elems, int t, bool live, int rowb) {
  return make_rsrc_wave(p0 + (live ? (int64_t)t * row_elems : 0), live ? rowb : 0);
}

// N consecutive elements of T from LDS, starting at element e0, as floats.
// EVEN: e0 and N are even (32-bit reads of 16-bit pairs).
template <typename T, int N, bool EVEN>
__device__ __forceinline__ void lds_elems(const uint8_t* seg, int e0, float (&out)[N]) {
  if constexpr (sizeof(T) == 4) {
    const float* p = reinterpret_cast<const float*>(seg) + e0;
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = p[i];
  } else if constexpr (EVEN) {
    const uint32_t* p = reinterpret_cast<const uint32_t*>(seg + e0 * 2);
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
      const uint32_t v = p[i];
      T e[2];
      __builtin_memcpy(e, &v, 4);
      out[2 * i] = (float)e[0];
      out[2 * i + 1] = (float)e[1];
    }
  } else {
    const uint16_t* p = reinterpret_cast<const uint16_t*>(seg) + e0;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const uint16_t v = p[i];
      T e;
      __builtin_memcpy(&e, &v, 2);
      out[i] = (float)e;
    }
  }
}

// A lane's CPL products dy * x added in channel order (its share of a head sum).
template <int CPL>
__device__ __forceinline__ float lane_sum(const float (&dy)[CPL], const float (&x)[CPL]) {
  float s = dy[0] * x[0];
#pragma unroll
  for (int j = 1; j < CPL; ++j) s = fmaf(dy[j], x[j], s);
  return s;
}

// ------------------------------------------------------------------ forward
template <typename T, int W, int CPL, bool H1, bool STATIC>
__global__ __launch_bounds__(256) void hw_fwd_wide(const T* __restrict__ x, const T* __restrict__ wt,
                                                   const T* __restrict__ sw, T* __restrict__ y, HwWideArgs a) {
  static_assert(CPL == 2 || !H1, "two heads per lane: two channels per lane");
  constexpr int ES = (int)sizeof(T);
  constexpr int COLS = 64 * CPL;  // channels per wavefront
  constexpr int NH = H1 ? 2 : 1;  // heads per lane
  constexpr int NB = wide_nb(H1, CPL), M = (W + NB - 1) / NB * NB;
  constexpr int NP = WideSeg<T, W, H1>::NP;
  constexpr bool EVEN = H1 || W % 2 == 0;
  typedef Raw<T, CPL> XR;
  __shared__ __attribute__((aligned(16))) uint8_t stg[4][NP * 1024];

  const int lb = xcd_remap(blockIdx.x, a.nblk);
  const int wc = lb % a.nwc, sgp = lb / a.nwc;
  const int wave = wave_id(), lane = threadIdx.x & 63;
  const int s = sgp * 4 + wave;
  if (s >= a.nseg) return;
  const WideRun run(a, s);
  const int t0 = run.t0, t1 = run.t1;
  const int D = a.D;
  const int c0 = wc * COLS + CPL * lane;  // the lane's first channel
  const int rowb = D * ES, wrowb = a.H * W * ES;
  const int64_t WH = (int64_t)a.H * W;
  const T* const xs = x + (int64_t)run.b * a.Tn * D;  // the sequence's first rows
  T* const ys = y + (int64_t)run.b * a.Tn * D;
  const T* const ws = wt + (int64_t)run.b * a.Tn * WH;
  const int xlo = c0 * ES;
  const int wseg = ((wc * COLS) >> a.hs_shift) * W * ES;  // the wavefront's segment in a weight row
  int wpo[NP];  // the lane's 16-byte pieces of the segment (past it: out of range)
#pragma unroll
  for (int i = 0; i < NP; ++i) wpo[i] = (i * 64 + lane) * 16 < a.sbytes ? wseg + (i * 64 + lane) * 16 : kHwLaneOob;
  // the lane's weights in the segment: element offset of its (first) head
  const int we0 = H1 ? 2 * lane * W : ((CPL * lane) >> a.hs_shift) * W;
  uint8_t* const my = stg[wave];

  float swf[W][CPL];
#pragma unroll
  for (int k = 0; k < W; ++k) {
    if constexpr (STATIC) {
      float v[CPL];
      load_vals<T, CPL>(sw + (int64_t)k * D + c0, v);
#pragma unroll
      for (int j = 0; j < CPL; ++j) swf[k][j] = v[j];
    }
  }
  // x ring: row t in slot (t - t0) mod W; rows before 0 read 0 (negative offsets are out of range)
  float xf[M][CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) xf[0][j] = 0.f;
#pragma unroll
  for (int i = 1; i < W; ++i) {
    XR h;
    bload_raw(h, row_rsrc(xs, D, t0 - i, t0 - i >= 0, rowb), xlo);
    h.to_float(xf[M - i]);
  }

  XR xr[NB];
  u32x4 wr[NB][NP];
  auto load_row = [&](int t, int buf) {
    const bool live = t < t1;
    bload_raw<kNt>(xr[buf], row_rsrc(xs, D, t, live, rowb), xlo);
    const rsrc_t rw = row_rsrc(ws, WH, t, live, wrowb);
#pragma unroll
    for (int i = 0; i < NP; ++i) wr[buf][i] = bload128<kNt>(rw, wpo[i]);
  };
#pragma unroll
  for (int i = 0; i < NB; ++i) load_row(t0 + i, i);
  for (int tb = t0; tb < t1; tb += M) {
#pragma unroll
    for (int u = 0; u < M; ++u) {
      const int t = tb + u;
      const int p = u % M, buf = u % NB;
      xr[buf].to_float(xf[p]);
      __builtin_amdgcn_wave_barrier();  // the previous row's reads of the slot are done
#pragma unroll
      for (int i = 0; i < NP; ++i) reinterpret_cast<u32x4*>(my)[i * 64 + lane] = wr[buf][i];
      load_row(t + NB, buf);
      __builtin_amdgcn_wave_barrier();
      float wv[NH * W];
      lds_elems<T, NH * W, EVEN>(my, we0, wv);
      float acc[CPL];
#pragma unroll
      for (int j = 0; j < CPL; ++j) acc[j] = a.residual ? xf[p][j] : 0.f;
#pragma unroll
      for (int k = 0; k < W; ++k) {
        const int q = ((u - k) % M + M) % M;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
          float tap = wv[(H1 ? j : 0) * W + k];
          if constexpr (STATIC) tap += swf[k][j];
          acc[j] = fmaf(tap, xf[q][j], acc[j]);
        }
      }
      bstore_vals<T, CPL, true>(row_rsrc(ys, D, t, t < t1, rowb), xlo, acc);
    }
  }
}

// ----------------------------------------------------------------- backward
// LPH: lanes per head: 0 at head size 1 with two channels per lane (two
// heads per lane), 1 for a lane's own head, 2..64 a compile-time group, -1 the
// run-time a.lph (the one-channel kernels above W 16).
template <typename T, int W, int CPL, int LPH, bool STATIC>
__global__ __launch_bounds__(256) void hw_bwd_wide(const T* __restrict__ x, const T* __restrict__ wt,
                                                   const T* __restrict__ sw, const T* __restrict__ dy,
                                                   T* __restrict__ dx, T* __restrict__ dwt,
                                                   float* __restrict__ part, HwWideArgs a) {
  constexpr int ES = (int)sizeof(T);
  constexpr bool H1 = LPH == 0;
  static_assert(CPL == 2 || !H1, "two heads per lane: two channels per lane");
  constexpr int COLS = 64 * CPL;  // channels per wavefront
  constexpr int NH = H1 ? 2 : 1;
  // With a static filter the dstatic_w sums go to LDS (registers held the
  // static backward at one wavefront per SIMD: W 12 head size 32 214 -> 163 us,
  // W 16 358 -> 207 us), except at head size 1 up to W 12, where registers are
  // faster (372 against 385 us); above W 12 two row buffers.
  constexpr bool WIDE_ST = STATIC && (W > 12 || !H1);
  constexpr int NB = STATIC && W > 12 ? 2 : wide_nb(H1, CPL), M = (W + NB - 1) / NB * NB;
  constexpr int NP = WideSeg<T, W, H1>::NP;
  constexpr bool EVEN = H1 || W % 2 == 0;
  typedef Raw<T, CPL> XR;
  __shared__ __attribute__((aligned(16))) uint8_t stg[4][NP * 1024];
  __shared__ __attribute__((aligned(8))) float dsr[STATIC ? 4 : 1][STATIC ? W * COLS : 1];

  const int lb = xcd_remap(blockIdx.x, a.nblk);
  const int wc = lb % a.nwc, sgp = lb / a.nwc;
  const int wave = wave_id(), lane = threadIdx.x & 63;
  const int s = sgp * 4 + wave;
  // Wavefronts past the last run take part in the workgroup's dstatic_w sum
  // (barrier) with zeros: their loop runs no row.
  const bool has_run = s < a.nseg;
  const WideRun run(a, has_run ? s : 0);
  const int t0 = run.t0, t1 = has_run ? run.t1 : run.t0;
  const int D = a.D, Tn = a.Tn;
  const int c0 = wc * COLS + CPL * lane;
  const int rowb = D * ES, wrowb = a.H * W * ES;
  const int64_t WH = (int64_t)a.H * W;
  const int64_t so = (int64_t)run.b * Tn;  // the sequence's first row
  const T* const xs = x + so * D;
  const T* const dys = dy + so * D;
  T* const dxs = dx + so * D;
  const T* const ws = wt + so * WH;
  T* const dws = dwt + so * WH;
  const int xlo = c0 * ES;
  const int wseg = ((wc * COLS) >> a.hs_shift) * W * ES;
  int wpo[NP];
#pragma unroll
  for (int i = 0; i < NP; ++i) wpo[i] = (i * 64 + lane) * 16 < a.sbytes ? wseg + (i * 64 + lane) * 16 : kHwLaneOob;
  const int hl = H1 ? 2 * lane : (CPL * lane) >> a.hs_shift;  // the lane's (first) head in the segment
  const int we0 = hl * W;
  uint8_t* const my = stg[wave];
  const float res = a.residual ? 1.f : 0.f;  // tap 0's weight + 1: the residual's dy term
  // dstatic_w sums of the lane's channels over the run: in the wavefront's LDS
  // slot (tap k at dsl[k * COLS]; each lane reads and writes only its own), or in
  // registers (WIDE_ST false)
  float dsw[WIDE_ST ? 1 : W][CPL];
  float* const dsl = dsr[wave] + CPL * lane;
  if constexpr (STATIC) {
#pragma unroll
    for (int k = 0; k < W; ++k)
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        if constexpr (WIDE_ST)
          dsl[k * COLS + j] = 0.f;
        else
          dsw[k][j] = 0.f;
      }
  }
  // the static filter of the lane's channels, in registers for the run (read
  // from LDS per row it took 150 more registers in the unrolled row blocks)
  float swf[STATIC ? W : 1][CPL];
  if constexpr (STATIC) {
#pragma unroll
    for (int k = 0; k < W; ++k) load_vals<T, CPL>(sw + (int64_t)k * D + c0, swf[k]);
  }
  float xf[M][CPL], dxr[M][CPL];
#pragma unroll
  for (int i = 0; i < M; ++i)
#pragma unroll
    for (int j = 0; j < CPL; ++j) dxr[i][j] = 0.f;
#pragma unroll
  for (int j = 0; j < CPL; ++j) xf[0][j] = 0.f;
#pragma unroll
  for (int i = 1; i < W; ++i) {
    XR h;
    bload_raw(h, row_rsrc(xs, D, t0 - i, has_run && t0 - i >= 0, rowb), xlo);
    h.to_float(xf[M - i]);
  }

  // Rows s in [t0, tend): x of rows < t1 (dweight, dstatic_w); dy and w of
  // rows < tend (their dx terms reach rows < t1).
  const int tend = has_run ? t1 + W - 1 : t1;
  XR xr[NB], dr[NB];
  u32x4 wr[NB][NP];
  auto load_row = [&](int t, int buf) {
    bload_raw<kNt>(xr[buf], row_rsrc(xs, D, t, t < t1, rowb), xlo);
    const bool ylive = t < tend && t < Tn;
    bload_raw<kNt>(dr[buf], row_rsrc(dys, D, t, ylive, rowb), xlo);
    const rsrc_t rw = row_rsrc(ws, WH, t, ylive, wrowb);
#pragma unroll
    for (int i = 0; i < NP; ++i) wr[buf][i] = bload128<kNt>(rw, wpo[i]);
  };
#pragma unroll
  for (int i = 0; i < NB; ++i) load_row(t0 + i, i);
  for (int tb = t0; tb < tend; tb += M) {
#pragma unroll
    for (int u = 0; u < M; ++u) {
      const int t = tb + u;
      const int p = u % M, buf = u % NB;
      xr[buf].to_float(xf[p]);
      float dyv[CPL], dym[CPL];
      dr[buf].to_float(dyv);
#pragma unroll
      for (int j = 0; j < CPL; ++j) dym[j] = t < t1 ? dyv[j] : 0.f;  // rows past the run: dx terms only
      __builtin_amdgcn_wave_barrier();  // the previous row's reads of the slot are done
#pragma unroll
      for (int i = 0; i < NP; ++i) reinterpret_cast<u32x4*>(my)[i * 64 + lane] = wr[buf][i];
      load_row(t + NB, buf);
      __builtin_amdgcn_wave_barrier();
      float wv[NH * W];
      lds_elems<T, NH * W, EVEN>(my, we0, wv);

      // dx (scatter form); row t-W+1 is complete afterwards
#pragma unroll
      for (int k = 0; k < W; ++k) {
        const int q = ((u - k) % M + M) % M;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
          float tap = wv[(H1 ? j : 0) * W + k];
          if constexpr (STATIC) tap += swf[k][j];
          if (k == 0) tap += res;
          dxr[q][j] = fmaf(dyv[j], tap, dxr[q][j]);
        }
      }
      {
        const int q = ((u - W + 1) % M + M) % M;  // slot of row t-W+1
        const int td = t - W + 1;
        bstore_vals<T, CPL, true>(row_rsrc(dxs, D, td, td >= t0 && td < t1, rowb), xlo, dxr[q]);
#pragma unroll
        for (int j = 0; j < CPL; ++j) dxr[q][j] = 0.f;
      }

      // dweight row t: products dy[t] * x[t-k] summed over the head's channels
      __builtin_amdgcn_wave_barrier();  // the weight reads of the slot are done
      uint16_t* const my16 = reinterpret_cast<uint16_t*>(my);
      float* const my32 = reinterpret_cast<float*>(my);
      auto put = [&](int e, float v) {  // entry e of the wavefront's dweight segment
        if constexpr (ES == 4) {
          my32[e] = v;
        } else {
          const T tv = (T)v;
          uint16_t bits;
          __builtin_memcpy(&bits, &tv, 2);
          my16[e] = bits;
        }
      };
      if constexpr (H1) {
#pragma unroll
        for (int k = 0; k < W; ++k) {
          const int q = ((u - k) % M + M) % M;
#pragma unroll
          for (int j = 0; j < CPL; ++j) put(we0 + j * W + k, dym[j] * xf[q][j]);
        }
      } else if constexpr (LPH == 1) {  // a head per lane (head size CPL): the lane's head is its own
#pragma unroll
        for (int k = 0; k < W; ++k) {
          const int q = ((u - k) % M + M) % M;
          put(we0 + k, lane_sum(dym, xf[q]));
        }
      } else if constexpr (LPH < 0) {
        // run-time group of a.lph lanes (DPP steps selected by it, no branch);
        // the head's first lane puts the sums
        float v[W];
#pragma unroll
        for (int k = 0; k < W; ++k) {
          const int q = ((u - k) % M + M) % M;
          v[k] = group_sum_sel(lane_sum(dym, xf[q]), a.lph);
        }
        if ((lane & (a.lph - 1)) == 0) {
#pragma unroll
          for (int k = 0; k < W; ++k) put(we0 + k, v[k]);
        }
      } else {
        // head sums over LPH lanes of the lanes' two-channel sums (DPP butterflies, ds_bpermute
        // steps beyond 16 lanes); the head's first lane puts them in the segment
        float v[W];
#pragma unroll
        for (int k = 0; k < W; ++k) {
          const int q = ((u - k) % M + M) % M;
          v[k] = group_sum<LPH>(lane_sum(dym, xf[q]));
        }
        if ((lane & (LPH - 1)) == 0) {
#pragma unroll
          for (int k = 0; k < W; ++k) put(we0 + k, v[k]);
        }
      }
      __builtin_amdgcn_wave_barrier();
      const rsrc_t rdw = row_rsrc(dws, WH, t, t < t1, wrowb);
#pragma unroll
      for (int i = 0; i < NP; ++i) bstore128<true>(reinterpret_cast<const u32x4*>(my)[i * 64 + lane], rdw, wpo[i]);

      if constexpr (STATIC) {
#pragma unroll
        for (int k = 0; k < W; ++k) {
          const int q = ((u - k) % M + M) % M;
#pragma unroll
          for (int j = 0; j < CPL; ++j) {
            if constexpr (WIDE_ST)
              dsl[k * COLS + j] = fmaf(dym[j], xf[q][j], dsl[k * COLS + j]);
            else
              dsw[k][j] = fmaf(dym[j], xf[q][j], dsw[k][j]);
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);  // rows one after another: the rings are the live state
    }
  }

  if constexpr (STATIC) {
    // dstatic_w: the workgroup's 4 runs added in wave order, one fp32 partial
    // per workgroup row: part[sgp][k * D + channel]
    if constexpr (!WIDE_ST) {
#pragma unroll
      for (int k = 0; k < W; ++k)
#pragma unroll
        for (int j = 0; j < CPL; ++j) dsl[k * COLS + j] = dsw[k][j];
    }
    __syncthreads();
    for (int e = threadIdx.x; e < W * COLS; e += 256) {
      const float v = ((dsr[0][e] + dsr[1][e]) + dsr[2][e]) + dsr[3][e];
      const int k = e / COLS, cc = e - k * COLS;
      part[(int64_t)sgp * W * D + (int64_t)k * D + wc * COLS + cc] = v;
    }
  }
}

// ------------------------------------------------------------------ launch
template <typename T, int W, int CPL, bool H1, bool ST>
hipError_t launch_hw_fwd_wide(const HwProblem& p, const HwWideArgs& a) {
  hw_fwd_wide<T, W, CPL, H1, ST><<<a.nblk, 256, 0, p.stream>>>((const T*)p.x, (const T*)p.weight,
                                                               (const T*)p.static_w, (T*)p.y, a);
  return hipGetLastError();
}

template <typename T, int W, int CPL, int LPH, bool ST>
hipError_t launch_hw_bwd_wide(const HwProblem& p, const HwWideArgs& a) {
  hw_bwd_wide<T, W, CPL, LPH, ST><<<a.nblk, 256, 0, p.stream>>>((const T*)p.x, (const T*)p.weight,
                                                                (const T*)p.static_w, (const T*)p.dy, (T*)p.dx,
                                                                (T*)p.dweight, p.ws, a);
  return hipGetLastError();
}

template <typename T, int W, int CPL, int LPH>
hipError_t launch_hw_bwd_wide_s(const HwProblem& p, const HwWideArgs& a) {
  return p.static_w ? launch_hw_bwd_wide<T, W, CPL, LPH, true>(p, a) : launch_hw_bwd_wide<T, W, CPL, LPH, false>(p, a);
}

// Up to W 16: two channels per lane, head sums over compile-time lane groups;
// above: one channel per lane, head sums over the run-time group a.lph.
template <typename T, bool BWD, int W>
hipError_t launch_hw_wide_w(const HwProblem& p, const HwWideArgs& a) {
  const bool st = p.static_w != nullptr;
  if constexpr (W > kWideCplMaxW) {
    if constexpr (!BWD)
      return st ? launch_hw_fwd_wide<T, W, 1, false, true>(p, a) : launch_hw_fwd_wide<T, W, 1, false, false>(p, a);
    else
      return launch_hw_bwd_wide_s<T, W, 1, -1>(p, a);
  } else if constexpr (!BWD) {
    if (a.hs_shift == 0)
      return st ? launch_hw_fwd_wide<T, W, 2, true, true>(p, a) : launch_hw_fwd_wide<T, W, 2, true, false>(p, a);
    return st ? launch_hw_fwd_wide<T, W, 2, false, true>(p, a) : launch_hw_fwd_wide<T, W, 2, false, false>(p, a);
  } else {
    switch (a.hs_shift) {  // lanes per head: head size / 2 (a lane holds two channels)
      case 0: return launch_hw_bwd_wide_s<T, W, 2, 0>(p, a);
      case 1: return launch_hw_bwd_wide_s<T, W, 2, 1>(p, a);
      case 2: return launch_hw_bwd_wide_s<T, W, 2, 2>(p, a);
      case 3: return launch_hw_bwd_wide_s<T, W, 2, 4>(p, a);
      case 4: return launch_hw_bwd_wide_s<T, W, 2, 8>(p, a);
      case 5: return launch_hw_bwd_wide_s<T, W, 2, 16>(p, a);
      case 6: return launch_hw_bwd_wide_s<T, W, 2, 32>(p, a);
      default: return launch_hw_bwd_wide_s<T, W, 2, 64>(p, a);
    }
  }
}

// The wide kernels for p (host checks: hw_wide_ok); the backward's dstatic_w
// partials are summed by the caller.
template <typename T, bool BWD>
hipError_t dispatch_wide(const HwProblem& p, const HwWideArgs& a) {
  switch (p.W) {
#define DC_HW_WIDE(WW) \
  case WW: return launch_hw_wide_w<T, BWD, WW>(p, a);
    DC_HW_WIDE(9) DC_HW_WIDE(10) DC_HW_WIDE(11) DC_HW_WIDE(12) DC_HW_WIDE(13) DC_HW_WIDE(14) DC_HW_WIDE(15)
    DC_HW_WIDE(16) DC_HW_WIDE(17) DC_HW_WIDE(18) DC_HW_WIDE(19) DC_HW_WIDE(20) DC_HW_WIDE(21) DC_HW_WIDE(22)
    DC_HW_WIDE(23) DC_HW_WIDE(24) DC_HW_WIDE(25) DC_HW_WIDE(26) DC_HW_WIDE(27) DC_HW_WIDE(28) DC_HW_WIDE(29)
    DC_HW_WIDE(30) DC_HW_WIDE(31) DC_HW_WIDE(32)
#undef DC_HW_WIDE
    default: return hipErrorInvalidValue;
  }
}

}  // namespace dc
