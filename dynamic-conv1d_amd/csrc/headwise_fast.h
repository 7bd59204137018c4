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
// (t - t0) mod W.  The row loop is unrolled by a multiple of W so every ring
// index is a compile-time constant.  Each row costs exactly one 128-bit load
// of x (and dy), one contiguous load of the lane's NHL*W weights, and one
// 128-bit store: the HBM traffic is the algorithmic traffic plus a W-1 row
// halo per run.  64 lanes of a wavefront cover 64*VEC consecutive channels
// (a 1 KiB contiguous row segment per load instruction); a 256-thread
// workgroup stacks 4 wavefronts on 4 consecutive runs of the same channels,
// so a run's halo rows were just read by the wavefront above it.
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
// pieces that are contiguous across the wavefront (TDW).  dstatic_w partial sums stay in registers
// for the whole run, are added across the 4 wavefronts of the workgroup in
// LDS in a fixed order, and one fp32 partial per workgroup is summed by
// reduce_partials (no atomics: bitwise deterministic).
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

// Rows per unrolled chunk: a multiple of W, at least 4.
template <int W> struct Unroll { static constexpr int value = (W >= 4) ? W : W * (4 / W); };

template <int W>
__device__ __forceinline__ constexpr int ring(int u, int k) {
  return ((u - k) % W + W) % W;
}

// ------------------------------------------------------------------ forward
template <typename T, int W, int HSV>
__global__ __launch_bounds__(256) void hw_fwd_fast(const T* __restrict__ x, const T* __restrict__ wt,
                                                   const T* __restrict__ sw, T* __restrict__ y, HwArgs a) {
  constexpr int VEC = VecOf<T>::value;
  constexpr int NWE = (VEC / HSV) * W;
  constexpr int U = Unroll<W>::value;
  typedef Raw<T, VEC> XR;
  typedef Raw<T, NWE> WR;
  const int lb = xcd_remap(blockIdx.x, a.nblk);
  const int vg = lb % a.nvg, sgp = lb / a.nvg;
  const int wave = wave_id(), lane = threadIdx.x & 63;
  const int vc = vg * 64 + lane;
  const int s = sgp * 4 + wave;
  if (s >= a.nseg || vc >= a.nvc) return;
  const int b = s / a.nspb;
  const int t0 = (s - b * a.nspb) * a.seg;
  const int t1 = min(t0 + a.seg, a.Tn);
  const int d0 = vc * VEC;
  const int h0 = d0 >> a.hs_shift;
  const int64_t row0 = (int64_t)b * a.Tn;
  const int64_t D = a.D;
  const int64_t wrs = (int64_t)a.H * W;
  const T* xp = x + row0 * D + d0;
  const T* wp = wt + (row0 * a.H + h0) * W;
  T* yp = y + row0 * D + d0;

  XR swr[W];
#pragma unroll
  for (int k = 0; k < W; ++k) {
    if (a.has_static)
      swr[k].load(sw + (int64_t)k * D + d0);
    else
      swr[k].zero();
  }
  // x ring: row t lives in slot (t - t0) mod W.
  XR xr[W];
  xr[0].zero();
#pragma unroll
  for (int i = 1; i < W; ++i) {
    const int t = t0 - i;
    if (t >= 0)
      xr[W - i].load(xp + (int64_t)t * D);
    else
      xr[W - i].zero();
  }
  // Rows of the current chunk and, in flight meanwhile, of the next one.
  XR xc[U], xn[U];
  WR wc[U], wn[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int t = t0 + u;
    if (t < t1) {
      xc[u].load(xp + (int64_t)t * D);
      wc[u].load(wp + (int64_t)t * wrs);
    }
  }
  for (int tc = t0; tc < t1; tc += U) {
    if (tc + U < t1) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int t = tc + U + u;
        if (t < t1) {
          xn[u].load(xp + (int64_t)t * D);
          wn[u].load(wp + (int64_t)t * wrs);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = tc + u;
      if (t < t1) {
        const int p = u % W;
        xr[p] = xc[u];
        float acc[VEC];
        zero_vals<VEC>(acc);
#pragma unroll
        for (int k = 0; k < W; ++k) {
          const int q = ring<W>(u, k);
#pragma unroll
          for (int j = 0; j < VEC; ++j)
            acc[j] = fmaf(wc[u].get((j / HSV) * W + k) + swr[k].get(j), xr[q].get(j), acc[j]);
        }
        if (a.residual) {
#pragma unroll
          for (int j = 0; j < VEC; ++j) acc[j] += xr[p].get(j);
        }
        store_vals<T, VEC, true>(yp + (int64_t)t * D, acc);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      xc[u] = xn[u];
      wc[u] = wn[u];
    }
  }
}

// ----------------------------------------------------------------- backward
// Transposed dweight store possible: 16-byte pieces, more than one per lane.
template <typename T, int W, int HSV> struct TdwOf {
  static constexpr int BYTES = (VecOf<T>::value / HSV) * W * (int)sizeof(T);
  static constexpr bool value = BYTES % 16 == 0 && BYTES > 16;
  static constexpr int NP = BYTES / 16;  // pieces per lane
};

template <typename T, int W, int HSV, bool HAS_STATIC, bool TDW>
__global__ __launch_bounds__(256) void hw_bwd_fast(const T* __restrict__ x, const T* __restrict__ wt,
                                                   const T* __restrict__ sw, const T* __restrict__ dy,
                                                   T* __restrict__ dx, T* __restrict__ dwt_,
                                                   float* __restrict__ part, HwArgs a) {
  constexpr int VEC = VecOf<T>::value;
  constexpr int NHL = VEC / HSV;
  constexpr int NWE = NHL * W;
  constexpr int U = Unroll<W>::value;
  typedef Raw<T, VEC> XR;
  typedef Raw<T, NWE> WR;
  const int lb = xcd_remap(blockIdx.x, a.nblk);
  const int vg = lb % a.nvg, sgp = lb / a.nvg;
  const int wave = wave_id(), lane = threadIdx.x & 63;
  const int vc = vg * 64 + lane;
  const int s = sgp * 4 + wave;
  const bool active = (s < a.nseg) && (vc < a.nvc);
  // TDW: the host guarantees nvc % 64 == 0, so `active` is wave-uniform.
  constexpr int NP = TDW ? TdwOf<T, W, HSV>::NP : 1;
  __shared__ u32x4 dwt[4][TDW ? NP * 64 : 1];

  float dsw[W][VEC];
#pragma unroll
  for (int k = 0; k < W; ++k) zero_vals<VEC>(dsw[k]);

  // Lanes of a head are aligned groups of `lph` consecutive columns and a
  // wavefront of one run holds whole heads, so every lane of a group shares
  // `active`; inactive lanes never take part in a shuffle.
  if (active) {
    const int b = s / a.nspb;
    const int t0 = (s - b * a.nspb) * a.seg;
    const int t1 = min(t0 + a.seg, a.Tn);
    const int tend = t1 + W - 1;        // steps t0 .. tend-1: dx of row t needs dy, w of rows t .. t+W-1
    const int tload = min(tend, a.Tn);  // dy / w rows that exist
    const int d0 = vc * VEC;
    const int h0 = d0 >> a.hs_shift;
    const int64_t row0 = (int64_t)b * a.Tn;
    const int64_t D = a.D;
    const int64_t wrs = (int64_t)a.H * W;
    const T* xp = x + row0 * D + d0;
    const T* wp = wt + (row0 * a.H + h0) * W;
    const T* dyp = dy + row0 * D + d0;
    T* dxp = dx + row0 * D + d0;
    T* dwp = dwt_ + (row0 * a.H + h0) * W;
    // dweight row of the wavefront's lane 0 (TDW: lanes own consecutive heads)
    T* dwp0 = dwt_ + (row0 * a.H + (((vc - lane) * VEC) >> a.hs_shift)) * W;
    const bool leader = (vc & (a.lph - 1)) == 0;
    const int residual = a.residual, lph = a.lph;

    XR swr[W];
#pragma unroll
    for (int k = 0; k < W; ++k) {
      if (HAS_STATIC)
        swr[k].load(sw + (int64_t)k * D + d0);
      else
        swr[k].zero();
    }
    XR xr[W];
    float dxa[W][VEC];
#pragma unroll
    for (int k = 0; k < W; ++k) zero_vals<VEC>(dxa[k]);
    xr[0].zero();
#pragma unroll
    for (int i = 1; i < W; ++i) {
      const int t = t0 - i;
      if (t >= 0)
        xr[W - i].load(xp + (int64_t)t * D);
      else
        xr[W - i].zero();
    }
    XR dyc[U], dyn[U], xc[U], xn[U];
    WR wc[U], wn[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = t0 + u;
      if (t < tload) {
        dyc[u].load(dyp + (int64_t)t * D);
        wc[u].load(wp + (int64_t)t * wrs);
      } else {
        dyc[u].zero();
        wc[u].zero();
      }
      if (t < t1) xc[u].load(xp + (int64_t)t * D);
    }
    for (int tc = t0; tc < tend; tc += U) {
      if (tc + U < tend) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int t = tc + U + u;
          if (t < tload) {
            dyn[u].load(dyp + (int64_t)t * D);
            wn[u].load(wp + (int64_t)t * wrs);
          } else {
            dyn[u].zero();
            wn[u].zero();
          }
          if (t < t1) xn[u].load(xp + (int64_t)t * D);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int t = tc + u;
        if (t < tend) {
          const int p = u % W;
          const bool main_row = t < t1;
          float dyv[VEC];
          dyc[u].to_float(dyv);
          // dx[t-k] += dy[t] * (w[t, h, k] + sw[k]); row t opens with its k = 0 term.
#pragma unroll
          for (int j = 0; j < VEC; ++j) {
            const float v = dyv[j] * (wc[u].get((j / HSV) * W) + swr[0].get(j));
            dxa[p][j] = residual ? v + dyv[j] : v;
          }
#pragma unroll
          for (int k = 1; k < W; ++k) {
            const int q = ring<W>(u, k);
#pragma unroll
            for (int j = 0; j < VEC; ++j)
              dxa[q][j] = fmaf(dyv[j], wc[u].get((j / HSV) * W + k) + swr[k].get(j), dxa[q][j]);
          }
          if (main_row) {
            xr[p] = xc[u];
            float dwv[NWE];
#pragma unroll
            for (int k = 0; k < W; ++k) {
              const int q = ring<W>(u, k);
              float pr[VEC];
#pragma unroll
              for (int j = 0; j < VEC; ++j) pr[j] = dyv[j] * xr[q].get(j);
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
            if (lph > 1) {
#pragma unroll
              for (int k = 0; k < NWE; ++k) dwv[k] = group_sum(dwv[k], lph);
            }
            if constexpr (TDW) {
              // Lane l's piece j goes to slot l*NP + j; slot i*64 + l is then
              // the wavefront's i-th contiguous 1 KiB.  One wavefront writes
              // and reads its own slots, in order: no barrier.
              T e[NWE];
#pragma unroll
              for (int i = 0; i < NWE; ++i) e[i] = (T)dwv[i];
              u32x4 pc[NP];
              __builtin_memcpy(pc, e, sizeof(pc));
              u32x4* my = dwt[wave];
#pragma unroll
              for (int j = 0; j < NP; ++j) my[lane * NP + j] = pc[j];
              u32x4* dst = reinterpret_cast<u32x4*>(dwp0 + (int64_t)t * wrs);
#pragma unroll
              for (int i = 0; i < NP; ++i) __builtin_nontemporal_store(my[i * 64 + lane], dst + i * 64 + lane);
            } else {
              if (leader) store_vals<T, NWE>(dwp + (int64_t)t * wrs, dwv);
            }
          }
          const int tdone = t - (W - 1);
          if (tdone >= t0 && tdone < t1) store_vals<T, VEC, true>(dxp + (int64_t)tdone * D, dxa[(u + 1) % W]);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        dyc[u] = dyn[u];
        wc[u] = wn[u];
        xc[u] = xn[u];
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
  hw_fwd_fast<T, W, HSV><<<pl.nblk, 256, 0, p.stream>>>((const T*)p.x, (const T*)p.weight, (const T*)p.static_w,
                                                         (T*)p.y, pl.a);
  return hipGetLastError();
}

template <typename T, int W, int HSV, bool TDW>
void launch_bwd_kernel(const HwProblem& p, const HwPlan& pl) {
  if (p.static_w) {
    hw_bwd_fast<T, W, HSV, true, TDW><<<pl.nblk, 256, 0, p.stream>>>(
        (const T*)p.x, (const T*)p.weight, (const T*)p.static_w, (const T*)p.dy, (T*)p.dx, (T*)p.dweight, p.ws,
        pl.a);
  } else {
    hw_bwd_fast<T, W, HSV, false, TDW><<<pl.nblk, 256, 0, p.stream>>>(
        (const T*)p.x, (const T*)p.weight, nullptr, (const T*)p.dy, (T*)p.dx, (T*)p.dweight, nullptr, pl.a);
  }
}

template <typename T, int W, int HSV>
hipError_t launch_bwd_fast(const HwProblem& p, const HwPlan& pl) {
  if constexpr (TdwOf<T, W, HSV>::value) {
    if (pl.tdw)
      launch_bwd_kernel<T, W, HSV, true>(p, pl);
    else
      launch_bwd_kernel<T, W, HSV, false>(p, pl);
  } else {
    launch_bwd_kernel<T, W, HSV, false>(p, pl);
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
