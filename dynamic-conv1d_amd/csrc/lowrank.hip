// Lowrank dynamic causal short convolution: generic kernels and host dispatch.
//
//   Kw[b,t,k,d] = sum_r z[b,t,r] * U[r, k*D+d]   (+ static_w[k,d])
//   y[b,t,d]    = sum_{k<W} Kw[b,t,k,d] * x[b,t-k,d]  (+ x[b,t,d])
//
// Reference: lowrank.py:24-67 (forward), 87-140 (dU/dz), 159-205 (dx),
// 214-299 (autograd glue).  The static filter is the reference's extra rank
// with z == 1 and U row = static_w (lowrank.py:223-225); here it is an
// implicit rank R of the kernel, so no padded z or concatenated U is built.
//
// This file holds the generic kernels, for the shapes no fast path takes
// (lowrank_mfma_*.hip, lowrank_f32*.hip), plus the dispatch.  x (and dx) rows may be xld (dxld) elements apart,
// for inputs read out of a fused projection.
#include "lowrank_mfma.h"

namespace dc {

// Element offset of (row = b*T + t, channel d) in y / dy: row*D + d for
// [B, T, D] (hd == D), else b*T*D + (d/hd)*T*hd + t*hd + d%hd for the
// head-major [B, D/hd, T, hd].
__device__ __forceinline__ int64_t yoff(int64_t row, int d, int Tn, int D, int hd) {
  if (hd == D) return row * D + d;
  const int64_t b = row / Tn;
  const int t = (int)(row - b * Tn), h = d / hd;
  return (b * D + (int64_t)h * hd) * Tn + (int64_t)t * hd + (d - h * hd);
}

template <typename T>
__device__ __forceinline__ float zrank(const T* __restrict__ z, int64_t row, int R, int r) {
  return r < R ? (float)z[row * R + r] : 1.0f;
}

template <typename T>
__device__ __forceinline__ float urank(const T* __restrict__ U, const T* __restrict__ sw, int R, int64_t WD,
                                       int r, int64_t col) {
  return r < R ? (float)U[(int64_t)r * WD + col] : (float)sw[col];
}

// Per-token tap weight Kw[row, k, d] in fp32: sum over dynamic ranks, then
// the static filter (reference.py:29-31 order).
template <typename T>
__device__ __forceinline__ float lr_tap(const T* __restrict__ z, const T* __restrict__ U,
                                        const T* __restrict__ sw, int64_t row, int R, int64_t WD, int64_t col) {
  float w = 0.f;
  for (int r = 0; r < R; ++r) w = fmaf((float)z[row * R + r], (float)U[(int64_t)r * WD + col], w);
  if (sw) w += (float)sw[col];
  return w;
}

// Generic forward and dx: a job is a block of kGenRows consecutive rows.  The
// z rows it needs (fp32, ranks padded with zeros to a multiple of 4) are staged
// in LDS once per job; a thread takes channels d = tid, tid+256, .. and, per
// tap, loads each U element once for all rows of the job.  Per output the
// arithmetic is lr_tap's (ranks in order, then the static filter) and the taps
// add in order, as one thread per output would.  A grid-stride loop over jobs
// (the grid is capped).
constexpr int kGenRows = 16;
constexpr int kGenMaxR = 256;  // kernel ranks of the generic path (DC_MAX_R)

// z rows rb .. rb+nrows-1 of the job into zs[i * rp + r] (0 past R and past BT).
template <typename T>
__device__ __forceinline__ void stage_zrows(float* __restrict__ zs, const T* __restrict__ z, int64_t rb, int nrows,
                                            int R, int rp, int64_t BT) {
  for (int e = threadIdx.x; e < nrows * rp; e += 256) {
    const int i = e / rp, r = e - i * rp;
    const int64_t row = rb + i;
    zs[e] = row < BT && r < R ? (float)z[row * R + r] : 0.f;
  }
}

template <typename T>
__global__ __launch_bounds__(256) void lr_fwd_generic(const T* __restrict__ x, const T* __restrict__ z,
                                                      const T* __restrict__ U, const T* __restrict__ sw,
                                                      T* __restrict__ y, int64_t BT, int Tn, int D, int64_t xld,
                                                      int hd, int R, int W, int residual) {
  __shared__ __attribute__((aligned(16))) float zs[kGenRows * kGenMaxR];
  const int64_t WD = (int64_t)W * D;
  const int rp = (R + 3) / 4 * 4;
  const int64_t njobs = (BT + kGenRows - 1) / kGenRows;
  for (int64_t job = blockIdx.x; job < njobs; job += gridDim.x) {
    const int64_t rb = job * kGenRows;
    __syncthreads();  // the previous job's reads of zs are done
    stage_zrows(zs, z, rb, kGenRows, R, rp, BT);
    __syncthreads();
    int tpos[kGenRows];  // position of each row in its sequence, -1 past BT
#pragma unroll
    for (int i = 0; i < kGenRows; ++i) tpos[i] = rb + i < BT ? (int)((rb + i) % Tn) : -1;
    for (int d = threadIdx.x; d < D; d += 256) {
      float acc[kGenRows];
#pragma unroll
      for (int i = 0; i < kGenRows; ++i) acc[i] = 0.f;
      for (int k = 0; k < W; ++k) {
        float kw[kGenRows];
#pragma unroll
        for (int i = 0; i < kGenRows; ++i) kw[i] = 0.f;
        for (int r = 0; r < rp; r += 4) {
          float u[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) u[q] = r + q < R ? (float)U[(int64_t)(r + q) * WD + (int64_t)k * D + d] : 0.f;
#pragma unroll
          for (int i = 0; i < kGenRows; ++i) {
            const float4 zv = *reinterpret_cast<const float4*>(zs + i * rp + r);
            kw[i] = fmaf(zv.x, u[0], kw[i]);
            kw[i] = fmaf(zv.y, u[1], kw[i]);
            kw[i] = fmaf(zv.z, u[2], kw[i]);
            kw[i] = fmaf(zv.w, u[3], kw[i]);
          }
        }
        const float st = sw ? (float)sw[(int64_t)k * D + d] : 0.f;
#pragma unroll
        for (int i = 0; i < kGenRows; ++i) {
          const bool in = tpos[i] >= k;  // rows whose tap k reaches before the sequence add nothing
          const float xv = (float)x[(in ? rb + i - k : rb) * xld + d];
          if (in) acc[i] = fmaf(sw ? kw[i] + st : kw[i], xv, acc[i]);
        }
      }
#pragma unroll
      for (int i = 0; i < kGenRows; ++i) {
        if (tpos[i] < 0) continue;
        float v = acc[i];
        if (residual) v += (float)x[(rb + i) * xld + d];
        y[yoff(rb + i, d, Tn, D, hd)] = (T)v;
      }
    }
  }
}

// dx[row, d] = sum_k dy[row+k, d] * Kw[row+k, k, d] (+ dy): the job's taps
// k .. k+kGenTapChunk-1 need z of rows rb+k .. rb+k+kGenRows+kGenTapChunk-2.
// Up to W = kGenTapChunk those rows are staged once per job; wider W stages
// them per chunk of taps and per 256 channels, so the channel loop runs the
// same trip count in every thread (its barriers) and out-of-range channels
// only skip the arithmetic.
constexpr int kGenTapChunk = 32;
template <typename T>
__global__ __launch_bounds__(256) void lr_bwd_dx_generic(const T* __restrict__ z, const T* __restrict__ U,
                                                         const T* __restrict__ sw, const T* __restrict__ dy,
                                                         T* __restrict__ dx, int64_t BT, int Tn, int D,
                                                         int64_t dxld, int hd, int R, int W, int residual) {
  __shared__ __attribute__((aligned(16))) float zs[(kGenRows + kGenTapChunk - 1) * kGenMaxR / 4 * 4];
  const int64_t WD = (int64_t)W * D;
  const int rp = (R + 3) / 4 * 4;
  const bool restage = W > kGenTapChunk;  // uniform: several chunks of taps
  const int64_t njobs = (BT + kGenRows - 1) / kGenRows;
  for (int64_t job = blockIdx.x; job < njobs; job += gridDim.x) {
    const int64_t rb = job * kGenRows;
    int tpos[kGenRows];
#pragma unroll
    for (int i = 0; i < kGenRows; ++i) tpos[i] = rb + i < BT ? (int)((rb + i) % Tn) : -1;
    for (int d0 = 0; d0 < D; d0 += 256) {
      const int d = d0 + (int)threadIdx.x;
      const bool dv = d < D;
      float acc[kGenRows];
#pragma unroll
      for (int i = 0; i < kGenRows; ++i) acc[i] = 0.f;
      for (int kc = 0; kc < W; kc += kGenTapChunk) {
        const int kn = min(kGenTapChunk, W - kc);  // taps of this chunk
        if (restage || d0 == 0) {
          __syncthreads();  // earlier reads of zs are done
          stage_zrows(zs, z, rb + kc, kGenRows + kn - 1, R, rp, BT);
          __syncthreads();
        }
        if (!dv) continue;
        for (int kk = 0; kk < kn; ++kk) {
          const int k = kc + kk;
          float kw[kGenRows];
#pragma unroll
          for (int i = 0; i < kGenRows; ++i) kw[i] = 0.f;
          for (int r = 0; r < rp; r += 4) {
            float u[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) u[q] = r + q < R ? (float)U[(int64_t)(r + q) * WD + (int64_t)k * D + d] : 0.f;
#pragma unroll
            for (int i = 0; i < kGenRows; ++i) {
              const float4 zv = *reinterpret_cast<const float4*>(zs + (i + kk) * rp + r);  // row rb+i+k
              kw[i] = fmaf(zv.x, u[0], kw[i]);
              kw[i] = fmaf(zv.y, u[1], kw[i]);
              kw[i] = fmaf(zv.z, u[2], kw[i]);
              kw[i] = fmaf(zv.w, u[3], kw[i]);
            }
          }
          const float st = sw ? (float)sw[(int64_t)k * D + d] : 0.f;
#pragma unroll
          for (int i = 0; i < kGenRows; ++i) {
            const bool in = tpos[i] >= 0 && tpos[i] + k < Tn;  // row rb+i+k in the same sequence
            const float dv2 = (float)dy[yoff(in ? rb + i + k : rb, d, Tn, D, hd)];
            if (in) acc[i] = fmaf(dv2, sw ? kw[i] + st : kw[i], acc[i]);
          }
        }
      }
      if (!dv) continue;
#pragma unroll
      for (int i = 0; i < kGenRows; ++i) {
        if (tpos[i] < 0) continue;
        float v = acc[i];
        if (residual) v += (float)dy[yoff(rb + i, d, Tn, D, hd)];
        dx[(rb + i) * dxld + d] = (T)v;
      }
    }
  }
}

// Sums of v[0 .. N) over the wavefront's 64 lanes, reduce-scattered: each step
// pairs lanes that differ in one bit (mask 32, 16, .., 1) and keeps the half of
// the entries that bit selects (upper when set), adding the partner's copy.
// Lane l ends with the totals of entries N/64 * l .. N/64 * l + N/64 - 1 in
// v[0 .. N/64).  Fixed order: deterministic.
template <int N>
__device__ __forceinline__ void wave_reduce_scatter(float (&v)[N], int lane) {
  static_assert(N % 64 == 0, "whole entries per lane");
  int n = N;
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const int half = n / 2;
    const bool upper = (lane & m) != 0;
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
      if (i < half) {
        const float send = upper ? v[i] : v[i + half];
        const float keep = upper ? v[i + half] : v[i];
        v[i] = keep + __shfl_xor(send, m);
      }
    }
    n = half;
  }
}

// dz[row, r] = sum_{k, d} dy[row, d] * x[row-k, d] * U[r, k*D+d].  A job is a
// block of kDzRows consecutive rows and kDzRanks ranks: each thread sums over
// the channels d = tid, tid+256, .. for all rows x ranks of the job in
// registers (every U element loaded once per job), then the 256 threads' sums
// are added: reduce-scattered within each wavefront, then the four wavefronts
// in wave order through LDS.  A grid-stride loop over jobs (the grid is capped).
constexpr int kDzRows = 16, kDzRanks = 8;
template <typename T>
__global__ __launch_bounds__(256) void lr_bwd_dz_generic(const T* __restrict__ x, const T* __restrict__ U,
                                                         const T* __restrict__ dy, T* __restrict__ dz, int64_t BT,
                                                         int Tn, int D, int64_t xld, int hd, int R, int W) {
  constexpr int NV = kDzRows * kDzRanks;
  __shared__ float red[4][NV];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t WD = (int64_t)W * D;
  const int nrc = (R + kDzRanks - 1) / kDzRanks;
  const int64_t njobs = (BT + kDzRows - 1) / kDzRows * nrc;
  for (int64_t job = blockIdx.x; job < njobs; job += gridDim.x) {
    const int64_t rb = job / nrc * kDzRows;
    const int r0 = (int)(job % nrc) * kDzRanks;
    float acc[NV];
#pragma unroll
    for (int e = 0; e < NV; ++e) acc[e] = 0.f;
    int tpos[kDzRows];  // position of each row in its sequence (-1 past BT): taps k <= t reach back
#pragma unroll
    for (int i = 0; i < kDzRows; ++i) tpos[i] = rb + i < BT ? (int)((rb + i) % Tn) : -1;
    for (int d = threadIdx.x; d < D; d += 256) {
      float dyv[kDzRows];
#pragma unroll
      for (int i = 0; i < kDzRows; ++i) {
        const int64_t row = rb + i;
        dyv[i] = row < BT ? (float)dy[yoff(row, d, Tn, D, hd)] : 0.f;
      }
      for (int k = 0; k < W; ++k) {
        float u[kDzRanks];
#pragma unroll
        for (int j = 0; j < kDzRanks; ++j)
          u[j] = r0 + j < R ? (float)U[(int64_t)(r0 + j) * WD + (int64_t)k * D + d] : 0.f;
        // branch-free, so that the 16 loads go out together: rows whose tap k
        // reaches before the sequence (or rows past BT) read their own row and add 0
        float g[kDzRows];
#pragma unroll
        for (int i = 0; i < kDzRows; ++i) {
          const bool in = tpos[i] >= k;
          const float xv = (float)x[(in ? rb + i - k : (tpos[i] < 0 ? rb : rb + i)) * xld + d];
          g[i] = in ? dyv[i] * xv : 0.f;
        }
#pragma unroll
        for (int i = 0; i < kDzRows; ++i)
#pragma unroll
          for (int j = 0; j < kDzRanks; ++j) acc[i * kDzRanks + j] = fmaf(g[i], u[j], acc[i * kDzRanks + j]);
      }
    }
    wave_reduce_scatter<NV>(acc, lane);
#pragma unroll
    for (int e = 0; e < NV / 64; ++e) red[wave][NV / 64 * lane + e] = acc[e];
    __syncthreads();
    if ((int)threadIdx.x < NV) {
      const int e = threadIdx.x;
      const float v = ((red[0][e] + red[1][e]) + red[2][e]) + red[3][e];
      const int64_t row = rb + e / kDzRanks;
      const int r = r0 + e % kDzRanks;
      if (row < BT && r < R) dz[row * R + r] = (T)v;
    }
    __syncthreads();
  }
}

// dU (and dstatic as kernel rank R) partials: a thread owns one column (k, d)
// of U for a slice of rows (blockIdx.y) and kDuRanks kernel ranks
// (blockIdx.z), all in registers, so each dy / x element is read once per
// chunk of ranks; z_eff of a row is the same for the whole workgroup.  Grid
// (ceil(W*D / 256), P, ceil(RK / kDuRanks)).
constexpr int kDuRanks = 16;
template <typename T>
__global__ __launch_bounds__(256) void lr_bwd_du_generic(const T* __restrict__ x, const T* __restrict__ z,
                                                         const T* __restrict__ dy, float* __restrict__ part,
                                                         int64_t BT, int Tn, int D, int64_t xld, int hd, int R,
                                                         int RK, int W, int64_t rows_per) {
  const int64_t WD = (int64_t)W * D;
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= WD) return;  // no barriers below
  const int k = (int)(c / D);
  const int d = (int)(c - (int64_t)k * D);
  const int r0 = (int)blockIdx.z * kDuRanks;
  const int64_t s0 = (int64_t)blockIdx.y * rows_per;
  const int64_t s1 = min(s0 + rows_per, BT);
  float acc[kDuRanks];
#pragma unroll
  for (int j = 0; j < kDuRanks; ++j) acc[j] = 0.f;
  // rows in steps of kDuStep, branch-free so that a step's loads go out
  // together: rows past the slice, or whose tap k reaches before the sequence,
  // read the slice's first row and add 0
  constexpr int kDuStep = 8;
  int t = (int)(s0 % Tn);  // the position in its sequence of the step's first row
  for (int64_t row = s0; row < s1; row += kDuStep) {
    float g[kDuStep];
    int tu = t;
#pragma unroll
    for (int u = 0; u < kDuStep; ++u) {
      const bool in = row + u < s1 && tu >= k;
      const int64_t rr = in ? row + u : s0;
      const float gv = (float)dy[yoff(rr, d, Tn, D, hd)] * (float)x[(in ? rr - k : rr) * xld + d];
      g[u] = in ? gv : 0.f;
      tu = tu + 1 == Tn ? 0 : tu + 1;
    }
#pragma unroll
    for (int u = 0; u < kDuStep; ++u) {
      const int64_t rr = row + u < s1 ? row + u : s0;
#pragma unroll
      for (int j = 0; j < kDuRanks; ++j) {
        const int r = r0 + j;
        if (r < RK) acc[j] = fmaf(zrank(z, rr, R, r), g[u], acc[j]);
      }
    }
    t = tu;
  }
#pragma unroll
  for (int j = 0; j < kDuRanks; ++j)
    if (r0 + j < RK) part[((int64_t)blockIdx.y * RK + r0 + j) * WD + c] = acc[j];
}

// ------------------------------------------------------------------- host
namespace {

bool aligned_to16(const void* p) { return aligned_to(p, 16); }
bool aligned_to8(const void* p) { return aligned_to(p, 8); }

// Workgroups of the generic dz launch: one per job (kDzRows rows x kDzRanks
// ranks), at most 65536 (a grid-stride loop takes the rest: HIP rejects grids
// above 2^32 work-items).
unsigned dz_grid(int64_t BT, int R) {
  const int64_t jobs = (BT + kDzRows - 1) / kDzRows * ((R + kDzRanks - 1) / kDzRanks);
  return (unsigned)(jobs < 65536 ? jobs : 65536);
}

// Workgroups of the generic forward / dx launches: one per job of kGenRows
// rows, at most 65536 (a grid-stride loop takes the rest).
unsigned gen_row_grid(int64_t BT) {
  const int64_t jobs = (BT + kGenRows - 1) / kGenRows;
  return (unsigned)(jobs < 65536 ? jobs : 65536);
}

int generic_partials(int64_t BT) {
  int64_t P = (BT + 255) / 256;
  return (int)(P > 64 ? 64 : (P < 1 ? 1 : P));
}

template <typename T>
hipError_t fwd_generic(const LrProblem& p) {
  const int64_t BT = p.B * p.T;
  lr_fwd_generic<T><<<gen_row_grid(BT), 256, 0, p.stream>>>(
      (const T*)p.x, (const T*)p.z, (const T*)p.U, (const T*)p.static_w, (T*)p.y, BT, (int)p.T, (int)p.D, p.xld(),
      (int)p.yhd(), (int)p.R, (int)p.W, p.residual);
  return hipGetLastError();
}

template <typename T>
hipError_t bwd_generic(const LrProblem& p) {
  const int64_t BT = p.B * p.T;
  const int RK = (int)p.R + (p.static_w ? 1 : 0);
  const int64_t WD = p.W * p.D;
  lr_bwd_dx_generic<T><<<gen_row_grid(BT), 256, 0, p.stream>>>(
      (const T*)p.z, (const T*)p.U, (const T*)p.static_w, (const T*)p.dy, (T*)p.dx, BT, (int)p.T, (int)p.D,
      p.dxld(), (int)p.yhd(), (int)p.R, (int)p.W, p.residual);
  lr_bwd_dz_generic<T><<<dz_grid(BT, (int)p.R), 256, 0, p.stream>>>((const T*)p.x, (const T*)p.U, (const T*)p.dy,
                                                          (T*)p.dz, BT, (int)p.T, (int)p.D, p.xld(), (int)p.yhd(),
                                                          (int)p.R, (int)p.W);
  const int P = generic_partials(BT);
  const int64_t rows_per = (BT + P - 1) / P;
  dim3 grid((unsigned)((WD + 255) / 256), (unsigned)P, (unsigned)((RK + kDuRanks - 1) / kDuRanks));
  lr_bwd_du_generic<T><<<grid, 256, 0, p.stream>>>((const T*)p.x, (const T*)p.z, (const T*)p.dy, p.ws, BT,
                                                   (int)p.T, (int)p.D, p.xld(), (int)p.yhd(), (int)p.R, RK,
                                                   (int)p.W, rows_per);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const PartialReduce jobs[2] = {
      {p.ws, RK * WD, P, p.R * WD, p.dU},
      {p.ws + p.R * WD, RK * WD, P, p.static_w ? WD : 0, p.dstatic_w},
  };
  return reduce_partials_multi(jobs, 2, p.dtype, p.stream);
}

}  // namespace

// Shapes, dtypes and alignments the MFMA kernels (lowrank_mfma_{fwd,bwd}.hip) take.
bool lr_mfma_ok(const LrProblem& p, bool bwd) {
  if (p.dtype != kBF16 && p.dtype != kFP16) return false;
  if (p.W < 1 || p.W > 32) return false;
  // every W <= 32 at every kernel rank <= 64: the forward stages W x RC
  // operand chunks (up to 128 KiB of LDS) and runs wider problems (above W 16
  // at one or two rank chunks, above W 8 at three or four) as passes of taps;
  // the backward runs wide W x RC as passes of taps (the runs' 32-row halo
  // covers a pass's look-back)
  // above kernel rank 64 (up to 256) as passes of ranks: the forward as passes of
  // 64 (each split into passes of at most 8 taps), at most kFwdMaxPasses of
  // them in all, since y is rounded after each; the backward as passes of 32
  // (also at kernel ranks 49-64 from W 2 on, lr_bwd_rank_split; any number:
  // past four its dx goes to an fp32 accumulator)
  const int64_t RK = p.R + (p.static_w ? 1 : 0);
  if (RK > kLrMfmaMaxRank) return false;
  if (!bwd && lr_fwd_npasses(p) > kFwdMaxPasses) return false;
  // buffer-offset range of a run (resources start at each run's base row, so
  // the sequence length is free): at least one tile must fit
  if ((bwd ? lr_bwd_max_run_tiles(p) : lr_fwd_max_run_tiles(p)) < 1) return false;
  if (!bwd) {
    // 16-byte row pieces of x at every row: xld a multiple of 8 elements
    if (p.D % 8 != 0 || p.xld() % 8 != 0) return false;
    if (p.yhd() % 8 != 0) return false;  // a lane's y octet inside one head
    return aligned_to16(p.x) && aligned_to16(p.U) && aligned_to16(p.static_w) && aligned_to16(p.y);
  }
  // whole 8-channel dz operand pieces (D % 8 == 0) and 4-byte-aligned row pieces of x / dx
  if (p.D % 8 != 0 || p.xld() % 4 != 0 || p.dxld() % 4 != 0) return false;
  // dU partial stores: byte offsets up to (RK + 16) rows of W*D fp32 stay below kOobLane
  if ((p.R + 1 + 16) * p.W * p.D * 4 > kOobLane) return false;
  if (p.yhd() != p.D && p.yhd() % 64 != 0) return false;  // a wavefront's dy channels inside one head
  return aligned_to8(p.x) && aligned_to8(p.dy) && aligned_to8(p.dx) && aligned_to16(p.U) && aligned_to16(p.static_w);
}

int64_t lr_zeff_bytes(const LrProblem& p) {
  if (!lr_mfma_ok(p, true)) return 0;
  const bool has_static = p.static_w != nullptr;
  const int64_t rc = (p.R + (has_static ? 1 : 0) + 15) / 16;
  // above kernel rank 64 the forward runs as passes of ranks and keeps no
  // z_eff: the backward pads z itself (one small launch next to its passes)
  if (rc > 4) return 0;
  // the backward reads z itself when its rows are what the kernel loads: R % 4
  // == 0 (8-byte loads) or, for two rank chunks and passes of 32 ranks, a
  // multiple of 32 dynamic ranks (16-byte loads)
  const bool k32 = rc == 2 || lr_bwd_rank_split(p.R + (has_static ? 1 : 0), p.W);
  const bool pad = k32 ? !(p.R % 32 == 0 && !has_static) : p.R % 4 != 0;
  return pad ? p.B * p.T * lr_bwd_zrow(p.R, has_static, p.W) * 2 : 0;
}

int64_t lr_bwd_ws_bytes(const LrProblem& p) {
  if (lr_mfma_ok(p, true)) return lr_mfma_ws_bytes(p);
  if (lr_f32m_bwd_ok(p) || lr_f32_ok(p)) {
    // fp32: the larger of the two fast paths' needs (alignment picks between them at the call)
    const int64_t m = lr_f32m_bwd_ok(p) ? lr_f32m_ws_bytes(p) : 0;
    const int64_t v = lr_f32_ok(p) ? lr_f32_ws_bytes(p) : 0;
    return m > v ? m : v;
  }
  const int64_t RK = p.R + (p.static_w ? 1 : 0);
  return (int64_t)generic_partials(p.B * p.T) * RK * p.W * p.D * (int64_t)sizeof(float);
}

// The dispatch order of lr_fwd / lr_bwd below, as dc_path codes.
int lr_path(const LrProblem& p, bool bwd) {
  if (lr_mfma_ok(p, bwd)) return 2;
  if (bwd ? lr_f32m_bwd_ok(p) : lr_f32m_fwd_ok(p)) return 3;
  if (lr_f32_ok(p)) return 4;
  return 0;
}

namespace {
bool all_mfma_ok(const LrProblem* p, int G, bool bwd) {
  for (int g = 0; g < G; ++g)
    if (!lr_mfma_ok(p[g], bwd)) return false;
  return true;
}
}  // namespace

// G problems of one shape (see dc_launch.h): one MFMA launch for all of them,
// or per group the fp32 kernels (matrix cores, else the VALU) or the generic
// launch sequence.
hipError_t lr_fwd(const LrProblem* p, int G) {
  if (G < 1 || G > kMaxGroups) return hipErrorInvalidValue;
  if (all_mfma_ok(p, G, false)) return lr_mfma_fwd(p, G);  // writes z_eff when asked
  if (p[0].zeff) {
    hipError_t e = lr_zeff_fill(p, G);
    if (e != hipSuccess) return e;
  }
  for (int g = 0; g < G; ++g) {
    hipError_t e;
    if (lr_f32m_fwd_ok(p[g])) {
      if ((e = lr_f32m_fwd(p[g])) != hipSuccess) return e;
      continue;
    }
    if (lr_f32_ok(p[g])) {
      if ((e = lr_f32(p[g], false)) != hipSuccess) return e;
      continue;
    }
    switch (p[g].dtype) {
      case kBF16: e = fwd_generic<bf16>(p[g]); break;
      case kFP16: e = fwd_generic<fp16>(p[g]); break;
      default: e = fwd_generic<float>(p[g]); break;
    }
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t lr_bwd(const LrProblem* p, int G) {
  if (G < 1 || G > kMaxGroups) return hipErrorInvalidValue;
  if (all_mfma_ok(p, G, true)) return lr_mfma_bwd(p, G);
  for (int g = 0; g < G; ++g) {
    hipError_t e;
    if (lr_f32m_bwd_ok(p[g])) {
      if ((e = lr_f32m_bwd(p[g])) != hipSuccess) return e;
      continue;
    }
    if (lr_f32_ok(p[g])) {
      if ((e = lr_f32(p[g], true)) != hipSuccess) return e;
      continue;
    }
    switch (p[g].dtype) {
      case kBF16: e = bwd_generic<bf16>(p[g]); break;
      case kFP16: e = bwd_generic<fp16>(p[g]); break;
      default: e = bwd_generic<float>(p[g]); break;
    }
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace dc
