// Headwise dynamic causal short convolution: host planning, generic kernels.
//
// The vectorised kernels (W <= 8) live in headwise_fast.h and the wide ones
// (9 <= W <= 16) in headwise_wide.h; both are instantiated per (dtype,
// direction) in headwise_fast_*.hip / headwise_wide_*.hip so they compile in
// parallel.
#include "headwise_wide.h"
#include "headwise_mma.h"

namespace dc {

extern template hipError_t dispatch_fast<bf16, false>(const HwProblem&, const HwPlan&);
extern template hipError_t dispatch_fast<bf16, true>(const HwProblem&, const HwPlan&);
extern template hipError_t dispatch_fast<fp16, false>(const HwProblem&, const HwPlan&);
extern template hipError_t dispatch_fast<fp16, true>(const HwProblem&, const HwPlan&);
extern template hipError_t dispatch_fast<float, false>(const HwProblem&, const HwPlan&);
extern template hipError_t dispatch_fast<float, true>(const HwProblem&, const HwPlan&);
extern template hipError_t dispatch_wide<bf16, false>(const HwProblem&, const HwWideArgs&);
extern template hipError_t dispatch_wide<bf16, true>(const HwProblem&, const HwWideArgs&);
extern template hipError_t dispatch_wide<fp16, false>(const HwProblem&, const HwWideArgs&);
extern template hipError_t dispatch_wide<fp16, true>(const HwProblem&, const HwWideArgs&);
extern template hipError_t dispatch_wide<float, false>(const HwProblem&, const HwWideArgs&);
extern template hipError_t dispatch_wide<float, true>(const HwProblem&, const HwWideArgs&);

// ------------------------------------------------------------ generic path
// Any D, any head size dividing D, any W <= DC_MAX_W, element alignment only.
// One thread per output element; used for shapes the vector path rejects and
// as an independent second implementation in the tests.
template <typename T>
__global__ __launch_bounds__(256) void hw_fwd_generic(const T* __restrict__ x, const T* __restrict__ wt,
                                                      const T* __restrict__ sw, T* __restrict__ y, int64_t BT,
                                                      int Tn, int D, int H, int hs, int W, int residual) {
  const int64_t n = BT * D;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t row = i / D;
    const int d = (int)(i - row * D);
    const int t = (int)(row % Tn);
    const int h = d / hs;
    float acc = 0.f;
    for (int k = 0; k < W && k <= t; ++k) {
      float tap = (float)wt[(row * H + h) * W + k];
      if (sw) tap += (float)sw[(int64_t)k * D + d];
      acc = fmaf(tap, (float)x[(row - k) * D + d], acc);
    }
    if (residual) acc += (float)x[i];
    y[i] = (T)acc;
  }
}

template <typename T>
__global__ __launch_bounds__(256) void hw_bwd_dx_generic(const T* __restrict__ wt, const T* __restrict__ sw,
                                                         const T* __restrict__ dy, T* __restrict__ dx,
                                                         int64_t BT, int Tn, int D, int H, int hs, int W,
                                                         int residual) {
  const int64_t n = BT * D;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t row = i / D;
    const int d = (int)(i - row * D);
    const int t = (int)(row % Tn);
    const int h = d / hs;
    float acc = 0.f;
    for (int k = 0; k < W && t + k < Tn; ++k) {
      float tap = (float)wt[((row + k) * H + h) * W + k];
      if (sw) tap += (float)sw[(int64_t)k * D + d];
      acc = fmaf((float)dy[(row + k) * D + d], tap, acc);
    }
    if (residual) acc += (float)dy[i];
    dx[i] = (T)acc;
  }
}

template <typename T>
__global__ __launch_bounds__(256) void hw_bwd_dw_generic(const T* __restrict__ x, const T* __restrict__ dy,
                                                         T* __restrict__ dwt, int64_t BT, int Tn, int D, int H,
                                                         int hs, int W) {
  const int64_t n = BT * H;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t row = i / H;
    const int h = (int)(i - row * H);
    const int t = (int)(row % Tn);
    for (int k = 0; k < W; ++k) {
      // Compensated (Neumaier) sum over the head: a plain running fp32 sum of
      // hundreds of products drifts well past the reference's blocked sum.
      float s = 0.f, comp = 0.f;
      if (k <= t) {
        const T* dyr = dy + row * D + (int64_t)h * hs;
        const T* xr = x + (row - k) * D + (int64_t)h * hs;
        for (int c = 0; c < hs; ++c) {
          // __fmul_rn / __fadd_rn: no contraction into an FMA, which would
          // make u differ from s + p and void the compensation
          const float p = __fmul_rn((float)dyr[c], (float)xr[c]);
          const float u = __fadd_rn(s, p);
          comp += fabsf(s) >= fabsf(p) ? __fadd_rn(__fsub_rn(s, u), p) : __fadd_rn(__fsub_rn(p, u), s);
          s = u;
        }
      }
      dwt[i * W + k] = (T)(s + comp);
    }
  }
}

// dstatic partials: grid (ceil(W*D/256), P); partial p covers rows
// [p*rows_per, (p+1)*rows_per) of the flattened B*T axis.
template <typename T>
__global__ __launch_bounds__(256) void hw_bwd_dsw_generic(const T* __restrict__ x, const T* __restrict__ dy,
                                                          float* __restrict__ part, int64_t BT, int Tn, int D,
                                                          int W, int64_t rows_per) {
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= (int64_t)W * D) return;
  const int k = (int)(c / D);
  const int d = (int)(c - (int64_t)k * D);
  const int64_t r0 = (int64_t)blockIdx.y * rows_per;
  const int64_t r1 = min(r0 + rows_per, BT);
  float acc = 0.f;
  for (int64_t row = r0; row < r1; ++row) {
    const int t = (int)(row % Tn);
    if (t >= k) acc = fmaf((float)dy[row * D + d], (float)x[(row - k) * D + d], acc);
  }
  part[(int64_t)blockIdx.y * W * D + c] = acc;
}

// --------------------------------------------------------------- host side
namespace {

constexpr int kMaxFastW = 8;

int ilog2(int64_t v) {
  int r = 0;
  while ((int64_t(1) << r) < v) ++r;
  return r;
}

int unroll_of(int W) { return W >= 4 ? W : W * (4 / W); }

bool aligned(const void* p, int a) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Run length: aim for `target_waves` wavefronts in total (1024 = one per
// SIMD of the 256 CUs: with the next chunk always in flight, fewer and longer
// runs measured faster than more, shorter ones), at least 4 rows, a multiple
// of the unroll.  Small problems get short runs so that the grid still covers
// the CUs: configs[0] (B2 T1024 D512, head size 1, fp32) forward 10.3 -> 6.4 us
// and backward 22.4 -> 13.0 us with a minimum of 4 rows instead of 16.
int choose_seg(int64_t B, int64_t T, int64_t nvg, int W, int target_waves) {
  const int u = unroll_of(W);
  int64_t seg = (B * T * nvg + target_waves - 1) / target_waves;
  if (seg < 4) seg = 4;
  seg = (seg + u - 1) / u * u;
  if (seg > T) seg = (T + u - 1) / u * u;
  return (int)seg;
}

// Bytes of the larger of a row of x and a row of weight.
int64_t max_row_bytes(const HwProblem& p) {
  const int64_t es = dtype_size(p.dtype);
  const int64_t xb = p.D * es, wb = p.H * p.W * es;
  return xb > wb ? xb : wb;
}

HwPlan make_plan(const HwProblem& p, bool bwd) {
  const int VEC = 16 / dtype_size(p.dtype);
  const int64_t hs = p.D / p.H;
  HwPlan pl;
  HwArgs& a = pl.a;
  a.Tn = (int)p.T;
  a.D = (int)p.D;
  a.H = (int)p.H;
  a.hs_shift = ilog2(hs);
  a.nvc = (int)(p.D / VEC);
  a.nvg = (a.nvc + 63) / 64;
  a.seg = choose_seg(p.B, p.T, a.nvg, (int)p.W, 1024);
  // a run's buffer resources span (seg + kHwSlackRows) rows at most kHwRunBytes
  const int u = unroll_of((int)p.W);
  const int64_t seg_cap = (kHwRunBytes / max_row_bytes(p) - kHwSlackRows) / u * u;
  if (a.seg > seg_cap) a.seg = (int)seg_cap;
  a.nspb = (int)((p.T + a.seg - 1) / a.seg);
  a.nseg = (int)(p.B * a.nspb);
  const int nsg = (a.nseg + 3) / 4;
  a.nblk = nsg * a.nvg;
  a.lph = hs > VEC ? (int)(hs / VEC) : 1;
  a.residual = p.residual;
  a.has_static = p.static_w != nullptr;
  pl.nblk = a.nblk;
  pl.tdw = a.nvc % 64 == 0;
  pl.P = nsg;
  return pl;
}

// ------------------------------------------------------------ wide path
// 9 <= W <= 32 (headwise_wide.h): power-of-two head sizes up to a wavefront's
// 64 * CPL channels, D a multiple of those, 16-byte weight-row segments per
// wavefront.  Runs are rounded to 4 rows (the kernels' row blocks are W
// rounded up to 2 or 4).
int wide_block(const HwProblem& p) { return ((int)p.W + 3) / 4 * 4; }

// Wavefronts per launch: two per SIMD (the backward's occupancy at up to 256
// registers per lane), runs of at least one row block.
constexpr int kWideTargetWaves = 2048;

HwWideArgs make_wide_args(const HwProblem& p) {
  const int64_t es = dtype_size(p.dtype);
  const int64_t hs = p.D / p.H;
  const int L = wide_block(p);
  HwWideArgs a;
  a.Tn = (int)p.T;
  a.D = (int)p.D;
  a.H = (int)p.H;
  const int cols = 64 * wide_cpl((int)p.W);
  a.hs_shift = ilog2(hs);
  a.lph = hs > cols / 64 ? (int)(hs / (cols / 64)) : 1;
  a.nwc = (int)(p.D / cols);
  int64_t seg = (p.B * p.T * a.nwc + kWideTargetWaves - 1) / kWideTargetWaves;
  seg = (seg + L - 1) / L * L;
  if (seg < L) seg = L;
  const int64_t tcap = (p.T + L - 1) / L * L;
  if (seg > tcap) seg = tcap;
  a.seg = (int)seg;
  a.nspb = (int)((p.T + seg - 1) / seg);
  a.nseg = (int)(p.B * a.nspb);
  a.nblk = ((a.nseg + 3) / 4) * a.nwc;
  a.sbytes = (int)((cols >> a.hs_shift) * p.W * es);
  a.residual = p.residual;
  return a;
}

bool hw_wide_ok(const HwProblem& p, bool bwd) {
  const int64_t es = dtype_size(p.dtype);
  const int64_t hs = p.D / p.H;
  if (p.W < kHwWideMinW || p.W > kHwWideMaxW) return false;
  const int64_t cols = 64 * wide_cpl((int)p.W);  // channels per wavefront
  if ((hs & (hs - 1)) != 0 || hs > cols) return false;  // a head within one wavefront
  if (p.D % cols != 0) return false;
  // the wavefront's weight segment and a weight row: whole 16-byte pieces
  if (((cols / hs) * p.W * es) % 16 != 0 || (p.H * p.W * es) % 16 != 0) return false;
  // each row has a resource of its own (any sequence length): a row's bytes, and
  // with them every in-row offset, stay below the out-of-range lane offset
  if (max_row_bytes(p) >= kHwLaneOob) return false;
  const int ea = (int)(wide_cpl((int)p.W) * es);  // a lane's channels
  if (!aligned(p.x, ea) || !aligned(p.static_w, ea) || !aligned(p.weight, 16)) return false;
  if (!bwd) return aligned(p.y, ea);
  return aligned(p.dy, ea) && aligned(p.dx, ea) && aligned(p.dweight, 16);
}

// ------------------------------------------------------- head-MFMA path
// The matrix-core kernels (headwise_mma.h): head sizes 8, 16, 32, 64 at
// 9 <= W <= 32 with whole 16-byte pieces of a wavefront's weight-row segment,
// bf16 / fp16, D a multiple of 64.  Runs of 16-row tiles; each run's resources
// reach 32 rows before it and 64 after it (the dy / weight look-ahead).
int64_t mma_max_run_tiles(const HwProblem& p) {
  const int64_t rowb = max_row_bytes(p);
  const int64_t rows = kMaxSeqBytes / rowb - kSeqSlackRows - kRunHaloRows - 64;
  return rows > 0 ? rows / 16 : 0;
}

bool hw_mma_ok(const HwProblem& p, bool bwd) {
  if (p.dtype != kBF16 && p.dtype != kFP16) return false;
  const int64_t hs = p.D / p.H;
  if (!hw_mma_width_ok((int)hs, (int)p.W) || p.D % 64 != 0) return false;
  if (mma_max_run_tiles(p) < 1) return false;
  // 16-byte pieces of x / dy rows and of the weight rows; y / dx a 16-bit element at a time
  if (!aligned(p.x, 16) || !aligned(p.weight, 16) || !aligned(p.static_w, 2)) return false;
  if (!bwd) return aligned(p.y, 2);
  return aligned(p.dy, 16) && aligned(p.dx, 2) && aligned(p.dweight, 16);
}

// Wavefronts per launch, all resident at once (one LDS region of 13-36 KiB and
// up to 256 VGPRs each): the backward one per SIMD, whose longer runs load
// their look-back and look-ahead blocks less often, the forward two.  B4 T4096
// D2048 head size 32 backward / forward: W 12 67 / 34 us, W 24 103 / 42 us;
// 1536 backward wavefronts 84 / 107 us (runs of 22 and 14 tiles), 2048 backward
// wavefronts at W 24 135 us (a second round: six fit per CU by LDS).
constexpr int kMmaBwdWaves = 1024, kMmaFwdWaves = 2048;

HwMmaArgs make_mma_args(const HwProblem& p, bool bwd) {
  HwMmaArgs a;
  a.Tn = (int)p.T;
  a.D = (int)p.D;
  a.H = (int)p.H;
  a.nwc = (int)(p.D / 64);
  const int64_t ntile = (p.T + 15) / 16;
  // runs per sequence: as many as the target allows, each at least one tile and
  // at most the resources' cap (tiles are split evenly among them)
  // the backward's wavefronts all resident: four per CU, or as many as fit by
  // LDS (head size 8 above W 20: three)
  int target = kMmaFwdWaves;
  if (bwd) {
    const int per = (160 * 1024) / ((hw_mma_bwd_lds_bytes((int)p.W, (int)(p.D / p.H)) + 1023) / 1024 * 1024);
    target = per >= 4 ? kMmaBwdWaves : 256 * per;
  }
  int64_t nspb = target / (p.B * a.nwc);
  if (nspb > ntile) nspb = ntile;
  const int64_t cap = mma_max_run_tiles(p);  // >= 1 (hw_mma_ok)
  if (nspb < (ntile + cap - 1) / cap) nspb = (ntile + cap - 1) / cap;
  if (nspb < 1) nspb = 1;
  a.nspb = (int)nspb;
  a.nseg = (int)(p.B * a.nspb);
  a.nblk = a.nseg * a.nwc;
  a.residual = p.residual;
  return a;
}

template <typename T>
hipError_t bwd_mma(const HwProblem& p) {
  const HwMmaArgs a = make_mma_args(p, true);
  const int hs = (int)(p.D / p.H);
  hipError_t e = p.static_w ? hw_bwd_mma_launch<T, true>(p, a, hs) : hw_bwd_mma_launch<T, false>(p, a, hs);
  if (e != hipSuccess || !p.static_w) return e;
  // one dstatic_w partial per run (row of wavefronts)
  return reduce_partials(p.ws, p.W * p.D, a.nseg, p.W * p.D, p.dstatic_w, p.dtype, p.stream);
}

template <typename T>
hipError_t fwd_mma(const HwProblem& p) {
  const HwMmaArgs a = make_mma_args(p, false);
  const int hs = (int)(p.D / p.H);
  return p.static_w ? hw_fwd_mma_launch<T, true>(p, a, hs) : hw_fwd_mma_launch<T, false>(p, a, hs);
}

template <typename T>
hipError_t fwd_wide(const HwProblem& p) {
  return dispatch_wide<T, false>(p, make_wide_args(p));
}

template <typename T>
hipError_t bwd_wide(const HwProblem& p) {
  const HwWideArgs a = make_wide_args(p);
  hipError_t e = dispatch_wide<T, true>(p, a);
  if (e != hipSuccess || !p.static_w) return e;
  return reduce_partials(p.ws, p.W * p.D, (a.nseg + 3) / 4, p.W * p.D, p.dstatic_w, p.dtype, p.stream);
}

unsigned generic_grid(int64_t n) {
  int64_t g = (n + 255) / 256;
  if (g > 65536) g = 65536;
  return (unsigned)(g < 1 ? 1 : g);
}

template <typename T>
hipError_t fwd_generic(const HwProblem& p) {
  const int64_t BT = p.B * p.T;
  hw_fwd_generic<T><<<generic_grid(BT * p.D), 256, 0, p.stream>>>(
      (const T*)p.x, (const T*)p.weight, (const T*)p.static_w, (T*)p.y, BT, (int)p.T, (int)p.D, (int)p.H,
      (int)(p.D / p.H), (int)p.W, p.residual);
  return hipGetLastError();
}

int generic_partials(int64_t BT) {
  int64_t P = (BT + 255) / 256;
  return (int)(P > 64 ? 64 : (P < 1 ? 1 : P));
}

template <typename T>
hipError_t bwd_generic(const HwProblem& p) {
  const int64_t BT = p.B * p.T;
  const int hs = (int)(p.D / p.H);
  hw_bwd_dx_generic<T><<<generic_grid(BT * p.D), 256, 0, p.stream>>>(
      (const T*)p.weight, (const T*)p.static_w, (const T*)p.dy, (T*)p.dx, BT, (int)p.T, (int)p.D, (int)p.H, hs,
      (int)p.W, p.residual);
  hw_bwd_dw_generic<T><<<generic_grid(BT * p.H), 256, 0, p.stream>>>(
      (const T*)p.x, (const T*)p.dy, (T*)p.dweight, BT, (int)p.T, (int)p.D, (int)p.H, hs, (int)p.W);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !p.static_w) return e;
  const int P = generic_partials(BT);
  const int64_t rows_per = (BT + P - 1) / P;
  dim3 grid((unsigned)((p.W * p.D + 255) / 256), (unsigned)P);
  hw_bwd_dsw_generic<T><<<grid, 256, 0, p.stream>>>((const T*)p.x, (const T*)p.dy, p.ws, BT, (int)p.T, (int)p.D,
                                                    (int)p.W, rows_per);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  return reduce_partials(p.ws, p.W * p.D, P, p.W * p.D, p.dstatic_w, p.dtype, p.stream);
}

}  // namespace

bool hw_fast_ok(const HwProblem& p, bool bwd) {
  const int es = dtype_size(p.dtype);
  const int VEC = 16 / es;
  const int64_t hs = p.D / p.H;
  if (p.W < 1 || p.W > kMaxFastW) return false;
  if (p.D % VEC != 0) return false;
  if ((hs & (hs - 1)) != 0) return false;  // power-of-two head size
  if (hs > 64 * VEC) return false;         // a head must fit in one wavefront
  // buffer offsets: a run of at least one chunk must fit the resource range
  if ((unroll_of((int)p.W) + kHwSlackRows) * max_row_bytes(p) > kHwRunBytes) return false;
  if (!aligned(p.x, 16) || !aligned(p.static_w, 16)) return false;
  // weight rows start at multiples of NHL*W elements; require that alignment.
  const int64_t nwe_bytes = (hs < VEC ? VEC / hs : 1) * p.W * es;
  const int wa = (nwe_bytes % 16 == 0) ? 16 : (nwe_bytes % 8 == 0) ? 8 : (nwe_bytes % 4 == 0) ? 4 : 2;
  if (!aligned(p.weight, wa)) return false;
  if (!bwd) return aligned(p.y, 16);
  return aligned(p.dy, 16) && aligned(p.dx, 16) && aligned(p.dweight, wa);
}

int64_t hw_bwd_ws_bytes(const HwProblem& p) {
  if (!p.static_w) return 0;
  int P;
  if (hw_fast_ok(p, true))
    P = make_plan(p, true).P;
  else if (hw_mma_ok(p, true))
    P = make_mma_args(p, true).nseg;
  else if (hw_wide_ok(p, true))
    P = (make_wide_args(p).nseg + 3) / 4;
  else
    P = generic_partials(p.B * p.T);
  return (int64_t)P * p.W * p.D * (int64_t)sizeof(float);
}

int hw_path(const HwProblem& p, bool bwd) {
  return hw_fast_ok(p, bwd) ? 1 : hw_mma_ok(p, bwd) ? 6 : hw_wide_ok(p, bwd) ? 5 : 0;
}

hipError_t hw_fwd(const HwProblem& p) {
  if (hw_fast_ok(p, false)) {
    const HwPlan pl = make_plan(p, false);
    switch (p.dtype) {
      case kBF16: return dispatch_fast<bf16, false>(p, pl);
      case kFP16: return dispatch_fast<fp16, false>(p, pl);
      default: return dispatch_fast<float, false>(p, pl);
    }
  }
  if (hw_mma_ok(p, false)) return p.dtype == kBF16 ? fwd_mma<bf16>(p) : fwd_mma<fp16>(p);
  if (hw_wide_ok(p, false)) {
    switch (p.dtype) {
      case kBF16: return fwd_wide<bf16>(p);
      case kFP16: return fwd_wide<fp16>(p);
      default: return fwd_wide<float>(p);
    }
  }
  switch (p.dtype) {
    case kBF16: return fwd_generic<bf16>(p);
    case kFP16: return fwd_generic<fp16>(p);
    default: return fwd_generic<float>(p);
  }
}

hipError_t hw_bwd(const HwProblem& p) {
  if (hw_fast_ok(p, true)) {
    const HwPlan pl = make_plan(p, true);
    switch (p.dtype) {
      case kBF16: return dispatch_fast<bf16, true>(p, pl);
      case kFP16: return dispatch_fast<fp16, true>(p, pl);
      default: return dispatch_fast<float, true>(p, pl);
    }
  }
  if (hw_mma_ok(p, true)) return p.dtype == kBF16 ? bwd_mma<bf16>(p) : bwd_mma<fp16>(p);
  if (hw_wide_ok(p, true)) {
    switch (p.dtype) {
      case kBF16: return bwd_wide<bf16>(p);
      case kFP16: return bwd_wide<fp16>(p);
      default: return bwd_wide<float>(p);
    }
  }
  switch (p.dtype) {
    case kBF16: return bwd_generic<bf16>(p);
    case kFP16: return bwd_generic<fp16>(p);
    default: return bwd_generic<float>(p);
  }
}

}  // namespace dc
