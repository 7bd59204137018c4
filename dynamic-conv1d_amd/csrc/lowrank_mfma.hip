// Lowrank dynamic convolution on gfx950 matrix cores (bf16 / fp16).
//
//   Kw[t, k, d] = sum_r z_eff[t, r] * U_eff[r, k*D + d]      (MFMA, fp32 accumulate)
//   y[t, d]     = sum_k Kw[t, k, d] * x[t-k, d]  (+ x[t, d])
//
// z_eff / U_eff are z / U extended by the static filter as rank R with
// z == 1 and U row = static_w (the reference's fusion, lowrank.py:223-225),
// and by zero ranks up to a multiple of 16; neither is materialised.
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
#include "dc_common.h"
#include "dc_launch.h"

namespace dc {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 h16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <typename T> struct Mma16;
template <> struct Mma16<bf16> {
  static constexpr uint16_t kOne = 0x3F80;  // 1.0
  __device__ static __forceinline__ f32x4 run(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a), __builtin_bit_cast(s16x4, b), c,
                                                      0, 0, 0);
  }
  __device__ static __forceinline__ float to_f(uint32_t bits) { return __uint_as_float(bits << 16); }
};
template <> struct Mma16<fp16> {
  static constexpr uint16_t kOne = 0x3C00;  // 1.0
  __device__ static __forceinline__ f32x4 run(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(h16x4, a), __builtin_bit_cast(h16x4, b), c, 0,
                                                 0, 0);
  }
  __device__ static __forceinline__ float to_f(uint32_t bits) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
  }
};

// 16-bit element j (0..7) of a 128-bit row piece, in the low half of a word.
__device__ __forceinline__ uint32_t elem16(const u32x4& v, int j) {
  const uint32_t w = v[j >> 1];
  return (j & 1) ? (w >> 16) : (w & 0xFFFFu);
}

template <typename T>
__device__ __forceinline__ uint32_t f2bits(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (T)f);
}

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
  int nblk;        // grid size
};

// z_eff[row, r] as raw 16-bit bits (row < T checked by the caller).
template <typename T>
__device__ __forceinline__ uint32_t zbits(const uint16_t* __restrict__ z, int64_t row, int R, int RK, int r) {
  if (r < R) return z[row * R + r];
  return r < RK ? Mma16<T>::kOne : 0u;
}

// Packed B operands of one 128-channel chunk, staged once per workgroup:
// ub[(k*RC + c)*8 + j][lane] = U_eff[16c + 4q + kk, k*D + dl + j], kk = 0..3.
template <int W, int RC>
__device__ __forceinline__ void stage_u(u32x2* __restrict__ lds, const uint16_t* __restrict__ U,
                                        const uint16_t* __restrict__ sw, int R, int RK, int D, int dl, bool chv,
                                        int q, int lane, int wave) {
  const int64_t WD = (int64_t)W * D;
  for (int kc = wave; kc < W * RC; kc += 4) {
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

template <typename T, int W, int RC>
__global__ __launch_bounds__(256) void lr_fwd_mfma(const T* __restrict__ x_, const T* __restrict__ z_,
                                                   const T* __restrict__ U_, const T* __restrict__ sw_,
                                                   T* __restrict__ y_, LrArgs a) {
  const uint16_t* __restrict__ x = reinterpret_cast<const uint16_t*>(x_);
  const uint16_t* __restrict__ z = reinterpret_cast<const uint16_t*>(z_);
  const uint16_t* __restrict__ U = reinterpret_cast<const uint16_t*>(U_);
  const uint16_t* __restrict__ sw = reinterpret_cast<const uint16_t*>(sw_);
  uint16_t* __restrict__ y = reinterpret_cast<uint16_t*>(y_);
  __shared__ u32x2 ub[W * RC * 8 * 64];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q = lane >> 4, n = lane & 15;
  const int lb = xcd_remap(blockIdx.x, a.nblk);
  const int chunk = lb % a.nch, sgp = lb / a.nch;  // 4 wavefronts: one chunk, 4 consecutive runs
  const int D = a.D;
  const int dl = chunk * 128 + 8 * n;  // first channel of the lane's octet
  const bool chv = dl < D;             // D % 8 == 0: octets are whole
  stage_u<W, RC>(ub, U, sw, a.R, a.RK, D, dl, chv, q, lane, wave);
  __syncthreads();

  const int sg = sgp * 4 + wave;
  if (sg >= a.nseg) return;
  const int b = sg / a.nspb;
  const int ntile = (a.Tn + 15) >> 4;
  const int tile0 = (sg - b * a.nspb) * a.seg;
  const int tile1 = min(tile0 + a.seg, ntile);

  const int64_t row0 = (int64_t)b * a.Tn;
  for (int tile = tile0; tile < tile1; ++tile) {
    const int t0 = tile * 16;
    // A operands: z_eff[t0 + n, 16c + 4q + kk].
    u32x2 za[RC];
    {
      const int t = t0 + n;
#pragma unroll
      for (int c = 0; c < RC; ++c) {
        uint32_t e[4];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) e[kk] = t < a.Tn ? zbits<T>(z, row0 + t, a.R, a.RK, 16 * c + 4 * q + kk) : 0u;
        za[c][0] = e[0] | (e[1] << 16);
        za[c][1] = e[2] | (e[3] << 16);
      }
    }
    // x rows t0 + 4q - (W-1) .. t0 + 4q + 3.
    u32x4 xr[W + 3];
#pragma unroll
    for (int m = 0; m < W + 3; ++m) {
      const int t = t0 + 4 * q - (W - 1) + m;
      xr[m] = (chv && t >= 0 && t < a.Tn) ? *reinterpret_cast<const u32x4*>(x + (row0 + t) * D + dl)
                                          : u32x4{0u, 0u, 0u, 0u};
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
        for (int c = 0; c < RC; ++c) wk = Mma16<T>::run(za[c], ub[((k * RC + c) * 8 + j) * 64 + lane], wk);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          acc[i][j] = fmaf(wk[i], Mma16<T>::to_f(elem16(xr[i - k + W - 1], j)), acc[i][j]);
      }
      // Consume tap k's weights before issuing tap k+1's products: keeps the
      // live accumulators at 8 x 4 instead of W x 8 x 4 (occupancy).
      __builtin_amdgcn_sched_barrier(0);
    }
    if (a.residual) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] += Mma16<T>::to_f(elem16(xr[i + W - 1], j));
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = t0 + 4 * q + i;
      if (chv && t < a.Tn) {
        u32x4 o;
#pragma unroll
        for (int h = 0; h < 4; ++h) o[h] = f2bits<T>(acc[i][2 * h]) | (f2bits<T>(acc[i][2 * h + 1]) << 16);
        *reinterpret_cast<u32x4*>(y + (row0 + t) * D + dl) = o;
      }
    }
  }
}

// ------------------------------------------------------------------- host
namespace {

bool aligned16(const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

LrArgs make_args(const LrProblem& p, int target_waves) {
  LrArgs a;
  a.Tn = (int)p.T;
  a.D = (int)p.D;
  a.R = (int)p.R;
  a.RK = (int)p.R + (p.static_w ? 1 : 0);
  a.has_static = p.static_w != nullptr;
  a.residual = p.residual;
  a.nch = (int)((p.D + 127) / 128);
  a.ncg = 0;
  const int64_t ntile = (p.T + 15) / 16;
  int64_t seg = (p.B * ntile * a.nch + target_waves - 1) / target_waves;
  if (seg < 1) seg = 1;
  if (seg > ntile) seg = ntile;
  a.seg = (int)seg;
  a.nspb = (int)((ntile + seg - 1) / seg);
  a.nseg = (int)(p.B * a.nspb);
  a.nblk = ((a.nseg + 3) / 4) * a.nch;
  return a;
}

template <typename T, int W, int RC>
hipError_t launch_fwd(const LrProblem& p) {
  const LrArgs a = make_args(p, 2048);
  lr_fwd_mfma<T, W, RC><<<a.nblk, 256, 0, p.stream>>>((const T*)p.x, (const T*)p.z, (const T*)p.U,
                                                       (const T*)p.static_w, (T*)p.y, a);
  return hipGetLastError();
}

template <typename T>
hipError_t dispatch_fwd(const LrProblem& p) {
  const int rc = (int)((p.R + (p.static_w ? 1 : 0) + 15) / 16);
#define DC_LR_CASE(WW, CC) \
  if (p.W == WW && rc == CC) return launch_fwd<T, WW, CC>(p);
  DC_LR_CASE(1, 1) DC_LR_CASE(1, 2) DC_LR_CASE(1, 3) DC_LR_CASE(1, 4)
  DC_LR_CASE(2, 1) DC_LR_CASE(2, 2) DC_LR_CASE(2, 3) DC_LR_CASE(2, 4)
  DC_LR_CASE(3, 1) DC_LR_CASE(3, 2)
  DC_LR_CASE(4, 1) DC_LR_CASE(4, 2)
  DC_LR_CASE(5, 1) DC_LR_CASE(6, 1) DC_LR_CASE(7, 1) DC_LR_CASE(8, 1)
#undef DC_LR_CASE
  return hipErrorInvalidValue;
}

}  // namespace

bool lr_mfma_ok_impl(const LrProblem& p, bool bwd) {
  if (bwd) return false;  // backward: lowrank.hip kernels
  if (p.dtype != kBF16 && p.dtype != kFP16) return false;
  if (p.W < 1 || p.W > 8) return false;
  if (p.D % 8 != 0) return false;
  const int64_t rc = (p.R + (p.static_w ? 1 : 0) + 15) / 16;
  if (rc > 4 || p.W * rc > 8) return false;  // staged operands: W*RC*4 KiB of LDS, at most 32 KiB
  return aligned16(p.x) && aligned16(p.U) && aligned16(p.static_w) && aligned16(p.y);
}

int64_t lr_mfma_ws_bytes(const LrProblem&) { return 0; }

hipError_t lr_mfma_fwd(const LrProblem& p) {
  return p.dtype == kBF16 ? dispatch_fwd<bf16>(p) : dispatch_fwd<fp16>(p);
}

hipError_t lr_mfma_bwd(const LrProblem&) { return hipErrorInvalidValue; }

}  // namespace dc
