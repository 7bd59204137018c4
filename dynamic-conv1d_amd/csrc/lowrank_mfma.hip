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

// v_mfma_f32_16x16x32 (gfx950): lane l gives A[l%16][8(l/16)..+7] and B[8(l/16)..+7][l%16].
typedef __bf16 b16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 h16x8 __attribute__((ext_vector_type(8)));
template <typename T> struct Mma32;
template <> struct Mma32<bf16> {
  __device__ static __forceinline__ f32x4 run(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(b16x8, a), __builtin_bit_cast(b16x8, b), c, 0, 0,
                                                   0);
  }
};
template <> struct Mma32<fp16> {
  __device__ static __forceinline__ f32x4 run(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h16x8, a), __builtin_bit_cast(h16x8, b), c, 0, 0,
                                                  0);
  }
};

// 16-bit element j (0..3) of a 64-bit quartet, in the low half of a word.
__device__ __forceinline__ uint32_t elem16x2(const u32x2& v, int j) {
  const uint32_t w = v[j >> 1];
  return (j & 1) ? (w >> 16) : (w & 0xFFFFu);
}

// 16-bit element j (0..7) of a 128-bit row piece, in the low half of a word.
__device__ __forceinline__ uint32_t elem16(const u32x4& v, int j) {
  const uint32_t w = v[j >> 1];
  return (j & 1) ? (w >> 16) : (w & 0xFFFFu);
}

template <typename T>
__device__ __forceinline__ uint32_t f2bits(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (T)f);
}

template <typename T> struct Pair16;
template <> struct Pair16<bf16> { typedef __bf16 type __attribute__((ext_vector_type(2))); };
template <> struct Pair16<fp16> { typedef _Float16 type __attribute__((ext_vector_type(2))); };
typedef float f32x2 __attribute__((ext_vector_type(2)));

// Two floats rounded to nearest-even into one word (a in the low half): v_cvt_pk_{bf16,f16}_f32.
template <typename T>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  const f32x2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, typename Pair16<T>::type));
}
// Element j (0..3) of a 64-bit quartet as float.
template <typename T>
__device__ __forceinline__ float q4f(const u32x2& v, int j) {
  return Mma16<T>::to_f(elem16x2(v, j));
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


// ---------------------------------------------------------------- backward
//
// One pass over x and dy produces dx, dz, dU and dstatic_w (reference:
// lowrank.py:87-140 and 159-205, two kernels that both read dy).
//
// Tile: a wavefront owns 16 rows x 64 channels; lane l = 16q + n owns rows
// 4q..4q+3 and the channel quartet 4n..4n+3 (64-bit loads, 128 contiguous
// bytes per row across the 16 lanes of a row group).  With
// G_k[t, d] = bf16(dy[t, d] * x[t-k, d]) (the reference also rounds this
// product to bf16 before its dot products, lowrank.py:128):
//   * dU[r, kD+d] += sum_t z_eff[t, r] G_k[t, d]: MFMA with K = the 16 rows.
//     For each j the lane's four G values of column 4n+j are exactly the
//     B operand (rows 4q..4q+3 of column n); A is z_eff transposed.
//   * dz[t, r] += sum_d G_k[t, d] U_eff[r, kD+d]: needs K = channels.  The
//     same packed G registers fed as the *A* operand of an MFMA against the
//     16x16 identity return G transposed (lane now holds one row and four
//     channels 4(4q+i)+j), which is the A operand of the dz MFMA.  All
//     values are bf16-exact, so the transpose is exact.
//   * dx[t, d] = sum_k dy[t+k, d] Kw[t+k, k, d] (+ dy): the tap weights of
//     rows 4q..4q+3+W-1 come from NB = ceil((W+3)/4) MFMA row blocks (A rows
//     shifted by 4), so every lane has the look-ahead rows it needs without
//     cross-lane traffic; dy rows 4q..4q+W+2 are read from L1.
// A workgroup is 4 wavefronts on 4 adjacent 64-channel chunks of the same
// rows.  dz partial sums over the 256 channels are added in LDS per tile in
// wave order and written as one fp32 partial per 256-channel group; dU
// accumulates in registers over the wavefront's run of tiles and is written
// as one fp32 partial per run.  reduce_partials sums both deterministically.

struct LrBwdArgs {
  int Tn, D, R, RK, residual;
  int nch;    // ceil(D / 64) channel chunks
  int ncg;    // ceil(nch / 4) chunk groups: one workgroup column
  int seg;    // tiles per run
  int nspb;   // runs per sequence
  int nseg;   // B * nspb
  int nblk;   // ncg * nseg
  int64_t BT;
};


// U_eff operands of one wavefront's 64-channel chunk, staged once per run (the
// chunk never changes across it): the dz operands always in LDS, the tap-weight
// operands in registers when W*RC <= 4 (UWREG) and in LDS otherwise.  For tap k
// and rank chunk c, lane (q, n) reads
//   uw[j] (j = 0..3): ranks 16c+4q..16c+4q+3 of channel 4n+j, packed (B operand
//                     of the 16x16x16 tap-weight MFMA);
//   uz[s] (s = 0, 1): rank 16c+n, channels 32s+8q..32s+8q+7 as they lie in U
//                     (B operand of the 16x16x32 dz MFMA).
template <int W, int RC, bool UWREG>
__device__ __forceinline__ void stage_uops(u32x2* __restrict__ uw_lds, u32x2 (&uw_reg)[UWREG ? W * RC * 4 : 1],
                                           u32x4* __restrict__ uz_lds, const uint16_t* __restrict__ U,
                                           const uint16_t* __restrict__ sw, int R, int RK, int D, int d0, int q,
                                           int n, int lane) {
  const int64_t WD = (int64_t)W * D;
  const bool chv = d0 + 4 * n < D;
#pragma unroll
  for (int k = 0; k < W; ++k) {
#pragma unroll
    for (int c = 0; c < RC; ++c) {
      u32x2 rows[4];
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int r = 16 * c + 4 * q + kk;
        const uint16_t* src = nullptr;
        if (chv && r < R) src = U + (int64_t)r * WD + (int64_t)k * D + d0 + 4 * n;
        else if (chv && r < RK) src = sw + (int64_t)k * D + d0 + 4 * n;
        rows[kk] = src ? *reinterpret_cast<const u32x2*>(src) : u32x2{0u, 0u};
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        u32x2 uw;
        uw[0] = elem16x2(rows[0], j) | (elem16x2(rows[1], j) << 16);
        uw[1] = elem16x2(rows[2], j) | (elem16x2(rows[3], j) << 16);
        if constexpr (UWREG)
          uw_reg[(k * RC + c) * 4 + j] = uw;
        else
          uw_lds[((k * RC + c) * 4 + j) * 64 + lane] = uw;
      }
      const int r = 16 * c + n;
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        const int dd = d0 + 32 * s2 + 8 * q;  // multiple of 8; D % 16 == 0, so dd < D means dd + 8 <= D
        const uint16_t* src = nullptr;
        if (dd < D && r < R) src = U + (int64_t)r * WD + (int64_t)k * D + dd;
        else if (dd < D && r < RK) src = sw + (int64_t)k * D + dd;
        uz_lds[((k * RC + c) * 2 + s2) * 64 + lane] = src ? *reinterpret_cast<const u32x4*>(src) : u32x4{0u, 0u, 0u, 0u};
      }
    }
  }
}

// Raw buffer resources.  A descriptor covers one sequence ([T, C] elements);
// the hardware returns 0 for loads and drops stores whose VGPR byte offset is
// >= the range, which handles rows before 0 (negative offsets wrap to large
// unsigned values), rows past T and channels past D (lane offset kOobLane)
// without branches or clamped addresses.  The host only takes this path when
// one sequence spans at most kMaxSeqBytes, so no offset can wrap back into range.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int kOobLane = 0x60000000;
constexpr int64_t kMaxSeqBytes = int64_t(1) << 29;

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x2 bload64(rsrc_t r, int off) { return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0); }
__device__ __forceinline__ uint32_t bload16(rsrc_t r, int off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}
__device__ __forceinline__ void bstore64(u32x2 v, rsrc_t r, int off) { __builtin_amdgcn_raw_buffer_store_b64(v, r, off, 0, 0); }

template <typename T, int W, int RC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(W <= 4 && RC == 1 ? 2 : 1, 8))) void lr_bwd_mfma(
    const T* __restrict__ x_, const T* __restrict__ z_, const T* __restrict__ U_, const T* __restrict__ sw_,
    const T* __restrict__ dy_, T* __restrict__ dx_, float* __restrict__ part_dz, float* __restrict__ part_du,
    LrBwdArgs a) {
  constexpr int NB = (W + 6) / 4;  // MFMA row blocks for the dx look-ahead
  constexpr int NR = W + 3;        // x rows 4q-W+1 .. 4q+3 and dy rows 4q .. 4q+W+2 per lane
  constexpr bool UWREG = W * RC <= 4;   // tap-weight operands in registers
  constexpr int NUW = W * RC * 4;  // packed tap-weight operands per lane
  constexpr int NUZ = W * RC * 2;  // dz operands per lane
  constexpr int GROW = 72;         // G tile row pitch (64 channels + 8 pad: conflict-free reads)
  const uint16_t* __restrict__ x = reinterpret_cast<const uint16_t*>(x_);
  const uint16_t* __restrict__ z = reinterpret_cast<const uint16_t*>(z_);
  const uint16_t* __restrict__ U = reinterpret_cast<const uint16_t*>(U_);
  const uint16_t* __restrict__ sw = reinterpret_cast<const uint16_t*>(sw_);
  const uint16_t* __restrict__ dy = reinterpret_cast<const uint16_t*>(dy_);
  uint16_t* __restrict__ dx = reinterpret_cast<uint16_t*>(dx_);
  __shared__ u32x2 uw_lds[4][UWREG ? 1 : NUW * 64];
  __shared__ u32x4 uz_lds[4][NUZ * 64];
  __shared__ __attribute__((aligned(16))) uint16_t gtile[4][16 * GROW];
  // dz partial sums of the workgroup's 4 chunks, gathered for DZB tiles and
  // reduced once per batch (double-buffered: one barrier per batch).
  constexpr int DZB = (UWREG && RC == 1) ? 4 : 1;
  __shared__ float dzred[2][4][DZB][RC * 256];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q = lane >> 4, n = lane & 15;
  const int lb = xcd_remap(blockIdx.x, a.nblk);
  const int cg = lb % a.ncg, sg = lb / a.ncg;
  const int chunk = cg * 4 + wave;
  const int D = a.D, Tn = a.Tn;
  const int d0 = chunk * 64;
  const bool chv = d0 + 4 * n < D;  // lane quartet inside D (D % 16 == 0)
  const int col = d0 + 4 * n;
  const int64_t WD = (int64_t)W * D;
  const int b = sg / a.nspb;
  const int ntile = (Tn + 15) >> 4;
  const int tile0 = (sg - b * a.nspb) * a.seg;
  const int tile1 = min(tile0 + a.seg, ntile);
  const int64_t row0 = (int64_t)b * Tn;
  const int R = a.R, RK = a.RK;
  const bool zvec = (R & 3) == 0;
  u32x2* __restrict__ my_uw = uw_lds[wave];
  u32x4* __restrict__ my_uz = uz_lds[wave];
  uint16_t* __restrict__ my_g = gtile[wave];
  const int rowb = D * 2;
  const int64_t seqb = (int64_t)Tn * rowb;
  const rsrc_t rx = make_rsrc(x + row0 * D, seqb);
  const rsrc_t rdy = make_rsrc(dy + row0 * D, seqb);
  const rsrc_t rdx = make_rsrc(dx + row0 * D, seqb);
  const rsrc_t rz = make_rsrc(z + row0 * R, (int64_t)Tn * R * 2);
  const int lane_off = chv ? (4 * q * D + col) * 2 : kOobLane;  // byte offset of the lane's row 4q quartet

  u32x2 uw_reg[UWREG ? NUW : 1];
  stage_uops<W, RC, UWREG>(my_uw, uw_reg, my_uz, U, sw, R, RK, D, d0, q, n, lane);

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

  f32x4 du[W][RC][4];
#pragma unroll
  for (int k = 0; k < W; ++k)
#pragma unroll
    for (int c = 0; c < RC; ++c)
#pragma unroll
      for (int j = 0; j < 4; ++j) du[k][c][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int tile = tile0; tile < tile1; ++tile) {
    const int t0 = tile * 16;
    // ---- tile inputs (buffer loads: out-of-range rows / channels read as 0)
    const int toff = t0 * rowb;
    u32x2 xr[NR], dyr[NR];
#pragma unroll
    for (int m = 0; m < NR; ++m) {
      xr[m] = bload64(rx, lane_off + toff + (m - (W - 1)) * rowb);
      dyr[m] = bload64(rdy, lane_off + toff + m * rowb);
    }
    // z_eff rows t0+4bb+n, ranks 16c+4q..+3: A operand of the tap-weight MFMA.
    u32x2 zA[NB][RC];
#pragma unroll
    for (int bb = 0; bb < NB; ++bb) {
      const int t = t0 + 4 * bb + n;
#pragma unroll
      for (int c = 0; c < RC; ++c) {
        const int r0 = 16 * c + 4 * q;
        if (zvec && r0 + 3 < R) {  // 4 dynamic ranks, 8-byte aligned (R % 4 == 0)
          zA[bb][c] = bload64(rz, (t * R + r0) * 2);
        } else {
          uint32_t e[4];
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) {
            const int r = r0 + kk;
            const uint32_t v = bload16(rz, (t * R + min(r, R - 1)) * 2);
            e[kk] = r < R ? v : ((r < RK && t < Tn) ? (uint32_t)Mma16<T>::kOne : 0u);
          }
          zA[bb][c][0] = e[0] | (e[1] << 16);
          zA[bb][c][1] = e[2] | (e[3] << 16);
        }
      }
    }
    // z_eff transposed (rank n, rows 4q..4q+3), the A operand of the dU MFMA,
    // from row block 0 through the exact identity transpose.
    u32x2 zT[RC];
#pragma unroll
    for (int c = 0; c < RC; ++c) {
      const f32x4 tz = Mma16<T>::run(zA[0][c], ident, f32x4{0.f, 0.f, 0.f, 0.f});
      zT[c][0] = pack2<T>(tz[0], tz[1]);
      zT[c][1] = pack2<T>(tz[2], tz[3]);
    }

    float dyf[NR][4];
#pragma unroll
    for (int m = 0; m < NR; ++m)
#pragma unroll
      for (int j = 0; j < 4; ++j) dyf[m][j] = q4f<T>(dyr[m], j);

    float dxa[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) dxa[i][j] = 0.f;
    f32x4 dz[RC];
#pragma unroll
    for (int c = 0; c < RC; ++c) dz[c] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int k = 0; k < W; ++k) {
      // G_k = bf16(dy * x_shift) for rows 4q..4q+3, channels 4n..4n+3 (fp32 products).
      float gf[4][4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) gf[i][j] = dyf[i][j] * q4f<T>(xr[i - k + W - 1], j);
      // Row-major copy of the G tile in this wavefront's LDS, read back below as
      // the transposed (channel-contiguous) A operand of the dz MFMA.
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        u32x2 w;
        w[0] = pack2<T>(gf[i][0], gf[i][1]);
        w[1] = pack2<T>(gf[i][2], gf[i][3]);
        *reinterpret_cast<u32x2*>(my_g + (4 * q + i) * GROW + 4 * n) = w;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // dx += dy[4q+i+k] * Kw[4q+i+k, k]: tap weights of the row blocks that hold rows k..k+3.
#pragma unroll
        for (int bb = 0; bb < NB; ++bb) {
          if (4 * bb > 3 + k || 4 * bb + 3 < k) continue;
          f32x4 wk = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int c = 0; c < RC; ++c)
            wk = Mma16<T>::run(zA[bb][c], UWREG ? uw_reg[UWREG ? (k * RC + c) * 4 + j : 0]
                                                : my_uw[((k * RC + c) * 4 + j) * 64 + lane], wk);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int tr = i + k;  // row offset of dy / Kw in the lane window
            if (tr >= 4 * bb && tr < 4 * bb + 4) dxa[i][j] = fmaf(dyf[tr][j], wk[tr - 4 * bb], dxa[i][j]);
          }
        }
        // dU (K = rows): column j of G, rows 4q..4q+3, is the B operand as it lies.
        u32x2 g;
        g[0] = pack2<T>(gf[0][j], gf[1][j]);
        g[1] = pack2<T>(gf[2][j], gf[3][j]);
#pragma unroll
        for (int c = 0; c < RC; ++c) du[k][c][j] = Mma16<T>::run(zT[c], g, du[k][c][j]);
      }
      // dz (K = 32 channels): A = G row n (this lane: row = lane % 16), channels 32s+8q..+7.
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        const u32x4 ga = *reinterpret_cast<const u32x4*>(my_g + n * GROW + 32 * s2 + 8 * q);
#pragma unroll
        for (int c = 0; c < RC; ++c) dz[c] = Mma32<T>::run(ga, my_uz[((k * RC + c) * 2 + s2) * 64 + lane], dz[c]);
      }
    }

    // ---- dx rows 4q..4q+3 (+ residual dy); out-of-range stores are dropped
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = a.residual ? dxa[i][j] + dyf[i][j] : dxa[i][j];
      u32x2 o;
      o[0] = pack2<T>(v[0], v[1]);
      o[1] = pack2<T>(v[2], v[3]);
      bstore64(o, rdx, lane_off + toff + i * rowb);
    }
    // ---- dz: gather this wavefront's tile sums; every DZB tiles (and at the end of
    // the run) add the 4 chunk wavefronts in wave order, one partial per group.
    const int slot = (tile - tile0) % DZB;
    const int buf = ((tile - tile0) / DZB) & 1;
#pragma unroll
    for (int c = 0; c < RC; ++c)
#pragma unroll
      for (int i = 0; i < 4; ++i) dzred[buf][wave][slot][c * 256 + (4 * q + i) * 16 + n] = dz[c][i];
    if (slot == DZB - 1 || tile == tile1 - 1) {
      __syncthreads();
      const int tb = t0 - slot * 16;  // first row of the batch
      for (int e = threadIdx.x; e < (slot + 1) * RC * 256; e += 256) {
        const int sl = e / (RC * 256), rem = e - sl * (RC * 256);
        const int c = rem >> 8, rr = (rem >> 4) & 15, nn = rem & 15;
        const int r = 16 * c + nn;
        const int t = tb + sl * 16 + rr;
        const float v = ((dzred[buf][0][sl][rem] + dzred[buf][1][sl][rem]) + dzred[buf][2][sl][rem]) +
                        dzred[buf][3][sl][rem];
        if (r < R && t < Tn) part_dz[((int64_t)cg * a.BT + row0 + t) * R + r] = v;
      }
    }
  }

  // ---- dU partial of this run: rows r < RK of U_eff, the wavefront's 64 columns per tap
#pragma unroll
  for (int k = 0; k < W; ++k)
#pragma unroll
    for (int c = 0; c < RC; ++c)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 16 * c + 4 * q + i;
          if (r < RK && chv) part_du[((int64_t)sg * RK + r) * WD + (int64_t)k * D + col + j] = du[k][c][j][i];
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

LrBwdArgs make_bwd_args(const LrProblem& p, int target_waves) {
  LrBwdArgs a;
  a.Tn = (int)p.T;
  a.D = (int)p.D;
  a.R = (int)p.R;
  a.RK = (int)p.R + (p.static_w ? 1 : 0);
  a.residual = p.residual;
  a.nch = (int)((p.D + 63) / 64);
  a.ncg = (a.nch + 3) / 4;
  const int64_t ntile = (p.T + 15) / 16;
  int64_t seg = (p.B * ntile * a.ncg * 4 + target_waves - 1) / target_waves;
  if (seg < 1) seg = 1;
  if (seg > ntile) seg = ntile;
  a.seg = (int)seg;
  a.nspb = (int)((ntile + seg - 1) / seg);
  a.nseg = (int)(p.B * a.nspb);
  a.nblk = a.nseg * a.ncg;
  a.BT = p.B * p.T;
  return a;
}

constexpr int kBwdTargetWaves = 2048;

// Workspace: [dz partials: ncg x BT x R fp32][dU partials: nseg x RK x W*D fp32], 256-byte aligned.
struct BwdWs {
  int64_t dz_off, du_off, total;
};
BwdWs bwd_ws(const LrProblem& p, const LrBwdArgs& a) {
  BwdWs w;
  const int64_t dz = (int64_t)a.ncg * a.BT * a.R * 4;
  w.dz_off = 0;
  w.du_off = (dz + 255) / 256 * 256;
  w.total = w.du_off + (int64_t)a.nseg * a.RK * p.W * p.D * 4;
  return w;
}

template <typename T, int W, int RC>
hipError_t launch_bwd(const LrProblem& p) {
  const LrBwdArgs a = make_bwd_args(p, kBwdTargetWaves);
  const BwdWs w = bwd_ws(p, a);
  float* pdz = (float*)((char*)p.ws + w.dz_off);
  float* pdu = (float*)((char*)p.ws + w.du_off);
  lr_bwd_mfma<T, W, RC><<<a.nblk, 256, 0, p.stream>>>((const T*)p.x, (const T*)p.z, (const T*)p.U,
                                                       (const T*)p.static_w, (const T*)p.dy, (T*)p.dx, pdz, pdu, a);
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

template <typename T>
hipError_t dispatch_bwd(const LrProblem& p) {
  const int rc = (int)((p.R + (p.static_w ? 1 : 0) + 15) / 16);
#define DC_LR_CASE(WW, CC) \
  if (p.W == WW && rc == CC) return launch_bwd<T, WW, CC>(p);
  DC_LR_CASE(1, 1) DC_LR_CASE(1, 2) DC_LR_CASE(1, 3) DC_LR_CASE(1, 4)
  DC_LR_CASE(2, 1) DC_LR_CASE(2, 2) DC_LR_CASE(2, 3)
  DC_LR_CASE(3, 1) DC_LR_CASE(3, 2)
  DC_LR_CASE(4, 1) DC_LR_CASE(4, 2)
  DC_LR_CASE(5, 1) DC_LR_CASE(6, 1) DC_LR_CASE(7, 1) DC_LR_CASE(8, 1)
#undef DC_LR_CASE
  return hipErrorInvalidValue;
}

bool aligned8(const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 7) == 0; }

}  // namespace

bool lr_mfma_ok_impl(const LrProblem& p, bool bwd) {
  if (p.dtype != kBF16 && p.dtype != kFP16) return false;
  if (p.W < 1 || p.W > 8) return false;
  const int64_t rc = (p.R + (p.static_w ? 1 : 0) + 15) / 16;
  if (rc > 4 || p.W * rc > 8) return false;  // staged operands / accumulators bound W*RC
  if (bwd && rc == 4 && p.W > 1) return false;  // backward LDS (operands + dz sums) above 160 KiB
  if (!bwd) {
    if (p.D % 8 != 0) return false;
    return aligned16(p.x) && aligned16(p.U) && aligned16(p.static_w) && aligned16(p.y);
  }
  if (p.D % 16 != 0) return false;
  if (p.T * p.D * 2 > kMaxSeqBytes) return false;  // buffer-offset range of one sequence
  return aligned8(p.x) && aligned8(p.dy) && aligned8(p.dx) && aligned16(p.U) && aligned16(p.static_w);
}

int64_t lr_mfma_ws_bytes(const LrProblem& p) { return bwd_ws(p, make_bwd_args(p, kBwdTargetWaves)).total; }

hipError_t lr_mfma_fwd(const LrProblem& p) {
  return p.dtype == kBF16 ? dispatch_fwd<bf16>(p) : dispatch_fwd<fp16>(p);
}

hipError_t lr_mfma_bwd(const LrProblem& p) {
  return p.dtype == kBF16 ? dispatch_bwd<bf16>(p) : dispatch_bwd<fp16>(p);
}

}  // namespace dc
