// Lowrank dynamic convolution on gfx950 matrix cores (bf16 / fp16).
//
//   Kw[t, k, d] = sum_r z_eff[t, r] * U_eff[r, k*D + d]      (MFMA, fp32 accumulate)
//   y[t, d]     = sum_k Kw[t, k, d] * x[t-k, d]  (+ x[t, d])
//
// z_eff / U_eff are z / U extended by the static filter as rank R with
// z == 1 and U row = static_w (the reference's fusion, lowrank.py:223-225),
// and by zero ranks up to a multiple of 16; neither is materialised.
//
// Shared device helpers of the MFMA kernels (lowrank_mfma_fwd_kernel.h,
// lowrank_mfma_bwd.hip): operand types, buffer resources, the z_eff loader.
#pragma once

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

// Buffer resources (dc_common.h) of the matrix-core lowrank kernels cover one
// run of tiles: they start at the run's base row rb = max(16 * tile0 - 32, 0)
// (the first tile's rows less a 32-row halo: the look-back of kofs + W - 1 <= 31
// rows of a pass of taps kofs .. kofs+W-1, W <= 32) and end at T, capped
// at kMaxSeqBytes - kSeqSlackRows rows (run_rsrc).  Rows before 0 (negative
// offsets wrap to large unsigned values), rows past T and channels past D
// (lane offset kOobLane) read 0 and drop stores, without branches or clamped
// addresses.  The host caps a run at lr_max_run_tiles, so every row a run
// touches (its tiles, the halo, the tile after it) lies below that cap: offsets
// stay within int32, and kOobTile, kOobTile less the halo and kOobLane are out
// of range.  A sequence of any length therefore takes these kernels.
constexpr int kOobLane = 0x40000000;
constexpr int64_t kMaxSeqBytes = int64_t(1) << 29;
constexpr int kSeqSlackRows = 32;

// A byte offset that every buffer access of a run treats as out of range
// (returns 0, touches no memory), also less 15 rows of halo.
constexpr int kOobTile = (int)kMaxSeqBytes;

// First row covered by the buffer resources of a run whose first tile is tile0.
constexpr int kRunHaloRows = 32;
__device__ __forceinline__ int run_base_row(int tile0) { return max(tile0 * 16 - kRunHaloRows, 0); }

// Byte counts of the per-pass (not per-run) buffer resources of the matrix-core
// lowrank kernels, as the kernels compute them; the host audit
// (dc_lowrank_plan_ranges) evaluates the same functions over every pass of a
// launch plan.  U rows from tap kofs of a pass of R dynamic ranks (rows uld
// elements apart, the pointer at row 0, tap kofs): R rows end kofs * D
// elements before R * uld; none when R == 0 (a pass of the static rank alone).
__host__ __device__ inline int64_t lr_u_bytes(int R, int64_t uld, int kofs, int64_t D, int es) {
  return R > 0 ? ((int64_t)R * uld - (int64_t)kofs * D) * es : 0;
}
// static_w from tap kofs: the pass's W taps of D elements (none without the static rank).
__host__ __device__ inline int64_t lr_sw_bytes(bool has, int W, int64_t D, int es) {
  return has ? (int64_t)W * D * es : 0;
}
// One dU partial of the backward from its pass's first rank row and tap kofs:
// RK rows of uld floats, less the kofs * D columns before the pointer.
__host__ __device__ inline int64_t lr_dupart_bytes(int RK, int64_t uld, int kofs, int64_t D) {
  return ((int64_t)RK * uld - (int64_t)kofs * D) * 4;
}
// A run resource (run_rsrc): nrows rows of rowb bytes, capped.
__host__ __device__ inline int64_t run_rsrc_bytes(int64_t nrows, int64_t rowb) {
  const int64_t bytes = nrows * rowb, cap = kMaxSeqBytes - kSeqSlackRows * rowb;
  return bytes < cap ? bytes : cap;
}

// Resource over rows [rb, rb + nrows) of `rowb` bytes each, starting at p (row
// rb), capped so that kOobTile less 15 rows stays out of range.
__device__ __forceinline__ rsrc_t run_rsrc(const void* p, int64_t nrows, int64_t rowb) {
  return make_rsrc(p, run_rsrc_bytes(nrows, rowb));
}

// A operands of a 16-row tile: z_eff[t, 16c+4q .. 16c+4q+3] for c < RC, where
// t is the lane's row (column n of the MFMA's A).  Split in two so the loads can
// stay in flight: ZRaw::load issues them without branches or uses of the
// results (vmcnt retires in order, so any use of a just-loaded value would also
// wait for every load issued before it), ZRaw::finish forms the operands once
// they are needed.  ZV (R % 4 == 0, z 8-byte aligned): one 8-byte load per rank
// chunk, whose four ranks are all dynamic or all not.  Otherwise (the forward
// only: the backward reads a padded z_eff copy instead), at two or five to
// eight rank chunks (ZW), one 8-byte load per rank chunk at the row's own
// 2-byte alignment (gfx950 under HSA serves unaligned vector memory accesses)
// that ends at rank min(r0 + 4, R), so it never reads past the row's R ranks,
// shifted into place by finish; else 2-byte element loads.  B4 T4096 D2048 W4
// forward against 2-byte loads: R31 + static without z_eff 33.6 -> 31.6 us,
// configs[4] 60.4 -> 59.5 us per call (58.8 -> 57.2 without z_eff), R95 +
// static 58.7 -> 50.7 us, R127 + static 73.8 -> 68.4 us; slower at one rank
// chunk (R15 + static 30.4 -> 33.3 us), three (R47 + static 40.9 -> 41.8 us)
// and four (R63 + static 45.4 -> 48.9 us), which keep the 2-byte loads.
// Ranks >= R load nothing (out-of-range offset); finish sets the static rank R
// (inside the sequence) to 1 and ranks beyond to 0.  `base` is the z byte
// offset of row t, or kOobTile for a tile that does not exist.
template <typename T, int RC, bool ZV>
struct ZRaw {
  // unaligned 8-byte windows (two, or five to eight, rank chunks) or 2-byte elements
  static constexpr bool ZW = RC == 2 || RC > 4;
  u32x2 v[ZV ? RC : 1];
  uint32_t e[ZV ? 1 : RC][ZV ? 1 : (ZW ? 2 : 4)];

  __device__ __forceinline__ void load(rsrc_t rz, int base, int R, int q) {
#pragma unroll
    for (int c = 0; c < RC; ++c) {
      const int r0 = 16 * c + 4 * q;
      if constexpr (ZV) {
        v[c] = bload64(rz, r0 < R ? base + r0 * 2 : kOobTile);
      } else if constexpr (ZW) {
        // R >= 16 (RC - 1): every chunk but the last holds dynamic ranks only
        const int s = c < RC - 1 || r0 + 4 <= R ? r0 : R - 4;  // the 4 ranks ending at min(r0 + 4, R)
        const u32x2 w = bload64(rz, c < RC - 1 || r0 < R ? base + s * 2 : kOobTile);
        e[c][0] = w[0];
        e[c][1] = w[1];
      } else {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) e[c][kk] = bload16(rz, r0 + kk < R ? base + (r0 + kk) * 2 : kOobTile);
      }
    }
  }
  __device__ __forceinline__ void finish(u32x2 (&za)[RC], int t, int R, int RK, int Tn, int q) const {
    const uint32_t one = (uint32_t)Mma16<T>::kOne;
#pragma unroll
    for (int c = 0; c < RC; ++c) {
      const int r0 = 16 * c + 4 * q;
      if constexpr (ZV) {
        // r0 == R < RK: the static rank opens this chunk
        const uint32_t s = (r0 == R && R < RK && t < Tn) ? one : 0u;
        za[c][0] = r0 < R ? v[c][0] : s;
        za[c][1] = r0 < R ? v[c][1] : 0u;
      } else if constexpr (ZW) {
        // m dynamic ranks in the group: when 0 < m < 4 the load holds ranks
        // R-4 .. R-1, so ranks r0 .. R-1 are its last m elements; they move to
        // the front, the static rank takes element m, zeros follow
        const int m = c < RC - 1 ? 4 : R - r0;
        const uint32_t e0 = e[c][0], e1 = e[c][1];
        const uint32_t st = (R < RK && t < Tn) ? one : 0u;
        const uint32_t mid = __builtin_amdgcn_alignbit(e1, e0, 16);  // elements 1, 2
        const uint32_t top = (e1 >> 16) | (st << 16);                // element 3, static
        uint32_t lo = e0, hi = e1;
        if (m < 4) {
          lo = m == 3 ? mid : m == 2 ? e1 : m == 1 ? top : m == 0 ? st : 0u;
          hi = m == 3 ? top : m == 2 ? st : 0u;
        }
        za[c][0] = lo;
        za[c][1] = hi;
      } else {
        uint32_t w[4];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const int r = r0 + kk;
          w[kk] = r < R ? (e[c][kk] & 0xFFFFu) : ((r < RK && t < Tn) ? one : 0u);
        }
        za[c][0] = w[0] | (w[1] << 16);
        za[c][1] = w[2] | (w[3] << 16);
      }
    }
  }
};

// dx of the backward over all kernel ranks in one launch (lowrank_mfma_dx.hip;
// the passes of ranks then form dz and dU only).
template <typename T>
hipError_t lr_dx_mfma_launch(const LrProblem* p, int G);

inline bool aligned_to(const void* p, int a) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Longest run (in 16-row tiles) whose rows fit the resource cap when rows are
// `rowb` bytes: the run's tiles, the halo, the tile after it and the slack
// rows.  0 when not even one tile fits.
inline int64_t run_tiles_cap(int64_t rowb) {
  const int64_t rows = kMaxSeqBytes / (rowb > 0 ? rowb : 1) - kSeqSlackRows - kRunHaloRows - 32;
  return rows > 0 ? rows / 16 : 0;
}

// The backward runs passes of 32 kernel ranks on the two-rank-chunk kernels
// above kernel rank 64, from W 2 on at kernel ranks 49-64 (four rank chunks
// hold the operands of one tap per pass) and from W 3 on at 33-48 (three rank
// chunks hold two taps per pass, at one wavefront per SIMD): B4 T4096 D2048
// backward R63 + static W4 327 -> 160 us (two passes of 32 + 32 ranks, 4 taps
// each, instead of four), R47 + static W4 171 -> 146 us, W8 369 -> 296 us.  At
// W 2 the one three-chunk pass stays (R47 + static: 78 us against 130 us).
inline bool lr_bwd_rank_split(int64_t RK, int64_t W) {
  return RK > 64 || (RK > 48 && W >= 2) || (RK > 32 && W >= 3);
}

// Ranks per row of the backward's padded z_eff copy: with passes of 32 ranks
// a multiple of 32 (each pass reads 32 of a row's ranks, 16 bytes per lane),
// else 32 for two rank chunks (17 <= RK <= 32) or RK rounded up to 4.
inline int64_t lr_bwd_zrow(int64_t R, bool has_static, int64_t W) {
  const int64_t rk = R + (has_static ? 1 : 0);
  if (lr_bwd_rank_split(rk, W)) return (rk + 31) / 32 * 32;
  return rk > 16 && rk <= 32 ? 32 : (rk + 3) / 4 * 4;
}
// Ranks per row of a problem's z_eff (a forward pass of taps: the whole problem's).
inline int64_t lr_zeff_rows(const LrProblem& p) {
  return p.zeff_rp > 0 ? p.zeff_rp : lr_bwd_zrow(p.R, p.static_w != nullptr, p.W);
}

// Largest kernel rank (R + static) of the matrix-core kernels: above 64 they
// run as passes of ranks.
constexpr int kLrMfmaMaxRank = 256;

// Field f of group g's entry in a kernel-argument table, by selects on the
// wave-uniform g (no dynamic indexing of the argument block).
template <class S, class F>
__device__ __forceinline__ F pick(const S (&a)[kMaxGroups], int g, F S::*f) {
  static_assert(kMaxGroups == 4, "pick() selects among four groups");
  return g == 0 ? a[0].*f : g == 1 ? a[1].*f : g == 2 ? a[2].*f : a[3].*f;
}

// Longest run (16-row tiles) of the MFMA forward / backward for p whose rows
// fit the buffer resources (0: not even one tile; the generic kernels take p).
int64_t lr_fwd_max_run_tiles(const LrProblem& p);
int64_t lr_bwd_max_run_tiles(const LrProblem& p);

// Passes of the matrix-core forward (lowrank_mfma_fwd.hip, fwd_plan): kernel
// ranks rofs .. rofs+RK-1 (R of them dynamic) and taps kofs .. kofs+W-1;
// accy: add to the y the earlier passes stored.  Above fwd_rank_pass(W)
// kernel ranks the ranks run as passes of that many.  lr_mfma_ok admits at
// most kFwdMaxPasses passes: y is rounded to the output type after each.
struct FwdPass {
  int rofs, R, RK, kofs, W;
  bool accy;
};
// Kernel ranks per forward pass: 128 up to W 4 (the W x 8 staged operand
// chunks take up to 128 KiB of LDS, on 8-wavefront workgroups), else 64.
constexpr int fwd_rank_pass(int W) { return W <= 4 ? 128 : 64; }
constexpr int kFwdMaxPasses = 4;
constexpr int kFwdMaxPlan = 64;  // room for every W <= 32, kernel rank <= 256 plan (rejected past kFwdMaxPasses)
int fwd_plan(const LrProblem& p, FwdPass* out);  // number of passes, or -1
int lr_fwd_npasses(const LrProblem& p);

// Passes of the matrix-core backward (lowrank_mfma_bwd.hip, bwd_plan): kernel
// ranks rofs .. rofs+RK-1 (R dynamic) and taps kofs .. kofs+W-1, dz partials in
// slot `slot`.  Where lr_bwd_rank_split holds the ranks run as passes of 32.
struct BwdPass {
  int rofs, R, RK, kofs, W, slot;
};
constexpr int kBwdMaxPlan = 8 * 32;  // kernel rank 256 (8 passes of ranks) x W 32 (up to 32 passes of taps)
int bwd_plan(const LrProblem& p, BwdPass* out);  // number of passes, or -1

// Host entry points of the two MFMA translation units.
hipError_t lr_mfma_fwd(const LrProblem* p, int G);
// Writes each group's z_eff (p[g].zeff, RP = lr_bwd_zrow ranks per row) from z:
// the forward's copy for the backward when the MFMA forward does not write it.
hipError_t lr_zeff_fill(const LrProblem* p, int G);
int64_t lr_mfma_ws_bytes(const LrProblem& p);
hipError_t lr_mfma_bwd(const LrProblem* p, int G);
// fp32 on matrix cores (lowrank_f32_mfma.hip), one problem per launch sequence.
bool lr_f32m_fwd_ok(const LrProblem& p);
hipError_t lr_f32m_fwd(const LrProblem& p);
bool lr_f32m_bwd_ok(const LrProblem& p);
int64_t lr_f32m_ws_bytes(const LrProblem& p);
hipError_t lr_f32m_bwd(const LrProblem& p);
// fp32 VALU kernels (lowrank_f32.hip), one problem per launch sequence.
bool lr_f32_ok(const LrProblem& p);
int64_t lr_f32_ws_bytes(const LrProblem& p);
hipError_t lr_f32(const LrProblem& p, bool bwd);

}  // namespace dc
