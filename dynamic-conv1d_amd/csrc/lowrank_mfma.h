// Lowrank dynamic convolution on gfx950 matrix cores (bf16 / fp16).
//
//   Kw[t, k, d] = sum_r z_eff[t, r] * U_eff[r, k*D + d]      (MFMA, fp32 accumulate)
//   y[t, d]     = sum_k Kw[t, k, d] * x[t-k, d]  (+ x[t, d])
//
// z_eff / U_eff are z / U extended by the static filter as rank R with
// z == 1 and U row = static_w (the reference's fusion, lowrank.py:223-225),
// and by zero ranks up to a multiple of 16; neither is materialised.
//
// Shared device helpers of the MFMA kernels (lowrank_mfma_fwd.hip,
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

// Raw buffer resources.  A descriptor covers one sequence ([T, C] elements);
// the hardware returns 0 for loads and drops stores whose VGPR byte offset is
// >= the range, which handles rows before 0 (negative offsets wrap to large
// unsigned values), rows past T and channels past D (lane offset kOobLane)
// without branches or clamped addresses.  The host takes these paths only when
// (T + kSeqSlackRows) rows of a sequence span at most kMaxSeqBytes: every
// offset a kernel forms (rows -7 .. T + 25, plus kOobLane) then stays below
// 2^31, and every wrapped negative offset stays above kMaxSeqBytes.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int kOobLane = 0x40000000;
constexpr int64_t kMaxSeqBytes = int64_t(1) << 29;
constexpr int kSeqSlackRows = 32;
// Cache-policy operand of a buffer store: nontemporal (gfx940 family `nt` bit).
constexpr int kNt = 2;

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 bload128(rsrc_t r, int off) { return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0); }
__device__ __forceinline__ u32x2 bload64(rsrc_t r, int off) { return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0); }
__device__ __forceinline__ uint32_t bload16(rsrc_t r, int off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}
template <bool NT>
__device__ __forceinline__ void bstore64(u32x2 v, rsrc_t r, int off) {
  __builtin_amdgcn_raw_buffer_store_b64(v, r, off, 0, NT ? kNt : 0);
}
template <bool NT>
__device__ __forceinline__ void bstore128(u32x4 v, rsrc_t r, int off) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, NT ? kNt : 0);
}

// A operands of a 16-row tile: z_eff[t, 16c+4q .. 16c+4q+3] for c < RC, where
// t is the lane's row (column n of the MFMA's A).  8-byte loads when R % 4 == 0
// (zvec) and the four ranks are dynamic; otherwise element loads, the static
// rank R as 1 (inside the sequence) and zero ranks beyond.
template <typename T, int RC>
__device__ __forceinline__ void load_za(u32x2 (&za)[RC], rsrc_t rz, int t, int R, int RK, int Tn, int q, bool zvec) {
#pragma unroll
  for (int c = 0; c < RC; ++c) {
    const int r0 = 16 * c + 4 * q;
    if (zvec && r0 + 3 < R) {
      za[c] = bload64(rz, (t * R + r0) * 2);
    } else {
      uint32_t e[4];
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int r = r0 + kk;
        const uint32_t v = bload16(rz, (t * R + min(r, R - 1)) * 2);
        e[kk] = r < R ? v : ((r < RK && t < Tn) ? (uint32_t)Mma16<T>::kOne : 0u);
      }
      za[c][0] = e[0] | (e[1] << 16);
      za[c][1] = e[2] | (e[3] << 16);
    }
  }
}

inline bool aligned_to(const void* p, int a) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Host entry points of the two MFMA translation units.
hipError_t lr_mfma_fwd(const LrProblem& p);
int64_t lr_mfma_ws_bytes(const LrProblem& p);
hipError_t lr_mfma_bwd(const LrProblem& p);

}  // namespace dc
