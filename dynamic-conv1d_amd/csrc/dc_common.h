// Shared device helpers for the gfx950 dynamic-convolution kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dc {

typedef __bf16 bf16;
typedef _Float16 fp16;

// ---------------------------------------------------------------- raw loads
// Load / store N elements of T that start at an address aligned to the largest
// power of two (<= 16 bytes) dividing N*sizeof(T).  Callers guarantee that
// alignment (checked on the host before a fast-path kernel is chosen).
constexpr int pow2_align(int bytes) {
  return (bytes % 16 == 0) ? 16 : (bytes % 8 == 0) ? 8 : (bytes % 4 == 0) ? 4 : 2;
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <int A> struct Unit;
template <> struct Unit<16> { typedef u32x4 type; };
template <> struct Unit<8> { typedef u32x2 type; };
template <> struct Unit<4> { typedef uint32_t type; };
template <> struct Unit<2> { typedef uint16_t type; };

template <typename T, int N>
__device__ __forceinline__ void load_vals(const T* __restrict__ p, float* out) {
  constexpr int BYTES = N * (int)sizeof(T);
  constexpr int A = pow2_align(BYTES);
  typedef typename Unit<A>::type U;
  constexpr int NU = BYTES / A;
  U u[NU];
  const U* q = reinterpret_cast<const U*>(p);
#pragma unroll
  for (int i = 0; i < NU; ++i) u[i] = q[i];
  T e[N];
  __builtin_memcpy(e, u, BYTES);
#pragma unroll
  for (int i = 0; i < N; ++i) out[i] = (float)e[i];
}

// NT: nontemporal store (`nt`), for outputs written in whole 128-byte lines
// that are not read again by the kernel; partial-line stores keep the default
// policy so the L2 merges them before write-back.
template <typename T, int N, bool NT = false>
__device__ __forceinline__ void store_vals(T* __restrict__ p, const float* in) {
  constexpr int BYTES = N * (int)sizeof(T);
  constexpr int A = pow2_align(BYTES);
  typedef typename Unit<A>::type U;
  constexpr int NU = BYTES / A;
  T e[N];
#pragma unroll
  for (int i = 0; i < N; ++i) e[i] = (T)in[i];  // round-to-nearest-even
  U u[NU];
  __builtin_memcpy(u, e, BYTES);
  U* q = reinterpret_cast<U*>(p);
#pragma unroll
  for (int i = 0; i < NU; ++i) {
    if constexpr (NT)
      __builtin_nontemporal_store(u[i], q + i);
    else
      q[i] = u[i];
  }
}

// N elements of T held as raw load units (no conversion): used to keep
// prefetched rows in flight while the previous rows are being computed.
template <typename T, int N>
struct Raw {
  static constexpr int BYTES = N * (int)sizeof(T);
  static constexpr int A = pow2_align(BYTES);
  typedef typename Unit<A>::type U;
  static constexpr int NU = BYTES / A;
  U u[NU];
  __device__ __forceinline__ void load(const T* __restrict__ p) {
    const U* q = reinterpret_cast<const U*>(p);
#pragma unroll
    for (int i = 0; i < NU; ++i) u[i] = q[i];
  }
  __device__ __forceinline__ void zero() { __builtin_memset(u, 0, sizeof(u)); }
  __device__ __forceinline__ float get(int i) const {
    T e[N];
    __builtin_memcpy(e, u, BYTES);
    return (float)e[i];
  }
  __device__ __forceinline__ void to_float(float* out) const {
    T e[N];
    __builtin_memcpy(e, u, BYTES);
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = (float)e[i];
  }
};

template <int N>
__device__ __forceinline__ void zero_vals(float* v) {
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = 0.f;
}

// Wavefront index within the workgroup, marked wave-uniform for the compiler
// (threadIdx.x >> 6 is, but divergence analysis cannot prove it): values
// derived from it (run, sequence, base addresses, buffer descriptors) then
// live in scalar registers.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// ------------------------------------------------------------- block remap
// The command processor hands workgroup i to XCD (i % 8).  Renumber so that
// each XCD receives one contiguous range of logical blocks: neighbouring
// tiles (which share the W-1 row halo) then meet in the same 4 MB L2.
// Bijective on [0, nblk) for every nblk.
__device__ __forceinline__ int xcd_remap(int bid, int nblk) {
  constexpr int NX = 8;
  const int q = nblk / NX, r = nblk % NX;
  const int xcd = bid % NX, slot = bid / NX;
  return (xcd < r) ? xcd * (q + 1) + slot : r * (q + 1) + (xcd - r) * q + slot;
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of `n` lanes (n a power of two, 1..64), leaving the
// group sum in every lane of the group.  Groups up to 16 lanes use DPP
// (quad_perm xor 1, xor 2, row_half_mirror, row_mirror: each pairs a lane
// with one of the other half of its group); 32 and 64 use ds_bpermute.
__device__ __forceinline__ float group_sum(float v, int n) {
  if (n >= 2) v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
  if (n >= 4) v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
  if (n >= 8) v += dpp_f<0x141>(v);  // row_half_mirror
  if (n >= 16) v += dpp_f<0x140>(v); // row_mirror
  if (n >= 32) v += __shfl_xor(v, 16);
  if (n >= 64) v += __shfl_xor(v, 32);
  return v;
}

}  // namespace dc
