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

template <typename T, int N>
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
  for (int i = 0; i < NU; ++i) q[i] = u[i];
}

template <int N>
__device__ __forceinline__ void zero_vals(float* v) {
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = 0.f;
}

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

// Sum over aligned groups of `n` lanes (n a power of two, 1..64).
__device__ __forceinline__ float group_sum(float v, int n) {
  for (int m = 1; m < n; m <<= 1) v += __shfl_xor(v, m);
  return v;
}

}  // namespace dc
