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

// ------------------------------------------------------- buffer resources
// Raw buffer resources: the hardware checks every lane's byte offset against
// the resource's range, returns 0 for loads and drops stores at or beyond it
// (offsets are unsigned, so a negative offset is out of range too).  Kernels
// use this for rows outside a sequence or run and lanes outside D, which keeps
// loads free of branches: a load under a branch, or one whose result is used
// at once, would make the compiler wait for every load issued before it
// (vmcnt counts in order).
typedef __amdgpu_buffer_rsrc_t rsrc_t;
// Cache-policy operand of a buffer access: nontemporal (gfx940 family `nt` bit).
// Stores of outputs take it.  Loads take it only where one instruction reads
// whole cache lines that nothing reads again soon (full 1 KiB rows of a
// wavefront): measured on a 64 MiB copy, nontemporal loads move 6.0 TB/s
// against 5.5 TB/s for default loads.  Loads whose lines are completed by the
// following instructions (strided per-lane pieces) or re-read as a halo keep
// the default policy: with `nt` those lines are fetched again.
constexpr int kNt = 2;

// Largest byte range a resource is given: 1 GiB.  Every kernel's lane
// out-of-range offset (1 << 30) lies at or past it, and the per-run resources
// stay below 512 MiB, under their row out-of-range offsets (host-capped runs).
// make_rsrc clamps the count into [0, MAX]: a negative count (an empty pass,
// or a slip in an offset) gives an empty range, where an unclamped one would
// wrap to a range of almost 4 GiB that takes the out-of-range offsets in.
// The host plans keep every count inside [0, MAX] anyway; the clamp is the
// backstop, and dc_lowrank_plan_ranges reports the counts for a test to check.
constexpr int64_t kRsrcMaxBytes = int64_t(1) << 30;

__host__ __device__ constexpr int64_t clamp_rsrc_bytes(int64_t bytes, int64_t max_bytes = kRsrcMaxBytes) {
  return bytes < 0 ? 0 : bytes > max_bytes ? max_bytes : bytes;
}

template <int64_t MAX = kRsrcMaxBytes>
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, int64_t bytes) {
  static_assert(MAX > 0 && MAX < (int64_t(1) << 31), "a range the 32-bit record count holds");
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)clamp_rsrc_bytes(bytes, MAX),
                                           0x00020000);
}
// make_rsrc for a base and count that are the same in every lane of the
// wavefront (a row, run or tile of the wavefront), both passed through
// readfirstlane.  The descriptor must sit in scalar registers.  When the
// compiler computes a uniform count on the vector unit (64-bit clamps and
// products do), it cannot prove the result uniform.  It then wraps every
// access through the resource in a readfirstlane loop over the lanes' distinct
// descriptors, and the register allocator has placed copies at the start of
// such a loop's exit block, before exec is restored, where they run with no
// lane enabled (lost values: the fp16 W 16 head-size-1 headwise backward lost
// a dx ring slot that way).  Callers guarantee the uniformity.
template <int64_t MAX = kRsrcMaxBytes>
__device__ __forceinline__ rsrc_t make_rsrc_wave(const void* base, int64_t bytes) {
  static_assert(MAX > 0 && MAX < (int64_t(1) << 31), "a range the 32-bit record count holds");
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32));
  const int n = __builtin_amdgcn_readfirstlane((int)clamp_rsrc_bytes(bytes, MAX));
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), (short)0, n,
                                           0x00020000);
}
template <int POL = 0>
__device__ __forceinline__ u32x4 bload128(rsrc_t r, int off) { return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, POL); }
template <int POL = 0>
__device__ __forceinline__ u32x2 bload64(rsrc_t r, int off) { return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, POL); }
template <int POL = 0>
__device__ __forceinline__ uint32_t bload32(rsrc_t r, int off) { return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, POL); }
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

// ds_read_b64_tr_b16 (gfx950): each lane addresses 8 bytes (four 16-bit
// elements) of LDS; within every group of 16 lanes, lane 4a+e receives as its
// element i the element e read by lane a+4i (a 4x4 transpose of 4-element
// chunks).  p must point into a __shared__ array, 8-byte aligned.
__device__ __forceinline__ u32x2 lds_read_tr16(const void* p) {
  typedef short v4i16 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
  const v4i16 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(p));
  return __builtin_bit_cast(u32x2, v);
}

// Load / store of one unit of A bytes (A = 2, 4, 8, 16) through a buffer resource.
template <int A> struct BufUnit;
template <> struct BufUnit<16> {
  template <int POL = 0>
  __device__ static __forceinline__ u32x4 load(rsrc_t r, int off) { return bload128<POL>(r, off); }
  template <bool NT> __device__ static __forceinline__ void store(u32x4 v, rsrc_t r, int off) { bstore128<NT>(v, r, off); }
};
template <> struct BufUnit<8> {
  template <int POL = 0>
  __device__ static __forceinline__ u32x2 load(rsrc_t r, int off) { return bload64<POL>(r, off); }
  template <bool NT> __device__ static __forceinline__ void store(u32x2 v, rsrc_t r, int off) { bstore64<NT>(v, r, off); }
};
template <> struct BufUnit<4> {
  template <int POL = 0>
  __device__ static __forceinline__ uint32_t load(rsrc_t r, int off) { return bload32<POL>(r, off); }
  template <bool NT> __device__ static __forceinline__ void store(uint32_t v, rsrc_t r, int off) {
    __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, NT ? kNt : 0);
  }
};
template <> struct BufUnit<2> {
  template <int POL = 0>
  __device__ static __forceinline__ uint16_t load(rsrc_t r, int off) {
    return (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, POL);
  }
  template <bool NT> __device__ static __forceinline__ void store(uint16_t v, rsrc_t r, int off) {
    __builtin_amdgcn_raw_buffer_store_b16(v, r, off, 0, NT ? kNt : 0);
  }
};

// Raw<T, N> through a buffer resource: unconditional loads (an out-of-range
// offset reads 0; POL is the cache-policy operand) and stores (an
// out-of-range offset writes nothing).
template <int POL = 0, typename T, int N>
__device__ __forceinline__ void bload_raw(Raw<T, N>& v, rsrc_t r, int off) {
  typedef Raw<T, N> R;
#pragma unroll
  for (int i = 0; i < R::NU; ++i) v.u[i] = BufUnit<R::A>::template load<POL>(r, off + i * R::A);
}
template <typename T, int N, bool NT = false>
__device__ __forceinline__ void bstore_vals(rsrc_t r, int off, const float* in) {
  typedef Raw<T, N> R;
  T e[N];
#pragma unroll
  for (int i = 0; i < N; ++i) e[i] = (T)in[i];  // round-to-nearest-even
  typename R::U u[R::NU];
  __builtin_memcpy(u, e, R::BYTES);
#pragma unroll
  for (int i = 0; i < R::NU; ++i) BufUnit<R::A>::template store<NT>(u[i], r, off + i * R::A);
}

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


}  // namespace dc
