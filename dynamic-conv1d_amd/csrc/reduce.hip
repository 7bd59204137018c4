// Deterministic cross-workgroup reduction of fp32 partial sums.
//
// The backward kernels write one fp32 partial per workgroup for quantities
// that sum over the batch and time axes (dstatic_w, dU) or over channel
// groups (dz).  The reference accumulates those with relaxed fp32 atomics
// (headwise.py:157-159, lowrank.py:136-137), so its results vary run to run;
// here every column is summed in a fixed order, then rounded once to the
// output dtype.
#include "dc_common.h"
#include "dc_launch.h"

namespace dc {

// 1024 threads: 64 columns x 16 partial lanes.  Lane pl sums partials
// pl, pl+16, ...; the 16 lane sums are then added in index order.
template <typename T>
__global__ __launch_bounds__(1024) void reduce_partials_kernel(const float* __restrict__ part, int64_t pstride,
                                                               int P, int64_t C, T* __restrict__ out) {
  __shared__ float red[16][65];
  const int cl = threadIdx.x & 63;
  const int pl = threadIdx.x >> 6;
  const int64_t c = (int64_t)blockIdx.x * 64 + cl;
  float s = 0.f;
  if (c < C) {
    const float* q = part + c;
    for (int p = pl; p < P; p += 16) s += q[(int64_t)p * pstride];
  }
  red[pl][cl] = s;
  __syncthreads();
  if (pl == 0 && c < C) {
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) t += red[i][cl];
    out[c] = (T)t;
  }
}

hipError_t reduce_partials(const float* part, int64_t pstride, int P, int64_t C, void* out, int dtype,
                           hipStream_t stream) {
  if (C <= 0) return hipSuccess;
  const unsigned grid = (unsigned)((C + 63) / 64);
  switch (dtype) {
    case kBF16:
      reduce_partials_kernel<bf16><<<grid, 1024, 0, stream>>>(part, pstride, P, C, (bf16*)out);
      break;
    case kFP16:
      reduce_partials_kernel<fp16><<<grid, 1024, 0, stream>>>(part, pstride, P, C, (fp16*)out);
      break;
    default:
      reduce_partials_kernel<float><<<grid, 1024, 0, stream>>>(part, pstride, P, C, (float*)out);
      break;
  }
  return hipGetLastError();
}

}  // namespace dc
