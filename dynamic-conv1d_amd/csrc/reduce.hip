// Deterministic cross-workgroup reduction of fp32 partial sums.
//
// The backward kernels write one fp32 partial per workgroup (or per row run)
// for quantities that sum over the batch and time axes (dstatic_w, dU) or over
// channel groups (dz).  The reference accumulates those with relaxed fp32
// atomics (headwise.py:157-159, lowrank.py:136-137), so its results vary run
// to run; here every column is summed in a fixed order, then rounded once to
// the output dtype.  Up to kMaxJobs reductions share one launch (three per
// lowrank problem: dU, dstatic_w, dz; a grouped launch has up to kMaxGroups).
#include "dc_common.h"
#include "dc_launch.h"

namespace dc {

constexpr int kMaxJobs = kMaxReduceJobs;

struct ReduceJob {
  const float* part;  // partial p, column c at part[p * pstride + c]
  int64_t pstride;
  int64_t C;          // columns
  void* out;          // C outputs of the launch dtype
  int P;              // partials
  int vec;            // 4: columns, pstride and pointers allow float4 access
  int plog;           // log2 of the partial lanes per column (PL = 1 .. 16)
  int block0;         // first block of this job
};

struct ReduceJobs {
  ReduceJob j[kMaxJobs];
  int n;
};

// 256 threads = 256/PL column lanes x PL partial lanes (PL a power of two, so
// each thread adds about 8-16 partials, whose loads are independent and in
// flight together); a column lane owns 4 consecutive columns when `vec`
// (float4 loads), else 1.  Partial lane pl sums partials pl, pl+PL, ... in order; the
// PL lane sums are then added in lane order from LDS.  The order is fixed by
// (P, PL), so results are the same run to run.
template <typename T>
__global__ __launch_bounds__(256) void reduce_partials_kernel(ReduceJobs jobs) {
  __shared__ float4 red[256];
  int ji = 0;
#pragma unroll
  for (int i = 1; i < kMaxJobs; ++i)
    if (i < jobs.n && (int)blockIdx.x >= jobs.j[i].block0) ji = i;
  const ReduceJob& J = jobs.j[ji];
  const int PL = 1 << J.plog, CL = 256 >> J.plog;
  const int cl = threadIdx.x & (CL - 1), pl = threadIdx.x >> (8 - J.plog);
  const int per = J.vec;  // columns per lane
  const int64_t c0 = ((int64_t)(blockIdx.x - J.block0) * CL + cl) * per;
  float4 s = {0.f, 0.f, 0.f, 0.f};
  if (c0 < J.C) {
    const float* q = J.part + c0;
    if (per == 4) {
#pragma unroll 8
      for (int p = pl; p < J.P; p += PL) {
        const float4 v = *reinterpret_cast<const float4*>(q + (int64_t)p * J.pstride);
        s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
      }
    } else {
#pragma unroll 4
      for (int p = pl; p < J.P; p += PL) s.x += q[(int64_t)p * J.pstride];
    }
  }
  red[threadIdx.x] = s;
  __syncthreads();
  if (pl == 0 && c0 < J.C) {
    float4 t = red[cl];
    for (int i = 1; i < PL; ++i) {
      const float4 u = red[i * CL + cl];
      t.x += u.x; t.y += u.y; t.z += u.z; t.w += u.w;
    }
    T* o = reinterpret_cast<T*>(J.out) + c0;
    o[0] = (T)t.x;
    if (per == 4) {
      o[1] = (T)t.y;
      o[2] = (T)t.z;
      o[3] = (T)t.w;
    }
  }
}

// The range audit's hook (dc_lowrank_plan_ranges installs it on its thread).
thread_local RangeAudit* g_range_audit = nullptr;

hipError_t reduce_partials_multi(const PartialReduce* r, int n, int dtype, hipStream_t stream) {
  if (auditing()) return hipSuccess;  // plain pointers: no buffer resources to record
  ReduceJobs jobs{};
  int blocks = 0;
  for (int i = 0; i < n; ++i) {
    if (r[i].C <= 0) continue;
    if (jobs.n == kMaxJobs) return hipErrorInvalidValue;
    ReduceJob& J = jobs.j[jobs.n++];
    J.part = r[i].part;
    J.pstride = r[i].pstride;
    J.C = r[i].C;
    J.out = r[i].out;
    J.P = r[i].P;
    const int es = dtype_size(dtype);
    const bool v4 = (r[i].C % 4 == 0) && (r[i].pstride % 4 == 0) &&
                    (reinterpret_cast<uintptr_t>(r[i].part) % 16 == 0) &&
                    (reinterpret_cast<uintptr_t>(r[i].out) % (4 * es) == 0);
    J.vec = v4 ? 4 : 1;
    // partial lanes: the largest power of two <= P/8, between 1 and 16 (about
    // 8 partials per thread: lowrank backward B4 T4096 D2048 R16 60.2 -> 59.2 us,
    // B2 T8192 D4096 R31+static 158.5 -> 155.1 us, against about 4)
    int plog = 0;
    while (plog < 4 && (8 << (plog + 1)) <= J.P) ++plog;
    J.plog = plog;
    const int64_t cols = (int64_t)(256 >> plog) * J.vec;  // columns per block
    J.block0 = blocks;
    blocks += (int)((J.C + cols - 1) / cols);
  }
  if (jobs.n == 0) return hipSuccess;
  switch (dtype) {
    case kBF16: reduce_partials_kernel<bf16><<<blocks, 256, 0, stream>>>(jobs); break;
    case kFP16: reduce_partials_kernel<fp16><<<blocks, 256, 0, stream>>>(jobs); break;
    default: reduce_partials_kernel<float><<<blocks, 256, 0, stream>>>(jobs); break;
  }
  return hipGetLastError();
}

hipError_t reduce_partials(const float* part, int64_t pstride, int P, int64_t C, void* out, int dtype,
                           hipStream_t stream) {
  const PartialReduce r{part, pstride, P, C, out};
  return reduce_partials_multi(&r, 1, dtype, stream);
}

}  // namespace dc
