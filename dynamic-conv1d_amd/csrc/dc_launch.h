// Internal host-side launch interface between the C ABI (capi.cpp) and the
// kernel translation units.  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dc {

enum DType { kBF16 = 0, kFP16 = 1, kFP32 = 2 };

inline int dtype_size(int dt) { return dt == kFP32 ? 4 : 2; }

// ---------------------------------------------------------------- headwise
struct HwProblem {
  const void* x;
  const void* weight;
  const void* static_w;  // may be null
  const void* dy;        // bwd only
  void* y;               // fwd output
  void* dx;
  void* dweight;
  void* dstatic_w;       // may be null
  float* ws;             // bwd partials (may be null when no static filter)
  int64_t B, T, D, H, W;
  int dtype;
  int residual;
  hipStream_t stream;
};

// Shape/alignment test for the vectorised kernels.  Pure host logic.
bool hw_fast_ok(const HwProblem& p, bool bwd);
// Bytes of fp32 partials the backward needs (0 without a static filter).
int64_t hw_bwd_ws_bytes(const HwProblem& p);
// dc_path code of the kernels hw_fwd / hw_bwd run for p.
int hw_path(const HwProblem& p, bool bwd);
hipError_t hw_fwd(const HwProblem& p);
hipError_t hw_bwd(const HwProblem& p);

// ----------------------------------------------------------------- lowrank
struct LrProblem {
  const void* x;
  const void* z;
  const void* U;
  const void* static_w;  // may be null: then the kernel rank is R, else R + 1
  const void* dy;
  void* y;
  void* dx;
  void* dz;
  void* dU;
  void* dstatic_w;
  float* ws;
  // Padded z_eff [B*T, RP] of z's type (RP = lr_bwd_zrow), or null: the forward
  // writes it, the backward reads it instead of building it (lowrank only).
  void* zeff;
  int64_t B, T, D, R, W;  // R = dynamic rank (z.shape[-1])
  int64_t x_ld;           // row stride of x in elements (0: D, contiguous)
  int64_t dx_ld;          // row stride of dx in elements (0: D, contiguous)
  // Layout of y (forward) and dy (backward): 0 or D for [B, T, D]; otherwise
  // the head dim hd of the head-major layout [B, D/hd, T, hd] (D % hd == 0),
  // in which element (b, t, d) sits at b*T*D + (d/hd)*T*hd + t*hd + d%hd.
  int64_t y_hd;
  int dtype;
  int residual;
  hipStream_t stream;
  // A forward pass over taps kofs .. kofs+W-1 of a wider problem (the
  // matrix-core forward above W 16): U's row stride in elements (0: W*D; U and
  // static_w then point at tap kofs), and accy: add to the y an earlier pass
  // stored.
  int64_t u_ld;
  int kofs;
  int accy;
  // z's row stride in elements (0: R): a pass over kernel ranks rofs .. of a
  // wider problem reads z from column rofs of rows z_ld apart (fp32 forward)
  int64_t z_ld;
  // Ranks per row of zeff (0: those of this problem, lr_zeff_rows): a forward
  // pass over some of a wider problem's taps writes the whole problem's rows.
  int64_t zeff_rp;
  int64_t xld() const { return x_ld > 0 ? x_ld : D; }
  int64_t uld() const { return u_ld > 0 ? u_ld : W * D; }
  int64_t zld() const { return z_ld > 0 ? z_ld : R; }
  int64_t dxld() const { return dx_ld > 0 ? dx_ld : D; }
  int64_t yhd() const { return y_hd > 0 ? y_hd : D; }
};

// Independent problems launched together (the q / k / v convolutions of one
// layer): every group shares B, T, D, R, W, dtype, residual, the presence of
// static_w and the x / dx row strides; pointers differ.  The backward's
// workspace is G consecutive per-group workspaces.
constexpr int kMaxGroups = 4;

bool lr_mfma_ok(const LrProblem& p, bool bwd);
// dc_path code of the kernels lr_fwd / lr_bwd run for one problem p.
int lr_path(const LrProblem& p, bool bwd);
int64_t lr_bwd_ws_bytes(const LrProblem& p);
// Bytes of the padded z_eff the MFMA backward builds for p (0: it reads z itself).
int64_t lr_zeff_bytes(const LrProblem& p);
hipError_t lr_fwd(const LrProblem* p, int G);
hipError_t lr_bwd(const LrProblem* p, int G);

// ---------------------------------------------------------------- proj_in
// z = pre_z W_in^T and its backward (proj_in.hip): pre_z [M, K], W_in [G*R, K],
// z / dz as G tensors [M, R] (group g holds ranks g*R .. g*R+R-1).
struct ProjProblem {
  const void* pre_z;
  const void* w_in;
  void* z[kMaxGroups];         // forward outputs
  const void* dz[kMaxGroups];  // backward inputs
  void* dpre_z;
  void* dw_in;
  float* ws;                   // backward: dW_in partials
  int64_t G, M, K, R;
  int dtype;
  hipStream_t stream;
};
bool proj_shape_ok(const ProjProblem& p);
int64_t proj_bwd_ws_bytes(const ProjProblem& p);
hipError_t proj_fwd_launch(const ProjProblem& p);
hipError_t proj_bwd_launch(const ProjProblem& p);

// ------------------------------------------------------------ range audit
// dc_lowrank_plan_ranges: while a RangeAudit is installed on the calling
// thread, the lowrank launch functions record, for every kernel launch of the
// plan, the byte count each buffer resource of that kernel gets (before
// make_rsrc's clamp, from the same functions the kernels call) with the bound
// it must stay within, and launch nothing (no HIP call is made).  Per-run
// resources are recorded for the longest run (from row 0).
struct RangeAudit {
  int64_t* out;  // pairs (bytes, bound): the count must lie in [0, bound]
  int64_t cap;   // pairs out can hold
  int64_t n;     // pairs recorded (counted past cap too)
};
extern thread_local RangeAudit* g_range_audit;
inline bool auditing() { return g_range_audit != nullptr; }
inline void audit_range(int64_t bytes, int64_t bound) {
  RangeAudit* a = g_range_audit;
  if (a->n < a->cap) {
    a->out[2 * a->n] = bytes;
    a->out[2 * a->n + 1] = bound;
  }
  ++a->n;
}

// ------------------------------------------------------------------ shared
// out[c] = (T) sum_{p < P} part[p * pstride + c] for c < C, summed in a fixed
// order (deterministic).
hipError_t reduce_partials(const float* part, int64_t pstride, int P, int64_t C, void* out, int dtype,
                           hipStream_t stream);

// Up to kMaxReduceJobs such reductions in one launch (jobs with C <= 0 are skipped).
constexpr int kMaxReduceJobs = 3 * kMaxGroups;
struct PartialReduce {
  const float* part;
  int64_t pstride;
  int P;
  int64_t C;
  void* out;
};
hipError_t reduce_partials_multi(const PartialReduce* r, int n, int dtype, hipStream_t stream);

}  // namespace dc
