/*
 * dynconv.h -- C ABI of libdynconv.so, the MI355X (gfx950) implementation of
 * the dynamic short-convolution kernels.
 *
 * The reference drives its kernels from Python through Triton launches; each
 * entry point below replaces the launch(es) and host-side tensor plumbing of
 * one autograd direction:
 *
 *   dc_headwise_fwd   <- headwise.py:219-254  (_HeadwiseDynamicConvolutionFn.forward,
 *                                              causal_conv1d_fwd_kernel launch 234-248)
 *   dc_headwise_bwd   <- headwise.py:256-309  (.backward, causal_conv1d_bwd_kernel
 *                                              launch 283-300, dstatic fp32 accumulate
 *                                              and cast 270-275, 304-305)
 *   dc_lowrank_fwd    <- lowrank.py:214-249   (_LowrankDynamicConvolutionFn.forward,
 *                                              static-as-rank fusion 223-225, launch 230-242)
 *   dc_lowrank_bwd    <- lowrank.py:251-299   (.backward, launches 266-292, dU cast and
 *                                              static split 294-299)
 *   dc_lowrank_fwd_grouped, dc_lowrank_bwd_grouped
 *                     <- README.md:57-110 (the QKV usage: three lowrank_dynamic_convolution
 *                                              calls, lowrank.py:302-338, on .contiguous()
 *                                              slices of one fused projection, and the
 *                                              .view(B, T, H, hd).transpose(1, 2) of
 *                                              their outputs, README.md:106-110)
 *
 * Conventions
 *   - Every tensor pointer is a DEVICE pointer to a contiguous row-major array:
 *       x, y, dy, dx        [B, T, D]
 *       weight, dweight     [B, T, H, W]        (headwise; head_size = D / H)
 *       z, dz               [B, T, R]           (lowrank; R = dynamic rank, without static)
 *       U, dU               [R, W * D]          (tap k occupies columns k*D .. k*D+D-1)
 *       static_w, dstatic_w [W, D]              (may be NULL: no static filter)
 *     All tensors of one call share `dtype`.  The grouped lowrank calls read x
 *     (and write dx) as G column slices of one [B, T, x_ld] array.
 *   - Sizes are int64.  Returns DC_OK (0) or a negative dc_status.
 *   - Arguments are validated before any HIP call; nothing is launched on error.
 *   - No call allocates device memory, synchronises, or throws.  Scratch for
 *     the deterministic cross-workgroup reductions of the backward passes is a
 *     caller-provided workspace of at least *_bwd_ws_bytes(...) bytes
 *     (256-byte aligned); its contents on entry do not matter.
 *   - Kernels are enqueued on `stream` (a hipStream_t; NULL = default stream)
 *     of the current HIP device.  Calls are safe from any host thread.
 *   - Results are deterministic: the same inputs give bitwise-identical
 *     outputs run to run (no floating-point atomics).
 */
#ifndef DYNCONV_H_
#define DYNCONV_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DC_ABI_VERSION 7

/* Largest convolution width and (kernel) rank accepted.  Every width up to 32
 * and kernel rank up to 256 runs on the vectorised / row-ring / matrix-core
 * kernels, subject to shape and alignment (dc_headwise_path, dc_lowrank_path
 * name the family); the rest, and every width 33 .. DC_MAX_W, take the generic
 * kernels.  Above kernel rank 64 the lowrank kernels run as passes of ranks
 * (the forward's at most four passes of ranks x taps, since y is rounded after
 * each). */
#define DC_MAX_W 1024
#define DC_MAX_R 256
/* Largest number of problems in one grouped lowrank call. */
#define DC_MAX_GROUPS 4

typedef enum dc_dtype {
  DC_DTYPE_BF16 = 0,
  DC_DTYPE_FP16 = 1,
  DC_DTYPE_FP32 = 2
} dc_dtype;

typedef enum dc_status {
  DC_OK = 0,
  DC_ERR_NULL = -1,        /* a required pointer is NULL                          */
  DC_ERR_SHAPE = -2,       /* a size <= 0, D % H != 0, or a size too large         */
  DC_ERR_DTYPE = -3,       /* dtype is not a dc_dtype                              */
  DC_ERR_UNSUPPORTED = -4, /* W > DC_MAX_W, R(+1) > DC_MAX_R, head_size too large  */
  DC_ERR_WORKSPACE = -5,   /* workspace (or z_eff) NULL or below its size query    */
  DC_ERR_ALIGN = -6,       /* a pointer is not aligned to its element size          */
  DC_ERR_DEVICE = -7,      /* no HIP device available                               */
  DC_ERR_LAUNCH = -8,      /* the HIP runtime rejected a kernel launch              */
  DC_ERR_SCRATCH = -9      /* the problem needs more than DC_NOALLOC_SCRATCH_BYTES  */
} dc_status;

/* Kernel family a call of a given shape runs (dc_headwise_path, dc_lowrank_path). */
typedef enum dc_path {
  DC_PATH_GENERIC = 0,   /* one thread per output element (any shape; slow)        */
  DC_PATH_VECTOR = 1,    /* headwise: 128-bit register-ring kernels                 */
  DC_PATH_MFMA = 2,      /* lowrank bf16 / fp16: matrix-core kernels                */
  DC_PATH_F32_MFMA = 3,  /* lowrank fp32: fp32 matrix-core kernels                  */
  DC_PATH_F32_VALU = 4,  /* lowrank fp32: vector-ALU kernels                        */
  DC_PATH_WIDE = 5,      /* headwise 9 <= W <= 32: row-ring kernels, staged weights */
  DC_PATH_HEAD_MFMA = 6  /* headwise, head sizes 8-64 at 9 <= W <= 32: matrix cores */
} dc_path;

/* DC_ABI_VERSION of the loaded library. */
int dc_abi_version(void);

/* Static, human-readable text for a dc_status value. */
const char* dc_status_string(int status);

/* y = headwise dynamic convolution of x (+ x if residual != 0).
 * Replaces headwise.py:219-254.  static_w may be NULL. */
int dc_headwise_fwd(const void* x, const void* weight, const void* static_w, void* y,
                    int64_t B, int64_t T, int64_t D, int64_t H, int64_t W,
                    int dtype, int residual, void* stream);

/* The dc_path that dc_headwise_fwd (bwd = 0) or dc_headwise_bwd (bwd = 1)
 * takes for these sizes with 256-byte aligned tensors, or a negative
 * dc_status for invalid sizes.  No counterpart in the reference, whose
 * autotuner picks among tile sizes of one kernel (headwise.py:8-23). */
int dc_headwise_path(int64_t B, int64_t T, int64_t D, int64_t H, int64_t W, int dtype, int has_static,
                     int bwd);

/* Workspace bytes needed by dc_headwise_bwd for these sizes (>= 0), or a
 * negative dc_status for invalid sizes. */
int64_t dc_headwise_bwd_ws_bytes(int64_t B, int64_t T, int64_t D, int64_t H, int64_t W,
                                 int dtype, int has_static);

/* dx, dweight and (when static_w != NULL) dstatic_w from dy.
 * Replaces headwise.py:256-309.  static_w and dstatic_w are both NULL or both set. */
int dc_headwise_bwd(const void* x, const void* weight, const void* static_w, const void* dy,
                    void* dx, void* dweight, void* dstatic_w,
                    void* workspace, int64_t ws_bytes,
                    int64_t B, int64_t T, int64_t D, int64_t H, int64_t W,
                    int dtype, int residual, void* stream);

/* dc_headwise_bwd for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc):
 * the same kernels and results, bitwise, with the workspace replaced by a
 * fixed scratch array of DC_NOALLOC_SCRATCH_BYTES that the library holds on
 * every GPU it runs on until the process ends.  No counterpart in the
 * reference.  Returns DC_ERR_SCRATCH when dc_headwise_bwd_ws_bytes(...)
 * exceeds DC_NOALLOC_SCRATCH_BYTES.  Every call on one GPU shares that GPU's
 * array: calls that overlap on one GPU (on different streams, or from several
 * host threads) race; calls ordered on one stream do not.  The array needs no
 * initial contents (each call overwrites what it reads).  Nothing here calls
 * hipMalloc, hipFree or an allocating library routine. */
#define DC_NOALLOC_SCRATCH_BYTES (8 << 20)
int dc_headwise_bwd_noalloc(const void* x, const void* weight, const void* static_w, const void* dy,
                            void* dx, void* dweight, void* dstatic_w,
                            int64_t B, int64_t T, int64_t D, int64_t H, int64_t W,
                            int dtype, int residual, void* stream);

/* Bytes of the padded z_eff (z with the static column and zero ranks, rows of
 * 4*k ranks, or of a multiple of 32 where the backward reads 32 ranks of a row
 * at a time: two rank chunks, passes of 32 ranks) that dc_lowrank_bwd builds before its main kernel for this
 * shape, or 0 when it reads z itself, or a negative dc_status.  A caller that
 * keeps such a buffer from the forward to the backward saves that pass: the
 * forward writes it as a by-product (z_eff of dc_lowrank_fwd) and the backward
 * reads it (z_eff of dc_lowrank_bwd).  No counterpart in the reference, whose
 * forward saves the padded z and concatenated U (lowrank.py:223-225, 244). */
int64_t dc_lowrank_zeff_bytes(int64_t B, int64_t T, int64_t D, int64_t R, int64_t W,
                              int dtype, int has_static);

/* y = lowrank dynamic convolution; the per-token weights z @ U (+ static_w as an
 * implicit extra rank with z == 1) are formed on chip and never written out.
 * Replaces lowrank.py:214-249.  R is the dynamic rank (z.shape[-1]).  z_eff is
 * NULL or a 16-byte aligned buffer of z_eff_bytes >= dc_lowrank_zeff_bytes(...)
 * bytes (DC_ERR_WORKSPACE otherwise), which the forward then fills for the
 * backward; when that size query is 0 the buffer is not used. */
int dc_lowrank_fwd(const void* x, const void* z, const void* U, const void* static_w, void* y,
                   void* z_eff, int64_t z_eff_bytes, int64_t B, int64_t T, int64_t D, int64_t R,
                   int64_t W, int dtype, int residual, void* stream);

/* The dc_path that dc_lowrank_fwd (bwd = 0) or dc_lowrank_bwd (bwd = 1) takes
 * for these sizes with contiguous, 256-byte aligned tensors, or a negative
 * dc_status.  No counterpart in the reference (lowrank.py:14-23, 75-85 and
 * 148-157 autotune tile sizes of one kernel each). */
int dc_lowrank_path(int64_t B, int64_t T, int64_t D, int64_t R, int64_t W, int dtype, int has_static, int bwd);

/* Test hook, no counterpart in the reference: the byte ranges that the
 * matrix-core and fp32 lowrank kernels of dc_lowrank_fwd (bwd = 0) or
 * dc_lowrank_bwd (bwd = 1) give their buffer resources for these sizes (with
 * contiguous, 256-byte aligned tensors), over every pass of the launch plan,
 * as the kernels compute them before clamping: per pass U, static_w and (in
 * the backward) the dU partial; per tensor the range of the longest run.
 * Writes up to max_pairs pairs (bytes, bound) to out, where each count must
 * lie in [0, bound] for every out-of-range offset the kernel uses to stay out
 * of range, and returns the number of pairs (0 for the generic kernels), or a
 * negative dc_status.  Launches nothing and makes no HIP call. */
int64_t dc_lowrank_plan_ranges(int64_t B, int64_t T, int64_t D, int64_t R, int64_t W, int dtype, int has_static,
                               int bwd, int64_t* out, int64_t max_pairs);

/* Workspace bytes needed by dc_lowrank_bwd, or a negative dc_status. */
int64_t dc_lowrank_bwd_ws_bytes(int64_t B, int64_t T, int64_t D, int64_t R, int64_t W,
                                int dtype, int has_static);

/* dx, dz, dU and (when static_w != NULL) dstatic_w from dy, in one pass over
 * x and dy.  Replaces lowrank.py:251-299.  z_eff is NULL or the buffer (of
 * z_eff_bytes, checked as in dc_lowrank_fwd) that dc_lowrank_fwd filled for
 * the same z and static_w presence; its contents are trusted, not checked. */
int dc_lowrank_bwd(const void* x, const void* z, const void* U, const void* static_w,
                   const void* z_eff, int64_t z_eff_bytes, const void* dy, void* dx, void* dz,
                   void* dU, void* dstatic_w,
                   void* workspace, int64_t ws_bytes,
                   int64_t B, int64_t T, int64_t D, int64_t R, int64_t W,
                   int dtype, int residual, void* stream);

/* G (1 .. DC_MAX_GROUPS) lowrank forwards of one shape in one launch, e.g. the
 * q, k and v convolutions of an attention layer.  Group g reads x + g*D, whose
 * rows are x_ld >= G*D elements apart (the column slices of a fused [B, T, G*D]
 * projection, read in place); z, U, y are arrays of G device pointers, each a
 * contiguous tensor as in dc_lowrank_fwd; static_w is NULL (no static filter in
 * any group) or an array of G non-NULL pointers.  Each group's y equals what
 * dc_lowrank_fwd computes for it.  y_hd = 0 writes each y as [B, T, D]; a head
 * dim y_hd > 0 (D % y_hd == 0) writes it head-major, [B, D/y_hd, T, y_hd]
 * contiguous: the layout attention reads.  The values are bitwise those of the
 * [B, T, D] layout when y_hd is a multiple of 64 (fp32) or 8 (bf16 / fp16);
 * other head dims take the generic kernels (same tolerance).  Replaces the
 * three calls of README.md:57-110 (lowrank.py:302-338 each), the .contiguous()
 * copies of their inputs and the head transposes of their outputs.  z_eff is
 * NULL or an array of G buffers of z_eff_bytes each, as z_eff of dc_lowrank_fwd. */
int dc_lowrank_fwd_grouped(int64_t G, const void* x, int64_t x_ld, const void* const* z,
                           const void* const* U, const void* const* static_w, void* const* y,
                           void* const* z_eff, int64_t z_eff_bytes, int64_t y_hd, int64_t B,
                           int64_t T, int64_t D, int64_t R, int64_t W, int dtype, int residual,
                           void* stream);

/* Workspace bytes needed by dc_lowrank_bwd_grouped, or a negative dc_status. */
int64_t dc_lowrank_bwd_grouped_ws_bytes(int64_t G, int64_t B, int64_t T, int64_t D, int64_t R,
                                        int64_t W, int dtype, int has_static);

/* The G backwards of dc_lowrank_fwd_grouped in one pass: group g writes its dx
 * into dx + g*D (rows dx_ld >= G*D elements apart: the gradient of the fused
 * projection, written in place), and dz[g], dU[g] (and dstatic_w[g]) as
 * dc_lowrank_bwd does; dy is an array of G contiguous gradients, [B, T, D]
 * when dy_hd = 0 and head-major [B, D/dy_hd, T, dy_hd] otherwise (the layout
 * of dc_lowrank_fwd_grouped's y_hd).  dstatic_w is NULL exactly when static_w
 * is.  Per group, results are bitwise those of dc_lowrank_bwd (with a head
 * dim: when it is a multiple of 64, else the generic kernels).  Replaces
 * README.md:57-110's three backwards (lowrank.py:251-299 each) and the
 * concatenation of dq, dk, dv.  z_eff is NULL or the array of G buffers (of
 * z_eff_bytes each) that dc_lowrank_fwd_grouped filled. */
int dc_lowrank_bwd_grouped(int64_t G, const void* x, int64_t x_ld, const void* const* z,
                           const void* const* U, const void* const* static_w,
                           const void* const* z_eff, int64_t z_eff_bytes,
                           const void* const* dy, int64_t dy_hd,
                           void* dx, int64_t dx_ld,
                           void* const* dz, void* const* dU, void* const* dstatic_w,
                           void* workspace, int64_t ws_bytes,
                           int64_t B, int64_t T, int64_t D, int64_t R, int64_t W,
                           int dtype, int residual, void* stream);

/* ------------------------------------------------------------- proj_in
 * The lowrank module's upstream projection z = pre_z @ W_in^T (README.md:67,
 * 75: nn.Linear(d_model, R, bias=False) applied to pre_z) and its backward,
 * for G modules at once (the grouped q / k / v module: W_in rows g*R ..
 * g*R+R-1 belong to group g).  pre_z [M, K] (M = B*T, K = d_model), W_in
 * [G*R, K], z and dz: arrays of G tensors [M, R], dpre_z [M, K], dW_in
 * [G*R, K]; bf16 or fp16, fp32 accumulation.  Needs G*R <= 128 and K % 8 == 0
 * (DC_ERR_UNSUPPORTED otherwise, also for fp32: callers use a library GEMM
 * then) and 16-byte aligned pre_z, W_in and dpre_z. */

/* z[g] = (pre_z @ W_in^T)[:, g*R : g*R+R] for g < G. */
int dc_proj_in_fwd(const void* pre_z, const void* w_in, void* const* z, int64_t G, int64_t M, int64_t K,
                   int64_t R, int dtype, void* stream);

/* Workspace bytes needed by dc_proj_in_bwd (fp32 partial sums of dW_in), or a
 * negative dc_status. */
int64_t dc_proj_in_bwd_ws_bytes(int64_t G, int64_t M, int64_t K, int64_t R, int dtype);

/* dpre_z = dz_cat @ W_in and dW_in = dz_cat^T @ pre_z, where dz_cat is the G
 * tensors dz[g] side by side ([M, G*R]), in one pass over pre_z; dW_in is
 * summed in a fixed order (deterministic). */
int dc_proj_in_bwd(const void* pre_z, const void* w_in, const void* const* dz, void* dpre_z, void* dw_in,
                   void* workspace, int64_t ws_bytes, int64_t G, int64_t M, int64_t K, int64_t R, int dtype,
                   void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DYNCONV_H_ */
