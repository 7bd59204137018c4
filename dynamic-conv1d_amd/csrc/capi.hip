// C ABI of libdynconv.so (declared in include/dynconv.h).
//
// Every entry point validates its arguments on the host before touching the
// HIP runtime and returns a dc_status; nothing here allocates, synchronises
// or throws.  The only process-wide state is the once-initialised device
// probe and the per-device address of the allocation-free scratch array below.
#include <atomic>
#include <mutex>

#include "dynconv.h"
#include "dc_launch.h"

namespace {

constexpr int64_t kI32Max = 2147483647;
static_assert(DC_MAX_GROUPS == dc::kMaxGroups, "group table size");

int device_status() {
  static std::once_flag once;
  static int status = DC_OK;
  std::call_once(once, [] {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) status = DC_ERR_DEVICE;
  });
  return status;
}

bool dtype_ok(int dt) { return dt == DC_DTYPE_BF16 || dt == DC_DTYPE_FP16 || dt == DC_DTYPE_FP32; }

bool aligned_to(const void* p, int a) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Shared size checks: positive, indexable with int32 rows/channels and int64
// element offsets.
int check_btd(int64_t B, int64_t T, int64_t D, int64_t W) {
  if (B <= 0 || T <= 0 || D <= 0 || W <= 0) return DC_ERR_SHAPE;
  if (T > kI32Max || D > kI32Max || B > kI32Max || B * T > kI32Max) return DC_ERR_SHAPE;
  if (W > DC_MAX_W) return DC_ERR_UNSUPPORTED;
  return DC_OK;
}

int check_headwise(int64_t B, int64_t T, int64_t D, int64_t H, int64_t W, int dtype) {
  if (!dtype_ok(dtype)) return DC_ERR_DTYPE;
  int s = check_btd(B, T, D, W);
  if (s != DC_OK) return s;
  if (H <= 0 || D % H != 0) return DC_ERR_SHAPE;
  if (W * D > kI32Max) return DC_ERR_SHAPE;  // static_w / dstatic_w columns
  return DC_OK;
}

int check_lowrank(int64_t B, int64_t T, int64_t D, int64_t R, int64_t W, int dtype, bool has_static) {
  if (!dtype_ok(dtype)) return DC_ERR_DTYPE;
  int s = check_btd(B, T, D, W);
  if (s != DC_OK) return s;
  if (R <= 0) return DC_ERR_SHAPE;
  if (R + (has_static ? 1 : 0) > DC_MAX_R) return DC_ERR_UNSUPPORTED;
  if (W * D > kI32Max) return DC_ERR_SHAPE;
  return DC_OK;
}

int launch_status(hipError_t e) { return e == hipSuccess ? DC_OK : DC_ERR_LAUNCH; }

// Scratch of dc_headwise_bwd_noalloc: the fp32 dstatic_w partial sums that
// dc_headwise_bwd keeps in its caller's workspace.  Each GPU holds its own copy
// of this array (at its own address) for the life of the process.  In host
// code `scratch` names a host-side stand-in, not a device address: only the
// address hipGetSymbolAddress returns for the current device is passed on.
static __device__ __align__(256) char scratch[DC_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of the current device's scratch array, looked up once per
// device with that device current.  DC_ERR_DEVICE when there is none.
int scratch_of_current_device(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return DC_ERR_DEVICE;
  void* ptr = g_scratch[dev].load(std::memory_order_acquire);
  if (ptr == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    ptr = g_scratch[dev].load(std::memory_order_relaxed);
    if (ptr == nullptr) {
      if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr) return DC_ERR_DEVICE;
      g_scratch[dev].store(ptr, std::memory_order_release);
    }
  }
  *out = ptr;
  return DC_OK;
}

}  // namespace

extern "C" {

int dc_abi_version(void) { return DC_ABI_VERSION; }

const char* dc_status_string(int status) {
  switch (status) {
    case DC_OK: return "ok";
    case DC_ERR_NULL: return "a required pointer is NULL (or static_w/dstatic_w disagree)";
    case DC_ERR_SHAPE: return "invalid shape (non-positive size, D % H != 0, or size too large)";
    case DC_ERR_DTYPE: return "unsupported dtype";
    case DC_ERR_UNSUPPORTED: return "unsupported configuration (W or rank above the library maximum)";
    case DC_ERR_WORKSPACE: return "workspace (or z_eff buffer) missing or smaller than its size query";
    case DC_ERR_ALIGN: return "pointer not aligned to its element size";
    case DC_ERR_DEVICE: return "no HIP device available";
    case DC_ERR_LAUNCH: return "kernel launch failed";
    case DC_ERR_SCRATCH: return "problem needs more scratch than the allocation-free entry point holds";
    default: return "unknown dynconv status";
  }
}

int dc_headwise_fwd(const void* x, const void* weight, const void* static_w, void* y, int64_t B, int64_t T,
                    int64_t D, int64_t H, int64_t W, int dtype, int residual, void* stream) {
  int s = check_headwise(B, T, D, H, W, dtype);
  if (s != DC_OK) return s;
  if (!x || !weight || !y) return DC_ERR_NULL;
  const int es = dc::dtype_size(dtype);
  if (!aligned_to(x, es) || !aligned_to(weight, es) || !aligned_to(static_w, es) || !aligned_to(y, es))
    return DC_ERR_ALIGN;
  if ((s = device_status()) != DC_OK) return s;
  dc::HwProblem p{};
  p.x = x; p.weight = weight; p.static_w = static_w; p.y = y;
  p.B = B; p.T = T; p.D = D; p.H = H; p.W = W;
  p.dtype = dtype; p.residual = residual ? 1 : 0; p.stream = (hipStream_t)stream;
  return launch_status(dc::hw_fwd(p));
}

static_assert(DC_PATH_GENERIC == 0 && DC_PATH_VECTOR == 1 && DC_PATH_MFMA == 2 && DC_PATH_F32_MFMA == 3 &&
                  DC_PATH_F32_VALU == 4 && DC_PATH_WIDE == 5 && DC_PATH_HEAD_MFMA == 6,
              "dc_path codes returned by hw_path / lr_path");

int dc_headwise_path(int64_t B, int64_t T, int64_t D, int64_t H, int64_t W, int dtype, int has_static, int bwd) {
  int s = check_headwise(B, T, D, H, W, dtype);
  if (s != DC_OK) return s;
  static const char kAligned[16] __attribute__((aligned(256))) = {0};
  dc::HwProblem p{};
  p.x = p.weight = p.dy = kAligned;
  p.dx = p.dweight = p.y = (void*)kAligned;
  p.static_w = has_static ? kAligned : nullptr;
  p.dstatic_w = has_static ? (void*)kAligned : nullptr;
  p.B = B; p.T = T; p.D = D; p.H = H; p.W = W; p.dtype = dtype;
  return dc::hw_path(p, bwd != 0);
}

int64_t dc_headwise_bwd_ws_bytes(int64_t B, int64_t T, int64_t D, int64_t H, int64_t W, int dtype,
                                 int has_static) {
  int s = check_headwise(B, T, D, H, W, dtype);
  if (s != DC_OK) return s;
  // The fast path needs 16-byte aligned tensors; size for it whenever the
  // shape allows it (torch allocations are 256-byte aligned).  A generic-path
  // call never needs more than the fast path's count.
  static const char kAligned[16] __attribute__((aligned(256))) = {0};
  dc::HwProblem p{};
  p.x = p.weight = p.dy = kAligned;
  p.dx = p.dweight = p.y = (void*)kAligned;
  p.static_w = has_static ? kAligned : nullptr;
  p.B = B; p.T = T; p.D = D; p.H = H; p.W = W; p.dtype = dtype;
  int64_t fast = dc::hw_bwd_ws_bytes(p);
  p.x = kAligned + 2;  // force the generic sizing, take the larger of the two
  int64_t gen = dc::hw_bwd_ws_bytes(p);
  return fast > gen ? fast : gen;
}

int dc_headwise_bwd(const void* x, const void* weight, const void* static_w, const void* dy, void* dx,
                    void* dweight, void* dstatic_w, void* workspace, int64_t ws_bytes, int64_t B, int64_t T,
                    int64_t D, int64_t H, int64_t W, int dtype, int residual, void* stream) {
  int s = check_headwise(B, T, D, H, W, dtype);
  if (s != DC_OK) return s;
  if (!x || !weight || !dy || !dx || !dweight) return DC_ERR_NULL;
  if ((static_w == nullptr) != (dstatic_w == nullptr)) return DC_ERR_NULL;
  const int es = dc::dtype_size(dtype);
  if (!aligned_to(x, es) || !aligned_to(weight, es) || !aligned_to(static_w, es) || !aligned_to(dy, es) ||
      !aligned_to(dx, es) || !aligned_to(dweight, es) || !aligned_to(dstatic_w, es))
    return DC_ERR_ALIGN;
  const int64_t need = dc_headwise_bwd_ws_bytes(B, T, D, H, W, dtype, static_w != nullptr);
  if (need < 0) return (int)need;
  if (need > 0 && (workspace == nullptr || ws_bytes < need || !aligned_to(workspace, 16))) return DC_ERR_WORKSPACE;
  if ((s = device_status()) != DC_OK) return s;
  dc::HwProblem p{};
  p.x = x; p.weight = weight; p.static_w = static_w; p.dy = dy;
  p.dx = dx; p.dweight = dweight; p.dstatic_w = dstatic_w; p.ws = (float*)workspace;
  p.B = B; p.T = T; p.D = D; p.H = H; p.W = W;
  p.dtype = dtype; p.residual = residual ? 1 : 0; p.stream = (hipStream_t)stream;
  return launch_status(dc::hw_bwd(p));
}

int dc_headwise_bwd_noalloc(const void* x, const void* weight, const void* static_w, const void* dy, void* dx,
                            void* dweight, void* dstatic_w, int64_t B, int64_t T, int64_t D, int64_t H, int64_t W,
                            int dtype, int residual, void* stream) {
  int s = check_headwise(B, T, D, H, W, dtype);
  if (s != DC_OK) return s;
  if (!x || !weight || !dy || !dx || !dweight) return DC_ERR_NULL;
  if ((static_w == nullptr) != (dstatic_w == nullptr)) return DC_ERR_NULL;
  const int es = dc::dtype_size(dtype);
  if (!aligned_to(x, es) || !aligned_to(weight, es) || !aligned_to(static_w, es) || !aligned_to(dy, es) ||
      !aligned_to(dx, es) || !aligned_to(dweight, es) || !aligned_to(dstatic_w, es))
    return DC_ERR_ALIGN;
  const int64_t need = dc_headwise_bwd_ws_bytes(B, T, D, H, W, dtype, static_w != nullptr);
  if (need < 0) return (int)need;
  if (need > DC_NOALLOC_SCRATCH_BYTES) return DC_ERR_SCRATCH;
  if ((s = device_status()) != DC_OK) return s;
  void* ws = nullptr;
  if (need > 0 && (s = scratch_of_current_device(&ws)) != DC_OK) return s;
  dc::HwProblem p{};
  p.x = x; p.weight = weight; p.static_w = static_w; p.dy = dy;
  p.dx = dx; p.dweight = dweight; p.dstatic_w = dstatic_w; p.ws = (float*)ws;
  p.B = B; p.T = T; p.D = D; p.H = H; p.W = W;
  p.dtype = dtype; p.residual = residual ? 1 : 0; p.stream = (hipStream_t)stream;
  return launch_status(dc::hw_bwd(p));
}

int64_t dc_lowrank_zeff_bytes(int64_t B, int64_t T, int64_t D, int64_t R, int64_t W, int dtype, int has_static) {
  int s = check_lowrank(B, T, D, R, W, dtype, has_static != 0);
  if (s != DC_OK) return s;
  static const char kAligned[16] __attribute__((aligned(256))) = {0};
  dc::LrProblem p{};
  p.x = p.z = p.U = p.dy = kAligned;
  p.y = p.dx = p.dz = p.dU = (void*)kAligned;
  p.static_w = has_static ? kAligned : nullptr;
  p.dstatic_w = has_static ? (void*)kAligned : nullptr;
  p.B = B; p.T = T; p.D = D; p.R = R; p.W = W; p.dtype = dtype;
  return dc::lr_zeff_bytes(p);
}

// z_eff bytes a call needs (dc_lowrank_zeff_bytes; the shape is already valid).
static int64_t zeff_need(int64_t B, int64_t T, int64_t D, int64_t R, int64_t W, int dtype, bool has_static) {
  const int64_t n = dc_lowrank_zeff_bytes(B, T, D, R, W, dtype, has_static);
  return n > 0 ? n : 0;
}

// A caller's z_eff buffer: DC_ERR_WORKSPACE when the shape uses one and the
// buffer is shorter than the size query.
static int zeff_status(const void* z_eff, int64_t z_eff_bytes, int64_t need) {
  return z_eff && need > 0 && z_eff_bytes < need ? DC_ERR_WORKSPACE : DC_OK;
}

// The z_eff buffer a call uses: the caller's when the shape has one, else none.
static void* zeff_of(const void* z_eff, int64_t need) { return z_eff && need > 0 ? const_cast<void*>(z_eff) : nullptr; }

int dc_lowrank_fwd(const void* x, const void* z, const void* U, const void* static_w, void* y, void* z_eff,
                   int64_t z_eff_bytes, int64_t B, int64_t T, int64_t D, int64_t R, int64_t W, int dtype,
                   int residual, void* stream) {
  int s = check_lowrank(B, T, D, R, W, dtype, static_w != nullptr);
  if (s != DC_OK) return s;
  if (!x || !z || !U || !y) return DC_ERR_NULL;
  const int es = dc::dtype_size(dtype);
  if (!aligned_to(x, es) || !aligned_to(z, es) || !aligned_to(U, es) || !aligned_to(static_w, es) ||
      !aligned_to(y, es) || !aligned_to(z_eff, 16))
    return DC_ERR_ALIGN;
  const int64_t zneed = zeff_need(B, T, D, R, W, dtype, static_w != nullptr);
  if ((s = zeff_status(z_eff, z_eff_bytes, zneed)) != DC_OK) return s;
  if ((s = device_status()) != DC_OK) return s;
  dc::LrProblem p{};
  p.x = x; p.z = z; p.U = U; p.static_w = static_w; p.y = y;
  p.zeff = zeff_of(z_eff, zneed);
  p.B = B; p.T = T; p.D = D; p.R = R; p.W = W;
  p.dtype = dtype; p.residual = residual ? 1 : 0; p.stream = (hipStream_t)stream;
  return launch_status(dc::lr_fwd(&p, 1));
}

int dc_lowrank_path(int64_t B, int64_t T, int64_t D, int64_t R, int64_t W, int dtype, int has_static, int bwd) {
  int s = check_lowrank(B, T, D, R, W, dtype, has_static != 0);
  if (s != DC_OK) return s;
  static const char kAligned[16] __attribute__((aligned(256))) = {0};
  dc::LrProblem p{};
  p.x = p.z = p.U = p.dy = kAligned;
  p.y = p.dx = p.dz = p.dU = (void*)kAligned;
  p.static_w = has_static ? kAligned : nullptr;
  p.dstatic_w = has_static ? (void*)kAligned : nullptr;
  p.B = B; p.T = T; p.D = D; p.R = R; p.W = W; p.dtype = dtype;
  return dc::lr_path(p, bwd != 0);
}

int64_t dc_lowrank_plan_ranges(int64_t B, int64_t T, int64_t D, int64_t R, int64_t W, int dtype, int has_static,
                               int bwd, int64_t* out, int64_t max_pairs) {
  int s = check_lowrank(B, T, D, R, W, dtype, has_static != 0);
  if (s != DC_OK) return s;
  if (max_pairs < 0 || (max_pairs > 0 && !out)) return DC_ERR_NULL;
  // 256-byte aligned stand-in addresses: the dispatch only offsets them (nothing
  // is launched or read while the audit is installed)
  static const char kAligned[16] __attribute__((aligned(256))) = {0};
  dc::LrProblem p{};
  p.x = p.z = p.U = p.dy = kAligned;
  p.y = p.dx = p.dz = p.dU = (void*)kAligned;
  p.ws = (float*)kAligned;
  p.static_w = has_static ? kAligned : nullptr;
  p.dstatic_w = has_static ? (void*)kAligned : nullptr;
  p.B = B; p.T = T; p.D = D; p.R = R; p.W = W; p.dtype = dtype; p.residual = 1;
  if (dc::lr_path(p, bwd != 0) == DC_PATH_GENERIC) return 0;  // generic kernels: plain pointers
  dc::RangeAudit audit{out, max_pairs, 0};
  dc::g_range_audit = &audit;
  const hipError_t e = bwd ? dc::lr_bwd(&p, 1) : dc::lr_fwd(&p, 1);
  dc::g_range_audit = nullptr;
  return e == hipSuccess ? audit.n : DC_ERR_LAUNCH;
}

int64_t dc_lowrank_bwd_ws_bytes(int64_t B, int64_t T, int64_t D, int64_t R, int64_t W, int dtype,
                                int has_static) {
  int s = check_lowrank(B, T, D, R, W, dtype, has_static != 0);
  if (s != DC_OK) return s;
  static const char kAligned[16] __attribute__((aligned(256))) = {0};
  dc::LrProblem p{};
  p.x = p.z = p.U = p.dy = kAligned;
  p.y = p.dx = p.dz = p.dU = (void*)kAligned;
  p.static_w = has_static ? kAligned : nullptr;
  p.dstatic_w = has_static ? (void*)kAligned : nullptr;
  p.B = B; p.T = T; p.D = D; p.R = R; p.W = W; p.dtype = dtype;
  int64_t fast = dc::lr_bwd_ws_bytes(p);
  p.x = kAligned + 2;
  int64_t gen = dc::lr_bwd_ws_bytes(p);
  return fast > gen ? fast : gen;
}

int dc_lowrank_bwd(const void* x, const void* z, const void* U, const void* static_w, const void* z_eff,
                   int64_t z_eff_bytes, const void* dy, void* dx, void* dz, void* dU, void* dstatic_w,
                   void* workspace, int64_t ws_bytes, int64_t B, int64_t T, int64_t D, int64_t R, int64_t W,
                   int dtype, int residual, void* stream) {
  int s = check_lowrank(B, T, D, R, W, dtype, static_w != nullptr);
  if (s != DC_OK) return s;
  if (!x || !z || !U || !dy || !dx || !dz || !dU) return DC_ERR_NULL;
  if ((static_w == nullptr) != (dstatic_w == nullptr)) return DC_ERR_NULL;
  const int es = dc::dtype_size(dtype);
  if (!aligned_to(x, es) || !aligned_to(z, es) || !aligned_to(U, es) || !aligned_to(static_w, es) ||
      !aligned_to(dy, es) || !aligned_to(dx, es) || !aligned_to(dz, es) || !aligned_to(dU, es) ||
      !aligned_to(dstatic_w, es) || !aligned_to(z_eff, 16))
    return DC_ERR_ALIGN;
  const int64_t need = dc_lowrank_bwd_ws_bytes(B, T, D, R, W, dtype, static_w != nullptr);
  if (need < 0) return (int)need;
  if (need > 0 && (workspace == nullptr || ws_bytes < need || !aligned_to(workspace, 16))) return DC_ERR_WORKSPACE;
  const int64_t zneed = zeff_need(B, T, D, R, W, dtype, static_w != nullptr);
  if ((s = zeff_status(z_eff, z_eff_bytes, zneed)) != DC_OK) return s;
  if ((s = device_status()) != DC_OK) return s;
  dc::LrProblem p{};
  p.x = x; p.z = z; p.U = U; p.static_w = static_w; p.dy = dy;
  p.dx = dx; p.dz = dz; p.dU = dU; p.dstatic_w = dstatic_w; p.ws = (float*)workspace;
  p.zeff = zeff_of(z_eff, zneed);
  p.B = B; p.T = T; p.D = D; p.R = R; p.W = W;
  p.dtype = dtype; p.residual = residual ? 1 : 0; p.stream = (hipStream_t)stream;
  return launch_status(dc::lr_bwd(&p, 1));
}

// ------------------------------------------------------------------ grouped
// G problems of one shape in one launch; group g reads x + g*D with rows
// x_ld elements apart (the q / k / v slices of a fused projection) and, in the
// backward, writes dx + g*D with rows dx_ld elements apart.  y (dy) is
// [B, T, D] when y_hd (dy_hd) is 0, else head-major [B, D/hd, T, hd].

static bool head_dim_ok(int64_t hd, int64_t D) { return hd == 0 || (hd > 0 && hd <= D && D % hd == 0); }

int dc_lowrank_fwd_grouped(int64_t G, const void* x, int64_t x_ld, const void* const* z, const void* const* U,
                           const void* const* static_w, void* const* y, void* const* z_eff, int64_t z_eff_bytes,
                           int64_t y_hd, int64_t B, int64_t T, int64_t D, int64_t R, int64_t W, int dtype,
                           int residual, void* stream) {
  if (G < 1 || G > DC_MAX_GROUPS) return DC_ERR_UNSUPPORTED;
  int s = check_lowrank(B, T, D, R, W, dtype, static_w != nullptr);
  if (s != DC_OK) return s;
  if (x_ld < G * D || x_ld > kI32Max || !head_dim_ok(y_hd, D)) return DC_ERR_SHAPE;
  if (!x || !z || !U || !y) return DC_ERR_NULL;
  const int es = dc::dtype_size(dtype);
  if (!aligned_to(x, es)) return DC_ERR_ALIGN;
  const int64_t zneed = zeff_need(B, T, D, R, W, dtype, static_w != nullptr);
  dc::LrProblem p[DC_MAX_GROUPS] = {};
  for (int64_t g = 0; g < G; ++g) {
    const void* sw = static_w ? static_w[g] : nullptr;
    if (!z[g] || !U[g] || !y[g] || (static_w && !sw) || (z_eff && !z_eff[g])) return DC_ERR_NULL;
    if (!aligned_to(z[g], es) || !aligned_to(U[g], es) || !aligned_to(sw, es) || !aligned_to(y[g], es) ||
        (z_eff && !aligned_to(z_eff[g], 16)))
      return DC_ERR_ALIGN;
    dc::LrProblem& q = p[g];
    q.x = (const char*)x + g * D * es; q.z = z[g]; q.U = U[g]; q.static_w = sw; q.y = y[g];
    q.zeff = z_eff ? zeff_of(z_eff[g], zneed) : nullptr;
    q.B = B; q.T = T; q.D = D; q.R = R; q.W = W; q.x_ld = x_ld; q.y_hd = y_hd;
    q.dtype = dtype; q.residual = residual ? 1 : 0; q.stream = (hipStream_t)stream;
  }
  if (z_eff && (s = zeff_status(z_eff[0], z_eff_bytes, zneed)) != DC_OK) return s;
  if ((s = device_status()) != DC_OK) return s;
  return launch_status(dc::lr_fwd(p, (int)G));
}

// One group's share, rounded up to 256 bytes (each group's partials start aligned).
static int64_t grouped_ws_share(int64_t B, int64_t T, int64_t D, int64_t R, int64_t W, int dtype, int has_static) {
  const int64_t one = dc_lowrank_bwd_ws_bytes(B, T, D, R, W, dtype, has_static);
  return one < 0 ? one : (one + 255) / 256 * 256;
}

int64_t dc_lowrank_bwd_grouped_ws_bytes(int64_t G, int64_t B, int64_t T, int64_t D, int64_t R, int64_t W,
                                        int dtype, int has_static) {
  if (G < 1 || G > DC_MAX_GROUPS) return DC_ERR_UNSUPPORTED;
  const int64_t share = grouped_ws_share(B, T, D, R, W, dtype, has_static);
  return share < 0 ? share : G * share;
}

int dc_lowrank_bwd_grouped(int64_t G, const void* x, int64_t x_ld, const void* const* z, const void* const* U,
                           const void* const* static_w, const void* const* z_eff, int64_t z_eff_bytes,
                           const void* const* dy, int64_t dy_hd, void* dx,
                           int64_t dx_ld, void* const* dz, void* const* dU, void* const* dstatic_w,
                           void* workspace, int64_t ws_bytes, int64_t B, int64_t T, int64_t D, int64_t R,
                           int64_t W, int dtype, int residual, void* stream) {
  if (G < 1 || G > DC_MAX_GROUPS) return DC_ERR_UNSUPPORTED;
  int s = check_lowrank(B, T, D, R, W, dtype, static_w != nullptr);
  if (s != DC_OK) return s;
  if (x_ld < G * D || x_ld > kI32Max || dx_ld < G * D || dx_ld > kI32Max || !head_dim_ok(dy_hd, D))
    return DC_ERR_SHAPE;
  if (!x || !z || !U || !dy || !dx || !dz || !dU) return DC_ERR_NULL;
  if ((static_w == nullptr) != (dstatic_w == nullptr)) return DC_ERR_NULL;
  const int es = dc::dtype_size(dtype);
  if (!aligned_to(x, es) || !aligned_to(dx, es)) return DC_ERR_ALIGN;
  const int64_t share = grouped_ws_share(B, T, D, R, W, dtype, static_w != nullptr);
  if (share < 0) return (int)share;
  if (share > 0 && (workspace == nullptr || ws_bytes < G * share || !aligned_to(workspace, 256)))
    return DC_ERR_WORKSPACE;
  const int64_t zneed = zeff_need(B, T, D, R, W, dtype, static_w != nullptr);
  dc::LrProblem p[DC_MAX_GROUPS] = {};
  for (int64_t g = 0; g < G; ++g) {
    const void* sw = static_w ? static_w[g] : nullptr;
    void* dsw = dstatic_w ? dstatic_w[g] : nullptr;
    if (!z[g] || !U[g] || !dy[g] || !dz[g] || !dU[g] || (static_w && (!sw || !dsw)) || (z_eff && !z_eff[g]))
      return DC_ERR_NULL;
    if (!aligned_to(z[g], es) || !aligned_to(U[g], es) || !aligned_to(sw, es) || !aligned_to(dy[g], es) ||
        !aligned_to(dz[g], es) || !aligned_to(dU[g], es) || !aligned_to(dsw, es) ||
        (z_eff && !aligned_to(z_eff[g], 16)))
      return DC_ERR_ALIGN;
    dc::LrProblem& q = p[g];
    q.x = (const char*)x + g * D * es; q.z = z[g]; q.U = U[g]; q.static_w = sw; q.dy = dy[g];
    q.dx = (char*)dx + g * D * es; q.dz = dz[g]; q.dU = dU[g]; q.dstatic_w = dsw;
    q.zeff = z_eff ? zeff_of(z_eff[g], zneed) : nullptr;
    q.ws = share > 0 ? (float*)((char*)workspace + g * share) : nullptr;
    q.B = B; q.T = T; q.D = D; q.R = R; q.W = W; q.x_ld = x_ld; q.dx_ld = dx_ld; q.y_hd = dy_hd;
    q.dtype = dtype; q.residual = residual ? 1 : 0; q.stream = (hipStream_t)stream;
  }
  if (z_eff && (s = zeff_status(z_eff[0], z_eff_bytes, zneed)) != DC_OK) return s;
  if ((s = device_status()) != DC_OK) return s;
  return launch_status(dc::lr_bwd(p, (int)G));
}

// ------------------------------------------------------------------ proj_in

static int check_proj(int64_t G, int64_t M, int64_t K, int64_t R, int dtype, dc::ProjProblem* p) {
  if (!dtype_ok(dtype)) return DC_ERR_DTYPE;
  if (G < 1 || M <= 0 || K <= 0 || R <= 0) return DC_ERR_SHAPE;
  if (G > DC_MAX_GROUPS) return DC_ERR_UNSUPPORTED;
  if (M > kI32Max || K > kI32Max || G * R > kI32Max) return DC_ERR_SHAPE;
  *p = dc::ProjProblem{};
  p->G = G; p->M = M; p->K = K; p->R = R; p->dtype = dtype;
  return dc::proj_shape_ok(*p) ? DC_OK : DC_ERR_UNSUPPORTED;
}

int dc_proj_in_fwd(const void* pre_z, const void* w_in, void* const* z, int64_t G, int64_t M, int64_t K, int64_t R,
                   int dtype, void* stream) {
  dc::ProjProblem p;
  int s = check_proj(G, M, K, R, dtype, &p);
  if (s != DC_OK) return s;
  if (!pre_z || !w_in || !z) return DC_ERR_NULL;
  if (!aligned_to(pre_z, 16) || !aligned_to(w_in, 16)) return DC_ERR_ALIGN;
  for (int64_t g = 0; g < G; ++g) {
    if (!z[g]) return DC_ERR_NULL;
    if (!aligned_to(z[g], 2)) return DC_ERR_ALIGN;
    p.z[g] = z[g];
  }
  if ((s = device_status()) != DC_OK) return s;
  p.pre_z = pre_z; p.w_in = w_in; p.stream = (hipStream_t)stream;
  return launch_status(dc::proj_fwd_launch(p));
}

int64_t dc_proj_in_bwd_ws_bytes(int64_t G, int64_t M, int64_t K, int64_t R, int dtype) {
  dc::ProjProblem p;
  int s = check_proj(G, M, K, R, dtype, &p);
  if (s != DC_OK) return s;
  return dc::proj_bwd_ws_bytes(p);
}

int dc_proj_in_bwd(const void* pre_z, const void* w_in, const void* const* dz, void* dpre_z, void* dw_in,
                   void* workspace, int64_t ws_bytes, int64_t G, int64_t M, int64_t K, int64_t R, int dtype,
                   void* stream) {
  dc::ProjProblem p;
  int s = check_proj(G, M, K, R, dtype, &p);
  if (s != DC_OK) return s;
  if (!pre_z || !w_in || !dz || !dpre_z || !dw_in) return DC_ERR_NULL;
  if (!aligned_to(pre_z, 16) || !aligned_to(w_in, 16) || !aligned_to(dpre_z, 16) || !aligned_to(dw_in, 2))
    return DC_ERR_ALIGN;
  for (int64_t g = 0; g < G; ++g) {
    if (!dz[g]) return DC_ERR_NULL;
    if (!aligned_to(dz[g], 2)) return DC_ERR_ALIGN;
    p.dz[g] = dz[g];
  }
  const int64_t need = dc::proj_bwd_ws_bytes(p);
  if (workspace == nullptr || ws_bytes < need || !aligned_to(workspace, 16)) return DC_ERR_WORKSPACE;
  if ((s = device_status()) != DC_OK) return s;
  p.pre_z = pre_z; p.w_in = w_in; p.dpre_z = dpre_z; p.dw_in = dw_in; p.ws = (float*)workspace;
  p.stream = (hipStream_t)stream;
  return launch_status(dc::proj_bwd_launch(p));
}

}  // extern "C"
