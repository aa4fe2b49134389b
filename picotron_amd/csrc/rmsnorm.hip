// C ABI of the RMSNorm kernels: argument validation, shape/alignment selection, and
// the deterministic weight-gradient finish pass.  Kernels live in rmsnorm_impl.hpp.
#include <mutex>
#include <string>

#include "rmsnorm_impl.hpp"

namespace pt {
namespace rmsnorm {

__global__ __launch_bounds__(256) void rmsnorm_dw_finish_kernel(const float* __restrict__ partial,
                                                                int64_t nparts, int cols,
                                                                void* __restrict__ dw, int wdt) {
  __shared__ float lds[kFinishGroups][kFinishCols + 1];
  const int col = threadIdx.x % kFinishCols;
  const int grp = threadIdx.x / kFinishCols;
  const int c = blockIdx.x * kFinishCols + col;
  lds[grp][col] = c < cols ? column_group_sum(partial, nparts, cols, c, grp) : 0.0f;
  __syncthreads();
  if (grp == 0 && c < cols) {
    float t = lds[0][col];
#pragma unroll
    for (int g = 1; g < kFinishGroups; ++g) t += lds[g][col];
    store_any(dw, c, wdt, t);
  }
}

namespace {

bool rows_aligned(int xdt, const void* p, int64_t stride) {
  return aligned16(p) && ((stride * dtype_size(xdt)) % 16) == 0;
}

int cap_of(int v) { return v < 1 ? 1 : (v > 8 ? 8 : v); }

int validate(const char* fn, int64_t rows, int64_t cols, int xdt, int wdt, bool backward,
             Shape* s) {
  if (!valid_dtype(xdt) || !valid_dtype(wdt))
    return fail(PT_EINVAL, std::string(fn) + ": unknown dtype code");
  if (rows < 0 || cols <= 0)
    return fail(PT_EINVAL, std::string(fn) + ": rows must be >= 0 and cols > 0");
  // Bounds the per-block row-group count (an int) for any grid.
  if (rows > (int64_t{1} << 36)) return fail(PT_EUNSUPPORTED, std::string(fn) + ": rows too large");
  const int vec = 16 / dtype_size(xdt);
  const int cap = cap_of(backward ? bwd_vpl_cap_for(tuning().bwd_vpl_cap, cols, vec)
                                  : fwd_vpl_cap_for(tuning().fwd_vpl_cap, vec));
  if (!choose_shape(cols, vec, cap, s))
    return fail(PT_EUNSUPPORTED, std::string(fn) + ": hidden size " + std::to_string(cols) +
                                     " exceeds the register-resident row capacity (" +
                                     std::to_string(64 * 16 * 16 * vec) + " elements)");
  return PT_OK;
}

}  // namespace
}  // namespace rmsnorm
}  // namespace pt

namespace pt {
namespace rmsnorm {
namespace {

int fwd_impl(const char* fn, const void* x, int64_t xs, const void* res, int64_t res_s,
             const void* weight, void* h, int64_t hs, void* y, int64_t ys, float* rstd,
             int64_t rows, int64_t cols, float eps, int x_dtype, int w_dtype, void* stream) {
  Shape s;
  if (int rc = validate(fn, rows, cols, x_dtype, w_dtype, false, &s)) return rc;
  if (rows == 0) return ok();
  const bool fused = res != nullptr || h != nullptr;
  if (!x || !weight || !y || !rstd || (fused && (!res || !h)))
    return fail(PT_EINVAL, std::string(fn) + ": null pointer");
  if (rows > 1 && (xs < cols || ys < cols || (fused && (res_s < cols || hs < cols))))
    return fail(PT_EINVAL, std::string(fn) + ": row stride smaller than cols");
  if (fused && (h == x || h == res || h == y))
    return fail(PT_EINVAL, std::string(fn) + ": h must not alias x, residual or y");
  const int vec = 16 / dtype_size(x_dtype);
  FwdArgs a{};
  a.x = x;
  a.xs = xs;
  a.w = weight;
  a.wdt = w_dtype;
  a.y = y;
  a.ys = ys;
  a.rstd = rstd;
  a.rows = rows;
  a.cols = static_cast<int>(cols);
  a.eps = eps;
  a.xdt = x_dtype;
  a.res = fused ? res : nullptr;
  a.res_s = res_s;
  a.h = fused ? h : nullptr;
  a.h_s = hs;
  a.aligned = (cols % vec == 0) && rows_aligned(x_dtype, x, xs) && rows_aligned(x_dtype, y, ys) &&
              (!fused || (rows_aligned(x_dtype, res, res_s) && rows_aligned(x_dtype, h, hs))) &&
              aligned16(weight) && vector_weight(x_dtype, w_dtype);
  a.shape = a.aligned ? s : unaligned_shape(cols, vec);
  a.blocks = fwd_blocks(rows, a.shape, num_cus());
  a.st = as_stream(stream);
  bool launched;
  if (x_dtype == PT_FLOAT32) {
    launched = launch_fwd<float>(a);
  } else if (x_dtype == PT_FLOAT16) {
    launched = launch_fwd<_Float16>(a);
  } else {
    launched = launch_fwd<__bf16>(a);
  }
  if (!launched) return fail(PT_EUNSUPPORTED, std::string(fn) + ": no kernel for this shape");
  return check_launch(fn);
}

int bwd_impl(const char* fn, const void* dy, int64_t dys, const void* dh_in, int64_t dh_in_s,
             const void* x, int64_t xs, const void* weight, const float* rstd, void* dx,
             int64_t dxs, void* dweight, void* workspace, size_t workspace_bytes, int64_t rows,
             int64_t cols, int x_dtype, int w_dtype, void* stream, bool static_scratch = false) {
  Shape s;
  if (int rc = validate(fn, rows, cols, x_dtype, w_dtype, true, &s)) return rc;
  hipStream_t st = as_stream(stream);
  if (rows == 0) {
    // Empty batch: the weight gradient is a sum over no rows.
    if (dweight) return fill(dweight, cols, dtype_size(w_dtype), 0u, st);
    return ok();
  }
  if (!dy || !x || !weight || !rstd || (dh_in && !dx))
    return fail(PT_EINVAL, std::string(fn) + ": null pointer");
  if (rows > 1 && (dys < cols || xs < cols || (dx && dxs < cols) || (dh_in && dh_in_s < cols)))
    return fail(PT_EINVAL, std::string(fn) + ": row stride smaller than cols");
  const int vec = 16 / dtype_size(x_dtype);
  BwdArgs a{};
  a.aligned = (cols % vec == 0) && rows_aligned(x_dtype, dy, dys) &&
              rows_aligned(x_dtype, x, xs) && (dx == nullptr || rows_aligned(x_dtype, dx, dxs)) &&
              (dh_in == nullptr || rows_aligned(x_dtype, dh_in, dh_in_s)) && aligned16(weight) &&
              vector_weight(x_dtype, w_dtype);
  a.shape = a.aligned ? s : unaligned_shape(cols, vec);
  a.blocks = bwd_blocks(rows, a.shape);
  float* partial = nullptr;
  if (dweight) {
    const size_t need = static_cast<size_t>(a.blocks) * static_cast<size_t>(cols) * sizeof(float);
    if (static_scratch && need > workspace_bytes)
      return fail(PT_EUNSUPPORTED,
                  std::string(fn) + ": the weight-gradient partials need " + std::to_string(need) +
                      " bytes, more than the library's static scratch of " +
                      std::to_string(workspace_bytes) + " bytes; use pt_rmsnorm_bwd");
    if (!workspace || workspace_bytes < need)
      return fail(PT_EINVAL, std::string(fn) + ": workspace smaller than pt_rmsnorm_bwd_workspace_bytes()");
    if (!aligned16(workspace)) return fail(PT_EINVAL, std::string(fn) + ": workspace not aligned");
    // LDS combining the row slots' weight-gradient sums holds one fp32 per column.
    if (bwd_waves(a.shape) / a.shape.wpr > 1 && cols * 4 > 160 * 1024)
      return fail(PT_EUNSUPPORTED, std::string(fn) + ": hidden size too large for the LDS combine");
    partial = static_cast<float*>(workspace);
  }
  a.dy = dy;
  a.dys = dys;
  a.x = x;
  a.xs = xs;
  a.w = weight;
  a.wdt = w_dtype;
  a.rstd = rstd;
  a.dx = dx;
  a.dxs = dxs;
  a.partial = partial;
  a.rows = rows;
  a.cols = static_cast<int>(cols);
  a.xdt = x_dtype;
  a.st = st;
  a.dh_in = dh_in;
  a.dh_in_s = dh_in_s;
  bool launched;
  if (x_dtype == PT_FLOAT32) {
    launched = launch_bwd<float>(a);
  } else if (x_dtype == PT_FLOAT16) {
    launched = launch_bwd<_Float16>(a);
  } else {
    launched = launch_bwd<__bf16>(a);
  }
  if (!launched) return fail(PT_EUNSUPPORTED, std::string(fn) + ": no kernel for this shape");
  if (int rc = check_launch(fn)) return rc;
  if (dweight) {
    const unsigned fblocks = static_cast<unsigned>((cols + kFinishCols - 1) / kFinishCols);
    hipLaunchKernelGGL(rmsnorm_dw_finish_kernel, dim3(fblocks), dim3(256), 0, st, partial,
                       a.blocks, static_cast<int>(cols), dweight, w_dtype);
    return check_launch(fn);
  }
  return ok();
}

}  // namespace
}  // namespace rmsnorm
}  // namespace pt

namespace pt {
namespace rmsnorm {

// Scratch of pt_rmsnorm_bwd_noalloc: the fp32 weight-gradient partial rows, [blocks, cols]
// (512 x 4096 at 16384 x 4096, 8 MiB).  A file-scope device array, so that entry point
// allocates nothing; every device the library runs on holds one copy until the process
// ends.  Each call overwrites every partial it reads (each block writes its whole row), so
// nothing needs clearing between calls; calls that overlap on one device race on it.
constexpr size_t kScratchBytes = size_t{16} << 20;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

namespace {

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
bool g_scratch_looked_up[kScratchDevices];
void* g_scratch_ptr[kScratchDevices];
hipError_t g_scratch_err[kScratchDevices];

// Device address of the current device's copy of `scratch`, looked up once per device with
// that device current.  In host code the array's name is only a host-side stand-in for the
// symbol: kernels and copies must be given this address instead.  The lookup is kept out of
// graph captures (it may load the library's code on the device): the first call on a device
// must not be captured, and is refused if it is.
int scratch_address(const char* fn, hipStream_t st, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kScratchDevices)
    return fail(PT_EDEVICE, std::string(fn) + ": no current HIP device");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_looked_up[dev]) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) {
      (void)hipGetLastError();
      return fail(PT_EUNSUPPORTED, std::string(fn) +
                                       ": the first call on a device looks up the library's "
                                       "scratch and cannot be captured; call it once before "
                                       "capturing");
    }
    void* p = nullptr;
    g_scratch_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_scratch_ptr[dev] = g_scratch_err[dev] == hipSuccess ? p : nullptr;
    g_scratch_looked_up[dev] = true;
  }
  if (g_scratch_err[dev] != hipSuccess || g_scratch_ptr[dev] == nullptr)
    return fail(PT_EDEVICE, std::string(fn) + ": hipGetSymbolAddress(scratch) failed: " +
                                hipGetErrorString(g_scratch_err[dev]));
  *out = g_scratch_ptr[dev];
  return PT_OK;
}

}  // namespace
}  // namespace rmsnorm
}  // namespace pt

using namespace pt;
using namespace pt::rmsnorm;

extern "C" {

int pt_rmsnorm_fwd(const void* x, int64_t x_row_stride, const void* weight, void* y,
                   int64_t y_row_stride, float* rstd, int64_t rows, int64_t cols, float eps,
                   int x_dtype, int w_dtype, void* stream) {
  return fwd_impl("pt_rmsnorm_fwd", x, x_row_stride, nullptr, 0, weight, nullptr, 0, y,
                  y_row_stride, rstd, rows, cols, eps, x_dtype, w_dtype, stream);
}

size_t pt_rmsnorm_bwd_workspace_bytes(int64_t rows, int64_t cols, int x_dtype) {
  Shape s;
  if (rows <= 0 || cols <= 0 || !valid_dtype(x_dtype)) return 0;
  const int vec = 16 / dtype_size(x_dtype);
  if (!choose_shape(cols, vec, cap_of(bwd_vpl_cap_for(tuning().bwd_vpl_cap, cols, vec)), &s))
    return 0;
  // Enough for either path (aligned shape or the unaligned subset).
  int64_t blocks = bwd_blocks(rows, s);
  const int64_t ublocks = bwd_blocks(rows, unaligned_shape(cols, vec));
  if (ublocks > blocks) blocks = ublocks;
  return static_cast<size_t>(blocks) * static_cast<size_t>(cols) * sizeof(float);
}

int pt_rmsnorm_bwd(const void* dy, int64_t dy_row_stride, const void* x, int64_t x_row_stride,
                   const void* weight, const float* rstd, void* dx, int64_t dx_row_stride,
                   void* dweight, void* workspace, size_t workspace_bytes, int64_t rows,
                   int64_t cols, int x_dtype, int w_dtype, void* stream) {
  return bwd_impl("pt_rmsnorm_bwd", dy, dy_row_stride, nullptr, 0, x, x_row_stride, weight, rstd,
                  dx, dx_row_stride, dweight, workspace, workspace_bytes, rows, cols, x_dtype,
                  w_dtype, stream);
}

int pt_rmsnorm_bwd_noalloc(const void* dy, int64_t dy_row_stride, const void* x,
                           int64_t x_row_stride, const void* weight, const float* rstd, void* dx,
                           int64_t dx_row_stride, void* dweight, int64_t rows, int64_t cols,
                           int x_dtype, int w_dtype, void* stream) {
  static const char* const fn = "pt_rmsnorm_bwd_noalloc";
  void* ws = nullptr;
  if (dweight != nullptr && rows > 0) {
    if (int rc = scratch_address(fn, as_stream(stream), &ws)) return rc;
  }
  return bwd_impl(fn, dy, dy_row_stride, nullptr, 0, x, x_row_stride, weight, rstd, dx,
                  dx_row_stride, dweight, ws, ws ? kScratchBytes : 0, rows, cols, x_dtype, w_dtype,
                  stream, true);
}

int pt_residual_rmsnorm_fwd(const void* x, int64_t x_row_stride, const void* residual,
                            int64_t residual_row_stride, const void* weight, void* h,
                            int64_t h_row_stride, void* y, int64_t y_row_stride, float* rstd,
                            int64_t rows, int64_t cols, float eps, int x_dtype, int w_dtype,
                            void* stream) {
  if (!residual || !h) return fail(PT_EINVAL, "pt_residual_rmsnorm_fwd: null pointer");
  return fwd_impl("pt_residual_rmsnorm_fwd", x, x_row_stride, residual, residual_row_stride,
                  weight, h, h_row_stride, y, y_row_stride, rstd, rows, cols, eps, x_dtype,
                  w_dtype, stream);
}

int pt_residual_rmsnorm_bwd(const void* dy, int64_t dy_row_stride, const void* dh_in,
                            int64_t dh_in_row_stride, const void* h, int64_t h_row_stride,
                            const void* weight, const float* rstd, void* dh, int64_t dh_row_stride,
                            void* dweight, void* workspace, size_t workspace_bytes, int64_t rows,
                            int64_t cols, int x_dtype, int w_dtype, void* stream) {
  if (!dh) return fail(PT_EINVAL, "pt_residual_rmsnorm_bwd: null pointer");
  return bwd_impl("pt_residual_rmsnorm_bwd", dy, dy_row_stride, dh_in, dh_in_row_stride, h,
                  h_row_stride, weight, rstd, dh, dh_row_stride, dweight, workspace,
                  workspace_bytes, rows, cols, x_dtype, w_dtype, stream);
}

}  // extern "C"
