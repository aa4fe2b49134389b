// C ABI of the RMSNorm kernels: argument validation, shape/alignment selection, and
// the deterministic weight-gradient finish pass.  Kernels live in rmsnorm_impl.hpp.
#include <string>

#include "rmsnorm_impl.hpp"

namespace pt {
namespace rmsnorm {

__global__ __launch_bounds__(256) void rmsnorm_dw_finish_kernel(const float* __restrict__ partial,
                                                                int64_t nparts, int cols,
                                                                void* __restrict__ dw, int wdt) {
  __shared__ float lds[4][64];
  const int lane = threadIdx.x % 64;
  const int wave = threadIdx.x / 64;
  const int c = blockIdx.x * 64 + lane;
  float s = 0.0f;
  if (c < cols) {
    for (int64_t p = wave; p < nparts; p += 4) s += partial[p * cols + c];
  }
  lds[wave][lane] = s;
  __syncthreads();
  if (wave == 0 && c < cols) {
    const float t = ((lds[0][lane] + lds[1][lane]) + lds[2][lane]) + lds[3][lane];
    store_any(dw, c, wdt, t);
  }
}

namespace {

template <typename T>
bool row_aligned(const void* p, int64_t stride) {
  return aligned16(p) && ((stride * static_cast<int64_t>(sizeof(T))) % 16) == 0;
}

bool rows_aligned(int xdt, const void* p, int64_t stride) {
  return aligned16(p) && ((stride * dtype_size(xdt)) % 16) == 0;
}

int validate(const char* fn, int64_t rows, int64_t cols, int xdt, int wdt, bool backward,
             Shape* s) {
  if (!valid_dtype(xdt) || !valid_dtype(wdt))
    return fail(PT_EINVAL, std::string(fn) + ": unknown dtype code");
  if (rows < 0 || cols <= 0)
    return fail(PT_EINVAL, std::string(fn) + ": rows must be >= 0 and cols > 0");
  if (rows > (int64_t{1} << 40)) return fail(PT_EUNSUPPORTED, std::string(fn) + ": rows too large");
  const int vec = 16 / dtype_size(xdt);
  if (!choose_shape(cols, vec, backward, s))
    return fail(PT_EUNSUPPORTED, std::string(fn) + ": hidden size " + std::to_string(cols) +
                                     " exceeds the register-resident row capacity (" +
                                     std::to_string(64 * 16 * 16 * vec) + " elements)");
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
  Shape s;
  if (int rc = validate("pt_rmsnorm_fwd", rows, cols, x_dtype, w_dtype, false, &s)) return rc;
  if (rows == 0) return ok();
  if (!x || !weight || !y || !rstd) return fail(PT_EINVAL, "pt_rmsnorm_fwd: null pointer");
  {
    // One wave per row (four rows per 256-thread block) or 64*wpr threads per row; an HSA
    // grid holds at most 2^32 - 1 work-items.
    const int64_t threads = s.wpr == 1 ? (rows + kFwdWavesWpr1 - 1) / kFwdWavesWpr1 * 64 * kFwdWavesWpr1
                                       : rows * 64 * s.wpr;
    if (threads > 0xffffffffLL)
      return fail(PT_EUNSUPPORTED, "pt_rmsnorm_fwd: too many rows for one launch");
  }
  if (rows > 1 && (x_row_stride < cols || y_row_stride < cols))
    return fail(PT_EINVAL, "pt_rmsnorm_fwd: row stride smaller than cols");
  const int vec = 16 / dtype_size(x_dtype);
  FwdArgs a{};
  a.x = x;
  a.xs = x_row_stride;
  a.w = weight;
  a.wdt = w_dtype;
  a.y = y;
  a.ys = y_row_stride;
  a.rstd = rstd;
  a.rows = rows;
  a.cols = static_cast<int>(cols);
  a.eps = eps;
  a.xdt = x_dtype;
  a.aligned = (cols % vec == 0) && rows_aligned(x_dtype, x, x_row_stride) &&
              rows_aligned(x_dtype, y, y_row_stride) && aligned16(weight);
  a.shape = s;
  a.st = as_stream(stream);
  if (x_dtype == PT_FLOAT32) {
    launch_fwd<float>(a);
  } else if (x_dtype == PT_FLOAT16) {
    launch_fwd<_Float16>(a);
  } else {
    launch_fwd<__bf16>(a);
  }
  return check_launch("pt_rmsnorm_fwd");
}

size_t pt_rmsnorm_bwd_workspace_bytes(int64_t rows, int64_t cols, int x_dtype) {
  Shape s;
  if (rows <= 0 || cols <= 0 || !valid_dtype(x_dtype)) return 0;
  if (!choose_shape(cols, 16 / dtype_size(x_dtype), true, &s)) return 0;
  int64_t blocks = 0, rpb = 0;
  bwd_grid(rows, s, &blocks, &rpb);
  return static_cast<size_t>(blocks) * static_cast<size_t>(cols) * sizeof(float);
}

int pt_rmsnorm_bwd(const void* dy, int64_t dy_row_stride, const void* x, int64_t x_row_stride,
                   const void* weight, const float* rstd, void* dx, int64_t dx_row_stride,
                   void* dweight, void* workspace, size_t workspace_bytes, int64_t rows,
                   int64_t cols, int x_dtype, int w_dtype, void* stream) {
  Shape s;
  if (int rc = validate("pt_rmsnorm_bwd", rows, cols, x_dtype, w_dtype, true, &s)) return rc;
  hipStream_t st = as_stream(stream);
  if (rows == 0) {
    // Empty batch: the weight gradient is a sum over no rows.
    if (dweight) return fill(dweight, cols, dtype_size(w_dtype), 0u, st);
    return ok();
  }
  if (!dy || !x || !weight || !rstd) return fail(PT_EINVAL, "pt_rmsnorm_bwd: null pointer");
  if (rows > 1 && (dy_row_stride < cols || x_row_stride < cols || (dx && dx_row_stride < cols)))
    return fail(PT_EINVAL, "pt_rmsnorm_bwd: row stride smaller than cols");
  int64_t blocks = 0, rpb = 0;
  bwd_grid(rows, s, &blocks, &rpb);
  float* partial = nullptr;
  if (dweight) {
    const size_t need = static_cast<size_t>(blocks) * static_cast<size_t>(cols) * sizeof(float);
    if (!workspace || workspace_bytes < need)
      return fail(PT_EINVAL,
                  "pt_rmsnorm_bwd: workspace smaller than pt_rmsnorm_bwd_workspace_bytes()");
    if (!aligned16(workspace)) return fail(PT_EINVAL, "pt_rmsnorm_bwd: workspace not aligned");
    partial = static_cast<float*>(workspace);
  }
  const int vec = 16 / dtype_size(x_dtype);
  BwdArgs a{};
  a.dy = dy;
  a.dys = dy_row_stride;
  a.x = x;
  a.xs = x_row_stride;
  a.w = weight;
  a.wdt = w_dtype;
  a.rstd = rstd;
  a.dx = dx;
  a.dxs = dx_row_stride;
  a.partial = partial;
  a.blocks = blocks;
  a.rpb = rpb;
  a.rows = rows;
  a.cols = static_cast<int>(cols);
  a.xdt = x_dtype;
  a.aligned = (cols % vec == 0) && rows_aligned(x_dtype, dy, dy_row_stride) &&
              rows_aligned(x_dtype, x, x_row_stride) &&
              (dx == nullptr || rows_aligned(x_dtype, dx, dx_row_stride)) && aligned16(weight);
  a.shape = s;
  a.st = st;
  if (x_dtype == PT_FLOAT32) {
    launch_bwd<float>(a);
  } else if (x_dtype == PT_FLOAT16) {
    launch_bwd<_Float16>(a);
  } else {
    launch_bwd<__bf16>(a);
  }
  if (int rc = check_launch("pt_rmsnorm_bwd")) return rc;
  if (dweight) {
    const unsigned fblocks = static_cast<unsigned>((cols + 63) / 64);
    hipLaunchKernelGGL(rmsnorm_dw_finish_kernel, dim3(fblocks), dim3(256), 0, st, partial, blocks,
                       static_cast<int>(cols), dweight, w_dtype);
    return check_launch("pt_rmsnorm_bwd (dW finish)");
  }
  return ok();
}

}  // extern "C"
