// C ABI of the RMSNorm kernels: argument validation, shape/alignment selection, and
// the deterministic weight-gradient finish pass.  Kernels live in rmsnorm_impl.hpp.
#include <string>

#include "rmsnorm_impl.hpp"

namespace pt {
namespace rmsnorm {

__global__ __launch_bounds__(256) void rmsnorm_dw_finish_kernel(const float* __restrict__ partial,
                                                                int64_t nparts, int cols,
                                                                void* __restrict__ dw, int wdt) {
  constexpr int kGroups = 256 / kFinishCols;
  constexpr int kUnroll = 64;
  __shared__ float lds[kGroups][kFinishCols + 1];
  const int col = threadIdx.x % kFinishCols;
  const int grp = threadIdx.x / kFinishCols;
  const int c = blockIdx.x * kFinishCols + col;
  float s = 0.0f;
  if (c < cols) {
    const float* p = partial + c;
    int64_t i = grp;
    for (; i + static_cast<int64_t>(kGroups) * (kUnroll - 1) < nparts;
         i += static_cast<int64_t>(kGroups) * kUnroll) {
      float v[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) v[u] = p[(i + u * kGroups) * cols];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) s += v[u];
    }
    for (; i < nparts; i += kGroups) s += p[i * cols];
  }
  lds[grp][col] = s;
  __syncthreads();
  if (grp == 0 && c < cols) {
    float t = lds[0][col];
#pragma unroll
    for (int g = 1; g < kGroups; ++g) t += lds[g][col];
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
  const int cap = cap_of(backward ? tuning().bwd_vpl_cap : tuning().fwd_vpl_cap);
  if (!choose_shape(cols, vec, cap, s))
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
              rows_aligned(x_dtype, y, y_row_stride) && aligned16(weight) &&
              vector_weight(x_dtype, w_dtype);
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
  if (!launched) return fail(PT_EUNSUPPORTED, "pt_rmsnorm_fwd: no kernel for this shape");
  return check_launch("pt_rmsnorm_fwd");
}

size_t pt_rmsnorm_bwd_workspace_bytes(int64_t rows, int64_t cols, int x_dtype) {
  Shape s;
  if (rows <= 0 || cols <= 0 || !valid_dtype(x_dtype)) return 0;
  const int vec = 16 / dtype_size(x_dtype);
  if (!choose_shape(cols, vec, cap_of(tuning().bwd_vpl_cap), &s)) return 0;
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
  const int vec = 16 / dtype_size(x_dtype);
  BwdArgs a{};
  a.aligned = (cols % vec == 0) && rows_aligned(x_dtype, dy, dy_row_stride) &&
              rows_aligned(x_dtype, x, x_row_stride) &&
              (dx == nullptr || rows_aligned(x_dtype, dx, dx_row_stride)) && aligned16(weight) &&
              vector_weight(x_dtype, w_dtype);
  a.shape = a.aligned ? s : unaligned_shape(cols, vec);
  a.blocks = bwd_blocks(rows, a.shape);
  float* partial = nullptr;
  if (dweight) {
    const size_t need = static_cast<size_t>(a.blocks) * static_cast<size_t>(cols) * sizeof(float);
    if (!workspace || workspace_bytes < need)
      return fail(PT_EINVAL,
                  "pt_rmsnorm_bwd: workspace smaller than pt_rmsnorm_bwd_workspace_bytes()");
    if (!aligned16(workspace)) return fail(PT_EINVAL, "pt_rmsnorm_bwd: workspace not aligned");
    // LDS combining the row slots' weight-gradient sums holds one fp32 per column.
    if (bwd_waves(a.shape) / a.shape.wpr > 1 && cols * 4 > 160 * 1024)
      return fail(PT_EUNSUPPORTED, "pt_rmsnorm_bwd: hidden size too large for the LDS combine");
    partial = static_cast<float*>(workspace);
  }
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
  a.rows = rows;
  a.cols = static_cast<int>(cols);
  a.xdt = x_dtype;
  a.st = st;
  bool launched;
  if (x_dtype == PT_FLOAT32) {
    launched = launch_bwd<float>(a);
  } else if (x_dtype == PT_FLOAT16) {
    launched = launch_bwd<_Float16>(a);
  } else {
    launched = launch_bwd<__bf16>(a);
  }
  if (!launched) return fail(PT_EUNSUPPORTED, "pt_rmsnorm_bwd: no kernel for this shape");
  if (int rc = check_launch("pt_rmsnorm_bwd")) return rc;
  if (dweight) {
    const unsigned fblocks = static_cast<unsigned>((cols + kFinishCols - 1) / kFinishCols);
    hipLaunchKernelGGL(rmsnorm_dw_finish_kernel, dim3(fblocks), dim3(256), 0, st, partial,
                       a.blocks, static_cast<int>(cols), dweight, w_dtype);
    return check_launch("pt_rmsnorm_bwd (dW finish)");
  }
  return ok();
}

}  // extern "C"
