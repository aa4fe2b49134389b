// Fused cross-entropy (mean over non-ignored rows) with its gradient written in place.
//
// Reference semantics (AndyMLAndAI/picotron):
//   src/picotron/nn/triton_kernels/cross_entropy.py:97-109 -> F.cross_entropy(logits,
//   targets) with torch's defaults (reduction "mean", ignore_index -100); the Triton kernel
//   at cross_entropy.py:28-45 computes lse - logit[target] per row (forward only).
//   Gradient of the mean: d/dx_j = (softmax_j - [j == target]) / n_valid, 0 on ignored rows.
//
// Three launches per call, no host synchronisation and no device-scope fences:
//   1. ce_prepare: one block counts the non-ignored targets (n_valid) into the workspace
//      and clears the status word.
//   2. ce_rows: one 1024-thread workgroup per row.  The row is loaded once into registers
//      (VPT 16-byte vectors per thread) and reduced to its max; exp(x - max) is then
//      computed once per element, summed in fp32 and kept in the registers in place of the
//      logit, so the gradient softmax / n_valid is written from registers without a second
//      exponential: HBM sees one read and one write of the logits.  The target element's
//      gradient (softmax_t - 1) / n_valid is computed from the exact fp32 target logit.
//      Rows too long for registers, or not 16-byte aligned, use ce_rows_stream (online
//      max / sum, then a second read).  Each row's fp32 loss goes to the workspace.
//   3. ce_finish: one block sums the per-row losses in a fixed order and divides by
//      n_valid, so the loss is bitwise reproducible.
// exp(x - m) is evaluated as exp2((x - m) * log2(e)) on the hardware exp2 unit.
#include <cmath>
#include <type_traits>

#include "pt_common.hpp"

namespace pt {
namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr float kLog2e = 1.4426950408889634f;

struct CeWork {
  float n_valid;  // number of non-ignored targets (exact below 2^24)
  int reserved;
  int status;     // bit 0: a non-ignored target outside [0, vocab)
  int pad;
  // followed by float row_loss[rows], 16-byte aligned
};

constexpr size_t kHeader = 16;

__device__ __forceinline__ float* row_losses(CeWork* ws) {
  return reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + kHeader);
}

__device__ __forceinline__ float exp2_(float x) { return __builtin_amdgcn_exp2f(x); }

// exp(x - m) on the hardware exp2 unit.  x - m is exact when x is within a factor of two of
// m, so the row max contributes exactly 1 to the sum and a one-class row has loss 0.
__device__ __forceinline__ float exp_shifted(float x, float m) { return exp2_((x - m) * kLog2e); }

__device__ __forceinline__ float block_reduce_max(float v, float* red) {
  v = wave_max(v);
  const int wave = threadIdx.x / 64;
  const int lane = threadIdx.x % 64;
  __syncthreads();  // previous users of red are done
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = red[0];
#pragma unroll
  for (int i = 1; i < kWaves; ++i) t = fmaxf(t, red[i]);
  return t;
}

__device__ __forceinline__ float block_reduce_sum(float v, float* red) {
  v = wave_sum(v);
  const int wave = threadIdx.x / 64;
  const int lane = threadIdx.x % 64;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = 0.0f;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) t += red[i];
  return t;
}

__global__ __launch_bounds__(kThreads) void ce_prepare_kernel(const int64_t* __restrict__ targets,
                                                               int64_t inner, int64_t tos,
                                                               int64_t tis, int64_t rows,
                                                               int64_t ignore_index,
                                                               CeWork* __restrict__ ws,
                                                               float* __restrict__ loss_out) {
  __shared__ float red[kWaves];
  float cnt = 0.0f;
  for (int64_t r = threadIdx.x; r < rows; r += kThreads) {
    const int64_t o = r / inner, i = r - (r / inner) * inner;
    cnt += (targets[o * tos + i * tis] != ignore_index) ? 1.0f : 0.0f;
  }
  const float total = block_reduce_sum(cnt, red);
  if (threadIdx.x == 0) {
    ws->n_valid = total;
    ws->status = 0;
    if (rows == 0) *loss_out = NAN;  // mean over an empty batch: 0/0, as torch returns
  }
}

// Common start of both row kernels: locates the row and its target.  An ignored row gets a
// zero gradient and a zero loss, and the function returns false.  Otherwise thread 0 reads
// the target logit into *s_target_logit (NaN for a target outside [0, vocab), which also
// sets status bit 0) before any thread of the block can overwrite the row: the block
// passes at least two barriers before its first gradient store.
template <typename T, int V, bool ALIGNED>
__device__ __forceinline__ bool ce_row_begin(T* logits, int64_t inner, int64_t os, int64_t is,
                                             int vocab, const int64_t* targets, int64_t tos,
                                             int64_t tis, int64_t ignore_index, int write_grad,
                                             CeWork* ws, T** p_out, int* tgt_out,
                                             float* s_target_logit) {
  const int64_t row = blockIdx.x;
  const int64_t o = row / inner, ii = row - (row / inner) * inner;
  T* p = logits + o * os + ii * is;
  const int64_t tgt = targets[o * tos + ii * tis];
  if (tgt == ignore_index) {
    if (write_grad) {
      for (int e = threadIdx.x * V; e < vocab; e += kThreads * V) {
        if constexpr (ALIGNED) {
          store16<true>(p + e, u32x4{0u, 0u, 0u, 0u});
        } else {
          p[e] = Elem<T>::from_f32(0.0f);
        }
      }
    }
    if (threadIdx.x == 0) row_losses(ws)[row] = 0.0f;
    return false;
  }
  const bool bad = tgt < 0 || tgt >= vocab;
  if (threadIdx.x == 0) {
    *s_target_logit = bad ? NAN : Elem<T>::to_f32(p[tgt]);
    if (bad) atomicOr(&ws->status, 1);
  }
  *p_out = p;
  *tgt_out = bad ? -1 : static_cast<int>(tgt);
  return true;
}

// Row loss lse - x_t, written (max - x_t) + ln(sum exp(x - max)): exact when the target is
// the row max and free of the cancellation of two large numbers.
__device__ __forceinline__ float row_loss(float mx, float se, float xt) {
  return (mx - xt) + __logf(se);
}

// Gradient of the target element, (softmax_t - 1) / n_valid, from the exact fp32 target
// logit as exp(x_t - max) / sum: when softmax_t is close to 1 the difference x_t - max is
// small and exact, so the result keeps fp32's relative accuracy (exactly 0 for one class).
__device__ __forceinline__ float target_grad(float mx, float se, float xt, float inv_n) {
  return (exp_shifted(xt, mx) / se - 1.0f) * inv_n;
}

// exp(x - max) is kept in the storage type in place of the logit.  fp16 holds it scaled by
// 2^15 (at most 32768 < 65504), so that values down to 2^-29 keep full fp16 precision
// instead of going subnormal; fp32 and bf16 have fp32's exponent range and need no scale.
template <typename T>
constexpr float kExpScale = std::is_same<T, _Float16>::value ? 32768.0f : 1.0f;

template <typename T, int VPT>
__global__ __launch_bounds__(kThreads) void ce_rows_kernel(
    T* __restrict__ logits, int64_t inner, int64_t os, int64_t is, int vocab,
    const int64_t* __restrict__ targets, int64_t tos, int64_t tis, int64_t ignore_index,
    int write_grad, CeWork* __restrict__ ws) {
  constexpr int V = Elem<T>::VEC;
  __shared__ float red[kWaves];
  __shared__ float s_target_logit;
  T* p = nullptr;
  int tgt = 0;
  if (!ce_row_begin<T, V, true>(logits, inner, os, is, vocab, targets, tos, tis, ignore_index,
                                write_grad, ws, &p, &tgt, &s_target_logit))
    return;

  Vec16<T> v[VPT];
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int e = (threadIdx.x + k * kThreads) * V;
    if (e < vocab) v[k].raw = load16<true>(p + e);
  }
  float mx = -INFINITY;
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int e = (threadIdx.x + k * kThreads) * V;
    if (e < vocab) {
#pragma unroll
      for (int i = 0; i < V; ++i) mx = fmaxf(mx, Elem<T>::to_f32(v[k].e[i]));
    }
  }
  mx = block_reduce_max(mx, red);
  float se = 0.0f;
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int e = (threadIdx.x + k * kThreads) * V;
    if (e < vocab) {
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const float ex = exp_shifted(Elem<T>::to_f32(v[k].e[i]), mx);
        se += ex;
        v[k].e[i] = Elem<T>::from_f32(ex * kExpScale<T>);
      }
    }
  }
  se = block_reduce_sum(se, red);
  const float xt = s_target_logit;
  if (threadIdx.x == 0) row_losses(ws)[blockIdx.x] = row_loss(mx, se, xt);
  if (!write_grad) return;

  const float inv_n = 1.0f / ws->n_valid;
  const float scale = (inv_n / se) * (1.0f / kExpScale<T>);
  const float gt = target_grad(mx, se, xt, inv_n);
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int e = (threadIdx.x + k * kThreads) * V;
    if (e < vocab) {
      float g[V];
#pragma unroll
      for (int i = 0; i < V; ++i) g[i] = Elem<T>::to_f32(v[k].e[i]) * scale;
      if (static_cast<unsigned>(tgt - e) < static_cast<unsigned>(V)) {
#pragma unroll
        for (int i = 0; i < V; ++i)
          if (e + i == tgt) g[i] = gt;
      }
      store_f32<T, true, true>(p + e, g, V);
    }
  }
}

// Rows too long for registers, or not 16-byte aligned: pass 1 streams the row once with an
// online max / sum-exp per thread; pass 2 re-reads it (largely from L2 / MALL) to write the
// gradient.
template <typename T, bool ALIGNED>
__global__ __launch_bounds__(kThreads) void ce_rows_stream_kernel(
    T* __restrict__ logits, int64_t inner, int64_t os, int64_t is, int vocab,
    const int64_t* __restrict__ targets, int64_t tos, int64_t tis, int64_t ignore_index,
    int write_grad, CeWork* __restrict__ ws) {
  constexpr int V = ALIGNED ? Elem<T>::VEC : 1;
  __shared__ float red[kWaves];
  __shared__ float s_target_logit;
  T* p = nullptr;
  int tgt = 0;
  if (!ce_row_begin<T, V, ALIGNED>(logits, inner, os, is, vocab, targets, tos, tis,
                                   ignore_index, write_grad, ws, &p, &tgt, &s_target_logit))
    return;

  auto load = [&](int e, float(&x)[V]) {
    if constexpr (ALIGNED) {
      Vec16<T> r;
      r.raw = load16<false>(p + e);
#pragma unroll
      for (int i = 0; i < V; ++i) x[i] = Elem<T>::to_f32(r.e[i]);
    } else {
      x[0] = Elem<T>::to_f32(p[e]);
    }
  };
  float m = -INFINITY, s = 0.0f;  // running max and sum of exp(x - m)
  for (int e = threadIdx.x * V; e < vocab; e += kThreads * V) {
    float x[V];
    load(e, x);
    float mv = x[0];
#pragma unroll
    for (int i = 1; i < V; ++i) mv = fmaxf(mv, x[i]);
    if (mv > m) {
      s *= exp_shifted(m, mv);
      m = mv;
    }
    if (m == -INFINITY) continue;  // all -inf so far: nothing to add (and -inf - -inf is NaN)
#pragma unroll
    for (int i = 0; i < V; ++i) s += exp_shifted(x[i], m);
  }
  const float mx = block_reduce_max(m, red);
  // rescale each thread's sum to the row max (threads without finite elements hold s = 0)
  const float mine = (s > 0.0f) ? s * exp_shifted(m, mx) : 0.0f;
  const float se = block_reduce_sum(mine, red);
  const float xt = s_target_logit;
  if (threadIdx.x == 0) row_losses(ws)[blockIdx.x] = row_loss(mx, se, xt);
  if (!write_grad) return;

  const float inv_n = 1.0f / ws->n_valid;
  const float scale = inv_n / se;
  const float gt = target_grad(mx, se, xt, inv_n);
  for (int e = threadIdx.x * V; e < vocab; e += kThreads * V) {
    float x[V];
    load(e, x);
    float g[V];
#pragma unroll
    for (int i = 0; i < V; ++i) g[i] = (e + i == tgt) ? gt : exp_shifted(x[i], mx) * scale;
    if constexpr (ALIGNED) {
      store_f32<T, true>(p + e, g, V);
    } else {
      p[e] = Elem<T>::from_f32(g[0]);
    }
  }
}

// loss = sum(row_loss) / n_valid, summed by one block in a fixed order.
__global__ __launch_bounds__(kThreads) void ce_finish_kernel(CeWork* __restrict__ ws,
                                                              int64_t rows,
                                                              float* __restrict__ loss_out) {
  __shared__ float red[kWaves];
  const float* rl = row_losses(ws);
  float acc = 0.0f;
  for (int64_t r = threadIdx.x; r < rows; r += kThreads) acc += rl[r];
  const float total = block_reduce_sum(acc, red);
  if (threadIdx.x == 0) *loss_out = total / ws->n_valid;
}

// In-place gradient scaling by a device scalar; a no-op when the scalar is exactly 1.
// Ignored rows stay zero whatever the scalar is (torch's nll_loss backward leaves them 0).
// Block b scales elements [c*kScaleChunk, (c+1)*kScaleChunk) of row b / chunks.
constexpr int kScaleChunk = 256 * 8;

template <typename T>
__global__ __launch_bounds__(256) void ce_scale_kernel(T* __restrict__ logits, int64_t inner,
                                                       int64_t os, int64_t is, int vocab,
                                                       int64_t chunks,
                                                       const int64_t* __restrict__ targets,
                                                       int64_t tos, int64_t tis,
                                                       int64_t ignore_index,
                                                       const float* __restrict__ scale) {
  const float sc = *scale;
  if (sc == 1.0f) return;
  const int64_t row = blockIdx.x / chunks;
  const int64_t c = blockIdx.x - row * chunks;
  const int64_t o = row / inner, ii = row - (row / inner) * inner;
  if (targets[o * tos + ii * tis] == ignore_index) return;
  T* p = logits + o * os + ii * is;
  const int64_t e0 = c * kScaleChunk;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int64_t e = e0 + k * 256 + threadIdx.x;
    if (e < vocab) p[e] = Elem<T>::from_f32(Elem<T>::to_f32(p[e]) * sc);
  }
}

template <typename T, int VPT>
void launch_rows(void* logits, int64_t inner, int64_t os, int64_t is, int vocab,
                 const int64_t* targets, int64_t tos, int64_t tis, int64_t ignore_index,
                 int write_grad, CeWork* ws, int64_t rows, hipStream_t st) {
  hipLaunchKernelGGL((ce_rows_kernel<T, VPT>), dim3(static_cast<unsigned>(rows)), dim3(kThreads),
                     0, st, static_cast<T*>(logits), inner, os, is, vocab, targets, tos, tis,
                     ignore_index, write_grad, ws);
}

// Register-resident rows for up to 16 vectors per thread (131072 fp16/bf16 or 65536 fp32
// elements); longer or unaligned rows stream.
template <typename T>
void dispatch_rows(bool aligned, void* logits, int64_t inner, int64_t os, int64_t is, int vocab,
                   const int64_t* targets, int64_t tos, int64_t tis, int64_t ignore_index,
                   int write_grad, CeWork* ws, int64_t rows, hipStream_t st) {
  const int64_t per_thread = (static_cast<int64_t>(vocab) + int64_t{kThreads} * Elem<T>::VEC - 1) /
                             (int64_t{kThreads} * Elem<T>::VEC);
  if (aligned) {
#define PT_CE_CASE(N)                                                                        \
  if (per_thread <= N) {                                                                     \
    launch_rows<T, N>(logits, inner, os, is, vocab, targets, tos, tis, ignore_index,         \
                      write_grad, ws, rows, st);                                             \
    return;                                                                                  \
  }
    PT_CE_CASE(1)
    PT_CE_CASE(2)
    PT_CE_CASE(4)
    PT_CE_CASE(8)
    PT_CE_CASE(16)
#undef PT_CE_CASE
    hipLaunchKernelGGL((ce_rows_stream_kernel<T, true>), dim3(static_cast<unsigned>(rows)),
                       dim3(kThreads), 0, st, static_cast<T*>(logits), inner, os, is, vocab,
                       targets, tos, tis, ignore_index, write_grad, ws);
  } else {
    hipLaunchKernelGGL((ce_rows_stream_kernel<T, false>), dim3(static_cast<unsigned>(rows)),
                       dim3(kThreads), 0, st, static_cast<T*>(logits), inner, os, is, vocab,
                       targets, tos, tis, ignore_index, write_grad, ws);
  }
}

}  // namespace
}  // namespace pt

using namespace pt;

extern "C" {

size_t pt_cross_entropy_workspace_bytes(int64_t rows) {
  if (rows < 0) return 0;
  return kHeader + static_cast<size_t>(rows) * sizeof(float);
}

int32_t* pt_cross_entropy_status(void* workspace) {
  return workspace == nullptr ? nullptr : &static_cast<CeWork*>(workspace)->status;
}

int pt_cross_entropy(void* logits, int64_t outer, int64_t inner, int64_t outer_stride,
                     int64_t inner_stride, int64_t vocab, const int64_t* targets,
                     int64_t t_outer_stride, int64_t t_inner_stride, int64_t ignore_index,
                     float* loss_out, int write_grad, void* workspace, size_t workspace_bytes,
                     int dtype, void* stream) {
  if (!valid_dtype(dtype)) return fail(PT_EINVAL, "pt_cross_entropy: unknown dtype code");
  if (outer < 0 || inner < 0 || vocab <= 0)
    return fail(PT_EINVAL, "pt_cross_entropy: bad shape");
  if (vocab > (int64_t{1} << 30)) return fail(PT_EUNSUPPORTED, "pt_cross_entropy: vocab too large");
  const int64_t rows = outer * inner;
  // One 1024-thread workgroup per row; an HSA grid holds at most 2^32 - 1 work-items.
  if (rows * kThreads > 0xffffffffLL)
    return fail(PT_EUNSUPPORTED, "pt_cross_entropy: more than 4194303 rows");
  if (!loss_out || !workspace) return fail(PT_EINVAL, "pt_cross_entropy: null pointer");
  if (rows > 0 && (!logits || !targets)) return fail(PT_EINVAL, "pt_cross_entropy: null pointer");
  if (workspace_bytes < pt_cross_entropy_workspace_bytes(rows) || !aligned16(workspace))
    return fail(PT_EINVAL, "pt_cross_entropy: workspace too small or not 16-byte aligned");
  hipStream_t st = as_stream(stream);
  CeWork* ws = static_cast<CeWork*>(workspace);
  const int64_t inner_nz = inner > 0 ? inner : 1;
  hipLaunchKernelGGL(ce_prepare_kernel, dim3(1), dim3(kThreads), 0, st, targets, inner_nz,
                     t_outer_stride, t_inner_stride, rows, ignore_index, ws, loss_out);
  if (int rc = check_launch("pt_cross_entropy (prepare)")) return rc;
  if (rows == 0) return ok();
  const int esize = dtype_size(dtype);
  const bool aligned = aligned16(logits) && (vocab * esize) % 16 == 0 &&
                       (outer <= 1 || (outer_stride * esize) % 16 == 0) &&
                       (inner <= 1 || (inner_stride * esize) % 16 == 0);
  const int v = static_cast<int>(vocab);
  if (dtype == PT_FLOAT32) {
    dispatch_rows<float>(aligned, logits, inner_nz, outer_stride, inner_stride, v, targets,
                         t_outer_stride, t_inner_stride, ignore_index, write_grad, ws, rows, st);
  } else if (dtype == PT_FLOAT16) {
    dispatch_rows<_Float16>(aligned, logits, inner_nz, outer_stride, inner_stride, v, targets,
                            t_outer_stride, t_inner_stride, ignore_index, write_grad, ws, rows,
                            st);
  } else {
    dispatch_rows<__bf16>(aligned, logits, inner_nz, outer_stride, inner_stride, v, targets,
                          t_outer_stride, t_inner_stride, ignore_index, write_grad, ws, rows, st);
  }
  if (int rc = check_launch("pt_cross_entropy (rows)")) return rc;
  hipLaunchKernelGGL(ce_finish_kernel, dim3(1), dim3(kThreads), 0, st, ws, rows, loss_out);
  return check_launch("pt_cross_entropy (finish)");
}

int pt_cross_entropy_scale_grad(void* logits, int64_t outer, int64_t inner,
                                int64_t outer_stride, int64_t inner_stride, int64_t vocab,
                                const int64_t* targets, int64_t t_outer_stride,
                                int64_t t_inner_stride, int64_t ignore_index,
                                const float* grad_output, int dtype, void* stream) {
  if (!valid_dtype(dtype)) return fail(PT_EINVAL, "pt_cross_entropy_scale_grad: unknown dtype");
  if (outer < 0 || inner < 0 || vocab <= 0 || vocab > (int64_t{1} << 30))
    return fail(PT_EINVAL, "pt_cross_entropy_scale_grad: bad shape");
  const int64_t rows = outer * inner;
  if (rows == 0) return ok();
  if (!logits || !targets || !grad_output)
    return fail(PT_EINVAL, "pt_cross_entropy_scale_grad: null pointer");
  const int64_t chunks = (vocab + kScaleChunk - 1) / kScaleChunk;
  const int64_t blocks = rows * chunks;
  if (blocks * 256 > 0xffffffffLL)
    return fail(PT_EUNSUPPORTED, "pt_cross_entropy_scale_grad: grid too large");
  hipStream_t st = as_stream(stream);
  const int v = static_cast<int>(vocab);
  const int64_t inner_nz = inner > 0 ? inner : 1;
  if (dtype == PT_FLOAT32) {
    hipLaunchKernelGGL(ce_scale_kernel<float>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       st, static_cast<float*>(logits), inner_nz, outer_stride, inner_stride, v,
                       chunks, targets, t_outer_stride, t_inner_stride, ignore_index,
                       grad_output);
  } else if (dtype == PT_FLOAT16) {
    hipLaunchKernelGGL(ce_scale_kernel<_Float16>, dim3(static_cast<unsigned>(blocks)), dim3(256),
                       0, st, static_cast<_Float16*>(logits), inner_nz, outer_stride,
                       inner_stride, v, chunks, targets, t_outer_stride, t_inner_stride,
                       ignore_index, grad_output);
  } else {
    hipLaunchKernelGGL(ce_scale_kernel<__bf16>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       st, static_cast<__bf16*>(logits), inner_nz, outer_stride, inner_stride, v,
                       chunks, targets, t_outer_stride, t_inner_stride, ignore_index,
                       grad_output);
  }
  return check_launch("pt_cross_entropy_scale_grad");
}

}  // extern "C"
