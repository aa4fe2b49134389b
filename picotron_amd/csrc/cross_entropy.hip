// Fused cross-entropy (mean over non-ignored rows) with its gradient written in place.
//
// Reference semantics (AndyMLAndAI/picotron):
//   src/picotron/nn/triton_kernels/cross_entropy.py:97-109 -> F.cross_entropy(logits,
//   targets) with torch's defaults (reduction "mean", ignore_index -100); the Triton kernel
//   at cross_entropy.py:28-45 computes lse - logit[target] per row (forward only).
//   Gradient of the mean: d/dx_j = (softmax_j - [j == target]) / n_valid, 0 on ignored rows.
//
// Passes per call:
//   1. ce_prepare: one block counts non-ignored targets into the workspace (n_valid), and
//      clears the completion ticket and the status word.  No host synchronisation.
//   2. ce_rows: one workgroup per row.  The row is loaded once into registers (1024
//      threads x VPT 16-byte vectors), reduced to max and sum(exp(x - max)) in fp32, and
//      (if requested) the gradient is written over the logits from the same registers,
//      so HBM sees exactly one read and one write of the logits.  Each row's fp32 loss
//      goes to the workspace; the block that takes the last completion ticket sums them
//      in a fixed order and writes the mean, so the loss is bitwise reproducible.
#include <cmath>

#include "pt_common.hpp"

namespace pt {
namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;

struct CeWork {
  float n_valid;     // number of non-ignored targets (exact below 2^24)
  unsigned ticket;   // completion counter of ce_rows blocks
  int status;        // bit 0: a non-ignored target outside [0, vocab)
  int pad;
  // followed by float row_loss[rows], 16-byte aligned
};

constexpr size_t kHeader = 16;

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
    ws->ticket = 0u;
    ws->status = 0;
    if (rows == 0) *loss_out = NAN;  // mean over an empty batch: 0/0, as torch returns
  }
}

// exp(x) via the hardware exp2 unit: x * log2(e), then v_exp_f32.
__device__ __forceinline__ float exp_(float x) { return __expf(x); }

template <typename T, int VPT, bool ALIGNED>
__global__ __launch_bounds__(kThreads) void ce_rows_kernel(
    T* __restrict__ logits, int64_t inner, int64_t os, int64_t is, int vocab,
    const int64_t* __restrict__ targets, int64_t tos, int64_t tis, int64_t ignore_index,
    int write_grad, CeWork* __restrict__ ws, float* __restrict__ loss_out, int64_t rows) {
  constexpr int V = ALIGNED ? Elem<T>::VEC : 1;
  __shared__ float red[kWaves];
  __shared__ float s_target_logit;
  __shared__ bool s_last;
  float* row_loss = reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + kHeader);

  const int64_t row = blockIdx.x;
  const int64_t o = row / inner, ii = row - (row / inner) * inner;
  T* p = logits + o * os + ii * is;
  const int64_t tgt = targets[o * tos + ii * tis];
  const bool ignored = tgt == ignore_index;
  const bool bad = !ignored && (tgt < 0 || tgt >= vocab);

  if (ignored) {
    if (write_grad) {
      for (int e = threadIdx.x * V; e < vocab; e += kThreads * V) {
        if constexpr (ALIGNED) {
          store16<true>(p + e, u32x4{0u, 0u, 0u, 0u});
        } else {
          p[e] = Elem<T>::from_f32(0.0f);
        }
      }
    }
    if (threadIdx.x == 0) row_loss[row] = 0.0f;
  } else {
    if (threadIdx.x == 0) {
      // Read before any thread of this block overwrites the row (barriers follow).
      s_target_logit = bad ? NAN : Elem<T>::to_f32(p[tgt]);
      if (bad) atomicOr(&ws->status, 1);
    }
    Vec16<T> v[VPT];
    float mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const int e = (threadIdx.x + k * kThreads) * V;
      if constexpr (ALIGNED) {
        if (e < vocab) {
          v[k].raw = load16<true>(p + e);
#pragma unroll
          for (int i = 0; i < V; ++i) mx = fmaxf(mx, Elem<T>::to_f32(v[k].e[i]));
        }
      } else {
        if (e < vocab) {
          v[k].e[0] = p[e];
          mx = fmaxf(mx, Elem<T>::to_f32(v[k].e[0]));
        }
      }
    }
    mx = block_reduce_max(mx, red);
    float se = 0.0f;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const int e = (threadIdx.x + k * kThreads) * V;
      if (e < vocab) {
#pragma unroll
        for (int i = 0; i < V; ++i) se += exp_(Elem<T>::to_f32(v[k].e[i]) - mx);
      }
    }
    se = block_reduce_sum(se, red);
    const float lse = mx + __logf(se);
    if (threadIdx.x == 0) row_loss[row] = lse - s_target_logit;

    if (write_grad) {
      const float inv_n = 1.0f / ws->n_valid;
#pragma unroll
      for (int k = 0; k < VPT; ++k) {
        const int e = (threadIdx.x + k * kThreads) * V;
        if (e < vocab) {
          float g[V];
#pragma unroll
          for (int i = 0; i < V; ++i) {
            const float pr = exp_(Elem<T>::to_f32(v[k].e[i]) - lse);
            g[i] = (pr - ((e + i) == tgt ? 1.0f : 0.0f)) * inv_n;
          }
          if constexpr (ALIGNED) {
            Vec16<T> out;
#pragma unroll
            for (int i = 0; i < V; ++i) out.e[i] = Elem<T>::from_f32(g[i]);
            store16<true>(p + e, out.raw);
          } else {
            p[e] = Elem<T>::from_f32(g[0]);
          }
        }
      }
    }
  }

  // Completion ticket: the last block to finish sums the per-row losses.
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned t = atomicAdd(&ws->ticket, 1u);
    s_last = (t == static_cast<unsigned>(rows - 1));
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  float acc = 0.0f;
  for (int64_t r = threadIdx.x; r < rows; r += kThreads) acc += row_loss[r];
  const float total = block_reduce_sum(acc, red);
  if (threadIdx.x == 0) {
    *loss_out = total / ws->n_valid;
    ws->ticket = 0u;
  }
}

// Rows too long for registers (or not 16-byte aligned): pass 1 streams the row once
// with an online max / sum-exp per thread; pass 2 re-reads it (mostly from L2 / MALL) to
// write the gradient.
template <typename T, bool ALIGNED>
__global__ __launch_bounds__(kThreads) void ce_rows_stream_kernel(
    T* __restrict__ logits, int64_t inner, int64_t os, int64_t is, int vocab,
    const int64_t* __restrict__ targets, int64_t tos, int64_t tis, int64_t ignore_index,
    int write_grad, CeWork* __restrict__ ws, float* __restrict__ loss_out, int64_t rows) {
  constexpr int V = ALIGNED ? Elem<T>::VEC : 1;
  __shared__ float red[kWaves];
  __shared__ float s_target_logit;
  __shared__ bool s_last;
  float* row_loss = reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + kHeader);

  const int64_t row = blockIdx.x;
  const int64_t o = row / inner, ii = row - (row / inner) * inner;
  T* p = logits + o * os + ii * is;
  const int64_t tgt = targets[o * tos + ii * tis];
  const bool ignored = tgt == ignore_index;
  const bool bad = !ignored && (tgt < 0 || tgt >= vocab);

  if (ignored) {
    if (write_grad) {
      for (int e = threadIdx.x * V; e < vocab; e += kThreads * V) {
        if constexpr (ALIGNED) {
          store16<false>(p + e, u32x4{0u, 0u, 0u, 0u});
        } else {
          p[e] = Elem<T>::from_f32(0.0f);
        }
      }
    }
    if (threadIdx.x == 0) row_loss[row] = 0.0f;
  } else {
    if (threadIdx.x == 0) {
      s_target_logit = bad ? NAN : Elem<T>::to_f32(p[tgt]);
      if (bad) atomicOr(&ws->status, 1);
    }
    float m = -INFINITY, se = 0.0f;
    for (int e = threadIdx.x * V; e < vocab; e += kThreads * V) {
      float x[V];
      if constexpr (ALIGNED) {
        load_f32<T, true>(p + e, x, V);
      } else {
        x[0] = Elem<T>::to_f32(p[e]);
      }
      float mv = x[0];
#pragma unroll
      for (int i = 1; i < V; ++i) mv = fmaxf(mv, x[i]);
      if (mv > m) {
        se *= exp_(m - mv);
        m = mv;
      }
#pragma unroll
      for (int i = 0; i < V; ++i) se += exp_(x[i] - m);
    }
    const float mx = block_reduce_max(m, red);
    // rescale each thread's partial sum to the row maximum (threads without elements
    // hold m = -inf and se = 0, contributing 0)
    const float mine = (se > 0.0f) ? se * exp_(m - mx) : 0.0f;
    const float total = block_reduce_sum(mine, red);
    const float lse = mx + __logf(total);
    if (threadIdx.x == 0) row_loss[row] = lse - s_target_logit;

    if (write_grad) {
      const float inv_n = 1.0f / ws->n_valid;
      for (int e = threadIdx.x * V; e < vocab; e += kThreads * V) {
        float x[V];
        if constexpr (ALIGNED) {
          load_f32<T, true>(p + e, x, V);
        } else {
          x[0] = Elem<T>::to_f32(p[e]);
        }
        float gr[V];
#pragma unroll
        for (int i = 0; i < V; ++i) {
          gr[i] = (exp_(x[i] - lse) - ((e + i) == tgt ? 1.0f : 0.0f)) * inv_n;
        }
        if constexpr (ALIGNED) {
          store_f32<T, true>(p + e, gr, V);
        } else {
          p[e] = Elem<T>::from_f32(gr[0]);
        }
      }
    }
  }

  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned t = atomicAdd(&ws->ticket, 1u);
    s_last = (t == static_cast<unsigned>(rows - 1));
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  float acc = 0.0f;
  for (int64_t r = threadIdx.x; r < rows; r += kThreads) acc += row_loss[r];
  const float total = block_reduce_sum(acc, red);
  if (threadIdx.x == 0) {
    *loss_out = total / ws->n_valid;
    ws->ticket = 0u;
  }
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

template <typename T, int VPT, bool ALIGNED>
void launch_rows(void* logits, int64_t inner, int64_t os, int64_t is, int vocab,
                 const int64_t* targets, int64_t tos, int64_t tis, int64_t ignore_index,
                 int write_grad, CeWork* ws, float* loss_out, int64_t rows, hipStream_t st) {
  hipLaunchKernelGGL((ce_rows_kernel<T, VPT, ALIGNED>), dim3(static_cast<unsigned>(rows)),
                     dim3(kThreads), 0, st, static_cast<T*>(logits), inner, os, is, vocab,
                     targets, tos, tis, ignore_index, write_grad, ws, loss_out, rows);
}

template <typename T>
int dispatch_rows(bool aligned, void* logits, int64_t inner, int64_t os, int64_t is, int vocab,
                  const int64_t* targets, int64_t tos, int64_t tis, int64_t ignore_index,
                  int write_grad, CeWork* ws, float* loss_out, int64_t rows, hipStream_t st) {
  const int V = aligned ? Elem<T>::VEC : 1;
  const int64_t per_thread = (static_cast<int64_t>(vocab) + int64_t{kThreads} * V - 1) /
                             (int64_t{kThreads} * V);
#define PT_CE_CASE(N)                                                                         \
  if (per_thread <= N) {                                                                      \
    launch_rows<T, N, true>(logits, inner, os, is, vocab, targets, tos, tis, ignore_index,    \
                            write_grad, ws, loss_out, rows, st);                              \
    return PT_OK;                                                                             \
  }
  if (aligned) {
    PT_CE_CASE(1)
    PT_CE_CASE(2)
    PT_CE_CASE(4)
    PT_CE_CASE(8)
    PT_CE_CASE(16)
  }
#undef PT_CE_CASE
  if (aligned) {
    hipLaunchKernelGGL((ce_rows_stream_kernel<T, true>), dim3(static_cast<unsigned>(rows)),
                       dim3(kThreads), 0, st, static_cast<T*>(logits), inner, os, is, vocab,
                       targets, tos, tis, ignore_index, write_grad, ws, loss_out, rows);
  } else {
    hipLaunchKernelGGL((ce_rows_stream_kernel<T, false>), dim3(static_cast<unsigned>(rows)),
                       dim3(kThreads), 0, st, static_cast<T*>(logits), inner, os, is, vocab,
                       targets, tos, tis, ignore_index, write_grad, ws, loss_out, rows);
  }
  return PT_OK;
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
  int rc;
  const int v = static_cast<int>(vocab);
  if (dtype == PT_FLOAT32) {
    rc = dispatch_rows<float>(aligned, logits, inner_nz, outer_stride, inner_stride, v, targets,
                              t_outer_stride, t_inner_stride, ignore_index, write_grad, ws,
                              loss_out, rows, st);
  } else if (dtype == PT_FLOAT16) {
    rc = dispatch_rows<_Float16>(aligned, logits, inner_nz, outer_stride, inner_stride, v,
                                 targets, t_outer_stride, t_inner_stride, ignore_index,
                                 write_grad, ws, loss_out, rows, st);
  } else {
    rc = dispatch_rows<__bf16>(aligned, logits, inner_nz, outer_stride, inner_stride, v, targets,
                               t_outer_stride, t_inner_stride, ignore_index, write_grad, ws,
                               loss_out, rows, st);
  }
  if (rc != PT_OK)
    return fail(rc, "pt_cross_entropy: vocab " + std::to_string(vocab) +
                        " exceeds the register-resident row capacity");
  return check_launch("pt_cross_entropy");
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
