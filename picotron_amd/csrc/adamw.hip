// Multi-tensor AdamW step for gfx950 (fp32 parameters and states).
//
// Reference semantics: AndyMLAndAI/picotron builds torch.optim.AdamW(params, lr, betas,
// eps, weight_decay) (src/picotron/training/train_loop.py:308-325) and its fused hook
// (src/picotron/nn/triton_kernels/adamw.py:14-47) always falls back to
// optimizer.step().  The arithmetic restated here is torch's single-tensor AdamW
// (amsgrad=False, maximize=False), per element, in fp32:
//   p  = p * (1 - lr*wd)
//   m  = lerp(m, g, 1 - beta1)          (m + w*(g - m) for w < 0.5, else g - (g - m)*(1 - w))
//   v  = v * beta2 + ((1 - beta2) * g) * g
//   p  = p + (-step_size) * (m / (sqrt(v) / bc2_sqrt + eps))
// with step_size = lr / (1 - beta1^t) and bc2_sqrt = (1 - beta2^t)^0.5 computed in double
// on the host, then rounded to fp32 as torch rounds Python scalars for fp32 tensors.
//
// One launch covers every tensor: block b finds its tensor by a 16-way search over the
// per-tensor first-block indices in the device table, then streams its chunk of
// kBlockElems elements (16-byte vectors when all four pointers are aligned).
//
// Gradient clipping fused into the step (torch.nn.utils.clip_grad_norm_, which the train
// loop runs right before the step, src/picotron/training/train_loop.py:163-168,338-350):
// pt_clip_grad_norm computes total_norm = ||all grads||_2 and
// clip_coef = min(max_norm / (total_norm + 1e-6), 1) on the device (one read of the
// grads, per-block fp32 partial sums of squares added in double in a fixed order), and
// pt_adamw_step_scaled multiplies each gradient by that device scalar as it reads it --
// optionally writing the clipped gradient back -- instead of a separate read-modify-write
// pass over every gradient.
#include <cmath>

#include "pt_common.hpp"

namespace pt {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 1;
constexpr int64_t kBlockElems = int64_t{kThreads} * 4 * kUnroll;  // 1024 fp32 per block

struct AdamRec {
  int64_t p, g, m, v, n, first_block;
};

struct AdamScalars {
  float decay;      // 1 - lr*wd
  float w1;         // 1 - beta1 (lerp weight)
  float beta2;
  float omb2;       // 1 - beta2
  float neg_step;   // -lr / (1 - beta1^t)
  float bc2_sqrt;   // sqrt(1 - beta2^t)
  float eps;
};

// The record whose blocks include block `blk`: the last i with table[i].first_block <= blk
// (first_block increases from 0 along the table).  A kSearchWays-way search: each round
// loads its probes' first_block values together (independent scalar loads, one wait), so a
// table of n records costs about log17(n) dependent rounds instead of a binary search's
// log2(n): one round up to 17 records, two up to 273, three up to 4369.
// Every round shrinks [lo, hi] (lo rises or hi falls), so the loop ends on any table.
// Block indexes and record counts are below 2^24 (checked before every launch), so the
// search runs in 32 bits and reads the low word of each first_block.
constexpr int kSearchWays = 16;

__device__ __forceinline__ uint32_t first_block_of(const AdamRec* __restrict__ table, uint32_t i) {
  return *reinterpret_cast<const uint32_t*>(&table[i].first_block);
}

__device__ __forceinline__ int64_t find_tensor(const AdamRec* __restrict__ table, int64_t ntensors,
                                               int64_t block) {
  const uint32_t blk = static_cast<uint32_t>(block);
  uint32_t lo = 0, hi = static_cast<uint32_t>(ntensors - 1);
  while (lo < hi) {
    // probe k at lo + ceil((k + 1) * len / kSearchWays): nondecreasing, in (lo, hi], and
    // every index of (lo, hi] when len <= kSearchWays (the last round)
    const uint32_t len = hi - lo;
    uint32_t fb[kSearchWays];
#pragma unroll
    for (int k = 0; k < kSearchWays; ++k)
      fb[k] = first_block_of(table, lo + ((k + 1) * len + kSearchWays - 1) / kSearchWays);
    uint32_t new_lo = lo, new_hi = hi;
#pragma unroll
    for (int k = kSearchWays - 1; k >= 0; --k) {
      const uint32_t probe = lo + ((k + 1) * len + kSearchWays - 1) / kSearchWays;
      if (fb[k] <= blk) {
        if (probe > new_lo) new_lo = probe;
      } else {
        new_hi = probe - 1;  // the loop runs downward: ends at the first probe past blk
      }
    }
    lo = new_lo;
    hi = new_hi;
  }
  return lo;
}

__device__ __forceinline__ void adam_elem(float& p, float g, float& m, float& v,
                                          const AdamScalars& s) {
  p = p * s.decay;
  m = (fabsf(s.w1) < 0.5f) ? m + s.w1 * (g - m) : g - (g - m) * (1.0f - s.w1);
  v = v * s.beta2;
  v = v + (s.omb2 * g) * g;
  const float denom = __fdiv_rn(__fsqrt_rn(v), s.bc2_sqrt) + s.eps;
  p = p + s.neg_step * __fdiv_rn(m, denom);
}

// Step counts on the device (torch's capturable AdamW keeps each parameter's step as an
// fp32 scalar next to it, advanced by the caller before the update): `steps[i]` is the
// address of table row i's step.  Each workgroup reads its tensor's step and forms the bias
// corrections in fp32, step_size = lr / (1 - beta1^t) and bc2_sqrt = sqrt(1 - beta2^t), in
// place of the host-computed ones; nothing in the launch depends on the step's value, so a
// captured graph replays correctly as the step advances.
struct DevStep {
  const int64_t* steps;
  float lr, beta1, beta2;
};

__device__ __forceinline__ void device_step_scalars(AdamScalars& s, const DevStep& d, int64_t row) {
  const float t = *as_global<const float>(d.steps[row]);
  s.neg_step = -__fdiv_rn(d.lr, 1.0f - powf(d.beta1, t));
  s.bc2_sqrt = __fsqrt_rn(1.0f - powf(d.beta2, t));
}

// SCALED: the gradient is multiplied by *grad_scale as it is read (torch's clipping
// multiplies the stored gradient, g = g * coef, before the step reads it), and written back
// when write_grad != 0.  DEVSTEP: bias corrections from the device step counts (DevStep).
// `found` (may be null): the overflow flag of the gradient statistics, read on the device;
// when it is set the step is skipped -- parameters and moments untouched -- and each
// workgroup only unscales its block of the gradient by *inv_scale, as GradScaler.unscale_
// leaves a skipped step's gradients (the caller advances no step count then).
template <bool SCALED, bool DEVSTEP>
__global__ __launch_bounds__(kThreads) void adamw_kernel(const AdamRec* __restrict__ table,
                                                         int64_t ntensors, AdamScalars s,
                                                         const float* __restrict__ grad_scale,
                                                         int write_grad, DevStep ds,
                                                         const int* __restrict__ found,
                                                         const float* __restrict__ inv_scale) {
  const int64_t blk = blockIdx.x;
  const int64_t row = find_tensor(table, ntensors, blk);
  const AdamRec r = table[row];
  const int64_t start = (blk - r.first_block) * kBlockElems;
  const int64_t end = (start + kBlockElems < r.n) ? start + kBlockElems : r.n;
  const gptr<float> G = as_global<float>(r.g);
  if (found != nullptr && *found != 0) {
    const float is = *inv_scale;
    for (int64_t i = start + threadIdx.x; i < end; i += kThreads) G[i] = G[i] * is;
    return;
  }
  if constexpr (DEVSTEP) device_step_scalars(s, ds, row);
  const float gs = SCALED ? *grad_scale : 1.0f;
  const gptr<float> P = as_global<float>(r.p);
  const gptr<float> M = as_global<float>(r.m);
  const gptr<float> Vv = as_global<float>(r.v);
  const bool vec_ok = ((r.p | r.g | r.m | r.v) & 15) == 0;

  if (vec_ok && end - start == kBlockElems) {
    // The block's chunk of each stream through a buffer resource, so that the stores can
    // be written through L2 (nontemporal, device scope): 1.2e9 parameters, one process,
    // alternated: 5282 against 5290 us per step (one tensor) and 5298 against 5329 (100
    // tensors) with nontemporal global stores.
    constexpr int kChunkBytes = static_cast<int>(kBlockElems * 4);
    const auto pb = uniform_buffer(reinterpret_cast<const void*>(r.p + start * 4), kChunkBytes);
    const auto mb = uniform_buffer(reinterpret_cast<const void*>(r.m + start * 4), kChunkBytes);
    const auto vb = uniform_buffer(reinterpret_cast<const void*>(r.v + start * 4), kChunkBytes);
    const auto gb = uniform_buffer(reinterpret_cast<const void*>(r.g + start * 4), kChunkBytes);
    f32x4 pv[kUnroll], gv[kUnroll], mv[kUnroll], vv[kUnroll];
#pragma unroll
    for (int k = 0; k < kUnroll; ++k) {
      const int64_t i = start + (static_cast<int64_t>(k) * kThreads + threadIdx.x) * 4;
      pv[k] = __builtin_nontemporal_load(reinterpret_cast<gptr<const f32x4>>(P + i));
      gv[k] = __builtin_nontemporal_load(reinterpret_cast<gptr<const f32x4>>(G + i));
      mv[k] = __builtin_nontemporal_load(reinterpret_cast<gptr<const f32x4>>(M + i));
      vv[k] = __builtin_nontemporal_load(reinterpret_cast<gptr<const f32x4>>(Vv + i));
    }
#pragma unroll
    for (int k = 0; k < kUnroll; ++k) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float pp = pv[k][j], mm = mv[k][j], v2 = vv[k][j];
        if constexpr (SCALED) gv[k][j] = gv[k][j] * gs;
        adam_elem(pp, gv[k][j], mm, v2, s);
        pv[k][j] = pp;
        mv[k][j] = mm;
        vv[k][j] = v2;
      }
      const int off = (k * kThreads + static_cast<int>(threadIdx.x)) * 16;
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, pv[k]), pb, off, 0, kWriteThrough);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, mv[k]), mb, off, 0, kWriteThrough);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, vv[k]), vb, off, 0, kWriteThrough);
      if (SCALED && write_grad)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, gv[k]), gb, off, 0, kWriteThrough);
    }
  } else {
    for (int64_t i = start + threadIdx.x; i < end; i += kThreads) {
      float pp = P[i], mm = M[i], v2 = Vv[i];
      float g = G[i];
      if constexpr (SCALED) g = g * gs;
      adam_elem(pp, g, mm, v2, s);
      P[i] = pp;
      M[i] = mm;
      Vv[i] = v2;
      if (SCALED && write_grad) G[i] = g;
    }
  }
}

// Statistics of the gradients (table layout as the step; only the g, n and first_block
// fields are read): per workgroup, the partial sum of squares of u = g * inv_scale (the
// unscaled gradient, inv_scale = 1 when absent) and, when `nonfinite` is given, whether any
// g it read is inf or NaN.  A grid of a few workgroups per CU walks the table's blocks,
// kWalkUnroll at a time (their loads in flight together), so the finish pass adds a few
// thousand partials; the walk order is fixed by the grid, so the sum is reproducible.
constexpr int kWalkUnroll = 4;

struct BlockSpan {
  gptr<float> g;
  int64_t start, end;
  bool vec;  // a whole 16-byte-aligned block: one float4 per thread
};

// `row` carries the record of the previous block of the same walk step (-1 for the first):
// consecutive blocks stay in that record or move on by one, since every record has a block.
__device__ __forceinline__ BlockSpan block_span(const AdamRec* __restrict__ table,
                                                int64_t ntensors, int64_t vb, int64_t& row) {
  if (row < 0) {
    row = find_tensor(table, ntensors, vb);
  } else {
    while (row + 1 < ntensors && table[row + 1].first_block <= vb) ++row;
  }
  const AdamRec r = table[row];
  BlockSpan b;
  b.g = as_global<float>(r.g);
  b.start = (vb - r.first_block) * kBlockElems;
  b.end = (b.start + kBlockElems < r.n) ? b.start + kBlockElems : r.n;
  b.vec = (r.g & 15) == 0 && b.end - b.start == kBlockElems;
  return b;
}

__global__ __launch_bounds__(kThreads) void grad_stats_kernel(const AdamRec* __restrict__ table,
                                                              int64_t ntensors, int64_t nblocks,
                                                              const float* __restrict__ inv_scale,
                                                              float* __restrict__ partial,
                                                              int* __restrict__ nonfinite) {
  __shared__ float red[kThreads / 64];
  const float s = inv_scale != nullptr ? *inv_scale : 1.0f;
  float acc = 0.0f;
  bool bad = false;
  const int64_t step = static_cast<int64_t>(gridDim.x) * kWalkUnroll;
  for (int64_t base = static_cast<int64_t>(blockIdx.x) * kWalkUnroll; base < nblocks; base += step) {
    BlockSpan sp[kWalkUnroll];
    f32x4 gv[kWalkUnroll];
    int64_t row = -1;
#pragma unroll
    for (int u = 0; u < kWalkUnroll; ++u) {
      sp[u].g = nullptr;
      sp[u].vec = false;
      sp[u].start = sp[u].end = 0;
      if (base + u < nblocks) {
        sp[u] = block_span(table, ntensors, base + u, row);
        if (sp[u].vec)
          gv[u] = __builtin_nontemporal_load(
              reinterpret_cast<gptr<const f32x4>>(sp[u].g + sp[u].start + threadIdx.x * 4));
      }
    }
#pragma unroll
    for (int u = 0; u < kWalkUnroll; ++u) {
      if (sp[u].vec) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float x = gv[u][j] * s;
          acc += x * x;
          bad |= !__builtin_isfinite(gv[u][j]);
        }
      } else {
        for (int64_t i = sp[u].start + threadIdx.x; i < sp[u].end; i += kThreads) {
          const float x = sp[u].g[i] * s;
          acc += x * x;
          bad |= !__builtin_isfinite(sp[u].g[i]);
        }
      }
    }
  }
  acc = wave_sum(acc);
  const int any_bad = __syncthreads_or(bad ? 1 : 0);
  if (threadIdx.x % 64 == 0) red[threadIdx.x / 64] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.0f;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) t += red[w];
    partial[blockIdx.x] = t;
    if (nonfinite != nullptr) nonfinite[blockIdx.x] = any_bad;
  }
}

// Number of workgroups of the statistics and scaling walks.
int walk_grid(int64_t nblocks) {
  const int64_t want = (nblocks + kWalkUnroll - 1) / kWalkUnroll;
  const int64_t cap = static_cast<int64_t>(num_cus()) * 32;
  return static_cast<int>(want < cap ? (want < 1 ? 1 : want) : cap);
}

// total_norm = sqrt(sum of the partials, added in double in a fixed order), the gradient
// multiplier and the non-finite flag, as device scalars.  With max_norm >= 0 the clip
// coefficient is computed as both clipping routines compute it,
//   c = (1 / (total_norm + 1e-6)) * max_norm   (Python's max_norm / tensor),
// and applied as torch.nn.utils.clip_grad_norm_ does (CLIP_CLAMP: min(c, 1), NaN stays NaN)
// or as picotron's ZeRO optimizer does (CLIP_IF_BELOW_ONE: c if c < 1 else 1).  The
// multiplier is inv_scale * coefficient (inv_scale = 1 when absent).
enum ClipMode { CLIP_CLAMP = 0, CLIP_IF_BELOW_ONE = 1 };

__global__ __launch_bounds__(1024) void grad_stats_finish_kernel(
    const float* __restrict__ partial, const int* __restrict__ nonfinite, int64_t nblocks,
    float max_norm, int clip_mode, const float* __restrict__ inv_scale,
    float* __restrict__ total_out, float* __restrict__ scale_out, int* __restrict__ found_out) {
  __shared__ double red[16];
  double acc = 0.0;
  int bad = 0;
  for (int64_t i = threadIdx.x; i < nblocks; i += 1024) {
    acc += static_cast<double>(partial[i]);
    if (nonfinite != nullptr) bad |= nonfinite[i];
  }
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) acc += __shfl_xor(acc, m);
  const int any_bad = __syncthreads_or(bad);
  if (threadIdx.x % 64 == 0) red[threadIdx.x / 64] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    double t = 0.0;
#pragma unroll
    for (int w = 0; w < 16; ++w) t += red[w];
    const float total = static_cast<float>(sqrt(t));
    float coef = 1.0f;
    if (max_norm >= 0.0f) {
      const float c = (1.0f / (total + 1e-6f)) * max_norm;
      coef = clip_mode == CLIP_CLAMP ? (c > 1.0f ? 1.0f : c) : (c < 1.0f ? c : 1.0f);
    }
    *total_out = total;
    *scale_out = (inv_scale != nullptr ? *inv_scale : 1.0f) * coef;
    if (found_out != nullptr) *found_out = any_bad;
  }
}

// In-place g *= *scale over every gradient of the table; nothing at all when the scale is
// exactly 1 (a clip that does not clip).  Walks the table like grad_stats_kernel.
__global__ __launch_bounds__(kThreads) void grad_scale_kernel(const AdamRec* __restrict__ table,
                                                              int64_t ntensors, int64_t nblocks,
                                                              const float* __restrict__ scale) {
  const float s = *scale;
  if (s == 1.0f) return;
  const int64_t step = static_cast<int64_t>(gridDim.x) * kWalkUnroll;
  for (int64_t base = static_cast<int64_t>(blockIdx.x) * kWalkUnroll; base < nblocks; base += step) {
    BlockSpan sp[kWalkUnroll];
    f32x4 gv[kWalkUnroll];
    int64_t row = -1;
#pragma unroll
    for (int u = 0; u < kWalkUnroll; ++u) {
      sp[u].g = nullptr;
      sp[u].vec = false;
      sp[u].start = sp[u].end = 0;
      if (base + u < nblocks) {
        sp[u] = block_span(table, ntensors, base + u, row);
        if (sp[u].vec)
          gv[u] = __builtin_nontemporal_load(
              reinterpret_cast<gptr<const f32x4>>(sp[u].g + sp[u].start + threadIdx.x * 4));
      }
    }
#pragma unroll
    for (int u = 0; u < kWalkUnroll; ++u) {
      const gptr<float> G = sp[u].g;
      if (sp[u].vec) {
#pragma unroll
        for (int j = 0; j < 4; ++j) gv[u][j] = gv[u][j] * s;
        __builtin_nontemporal_store(gv[u], reinterpret_cast<gptr<f32x4>>(G + sp[u].start + threadIdx.x * 4));
      } else {
        for (int64_t i = sp[u].start + threadIdx.x; i < sp[u].end; i += kThreads) G[i] = G[i] * s;
      }
    }
  }
}

// Resident step workgroups per CU (each thread keeps four 16-byte loads in flight): at
// 1.2e9 parameters the plain step measured 5.67-5.75 ms with the full 8 and 5.22-5.62 ms
// at 3; with the clip fused, 7.50-7.52 ms against 7.10-7.11 ms.  PT_ADAMW_BLOCKS_PER_CU
// overrides it (0: no limit).
int step_occupancy() {
  static const int v = static_cast<int>(env_int("PT_ADAMW_BLOCKS_PER_CU", 3));
  return v;
}

template <bool SCALED, bool DEVSTEP>
int launch_step(const int64_t* table, int64_t n_tensors, int64_t total_blocks, AdamScalars s,
                const float* grad_scale, int write_grad, DevStep d, void* stream, const char* fn,
                const int* found = nullptr, const float* inv_scale = nullptr) {
  const auto kernel = adamw_kernel<SCALED, DEVSTEP>;
  size_t lds = occupancy_lds(step_occupancy(), 0);
  if (allow_dynamic_lds(reinterpret_cast<const void*>(kernel), lds) != PT_OK) lds = 0;
  hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(total_blocks)), dim3(kThreads), lds,
                     as_stream(stream), reinterpret_cast<const AdamRec*>(table), n_tensors, s,
                     grad_scale, write_grad, d, found, inv_scale);
  return check_launch(fn);
}

AdamScalars host_scalars(double lr, double beta1, double beta2, double eps, double weight_decay,
                         double step) {
  // torch.optim.adamw._single_tensor_adamw, in Python floats (double):
  const double bias_correction1 = 1.0 - std::pow(beta1, step);
  const double bias_correction2 = 1.0 - std::pow(beta2, step);
  const double step_size = lr / bias_correction1;
  const double bc2_sqrt = std::pow(bias_correction2, 0.5);
  AdamScalars s;
  s.decay = static_cast<float>(1.0 - lr * weight_decay);
  s.w1 = static_cast<float>(1.0 - beta1);
  s.beta2 = static_cast<float>(beta2);
  s.omb2 = static_cast<float>(1.0 - beta2);
  s.neg_step = static_cast<float>(-step_size);
  s.bc2_sqrt = static_cast<float>(bc2_sqrt);
  s.eps = static_cast<float>(eps);
  return s;
}

int check_table(const char* fn, const int64_t* table, int64_t n_tensors, int64_t total_blocks) {
  const std::string name(fn);
  if (n_tensors < 0 || total_blocks < 0) return fail(PT_EINVAL, name + ": negative count");
  if (n_tensors == 0 || total_blocks == 0) return -1;  // nothing to do
  if (!table) return fail(PT_EINVAL, name + ": null table");
  if ((reinterpret_cast<uintptr_t>(table) & 7u) != 0)
    return fail(PT_EINVAL, name + ": table not 8-byte aligned");
  if (total_blocks * kThreads > 0xffffffffLL)
    return fail(PT_EUNSUPPORTED, name + ": more than 2^24 blocks in one launch");
  if (n_tensors > total_blocks)
    return fail(PT_EINVAL, name + ": more records than blocks (every record needs a block; "
                                  "leave empty tensors out of the table)");
  return PT_OK;
}

}  // namespace
}  // namespace pt

using namespace pt;

extern "C" {

int64_t pt_adamw_block_elems(void) { return kBlockElems; }

int pt_adamw_step(const int64_t* table, int64_t n_tensors, int64_t total_blocks, double lr,
                  double beta1, double beta2, double eps, double weight_decay, double step,
                  void* stream) {
  const int rc = check_table("pt_adamw_step", table, n_tensors, total_blocks);
  if (rc == -1) return ok();
  if (rc != PT_OK) return rc;
  if (!(step >= 1.0)) return fail(PT_EINVAL, "pt_adamw_step: step must be >= 1");
  return launch_step<false, false>(table, n_tensors, total_blocks,
                                   host_scalars(lr, beta1, beta2, eps, weight_decay, step), nullptr,
                                   0, DevStep{}, stream, "pt_adamw_step");
}

int pt_adamw_step_scaled(const int64_t* table, int64_t n_tensors, int64_t total_blocks, double lr,
                         double beta1, double beta2, double eps, double weight_decay, double step,
                         const float* grad_scale, int write_grad, void* stream) {
  const int rc = check_table("pt_adamw_step_scaled", table, n_tensors, total_blocks);
  if (rc == -1) return ok();
  if (rc != PT_OK) return rc;
  if (!(step >= 1.0)) return fail(PT_EINVAL, "pt_adamw_step_scaled: step must be >= 1");
  if (!grad_scale) return fail(PT_EINVAL, "pt_adamw_step_scaled: null grad_scale");
  return launch_step<true, false>(table, n_tensors, total_blocks,
                                  host_scalars(lr, beta1, beta2, eps, weight_decay, step),
                                  grad_scale, write_grad, DevStep{}, stream, "pt_adamw_step_scaled");
}

int pt_adamw_step_device_step(const int64_t* table, int64_t n_tensors, int64_t total_blocks,
                              const int64_t* step_table, double lr, double beta1, double beta2,
                              double eps, double weight_decay, const float* grad_scale,
                              int write_grad, void* stream) {
  const int rc = check_table("pt_adamw_step_device_step", table, n_tensors, total_blocks);
  if (rc == -1) return ok();
  if (rc != PT_OK) return rc;
  if (!step_table || (reinterpret_cast<uintptr_t>(step_table) & 7u) != 0)
    return fail(PT_EINVAL, "pt_adamw_step_device_step: null or misaligned step table");
  // decay, lerp weight, beta2 and eps as for a host step; the bias corrections per workgroup
  const AdamScalars s = host_scalars(lr, beta1, beta2, eps, weight_decay, 1.0);
  const DevStep d{step_table, static_cast<float>(lr), static_cast<float>(beta1),
                  static_cast<float>(beta2)};
  if (grad_scale)
    return launch_step<true, true>(table, n_tensors, total_blocks, s, grad_scale, write_grad, d,
                                   stream, "pt_adamw_step_device_step");
  return launch_step<false, true>(table, n_tensors, total_blocks, s, nullptr, 0, d, stream,
                                  "pt_adamw_step_device_step");
}

int pt_adamw_step_device_step_guarded(const int64_t* table, int64_t n_tensors,
                                      int64_t total_blocks, const int64_t* step_table, double lr,
                                      double beta1, double beta2, double eps,
                                      double weight_decay, const float* grad_scale,
                                      int write_grad, const int32_t* found_inf,
                                      const float* inv_scale, void* stream) {
  const char* fn = "pt_adamw_step_device_step_guarded";
  const int rc = check_table(fn, table, n_tensors, total_blocks);
  if (rc == -1) return ok();
  if (rc != PT_OK) return rc;
  if (!step_table || (reinterpret_cast<uintptr_t>(step_table) & 7u) != 0)
    return fail(PT_EINVAL, std::string(fn) + ": null or misaligned step table");
  if (!grad_scale || !found_inf || !inv_scale)
    return fail(PT_EINVAL, std::string(fn) + ": null grad_scale, found_inf or inv_scale");
  const AdamScalars s = host_scalars(lr, beta1, beta2, eps, weight_decay, 1.0);
  const DevStep d{step_table, static_cast<float>(lr), static_cast<float>(beta1),
                  static_cast<float>(beta2)};
  return launch_step<true, true>(table, n_tensors, total_blocks, s, grad_scale, write_grad, d,
                                 stream, fn, found_inf, inv_scale);
}

// One fp32 partial (and one int flag) per workgroup of the statistics walk, which has at
// most ceil(total_blocks / kWalkUnroll) workgroups.
size_t pt_clip_grad_norm_workspace_bytes(int64_t total_blocks) {
  if (total_blocks < 0) return 0;
  return static_cast<size_t>((total_blocks + kWalkUnroll - 1) / kWalkUnroll) * sizeof(float);
}

size_t pt_grad_stats_workspace_bytes(int64_t total_blocks) {
  if (total_blocks < 0) return 0;
  const size_t parts = static_cast<size_t>((total_blocks + kWalkUnroll - 1) / kWalkUnroll);
  return (parts * sizeof(float) + 15) / 16 * 16 + parts * sizeof(int);
}

}  // extern "C"

namespace {

// Launches the statistics pass and its finish.  `nonfinite` (blocks ints) may be null.
int grad_stats_run(const char* fn, const int64_t* table, int64_t n_tensors, int64_t total_blocks,
                   const float* inv_scale, double max_norm, int clip_mode, float* total_out,
                   float* scale_out, int* found_out, float* partial, int* nonfinite,
                   hipStream_t st) {
  int rc = check_table(fn, table, n_tensors, total_blocks);
  if (rc != -1 && rc != PT_OK) return rc;
  int64_t nparts = 0;  // no gradients: the norm of nothing is 0
  if (rc == PT_OK) {
    const int grid = walk_grid(total_blocks);
    hipLaunchKernelGGL(grad_stats_kernel, dim3(grid), dim3(kThreads), 0, st,
                       reinterpret_cast<const AdamRec*>(table), n_tensors, total_blocks, inv_scale,
                       partial, nonfinite);
    if (int lrc = check_launch(fn)) return lrc;
    nparts = grid;
  }
  hipLaunchKernelGGL(grad_stats_finish_kernel, dim3(1), dim3(1024), 0, st, partial, nonfinite,
                     nparts, static_cast<float>(max_norm), clip_mode, inv_scale, total_out,
                     scale_out, found_out);
  return check_launch(fn);
}

}  // namespace

extern "C" {

int pt_clip_grad_norm(const int64_t* table, int64_t n_tensors, int64_t total_blocks,
                      double max_norm, float* total_norm_out, float* clip_coef_out,
                      void* workspace, size_t workspace_bytes, void* stream) {
  if (!total_norm_out || !clip_coef_out)
    return fail(PT_EINVAL, "pt_clip_grad_norm: null output");
  if (!(max_norm >= 0.0)) return fail(PT_EINVAL, "pt_clip_grad_norm: max_norm must be >= 0");
  if (n_tensors > 0 && total_blocks > 0 &&
      (!workspace || workspace_bytes < pt_clip_grad_norm_workspace_bytes(total_blocks) ||
       !aligned16(workspace)))
    return fail(PT_EINVAL, "pt_clip_grad_norm: workspace too small or not 16-byte aligned");
  return grad_stats_run("pt_clip_grad_norm", table, n_tensors, total_blocks, nullptr, max_norm,
                        CLIP_CLAMP, total_norm_out, clip_coef_out, nullptr,
                        static_cast<float*>(workspace), nullptr, as_stream(stream));
}

int pt_grad_stats(const int64_t* table, int64_t n_tensors, int64_t total_blocks,
                  const float* inv_scale, double max_norm, int clip_mode, float* total_norm_out,
                  float* grad_scale_out, int32_t* found_inf_out, void* workspace,
                  size_t workspace_bytes, void* stream) {
  if (!total_norm_out || !grad_scale_out || !found_inf_out)
    return fail(PT_EINVAL, "pt_grad_stats: null output");
  if (clip_mode != CLIP_CLAMP && clip_mode != CLIP_IF_BELOW_ONE)
    return fail(PT_EINVAL, "pt_grad_stats: unknown clip mode");
  if (n_tensors > 0 && total_blocks > 0 &&
      (!workspace || workspace_bytes < pt_grad_stats_workspace_bytes(total_blocks) ||
       !aligned16(workspace)))
    return fail(PT_EINVAL, "pt_grad_stats: workspace too small or not 16-byte aligned");
  float* partial = static_cast<float*>(workspace);
  const int64_t parts = (total_blocks + kWalkUnroll - 1) / kWalkUnroll;
  int* nonfinite = partial != nullptr
                       ? reinterpret_cast<int*>(reinterpret_cast<char*>(partial) +
                                                (parts * sizeof(float) + 15) / 16 * 16)
                       : nullptr;
  return grad_stats_run("pt_grad_stats", table, n_tensors, total_blocks, inv_scale, max_norm,
                        clip_mode, total_norm_out, grad_scale_out, found_inf_out, partial,
                        nonfinite, as_stream(stream));
}

int pt_grad_scale(const int64_t* table, int64_t n_tensors, int64_t total_blocks,
                  const float* scale, void* stream) {
  const int rc = check_table("pt_grad_scale", table, n_tensors, total_blocks);
  if (rc == -1) return ok();
  if (rc != PT_OK) return rc;
  if (!scale) return fail(PT_EINVAL, "pt_grad_scale: null scale");
  hipLaunchKernelGGL(grad_scale_kernel, dim3(walk_grid(total_blocks)), dim3(kThreads), 0,
                     as_stream(stream), reinterpret_cast<const AdamRec*>(table), n_tensors,
                     total_blocks, scale);
  return check_launch("pt_grad_scale");
}

}  // extern "C"
