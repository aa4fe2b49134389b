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
// One launch covers every tensor: block b finds its tensor by binary search over the
// per-tensor first-block indices in the device table, then streams its chunk of
// kBlockElems elements (16-byte vectors when all four pointers are aligned).
#include <cmath>

#include "pt_common.hpp"

namespace pt {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;
constexpr int64_t kBlockElems = int64_t{kThreads} * 4 * kUnroll;  // 4096 fp32 per block

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

__device__ __forceinline__ void adam_elem(float& p, float g, float& m, float& v,
                                          const AdamScalars& s) {
  p = p * s.decay;
  m = (fabsf(s.w1) < 0.5f) ? m + s.w1 * (g - m) : g - (g - m) * (1.0f - s.w1);
  v = v * s.beta2;
  v = v + (s.omb2 * g) * g;
  const float denom = __fdiv_rn(__fsqrt_rn(v), s.bc2_sqrt) + s.eps;
  p = p + s.neg_step * __fdiv_rn(m, denom);
}

__global__ __launch_bounds__(kThreads) void adamw_kernel(const AdamRec* __restrict__ table,
                                                         int64_t ntensors, AdamScalars s) {
  const int64_t blk = blockIdx.x;
  int64_t lo = 0, hi = ntensors - 1;
  while (lo < hi) {
    const int64_t mid = (lo + hi + 1) / 2;
    if (table[mid].first_block <= blk) {
      lo = mid;
    } else {
      hi = mid - 1;
    }
  }
  const AdamRec r = table[lo];
  const int64_t start = (blk - r.first_block) * kBlockElems;
  const int64_t end = (start + kBlockElems < r.n) ? start + kBlockElems : r.n;
  float* P = reinterpret_cast<float*>(r.p);
  const float* G = reinterpret_cast<const float*>(r.g);
  float* M = reinterpret_cast<float*>(r.m);
  float* Vv = reinterpret_cast<float*>(r.v);
  const bool vec_ok = ((r.p | r.g | r.m | r.v) & 15) == 0;

  if (vec_ok && end - start == kBlockElems) {
    f32x4 pv[kUnroll], gv[kUnroll], mv[kUnroll], vv[kUnroll];
#pragma unroll
    for (int k = 0; k < kUnroll; ++k) {
      const int64_t i = start + (static_cast<int64_t>(k) * kThreads + threadIdx.x) * 4;
      pv[k] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(P + i));
      gv[k] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(G + i));
      mv[k] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(M + i));
      vv[k] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(Vv + i));
    }
#pragma unroll
    for (int k = 0; k < kUnroll; ++k) {
      const int64_t i = start + (static_cast<int64_t>(k) * kThreads + threadIdx.x) * 4;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float pp = pv[k][j], mm = mv[k][j], v2 = vv[k][j];
        adam_elem(pp, gv[k][j], mm, v2, s);
        pv[k][j] = pp;
        mv[k][j] = mm;
        vv[k][j] = v2;
      }
      __builtin_nontemporal_store(pv[k], reinterpret_cast<f32x4*>(P + i));
      __builtin_nontemporal_store(mv[k], reinterpret_cast<f32x4*>(M + i));
      __builtin_nontemporal_store(vv[k], reinterpret_cast<f32x4*>(Vv + i));
    }
  } else {
    for (int64_t i = start + threadIdx.x; i < end; i += kThreads) {
      float pp = P[i], mm = M[i], v2 = Vv[i];
      adam_elem(pp, G[i], mm, v2, s);
      P[i] = pp;
      M[i] = mm;
      Vv[i] = v2;
    }
  }
}

}  // namespace
}  // namespace pt

using namespace pt;

extern "C" {

int64_t pt_adamw_block_elems(void) { return kBlockElems; }

int pt_adamw_step(const int64_t* table, int64_t n_tensors, int64_t total_blocks, double lr,
                  double beta1, double beta2, double eps, double weight_decay, double step,
                  void* stream) {
  if (n_tensors < 0 || total_blocks < 0) return fail(PT_EINVAL, "pt_adamw_step: negative count");
  if (n_tensors == 0 || total_blocks == 0) return ok();
  if (!table) return fail(PT_EINVAL, "pt_adamw_step: null table");
  if ((reinterpret_cast<uintptr_t>(table) & 7u) != 0)
    return fail(PT_EINVAL, "pt_adamw_step: table not 8-byte aligned");
  if (total_blocks * kThreads > 0xffffffffLL)
    return fail(PT_EUNSUPPORTED, "pt_adamw_step: more than 2^24 blocks in one launch");
  if (!(step >= 1.0)) return fail(PT_EINVAL, "pt_adamw_step: step must be >= 1");
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
  hipLaunchKernelGGL(adamw_kernel, dim3(static_cast<unsigned>(total_blocks)), dim3(kThreads), 0,
                     as_stream(stream), reinterpret_cast<const AdamRec*>(table), n_tensors, s);
  return check_launch("pt_adamw_step");
}

}  // extern "C"
