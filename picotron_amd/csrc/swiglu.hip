// SwiGLU activation forward and backward for gfx950: pure HBM streams.
//
// Reference semantics (AndyMLAndAI/picotron):
//   forward  src/picotron/nn/triton_kernels/swiglu.py:26-41   y = (g * (1 / (1 + exp(-g)))) * u
//   backward src/picotron/nn/triton_kernels/swiglu.py:71-81   s = sigmoid(g);
//            dg = (dy * u) * (s * (1 + g * (1 - s)));  du = dy * (g * s)
// All arithmetic is fp32; the reference backward runs in the input type, this one rounds
// once on store.
//
// Each thread moves UNROLL independent 16-byte vectors per stream before touching any of
// them, so a wave keeps UNROLL KiB in flight per stream.  Streams larger than the caches
// use nontemporal loads/stores (they are touched exactly once).  Elements past the last
// whole vector, and inputs whose pointers are not 16-byte aligned, take the element path.
#include "pt_common.hpp"

namespace pt {
namespace {

__device__ __forceinline__ float sigmoidf_(float g) {
  // 1 / (1 + exp(-g)); exp(-g) = 2^(-g*log2(e)) on the hardware exp2 unit.  For very
  // negative g the exponential overflows to +inf and the reciprocal gives 0.
  const float e = __expf(-g);
  return __builtin_amdgcn_rcpf(1.0f + e);
}

template <typename T, int UNROLL, bool NT>
__global__ __launch_bounds__(256) void swiglu_fwd_kernel(const T* __restrict__ g,
                                                         const T* __restrict__ u,
                                                         T* __restrict__ o, int64_t nvec) {
  constexpr int V = Elem<T>::VEC;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256 * UNROLL;
  for (int64_t base = static_cast<int64_t>(blockIdx.x) * 256 * UNROLL + threadIdx.x; base < nvec;
       base += stride) {
    Vec16<T> gv[UNROLL], uv[UNROLL];
#pragma unroll
    for (int k = 0; k < UNROLL; ++k) {
      const int64_t i = base + static_cast<int64_t>(k) * 256;
      if (i < nvec) {
        gv[k].raw = load16<NT>(g + i * V);
        uv[k].raw = load16<NT>(u + i * V);
      }
    }
#pragma unroll
    for (int k = 0; k < UNROLL; ++k) {
      const int64_t i = base + static_cast<int64_t>(k) * 256;
      if (i < nvec) {
        Vec16<T> ov;
#pragma unroll
        for (int j = 0; j < V; ++j) {
          const float gf = Elem<T>::to_f32(gv[k].e[j]);
          const float uf = Elem<T>::to_f32(uv[k].e[j]);
          ov.e[j] = Elem<T>::from_f32((gf * sigmoidf_(gf)) * uf);
        }
        store16<NT>(o + i * V, ov.raw);
      }
    }
  }
}

// WT: the two gradients are stored through buffer resources with the write-through policy
// (host-checked: every byte offset fits 31 bits) instead of nontemporal global stores.
template <typename T, int UNROLL, bool NT, bool WT>
__global__ __launch_bounds__(256) void swiglu_bwd_kernel(const T* __restrict__ dy,
                                                         const T* __restrict__ g,
                                                         const T* __restrict__ u,
                                                         T* __restrict__ dg, T* __restrict__ du,
                                                         int64_t nvec) {
  constexpr int V = Elem<T>::VEC;
  const int bytes = WT ? static_cast<int>(nvec * 16) : 0;
  const auto gbuf = uniform_buffer(dg, dg != nullptr ? bytes : 0);
  const auto ubuf = uniform_buffer(du, du != nullptr ? bytes : 0);
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256 * UNROLL;
  for (int64_t base = static_cast<int64_t>(blockIdx.x) * 256 * UNROLL + threadIdx.x; base < nvec;
       base += stride) {
    Vec16<T> dv[UNROLL], gv[UNROLL], uv[UNROLL];
#pragma unroll
    for (int k = 0; k < UNROLL; ++k) {
      const int64_t i = base + static_cast<int64_t>(k) * 256;
      if (i < nvec) {
        dv[k].raw = load16<NT>(dy + i * V);
        gv[k].raw = load16<NT>(g + i * V);
        uv[k].raw = load16<NT>(u + i * V);
      }
    }
#pragma unroll
    for (int k = 0; k < UNROLL; ++k) {
      const int64_t i = base + static_cast<int64_t>(k) * 256;
      if (i < nvec) {
        Vec16<T> gov, uov;
#pragma unroll
        for (int j = 0; j < V; ++j) {
          const float d = Elem<T>::to_f32(dv[k].e[j]);
          const float gf = Elem<T>::to_f32(gv[k].e[j]);
          const float uf = Elem<T>::to_f32(uv[k].e[j]);
          const float s = sigmoidf_(gf);
          gov.e[j] = Elem<T>::from_f32((d * uf) * (s * (1.0f + gf * (1.0f - s))));
          uov.e[j] = Elem<T>::from_f32(d * (gf * s));
        }
        if constexpr (WT) {
          const int off = static_cast<int>(i * 16);
          if (dg != nullptr) __builtin_amdgcn_raw_buffer_store_b128(gov.raw, gbuf, off, 0, kWriteThrough);
          if (du != nullptr) __builtin_amdgcn_raw_buffer_store_b128(uov.raw, ubuf, off, 0, kWriteThrough);
        } else {
          if (dg != nullptr) store16<NT>(dg + i * V, gov.raw);
          if (du != nullptr) store16<NT>(du + i * V, uov.raw);
        }
      }
    }
  }
}

// Element-wise path for [start, n): unaligned inputs and the sub-vector tail.
template <typename T>
__global__ __launch_bounds__(256) void swiglu_fwd_elem_kernel(const T* __restrict__ g,
                                                              const T* __restrict__ u,
                                                              T* __restrict__ o, int64_t start,
                                                              int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t i = start + static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += stride) {
    const float gf = Elem<T>::to_f32(g[i]);
    o[i] = Elem<T>::from_f32((gf * sigmoidf_(gf)) * Elem<T>::to_f32(u[i]));
  }
}

template <typename T>
__global__ __launch_bounds__(256) void swiglu_bwd_elem_kernel(const T* __restrict__ dy,
                                                              const T* __restrict__ g,
                                                              const T* __restrict__ u,
                                                              T* __restrict__ dg,
                                                              T* __restrict__ du, int64_t start,
                                                              int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t i = start + static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += stride) {
    const float d = Elem<T>::to_f32(dy[i]);
    const float gf = Elem<T>::to_f32(g[i]);
    const float uf = Elem<T>::to_f32(u[i]);
    const float s = sigmoidf_(gf);
    if (dg != nullptr) dg[i] = Elem<T>::from_f32((d * uf) * (s * (1.0f + gf * (1.0f - s))));
    if (du != nullptr) du[i] = Elem<T>::from_f32(d * (gf * s));
  }
}

// Vectors per stream per thread.  The backward (3 streams read, 2 written) keeps two in
// flight and runs 2 workgroups per CU: [16384, 14336] bf16 366-367 us, against 383 us with
// four vectors at full occupancy and 395-399 us with two at full occupancy.  The forward
// is fastest with four vectors and no limit (212-216 us at every limit tried).
// Store policy of the streaming launches (one process, alternated): the backward's two
// gradients written through L2 (nontemporal, device scope) 361.0 us against 366.3 with
// nontemporal global stores (364.9 device scope alone, 368.2 nontemporal buffer stores,
// 366.0 at system scope); the forward's one output 221.3 against 219.0, so it keeps them.
constexpr int kFwdUnroll = 4;
constexpr int kBwdUnroll = 2;
// Streams above this many bytes bypass cache retention (nontemporal).
constexpr int64_t kNontemporalBytes = int64_t{64} << 20;

// Resident workgroups per CU of the vector kernels (0: no limit); PT_SWIGLU_FWD_OCCUPANCY
// and PT_SWIGLU_BWD_OCCUPANCY override them.
int fwd_occupancy() {
  static const int v = static_cast<int>(env_int("PT_SWIGLU_FWD_OCCUPANCY", 0));
  return v;
}
int bwd_occupancy() {
  static const int v = static_cast<int>(env_int("PT_SWIGLU_BWD_OCCUPANCY", 2));
  return v;
}

// Launches `kernel` with the dynamic LDS that limits it to `per_cu` resident workgroups
// per CU (or without a limit when the runtime refuses the allocation).
template <typename K, typename... Args>
void launch_limited(K kernel, int per_cu, unsigned grid, hipStream_t st, Args... args) {
  size_t lds = occupancy_lds(per_cu, 0);
  if (allow_dynamic_lds(reinterpret_cast<const void*>(kernel), lds) != PT_OK) lds = 0;
  hipLaunchKernelGGL(kernel, dim3(grid), dim3(256), lds, st, args...);
}

unsigned grid_for(int64_t items, int per_block) {
  int64_t b = (items + per_block - 1) / per_block;
  const int64_t cap = static_cast<int64_t>(num_cus()) * 256;
  if (b > cap) b = cap;
  if (b < 1) b = 1;
  return static_cast<unsigned>(b);
}

template <typename T>
void launch_fwd(const void* g, const void* u, void* o, int64_t n, hipStream_t st) {
  constexpr int V = Elem<T>::VEC;
  const bool aligned = aligned16(g) && aligned16(u) && aligned16(o);
  const int64_t nvec = aligned ? n / V : 0;
  const T* gp = static_cast<const T*>(g);
  const T* up = static_cast<const T*>(u);
  T* op = static_cast<T*>(o);
  if (nvec > 0) {
    const bool nt = n * static_cast<int64_t>(sizeof(T)) > kNontemporalBytes;
    const unsigned grid = grid_for(nvec, 256 * kFwdUnroll);
    if (nt) {
      launch_limited(swiglu_fwd_kernel<T, kFwdUnroll, true>, fwd_occupancy(), grid, st, gp, up, op,
                     nvec);
    } else {
      launch_limited(swiglu_fwd_kernel<T, kFwdUnroll, false>, fwd_occupancy(), grid, st, gp, up,
                     op, nvec);
    }
  }
  const int64_t start = nvec * V;
  if (start < n) {
    hipLaunchKernelGGL(swiglu_fwd_elem_kernel<T>, dim3(grid_for(n - start, 256)), dim3(256), 0,
                       st, gp, up, op, start, n);
  }
}

template <typename T>
void launch_bwd(const void* dy, const void* g, const void* u, void* dg, void* du, int64_t n,
                hipStream_t st) {
  constexpr int V = Elem<T>::VEC;
  const bool aligned = aligned16(dy) && aligned16(g) && aligned16(u) &&
                       (dg == nullptr || aligned16(dg)) && (du == nullptr || aligned16(du));
  const int64_t nvec = aligned ? n / V : 0;
  const T* dyp = static_cast<const T*>(dy);
  const T* gp = static_cast<const T*>(g);
  const T* up = static_cast<const T*>(u);
  T* dgp = static_cast<T*>(dg);
  T* dup = static_cast<T*>(du);
  if (nvec > 0) {
    const bool nt = n * static_cast<int64_t>(sizeof(T)) > kNontemporalBytes;
    const unsigned grid = grid_for(nvec, 256 * kBwdUnroll);
    if (nt && nvec <= 0x7fffffff / 16) {
      launch_limited(swiglu_bwd_kernel<T, kBwdUnroll, true, true>, bwd_occupancy(), grid, st, dyp,
                     gp, up, dgp, dup, nvec);
    } else if (nt) {
      launch_limited(swiglu_bwd_kernel<T, kBwdUnroll, true, false>, bwd_occupancy(), grid, st, dyp,
                     gp, up, dgp, dup, nvec);
    } else {
      launch_limited(swiglu_bwd_kernel<T, kBwdUnroll, false, false>, bwd_occupancy(), grid, st,
                     dyp, gp, up, dgp, dup, nvec);
    }
  }
  const int64_t start = nvec * V;
  if (start < n) {
    hipLaunchKernelGGL(swiglu_bwd_elem_kernel<T>, dim3(grid_for(n - start, 256)), dim3(256), 0,
                       st, dyp, gp, up, dgp, dup, start, n);
  }
}

}  // namespace
}  // namespace pt

using namespace pt;

extern "C" {

int pt_swiglu_fwd(const void* gate, const void* up, void* out, int64_t n, int dtype,
                  void* stream) {
  if (!valid_dtype(dtype)) return fail(PT_EINVAL, "pt_swiglu_fwd: unknown dtype code");
  if (n < 0) return fail(PT_EINVAL, "pt_swiglu_fwd: negative element count");
  if (n == 0) return ok();
  if (!gate || !up || !out) return fail(PT_EINVAL, "pt_swiglu_fwd: null pointer");
  hipStream_t st = as_stream(stream);
  if (dtype == PT_FLOAT32) {
    launch_fwd<float>(gate, up, out, n, st);
  } else if (dtype == PT_FLOAT16) {
    launch_fwd<_Float16>(gate, up, out, n, st);
  } else {
    launch_fwd<__bf16>(gate, up, out, n, st);
  }
  return check_launch("pt_swiglu_fwd");
}

int pt_swiglu_bwd(const void* dout, const void* gate, const void* up, void* dgate, void* dup,
                  int64_t n, int dtype, void* stream) {
  if (!valid_dtype(dtype)) return fail(PT_EINVAL, "pt_swiglu_bwd: unknown dtype code");
  if (n < 0) return fail(PT_EINVAL, "pt_swiglu_bwd: negative element count");
  if (n == 0 || (dgate == nullptr && dup == nullptr)) return ok();
  if (!dout || !gate || !up) return fail(PT_EINVAL, "pt_swiglu_bwd: null pointer");
  hipStream_t st = as_stream(stream);
  if (dtype == PT_FLOAT32) {
    launch_bwd<float>(dout, gate, up, dgate, dup, n, st);
  } else if (dtype == PT_FLOAT16) {
    launch_bwd<_Float16>(dout, gate, up, dgate, dup, n, st);
  } else {
    launch_bwd<__bf16>(dout, gate, up, dgate, dup, n, st);
  }
  return check_launch("pt_swiglu_bwd");
}

}  // extern "C"
