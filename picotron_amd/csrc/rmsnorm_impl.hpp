// RMSNorm forward and backward kernels for gfx950.  Templates only: the per-storage-type
// launchers are instantiated in rmsnorm_{fwd,bwd}_{f32,f16,bf16}.hip (compiled in
// parallel) and called from the C ABI in rmsnorm.hip.
//
// Reference semantics (AndyMLAndAI/picotron):
//   forward  src/picotron/nn/triton_kernels/rmsnorm.py:49-60   r = rsqrt(mean(x^2) + eps),
//            y = (x * r) * w in fp32, stored in x's type
//   backward src/picotron/nn/triton_kernels/rmsnorm.py:110-134
//            wg = g * w; dm = mean(wg * x); dx = r * (wg - (x * r^2) * dm);
//            dW = sum_rows((g * x) * r)
//
// Layout: rows are `cols` contiguous elements, consecutive rows `*_row_stride` apart.
// A row is owned by WPR waves (64*WPR lanes).  Lane `rl` of the row holds the 16-byte
// vectors rl, rl + 64*WPR, ... (VPL of them), so each wave instruction moves 1 KiB of
// contiguous memory, and the whole row stays in registers (packed in its storage type)
// between the reduction and the elementwise pass: x and dy are read from HBM once.
//
// Backward weight gradient: each block accumulates sum((g*x)*r) for its rows in fp32
// registers, combines its row slots in LDS in slot order, and writes one fp32 partial
// row to the workspace; a second kernel sums the partial rows in a fixed order.  No
// atomics, so dW is bitwise reproducible for a given (rows, cols).
#pragma once

#include <string>
#include <type_traits>

#include "pt_common.hpp"

namespace pt {
namespace rmsnorm {

// Upper bound on weight-gradient partial rows (= blocks of the backward row pass).
constexpr int64_t kMaxPartials = 512;
// Waves per block for one-wave rows.
constexpr int kFwdWavesWpr1 = 4;
constexpr int kBwdWavesWpr1 = 8;

// ------------------------------------------------------------------ device helpers

// Loads N consecutive weights starting at element `e` as fp32.
//   WT == void : runtime dtype `wdt`, element loads (any alignment / type)
//   VECTOR     : N*sizeof(WT) bytes as 16/32-byte vector loads (aligned)
template <typename WT, int N, bool VECTOR>
__device__ __forceinline__ void load_weight(const void* w, int wdt, int64_t e, int valid,
                                            float (&out)[N]) {
  if constexpr (std::is_void_v<WT>) {
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = (i < valid) ? load_any(w, e + i, wdt) : 0.0f;
  } else if constexpr (VECTOR) {
    const WT* p = reinterpret_cast<const WT*>(w) + e;
    constexpr int kBytes = N * static_cast<int>(sizeof(WT));
    static_assert(kBytes == 16 || kBytes == 32, "weight vector size");
    constexpr int kLoads = kBytes / 16;
    constexpr int kPer = N / kLoads;
#pragma unroll
    for (int l = 0; l < kLoads; ++l) {
      union {
        u32x4 raw;
        WT e[kPer];
      } u;
      u.raw = *reinterpret_cast<const u32x4*>(p + l * kPer);
#pragma unroll
      for (int i = 0; i < kPer; ++i) out[l * kPer + i] = static_cast<float>(u.e[i]);
    }
  } else {
    const WT* p = reinterpret_cast<const WT*>(w) + e;
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = (i < valid) ? static_cast<float>(p[i]) : 0.0f;
  }
}

// The 16-byte vectors of one row held by a lane, packed in the storage type.
template <typename T, int VPL>
struct RowRegs {
  Vec16<T> v[VPL];

  __device__ __forceinline__ float at(int k, int i) const { return Elem<T>::to_f32(v[k].e[i]); }

  // Tells the compiler the packed words may have changed, so fp32 values converted
  // before this point are not kept alive past it (they are re-derived from the packed
  // words instead).  Keeps the row at 2 bytes/element of registers across the
  // reduction for 16-bit types.
  __device__ __forceinline__ void opaque() {
#pragma unroll
    for (int k = 0; k < VPL; ++k) asm volatile("" : "+v"(v[k].raw));
  }
};

// Loads the lane's VPL vectors of a row.  Out-of-range vectors are zero-filled.
template <typename T, int VPL, int LANES, bool ALIGNED>
__device__ __forceinline__ void load_row(const T* __restrict__ row, int rl, int cols,
                                         RowRegs<T, VPL>& r) {
  constexpr int V = Elem<T>::VEC;
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int e = (rl + k * LANES) * V;
    const int valid = cols - e;
    if constexpr (ALIGNED) {
      if (valid > 0) {
        r.v[k].raw = load16<false>(row + e);
      } else {
        r.v[k].raw = u32x4{0u, 0u, 0u, 0u};
      }
    } else {
#pragma unroll
      for (int i = 0; i < V; ++i) {
        r.v[k].e[i] = (i < valid) ? row[e + i] : Elem<T>::from_f32(0.0f);
      }
    }
  }
}

template <typename T, int LANES, bool ALIGNED>
__device__ __forceinline__ void store_vec(T* __restrict__ row, int rl, int k, int cols,
                                          const float (&o)[Elem<T>::VEC]) {
  constexpr int V = Elem<T>::VEC;
  const int e = (rl + k * LANES) * V;
  const int valid = cols - e;
  if (valid > 0) store_f32<T, ALIGNED>(row + e, o, valid);
}

// Sum over the WPR waves that share a row.  `red` holds 2*WPR floats, double buffered
// by `parity` so consecutive rows need one barrier each.
template <int WPR>
__device__ __forceinline__ float row_sum(float v, float* red, int wave, int lane, int parity) {
  v = wave_sum(v);
  if constexpr (WPR > 1) {
    float* buf = red + parity * WPR;
    if (lane == 0) buf[wave] = v;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int i = 0; i < WPR; ++i) t += buf[i];
    v = t;
  }
  return v;
}

// ------------------------------------------------------------------ forward

template <typename T, typename WT, int VPL, int WPR, int WAVES, bool ALIGNED>
__global__ __launch_bounds__(WAVES * 64) void rmsnorm_fwd_kernel(
    const T* __restrict__ x, int64_t xs, const void* __restrict__ w, int wdt, T* __restrict__ y,
    int64_t ys, float* __restrict__ rstd, int64_t rows, int cols, float eps) {
  static_assert(WPR == 1 || WPR == WAVES, "multi-wave rows use one row per block");
  constexpr int V = Elem<T>::VEC;
  constexpr int RPB = WAVES / WPR;
  constexpr int LANES = 64 * WPR;
  __shared__ float red[2 * WPR];

  const int wave = threadIdx.x / 64;
  const int lane = threadIdx.x % 64;
  const int rl = (wave % WPR) * 64 + lane;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * RPB + wave / WPR;
  // One-wave rows may have a partial last block; multi-wave rows launch exactly `rows`
  // blocks, so every wave of a block reaches the barrier in row_sum.
  if (WPR == 1 && row >= rows) return;

  RowRegs<T, VPL> xr;
  load_row<T, VPL, LANES, ALIGNED>(x + row * xs, rl, cols, xr);

  float ss = 0.0f;
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const float f = xr.at(k, i);
      ss += f * f;
    }
  }
  xr.opaque();
  ss = row_sum<WPR>(ss, red, wave, lane, 0);
  const float r = 1.0f / sqrtf(ss / static_cast<float>(cols) + eps);
  if (rl == 0) rstd[row] = r;

  T* yr = y + row * ys;
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int e = (rl + k * LANES) * V;
    if (e >= cols) continue;
    float wv[V];
    load_weight<WT, V, ALIGNED>(w, wdt, e, cols - e, wv);
    float o[V];
#pragma unroll
    for (int i = 0; i < V; ++i) o[i] = (xr.at(k, i) * r) * wv[i];
    store_vec<T, LANES, ALIGNED>(yr, rl, k, cols, o);
  }
}

// ------------------------------------------------------------------ backward

template <typename T, typename WT, int VPL, int WPR, int WAVES, bool ALIGNED>
__global__ __launch_bounds__(WAVES * 64) void rmsnorm_bwd_kernel(
    const T* __restrict__ dy, int64_t dys, const T* __restrict__ x, int64_t xs,
    const void* __restrict__ w, int wdt, const float* __restrict__ rstd, T* __restrict__ dx,
    int64_t dxs, float* __restrict__ partial, int64_t rows, int cols, int64_t rows_per_block) {
  static_assert(WPR == 1 || WPR == WAVES, "multi-wave rows use one row per block");
  constexpr int V = Elem<T>::VEC;
  constexpr int RPB = WAVES / WPR;
  constexpr int LANES = 64 * WPR;
  __shared__ float red[2 * WPR];
  extern __shared__ float lds_dw[];  // [cols] when RPB > 1 and partial != nullptr

  const int wave = threadIdx.x / 64;
  const int lane = threadIdx.x % 64;
  const int slot = wave / WPR;
  const int rl = (wave % WPR) * 64 + lane;
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * rows_per_block;
  const int64_t r1 = (r0 + rows_per_block < rows) ? r0 + rows_per_block : rows;
  const bool want_dw = partial != nullptr;
  const float inv_cols = 1.0f / static_cast<float>(cols);

  float acc[VPL][V];
#pragma unroll
  for (int k = 0; k < VPL; ++k)
#pragma unroll
    for (int i = 0; i < V; ++i) acc[k][i] = 0.0f;

  int parity = 0;
  // Multi-wave rows: RPB == 1 and every wave of the block walks the same rows, so the
  // barrier in row_sum is reached uniformly.
  for (int64_t row = r0 + slot; row < r1; row += RPB) {
    RowRegs<T, VPL> gr, xr;
    load_row<T, VPL, LANES, ALIGNED>(dy + row * dys, rl, cols, gr);
    load_row<T, VPL, LANES, ALIGNED>(x + row * xs, rl, cols, xr);
    const float r = rstd[row];

    float dot = 0.0f;
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      const int e = (rl + k * LANES) * V;
      if (e >= cols) continue;
      float wv[V];
      load_weight<WT, V, ALIGNED>(w, wdt, e, cols - e, wv);
#pragma unroll
      for (int i = 0; i < V; ++i) dot += (gr.at(k, i) * wv[i]) * xr.at(k, i);
    }
    gr.opaque();
    xr.opaque();
    dot = row_sum<WPR>(dot, red, wave, lane, parity);
    parity ^= 1;
    const float dm = dot * inv_cols;
    const float r2 = r * r;

    T* dxr = dx + row * dxs;
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      const int e = (rl + k * LANES) * V;
      if (e >= cols) continue;
      if (dx != nullptr) {
        float wv[V];
        load_weight<WT, V, ALIGNED>(w, wdt, e, cols - e, wv);
        float o[V];
#pragma unroll
        for (int i = 0; i < V; ++i) o[i] = r * (gr.at(k, i) * wv[i] - (xr.at(k, i) * r2) * dm);
        store_vec<T, LANES, ALIGNED>(dxr, rl, k, cols, o);
      }
      if (want_dw) {
#pragma unroll
        for (int i = 0; i < V; ++i) acc[k][i] += (gr.at(k, i) * xr.at(k, i)) * r;
      }
    }
  }
  if (!want_dw) return;

  float* prow = partial + static_cast<int64_t>(blockIdx.x) * cols;
  if constexpr (RPB == 1) {
    // The block's single row slot: each lane owns distinct columns.
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      const int e = (rl + k * LANES) * V;
#pragma unroll
      for (int i = 0; i < V; ++i)
        if (e + i < cols) prow[e + i] = acc[k][i];
    }
  } else {
    // Row slots hold the same columns: combine them in LDS in slot order.
    for (int s = 0; s < RPB; ++s) {
      if (slot == s) {
#pragma unroll
        for (int k = 0; k < VPL; ++k) {
          const int e = (rl + k * LANES) * V;
#pragma unroll
          for (int i = 0; i < V; ++i) {
            if (e + i < cols) lds_dw[e + i] = (s == 0) ? acc[k][i] : lds_dw[e + i] + acc[k][i];
          }
        }
      }
      __syncthreads();
    }
    for (int c = threadIdx.x; c < cols; c += WAVES * 64) prow[c] = lds_dw[c];
  }
}

// dW[c] = sum_p partial[p][c] in increasing p, cast to the weight type.  A block covers
// 64 columns; its 4 waves take p = wave, wave+4, ... and are combined in wave order.
__global__ __launch_bounds__(256) void rmsnorm_dw_finish_kernel(const float* __restrict__ partial,
                                                                int64_t nparts, int cols,
                                                                void* __restrict__ dw, int wdt);

// ------------------------------------------------------------------ host-side shapes

struct Shape {
  int vpl = 0;  // 16-byte vectors per lane
  int wpr = 0;  // waves per row
};

// Chooses vectors-per-lane (a power of two, at least 4 once a row spans several waves)
// and waves-per-row (1, 4 or 16) so one row fits in registers.  The backward holds dy,
// x and the fp32 weight-gradient accumulator per lane, so it caps VPL at 8 below 16
// waves per row.
inline bool choose_shape(int64_t cols, int vec, bool backward, Shape* s) {
  const int64_t nvec = (cols + vec - 1) / vec;
  const int wprs[3] = {1, 4, 16};
  for (int wpr : wprs) {
    const int64_t per_lane = (nvec + 64 * wpr - 1) / (64 * wpr);
    const int64_t cap = (backward && wpr < 16) ? 8 : 16;
    if (per_lane > cap) continue;
    int vpl = wpr == 1 ? 1 : 4;
    while (vpl < per_lane) vpl *= 2;
    *s = {vpl, wpr};
    return true;
  }
  return false;
}

// Number of backward blocks (= weight-gradient partial rows) and rows per block.
inline void bwd_grid(int64_t rows, const Shape& s, int64_t* blocks, int64_t* rpb) {
  const int64_t slots = s.wpr == 1 ? kBwdWavesWpr1 : 1;
  int64_t b = (rows + slots - 1) / slots;
  if (b > kMaxPartials) b = kMaxPartials;
  if (b < 1) b = 1;
  const int64_t per = rows > 0 ? (rows + b - 1) / b : 1;
  b = (rows + per - 1) / per;
  if (b < 1) b = 1;
  *blocks = b;
  *rpb = per;
}

// Maps a runtime Shape onto the instantiated <VPL, WPR, WAVES> set and calls
// f.template run<VPL, WPR, WAVES>().  WAVES_1 is the block size (in waves) for one-wave
// rows; multi-wave rows use one row per block.
template <int WAVES_1, typename F>
void dispatch_shape(const Shape& s, const F& f) {
  if (s.wpr == 1) {
    switch (s.vpl) {
      case 1: f.template run<1, 1, WAVES_1>(); break;
      case 2: f.template run<2, 1, WAVES_1>(); break;
      case 4: f.template run<4, 1, WAVES_1>(); break;
      case 8: f.template run<8, 1, WAVES_1>(); break;
      default: f.template run<16, 1, WAVES_1>(); break;
    }
  } else if (s.wpr == 4) {
    switch (s.vpl) {
      case 4: f.template run<4, 4, 4>(); break;
      case 8: f.template run<8, 4, 4>(); break;
      default: f.template run<16, 4, 4>(); break;
    }
  } else {
    switch (s.vpl) {
      case 4: f.template run<4, 16, 16>(); break;
      case 8: f.template run<8, 16, 16>(); break;
      default: f.template run<16, 16, 16>(); break;
    }
  }
}

struct FwdArgs {
  const void* x;
  int64_t xs;
  const void* w;
  int wdt;
  void* y;
  int64_t ys;
  float* rstd;
  int64_t rows;
  int cols;
  float eps;
  int xdt;
  bool aligned;
  Shape shape;
  hipStream_t st;
};

struct BwdArgs {
  const void* dy;
  int64_t dys;
  const void* x;
  int64_t xs;
  const void* w;
  int wdt;
  const float* rstd;
  void* dx;
  int64_t dxs;
  float* partial;
  int64_t blocks;
  int64_t rpb;
  int64_t rows;
  int cols;
  int xdt;
  bool aligned;
  Shape shape;
  hipStream_t st;
};

template <typename T, typename WT, bool ALIGNED>
struct FwdLaunch {
  const FwdArgs& a;
  template <int VPL, int WPR, int WAVES>
  void run() const {
    constexpr int RPB = WAVES / WPR;
    const int64_t blocks = (a.rows + RPB - 1) / RPB;
    hipLaunchKernelGGL((rmsnorm_fwd_kernel<T, WT, VPL, WPR, WAVES, ALIGNED>),
                       dim3(static_cast<unsigned>(blocks)), dim3(WAVES * 64), 0, a.st,
                       static_cast<const T*>(a.x), a.xs, a.w, a.wdt, static_cast<T*>(a.y), a.ys,
                       a.rstd, a.rows, a.cols, a.eps);
  }
};

template <typename T, typename WT, bool ALIGNED>
struct BwdLaunch {
  const BwdArgs& a;
  template <int VPL, int WPR, int WAVES>
  void run() const {
    constexpr int RPB = WAVES / WPR;
    const size_t lds =
        (RPB > 1 && a.partial != nullptr) ? static_cast<size_t>(a.cols) * sizeof(float) : 0;
    hipLaunchKernelGGL((rmsnorm_bwd_kernel<T, WT, VPL, WPR, WAVES, ALIGNED>),
                       dim3(static_cast<unsigned>(a.blocks)), dim3(WAVES * 64), lds, a.st,
                       static_cast<const T*>(a.dy), a.dys, static_cast<const T*>(a.x), a.xs,
                       a.w, a.wdt, a.rstd, static_cast<T*>(a.dx), a.dxs, a.partial, a.rows,
                       a.cols, a.rpb);
  }
};

// Per-storage-type launchers.  The vector path is instantiated for weights in
// {x's type, fp32}; other weight types and unaligned rows take the element-wise path.
template <typename T>
void launch_fwd(const FwdArgs& a) {
  if (a.aligned && a.wdt == a.xdt) {
    dispatch_shape<kFwdWavesWpr1>(a.shape, FwdLaunch<T, T, true>{a});
  } else if (a.aligned && a.wdt == PT_FLOAT32) {
    dispatch_shape<kFwdWavesWpr1>(a.shape, FwdLaunch<T, float, true>{a});
  } else {
    dispatch_shape<kFwdWavesWpr1>(a.shape, FwdLaunch<T, void, false>{a});
  }
}

template <typename T>
void launch_bwd(const BwdArgs& a) {
  if (a.aligned && a.wdt == a.xdt) {
    dispatch_shape<kBwdWavesWpr1>(a.shape, BwdLaunch<T, T, true>{a});
  } else if (a.aligned && a.wdt == PT_FLOAT32) {
    dispatch_shape<kBwdWavesWpr1>(a.shape, BwdLaunch<T, float, true>{a});
  } else {
    dispatch_shape<kBwdWavesWpr1>(a.shape, BwdLaunch<T, void, false>{a});
  }
}

extern template void launch_fwd<float>(const FwdArgs&);
extern template void launch_fwd<_Float16>(const FwdArgs&);
extern template void launch_fwd<__bf16>(const FwdArgs&);
extern template void launch_bwd<float>(const BwdArgs&);
extern template void launch_bwd<_Float16>(const BwdArgs&);
extern template void launch_bwd<__bf16>(const BwdArgs&);

}  // namespace rmsnorm
}  // namespace pt
