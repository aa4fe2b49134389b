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

#include <cstdlib>
#include <string>
#include <type_traits>

#include "pt_common.hpp"

namespace pt {
namespace rmsnorm {

// Waves per block: the backward uses 8 (one weight-gradient partial per 8 waves) and the
// forward 4, or in both cases as many as a row spans when that is more.
constexpr int kBwdWaves = 8;
constexpr int kFwdWaves = 4;
// Cache policy of the row loads (x, dy): nontemporal, the measured optimum on MI355X for data
// read once per kernel.  The row stores: RowStore.
constexpr bool kLoadNT = true;

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

// Loads the weights of a lane's VPL vectors as fp32.  Vector path: branch-free -- a vector
// past the row end loads the row's first weights instead (its products are never stored
// or summed), so the loads issue back to back and their one wait comes at first use.
// Element path: zero past the row end.
template <typename WT, int VPL, int N, bool VECTOR>
__device__ __forceinline__ void load_lane_weights(const void* w, int wdt, int rl, int lanes,
                                                  int cols, float (&wv)[VPL][N]) {
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int e = (rl + k * lanes) * N;
    if constexpr (VECTOR) {
      load_weight<WT, N, true>(w, wdt, e < cols ? e : 0, N, wv[k]);
    } else {
      load_weight<WT, N, false>(w, wdt, e, cols - e, wv[k]);
    }
  }
}

// A lane's weights kept as loaded and converted to fp32 at each use, which halves their
// registers for 16-bit weights.  Vector path: 16-byte words, branch-free (a vector past the
// row end loads the row's first weights; its products are never stored or summed).
// Element path (runtime weight type): fp32 values, zero past the row end.
template <typename WT, int VPL, int N, bool VECTOR>
struct LaneWeights {
  float f[VPL][N];
  __device__ __forceinline__ void load(const void* w, int wdt, int rl, int lanes, int cols) {
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      const int e = (rl + k * lanes) * N;
      load_weight<WT, N, false>(w, wdt, e, cols - e, f[k]);
    }
  }
  __device__ __forceinline__ float at(int k, int i) const { return f[k][i]; }
};

template <typename WT, int VPL, int N>
struct LaneWeights<WT, VPL, N, true> {
  static constexpr int kPer = 16 / static_cast<int>(sizeof(WT));  // weights per 16-byte word
  static constexpr int kWords = N / kPer;
  static_assert(kWords * kPer == N, "weights of one vector fill whole 16-byte words");
  union Word {
    u32x4 raw;
    WT e[kPer];
  };
  Word wd[VPL][kWords];
  __device__ __forceinline__ void load(const void* w, int, int rl, int lanes, int cols) {
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      const int e = (rl + k * lanes) * N;
      const WT* p = reinterpret_cast<const WT*>(w) + (e < cols ? e : 0);
#pragma unroll
      for (int l = 0; l < kWords; ++l) wd[k][l].raw = *reinterpret_cast<const u32x4*>(p + l * kPer);
    }
  }
  __device__ __forceinline__ float at(int k, int i) const {
    return static_cast<float>(wd[k][i / kPer].e[i % kPer]);
  }
};

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

// Stand-in for an absent row buffer (template variants without a residual stream).
struct NoRegs {
  __device__ __forceinline__ void opaque() {}
};

// Residual stream of the fused add + norm (decoder block: h = x + res, then norm(h)).
template <typename T>
struct ResidualIn {
  const T* res;
  int64_t res_stride;
  T* h;
  int64_t h_stride;
};

// Incoming gradient of h added to the norm's input gradient (h also feeds the block's
// final residual add): dh = norm_backward(dy) + dh_in.
template <typename T>
struct ResidualGrad {
  const T* dh_in;
  int64_t dh_in_stride;
};

// Loads the lane's VPL vectors of a row.  Aligned path: branch-free and unmasked -- a
// lane whose vector lies past the row end loads the row's first vector instead, and the
// caller ignores it (in_row()).  Nothing may consume the loaded registers here: loads
// under divergent branches, or a select right after them, make the compiler wait for the
// data at load time and so drain the next row's prefetch.  Element path: out-of-range
// elements are zero-filled.
template <typename T, int VPL, int LANES, bool ALIGNED, bool NT>
__device__ __forceinline__ void load_row(const T* __restrict__ row, int rl, int cols,
                                         RowRegs<T, VPL>& r) {
  constexpr int V = Elem<T>::VEC;
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int e = (rl + k * LANES) * V;
    const int valid = cols - e;
    if constexpr (ALIGNED) {
      r.v[k].raw = load16<NT>(row + (valid > 0 ? e : 0));
    } else {
#pragma unroll
      for (int i = 0; i < V; ++i) {
        r.v[k].e[i] = (i < valid) ? row[e + i] : Elem<T>::from_f32(0.0f);
      }
    }
  }
}

// True if vector k of lane rl lies inside the row (aligned path: whole vectors).
template <typename T, int LANES>
__device__ __forceinline__ bool in_row(int rl, int k, int cols) {
  return (rl + k * LANES) * Elem<T>::VEC < cols;
}

// Stores of one row's 16-byte vectors.  Aligned rows: buffer stores with cache policy
// POLICY through a resource over the row, whose base is wave-uniform (all lanes of a wave
// work on the same row); the resource's range check drops vectors past the row end, so the
// stores need no branch.  Unaligned rows: element stores of the in-range elements.
// The forward's stores are write-through (kWriteThrough: 43.9 against 44.3 us per launch at
// [16384, 4096] bf16), the backward's nontemporal (kNonTemporal: 71.9 against 72.2 us: with
// two read streams beside it, write-through costs more than it saves).
template <typename T, int LANES, bool ALIGNED, int POLICY>
struct RowStore {
  T* row;
  int cols;
  __amdgpu_buffer_rsrc_t rsrc;
  __device__ __forceinline__ RowStore(T* r, int c) : row(r), cols(c) {
    if constexpr (ALIGNED) rsrc = uniform_buffer(r, c * static_cast<int>(sizeof(T)));
  }
  __device__ __forceinline__ void store(int rl, int k, const float (&o)[Elem<T>::VEC]) const {
    constexpr int V = Elem<T>::VEC;
    const int e = (rl + k * LANES) * V;
    if constexpr (ALIGNED) {
      Vec16<T> v;
#pragma unroll
      for (int i = 0; i < V; ++i) v.e[i] = Elem<T>::from_f32(o[i]);
      __builtin_amdgcn_raw_buffer_store_b128(v.raw, rsrc, e * static_cast<int>(sizeof(T)), 0,
                                             POLICY);
    } else {
      const int valid = cols - e;
      if (valid > 0) store_f32<T, false>(row + e, o, valid);
    }
  }
};

// Sum over the WPR waves that share a row.  `red` holds 2*WAVES floats; `buf` alternates
// between consecutive calls so one barrier per row suffices (a wave cannot overwrite a
// buffer before every wave has passed the barrier of the call in between).  Waves sum the
// partials of their row in wave order, so every wave of a row gets the same value.
template <int WPR, int WAVES>
__device__ __forceinline__ float row_sum(float v, float* red, int wave, int lane, int buf) {
  v = wave_sum(v);
  if constexpr (WPR > 1) {
    float* b = red + buf * WAVES;
    if (lane == 0) b[wave] = v;
    __syncthreads();
    const int first = (wave / WPR) * WPR;
    float t = 0.0f;
#pragma unroll
    for (int i = 0; i < WPR; ++i) t += b[first + i];
    v = t;
  }
  return v;
}

// ------------------------------------------------------------------ forward
//
// Row groups: a block has WAVES/WPR row slots; at step `it` block b works on the group of
// rows starting at (it * gridDim.x + b) * slots, so at any moment all blocks work on one
// compact window of rows (DRAM-friendly, like a non-persistent grid).  With a grid that
// covers every row once (the default) each wave handles one row; smaller grids loop, and
// the next row is then loaded into the second register buffer before the current one is
// reduced (PERSIST).  Weights are loaded once per wave, kept packed.  Without PERSIST the
// kernel holds one row buffer only: fewer registers, more waves in flight per CU.

// ADD: the fused residual add.  h = x + res is computed in fp32, rounded to the storage
// type and written; the norm is taken of the rounded h, as the unfused graph normalises the
// stored sum.

template <typename T, typename WT, int VPL, int WPR, int WAVES, bool ALIGNED, bool LOAD_NT,
          bool PERSIST, bool ADD>
__global__ __launch_bounds__(WAVES * 64) void rmsnorm_fwd_kernel(
    const T* __restrict__ x, int64_t xs, const void* __restrict__ w, int wdt, T* __restrict__ y,
    int64_t ys, float* __restrict__ rstd, int64_t rows, int cols, float eps, int iters,
    ResidualIn<T> rin) {
  static_assert(WAVES % WPR == 0, "row slots must tile the block");
  constexpr int V = Elem<T>::VEC;
  constexpr int RPB = WAVES / WPR;
  constexpr int LANES = 64 * WPR;
  __shared__ float red[2 * WAVES];

  const int wave = threadIdx.x / 64;
  const int lane = threadIdx.x % 64;
  const int slot = wave / WPR;
  const int rl = (wave % WPR) * 64 + lane;
  // iters = ceil(rows / group_stride), computed on the host: the same for every wave.
  const int64_t group_stride = static_cast<int64_t>(gridDim.x) * RPB;
  const int64_t r1 = rows;
  const float inv_cols = 1.0f / static_cast<float>(cols);

  LaneWeights<WT, VPL, V, ALIGNED> wv;
  wv.load(w, wdt, rl, LANES, cols);

  using ResRegs = std::conditional_t<ADD, RowRegs<T, VPL>, NoRegs>;
  struct Row {
    RowRegs<T, VPL> x;
    ResRegs res;
  };
  auto process = [&](Row& rw, int64_t row, int buf) {
    RowRegs<T, VPL>& xr = rw.x;
    const bool active = row < r1;
    if constexpr (ADD) {
      const RowStore<T, LANES, ALIGNED, kWriteThrough> hs(rin.h + row * rin.h_stride, cols);
#pragma unroll
      for (int k = 0; k < VPL; ++k) {
        float o[V];
#pragma unroll
        for (int i = 0; i < V; ++i) {
          xr.v[k].e[i] = Elem<T>::from_f32(xr.at(k, i) + rw.res.at(k, i));
          o[i] = xr.at(k, i);
        }
        if (active) hs.store(rl, k, o);
      }
    }
    float ss = 0.0f;
    if (active) {
#pragma unroll
      for (int k = 0; k < VPL; ++k) {
        float part = 0.0f;
#pragma unroll
        for (int i = 0; i < V; ++i) {
          const float f = xr.at(k, i);
          part += f * f;
        }
        ss += in_row<T, LANES>(rl, k, cols) ? part : 0.0f;
      }
    }
    xr.opaque();
    ss = row_sum<WPR, WAVES>(ss, red, wave, lane, buf);
    if (!active) return;
    const float r = 1.0f / sqrtf(ss * inv_cols + eps);
    if (rl == 0) rstd[row] = r;
    const RowStore<T, LANES, ALIGNED, kWriteThrough> yst(y + row * ys, cols);
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      float o[V];
#pragma unroll
      for (int i = 0; i < V; ++i) o[i] = (xr.at(k, i) * r) * wv.at(k, i);
      yst.store(rl, k, o);
    }
  };

  // Rows past the end are clamped to the last row for loading (keeping the loads
  // unconditional) and skipped by process().
  auto load = [&](Row& rw, int64_t row) {
    const int64_t lr = row < r1 ? row : r1 - 1;
    load_row<T, VPL, LANES, ALIGNED, LOAD_NT>(x + lr * xs, rl, cols, rw.x);
    if constexpr (ADD)
      load_row<T, VPL, LANES, ALIGNED, LOAD_NT>(rin.res + lr * rin.res_stride, rl, cols, rw.res);
  };
  int64_t ra = static_cast<int64_t>(blockIdx.x) * RPB + slot;
  if constexpr (!PERSIST) {
    Row a;
    load(a, ra);
    process(a, ra, 0);
  } else {
    // Unconditional prefetches inside the loop, the last one or two rows peeled (as in the
    // backward: a prefetch under a branch makes the compiler wait for it at the join).
    Row a, b;
    load(a, ra);
    int it = 0;
    for (; it + 2 < iters; it += 2) {
      const int64_t rb = ra + group_stride;
      load(b, rb);
      process(a, ra, 0);
      const int64_t rc = rb + group_stride;
      load(a, rc);
      process(b, rb, 1);
      ra = rc;
    }
    if (it + 1 < iters) {
      const int64_t rb = ra + group_stride;
      load(b, rb);
      process(a, ra, 0);
      process(b, rb, 1);
    } else {
      process(a, ra, 0);
    }
  }
}

// ------------------------------------------------------------------ weight-gradient sum
//
// dW[c] = sum_p partial[p][c] in a fixed order, cast to the weight type: 256 threads cover
// kFinishCols columns with kFinishGroups groups of 32 lanes; group g sums p = g, g+8, ... in
// increasing p (up to 64 loads in flight per lane: one round trip at 512 partials), then the
// groups are added in group order (rmsnorm_dw_finish_kernel).
constexpr int kFinishCols = 32;
constexpr int kFinishGroups = 8;

__device__ __forceinline__ float column_group_sum(const float* __restrict__ partial,
                                                  int64_t nparts, int cols, int c, int grp) {
  constexpr int kUnroll = 64;
  const float* p = partial + c;
  float s = 0.0f;
  int64_t i = grp;
  for (; i + static_cast<int64_t>(kFinishGroups) * (kUnroll - 1) < nparts;
       i += static_cast<int64_t>(kFinishGroups) * kUnroll) {
    float v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) v[u] = p[(i + u * kFinishGroups) * cols];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) s += v[u];
  }
  // The remainder (fewer than kUnroll partials per group) in batches of 16 independent
  // loads, so that it costs a few round trips rather than one per partial.
#pragma unroll 16
  for (; i < nparts; i += kFinishGroups) s += p[i * cols];
  return s;
}

__global__ __launch_bounds__(256) void rmsnorm_dw_finish_kernel(const float* __restrict__ partial,
                                                                int64_t nparts, int cols,
                                                                void* __restrict__ dw, int wdt);

// ------------------------------------------------------------------ backward
//
// Persistent blocks walking the same interleaved row groups as the forward (step `it`:
// rows (it * gridDim.x + b) * slots + slot), with the next row double-buffered in
// registers.  Per row: dot = sum((g*w)*x) over the row (fp32, wave + LDS reduction),
// dx = r*((g*w) - (x*r^2)*dm) written from the registers, and sum((g*x)*r) accumulated
// per lane in fp32.  Spreading a row over WPR waves divides that accumulator (and the row
// registers) by WPR.  At the end the row slots are combined in LDS in slot order and the
// block writes one fp32 partial row; the partial count (the grid) is fixed for a given
// shape and tuning, so the weight gradient is reproducible.

// ADD: dx = norm_backward(dy) + dh_in, summed in fp32 and rounded once (the fused residual
// add's backward; dx may alias dh_in, each element being read before it is written by the
// same lane).

template <typename T, typename WT, int VPL, int WPR, int WAVES, bool ALIGNED, bool LOAD_NT,
          bool ADD>
__global__ __launch_bounds__(WAVES * 64) void rmsnorm_bwd_kernel(
    const T* __restrict__ dy, int64_t dys, const T* __restrict__ x, int64_t xs,
    const void* __restrict__ w, int wdt, const float* __restrict__ rstd, T* dx,
    int64_t dxs, float* __restrict__ partial, int64_t rows, int cols, int iters,
    ResidualGrad<T> rg) {
  static_assert(WAVES % WPR == 0, "row slots must tile the block");
  constexpr int V = Elem<T>::VEC;
  constexpr int RPB = WAVES / WPR;
  constexpr int LANES = 64 * WPR;
  __shared__ float red[2 * WAVES];
  extern __shared__ float lds_dw[];  // [cols] when RPB > 1 and partial != nullptr

  const int wave = threadIdx.x / 64;
  const int lane = threadIdx.x % 64;
  const int slot = wave / WPR;
  const int rl = (wave % WPR) * 64 + lane;
  // iters = ceil(rows / group_stride), computed on the host: the same for every wave.
  const int64_t group_stride = static_cast<int64_t>(gridDim.x) * RPB;
  const int64_t r1 = rows;
  const bool want_dw = partial != nullptr;
  const float inv_cols = 1.0f / static_cast<float>(cols);

  float wv[VPL][V];
  load_lane_weights<WT, VPL, V, ALIGNED>(w, wdt, rl, LANES, cols, wv);
  float acc[VPL][V];
#pragma unroll
  for (int k = 0; k < VPL; ++k)
#pragma unroll
    for (int i = 0; i < V; ++i) acc[k][i] = 0.0f;

  using ResRegs = std::conditional_t<ADD, RowRegs<T, VPL>, NoRegs>;
  struct Buf {
    RowRegs<T, VPL> g, x;
    ResRegs d;
    float r;
  };
  // Rows past the end are clamped to the last row for loading (keeping the loads
  // unconditional) and skipped by process().
  auto load = [&](Buf& bf, int64_t row) {
    const int64_t lr = row < r1 ? row : r1 - 1;
    load_row<T, VPL, LANES, ALIGNED, LOAD_NT>(dy + lr * dys, rl, cols, bf.g);
    load_row<T, VPL, LANES, ALIGNED, LOAD_NT>(x + lr * xs, rl, cols, bf.x);
    if constexpr (ADD)
      load_row<T, VPL, LANES, ALIGNED, LOAD_NT>(rg.dh_in + lr * rg.dh_in_stride, rl, cols, bf.d);
    bf.r = rstd[lr];
  };
  auto process = [&](Buf& bf, int64_t row, int buf) {
    const bool active = row < r1;
    float dot = 0.0f;
    if (active) {
#pragma unroll
      for (int k = 0; k < VPL; ++k) {
        float part = 0.0f;
#pragma unroll
        for (int i = 0; i < V; ++i) part += (bf.g.at(k, i) * wv[k][i]) * bf.x.at(k, i);
        dot += in_row<T, LANES>(rl, k, cols) ? part : 0.0f;
      }
    }
    bf.g.opaque();
    bf.x.opaque();
    bf.d.opaque();
    dot = row_sum<WPR, WAVES>(dot, red, wave, lane, buf);
    if (!active) return;
    const float r = bf.r;
    const float dm = dot * inv_cols;
    const float r2 = r * r;
    if (dx != nullptr) {
      const RowStore<T, LANES, ALIGNED, kNonTemporal> dxst(dx + row * dxs, cols);
#pragma unroll
      for (int k = 0; k < VPL; ++k) {
        float o[V];
#pragma unroll
        for (int i = 0; i < V; ++i) {
          o[i] = r * (bf.g.at(k, i) * wv[k][i] - (bf.x.at(k, i) * r2) * dm);
          if constexpr (ADD) o[i] += bf.d.at(k, i);
        }
        dxst.store(rl, k, o);
      }
    }
    if (want_dw) {
#pragma unroll
      for (int k = 0; k < VPL; ++k)
#pragma unroll
        for (int i = 0; i < V; ++i) acc[k][i] += (bf.g.at(k, i) * bf.x.at(k, i)) * r;
    }
  };

  // The next row is double-buffered in registers.  The loop body issues its two prefetches
  // unconditionally (both rows are within the block's iterations), so the wait for the row
  // being reduced counts only that row's loads: a prefetch under a branch would make the
  // compiler wait for everything at the join.  The last one or two rows are peeled.
  int64_t ra = static_cast<int64_t>(blockIdx.x) * RPB + slot;
  Buf a, b;
  load(a, ra);
  int it = 0;
  for (; it + 2 < iters; it += 2) {
    const int64_t rb = ra + group_stride;
    load(b, rb);
    process(a, ra, 0);
    const int64_t rc = rb + group_stride;
    load(a, rc);
    process(b, rb, 1);
    ra = rc;
  }
  if (it + 1 < iters) {
    const int64_t rb = ra + group_stride;
    load(b, rb);
    process(a, ra, 0);
    process(b, rb, 1);
  } else {
    process(a, ra, 0);
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

// ------------------------------------------------------------------ host-side shapes

struct Shape {
  int vpl = 0;  // 16-byte vectors per lane
  int wpr = 0;  // waves per row
};

// Launch tuning.  Defaults were chosen by measurement on MI355X; the environment can
// override them (PT_RMSNORM_FWD_VPL_CAP, PT_RMSNORM_BWD_VPL_CAP, PT_RMSNORM_FWD_BLOCKS_PER_CU,
// PT_RMSNORM_BWD_PARTIALS, PT_RMSNORM_FWD_OCCUPANCY, PT_RMSNORM_BWD_OCCUPANCY), read once
// per process.  The backward partial count fixes the
// weight-gradient summation order, so dW is reproducible for a given setting.
struct Tuning {
  int fwd_vpl_cap = 0;  // 0: by element size (fwd_vpl_cap_for)
  int bwd_vpl_cap = 0;  // 0: by row length (bwd_vpl_cap_for)
  int64_t fwd_blocks_per_cu = 0;  // 0: no cap (one row per row slot)
  int64_t bwd_partials = 512;
  int fwd_occupancy = 0;  // resident forward workgroups per CU (0: no limit)
  int bwd_occupancy = 0;  // resident backward workgroups per CU (0: no limit)
};

// Backward vectors per lane: one for rows of at most 256 16-byte vectors (bf16 hidden
// <= 2048; measured 960: 40.7 -> 34.1 us, 2048: 64.2 -> 62.1 us per fwd+bwd layer at 16384
// rows), two above (4096: 116.0 against 117.8 with one), unless the environment sets it.
inline int bwd_vpl_cap_for(int tuned, int64_t cols, int vec) {
  if (tuned > 0) return tuned;
  return (cols + vec - 1) / vec <= 256 ? 1 : 2;
}

// Forward vectors per lane: 32 elements per lane, four 16-byte vectors of a 16-bit type and
// eight of fp32 (two waves per 4096-wide row either way); measured at [16384, 4096], 4 layers:
// bf16 0.4628-0.4639 ms per step against 0.4660-0.4684 with two and 0.4747-0.4763 with eight,
// fp32 0.8769-0.8777 ms against 0.8868-0.8871 with four.
inline int fwd_vpl_cap_for(int tuned, int vec) { return tuned > 0 ? tuned : 32 / vec; }

inline int64_t env_positive(const char* name, int64_t fallback) {
  const char* v = std::getenv(name);
  if (v == nullptr || *v == '\0') return fallback;
  char* end = nullptr;
  const long long x = std::strtoll(v, &end, 10);
  return (end != v && x > 0) ? static_cast<int64_t>(x) : fallback;
}

inline const Tuning& tuning() {
  static const Tuning t = [] {
    Tuning d;
    d.fwd_vpl_cap = static_cast<int>(env_positive("PT_RMSNORM_FWD_VPL_CAP", d.fwd_vpl_cap));
    d.bwd_vpl_cap = static_cast<int>(env_positive("PT_RMSNORM_BWD_VPL_CAP", d.bwd_vpl_cap));
    d.fwd_blocks_per_cu = env_positive("PT_RMSNORM_FWD_BLOCKS_PER_CU", d.fwd_blocks_per_cu);
    d.bwd_partials = env_positive("PT_RMSNORM_BWD_PARTIALS", d.bwd_partials);
    d.fwd_occupancy = static_cast<int>(env_int("PT_RMSNORM_FWD_OCCUPANCY", d.fwd_occupancy));
    d.bwd_occupancy = static_cast<int>(env_int("PT_RMSNORM_BWD_OCCUPANCY", d.bwd_occupancy));
    return d;
  }();
  return t;
}

inline int pow2_at_least(int64_t n) {
  int v = 1;
  while (v < n) v *= 2;
  return v;
}

// Smallest waves-per-row in {1, 2, 4, 8, 16} whose vectors-per-lane fit under `cap`
// (VPL a power of two); past that, 16 waves per row with up to 16 vectors per lane.
inline bool choose_shape(int64_t cols, int vec, int cap, Shape* s) {
  const int64_t nvec = (cols + vec - 1) / vec;
  for (int wpr = 1; wpr <= 16; wpr *= 2) {
    const int64_t per_lane = (nvec + 64 * wpr - 1) / (64 * wpr);
    if (per_lane <= cap) {
      *s = {pow2_at_least(per_lane), wpr};
      return true;
    }
  }
  const int64_t per_lane = (nvec + 1023) / 1024;
  if (per_lane > 16) return false;
  *s = {pow2_at_least(per_lane), 16};
  return true;
}

// The element-wise (unaligned) path is instantiated for fewer shapes: 4 waves per row
// with 1..8 vectors per lane, or 16 waves per row with 8 or 16.
inline Shape unaligned_shape(int64_t cols, int vec) {
  const int64_t nvec = (cols + vec - 1) / vec;
  const int64_t per4 = (nvec + 255) / 256;
  if (per4 <= 8) return {pow2_at_least(per4), 4};
  const int64_t per16 = (nvec + 1023) / 1024;
  return {per16 <= 8 ? 8 : 16, 16};
}

// Calls f.template run<VPL, WPR>() for a runtime shape and returns true, or returns false
// if that shape is not instantiated.  FULL selects the complete set (vector path);
// otherwise the element-wise subset.
template <bool FULL, typename F>
bool dispatch_shape(const Shape& s, const F& f) {
#define PT_RMS_CASE(V, W)            \
  if (s.vpl == V && s.wpr == W) {    \
    f.template run<V, W>();          \
    return true;                     \
  }
  if constexpr (FULL) {
    PT_RMS_CASE(1, 1) PT_RMS_CASE(2, 1) PT_RMS_CASE(4, 1) PT_RMS_CASE(8, 1)
    PT_RMS_CASE(1, 2) PT_RMS_CASE(2, 2) PT_RMS_CASE(4, 2) PT_RMS_CASE(8, 2)
    PT_RMS_CASE(1, 4) PT_RMS_CASE(2, 4) PT_RMS_CASE(4, 4) PT_RMS_CASE(8, 4)
    PT_RMS_CASE(1, 8) PT_RMS_CASE(2, 8) PT_RMS_CASE(4, 8) PT_RMS_CASE(8, 8)
    PT_RMS_CASE(1, 16) PT_RMS_CASE(2, 16) PT_RMS_CASE(4, 16) PT_RMS_CASE(8, 16)
    PT_RMS_CASE(16, 16)
  } else {
    PT_RMS_CASE(1, 4) PT_RMS_CASE(2, 4) PT_RMS_CASE(4, 4) PT_RMS_CASE(8, 4)
    PT_RMS_CASE(8, 16) PT_RMS_CASE(16, 16)
  }
#undef PT_RMS_CASE
  return false;
}

inline int bwd_waves(const Shape& s) { return s.wpr > kBwdWaves ? s.wpr : kBwdWaves; }

// Backward grid = number of weight-gradient partial rows.
inline int64_t bwd_blocks(int64_t rows, const Shape& s) {
  const int64_t slots = bwd_waves(s) / s.wpr;
  int64_t b = (rows + slots - 1) / slots;
  if (b > tuning().bwd_partials) b = tuning().bwd_partials;
  return b < 1 ? 1 : b;
}

inline int fwd_waves(const Shape& s) { return s.wpr > kFwdWaves ? s.wpr : kFwdWaves; }

// Forward grid: one row per row slot (non-persistent, measured fastest), optionally capped
// at PT_RMSNORM_FWD_BLOCKS_PER_CU blocks per CU.
inline int64_t fwd_blocks(int64_t rows, const Shape& s, int ncu) {
  const int64_t slots = fwd_waves(s) / s.wpr;
  int64_t b = (rows + slots - 1) / slots;
  const int64_t per_cu = tuning().fwd_blocks_per_cu;
  if (per_cu > 0 && b > static_cast<int64_t>(ncu) * per_cu) b = static_cast<int64_t>(ncu) * per_cu;
  return b < 1 ? 1 : b;
}

// Row-group steps of a grid of `blocks` blocks with `slots` row slots each.
inline int row_iters(int64_t rows, int64_t blocks, int slots) {
  const int64_t stride = blocks * slots;
  return static_cast<int>((rows + stride - 1) / stride);
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
  int64_t blocks;
  hipStream_t st;
  // fused residual add (res == nullptr: plain norm)
  const void* res = nullptr;
  int64_t res_s = 0;
  void* h = nullptr;
  int64_t h_s = 0;
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
  int64_t rows;
  int cols;
  int xdt;
  bool aligned;
  Shape shape;
  hipStream_t st;
  // incoming gradient of h for the fused residual add (nullptr: plain norm backward)
  const void* dh_in = nullptr;
  int64_t dh_in_s = 0;
};

template <typename T, typename WT, bool ALIGNED>
struct FwdLaunch {
  const FwdArgs& a;
  template <int VPL, int WPR, bool PERSIST, bool ADD>
  void go(int iters) const {
    constexpr int WAVES = WPR > kFwdWaves ? WPR : kFwdWaves;
    const ResidualIn<T> rin{static_cast<const T*>(a.res), a.res_s, static_cast<T*>(a.h), a.h_s};
    const auto kernel =
        rmsnorm_fwd_kernel<T, WT, VPL, WPR, WAVES, ALIGNED, kLoadNT, PERSIST, ADD>;
    size_t lds = occupancy_lds(tuning().fwd_occupancy, 0);
    if (allow_dynamic_lds(reinterpret_cast<const void*>(kernel), lds) != PT_OK) lds = 0;
    hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(a.blocks)), dim3(WAVES * 64), lds, a.st,
                       static_cast<const T*>(a.x), a.xs, a.w, a.wdt, static_cast<T*>(a.y), a.ys,
                       a.rstd, a.rows, a.cols, a.eps, iters, rin);
  }
  template <int VPL, int WPR>
  void run() const {
    constexpr int WAVES = WPR > kFwdWaves ? WPR : kFwdWaves;
    const int iters = row_iters(a.rows, a.blocks, WAVES / WPR);
    if (a.res != nullptr) {
      if (iters == 1) {
        go<VPL, WPR, false, true>(iters);
      } else {
        go<VPL, WPR, true, true>(iters);
      }
    } else if (iters == 1) {
      go<VPL, WPR, false, false>(iters);
    } else {
      go<VPL, WPR, true, false>(iters);
    }
  }
};

template <typename T, typename WT, bool ALIGNED>
struct BwdLaunch {
  const BwdArgs& a;
  template <bool ADD, int VPL, int WPR, int WAVES>
  void go(size_t need, size_t lds, int iters) const {
    const auto kernel = rmsnorm_bwd_kernel<T, WT, VPL, WPR, WAVES, ALIGNED, kLoadNT, ADD>;
    if (allow_dynamic_lds(reinterpret_cast<const void*>(kernel), lds) != PT_OK) lds = need;
    const ResidualGrad<T> rg{static_cast<const T*>(a.dh_in), a.dh_in_s};
    hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(a.blocks)), dim3(WAVES * 64), lds, a.st,
                       static_cast<const T*>(a.dy), a.dys, static_cast<const T*>(a.x), a.xs, a.w,
                       a.wdt, a.rstd, static_cast<T*>(a.dx), a.dxs, a.partial, a.rows, a.cols,
                       iters, rg);
  }
  template <int VPL, int WPR>
  void run() const {
    constexpr int WAVES = WPR > kBwdWaves ? WPR : kBwdWaves;
    constexpr int RPB = WAVES / WPR;
    const size_t need =
        (RPB > 1 && a.partial != nullptr) ? static_cast<size_t>(a.cols) * sizeof(float) : 0;
    const size_t share = occupancy_lds(tuning().bwd_occupancy, 0);
    const size_t lds = share > need ? share : need;
    const int iters = row_iters(a.rows, a.blocks, RPB);
    if (a.dh_in != nullptr) {
      go<true, VPL, WPR, WAVES>(need, lds, iters);
    } else {
      go<false, VPL, WPR, WAVES>(need, lds, iters);
    }
  }
};

// True when the 16-byte vector kernels apply: rows aligned (checked by the caller) and a
// weight type with an instantiated vector path (x's type or fp32).
inline bool vector_weight(int xdt, int wdt) { return wdt == xdt || wdt == PT_FLOAT32; }

// Per-storage-type launchers; false if no kernel matched the shape (a bug, reported by
// the caller as an error rather than silently skipping the launch).
template <typename T>
bool launch_fwd(const FwdArgs& a) {
  if (a.aligned && a.wdt == a.xdt) return dispatch_shape<true>(a.shape, FwdLaunch<T, T, true>{a});
  if (a.aligned && a.wdt == PT_FLOAT32)
    return dispatch_shape<true>(a.shape, FwdLaunch<T, float, true>{a});
  return dispatch_shape<false>(a.shape, FwdLaunch<T, void, false>{a});
}

template <typename T>
bool launch_bwd(const BwdArgs& a) {
  if (a.aligned && a.wdt == a.xdt) return dispatch_shape<true>(a.shape, BwdLaunch<T, T, true>{a});
  if (a.aligned && a.wdt == PT_FLOAT32)
    return dispatch_shape<true>(a.shape, BwdLaunch<T, float, true>{a});
  return dispatch_shape<false>(a.shape, BwdLaunch<T, void, false>{a});
}

extern template bool launch_fwd<float>(const FwdArgs&);
extern template bool launch_fwd<_Float16>(const FwdArgs&);
extern template bool launch_fwd<__bf16>(const FwdArgs&);
extern template bool launch_bwd<float>(const BwdArgs&);
extern template bool launch_bwd<_Float16>(const BwdArgs&);
extern template bool launch_bwd<__bf16>(const BwdArgs&);

}  // namespace rmsnorm
}  // namespace pt
