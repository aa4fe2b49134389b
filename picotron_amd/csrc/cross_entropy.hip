// Fused cross-entropy (mean over non-ignored rows) with its gradient written in place, over
// the logits, or into a separate gradient buffer whose rows lie in the same 16-byte phase as
// the logits rows (the logits are then only read).
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
//      (VPT 16-byte vectors per thread, raw buffer loads whose hardware range check drops
//      the ragged end) and reduced by an online max / sum of exp(x - max) as the vectors
//      arrive; each exp is kept in the registers in place of its logit, so the gradient
//      softmax / n_valid is written from registers with one multiply per element and no
//      second exponential: HBM sees one read and one write of the logits.  The target
//      element's gradient (softmax_t - 1) / n_valid comes from the exact fp32 target logit.
//      Longer or unaligned rows use ce_rows_batched (two passes, batches of loads in flight,
//      the second pass served largely by the Infinity Cache).
//      Each row's fp32 loss goes to the workspace.  When no gradient is written in the
//      forward -- the loss alone, or fp16 logits, which are left as they are -- aligned rows
//      take ce_lse instead: a read-only stream, 256-thread workgroups several to a CU, that
//      also keeps the row's log-sum-exp for fp16, whose backward (ce_scale) then writes the
//      gradient with grad_output applied, rounding to fp16 once.
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
  // followed by float row_loss[rows] (16-byte aligned), then float row_lse[rows]
};

constexpr size_t kHeader = 16;

__device__ __forceinline__ float* row_losses(CeWork* ws) {
  return reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + kHeader);
}

// Log-sum-exp of each row, kept for a deferred gradient (fp16); `rows` is the call's row count.
__device__ __forceinline__ const float* row_lses(const CeWork* ws, int64_t rows) {
  return reinterpret_cast<const float*>(reinterpret_cast<const char*>(ws) + kHeader) + rows;
}
__device__ __forceinline__ float* row_lses(CeWork* ws, int64_t rows) {
  return row_losses(ws) + rows;
}

// What the row kernels do with the gradient.  kGradWrite: write d(mean loss)/d(logits) over
// the logits.  kGradDefer (fp16): leave the logits as they are and keep each row's
// log-sum-exp; the backward then writes the gradient, grad_output included, rounding to fp16
// once.  fp16 cannot hold softmax / n_valid (about 1e-10 for vocab 128256 over 8192 rows: below
// its smallest subnormal) until the loss scale of fp16 training, which only arrives with the
// backward, lifts it.
constexpr int kGradNone = 0;
constexpr int kGradWrite = 1;
constexpr int kGradDefer = 2;

__device__ __forceinline__ float inv_n_of(const CeWork* ws) { return 1.0f / ws->n_valid; }

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

// Loads per thread that the one-block kernels (ce_prepare, ce_finish) keep in flight together.
constexpr int kFinishBatch = 8;

// This thread's count of kept targets among rows tid, tid + kThreads, ...: kFinishBatch
// targets in flight together (a load under a branch would be waited for before the next is
// issued: one round trip each); a row without a target loads targets[0] and is not counted.
template <bool SMALL>
__device__ __forceinline__ float count_kept_batched(const int64_t* __restrict__ targets,
                                                    int64_t inner, int64_t valid_inner,
                                                    int64_t tos, int64_t tis, int64_t rows,
                                                    int64_t ignore_index) {
  float cnt = 0.0f;
  for (int64_t base = threadIdx.x; base < rows; base += int64_t{kThreads} * kFinishBatch) {
    int64_t t[kFinishBatch];
    bool kept[kFinishBatch];
#pragma unroll
    for (int u = 0; u < kFinishBatch; ++u) {
      const int64_t r = base + static_cast<int64_t>(u) * kThreads;
      int64_t o, i;
      if constexpr (SMALL) {
        const uint32_t o32 = static_cast<uint32_t>(r) / static_cast<uint32_t>(inner);
        o = o32;
        i = static_cast<uint32_t>(r) - o32 * static_cast<uint32_t>(inner);
      } else {
        o = r / inner;
        i = r - o * inner;
      }
      kept[u] = r < rows && i < valid_inner;
      t[u] = targets[kept[u] ? o * tos + i * tis : 0];
    }
#pragma unroll
    for (int u = 0; u < kFinishBatch; ++u) cnt += (kept[u] && t[u] != ignore_index) ? 1.0f : 0.0f;
  }
  return cnt;
}

__global__ __launch_bounds__(kThreads) void ce_prepare_kernel(const int64_t* __restrict__ targets,
                                                               int64_t inner, int64_t valid_inner,
                                                               int64_t tos, int64_t tis,
                                                               int64_t rows, int64_t ignore_index,
                                                               CeWork* __restrict__ ws,
                                                               float* __restrict__ loss_out) {
  __shared__ float red[kWaves];
  float cnt = 0.0f;
  // Row decode in 32 bits when the counts allow it (the 64-bit division is a long
  // instruction sequence per target).
  if (valid_inner > 0) {
    if (rows + int64_t{kThreads} * kFinishBatch <= 0xffffffffLL) {
      cnt = count_kept_batched<true>(targets, inner, valid_inner, tos, tis, rows, ignore_index);
    } else {
      cnt = count_kept_batched<false>(targets, inner, valid_inner, tos, tis, rows, ignore_index);
    }
  }
  const float total = block_reduce_sum(cnt, red);
  if (threadIdx.x == 0) {
    ws->n_valid = total;
    ws->status = 0;
    if (rows == 0) *loss_out = NAN;  // mean over an empty batch: 0/0, as torch returns
  }
}

// Start of the streaming row kernel: locates the row and its target.  An ignored row
// (target == ignore_index, or a position i >= valid_inner that has no target) gets a zero
// gradient and a zero loss, and the function returns false.  Otherwise thread 0 reads the
// target logit into *s_target_logit (NaN for a target outside [0, vocab), which also sets
// status bit 0) before any thread of the block can overwrite the row: the block passes at
// least two barriers before its first gradient store.
template <typename T, int V, bool ALIGNED>
__device__ __forceinline__ bool ce_row_begin(const T* logits, T* grad, int64_t inner,
                                             int64_t valid_inner, int64_t os, int64_t is,
                                             int64_t gos, int64_t gis, int vocab,
                                             const int64_t* targets, int64_t tos, int64_t tis,
                                             int64_t ignore_index, int write_grad, CeWork* ws,
                                             const T** p_out, T** g_out, int* tgt_out,
                                             float* s_target_logit) {
  const int64_t row = blockIdx.x;
  const int64_t o = row / inner, ii = row - (row / inner) * inner;
  const T* p = logits + o * os + ii * is;
  T* g = grad + o * gos + ii * gis;
  const int64_t tgt = ii < valid_inner ? targets[o * tos + ii * tis] : ignore_index;
  if (tgt == ignore_index) {
    if (write_grad == kGradWrite) {
      for (int e = threadIdx.x * V; e < vocab; e += kThreads * V) {
        if constexpr (ALIGNED) {
          store16<true>(g + e, u32x4{0u, 0u, 0u, 0u});
        } else {
          g[e] = Elem<T>::from_f32(0.0f);
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
  *g_out = g;
  *tgt_out = bad ? -1 : static_cast<int>(tgt);
  return true;
}

// Row loss lse - x_t, written (max - x_t) + ln(sum exp(x - max)), free of the cancellation
// of two large numbers (lse and x_t): max - x_t is exact when the target is within a factor
// of two of the max, and a dominant target's small loss ln(sum) carries only the rounding of
// the fp32 sum, a few units of 2^-24.
__device__ __forceinline__ float row_loss(float mx, float se, float xt) {
  return (mx - xt) + __logf(se);
}

// Gradient of the target element, (softmax_t - 1) / n_valid, from the exact fp32 target
// logit as exp(x_t - max) / sum - 1 (exactly 0 for one class).  For a dominant target the
// subtraction cancels: the result is then accurate to a few units of 2^-24 absolutely, the
// rounding of the fp32 sum, not relative to its own small size (torch's fp32 path,
// exp(log_softmax_t) - 1, cancels the same way).
__device__ __forceinline__ float target_grad(float mx, float se, float xt, float inv_n) {
  return (exp_shifted(xt, mx) / se - 1.0f) * inv_n;
}

// Where a row lives and what its target is; uniform across the block.  A row without a
// target (ignore_index, or a position i >= valid_inner) has skip set.
struct RowRef {
  int64_t off;   // of the logits row
  int64_t goff;  // of its gradient row
  int64_t tgt;
  bool skip;
};

__device__ __forceinline__ RowRef row_ref(int64_t row, int64_t inner, int64_t valid_inner,
                                          int64_t os, int64_t is,
                                          const int64_t* __restrict__ targets, int64_t tos,
                                          int64_t tis, int64_t ignore_index, int64_t gos = 0,
                                          int64_t gis = 0) {
  const int64_t o = row / inner, ii = row - o * inner;
  RowRef r;
  r.off = o * os + ii * is;
  r.goff = o * gos + ii * gis;
  r.tgt = ii < valid_inner ? targets[o * tos + ii * tis] : ignore_index;
  r.skip = r.tgt == ignore_index;
  return r;
}

// Raw buffer resource (stride 0) over `bytes` bytes at `base`: the hardware drops loads
// past the end (they return 0) and stores past the end, so a row's ragged last vectors need
// no branches.  The range check covers the VGPR offset plus the instruction's immediate offset
// but not the SGPR offset, so every access below puts its whole offset in the VGPR operand
// and passes an SGPR offset of 0 (kBufferWord3 and the cache-policy bits: pt_common.hpp).

__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_buffer(void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(base, 0, bytes, kBufferWord3);
}

// exp(x - m) kept in the storage type in place of the logit: fp16 holds it scaled by 2^15
// (at most 32768 < 65504), so that values down to 2^-29 keep full fp16 precision instead of
// going subnormal; fp32 and bf16 have fp32's exponent range and need no scale.
template <typename T>
constexpr float kExpScale = std::is_same<T, _Float16>::value ? 32768.0f : 1.0f;

// A cache line: the row kernels start their 16-byte vectors on one, so that each wave's
// 1024-byte access covers 8 whole lines rather than 9 partial ones.
constexpr int kLineBytes = 128;

// The bit pattern of two / one -inf in the storage type, for masking vectors past the row.
template <typename T>
constexpr uint32_t kNegInfWord = std::is_same<T, float>::value      ? 0xff800000u
                                 : std::is_same<T, _Float16>::value ? 0xfc00fc00u
                                                                    : 0xff80ff80u;

// Register-resident rows, VPT 16-byte vectors per thread, one 1024-thread workgroup per row
// (a CU holds one such workgroup; when it retires its stores drain while the next row's
// workgroup loads, which keeps reads and writes in flight together).  Per row:
//   1. an online max / sum per thread as the vectors arrive: chunk k's elements become
//      e = exp(x - m_k), m_k the thread's running max after the chunk, summed in fp32 and
//      kept in the storage type in place of the logits; then the max and the rescaled sums
//      are reduced across the wave by shuffles and across the block through LDS (one
//      barrier);
//   2. the gradient e * exp(m_k - M) / (S * n_valid), one multiply per element with a factor
//      per chunk.  The thread holding the target writes the row loss and, after its own
//      vector store of that address, the target element (softmax_t - 1) / n_valid.
// Keeping e rounds the softmax twice in 16-bit storage (once as e, once as the gradient),
// a relative error of at most 2 units of the storage type's last place.
// The launch picks the smallest VPT of 1, 2, 3, 4, 6, 7, 8, 10, 12, 14, 16 that covers the
// row; each is at most twice the one before, so the vectors of chunks k < VPT / 2 are always
// inside it.
// Up to 64 VGPRs a CU holds two of these workgroups, one loading while the other reduces or
// stores: bf16 rows of 32000 and 48000 logits (VPT 4 and 6, 53 and 62 VGPRs) stream at
// 6.1-6.2 TB/s against 4.8 TB/s for 50256 (VPT 8 online: 77 VGPRs, one workgroup).  VPT 7
// and 8 therefore take the thread's max over all its vectors first and every exp against
// that one reference (kMaxFirst: no per-chunk maxima to keep), which brings them under 64.
template <int VPT>
constexpr bool kMaxFirst = VPT == 7 || VPT == 8;

template <typename T, int VPT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(kMaxFirst<VPT> ? 8 : 1))) void ce_rows_kernel(
    const T* logits, T* grad, int64_t inner, int64_t valid_inner, int64_t os, int64_t is,
    int64_t gos, int64_t gis, int vocab, const int64_t* __restrict__ targets, int64_t tos,
    int64_t tis, int64_t ignore_index, int write_grad, CeWork* __restrict__ ws) {
  constexpr int V = Elem<T>::VEC;
  constexpr int kChunkBytes = kThreads * 16;
  __shared__ float red_m[kWaves];
  __shared__ float red_s[kWaves];
  const int tid = threadIdx.x;
  const int wave = tid / 64, lane = tid % 64;
  const int64_t row = blockIdx.x;
  const int row_bytes = vocab * static_cast<int>(sizeof(T));
  const int voff = tid * 16;
  const RowRef cur =
      row_ref(row, inner, valid_inner, os, is, targets, tos, tis, ignore_index, gos, gis);
  const auto buf = row_buffer(const_cast<T*>(logits) + cur.off, row_bytes);
  const auto gbuf = row_buffer(grad + cur.goff, row_bytes);

  if (cur.skip) {
    if (write_grad == kGradWrite) {
#pragma unroll
      for (int k = 0; k < VPT; ++k)
        __builtin_amdgcn_raw_buffer_store_b128(u32x4{0u, 0u, 0u, 0u}, gbuf,
                                               voff + k * kChunkBytes, 0, kNonTemporal);
    }
    if (tid == 0) row_losses(ws)[row] = 0.0f;
    return;
  }

  Vec16<T> v[VPT];
#pragma unroll
  for (int k = 0; k < VPT; ++k)
    v[k].raw = __builtin_amdgcn_raw_buffer_load_b128(buf, voff + k * kChunkBytes, 0, kNonTemporal);

  // The target's vector index, its owner thread, chunk and lane are uniform; the owner
  // picks the exact target logit out of its registers.  A target outside [0, vocab) sets
  // status bit 0 and gives the row a NaN loss, as no logit is its own.
  const bool bad = cur.tgt < 0 || cur.tgt >= vocab;
  const int tvec = bad ? 0 : static_cast<int>(cur.tgt / V);
  const int owner = bad ? 0 : tvec % kThreads;
  const int tk = tvec / kThreads, ti = bad ? 0 : static_cast<int>(cur.tgt % V);
  if (bad && tid == 0) atomicOr(&ws->status, 1);
  float xt = NAN;
  if (!bad && tid == owner) {
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      if (k == tk) {
#pragma unroll
        for (int i = 0; i < V; ++i)
          if (i == ti) xt = Elem<T>::to_f32(v[k].e[i]);
      }
    }
  }

  float m = -INFINITY, s = 0.0f;
  // the reference of the exps kept for chunk k: the running max after it (online), or the
  // thread's max over all its chunks (kMaxFirst, one entry)
  constexpr bool kFirst = kMaxFirst<VPT>;
  float mk[kFirst ? 1 : VPT];
  const auto masked = [&](int k) -> Vec16<T> {
    Vec16<T> r = v[k];
    if (k >= VPT / 2 && (tid + k * kThreads) * V >= vocab) {
      const uint32_t ninf = kNegInfWord<T>;
      r.raw = u32x4{ninf, ninf, ninf, ninf};
    }
    return r;
  };
  if constexpr (kFirst) {
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const Vec16<T> r = masked(k);
#pragma unroll
      for (int i = 0; i < V; ++i) m = fmaxf(m, Elem<T>::to_f32(r.e[i]));
    }
    const float ref = m == -INFINITY ? 0.0f : m;
    // The exps convert the packed vectors again rather than keep the first pass's fp32
    // values, which would take VPT * V registers.
#pragma unroll
    for (int k = 0; k < VPT; ++k) asm volatile("" : "+v"(v[k].raw));
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const Vec16<T> r = masked(k);
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const float e = exp_shifted(Elem<T>::to_f32(r.e[i]), ref);
        s += e;
        v[k].e[i] = Elem<T>::from_f32(e * kExpScale<T>);
      }
      asm volatile("" : "+v"(v[k].raw));  // packed here, as below
    }
    mk[0] = m;
  } else {
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const Vec16<T> r = masked(k);
      float x[V];
#pragma unroll
      for (int i = 0; i < V; ++i) x[i] = Elem<T>::to_f32(r.e[i]);
      float cm = x[0];
#pragma unroll
      for (int i = 1; i < V; ++i) cm = fmaxf(cm, x[i]);
      const float nm = fmaxf(m, cm);
      const float ref = nm == -INFINITY ? 0.0f : nm;
      float add = 0.0f;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const float e = exp_shifted(x[i], ref);
        add += e;
        v[k].e[i] = Elem<T>::from_f32(e * kExpScale<T>);
      }
      // Packed here: left to itself the optimiser would carry the fp32 exps across the
      // barrier into the gradient branch, twice the registers.
      asm volatile("" : "+v"(v[k].raw));
      s = s * exp_shifted(m, ref) + add;
      m = nm;
      mk[k] = nm;
    }
  }
  // Max first, then one rescale per partial sum (a max of -inf is shifted by 0, as above).
  const float mw = wave_max(m);
  const float sw = wave_sum(s * exp_shifted(m, mw == -INFINITY ? 0.0f : mw));
  if (lane == 0) {
    red_m[wave] = mw;
    red_s[wave] = sw;
  }
  __syncthreads();
  float M = red_m[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) M = fmaxf(M, red_m[w]);
  const float refM = M == -INFINITY ? 0.0f : M;
  float S = 0.0f;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) S += red_s[w] * exp_shifted(red_m[w], refM);
  if (tid == owner) row_losses(ws)[row] = row_loss(M, S, xt);
  if (write_grad == kGradDefer && tid == 0) row_lses(ws, gridDim.x)[row] = M + __logf(S);
  if (write_grad != kGradWrite) return;

  const float scale = inv_n_of(ws) / S;
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    Vec16<T> out;
    // exp(m_k - M) / (S n) per chunk; 0 for a chunk whose reference is -inf (it held only
    // -inf logits, whose exps are 0).
    const float f = exp_shifted(mk[kFirst ? 0 : k], M) * (scale / kExpScale<T>);
#pragma unroll
    for (int i = 0; i < V; ++i) {
      out.e[i] = Elem<T>::from_f32(Elem<T>::to_f32(v[k].e[i]) * f);
    }
    // One add per store rather than sixteen offsets held in registers across the row.
    // Gradient stores write through L2 (as the RMSNorm forward's do): a [8192, 128256] bf16
    // call measured 1-6 µs faster than with nontemporal stores alone, never slower.
    int vo = voff + k * kChunkBytes;
    asm volatile("" : "+v"(vo));
    __builtin_amdgcn_raw_buffer_store_b128(out.raw, gbuf, vo, 0, kWriteThrough);
  }
  if (!bad && tid == owner) {
    Vec16<T> one;
    one.e[0] = Elem<T>::from_f32(target_grad(M, S, xt, inv_n_of(ws)));
    const int toff = static_cast<int>(cur.tgt) * static_cast<int>(sizeof(T));
    if constexpr (sizeof(T) == 4) {
      __builtin_amdgcn_raw_buffer_store_b32(one.raw[0], gbuf, toff, 0, kWriteThrough);
    } else {
      __builtin_amdgcn_raw_buffer_store_b16(static_cast<unsigned short>(one.raw[0] & 0xffffu),
                                            gbuf, toff, 0, kWriteThrough);
    }
  }
}

// Forward without a gradient write (no gradient, or the fp16 deferred one): a read-only
// pass, so nothing of the row has to stay in registers and 256-thread workgroups (46-73
// VGPRs) share a CU six or more at a time, each streaming its own row; the register-resident
// kernel, one 1024-thread workgroup per CU, leaves the CU's loads idle while it reduces a
// row when there is no store phase to overlap.  A row is split as in the batched kernel: a
// head of up to V-1 elements before its first 16-byte boundary and a tail of up to V-1
// after its last (one element per thread, folded in before the body), and a body of 16-byte
// vectors (all of an aligned row).  Per thread, batches of kLseBatch 16-byte nontemporal
// loads of the body (raw buffer loads: the range check returns zeros past the body, masked
// to -inf here) feed an online max / sum-exp with one rescale per batch; the wave and block
// reductions are those of ce_rows_kernel.  Thread 0 reads the target logit at the start (in
// flight with the row) and writes the row loss and, for a deferred gradient, the row's
// log-sum-exp.
constexpr int kLseThreads = 256;
constexpr int kLseWaves = kLseThreads / 64;
constexpr int kLseBatch = 8;

template <typename T>
__global__ __launch_bounds__(kLseThreads) void ce_lse_kernel(
    const T* __restrict__ logits, int64_t inner, int64_t valid_inner, int64_t os, int64_t is,
    int vocab, const int64_t* __restrict__ targets, int64_t tos, int64_t tis,
    int64_t ignore_index, int write_grad, CeWork* __restrict__ ws) {
  constexpr int V = Elem<T>::VEC;
  __shared__ float red_m[kLseWaves];
  __shared__ float red_s[kLseWaves];
  const int tid = threadIdx.x;
  const int wave = tid / 64, lane = tid % 64;
  const int64_t row = blockIdx.x;
  const RowRef cur = row_ref(row, inner, valid_inner, os, is, targets, tos, tis, ignore_index);
  if (cur.skip) {
    if (tid == 0) row_losses(ws)[row] = 0.0f;
    return;
  }
  const T* p = logits + cur.off;
  const bool bad = cur.tgt < 0 || cur.tgt >= vocab;
  float xt = NAN;  // a target outside [0, vocab): NaN loss and status bit 0
  if (tid == 0) {
    if (bad) {
      atomicOr(&ws->status, 1);
    } else {
      xt = Elem<T>::to_f32(p[cur.tgt]);
    }
  }
  // head [0, head): the elements before the row's first 128-byte line, as in the batched
  // kernel; body [head, head + nvec * V); tail [head + nvec * V, vocab)
  const int lead = static_cast<int>(((kLineBytes - (reinterpret_cast<uintptr_t>(p) & (kLineBytes - 1))) &
                                     (kLineBytes - 1)) / sizeof(T));
  const int head = lead < vocab ? lead : vocab;
  const int nvec = (vocab - head) / V;
  const int tail_start = head + nvec * V;
  const auto buf = row_buffer(const_cast<T*>(p) + head, nvec * 16);
  float m = -INFINITY, s = 0.0f;
  if (tid < head || tid < vocab - tail_start) {
    const float a = tid < head ? Elem<T>::to_f32(p[tid]) : -INFINITY;
    const float b = tid < vocab - tail_start ? Elem<T>::to_f32(p[tail_start + tid]) : -INFINITY;
    m = fmaxf(a, b);
    const float ref = m == -INFINITY ? 0.0f : m;
    s = exp_shifted(a, ref) + exp_shifted(b, ref);
  }
  for (int base = tid; base < nvec; base += kLseThreads * kLseBatch) {
    Vec16<T> v[kLseBatch];
#pragma unroll
    for (int u = 0; u < kLseBatch; ++u)
      v[u].raw = __builtin_amdgcn_raw_buffer_load_b128(buf, (base + u * kLseThreads) * 16, 0,
                                                       kNonTemporal);
    float cm = -INFINITY;
#pragma unroll
    for (int u = 0; u < kLseBatch; ++u) {
      if (base + u * kLseThreads >= nvec) {
        const uint32_t ninf = kNegInfWord<T>;
        v[u].raw = u32x4{ninf, ninf, ninf, ninf};
      }
#pragma unroll
      for (int i = 0; i < V; ++i) cm = fmaxf(cm, Elem<T>::to_f32(v[u].e[i]));
    }
    const float nm = fmaxf(m, cm);
    const float ref = nm == -INFINITY ? 0.0f : nm;
    float add = 0.0f;
#pragma unroll
    for (int u = 0; u < kLseBatch; ++u) {
#pragma unroll
      for (int i = 0; i < V; ++i) add += exp_shifted(Elem<T>::to_f32(v[u].e[i]), ref);
    }
    s = s * exp_shifted(m, ref) + add;
    m = nm;
  }
  const float mw = wave_max(m);
  const float sw = wave_sum(s * exp_shifted(m, mw == -INFINITY ? 0.0f : mw));
  if (lane == 0) {
    red_m[wave] = mw;
    red_s[wave] = sw;
  }
  __syncthreads();
  if (tid == 0) {
    float M = red_m[0];
#pragma unroll
    for (int w = 1; w < kLseWaves; ++w) M = fmaxf(M, red_m[w]);
    const float refM = M == -INFINITY ? 0.0f : M;
    float S = 0.0f;
#pragma unroll
    for (int w = 0; w < kLseWaves; ++w) S += red_s[w] * exp_shifted(red_m[w], refM);
    row_losses(ws)[row] = row_loss(M, S, xt);
    if (write_grad == kGradDefer) row_lses(ws, gridDim.x)[row] = M + __logf(S);
  }
}

// Rows that the register-resident kernel does not take -- longer than it holds, or not
// starting on a 128-byte cache line -- with row_bytes + kStreamBatchBytes < 2^31: one
// 1024-thread workgroup per row; rows of up to 16 vectors per thread are held whole in
// registers and read once, longer ones in two passes.  A row is split
// into a head of the elements before its first 128-byte boundary (at most 127 bytes' worth,
// one per thread, from thread 0), a body of 16-byte vectors read in batches of kStreamBatch
// per thread with raw buffer loads (the hardware range check drops the ragged end), and a
// tail of up to V-1 elements (one per thread, from the last thread).  Starting the body on a
// line makes each wave's 1024-byte access cover 8 whole lines rather than 9 partial ones: a
// [8160, V] bf16 forward streams at 5.8-6.0 TB/s for V a multiple of 64 and 4.7-4.9 TB/s for
// other multiples of 8 when the body starts at the row (50000, 50256, 54000, 57000, 62000).
// The kept chunks are reduced and written as in ce_rows_kernel; the part of a longer row
// past them takes two passes:
//   1. cached loads (the row stays in the Infinity Cache for pass 2) and an online max /
//      sum per thread, reduced with the kept chunks' (one barrier);
//   2. the part re-read (nontemporal: last use), exp(x - M) / (S * n_valid) written over it;
//      the thread that wrote the target's element then stores (softmax_t - 1) / n_valid.
constexpr int kStreamBatch = 4;
constexpr int kStreamBatchBytes = kStreamBatch * kThreads * 16;
// Leading body chunks (1024 vectors each) held in registers as exps, as in ce_rows_kernel:
// the launch keeps as many as a row needs up to 16, and kKeepChunks of a longer row, whose
// body beyond them is read twice.
constexpr int kKeepChunks = 12;

template <int KEEP>
constexpr bool kBatchedMaxFirst = KEEP >= 6 && KEEP <= 8;

template <typename T, int KEEP>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(kBatchedMaxFirst<KEEP> ? 8 : 1))) void ce_rows_batched_kernel(
    const T* logits, T* grad, int64_t inner, int64_t valid_inner, int64_t os, int64_t is,
    int64_t gos, int64_t gis, int vocab, const int64_t* __restrict__ targets, int64_t tos,
    int64_t tis, int64_t ignore_index, int write_grad, CeWork* __restrict__ ws) {
  constexpr int V = Elem<T>::VEC;
  constexpr int kChunkBytes = kThreads * 16;
  __shared__ float red_m[kWaves];
  __shared__ float red_s[kWaves];
  __shared__ float s_xt;
  const int tid = threadIdx.x;
  const int wave = tid / 64, lane = tid % 64;
  const int64_t row = blockIdx.x;
  const RowRef cur =
      row_ref(row, inner, valid_inner, os, is, targets, tos, tis, ignore_index, gos, gis);
  const T* p = logits + cur.off;
  T* g = grad + cur.goff;  // in the same 16-byte phase as p (checked on the host)
  // head [0, head): the elements before the row's first 128-byte boundary; body [head,
  // head + nbody * V); tail [head + nbody * V, vocab)
  const int lead = static_cast<int>(((kLineBytes - (reinterpret_cast<uintptr_t>(p) & (kLineBytes - 1))) &
                                     (kLineBytes - 1)) / sizeof(T));
  const int head = lead < vocab ? lead : vocab;
  const int nbody = (vocab - head) / V;
  const int tail_start = head + nbody * V;
  const int ntail = vocab - tail_start;
  const int body_bytes = nbody * 16;
  // only kKeepChunks streams the body past its kept chunks (the launch gives the other
  // instances rows that their kept chunks cover; without the streaming loops they need
  // fewer registers)
  const int stream_end = KEEP == kKeepChunks ? body_bytes : 0;
  const auto buf = row_buffer(const_cast<T*>(p) + head, body_bytes);
  const auto gbuf = row_buffer(g + head, body_bytes);
  const int voff = tid * 16;
  // the one head or tail element of this thread, if any
  const int my_edge = tid < head ? tid : (kThreads - 1 - tid < ntail ? tail_start + (kThreads - 1 - tid) : -1);

  if (cur.skip) {
    if (write_grad == kGradWrite) {
      for (int b = 0; b < body_bytes; b += kChunkBytes)
        __builtin_amdgcn_raw_buffer_store_b128(u32x4{0u, 0u, 0u, 0u}, gbuf, voff + b, 0,
                                               kNonTemporal);
      if (my_edge >= 0) g[my_edge] = Elem<T>::from_f32(0.0f);
    }
    if (tid == 0) row_losses(ws)[row] = 0.0f;
    return;
  }
  Vec16<T> kv[KEEP];
#pragma unroll
  for (int k = 0; k < KEEP; ++k)
    kv[k].raw = __builtin_amdgcn_raw_buffer_load_b128(buf, voff + k * kChunkBytes, 0, kNonTemporal);
  const bool bad = cur.tgt < 0 || cur.tgt >= vocab;
  if (tid == 0) {
    s_xt = bad ? NAN : Elem<T>::to_f32(p[cur.tgt]);
    if (bad) atomicOr(&ws->status, 1);
  }

  float m = -INFINITY, s = 0.0f;
  if (my_edge >= 0) {
    m = Elem<T>::to_f32(p[my_edge]);
    s = m == -INFINITY ? 0.0f : 1.0f;  // exp(x - x); a lone -inf contributes nothing
  }
  // the reference of kept chunk k's exps: the running max after it, or for 6 to 8 kept
  // chunks (as in ce_rows_kernel, to stay under 64 VGPRs: 64 against 66-78 online) the
  // thread's max over its edge element and all its kept chunks
  constexpr bool kFirst = kBatchedMaxFirst<KEEP>;
  float mk[kFirst ? 1 : KEEP];
  const auto masked = [&](int k) -> Vec16<T> {
    Vec16<T> r = kv[k];
    if (voff + k * kChunkBytes >= body_bytes) {
      const uint32_t ninf = kNegInfWord<T>;
      r.raw = u32x4{ninf, ninf, ninf, ninf};
    }
    return r;
  };
  if constexpr (kFirst) {
    const float m0 = m;
#pragma unroll
    for (int k = 0; k < KEEP; ++k) {
      const Vec16<T> r = masked(k);
#pragma unroll
      for (int i = 0; i < V; ++i) m = fmaxf(m, Elem<T>::to_f32(r.e[i]));
    }
    const float ref = m == -INFINITY ? 0.0f : m;
    s *= exp_shifted(m0, ref);
#pragma unroll
    for (int k = 0; k < KEEP; ++k) asm volatile("" : "+v"(kv[k].raw));  // convert again
#pragma unroll
    for (int k = 0; k < KEEP; ++k) {
      const Vec16<T> r = masked(k);
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const float e = exp_shifted(Elem<T>::to_f32(r.e[i]), ref);
        s += e;
        kv[k].e[i] = Elem<T>::from_f32(e * kExpScale<T>);
      }
      asm volatile("" : "+v"(kv[k].raw));
    }
    mk[0] = m;
  } else {
#pragma unroll
    for (int k = 0; k < KEEP; ++k) {
      const Vec16<T> r = masked(k);
      float x[V];
#pragma unroll
      for (int i = 0; i < V; ++i) x[i] = Elem<T>::to_f32(r.e[i]);
      float cm = x[0];
#pragma unroll
      for (int i = 1; i < V; ++i) cm = fmaxf(cm, x[i]);
      const float nm = fmaxf(m, cm);
      const float ref = nm == -INFINITY ? 0.0f : nm;
      float add = 0.0f;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const float e = exp_shifted(x[i], ref);
        add += e;
        kv[k].e[i] = Elem<T>::from_f32(e * kExpScale<T>);
      }
      asm volatile("" : "+v"(kv[k].raw));  // packed here, not carried as fp32 across the barrier
      s = s * exp_shifted(m, ref) + add;
      m = nm;
      mk[k] = nm;
    }
  }
  for (int b = KEEP * kChunkBytes; b < stream_end; b += kStreamBatchBytes) {
    Vec16<T> v[kStreamBatch];
#pragma unroll
    for (int u = 0; u < kStreamBatch; ++u)
      v[u].raw = __builtin_amdgcn_raw_buffer_load_b128(buf, voff + b + u * kChunkBytes, 0, 0);
#pragma unroll
    for (int u = 0; u < kStreamBatch; ++u) {
      if (voff + b + u * kChunkBytes >= body_bytes) {
        const uint32_t ninf = kNegInfWord<T>;
        v[u].raw = u32x4{ninf, ninf, ninf, ninf};
      }
      float x[V];
#pragma unroll
      for (int i = 0; i < V; ++i) x[i] = Elem<T>::to_f32(v[u].e[i]);
      float cm = x[0];
#pragma unroll
      for (int i = 1; i < V; ++i) cm = fmaxf(cm, x[i]);
      const float nm = fmaxf(m, cm);
      const float ref = nm == -INFINITY ? 0.0f : nm;
      float add = 0.0f;
#pragma unroll
      for (int i = 0; i < V; ++i) add += exp_shifted(x[i], ref);
      s = s * exp_shifted(m, ref) + add;
      m = nm;
    }
  }
  const float mw = wave_max(m);
  const float sw = wave_sum(s * exp_shifted(m, mw == -INFINITY ? 0.0f : mw));
  if (lane == 0) {
    red_m[wave] = mw;
    red_s[wave] = sw;
  }
  __syncthreads();
  float M = red_m[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) M = fmaxf(M, red_m[w]);
  const float refM = M == -INFINITY ? 0.0f : M;
  float S = 0.0f;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) S += red_s[w] * exp_shifted(red_m[w], refM);
  const float xt = s_xt;
  if (tid == 0) row_losses(ws)[row] = row_loss(M, S, xt);
  if (write_grad == kGradDefer && tid == 0) row_lses(ws, gridDim.x)[row] = M + __logf(S);
  if (write_grad != kGradWrite) return;

  const float inv_n = inv_n_of(ws);
  const float scale = inv_n / S;
#pragma unroll
  for (int k = 0; k < KEEP; ++k) {
    // exp(m_k - M) / (S n) per chunk; 0 for a chunk whose reference is -inf
    const float f = exp_shifted(mk[kFirst ? 0 : k], M) * (scale / kExpScale<T>);
    Vec16<T> out;
#pragma unroll
    for (int i = 0; i < V; ++i) out.e[i] = Elem<T>::from_f32(Elem<T>::to_f32(kv[k].e[i]) * f);
    int vo = voff + k * kChunkBytes;
    asm volatile("" : "+v"(vo));
    __builtin_amdgcn_raw_buffer_store_b128(out.raw, gbuf, vo, 0, kWriteThrough);
  }
  for (int b = KEEP * kChunkBytes; b < stream_end; b += kStreamBatchBytes) {
    Vec16<T> v[kStreamBatch];
#pragma unroll
    for (int u = 0; u < kStreamBatch; ++u)
      v[u].raw = __builtin_amdgcn_raw_buffer_load_b128(buf, voff + b + u * kChunkBytes, 0,
                                                       kNonTemporal);
#pragma unroll
    for (int u = 0; u < kStreamBatch; ++u) {
      Vec16<T> out;
#pragma unroll
      for (int i = 0; i < V; ++i)
        out.e[i] = Elem<T>::from_f32(exp_shifted(Elem<T>::to_f32(v[u].e[i]), M) * scale);
      __builtin_amdgcn_raw_buffer_store_b128(out.raw, gbuf, voff + b + u * kChunkBytes, 0,
                                             kWriteThrough);
    }
  }
  if (my_edge >= 0) g[my_edge] = Elem<T>::from_f32(exp_shifted(Elem<T>::to_f32(p[my_edge]), M) * scale);
  if (!bad) {
    // The owner rewrites the target over its own earlier store of that element, through the
    // same kind of access (buffer store for the body, plain store for head and tail), so the
    // two stay in program order.
    const int t = static_cast<int>(cur.tgt);
    const bool in_body = t >= head && t < tail_start;
    const int owner = t < head ? t : (in_body ? ((t - head) / V) % kThreads
                                              : kThreads - 1 - (t - tail_start));
    if (tid == owner) {
      const T gt = Elem<T>::from_f32(target_grad(M, S, xt, inv_n));
      if (in_body) {
        Vec16<T> one;
        one.e[0] = gt;
        const int toff = (t - head) * static_cast<int>(sizeof(T));
        if constexpr (sizeof(T) == 4) {
          __builtin_amdgcn_raw_buffer_store_b32(one.raw[0], gbuf, toff, 0, kWriteThrough);
        } else {
          __builtin_amdgcn_raw_buffer_store_b16(static_cast<unsigned short>(one.raw[0] & 0xffffu),
                                                gbuf, toff, 0, kWriteThrough);
        }
      } else {
        g[t] = gt;
      }
    }
  }
}

// Rows of 2^31 bytes and more: pass 1 streams the row once with an online max / sum-exp per
// thread; pass 2 re-reads it to write the gradient.
template <typename T, bool ALIGNED>
__global__ __launch_bounds__(kThreads) void ce_rows_stream_kernel(
    const T* logits, T* grad, int64_t inner, int64_t valid_inner, int64_t os, int64_t is,
    int64_t gos, int64_t gis, int vocab, const int64_t* __restrict__ targets, int64_t tos,
    int64_t tis, int64_t ignore_index, int write_grad, CeWork* __restrict__ ws) {
  constexpr int V = ALIGNED ? Elem<T>::VEC : 1;
  __shared__ float red[kWaves];
  __shared__ float s_target_logit;
  const T* p = nullptr;
  T* g = nullptr;
  int tgt = 0;
  if (!ce_row_begin<T, V, ALIGNED>(logits, grad, inner, valid_inner, os, is, gos, gis, vocab,
                                   targets, tos, tis, ignore_index, write_grad, ws, &p, &g, &tgt,
                                   &s_target_logit))
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
  if (write_grad == kGradDefer && threadIdx.x == 0)
    row_lses(ws, gridDim.x)[blockIdx.x] = mx + __logf(se);
  if (write_grad != kGradWrite) return;

  const float inv_n = inv_n_of(ws);
  const float scale = inv_n / se;
  const float gt = target_grad(mx, se, xt, inv_n);
  for (int e = threadIdx.x * V; e < vocab; e += kThreads * V) {
    float x[V];
    load(e, x);
    float gv[V];
#pragma unroll
    for (int i = 0; i < V; ++i) gv[i] = (e + i == tgt) ? gt : exp_shifted(x[i], mx) * scale;
    if constexpr (ALIGNED) {
      store_f32<T, true>(g + e, gv, V);
    } else {
      g[e] = Elem<T>::from_f32(gv[0]);
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
  // kFinishBatch losses per thread in flight together, added in increasing row order (the
  // order of one load at a time); rows past the end load the last row's loss and add 0.
  for (int64_t base = threadIdx.x; base < rows; base += int64_t{kThreads} * kFinishBatch) {
    float v[kFinishBatch];
#pragma unroll
    for (int u = 0; u < kFinishBatch; ++u) {
      const int64_t r = base + static_cast<int64_t>(u) * kThreads;
      v[u] = rl[r < rows ? r : rows - 1];
    }
#pragma unroll
    for (int u = 0; u < kFinishBatch; ++u)
      acc += base + static_cast<int64_t>(u) * kThreads < rows ? v[u] : 0.0f;
  }
  const float total = block_reduce_sum(acc, red);
  if (threadIdx.x == 0) *loss_out = total / ws->n_valid;
}

// The backward.  fp32 and bf16: in-place gradient scaling by a device scalar, a no-op when the
// scalar is exactly 1.  fp16 (deferred gradient): each element x of the untouched logits
// (`src`: the gradient rows themselves when in place) gives the gradient element
// (exp(x - lse) - [j == target]) * (grad_output / n_valid), computed in fp32 and rounded to
// fp16 once (lse from the forward's workspace).  Ignored rows are zero whatever the
// scalar is (torch's nll_loss backward leaves them 0).
// The work items are (row, chunk of 1024 vectors or elements); a grid of up to 128 blocks
// per CU walks them (a one-shot grid streams no faster and makes the common
// grad_output == 1 launch several times dearer).  The body moves in 16-byte vectors (4 per
// thread per chunk, loads nontemporal: touched once); rows that do not start on a 128-byte
// line (!ALIGNED) split off a head of elements up to the line and a tail of fewer than one
// vector, one element per thread.
constexpr int kScaleVecs = 4;

template <typename T, bool ALIGNED>
__global__ __launch_bounds__(256) void ce_scale_kernel(T* logits, const T* src, int64_t inner,
                                                       int64_t valid_inner, int64_t os,
                                                       int64_t is, int64_t sos, int64_t sis,
                                                       int vocab, int64_t items, int64_t chunks,
                                                       const int64_t* __restrict__ targets,
                                                       int64_t tos, int64_t tis,
                                                       int64_t ignore_index,
                                                       const float* __restrict__ scale,
                                                       const CeWork* __restrict__ ws) {
  constexpr int V = Elem<T>::VEC;
  constexpr bool kDefer = std::is_same<T, _Float16>::value;
  float sc = *scale;
  if constexpr (kDefer) {
    sc = sc / ws->n_valid;  // grad_output / total_weight, as torch's nll_loss backward forms it
  } else {
    if (sc == 1.0f) return;
  }
  const int64_t rows = items / chunks;
  // Item decode in 32 bits when the counts allow it (the usual case; a uniform branch):
  // 64-bit divisions are long scalar sequences ahead of every item's loads.
  const bool small = items <= 0xffffffffLL && inner <= 0xffffffffLL;
  for (int64_t item = blockIdx.x; item < items; item += gridDim.x) {
    int64_t row, c, o, ii;
    if (small) {
      const uint32_t r32 = static_cast<uint32_t>(item) / static_cast<uint32_t>(chunks);
      const uint32_t o32 = r32 / static_cast<uint32_t>(inner);
      row = r32;
      c = static_cast<uint32_t>(item) - r32 * static_cast<uint32_t>(chunks);
      o = o32;
      ii = r32 - o32 * static_cast<uint32_t>(inner);
    } else {
      row = item / chunks;
      c = item - row * chunks;
      o = row / inner;
      ii = row - o * inner;
    }
    const int64_t tgt = ii < valid_inner ? targets[o * tos + ii * tis] : ignore_index;
    const bool skip = tgt == ignore_index;
    if (!kDefer && skip) continue;
    T* p = logits + o * os + ii * is;
    const T* q = src + o * sos + ii * sis;  // same 16-byte phase as p (checked on the host)
    // Rows not on 128-byte lines: a head of the elements before the first line (one per
    // thread), a body of 16-byte vectors and a tail of fewer than V elements; rows on lines
    // (ALIGNED) are all body.
    int lead = 0;
    if constexpr (!ALIGNED) {
      lead = static_cast<int>(((kLineBytes - (reinterpret_cast<uintptr_t>(p) & (kLineBytes - 1))) &
                               (kLineBytes - 1)) / sizeof(T));
      if (lead > vocab) lead = vocab;
    }
    const int nbody = (vocab - lead) / V;
    T* body = p + lead;
    // read whether or not the row is ignored (an ignored row's value is never used), so the
    // load does not wait for the target's
    const float lse = kDefer ? row_lses(ws, rows)[row] : 0.0f;
    // The gradient of element j (row index) holding x.
    const auto grad = [&](float x, int64_t j) -> float {
      if constexpr (kDefer) {
        float y = exp_shifted(x, lse);
        if (j == tgt) y -= 1.0f;
        return y * sc;
      } else {
        return x * sc;
      }
    };
    // The item's chunk of the body through a raw buffer resource sized to the part of the
    // chunk inside the row: loads past it return zeros and stores past it are dropped, so
    // the code has no branches, all four loads are in flight together and every gradient
    // is computed before the first store (a load waited for after a store waits for the
    // store too).  Within a row, indexes fit in 32 bits.
    const int cstart = static_cast<int>(c) * (256 * kScaleVecs);  // first vector of the chunk
    const int cvecs = nbody - cstart < 256 * kScaleVecs ? nbody - cstart : 256 * kScaleVecs;
    const int cbytes = cvecs > 0 ? cvecs * 16 : 0;
    T* cptr = body + static_cast<int64_t>(cstart) * V;
    const T* qptr = q + lead + static_cast<int64_t>(cstart) * V;
    // an ignored row (deferred gradient) reads nothing: its load resource is empty
    const auto lbuf = row_buffer(const_cast<T*>(qptr), skip ? 0 : cbytes);
    const auto sbuf = row_buffer(cptr, cbytes);
    // the target's index in the chunk, or -1 when it is not there (ignored, in another
    // chunk, in the head or tail of an unaligned row, or outside the row)
    const int64_t trel64 = tgt - lead - static_cast<int64_t>(cstart) * V;
    const int trel = (trel64 >= 0 && trel64 < int64_t{256} * kScaleVecs * V) ? static_cast<int>(trel64) : -1;
    const int tid = static_cast<int>(threadIdx.x);
    // In a row not on a line, the first item also takes the head elements and the item of
    // the body's last chunk the tail elements (one per thread), so that each end of the row
    // is written by one item; their loads go out with the vector loads, so that their
    // latency overlaps them rather than following the vector stores.
    T head_v{}, tail_v{};
    bool has_head = false, has_tail = false;
    const int tail_j = lead + nbody * V + tid;
    if constexpr (!ALIGNED) {
      const int last_c = nbody > 0 ? (nbody - 1) / (256 * kScaleVecs) : 0;
      const bool read = !(kDefer && skip);  // an ignored fp16 row is written as zeros
      has_head = c == 0 && tid < lead;
      has_tail = c == last_c && tid < V && tail_j < vocab;
      if (has_head && read) head_v = q[tid];
      if (has_tail && read) tail_v = q[tail_j];
    }
    Vec16<T> in[kScaleVecs];
#pragma unroll
    for (int k = 0; k < kScaleVecs; ++k)
      in[k].raw = __builtin_amdgcn_raw_buffer_load_b128(lbuf, (k * 256 + tid) * 16, 0, kNonTemporal);
    Vec16<T> out[kScaleVecs];
#pragma unroll
    for (int k = 0; k < kScaleVecs; ++k) {
#pragma unroll
      for (int i = 0; i < V; ++i) {
        float y;
        if constexpr (kDefer) {
          y = exp_shifted(Elem<T>::to_f32(in[k].e[i]), lse);
          if ((k * 256 + tid) * V + i == trel) y -= 1.0f;
          y = skip ? 0.0f : y * sc;
        } else {
          y = Elem<T>::to_f32(in[k].e[i]) * sc;
        }
        // rounded to fp32 and then to the storage type, as torch rounds (left alone, the
        // compiler fuses the multiply and the 16-bit conversion into one rounding)
        asm volatile("" : "+v"(y));
        out[k].e[i] = Elem<T>::from_f32(y);
      }
    }
#pragma unroll
    for (int k = 0; k < kScaleVecs; ++k)
      __builtin_amdgcn_raw_buffer_store_b128(out[k].raw, sbuf, (k * 256 + tid) * 16, 0, kWriteThrough);
    if constexpr (!ALIGNED) {
      // The value is rounded to fp32 before the conversion, as in the vector path (left
      // alone, the compiler fuses the last multiply and the fp16 conversion into one rounding).
      const auto fix = [&](T v, int64_t j) {
        float y = skip ? 0.0f : grad(Elem<T>::to_f32(v), j);
        asm volatile("" : "+v"(y));
        return Elem<T>::from_f32(y);
      };
      if (has_head) p[tid] = fix(head_v, tid);
      if (has_tail) p[tail_j] = fix(tail_v, tail_j);
    }
  }
}

// Row and target description shared by the launches of one call.  `grad` (strides gos, gis)
// receives the gradient: the logits themselves when in place.  For the backward, `logits`
// holds the gradient rows and `grad` the rows the fp16 gradient is computed from.
struct CeRows {
  void* logits;
  int64_t inner, valid_inner, os, is;
  int vocab;
  const int64_t* targets;
  int64_t tos, tis, ignore_index;
  void* grad;
  int64_t gos, gis;
};

// Resident row workgroups per CU (0: no limit); PT_CE_OCCUPANCY overrides it.
int rows_occupancy() {
  static const int v = static_cast<int>(env_int("PT_CE_OCCUPANCY", 0));
  return v;
}

// Dynamic LDS bytes that apply the row-kernel occupancy limit to `kernel` (0 when there is
// none, or when the runtime refuses the allocation).
size_t rows_lds(const void* kernel) {
  const size_t lds = occupancy_lds(rows_occupancy(), 0);
  return allow_dynamic_lds(kernel, lds) == PT_OK ? lds : 0;
}

template <typename T, int VPT>
void launch_rows(const CeRows& d, int write_grad, CeWork* ws, int64_t rows, hipStream_t st) {
  const auto kernel = ce_rows_kernel<T, VPT>;
  hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(rows)), dim3(kThreads),
                     rows_lds(reinterpret_cast<const void*>(kernel)), st,
                     static_cast<const T*>(d.logits), static_cast<T*>(d.grad), d.inner,
                     d.valid_inner, d.os, d.is, d.gos, d.gis, d.vocab, d.targets, d.tos, d.tis,
                     d.ignore_index, write_grad, ws);
}

// Register-resident rows for up to 16 vectors per thread (131072 fp16/bf16 or 65536 fp32
// elements) when every row is 16-byte aligned and, up to 8 vectors per thread, starts on a
// 128-byte line; other rows take the batched kernel (the element-wise stream only for rows
// of 2 GB and more).
template <typename T>
void dispatch_rows(bool aligned, bool lines, const CeRows& d, int write_grad, CeWork* ws, int64_t rows,
                   hipStream_t st) {
  const int64_t per_thread = (static_cast<int64_t>(d.vocab) + int64_t{kThreads} * Elem<T>::VEC - 1) /
                             (int64_t{kThreads} * Elem<T>::VEC);
  const int64_t row_bytes = static_cast<int64_t>(d.vocab) * static_cast<int64_t>(sizeof(T));
  if (write_grad != kGradWrite && row_bytes + int64_t{kLseThreads} * kLseBatch * 16 < (int64_t{1} << 31)) {
    hipLaunchKernelGGL(ce_lse_kernel<T>, dim3(static_cast<unsigned>(rows)), dim3(kLseThreads), 0,
                       st, static_cast<const T*>(d.logits), d.inner, d.valid_inner, d.os, d.is,
                       d.vocab, d.targets, d.tos, d.tis, d.ignore_index, write_grad, ws);
    return;
  }
  // fp16 never writes its gradient in the forward (it is deferred to the backward), and
  // neither does a loss-only call: their rows take ce_lse_kernel above (from 2 GB, the
  // stream kernel), so the register-resident and batched kernels have no fp16 instances.
  if constexpr (!std::is_same<T, _Float16>::value) {
    // rows that do not start on a line take the batched kernel, which starts its vectors on
    // one (up to 16 vectors per thread, the same single read of the row)
    if (aligned && lines) {
#define PT_CE_CASE(N)                                  \
  if (per_thread <= N) {                               \
    launch_rows<T, N>(d, write_grad, ws, rows, st);    \
    return;                                            \
  }
      PT_CE_CASE(1)
      PT_CE_CASE(2)
      PT_CE_CASE(3)
      PT_CE_CASE(4)
      PT_CE_CASE(6)
      PT_CE_CASE(7)
      PT_CE_CASE(8)
      PT_CE_CASE(10)
      PT_CE_CASE(12)
      PT_CE_CASE(14)
      PT_CE_CASE(16)
#undef PT_CE_CASE
    }
    if (row_bytes + kStreamBatchBytes < (int64_t{1} << 31)) {
      // Rows whose body fits in 1, 2, 4, 6, 7, 8, 10, 12, 14 or 16 kept chunks are read
      // once; longer rows keep kKeepChunks and stream the rest twice.  Up to 8 kept chunks
      // leave room for two workgroups per CU.
#define PT_CE_BATCHED(K)                                                                        \
  hipLaunchKernelGGL((ce_rows_batched_kernel<T, K>), dim3(static_cast<unsigned>(rows)),        \
                     dim3(kThreads),                                                           \
                     rows_lds(reinterpret_cast<const void*>(ce_rows_batched_kernel<T, K>)), st, \
                     static_cast<const T*>(d.logits), static_cast<T*>(d.grad), d.inner,          \
                     d.valid_inner, d.os, d.is, d.gos, d.gis, d.vocab, d.targets, d.tos, d.tis,  \
                     d.ignore_index, write_grad, ws)
      if (per_thread <= 1) {
        PT_CE_BATCHED(1);
      } else if (per_thread <= 2) {
        PT_CE_BATCHED(2);
      } else if (per_thread <= 4) {
        PT_CE_BATCHED(4);
      } else if (per_thread <= 6) {
        PT_CE_BATCHED(6);
      } else if (per_thread <= 7) {
        PT_CE_BATCHED(7);
      } else if (per_thread <= 8) {
        PT_CE_BATCHED(8);
      } else if (per_thread <= 10) {
        PT_CE_BATCHED(10);
      } else if (per_thread <= 12) {
        PT_CE_BATCHED(12);
      } else if (per_thread <= 14) {
        PT_CE_BATCHED(14);
      } else if (per_thread <= 16) {
        PT_CE_BATCHED(16);
      } else {
        PT_CE_BATCHED(kKeepChunks);
      }
#undef PT_CE_BATCHED
      return;
    }
  }
  if (aligned) {
    hipLaunchKernelGGL((ce_rows_stream_kernel<T, true>), dim3(static_cast<unsigned>(rows)),
                       dim3(kThreads), 0, st, static_cast<const T*>(d.logits),
                       static_cast<T*>(d.grad), d.inner, d.valid_inner, d.os, d.is, d.gos, d.gis,
                       d.vocab, d.targets, d.tos, d.tis, d.ignore_index, write_grad, ws);
  } else {
    hipLaunchKernelGGL((ce_rows_stream_kernel<T, false>), dim3(static_cast<unsigned>(rows)),
                       dim3(kThreads), 0, st, static_cast<const T*>(d.logits),
                       static_cast<T*>(d.grad), d.inner, d.valid_inner, d.os, d.is, d.gos, d.gis,
                       d.vocab, d.targets, d.tos, d.tis, d.ignore_index, write_grad, ws);
  }
}

// True when every row of `b` (strides bos, bis) starts in the same 16-byte phase as the
// matching row of `a` (strides aos, ais): the row kernels split a row at the logits' 16-byte
// boundaries and address the gradient row with the same offsets.
bool same_phase(const void* a, int64_t aos, int64_t ais, const void* b, int64_t bos, int64_t bis,
                int64_t outer, int64_t inner, int esize) {
  const int64_t base = static_cast<int64_t>(reinterpret_cast<uintptr_t>(b)) -
                       static_cast<int64_t>(reinterpret_cast<uintptr_t>(a));
  return base % 16 == 0 && (outer <= 1 || ((bos - aos) * esize) % 16 == 0) &&
         (inner <= 1 || ((bis - ais) * esize) % 16 == 0);
}

// The fused loss over outer x inner rows, of which positions i >= valid_inner carry no target.
int ce_run(const char* fn, const CeRows& d, int64_t outer, int64_t inner, int64_t vocab,
           float* loss_out, int write_grad, void* workspace, size_t workspace_bytes, int dtype,
           void* stream) {
  const std::string name(fn);
  if (!valid_dtype(dtype)) return fail(PT_EINVAL, name + ": unknown dtype code");
  if (outer < 0 || inner < 0 || vocab <= 0) return fail(PT_EINVAL, name + ": bad shape");
  if (vocab > (int64_t{1} << 30)) return fail(PT_EUNSUPPORTED, name + ": vocab too large");
  const int64_t rows = outer * inner;
  // One 1024-thread workgroup per row; an HSA grid holds at most 2^32 - 1 work-items.
  if (rows * kThreads > 0xffffffffLL)
    return fail(PT_EUNSUPPORTED, name + ": more than 4194303 rows");
  if (!loss_out || !workspace) return fail(PT_EINVAL, name + ": null pointer");
  if (rows > 0 && (!d.logits || (d.valid_inner > 0 && !d.targets)))
    return fail(PT_EINVAL, name + ": null pointer");
  if (workspace_bytes < pt_cross_entropy_workspace_bytes(rows) || !aligned16(workspace))
    return fail(PT_EINVAL, name + ": workspace too small or not 16-byte aligned");
  if (rows > 0 && d.grad != d.logits &&
      !same_phase(d.logits, d.os, d.is, d.grad, d.gos, d.gis, outer, inner, dtype_size(dtype)))
    return fail(PT_EINVAL, name + ": gradient rows must start in the same 16-byte phase as the "
                                  "logits rows");
  hipStream_t st = as_stream(stream);
  CeWork* ws = static_cast<CeWork*>(workspace);
  hipLaunchKernelGGL(ce_prepare_kernel, dim3(1), dim3(kThreads), 0, st, d.targets, d.inner,
                     d.valid_inner, d.tos, d.tis, rows, d.ignore_index, ws, loss_out);
  if (int rc = check_launch(fn)) return rc;
  if (rows == 0) return ok();
  const int esize = dtype_size(dtype);
  const bool aligned = aligned16(d.logits) && (vocab * esize) % 16 == 0 &&
                       (outer <= 1 || (d.os * esize) % 16 == 0) &&
                       (inner <= 1 || (d.is * esize) % 16 == 0);
  // every row starts on a 128-byte line
  const bool lines = reinterpret_cast<uintptr_t>(d.logits) % kLineBytes == 0 &&
                     (outer <= 1 || (d.os * esize) % kLineBytes == 0) &&
                     (inner <= 1 || (d.is * esize) % kLineBytes == 0);
  const int mode = !write_grad ? kGradNone : (dtype == PT_FLOAT16 ? kGradDefer : kGradWrite);
  if (dtype == PT_FLOAT32) {
    dispatch_rows<float>(aligned, lines, d, mode, ws, rows, st);
  } else if (dtype == PT_FLOAT16) {
    dispatch_rows<_Float16>(aligned, lines, d, mode, ws, rows, st);
  } else {
    dispatch_rows<__bf16>(aligned, lines, d, mode, ws, rows, st);
  }
  if (int rc = check_launch(fn)) return rc;
  hipLaunchKernelGGL(ce_finish_kernel, dim3(1), dim3(kThreads), 0, st, ws, rows, loss_out);
  return check_launch(fn);
}

template <typename T, bool ALIGNED>
void scale_launch_as(const CeRows& d, int64_t rows, const float* grad_output, const CeWork* ws,
                     hipStream_t st) {
  // (row, chunk of 256 * kScaleVecs body vectors) items; a row's body has at most
  // vocab / VEC vectors whether or not it is aligned.
  constexpr int64_t kChunk = 256 * Elem<T>::VEC * kScaleVecs;
  const int64_t chunks = (d.vocab + kChunk - 1) / kChunk;
  const int64_t items = rows * chunks;
  // fp32 / bf16 scaling: a walk of up to 128 workgroups per CU, at most 4 resident per CU
  // (four 16-byte vectors in flight per thread: [8192, 128256] bf16 761 -> 714 us, vocab
  // 151936 935 -> 846 us); a one-shot grid streams no faster and makes the common
  // grad_output == 1 launch, which returns at once, several times dearer.  fp16 (the deferred
  // gradient, always computed): one workgroup per item, at most 3 resident per CU, so that no
  // item's loads wait behind an earlier item's stores in the same wave ([4 x 2049, 128256]
  // 711 -> 659 us against the walk; 4 per CU 685 us, 2 per CU 791 us).  The grid stays below
  // 2^24 workgroups (the walk covers any remainder).  PT_CE_SCALE_BLOCKS_PER_CU,
  // PT_CE_SCALE_OCCUPANCY and PT_CE_DEFER_OCCUPANCY override the three figures.
  constexpr bool kDefer = std::is_same<T, _Float16>::value;
  static const int64_t walk_blocks = env_int("PT_CE_SCALE_BLOCKS_PER_CU", 128);
  const int64_t cap = (kDefer || walk_blocks <= 0) ? (int64_t{1} << 24) - 1
                                                   : static_cast<int64_t>(num_cus()) * walk_blocks;
  const unsigned grid = static_cast<unsigned>(items < cap ? items : cap);
  static const int walk_per_cu = static_cast<int>(env_int("PT_CE_SCALE_OCCUPANCY", 4));
  static const int defer_per_cu = static_cast<int>(env_int("PT_CE_DEFER_OCCUPANCY", 3));
  const int per_cu = kDefer ? defer_per_cu : walk_per_cu;
  const auto kernel = ce_scale_kernel<T, ALIGNED>;
  size_t lds = occupancy_lds(per_cu, 0);
  if (allow_dynamic_lds(reinterpret_cast<const void*>(kernel), lds) != PT_OK) lds = 0;
  hipLaunchKernelGGL(kernel, dim3(grid), dim3(256), lds, st, static_cast<T*>(d.logits),
                     static_cast<const T*>(d.grad), d.inner, d.valid_inner, d.os, d.is, d.gos,
                     d.gis, d.vocab, items, chunks, d.targets, d.tos, d.tis, d.ignore_index,
                     grad_output, ws);
}

template <typename T>
void scale_launch(bool aligned, const CeRows& d, int64_t rows, const float* grad_output,
                  const CeWork* ws, hipStream_t st) {
  if (aligned) {
    scale_launch_as<T, true>(d, rows, grad_output, ws, st);
  } else {
    scale_launch_as<T, false>(d, rows, grad_output, ws, st);
  }
}

int ce_scale_run(const char* fn, const CeRows& d, int64_t outer, int64_t inner, int64_t vocab,
                 const float* grad_output, const void* workspace, int dtype, void* stream) {
  const std::string name(fn);
  if (!valid_dtype(dtype)) return fail(PT_EINVAL, name + ": unknown dtype");
  if (outer < 0 || inner < 0 || vocab <= 0 || vocab > (int64_t{1} << 30))
    return fail(PT_EINVAL, name + ": bad shape");
  const int64_t rows = outer * inner;
  if (rows == 0) return ok();
  if (!d.logits || (d.valid_inner > 0 && !d.targets) || !grad_output)
    return fail(PT_EINVAL, name + ": null pointer");
  if (dtype == PT_FLOAT16 && (workspace == nullptr || !aligned16(workspace)))
    return fail(PT_EINVAL, name + ": fp16 gradients need the forward's workspace (16-byte aligned)");
  if (dtype == PT_FLOAT16 && d.grad != d.logits &&
      !same_phase(d.logits, d.os, d.is, d.grad, d.gos, d.gis, outer, inner, dtype_size(dtype)))
    return fail(PT_EINVAL, name + ": the logits rows must start in the same 16-byte phase as the "
                                  "gradient rows");
  const CeWork* ws = static_cast<const CeWork*>(workspace);
  hipStream_t st = as_stream(stream);
  const int esize = dtype_size(dtype);
  // all body: every row starts on a 128-byte line and holds whole 16-byte vectors
  const bool aligned = reinterpret_cast<uintptr_t>(d.logits) % kLineBytes == 0 &&
                       (vocab * esize) % 16 == 0 &&
                       (outer <= 1 || (d.os * esize) % kLineBytes == 0) &&
                       (inner <= 1 || (d.is * esize) % kLineBytes == 0);
  if (dtype == PT_FLOAT32) {
    scale_launch<float>(aligned, d, rows, grad_output, ws, st);
  } else if (dtype == PT_FLOAT16) {
    scale_launch<_Float16>(aligned, d, rows, grad_output, ws, st);
  } else {
    scale_launch<__bf16>(aligned, d, rows, grad_output, ws, st);
  }
  return check_launch(fn);
}

}  // namespace
}  // namespace pt

using namespace pt;

extern "C" {

size_t pt_cross_entropy_workspace_bytes(int64_t rows) {
  if (rows < 0) return 0;
  return kHeader + 2 * static_cast<size_t>(rows) * sizeof(float);
}

int32_t* pt_cross_entropy_status(void* workspace) {
  return workspace == nullptr ? nullptr : &static_cast<CeWork*>(workspace)->status;
}

int pt_cross_entropy(void* logits, int64_t outer, int64_t inner, int64_t outer_stride,
                     int64_t inner_stride, int64_t vocab, const int64_t* targets,
                     int64_t t_outer_stride, int64_t t_inner_stride, int64_t ignore_index,
                     float* loss_out, int write_grad, void* grad, int64_t grad_outer_stride,
                     int64_t grad_inner_stride, void* workspace, size_t workspace_bytes,
                     int dtype, void* stream) {
  const int64_t inner_nz = inner > 0 ? inner : 1;
  const bool out = grad != nullptr;
  const CeRows d{logits, inner_nz, inner_nz, outer_stride, inner_stride,
                 static_cast<int>(vocab > 0 && vocab <= (int64_t{1} << 30) ? vocab : 1),
                 targets, t_outer_stride, t_inner_stride, ignore_index,
                 out ? grad : logits, out ? grad_outer_stride : outer_stride,
                 out ? grad_inner_stride : inner_stride};
  return ce_run("pt_cross_entropy", d, outer, inner, vocab, loss_out, write_grad, workspace,
                workspace_bytes, dtype, stream);
}

int pt_cross_entropy_scale_grad(void* dlogits, int64_t outer, int64_t inner,
                                int64_t outer_stride, int64_t inner_stride, int64_t vocab,
                                const int64_t* targets, int64_t t_outer_stride,
                                int64_t t_inner_stride, int64_t ignore_index,
                                const float* grad_output, const void* logits,
                                int64_t logits_outer_stride, int64_t logits_inner_stride,
                                const void* workspace, int dtype, void* stream) {
  const int64_t inner_nz = inner > 0 ? inner : 1;
  const bool out = logits != nullptr && dtype == PT_FLOAT16;
  const CeRows d{dlogits, inner_nz, inner_nz, outer_stride, inner_stride,
                 static_cast<int>(vocab > 0 && vocab <= (int64_t{1} << 30) ? vocab : 1),
                 targets, t_outer_stride, t_inner_stride, ignore_index,
                 out ? const_cast<void*>(logits) : dlogits,
                 out ? logits_outer_stride : outer_stride, out ? logits_inner_stride : inner_stride};
  return ce_scale_run("pt_cross_entropy_scale_grad", d, outer, inner, vocab, grad_output,
                      workspace, dtype, stream);
}

// Rows (b, t) of (batch, seq, vocab) logits; row t < seq - 1 predicts input_ids[b, t + 1], so
// the targets start one position into input_ids and the last position has none.  `grad`
// (strides gbs, gss): where the gradient goes (nullptr: over the logits).
static CeRows shifted_rows(void* logits, int64_t seq, int64_t batch_stride, int64_t seq_stride,
                           int64_t vocab, const int64_t* input_ids, int64_t ids_batch_stride,
                           int64_t ids_seq_stride, int64_t ignore_index, void* grad, int64_t gbs,
                           int64_t gss) {
  const int64_t inner_nz = seq > 0 ? seq : 1;
  const int64_t valid = seq > 1 ? seq - 1 : 0;
  const int64_t* targets = (input_ids != nullptr && valid > 0) ? input_ids + ids_seq_stride : nullptr;
  const bool out = grad != nullptr;
  return CeRows{logits, inner_nz, valid, batch_stride, seq_stride,
                static_cast<int>(vocab > 0 && vocab <= (int64_t{1} << 30) ? vocab : 1),
                targets, ids_batch_stride, ids_seq_stride, ignore_index,
                out ? grad : logits, out ? gbs : batch_stride, out ? gss : seq_stride};
}

int pt_cross_entropy_shifted(void* logits, int64_t batch, int64_t seq, int64_t batch_stride,
                             int64_t seq_stride, int64_t vocab, const int64_t* input_ids,
                             int64_t ids_batch_stride, int64_t ids_seq_stride,
                             int64_t ignore_index, float* loss_out, int write_grad, void* grad,
                             int64_t grad_batch_stride, int64_t grad_seq_stride,
                             void* workspace, size_t workspace_bytes, int dtype, void* stream) {
  const CeRows d = shifted_rows(logits, seq, batch_stride, seq_stride, vocab, input_ids,
                                ids_batch_stride, ids_seq_stride, ignore_index, grad,
                                grad_batch_stride, grad_seq_stride);
  return ce_run("pt_cross_entropy_shifted", d, batch, seq, vocab, loss_out, write_grad,
                workspace, workspace_bytes, dtype, stream);
}

int pt_cross_entropy_shifted_scale_grad(void* dlogits, int64_t batch, int64_t seq,
                                        int64_t batch_stride, int64_t seq_stride, int64_t vocab,
                                        const int64_t* input_ids, int64_t ids_batch_stride,
                                        int64_t ids_seq_stride, int64_t ignore_index,
                                        const float* grad_output, const void* logits,
                                        int64_t logits_batch_stride, int64_t logits_seq_stride,
                                        const void* workspace, int dtype, void* stream) {
  const bool out = logits != nullptr && dtype == PT_FLOAT16;
  const CeRows d = shifted_rows(dlogits, seq, batch_stride, seq_stride, vocab, input_ids,
                                ids_batch_stride, ids_seq_stride, ignore_index,
                                out ? const_cast<void*>(logits) : nullptr, logits_batch_stride,
                                logits_seq_stride);
  return ce_scale_run("pt_cross_entropy_shifted_scale_grad", d, batch, seq, vocab, grad_output,
                      workspace, dtype, stream);
}

}  // extern "C"
