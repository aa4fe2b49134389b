// Shared device and host helpers for the gfx950 kernels of libpicotron_hip.so.
//
// Storage types are fp32, fp16 and bf16; all arithmetic is fp32.  Global memory is
// moved in 16-byte (128-bit) vectors wherever the caller's pointers and strides allow
// it, so one wave64 instruction moves 1 KiB of contiguous data.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "../../include/picotron_hip.h"

namespace pt {

// ------------------------------------------------------------------ host-side errors

// Records `msg` as the calling thread's last error and returns `code`.
int fail(int code, const std::string& msg);
// Clears the calling thread's last error and returns PT_OK.
int ok();
// Checks the last HIP launch; returns PT_OK or PT_ELAUNCH with the HIP message.
int check_launch(const char* what);
// Number of compute units of the current device (cached per device).
int num_cus();
// Resident-workgroup limit for streaming kernels.  A kernel that keeps several 16-byte loads
// in flight per thread moves more bytes per second with fewer workgroups per CU: the DRAM
// then sees fewer interleaved streams.  Measured on MI355X with one-shot grids of 256-thread
// workgroups: 4 fp32 streams read and 3 written, 5873 GB/s at the full 8 workgroups per CU
// against 6419 at 3; 3 read and 2 written, 5963 against 6374 at 2.  A plain copy with one
// load per thread is fastest uncapped.  The limit is a dynamic LDS allocation that the
// kernel never touches.
// Bytes of dynamic LDS that keep at most `per_cu` workgroups (each also holding
// `static_lds` bytes of its own) resident on one CU of the current device; 0 for
// per_cu <= 0 (no limit).
size_t occupancy_lds(int per_cu, size_t static_lds);
// Lets `kernel` launch with `bytes` of dynamic LDS (raises the 64 KB default once per
// kernel and device when needed); returns PT_OK, or PT_ELAUNCH when the runtime refuses
// (callers then launch without the limit: same results, default occupancy).
int allow_dynamic_lds(const void* kernel, size_t bytes);
// A non-negative integer from the environment variable `name`, or `fallback` when it is
// unset or not a number (callers read it once, into a static, for tuning experiments).
int64_t env_int(const char* name, int64_t fallback);
// Fills `count` elements of 4 or 2 bytes at device address `p` with `value` using a kernel
// (not hipMemsetAsync, so the call is safe inside captured graphs).
int fill(void* p, int64_t count, int elem_bytes, unsigned value, hipStream_t st);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int dtype_size(int dtype) { return dtype == PT_FLOAT32 ? 4 : 2; }
inline bool valid_dtype(int dtype) {
  return dtype == PT_FLOAT32 || dtype == PT_FLOAT16 || dtype == PT_BFLOAT16;
}

// ------------------------------------------------------------------ device types

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Storage-type traits.  VEC = elements per 16-byte vector.
template <typename T>
struct Elem;

template <>
struct Elem<float> {
  static constexpr int VEC = 4;
  static __device__ __forceinline__ float to_f32(float v) { return v; }
  static __device__ __forceinline__ float from_f32(float v) { return v; }
};

template <>
struct Elem<_Float16> {
  static constexpr int VEC = 8;
  static __device__ __forceinline__ float to_f32(_Float16 v) { return static_cast<float>(v); }
  // fptrunc is round-to-nearest-even, the same rounding as torch's .to(torch.float16).
  static __device__ __forceinline__ _Float16 from_f32(float v) { return static_cast<_Float16>(v); }
};

template <>
struct Elem<__bf16> {
  static constexpr int VEC = 8;
  static __device__ __forceinline__ float to_f32(__bf16 v) { return static_cast<float>(v); }
  // Lowers to gfx950's v_cvt_pk_bf16_f32: round-to-nearest-even, NaN preserved, the
  // same rounding as torch's .to(torch.bfloat16).
  static __device__ __forceinline__ __bf16 from_f32(float v) { return static_cast<__bf16>(v); }
};

// A 16-byte vector of storage elements, viewed either as raw 32-bit words (for the
// 128-bit global load/store) or as elements.
template <typename T>
union Vec16 {
  u32x4 raw;
  T e[16 / sizeof(T)];
};

// ------------------------------------------------------------------ buffer resources

// Data-format word of a raw (untyped, 32-bit) gfx9-family buffer resource.
constexpr int kBufferWord3 = 0x00020000;
// Cache-policy operand of buffer loads and stores on gfx950: bit 0 sc0, bit 1 nt, bit 4 sc1.
constexpr int kNonTemporal = 2;  // nt: no reuse expected
// nt | sc1: a store performed at device scope, written through the XCD's L2 rather than
// left dirty there for the write-back at the end of the kernel.  A 134 MB copy on MI355X
// (one 16-byte vector per thread, nontemporal loads, one-shot grid) takes 43.2-43.4 us per
// launch with these stores, 44.4-44.7 us with nontemporal write-back stores and 47.1 us with
// plain ones.
constexpr int kWriteThrough = 18;

// A raw buffer resource over `bytes` bytes at `base`, which must be the same in every active
// lane of the wave: it is read from the first active lane, so the resource lives in scalar
// registers and addresses are per-lane byte offsets from it.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t uniform_buffer(const void* base, int bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(a)));
  const uint32_t hi =
      static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(a >> 32)));
  void* b = reinterpret_cast<void*>((static_cast<uint64_t>(hi) << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(b, 0, bytes, kBufferWord3);
}

// Loads 16 bytes from `p` (16-byte aligned).  NT selects a nontemporal access, used
// for data that is touched exactly once (streams far larger than L2 + MALL).
template <bool NT>
__device__ __forceinline__ u32x4 load16(const void* p) {
  const u32x4* q = reinterpret_cast<const u32x4*>(p);
  if constexpr (NT) {
    return __builtin_nontemporal_load(q);
  } else {
    return *q;
  }
}

template <bool NT>
__device__ __forceinline__ void store16(void* p, u32x4 v) {
  u32x4* q = reinterpret_cast<u32x4*>(p);
  if constexpr (NT) {
    __builtin_nontemporal_store(v, q);
  } else {
    *q = v;
  }
}

// Loads VEC consecutive elements of storage type T as fp32.  ALIGNED: one 16-byte load
// (caller guarantees alignment and that all VEC elements are in range); otherwise
// element-wise loads of the first `valid` elements, zero-filling the rest.
template <typename T, bool ALIGNED, bool NT = false>
__device__ __forceinline__ void load_f32(const T* p, float (&out)[Elem<T>::VEC], int valid) {
  constexpr int V = Elem<T>::VEC;
  if constexpr (ALIGNED) {
    Vec16<T> v;
    v.raw = load16<NT>(p);
#pragma unroll
    for (int i = 0; i < V; ++i) out[i] = Elem<T>::to_f32(v.e[i]);
  } else {
#pragma unroll
    for (int i = 0; i < V; ++i) out[i] = (i < valid) ? Elem<T>::to_f32(p[i]) : 0.0f;
  }
}

template <typename T, bool ALIGNED, bool NT = false>
__device__ __forceinline__ void store_f32(T* p, const float (&in)[Elem<T>::VEC], int valid) {
  constexpr int V = Elem<T>::VEC;
  if constexpr (ALIGNED) {
    Vec16<T> v;
#pragma unroll
    for (int i = 0; i < V; ++i) v.e[i] = Elem<T>::from_f32(in[i]);
    store16<NT>(p, v.raw);
  } else {
#pragma unroll
    for (int i = 0; i < V; ++i)
      if (i < valid) p[i] = Elem<T>::from_f32(in[i]);
  }
}

// Loads one element of a runtime-typed array as fp32 (weights: tiny, cache-resident).
__device__ __forceinline__ float load_any(const void* p, int64_t i, int dtype) {
  if (dtype == PT_FLOAT32) return reinterpret_cast<const float*>(p)[i];
  if (dtype == PT_BFLOAT16) return static_cast<float>(reinterpret_cast<const __bf16*>(p)[i]);
  return static_cast<float>(reinterpret_cast<const _Float16*>(p)[i]);
}

__device__ __forceinline__ void store_any(void* p, int64_t i, int dtype, float v) {
  if (dtype == PT_FLOAT32) {
    reinterpret_cast<float*>(p)[i] = v;
  } else if (dtype == PT_BFLOAT16) {
    reinterpret_cast<__bf16*>(p)[i] = static_cast<__bf16>(v);
  } else {
    reinterpret_cast<_Float16*>(p)[i] = static_cast<_Float16>(v);
  }
}

// Device memory reached through an address held as an integer (a record table) in the
// global address space, so that the compiler emits global_* accesses: through a generic
// pointer it would emit flat_* accesses, which also count against the LDS wait counter.
template <typename T>
using gptr = T __attribute__((address_space(1)))*;

template <typename T>
__device__ __forceinline__ gptr<T> as_global(int64_t addr) {
  return reinterpret_cast<gptr<T>>(addr);
}

// ------------------------------------------------------------------ reductions

// Wave reductions on DPP lane moves (register-to-register, a few cycles each) instead of
// LDS permutes: two quad swaps, a half-row and a row mirror leave every lane of each
// 16-lane row holding that row's result (bitwise equal in all of its lanes, since each
// step combines the same two values in either order); the four row results are then read
// into scalars and combined in row order, so every lane receives the same total.  All 64
// lanes must be active.
namespace dpp {
constexpr int kQuadSwap1 = 0xb1;     // quad_perm [1, 0, 3, 2]
constexpr int kQuadSwap2 = 0x4e;     // quad_perm [2, 3, 0, 1]
constexpr int kRowHalfMirror = 0x141;
constexpr int kRowMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ float move(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

__device__ __forceinline__ float lane(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
}  // namespace dpp

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp::move<dpp::kQuadSwap1>(v);
  v += dpp::move<dpp::kQuadSwap2>(v);
  v += dpp::move<dpp::kRowHalfMirror>(v);
  v += dpp::move<dpp::kRowMirror>(v);
  return ((dpp::lane(v, 0) + dpp::lane(v, 16)) + dpp::lane(v, 32)) + dpp::lane(v, 48);
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp::move<dpp::kQuadSwap1>(v));
  v = fmaxf(v, dpp::move<dpp::kQuadSwap2>(v));
  v = fmaxf(v, dpp::move<dpp::kRowHalfMirror>(v));
  v = fmaxf(v, dpp::move<dpp::kRowMirror>(v));
  return fmaxf(fmaxf(dpp::lane(v, 0), dpp::lane(v, 16)), fmaxf(dpp::lane(v, 32), dpp::lane(v, 48)));
}

constexpr int kWave = 64;

}  // namespace pt
