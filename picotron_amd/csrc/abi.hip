// Library-wide C ABI: version, per-thread error message, device gate, and the
// 128-bit streaming copy used as the achievable-bandwidth reference.
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <map>
#include <string>
#include <utility>

#include "pt_common.hpp"

namespace pt {

namespace {
thread_local std::string g_last_error;

constexpr int kMaxDevices = 64;
int g_cus[kMaxDevices];
std::once_flag g_cus_once[kMaxDevices];
size_t g_lds[kMaxDevices];
std::once_flag g_lds_once[kMaxDevices];
std::mutex g_lds_mutex;
std::map<std::pair<int, const void*>, size_t> g_lds_raised;  // (device, kernel) -> bytes allowed

int current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return -1;
  return dev;
}

size_t lds_per_cu() {
  const int dev = current_device();
  if (dev < 0) return 163840;
  std::call_once(g_lds_once[dev], [dev] {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) !=
            hipSuccess ||
        n <= 0) {
      n = 163840;
    }
    g_lds[dev] = static_cast<size_t>(n);
  });
  return g_lds[dev];
}
}  // namespace

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int ok() {
  g_last_error.clear();
  return PT_OK;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return fail(PT_ELAUNCH, std::string(what) + ": " + hipGetErrorString(e));
  }
  return ok();
}

int num_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  std::call_once(g_cus_once[dev], [dev] {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0) {
      n = 256;
    }
    g_cus[dev] = n;
  });
  return g_cus[dev];
}

size_t occupancy_lds(int per_cu, size_t static_lds) {
  if (per_cu <= 0) return 0;
  // Each workgroup takes a 1/per_cu share of the CU's LDS, less a margin that keeps the
  // share above 1/(per_cu + 1) of it (true for per_cu <= 12), so exactly per_cu fit.
  // Larger per_cu values leave little or no share: the limit then fades to none.
  const int64_t share = static_cast<int64_t>(lds_per_cu() / static_cast<size_t>(per_cu)) - 1024 -
                        static_cast<int64_t>(static_lds);
  return share > 0 ? static_cast<size_t>(share) : 0;
}

int allow_dynamic_lds(const void* kernel, size_t bytes) {
  if (bytes <= 65536) return PT_OK;
  const int dev = current_device();
  std::lock_guard<std::mutex> lock(g_lds_mutex);
  size_t& allowed = g_lds_raised[{dev, kernel}];
  if (allowed >= bytes) return PT_OK;
  const hipError_t e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           static_cast<int>(bytes));
  if (e != hipSuccess) {
    (void)hipGetLastError();  // a refused attribute must not surface as the next launch's error
    return fail(PT_ELAUNCH, std::string("dynamic LDS limit: ") + hipGetErrorString(e));
  }
  allowed = bytes;
  return PT_OK;
}

int64_t env_int(const char* name, int64_t fallback) {
  const char* v = std::getenv(name);
  if (v == nullptr || *v == '\0') return fallback;
  char* end = nullptr;
  const long long x = std::strtoll(v, &end, 10);
  return (end != v && x >= 0) ? static_cast<int64_t>(x) : fallback;
}

// 16-byte nontemporal copy.  One-shot grid: thread t of block b moves vector b*256 + t, so
// every vector has its own thread and the grid drains once (measured on MI355X over 1 GiB:
// 6.46 TB/s, against 5.99 TB/s for a grid-stride loop over 32 workgroups per CU with four
// vectors in flight per thread).  `base` offsets the grid for copies of more vectors than
// one launch's work-item count can address.
__global__ __launch_bounds__(256) void copy16_kernel(const u32x4* __restrict__ src,
                                                     u32x4* __restrict__ dst, int64_t base,
                                                     int64_t nvec) {
  const int64_t i = base + static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < nvec) __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

__global__ __launch_bounds__(256) void fill_u32_kernel(unsigned* __restrict__ p, int64_t n,
                                                        unsigned value) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    p[i] = value;
  }
}

__global__ __launch_bounds__(256) void fill_u16_kernel(unsigned short* __restrict__ p, int64_t n,
                                                        unsigned short value) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    p[i] = value;
  }
}

int fill(void* p, int64_t count, int elem_bytes, unsigned value, hipStream_t st) {
  if (count <= 0) return PT_OK;
  int64_t blocks = (count + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  if (elem_bytes == 4) {
    hipLaunchKernelGGL(fill_u32_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st,
                       static_cast<unsigned*>(p), count, value);
  } else {
    hipLaunchKernelGGL(fill_u16_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st,
                       static_cast<unsigned short*>(p), count, static_cast<unsigned short>(value));
  }
  return check_launch("fill");
}

}  // namespace pt

extern "C" {

int pt_abi_version(void) { return PT_ABI_VERSION; }

const char* pt_last_error(void) { return pt::g_last_error.c_str(); }

int pt_device_supported(int device) {
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) return 0;
  return std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

int pt_copy(const void* src, void* dst, int64_t bytes, void* stream) {
  if (src == nullptr || dst == nullptr) return pt::fail(PT_EINVAL, "pt_copy: null pointer");
  if (bytes < 0 || (bytes & 15) != 0)
    return pt::fail(PT_EINVAL, "pt_copy: bytes must be a non-negative multiple of 16");
  if (!pt::aligned16(src) || !pt::aligned16(dst))
    return pt::fail(PT_EINVAL, "pt_copy: pointers must be 16-byte aligned");
  if (bytes == 0) return pt::ok();
  const int64_t nvec = bytes / 16;
  // A launch addresses fewer than 2^32 work-items: 2^23 workgroups (2^31 vectors, 32 GiB)
  // per launch.
  constexpr int64_t kChunk = int64_t{1} << 31;
  for (int64_t base = 0; base < nvec; base += kChunk) {
    const int64_t n = nvec - base < kChunk ? nvec - base : kChunk;
    hipLaunchKernelGGL(pt::copy16_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256),
                       0, pt::as_stream(stream), reinterpret_cast<const pt::u32x4*>(src),
                       reinterpret_cast<pt::u32x4*>(dst), base, nvec);
    if (int rc = pt::check_launch("pt_copy")) return rc;
  }
  return pt::check_launch("pt_copy");
}

}  // extern "C"
