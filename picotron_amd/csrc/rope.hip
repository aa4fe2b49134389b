// Rotary position embedding (forward and its inverse, the backward) for gfx950.
//
// Reference semantics (AndyMLAndAI/picotron):
//   tables   src/picotron/nn/rope.py:13-32    angle[s, i] = s * theta^(-2i/D); cos/sin
//   rotation src/picotron/nn/rope.py:35-51    interleaved pairs (2i, 2i+1):
//            (a, b) -> (a*c - b*s, a*s + b*c)
//   Triton   src/picotron/nn/triton_kernels/rope.py:25-49 (same pairs, forward only)
// The rotate-half layout pairs (i, i + D/2) with the same angle table.  The inverse
// rotation (a, b) -> (a*c + b*s, -a*s + b*c) is the exact transpose of the forward, so it
// is the backward of the forward.
//
// Work item = one 16-byte vector of a row (interleaved: V/2 pairs) or one vector from each
// half of a row (rotate-half: V pairs).  Rows are the (batch, head, seq) positions of a
// strided view whose head_dim is contiguous; the host orders the three row dimensions by
// decreasing stride so consecutive work items walk memory in address order.  Query and key
// are handled by one launch (blocks [0, nb0) and [nb0, nb0 + nb1)).
#include "pt_common.hpp"

namespace pt {
namespace {

// Work items per row: interleaved rows split into V-element vectors (V/2 pairs each, or one
// pair on the element path); rotate-half rows into P-pair groups taken from both halves.
template <typename T, int LAYOUT, bool ALIGNED>
__host__ __device__ constexpr int items_per_row(int head_dim) {
  return LAYOUT == 0 ? head_dim / (ALIGNED ? Elem<T>::VEC : 2)
                     : (head_dim / 2) / (ALIGNED ? Elem<T>::VEC : 1);
}

struct RopeTensor {
  const void* x;
  void* y;
  int64_t n[3];    // row dimensions, outer to inner (iteration order)
  int64_t xs[3];   // x strides of those dimensions (elements)
  int64_t ys[3];   // y strides
  int seq_dim;     // which of the three is the sequence dimension
  int64_t rows;    // n[0] * n[1] * n[2]
  int64_t items;   // rows * items_per_row
  int64_t blocks;  // blocks assigned to this tensor
  int64_t ybytes;  // bytes from y to the end of its last row
};

// One work item in two phases, so that a thread can have several items' loads in flight
// before it computes and stores any of them (the output may alias the input, so the
// compiler would not move a later item's loads above an earlier item's stores).  The pair
// members are held as a[p] (first) and b[p] (second): interleaved rows pair elements
// (2i, 2i+1) of one vector, rotate-half rows pair element i of the first half with element
// i of the second.  Item, row and the three row indices fit in 32 bits (pt_rope bounds
// items by 2^32), so they are decoded with 32-bit divisions; only memory offsets are 64-bit.
// WT (aligned rows only): stores through a buffer resource over y with the write-through
// policy instead of nontemporal global stores.
template <typename T, int LAYOUT, bool ALIGNED, bool NT, bool WT>
struct RopeWork {
  static constexpr int V = ALIGNED ? Elem<T>::VEC : 2;
  static constexpr int P = LAYOUT == 0 ? V / 2 : (ALIGNED ? Elem<T>::VEC : 1);  // pairs
  // Raw storage until store(): converting in load() would wait for the data there.
  Vec16<T> va, vb;  // aligned: interleaved vector (va) or the two half vectors (va, vb)
  T ea[2], eb[2];   // element path: interleaved (ea[0], ea[1]) or rotate-half (ea[0], eb[0])
  float c[P], s[P];
  T* ya;  // first members (interleaved: the whole vector)
  T* yb;  // second members (rotate-half)

  __device__ __forceinline__ void load(const RopeTensor& t, uint32_t item, int head_dim,
                                       const float* __restrict__ cos_t,
                                       const float* __restrict__ sin_t) {
    const int half = head_dim / 2;
    const uint32_t per_row = static_cast<uint32_t>(items_per_row<T, LAYOUT, ALIGNED>(head_dim));
    const uint32_t row = item / per_row;
    const int j = static_cast<int>(item - row * per_row);
    const uint32_t n2 = static_cast<uint32_t>(t.n[2]), n1 = static_cast<uint32_t>(t.n[1]);
    int64_t idx[3];
    const uint32_t r1 = row / n2;
    idx[2] = row - r1 * n2;
    idx[0] = r1 / n1;
    idx[1] = r1 - static_cast<uint32_t>(idx[0]) * n1;
    const int64_t xo = idx[0] * t.xs[0] + idx[1] * t.xs[1] + idx[2] * t.xs[2];
    const int64_t yo = idx[0] * t.ys[0] + idx[1] * t.ys[1] + idx[2] * t.ys[2];
    const int64_t pos = idx[t.seq_dim];
    const T* xr = static_cast<const T*>(t.x) + xo;
    T* yr = static_cast<T*>(t.y) + yo;
    const int i0 = j * P;  // first pair of the item
    if constexpr (LAYOUT == 0) {
      if constexpr (ALIGNED) {
        va.raw = load16<NT>(xr + j * V);
      } else {
        ea[0] = xr[2 * j];
        ea[1] = xr[2 * j + 1];
      }
      ya = yr + j * V;
      yb = ya;
    } else {
      if constexpr (ALIGNED) {
        va.raw = load16<NT>(xr + i0);
        vb.raw = load16<NT>(xr + half + i0);
      } else {
        ea[0] = xr[j];
        eb[0] = xr[half + j];
      }
      ya = yr + i0;
      yb = yr + half + i0;
    }
    const float* cr = cos_t + pos * half + i0;
    const float* sr = sin_t + pos * half + i0;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      c[p] = cr[p];
      s[p] = sr[p];
    }
  }

  template <int N>
  __device__ __forceinline__ static void put(__amdgpu_buffer_rsrc_t buf, const T* ybase, T* p,
                                             const float (&o)[N]) {
    Vec16<T> v;
#pragma unroll
    for (int i = 0; i < N; ++i) v.e[i] = Elem<T>::from_f32(o[i]);
    const uint32_t off = static_cast<uint32_t>(reinterpret_cast<const char*>(p) -
                                               reinterpret_cast<const char*>(ybase));
    __builtin_amdgcn_raw_buffer_store_b128(v.raw, buf, off, 0, kWriteThrough);
  }

  __device__ __forceinline__ void store(float sign, __amdgpu_buffer_rsrc_t buf,
                                        const T* ybase) const {
    float a[P], b[P];
    if constexpr (LAYOUT == 0) {
#pragma unroll
      for (int p = 0; p < P; ++p) {
        a[p] = Elem<T>::to_f32(ALIGNED ? va.e[2 * p] : ea[2 * p]);
        b[p] = Elem<T>::to_f32(ALIGNED ? va.e[2 * p + 1] : ea[2 * p + 1]);
      }
    } else {
#pragma unroll
      for (int p = 0; p < P; ++p) {
        a[p] = Elem<T>::to_f32(ALIGNED ? va.e[p] : ea[p]);
        b[p] = Elem<T>::to_f32(ALIGNED ? vb.e[p] : eb[p]);
      }
    }
    float oa[P], ob[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const float sn = sign * s[p];
      oa[p] = a[p] * c[p] - b[p] * sn;
      ob[p] = a[p] * sn + b[p] * c[p];
    }
    if constexpr (LAYOUT == 0) {
      float o[V];
#pragma unroll
      for (int p = 0; p < P; ++p) {
        o[2 * p] = oa[p];
        o[2 * p + 1] = ob[p];
      }
      if constexpr (ALIGNED && WT) {
        put(buf, ybase, ya, o);
      } else if constexpr (ALIGNED) {
        store_f32<T, true, NT>(ya, o, V);
      } else {
        ya[0] = Elem<T>::from_f32(o[0]);
        ya[1] = Elem<T>::from_f32(o[1]);
      }
    } else {
      if constexpr (ALIGNED && WT) {
        put(buf, ybase, ya, oa);
        put(buf, ybase, yb, ob);
      } else if constexpr (ALIGNED) {
        store_f32<T, true, NT>(ya, oa, P);
        store_f32<T, true, NT>(yb, ob, P);
      } else {
        ya[0] = Elem<T>::from_f32(oa[0]);
        yb[0] = Elem<T>::from_f32(ob[0]);
      }
    }
  }
};

// A block covers 256 * kItemsPerThread items of one tensor: thread t takes items
// base + t + 256 * u, all loaded before any is stored.  One item per thread measured best
// on q [8, 2048, 32, 128] + k [8, 2048, 8, 128] bf16 (54.1 us; two 55.8, four 57.5): more
// waves beat more loads per wave.
constexpr int kItemsPerThread = 1;

template <typename T, int LAYOUT, bool ALIGNED, bool NT, bool WT>
__global__ __launch_bounds__(256) void rope_kernel(RopeTensor t0, RopeTensor t1, int head_dim,
                                                   const float* __restrict__ cos_t,
                                                   const float* __restrict__ sin_t, float sign) {
  uint32_t b = blockIdx.x;
  const RopeTensor* t = &t0;
  if (b >= t0.blocks) {
    b -= static_cast<uint32_t>(t0.blocks);
    t = &t1;
  }
  const uint32_t base = b * (256u * kItemsPerThread) + threadIdx.x;
  const uint32_t items = static_cast<uint32_t>(t->items);
  RopeWork<T, LAYOUT, ALIGNED, NT, WT> w[kItemsPerThread];
#pragma unroll
  for (int u = 0; u < kItemsPerThread; ++u) {
    const uint32_t item = base + 256u * u;
    if (item < items) w[u].load(*t, item, head_dim, cos_t, sin_t);
  }
  // y's span fits a buffer resource whenever WT is set (checked on the host); unused otherwise
  const auto ybuf = uniform_buffer(t->y, WT ? static_cast<int>(t->ybytes) : 0);
#pragma unroll
  for (int u = 0; u < kItemsPerThread; ++u)
    if (base + 256u * u < items) w[u].store(sign, ybuf, static_cast<const T*>(t->y));
}

bool parse(const void* x, void* y, const int64_t* d, int64_t head_dim, int64_t table_rows,
           int esize, int layout, RopeTensor* t, bool* aligned, std::string* err) {
  const int64_t sz[3] = {d[0], d[1], d[2]};  // batch, heads, seq
  const int64_t xs[3] = {d[3], d[4], d[5]};
  const int64_t ys[3] = {d[6], d[7], d[8]};
  for (int i = 0; i < 3; ++i) {
    if (sz[i] < 0) {
      *err = "negative dimension";
      return false;
    }
  }
  if (sz[2] > table_rows) {
    *err = "sequence length exceeds the cos/sin table rows";
    return false;
  }
  // iteration order: dimensions by decreasing x stride (stable), so the innermost
  // iterated dimension has the smallest stride.
  int ord[3] = {0, 1, 2};
  for (int a = 0; a < 3; ++a)
    for (int b = a + 1; b < 3; ++b)
      if (xs[ord[b]] > xs[ord[a]]) {
        const int tmp = ord[a];
        ord[a] = ord[b];
        ord[b] = tmp;
      }
  t->x = x;
  t->y = y;
  for (int i = 0; i < 3; ++i) {
    t->n[i] = sz[ord[i]];
    t->xs[i] = xs[ord[i]];
    t->ys[i] = ys[ord[i]];
    if (ord[i] == 2) t->seq_dim = i;
  }
  t->rows = sz[0] * sz[1] * sz[2];
  // y's extent in bytes (-1 when a stride is negative): the write-through stores address y
  // through a buffer resource, so they need it to fit 31 bits
  int64_t last = head_dim;
  for (int i = 0; i < 3; ++i) {
    if (sz[i] > 1 && ys[i] < 0) last = -1;
    if (last >= 0 && sz[i] > 1) last += (sz[i] - 1) * ys[i];
  }
  t->ybytes = last < 0 ? -1 : last * esize;
  // 16-byte vectors need aligned bases, strides that keep every row aligned, and
  // (rotate-half) a half that is a whole number of vectors.
  const int vec = 16 / esize;
  bool al = aligned16(x) && aligned16(y) && head_dim % (2 * vec) == 0;
  for (int i = 0; i < 3; ++i) {
    if (sz[i] > 1 && ((xs[i] * esize) % 16 != 0 || (ys[i] * esize) % 16 != 0)) al = false;
  }
  if (layout == 0 && head_dim % vec != 0) al = false;
  *aligned = al;
  return true;
}

constexpr int64_t kNontemporalBytes = int64_t{64} << 20;

// Resident workgroups per CU; PT_ROPE_OCCUPANCY overrides it (0: no limit).  One item
// per thread keeps little in flight, so the limit stays high: at 6 the 4-layer q + k
// benchmark measured 54.3-54.5 us per launch against 54.7 with the full 8, and 60.5-66.1
// at 4 and 3.
int rope_occupancy() {
  static const int v = static_cast<int>(env_int("PT_ROPE_OCCUPANCY", 6));
  return v;
}

template <typename K>
void launch_limited(K kernel, unsigned grid, hipStream_t st, const RopeTensor& t0,
                    const RopeTensor& t1, int head_dim, const float* c, const float* s,
                    float sign) {
  size_t lds = occupancy_lds(rope_occupancy(), 0);
  if (allow_dynamic_lds(reinterpret_cast<const void*>(kernel), lds) != PT_OK) lds = 0;
  hipLaunchKernelGGL(kernel, dim3(grid), dim3(256), lds, st, t0, t1, head_dim, c, s, sign);
}

template <typename T, int LAYOUT, bool ALIGNED>
void launch(RopeTensor& t0, RopeTensor& t1, int head_dim, const float* c, const float* s,
            float sign, hipStream_t st) {
  const int per_row = items_per_row<T, LAYOUT, ALIGNED>(head_dim);
  t0.items = t0.rows * per_row;
  t1.items = t1.rows * per_row;
  constexpr int64_t kPerBlock = 256 * kItemsPerThread;
  t0.blocks = (t0.items + kPerBlock - 1) / kPerBlock;
  t1.blocks = (t1.items + kPerBlock - 1) / kPerBlock;
  const int64_t blocks = t0.blocks + t1.blocks;
  if (blocks == 0) return;
  // pt_rope has checked that (rows0 + rows1) * head_dim / 2 + 512 < 2^32, which bounds
  // blocks * 256 for every layout.  Streams larger than the caches are touched once:
  // nontemporal loads and stores.
  // Aligned streams whose outputs fit a buffer resource store through it with the
  // write-through policy: the q + k benchmark (4 layers, rotate-half bf16) measured 419.7
  // against 424.6 us per step with nontemporal global stores, the same bits.
  const int64_t bytes = (t0.rows + t1.rows) * head_dim * static_cast<int64_t>(sizeof(T));
  const auto fits = [](const RopeTensor& t) {
    return t.rows == 0 || (t.ybytes > 0 && t.ybytes <= 0x7fffffff);
  };
  if (bytes > kNontemporalBytes) {
    if (ALIGNED && fits(t0) && fits(t1)) {
      launch_limited(rope_kernel<T, LAYOUT, ALIGNED, true, ALIGNED>, static_cast<unsigned>(blocks),
                     st, t0, t1, head_dim, c, s, sign);
    } else {
      launch_limited(rope_kernel<T, LAYOUT, ALIGNED, true, false>, static_cast<unsigned>(blocks),
                     st, t0, t1, head_dim, c, s, sign);
    }
  } else {
    launch_limited(rope_kernel<T, LAYOUT, ALIGNED, false, false>, static_cast<unsigned>(blocks),
                   st, t0, t1, head_dim, c, s, sign);
  }
}

template <typename T>
void launch_t(int layout, bool aligned, RopeTensor& t0, RopeTensor& t1, int head_dim,
              const float* c, const float* s, float sign, hipStream_t st) {
  if (layout == 0) {
    if (aligned) {
      launch<T, 0, true>(t0, t1, head_dim, c, s, sign, st);
    } else {
      launch<T, 0, false>(t0, t1, head_dim, c, s, sign, st);
    }
  } else {
    if (aligned) {
      launch<T, 1, true>(t0, t1, head_dim, c, s, sign, st);
    } else {
      launch<T, 1, false>(t0, t1, head_dim, c, s, sign, st);
    }
  }
}

}  // namespace
}  // namespace pt

using namespace pt;

extern "C" {

int pt_rope(const void* x0, void* y0, const int64_t* desc0, const void* x1, void* y1,
            const int64_t* desc1, int64_t head_dim, const float* cos_table,
            const float* sin_table, int64_t table_rows, int layout, int inverse, int dtype,
            void* stream) {
  if (!valid_dtype(dtype)) return fail(PT_EINVAL, "pt_rope: unknown dtype code");
  if (layout != 0 && layout != 1) return fail(PT_EINVAL, "pt_rope: layout must be 0 or 1");
  if (head_dim <= 0 || head_dim % 2 != 0 || head_dim > (1 << 20))
    return fail(PT_EINVAL, "pt_rope: head_dim must be a positive even number");
  if (!cos_table || !sin_table) return fail(PT_EINVAL, "pt_rope: null cos/sin table");
  if (!desc0) return fail(PT_EINVAL, "pt_rope: null first tensor descriptor");
  if ((x1 == nullptr) != (y1 == nullptr) || (x1 != nullptr && desc1 == nullptr))
    return fail(PT_EINVAL, "pt_rope: second tensor needs x, y and desc");
  const int esize = dtype_size(dtype);
  RopeTensor t0{}, t1{};
  bool al0 = true, al1 = true;
  std::string err;
  if (!parse(x0, y0, desc0, head_dim, table_rows, esize, layout, &t0, &al0, &err))
    return fail(PT_EINVAL, "pt_rope: first tensor: " + err);
  if (x1 != nullptr) {
    if (!parse(x1, y1, desc1, head_dim, table_rows, esize, layout, &t1, &al1, &err))
      return fail(PT_EINVAL, "pt_rope: second tensor: " + err);
  } else {
    t1.n[0] = t1.n[1] = t1.n[2] = 1;
    t1.rows = 0;
  }
  // Empty tensors may carry null data pointers; non-empty ones may not.
  if (t0.rows > 0 && (!x0 || !y0)) return fail(PT_EINVAL, "pt_rope: null first tensor");
  const bool aligned = al0 && al1;
  if ((t0.rows + t1.rows) * (head_dim / 2) + 512 > 0xffffffffLL)
    return fail(PT_EUNSUPPORTED, "pt_rope: too many rows for one launch");
  const float sign = inverse ? -1.0f : 1.0f;
  hipStream_t st = as_stream(stream);
  const int hd = static_cast<int>(head_dim);
  if (dtype == PT_FLOAT32) {
    launch_t<float>(layout, aligned, t0, t1, hd, cos_table, sin_table, sign, st);
  } else if (dtype == PT_FLOAT16) {
    launch_t<_Float16>(layout, aligned, t0, t1, hd, cos_table, sin_table, sign, st);
  } else {
    launch_t<__bf16>(layout, aligned, t0, t1, hd, cos_table, sin_table, sign, st);
  }
  return check_launch("pt_rope");
}

}  // extern "C"
