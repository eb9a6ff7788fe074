// Jagged <-> padded-dense kernels for gfx950.
//
// Semantics follow fbgemm_gpu's jagged_to_padded_dense_forward,
// dense_to_jagged_forward, jagged_dense_elementwise_add_jagged_output and
// jagged_dense_elementwise_mul (upstream src/jagged_tensor_ops/, recalled;
// outside the dense the add gives x + 0 and the mul x * 0), restated from torch's own
// port of the same ops: torch/_inductor/jagged_lowerings.py:161-177 (masked
// load, else padding value) and :231-249 (jagged rows past max length become
// 0).
//
// Design: the ops are pure HBM streams.  One work item moves VEC bytes
// (16 when the row size and pointers allow it), consecutive work items walk
// a row, so every wave issues fully coalesced 1 KiB transactions.  With one
// jagged dim (the common case) a bag is a contiguous copy: one block row per
// bag, no per-item index arithmetic.  With more, the jagged coordinate of a
// dense row is found by walking the offsets levels (dense -> jagged) or by a
// binary search per level (jagged -> dense); the offsets are a few KB and
// stay in L2.
#include "mx_common.h"

namespace mx {
namespace {

struct JaggedMeta {
  const void* off[MX_MAX_JAGGED_DIM];
  int64_t off_len[MX_MAX_JAGGED_DIM];  // entries in each offsets array
  int64_t max_len[MX_MAX_JAGGED_DIM];
  int32_t ndim;
};

template <int VEC>
struct alignas(VEC) Chunk {
  uint8_t b[VEC];
};

template <typename I>
__device__ __forceinline__ int64_t off_at(const JaggedMeta& m, int k, int64_t i) {
  return static_cast<int64_t>(reinterpret_cast<const I*>(m.off[k])[i]);
}

// Dense row r (over B * prod(max_len)) -> jagged values row, or -1 for padding.
template <typename I>
__device__ int64_t dense_to_values_row(int64_t r, const JaggedMeta& m) {
  int64_t coord[MX_MAX_JAGGED_DIM];
  for (int k = m.ndim - 1; k >= 0; --k) {
    coord[k] = r % m.max_len[k];
    r /= m.max_len[k];
  }
  int64_t idx = r;  // b
  for (int k = 0; k < m.ndim; ++k) {
    const int64_t begin = off_at<I>(m, k, idx);
    const int64_t end = off_at<I>(m, k, idx + 1);
    if (coord[k] >= end - begin) return -1;
    idx = begin + coord[k];
  }
  return idx;
}

// Last p in [0, n-1) with off[p] <= x, or -1 when x is past the last offset.
template <typename I>
__device__ int64_t owner_of(const JaggedMeta& m, int k, int64_t x) {
  const int64_t n = m.off_len[k];
  if (n < 2 || x < off_at<I>(m, k, 0) || x >= off_at<I>(m, k, n - 1)) return -1;
  int64_t lo = 0, hi = n - 1;  // off[lo] <= x < off[hi]
  while (hi - lo > 1) {
    const int64_t mid = lo + ((hi - lo) >> 1);
    if (off_at<I>(m, k, mid) <= x)
      lo = mid;
    else
      hi = mid;
  }
  return lo;
}

// Jagged values row i -> dense row, or -1 if it has no dense position.
template <typename I>
__device__ int64_t values_to_dense_row(int64_t i, const JaggedMeta& m) {
  int64_t coord[MX_MAX_JAGGED_DIM];
  int64_t idx = i;
  bool inside = true;
  for (int k = m.ndim - 1; k >= 0; --k) {
    const int64_t p = owner_of<I>(m, k, idx);
    if (p < 0) return -1;
    coord[k] = idx - off_at<I>(m, k, p);
    if (coord[k] >= m.max_len[k]) inside = false;
    idx = p;
  }
  if (!inside) return -1;
  int64_t r = idx;
  for (int k = 0; k < m.ndim; ++k) r = r * m.max_len[k] + coord[k];
  return r;
}

template <int VEC, typename I>
__global__ void __launch_bounds__(256) j2pd_kernel(const uint8_t* __restrict__ values,
                                                   uint8_t* __restrict__ out, JaggedMeta m,
                                                   int64_t rows, int64_t vpr, Chunk<VEC> pad) {
  const int64_t total = rows * vpr;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t w = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; w < total;
       w += stride) {
    const int64_t r = w / vpr;
    const int64_t v = w - r * vpr;
    const int64_t src = dense_to_values_row<I>(r, m);
    Chunk<VEC> c = pad;
    if (src >= 0) c = reinterpret_cast<const Chunk<VEC>*>(values)[src * vpr + v];
    reinterpret_cast<Chunk<VEC>*>(out)[w] = c;
  }
}

template <int VEC, typename I>
__global__ void __launch_bounds__(256) d2j_kernel(const uint8_t* __restrict__ dense,
                                                  uint8_t* __restrict__ out, JaggedMeta m,
                                                  int64_t total_L, int64_t vpr) {
  const int64_t total = total_L * vpr;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t w = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; w < total;
       w += stride) {
    const int64_t i = w / vpr;
    const int64_t v = w - i * vpr;
    const int64_t dr = values_to_dense_row<I>(i, m);
    Chunk<VEC> c;
#pragma unroll
    for (int e = 0; e < VEC; ++e) c.b[e] = 0;
    if (dr >= 0) c = reinterpret_cast<const Chunk<VEC>*>(dense)[dr * vpr + v];
    reinterpret_cast<Chunk<VEC>*>(out)[w] = c;
  }
}

// ---- element arithmetic for the jagged + dense add ------------------------

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}
// Round to nearest even, NaN kept quiet (same rule as c10::BFloat16).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// x (op) y per element in the element type's arithmetic: f32/f64 natively,
// f16/bf16 computed in fp32 (sums and products of two such values are then
// rounded once to the element type, to nearest even).
template <int DT, bool MUL>
struct BinOp;

template <bool MUL>
struct BinOp<MX_DTYPE_F32, MUL> {
  static constexpr int kBytes = 4;
  __device__ static void apply(const uint8_t* x, const uint8_t* y, uint8_t* o) {
    const float a = *reinterpret_cast<const float*>(x), b = *reinterpret_cast<const float*>(y);
    *reinterpret_cast<float*>(o) = MUL ? a * b : a + b;
  }
};
template <bool MUL>
struct BinOp<MX_DTYPE_F64, MUL> {
  static constexpr int kBytes = 8;
  __device__ static void apply(const uint8_t* x, const uint8_t* y, uint8_t* o) {
    const double a = *reinterpret_cast<const double*>(x), b = *reinterpret_cast<const double*>(y);
    *reinterpret_cast<double*>(o) = MUL ? a * b : a + b;
  }
};
template <bool MUL>
struct BinOp<MX_DTYPE_F16, MUL> {
  static constexpr int kBytes = 2;
  __device__ static void apply(const uint8_t* x, const uint8_t* y, uint8_t* o) {
    const float a = __half2float(*reinterpret_cast<const __half*>(x));
    const float b = __half2float(*reinterpret_cast<const __half*>(y));
    *reinterpret_cast<__half*>(o) = __float2half_rn(MUL ? a * b : a + b);
  }
};
template <bool MUL>
struct BinOp<MX_DTYPE_BF16, MUL> {
  static constexpr int kBytes = 2;
  __device__ static void apply(const uint8_t* x, const uint8_t* y, uint8_t* o) {
    const float a = bf16_to_f32(*reinterpret_cast<const uint16_t*>(x));
    const float b = bf16_to_f32(*reinterpret_cast<const uint16_t*>(y));
    *reinterpret_cast<uint16_t*>(o) = f32_to_bf16(MUL ? a * b : a + b);
  }
};

template <int VEC, typename I, int DT, bool MUL>
__global__ void __launch_bounds__(256) jagged_add_kernel(const uint8_t* __restrict__ x,
                                                         const uint8_t* __restrict__ y,
                                                         uint8_t* __restrict__ out, JaggedMeta m,
                                                         int64_t total_L, int64_t vpr) {
  using Op = BinOp<DT, MUL>;
  const int64_t total = total_L * vpr;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t w = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; w < total;
       w += stride) {
    const int64_t i = w / vpr;
    const int64_t v = w - i * vpr;
    const int64_t dr = values_to_dense_row<I>(i, m);
    const Chunk<VEC> cx = reinterpret_cast<const Chunk<VEC>*>(x)[w];
    Chunk<VEC> cy;
#pragma unroll
    for (int e = 0; e < VEC; ++e) cy.b[e] = 0;  // +0 in every element type
    if (dr >= 0) cy = reinterpret_cast<const Chunk<VEC>*>(y)[dr * vpr + v];
    Chunk<VEC> co;
#pragma unroll
    for (int e = 0; e < VEC; e += Op::kBytes) Op::apply(cx.b + e, cy.b + e, co.b + e);
    reinterpret_cast<Chunk<VEC>*>(out)[w] = co;
  }
}

// ---- one jagged dimension: a bag is a contiguous copy ----------------------
//
// With a single jagged dim, bag b's values rows are [off[b], off[b+1]) and its
// dense rows [b*max_L, (b+1)*max_L): both contiguous, so each bag is one
// straight copy plus padding, with no per-chunk coordinate arithmetic.  Grid
// (x = bag, y = part of the bag); every thread keeps kJagItems chunks in
// flight.

constexpr int kJagItems = 4;
constexpr int64_t kJagSpan = 256 * kJagItems;

template <int VEC, typename I>
__global__ void __launch_bounds__(256)
    j2pd1_kernel(const uint8_t* __restrict__ values, uint8_t* __restrict__ out,
                 const I* __restrict__ off, int64_t max_L, int64_t vpr, Chunk<VEC> pad) {
  const int64_t b = blockIdx.x;
  const int64_t begin = static_cast<int64_t>(off[b]);
  int64_t len = static_cast<int64_t>(off[b + 1]) - begin;
  len = len < 0 ? 0 : (len > max_L ? max_L : len);
  const int64_t n_copy = len * vpr, n_all = max_L * vpr;
  const Chunk<VEC>* __restrict__ src = reinterpret_cast<const Chunk<VEC>*>(values) + begin * vpr;
  Chunk<VEC>* __restrict__ dst = reinterpret_cast<Chunk<VEC>*>(out) + b * n_all;
  for (int64_t base = blockIdx.y * kJagSpan; base < n_all; base += gridDim.y * kJagSpan) {
    Chunk<VEC> c[kJagItems];
#pragma unroll
    for (int it = 0; it < kJagItems; ++it) {
      const int64_t i = base + it * 256 + threadIdx.x;
      c[it] = i < n_copy ? src[i] : pad;
    }
#pragma unroll
    for (int it = 0; it < kJagItems; ++it) {
      const int64_t i = base + it * 256 + threadIdx.x;
      if (i < n_all) {
        // The dense output streams past the caches (config 1 cold round trip
        // 12.4 -> 11.8 us; the same for dense_to_jagged's output gained nothing).
        if constexpr (VEC == 16) {
          typedef unsigned int u4nt __attribute__((ext_vector_type(4)));
          __builtin_nontemporal_store(*reinterpret_cast<const u4nt*>(&c[it]),
                                      reinterpret_cast<u4nt*>(&dst[i]));
        } else {
          dst[i] = c[it];
        }
      }
    }
  }
}

// Values rows [r0, r1) whose first `copy_rows` rows take dense rows from
// `dense_row0` on and the rest 0; ADD combines x with them (x + y, or x * y
// with MUL), else the dense value is copied (dense -> jagged).
template <int VEC, bool ADD, int DT, bool MUL>
__device__ __forceinline__ void emit_rows(const uint8_t* __restrict__ dense,
                                          const uint8_t* __restrict__ x,
                                          uint8_t* __restrict__ out, int64_t r0, int64_t r1,
                                          int64_t copy_rows, int64_t dense_row0, int64_t vpr) {
  const int64_t n_all = (r1 - r0) * vpr, n_copy = copy_rows * vpr;
  const Chunk<VEC>* __restrict__ src = reinterpret_cast<const Chunk<VEC>*>(dense) + dense_row0 * vpr;
  Chunk<VEC>* __restrict__ dst = reinterpret_cast<Chunk<VEC>*>(out) + r0 * vpr;
  const Chunk<VEC>* __restrict__ xs = reinterpret_cast<const Chunk<VEC>*>(x) + r0 * vpr;
  for (int64_t base = blockIdx.y * kJagSpan; base < n_all; base += gridDim.y * kJagSpan) {
    Chunk<VEC> y[kJagItems];
#pragma unroll
    for (int it = 0; it < kJagItems; ++it) {
      const int64_t i = base + it * 256 + threadIdx.x;
      if (i < n_copy) {
        y[it] = src[i];
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) y[it].b[e] = 0;  // +0 in every element type
      }
    }
#pragma unroll
    for (int it = 0; it < kJagItems; ++it) {
      const int64_t i = base + it * 256 + threadIdx.x;
      if (i >= n_all) continue;
      if constexpr (ADD) {
        const Chunk<VEC> cx = xs[i];
        Chunk<VEC> co;
#pragma unroll
        for (int e = 0; e < VEC; e += BinOp<DT, MUL>::kBytes)
          BinOp<DT, MUL>::apply(cx.b + e, y[it].b + e, co.b + e);
        dst[i] = co;
      } else {
        dst[i] = y[it];
      }
    }
  }
}

// Block x < nbags: bag x.  Block x == nbags: the values rows no bag covers
// (before off[0], from off[nbags] on), which have no dense position.  Row
// ranges are clamped to [0, total_L], so malformed offsets never write out
// of bounds.
template <int VEC, typename I, bool ADD, int DT, bool MUL>
__global__ void __launch_bounds__(256)
    jagged_out1_kernel(const uint8_t* __restrict__ dense, const uint8_t* __restrict__ x,
                       uint8_t* __restrict__ out, const I* __restrict__ off, int64_t nbags,
                       int64_t max_L, int64_t total_L, int64_t vpr) {
  auto clamp = [&](int64_t v, int64_t lo) { return v < lo ? lo : (v > total_L ? total_L : v); };
  const int64_t b = blockIdx.x;
  if (b < nbags) {
    const int64_t r0 = clamp(static_cast<int64_t>(off[b]), 0);
    const int64_t r1 = clamp(static_cast<int64_t>(off[b + 1]), r0);
    const int64_t copy = r1 - r0 < max_L ? r1 - r0 : max_L;
    emit_rows<VEC, ADD, DT, MUL>(dense, x, out, r0, r1, copy, b * max_L, vpr);
  } else {
    const int64_t head = clamp(static_cast<int64_t>(off[0]), 0);
    const int64_t tail = clamp(static_cast<int64_t>(off[nbags]), head);
    emit_rows<VEC, ADD, DT, MUL>(dense, x, out, 0, head, 0, 0, vpr);
    emit_rows<VEC, ADD, DT, MUL>(dense, x, out, tail, total_L, 0, 0, vpr);
  }
}

// ---- host side ------------------------------------------------------------

// Grid of the single-jagged-dim kernels: one x per bag (plus extra), parts
// of a bag in y.
dim3 grid_1d(int64_t bags, int64_t chunks_per_bag) {
  int64_t parts = ceil_div(chunks_per_bag > 0 ? chunks_per_bag : 1, kJagSpan);
  if (parts > 64) parts = 64;  // the kernels loop over the rest
  return dim3(static_cast<uint32_t>(bags), static_cast<uint32_t>(parts));
}

int pick_vec(int64_t row_bytes, std::initializer_list<const void*> ptrs) {
  for (int vec : {16, 8, 4, 2, 1}) {
    if (row_bytes % vec) continue;
    bool ok = true;
    for (const void* p : ptrs)
      if (reinterpret_cast<uintptr_t>(p) % vec) ok = false;
    if (ok) return vec;
  }
  return 1;
}

int grid_for(int64_t items) {
  const int64_t blocks = ceil_div(items, 256);
  const int64_t cap = static_cast<int64_t>(num_cus()) * 32;
  return static_cast<int>(blocks < 1 ? 1 : (blocks > cap ? cap : blocks));
}

int build_meta(JaggedMeta& m, int32_t ndim, const void* const* offsets, int32_t offset_bytes,
               const int64_t* offsets_numel, const int64_t* max_lengths) {
  MX_REQUIRE(ndim >= 1 && ndim <= MX_MAX_JAGGED_DIM, "num_jagged_dim %d not in [1, %d]", ndim,
             MX_MAX_JAGGED_DIM);
  MX_REQUIRE(offset_bytes == 4 || offset_bytes == 8, "offsets must be int32 or int64");
  MX_REQUIRE(offsets != nullptr && offsets_numel != nullptr && max_lengths != nullptr,
             "null offsets/offsets_numel/max_lengths");
  m.ndim = ndim;
  for (int k = 0; k < ndim; ++k) {
    MX_REQUIRE(offsets_numel[k] >= 1, "offsets[%d] must have at least one entry", k);
    MX_REQUIRE(offsets[k] != nullptr, "null offsets[%d]", k);
    MX_REQUIRE(max_lengths[k] >= 0, "negative max_length[%d]", k);
    m.off[k] = offsets[k];
    m.off_len[k] = offsets_numel[k];
    m.max_len[k] = max_lengths[k];
  }
  for (int k = ndim; k < MX_MAX_JAGGED_DIM; ++k) {
    m.off[k] = nullptr;
    m.off_len[k] = 0;
    m.max_len[k] = 1;
  }
  return MX_OK;
}

bool valid_elem(int64_t eb) { return eb == 1 || eb == 2 || eb == 4 || eb == 8; }

int64_t dtype_bytes(int32_t dt) {
  switch (dt) {
    case MX_DTYPE_F32: return 4;
    case MX_DTYPE_F64: return 8;
    case MX_DTYPE_F16:
    case MX_DTYPE_BF16: return 2;
    default: return -1;
  }
}

}  // namespace
}  // namespace mx

using namespace mx;

#define MX_VEC_SWITCH(vec, ...)                             \
  switch (vec) {                                            \
    case 16: { constexpr int V = 16; __VA_ARGS__; break; } \
    case 8: { constexpr int V = 8; __VA_ARGS__; break; }   \
    case 4: { constexpr int V = 4; __VA_ARGS__; break; }   \
    case 2: { constexpr int V = 2; __VA_ARGS__; break; }   \
    default: { constexpr int V = 1; __VA_ARGS__; break; }  \
  }

extern "C" int mx_jagged_to_padded_dense(const void* values, int64_t elem_bytes, int64_t inner,
                                         int32_t num_jagged_dim, const void* const* offsets,
                                         int32_t offset_bytes, const int64_t* offsets_numel,
                                         const int64_t* max_lengths, uint64_t pad_bits,
                                         void* out, void* stream) {
  clear_error();
  JaggedMeta m;
  if (int rc = build_meta(m, num_jagged_dim, offsets, offset_bytes, offsets_numel, max_lengths))
    return rc;
  MX_REQUIRE(valid_elem(elem_bytes), "element size %lld not supported", (long long)elem_bytes);
  MX_REQUIRE(inner >= 0, "negative inner size");
  int64_t rows = offsets_numel[0] - 1;
  for (int k = 0; k < num_jagged_dim; ++k) rows *= max_lengths[k];
  const int64_t row_bytes = inner * elem_bytes;
  if (rows == 0 || row_bytes == 0) return MX_OK;
  MX_REQUIRE(out != nullptr, "null out");  // values may be empty (every row padding)
  int vec = pick_vec(row_bytes, {values, out});
  if (vec < elem_bytes) vec = static_cast<int>(elem_bytes);  // keep elements whole
  MX_REQUIRE(row_bytes % vec == 0, "misaligned tensors");
  uint8_t pat[16];  // padding pattern replicated over a 16-byte chunk
  for (int i = 0; i < 16; ++i) pat[i] = static_cast<uint8_t>(pad_bits >> (8 * (i % elem_bytes)));
  const int64_t vpr = row_bytes / vec;
  auto* s = as_stream(stream);
  const auto* v = static_cast<const uint8_t*>(values);
  auto* o = static_cast<uint8_t*>(out);
  const int64_t nbags = offsets_numel[0] - 1;
  const bool one = num_jagged_dim == 1 && nbags <= 0x7fffffffll;
  const int grid = one ? 0 : grid_for(rows * vpr);  // the one-dim grid is per bag
  MX_VEC_SWITCH(vec, {
    Chunk<V> pad;
    for (int i = 0; i < V; ++i) pad.b[i] = pat[i];
    if (one) {
      const dim3 g = grid_1d(nbags, max_lengths[0] * vpr);
      if (offset_bytes == 8)
        j2pd1_kernel<V, int64_t><<<g, 256, 0, s>>>(
            v, o, static_cast<const int64_t*>(offsets[0]), max_lengths[0], vpr, pad);
      else
        j2pd1_kernel<V, int32_t><<<g, 256, 0, s>>>(
            v, o, static_cast<const int32_t*>(offsets[0]), max_lengths[0], vpr, pad);
    } else if (offset_bytes == 8) {
      j2pd_kernel<V, int64_t><<<grid, 256, 0, s>>>(v, o, m, rows, vpr, pad);
    } else {
      j2pd_kernel<V, int32_t><<<grid, 256, 0, s>>>(v, o, m, rows, vpr, pad);
    }
  });
  MX_LAUNCH_CHECK();
  return MX_OK;
}

// Shared host path of dense_to_jagged (x_values == NULL) and of the
// jagged (op) dense elementwise ops (x_values != NULL; mul: x * y, else x + y).
static int jagged_output_op(const void* dense, int64_t elem_bytes, int64_t inner,
                            int32_t num_jagged_dim, const void* const* offsets,
                            int32_t offset_bytes, const int64_t* offsets_numel,
                            const int64_t* max_lengths, int64_t total_L, const void* x_values,
                            int32_t add_dtype, bool mul, void* out, void* stream) {
  JaggedMeta m;
  if (int rc = build_meta(m, num_jagged_dim, offsets, offset_bytes, offsets_numel, max_lengths))
    return rc;
  MX_REQUIRE(valid_elem(elem_bytes), "element size %lld not supported", (long long)elem_bytes);
  MX_REQUIRE(inner >= 0 && total_L >= 0, "negative size");
  const int64_t row_bytes = inner * elem_bytes;
  if (total_L == 0 || row_bytes == 0) return MX_OK;
  MX_REQUIRE(out != nullptr, "null out");
  int64_t dense_rows = offsets_numel[0] - 1;
  for (int k = 0; k < num_jagged_dim; ++k) dense_rows *= max_lengths[k];
  MX_REQUIRE(dense != nullptr || dense_rows == 0, "null dense");
  const int vec0 = x_values ? pick_vec(row_bytes, {dense, out, x_values})
                            : pick_vec(row_bytes, {dense, out});
  const int vec = vec0 < elem_bytes ? static_cast<int>(elem_bytes) : vec0;
  MX_REQUIRE(row_bytes % vec == 0, "misaligned tensors");
  const int64_t vpr = row_bytes / vec;
  auto* s = as_stream(stream);
  const auto* d = static_cast<const uint8_t*>(dense);
  auto* o = static_cast<uint8_t*>(out);
  const int64_t nbags = offsets_numel[0] - 1;
  const bool one = num_jagged_dim == 1 && nbags < 0x7fffffffll;
  const int grid = one ? 0 : grid_for(total_L * vpr);  // the one-dim grid is per bag
  const dim3 g1 = grid_1d(nbags + 1, max_lengths[0] * vpr);
  const int64_t L0 = max_lengths[0];
  if (x_values == nullptr) {
    MX_VEC_SWITCH(vec, {
      if (one) {
        if (offset_bytes == 8)
          jagged_out1_kernel<V, int64_t, false, MX_DTYPE_F32, false><<<g1, 256, 0, s>>>(
              d, nullptr, o, static_cast<const int64_t*>(offsets[0]), nbags, L0, total_L, vpr);
        else
          jagged_out1_kernel<V, int32_t, false, MX_DTYPE_F32, false><<<g1, 256, 0, s>>>(
              d, nullptr, o, static_cast<const int32_t*>(offsets[0]), nbags, L0, total_L, vpr);
      } else if (offset_bytes == 8) {
        d2j_kernel<V, int64_t><<<grid, 256, 0, s>>>(d, o, m, total_L, vpr);
      } else {
        d2j_kernel<V, int32_t><<<grid, 256, 0, s>>>(d, o, m, total_L, vpr);
      }
    });
    MX_LAUNCH_CHECK();
    return MX_OK;
  }
  MX_REQUIRE(dtype_bytes(add_dtype) == elem_bytes, "dtype %d does not match element size %lld",
             add_dtype, (long long)elem_bytes);
  const auto* x = static_cast<const uint8_t*>(x_values);
#define MX_OP_LAUNCH(DTC, MULC)                                                                 \
  MX_VEC_SWITCH(vec, {                                                                          \
    if constexpr (V >= BinOp<DTC, MULC>::kBytes) {                                              \
      if (one && offset_bytes == 8)                                                             \
        jagged_out1_kernel<V, int64_t, true, DTC, MULC><<<g1, 256, 0, s>>>(                     \
            d, x, o, static_cast<const int64_t*>(offsets[0]), nbags, L0, total_L, vpr);         \
      else if (one)                                                                             \
        jagged_out1_kernel<V, int32_t, true, DTC, MULC><<<g1, 256, 0, s>>>(                     \
            d, x, o, static_cast<const int32_t*>(offsets[0]), nbags, L0, total_L, vpr);         \
      else if (offset_bytes == 8)                                                               \
        jagged_add_kernel<V, int64_t, DTC, MULC><<<grid, 256, 0, s>>>(x, d, o, m, total_L, vpr); \
      else                                                                                      \
        jagged_add_kernel<V, int32_t, DTC, MULC><<<grid, 256, 0, s>>>(x, d, o, m, total_L, vpr); \
    }                                                                                           \
  })
#define MX_ADD_LAUNCH(DTC)    \
  if (mul) {                  \
    MX_OP_LAUNCH(DTC, true);  \
  } else {                    \
    MX_OP_LAUNCH(DTC, false); \
  }
  switch (add_dtype) {
    case MX_DTYPE_F32: MX_ADD_LAUNCH(MX_DTYPE_F32); break;
    case MX_DTYPE_F64: MX_ADD_LAUNCH(MX_DTYPE_F64); break;
    case MX_DTYPE_F16: MX_ADD_LAUNCH(MX_DTYPE_F16); break;
    case MX_DTYPE_BF16: MX_ADD_LAUNCH(MX_DTYPE_BF16); break;
    default: return set_error(MX_EUNSUPPORTED, "dtype %d not supported", add_dtype);
  }
#undef MX_ADD_LAUNCH
#undef MX_OP_LAUNCH
  MX_LAUNCH_CHECK();
  return MX_OK;
}

extern "C" int mx_dense_to_jagged(const void* dense, int64_t elem_bytes, int64_t inner,
                                  int32_t num_jagged_dim, const void* const* offsets,
                                  int32_t offset_bytes, const int64_t* offsets_numel,
                                  const int64_t* max_lengths, int64_t total_L, void* out,
                                  void* stream) {
  clear_error();
  return jagged_output_op(dense, elem_bytes, inner, num_jagged_dim, offsets, offset_bytes,
                          offsets_numel, max_lengths, total_L, nullptr, 0, false, out, stream);
}

extern "C" int mx_jagged_dense_elementwise_add(const void* x_values, const void* y_dense,
                                               int32_t dtype, int64_t inner,
                                               int32_t num_jagged_dim, const void* const* offsets,
                                               int32_t offset_bytes, const int64_t* offsets_numel,
                                               const int64_t* max_lengths, int64_t total_L,
                                               void* out, void* stream) {
  clear_error();
  const int64_t eb = dtype_bytes(dtype);
  if (eb < 0) return set_error(MX_EUNSUPPORTED, "dtype %d not supported", dtype);
  MX_REQUIRE(x_values != nullptr || total_L == 0, "null x_values");
  if (total_L == 0 || inner == 0) return MX_OK;
  return jagged_output_op(y_dense, eb, inner, num_jagged_dim, offsets, offset_bytes,
                          offsets_numel, max_lengths, total_L, x_values, dtype, false, out, stream);
}

extern "C" int mx_jagged_dense_elementwise_mul(const void* x_values, const void* y_dense,
                                               int32_t dtype, int64_t inner,
                                               int32_t num_jagged_dim, const void* const* offsets,
                                               int32_t offset_bytes, const int64_t* offsets_numel,
                                               const int64_t* max_lengths, int64_t total_L,
                                               void* out, void* stream) {
  clear_error();
  const int64_t eb = dtype_bytes(dtype);
  if (eb < 0) return set_error(MX_EUNSUPPORTED, "dtype %d not supported", dtype);
  MX_REQUIRE(x_values != nullptr || total_L == 0, "null x_values");
  if (total_L == 0 || inner == 0) return MX_OK;
  return jagged_output_op(y_dense, eb, inner, num_jagged_dim, offsets, offset_bytes,
                          offsets_numel, max_lengths, total_L, x_values, dtype, true, out, stream);
}
