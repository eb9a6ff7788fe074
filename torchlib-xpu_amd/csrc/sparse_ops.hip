// Sparse-feature helpers either side of the TBE lookup, for gfx950: the
// prefix sums that turn lengths into offsets, and the feature permute of a
// [T, B] batch of lengths and indices.
//
// Semantics (fbgemm_gpu sparse ops, recalled):
//  * asynchronous_exclusive_cumsum(x)[i] = x[0] + ... + x[i-1];
//    asynchronous_inclusive_cumsum(x)[i] = x[0] + ... + x[i];
//    asynchronous_complete_cumsum(x) = [0, inclusive...] (n + 1 entries; a
//    2-D input is summed per row).  int32 or int64, in the input's type (two's
//    complement wrap-around, as the integer adds of the GPU op).
//  * permute_2D_sparse_data(permute, lengths [T, B], indices, weights): output
//    feature f is input feature permute[f]: permuted_lengths[f, :] =
//    lengths[permute[f], :], and the indices (and weights) of each bag (f, b)
//    are the input's bag (permute[f], b), in order.  permute may repeat or
//    drop features.  permute_1D_sparse_data is the same with one bag per
//    feature (lengths [T]).
//  * offsets_range(offsets [N], range_size): out[j] = j - offsets[i] for j in
//    segment i = [offsets[i], offsets[i + 1]) (the last ends at range_size).
//  * expand_into_jagged_permute(permute [T], input_offsets, output_offsets,
//    output_size): out[output_offsets[t] + j] = input_offsets[permute[t]] + j
//    for j below output feature t's length.
//
// Design: integer work, HBM-bound.  The scans are reduce-then-scan with no
// waits between blocks: a block sums its 8192-element tile, then every block
// scans its tile from its prefix, the sum of the tiles before it (added up by
// the block itself up to 1024 tiles, beyond that scanned first by one block;
// a batch of one tile takes only the last launch).  A 2-D complete cumsum gives each
// row to one block.  The permute copies each output bag with one 16-lane
// group (consecutive elements, coalesced), from the two complete cumsums.
#include <type_traits>

#include "mx_common.h"

namespace mx {
namespace {

constexpr int kCsThreads = 1024;
constexpr int kCsItems = 8;
constexpr int64_t kCsTile = static_cast<int64_t>(kCsThreads) * kCsItems;

// Sums in the type's own wrap-around arithmetic (signed overflow is not
// defined in C++: add as unsigned).
template <typename T>
__device__ __forceinline__ T wadd(T a, T b) {
  using U = std::make_unsigned_t<T>;
  return static_cast<T>(static_cast<U>(a) + static_cast<U>(b));
}

template <typename T>
__device__ __forceinline__ T wsub(T a, T b) {
  using U = std::make_unsigned_t<T>;
  return static_cast<T>(static_cast<U>(a) - static_cast<U>(b));
}

// Exclusive scan of one value per thread over a block of kCsThreads; the
// block's total in *total.
template <typename T>
__device__ __forceinline__ T block_excl(T v, T* total) {
  __shared__ T wsum[kCsThreads / 64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  T incl = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const T o = __shfl_up(incl, d, 64);
    if (lane >= d) incl = wadd(incl, o);
  }
  if (lane == 63) wsum[w] = incl;
  __syncthreads();
  T before = 0, all = 0;
#pragma unroll
  for (int i = 0; i < kCsThreads / 64; ++i) {
    if (i < w) before = wadd(before, wsum[i]);
    all = wadd(all, wsum[i]);
  }
  __syncthreads();  // wsum is reused by the next call
  *total = all;
  return wsub(wadd(before, incl), v);
}

// A tile's sum: wrap-around integer sums do not depend on the order, so each
// thread adds a strided slice and every load instruction is coalesced.
template <typename T>
__global__ void __launch_bounds__(kCsThreads)
    cumsum_tile_kernel(const T* __restrict__ x, int64_t n, T* __restrict__ partial) {
  const int64_t tile0 = static_cast<int64_t>(blockIdx.x) * kCsTile;
  T s = 0;
#pragma unroll
  for (int it = 0; it < kCsItems; ++it) {
    const int64_t i = tile0 + it * kCsThreads + threadIdx.x;
    if (i < n) s = wadd(s, x[i]);
  }
  T total;
  (void)block_excl<T>(s, &total);
  if (threadIdx.x == 0) partial[blockIdx.x] = total;
}

// One block: the tile sums into their exclusive prefixes, in place.
template <typename T>
__global__ void __launch_bounds__(kCsThreads) cumsum_spine_kernel(T* __restrict__ partial,
                                                                   int64_t ntiles) {
  T carry = 0;
  for (int64_t c = 0; c < ntiles; c += kCsThreads) {
    const int64_t i = c + threadIdx.x;
    const T v = i < ntiles ? partial[i] : T(0);
    T total;
    const T ex = block_excl<T>(v, &total);
    if (i < ntiles) partial[i] = wadd(carry, ex);
    carry = wadd(carry, total);
  }
}

// KIND 0 exclusive, 1 inclusive, 2 complete (out[0] = 0, out[i + 1] = inclusive[i]).
// The tile passes through LDS both ways, so that the global loads and stores
// are coalesced while each thread scans kCsItems consecutive elements; a row
// of kCsItems elements takes kCsPad slots (fewer bank conflicts).
constexpr int kCsPad = kCsItems + 1;
__device__ __forceinline__ int cs_slot(int j) { return (j / kCsItems) * kCsPad + j % kCsItems; }

// prefix: null (one tile), the tiles' exclusive prefixes, or with `raw` the
// tiles' sums (at most kCsThreads tiles), which each block adds up to its own.
template <typename T, int KIND>
__global__ void __launch_bounds__(kCsThreads)
    cumsum_scan_kernel(const T* __restrict__ x, int64_t n, const T* __restrict__ prefix,
                       bool raw, T* __restrict__ out) {
  __shared__ T s_buf[kCsThreads * kCsPad];
  const int64_t tile0 = static_cast<int64_t>(blockIdx.x) * kCsTile;
  T pre = 0;
  if (raw) {  // block-uniform
    (void)block_excl<T>(threadIdx.x < blockIdx.x ? prefix[threadIdx.x] : T(0), &pre);
  } else if (prefix) {
    pre = prefix[blockIdx.x];
  }
#pragma unroll
  for (int it = 0; it < kCsItems; ++it) {
    const int j = it * kCsThreads + threadIdx.x;
    s_buf[cs_slot(j)] = tile0 + j < n ? x[tile0 + j] : T(0);
  }
  __syncthreads();
  T v[kCsItems];
  T s = 0;
#pragma unroll
  for (int it = 0; it < kCsItems; ++it) {
    v[it] = s_buf[threadIdx.x * kCsPad + it];
    s = wadd(s, v[it]);
  }
  T total;
  // block_excl's barriers also order every thread's reads above before the
  // writes below.
  T run = wadd(block_excl<T>(s, &total), pre);
#pragma unroll
  for (int it = 0; it < kCsItems; ++it) {
    const T before = run;
    run = wadd(run, v[it]);
    s_buf[threadIdx.x * kCsPad + it] = KIND == 0 ? before : run;
  }
  __syncthreads();
  if (KIND == 2 && blockIdx.x == 0 && threadIdx.x == 0) out[0] = 0;
#pragma unroll
  for (int it = 0; it < kCsItems; ++it) {
    const int j = it * kCsThreads + threadIdx.x;
    if (tile0 + j < n) out[tile0 + j + (KIND == 2 ? 1 : 0)] = s_buf[cs_slot(j)];
  }
}

// 2-D complete cumsum: block r scans row r of x [rows, n] into out [rows, n + 1].
template <typename T>
__global__ void __launch_bounds__(kCsThreads)
    cumsum_rows_kernel(const T* __restrict__ x, int64_t n, T* __restrict__ out) {
  const T* xr = x + static_cast<int64_t>(blockIdx.x) * n;
  T* orow = out + static_cast<int64_t>(blockIdx.x) * (n + 1);
  if (threadIdx.x == 0) orow[0] = 0;
  T carry = 0;
  for (int64_t c = 0; c < n; c += kCsTile) {
    const int64_t base = c + threadIdx.x * kCsItems;
    T v[kCsItems];
    T s = 0;
#pragma unroll
    for (int it = 0; it < kCsItems; ++it) {
      v[it] = base + it < n ? xr[base + it] : T(0);
      s = wadd(s, v[it]);
    }
    T total;
    T run = wadd(block_excl<T>(s, &total), carry);
#pragma unroll
    for (int it = 0; it < kCsItems; ++it) {
      if (base + it >= n) break;
      run = wadd(run, v[it]);
      orow[base + it + 1] = run;
    }
    carry = wadd(carry, total);
  }
}

template <typename T>
int cumsum_t(const T* x, int64_t n, int32_t kind, T* out, T* partial, hipStream_t s) {
  const int64_t nt = ceil_div(n > 0 ? n : 1, kCsTile);  // n = 0: one block writes out[0]
  MX_REQUIRE(nt <= 0x7fffffffll, "cumsum of %lld elements too long", (long long)n);
  const dim3 gd(static_cast<uint32_t>(nt));
  const T* prefix = nullptr;
  // Up to kCsThreads tiles each scan block adds the tile sums before its own
  // (one launch fewer than the spine kernel, which scans them beyond that).
  const bool raw = nt > 1 && nt <= kCsThreads;
  if (nt > 1) {
    cumsum_tile_kernel<T><<<gd, kCsThreads, 0, s>>>(x, n, partial);
    if (!raw) cumsum_spine_kernel<T><<<1, kCsThreads, 0, s>>>(partial, nt);
    prefix = partial;
  }
  if (kind == 0)
    cumsum_scan_kernel<T, 0><<<gd, kCsThreads, 0, s>>>(x, n, prefix, raw, out);
  else if (kind == 1)
    cumsum_scan_kernel<T, 1><<<gd, kCsThreads, 0, s>>>(x, n, prefix, raw, out);
  else
    cumsum_scan_kernel<T, 2><<<gd, kCsThreads, 0, s>>>(x, n, prefix, raw, out);
  MX_LAUNCH_CHECK();
  return MX_OK;
}

// ---- permute_2D_sparse_data --------------------------------------------------

template <typename L>
__global__ void __launch_bounds__(256)
    permute_lengths_kernel(const int32_t* __restrict__ permute, const L* __restrict__ lengths,
                           int32_t T, int64_t B, int64_t Tp, L* __restrict__ out) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < Tp * B;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t f = i / B, b = i - f * B;
    const int32_t src = permute[f];
    out[i] = src >= 0 && src < T ? lengths[static_cast<int64_t>(src) * B + b] : L(0);
  }
}

// A 16-lane group per output bag (f, b): copies the input bag (permute[f], b).
template <typename L, typename I, typename W>
__global__ void __launch_bounds__(256)
    permute_data_kernel(const int32_t* __restrict__ permute, const L* __restrict__ in_off,
                        const L* __restrict__ out_off, int32_t T, int64_t B, int64_t Tp,
                        const I* __restrict__ indices, const W* __restrict__ weights,
                        int64_t in_len, I* __restrict__ out_indices, W* __restrict__ out_weights,
                        int64_t out_len) {
  constexpr int G = 16;
  const int k = threadIdx.x % G;
  const int64_t ngrp = static_cast<int64_t>(gridDim.x) * (256 / G);
  for (int64_t bag = static_cast<int64_t>(blockIdx.x) * (256 / G) + threadIdx.x / G;
       bag < Tp * B; bag += ngrp) {
    const int64_t f = bag / B, b = bag - f * B;
    const int32_t src = permute[f];
    if (src < 0 || src >= T) continue;  // its length is 0
    const int64_t s0 = static_cast<int64_t>(in_off[static_cast<int64_t>(src) * B + b]);
    const int64_t d0 = static_cast<int64_t>(out_off[bag]);
    const int64_t len = static_cast<int64_t>(out_off[bag + 1]) - d0;
    if (s0 < 0 || d0 < 0) continue;  // negative lengths upstream: nothing in bounds to copy
    for (int64_t j = k; j < len; j += G) {
      // Lengths that disagree with the index count or the given output size
      // stop the copy instead of reading or writing past either array.
      if (d0 + j >= out_len || s0 + j >= in_len) break;
      out_indices[d0 + j] = indices[s0 + j];
      if (weights) out_weights[d0 + j] = weights[s0 + j];
    }
  }
}

// A 16-lane group per segment writes j - start over its range.
template <typename I>
__global__ void __launch_bounds__(256)
    offsets_range_kernel(const I* __restrict__ offsets, int64_t nseg, int64_t range_size,
                         I* __restrict__ out) {
  constexpr int G = 16;
  const int k = threadIdx.x % G;
  const int64_t ngrp = static_cast<int64_t>(gridDim.x) * (256 / G);
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * (256 / G) + threadIdx.x / G; i < nseg;
       i += ngrp) {
    int64_t s0 = static_cast<int64_t>(offsets[i]);
    int64_t s1 = i + 1 < nseg ? static_cast<int64_t>(offsets[i + 1]) : range_size;
    s0 = s0 < 0 ? 0 : s0;
    s1 = s1 > range_size ? range_size : s1;
    for (int64_t j = s0 + k; j < s1; j += G) out[j] = static_cast<I>(j - s0);
  }
}

// A 16-lane group per output feature t.
template <typename I>
__global__ void __launch_bounds__(256)
    expand_permute_kernel(const int32_t* __restrict__ permute, const I* __restrict__ in_off,
                          int64_t in_n, const I* __restrict__ out_off, int64_t T, bool out_has_end,
                          int64_t output_size, I* __restrict__ out) {
  constexpr int G = 16;
  const int k = threadIdx.x % G;
  const int64_t ngrp = static_cast<int64_t>(gridDim.x) * (256 / G);
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * (256 / G) + threadIdx.x / G; t < T;
       t += ngrp) {
    const int32_t src = permute[t];
    if (src < 0 || src >= in_n) continue;
    int64_t d0 = static_cast<int64_t>(out_off[t]);
    int64_t d1 = out_has_end || t + 1 < T ? static_cast<int64_t>(out_off[t + 1]) : output_size;
    d0 = d0 < 0 ? 0 : d0;
    d1 = d1 > output_size ? output_size : d1;
    const int64_t s0 = static_cast<int64_t>(in_off[src]);
    for (int64_t j = d0 + k; j < d1; j += G) out[j] = static_cast<I>(s0 + (j - d0));
  }
}

int grid_for(int64_t work, int64_t per_block) {
  const int64_t want = ceil_div(work > 0 ? work : 1, per_block);
  const int64_t cap = static_cast<int64_t>(num_cus()) * 16;
  return static_cast<int>(want < cap ? want : cap);
}

}  // namespace
}  // namespace mx

using namespace mx;

extern "C" size_t mx_cumsum_workspace_bytes(int64_t n, int32_t elem_bytes) {
  const int64_t nt = ceil_div(n > 0 ? n : 1, kCsTile);
  return static_cast<size_t>(nt) * static_cast<size_t>(elem_bytes > 0 ? elem_bytes : 8);
}

extern "C" int mx_cumsum(const void* in, int32_t elem_bytes, int64_t rows, int64_t n,
                         int32_t kind, void* out, void* workspace, size_t workspace_bytes,
                         void* stream) {
  clear_error();
  MX_REQUIRE(elem_bytes == 4 || elem_bytes == 8, "cumsum needs int32 or int64 elements");
  MX_REQUIRE(kind >= 0 && kind <= 2, "cumsum kind %d (0 exclusive, 1 inclusive, 2 complete)",
             kind);
  MX_REQUIRE(rows >= 1 && n >= 0, "cumsum of %lld rows of %lld", (long long)rows, (long long)n);
  MX_REQUIRE(rows == 1 || kind == 2, "a 2-D cumsum is complete only");
  auto* s = as_stream(stream);
  if (rows > 1) {
    MX_REQUIRE(rows <= 0x7fffffffll, "too many rows");
    MX_REQUIRE(out && (n == 0 || in), "null pointer argument");
    const dim3 gd(static_cast<uint32_t>(rows));
    if (elem_bytes == 8)
      cumsum_rows_kernel<int64_t><<<gd, kCsThreads, 0, s>>>(static_cast<const int64_t*>(in), n,
                                                            static_cast<int64_t*>(out));
    else
      cumsum_rows_kernel<int32_t><<<gd, kCsThreads, 0, s>>>(static_cast<const int32_t*>(in), n,
                                                            static_cast<int32_t*>(out));
    MX_LAUNCH_CHECK();
    return MX_OK;
  }
  if (n == 0) {
    if (kind != 2) return MX_OK;
    MX_REQUIRE(out, "null pointer argument");
    return elem_bytes == 8 ? cumsum_t<int64_t>(nullptr, 0, 2, static_cast<int64_t*>(out), nullptr, s)
                           : cumsum_t<int32_t>(nullptr, 0, 2, static_cast<int32_t*>(out), nullptr, s);
  }
  MX_REQUIRE(in && out, "null pointer argument");
  const int64_t nt = ceil_div(n, kCsTile);  // n > 0 here
  if (nt > 1 && (workspace == nullptr || workspace_bytes < mx_cumsum_workspace_bytes(n, elem_bytes)))
    return set_error(MX_EWORKSPACE, "workspace of %zu bytes needed",
                     mx_cumsum_workspace_bytes(n, elem_bytes));
  if (elem_bytes == 8)
    return cumsum_t<int64_t>(static_cast<const int64_t*>(in), n, kind, static_cast<int64_t*>(out),
                             static_cast<int64_t*>(workspace), s);
  return cumsum_t<int32_t>(static_cast<const int32_t*>(in), n, kind, static_cast<int32_t*>(out),
                           static_cast<int32_t*>(workspace), s);
}

extern "C" int mx_permute_2d_lengths(const int32_t* permute, int64_t T_out, const void* lengths,
                                     int32_t length_bytes, int32_t T, int64_t B,
                                     void* permuted_lengths, void* stream) {
  clear_error();
  MX_REQUIRE(length_bytes == 4 || length_bytes == 8, "lengths must be int32 or int64");
  MX_REQUIRE(T >= 0 && B >= 0 && T_out >= 0, "negative size");
  if (T_out * B == 0) return MX_OK;
  MX_REQUIRE(permute && permuted_lengths && (T == 0 || lengths), "null pointer argument");
  auto* s = as_stream(stream);
  const dim3 gd(static_cast<uint32_t>(grid_for(T_out * B, 256)));
  if (length_bytes == 8)
    permute_lengths_kernel<int64_t><<<gd, 256, 0, s>>>(permute, static_cast<const int64_t*>(lengths),
                                                       T, B, T_out,
                                                       static_cast<int64_t*>(permuted_lengths));
  else
    permute_lengths_kernel<int32_t><<<gd, 256, 0, s>>>(permute, static_cast<const int32_t*>(lengths),
                                                       T, B, T_out,
                                                       static_cast<int32_t*>(permuted_lengths));
  MX_LAUNCH_CHECK();
  return MX_OK;
}

extern "C" int mx_permute_2d_data(const int32_t* permute, int64_t T_out, int32_t T, int64_t B,
                                  const void* input_offsets, const void* output_offsets,
                                  int32_t offset_bytes, const void* indices, int32_t index_bytes,
                                  int64_t in_len, const float* weights, int64_t out_len,
                                  void* permuted_indices, float* permuted_weights,
                                  void* stream) {
  clear_error();
  MX_REQUIRE(offset_bytes == 4 || offset_bytes == 8, "offsets must be int32 or int64");
  MX_REQUIRE(index_bytes == 4 || index_bytes == 8, "indices must be int32 or int64");
  MX_REQUIRE(T >= 0 && B >= 0 && T_out >= 0 && out_len >= 0 && in_len >= 0, "negative size");
  MX_REQUIRE(!weights == !permuted_weights, "weights and permuted_weights go together");
  if (T_out * B == 0 || out_len == 0) return MX_OK;
  MX_REQUIRE(permute && input_offsets && output_offsets && indices && permuted_indices,
             "null pointer argument");
  auto* s = as_stream(stream);
  const dim3 gd(static_cast<uint32_t>(grid_for(T_out * B, 256 / 16)));
#define MX_PERM(L, I)                                                                       \
  permute_data_kernel<L, I, float><<<gd, 256, 0, s>>>(                                      \
      permute, static_cast<const L*>(input_offsets), static_cast<const L*>(output_offsets), \
      T, B, T_out, static_cast<const I*>(indices), weights, in_len,                          \
      static_cast<I*>(permuted_indices), permuted_weights, out_len)
  if (offset_bytes == 8) {
    if (index_bytes == 8)
      MX_PERM(int64_t, int64_t);
    else
      MX_PERM(int64_t, int32_t);
  } else {
    if (index_bytes == 8)
      MX_PERM(int32_t, int64_t);
    else
      MX_PERM(int32_t, int32_t);
  }
#undef MX_PERM
  MX_LAUNCH_CHECK();
  return MX_OK;
}

extern "C" int mx_offsets_range(const void* offsets, int32_t index_bytes, int64_t nseg,
                                int64_t range_size, void* out, void* stream) {
  clear_error();
  MX_REQUIRE(index_bytes == 4 || index_bytes == 8, "offsets must be int32 or int64");
  MX_REQUIRE(nseg >= 0 && range_size >= 0, "negative size");
  if (nseg == 0 || range_size == 0) return MX_OK;
  MX_REQUIRE(offsets && out, "null pointer argument");
  auto* s = as_stream(stream);
  const dim3 gd(static_cast<uint32_t>(grid_for(nseg, 256 / 16)));
  if (index_bytes == 8)
    offsets_range_kernel<int64_t><<<gd, 256, 0, s>>>(static_cast<const int64_t*>(offsets), nseg,
                                                     range_size, static_cast<int64_t*>(out));
  else
    offsets_range_kernel<int32_t><<<gd, 256, 0, s>>>(static_cast<const int32_t*>(offsets), nseg,
                                                     range_size, static_cast<int32_t*>(out));
  MX_LAUNCH_CHECK();
  return MX_OK;
}

extern "C" int mx_expand_into_jagged_permute(const int32_t* permute, int64_t T,
                                             const void* input_offsets, int64_t input_numel,
                                             const void* output_offsets, int64_t output_numel,
                                             int32_t index_bytes, int64_t output_size, void* out,
                                             void* stream) {
  clear_error();
  MX_REQUIRE(index_bytes == 4 || index_bytes == 8, "offsets must be int32 or int64");
  MX_REQUIRE(T >= 0 && output_size >= 0, "negative size");
  MX_REQUIRE(output_numel == T || output_numel == T + 1,
             "output_offsets must have T or T+1 entries (T=%lld, got %lld)", (long long)T,
             (long long)output_numel);
  if (T == 0 || output_size == 0) return MX_OK;
  MX_REQUIRE(permute && input_offsets && output_offsets && out, "null pointer argument");
  auto* s = as_stream(stream);
  const dim3 gd(static_cast<uint32_t>(grid_for(T, 256 / 16)));
  const bool has_end = output_numel == T + 1;
  if (index_bytes == 8)
    expand_permute_kernel<int64_t><<<gd, 256, 0, s>>>(
        permute, static_cast<const int64_t*>(input_offsets), input_numel,
        static_cast<const int64_t*>(output_offsets), T, has_end, output_size,
        static_cast<int64_t*>(out));
  else
    expand_permute_kernel<int32_t><<<gd, 256, 0, s>>>(
        permute, static_cast<const int32_t*>(input_offsets), input_numel,
        static_cast<const int32_t*>(output_offsets), T, has_end, output_size,
        static_cast<int32_t*>(out));
  MX_LAUNCH_CHECK();
  return MX_OK;
}
