// Device-wide exclusive prefix sum of 32-bit counts produced by a functor,
// in three launches: per-tile reduce, one-block scan of the tile sums, and
// per-tile scan + write.  The effective length may live on the device
// (`n_dev`, e.g. a run count), so no host synchronisation is needed; `n` is
// the host-side upper bound that sizes the grid.
#pragma once

#include "mx_common.h"

namespace mx {

constexpr int kScanThreads = 256;
constexpr int kScanItems = 16;
constexpr int64_t kScanTile = kScanThreads * kScanItems;

inline int64_t scan_tiles(int64_t n) { return ceil_div(n > 0 ? n : 1, kScanTile); }

// Inclusive scan over the 64 lanes of a wave.
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t o = __shfl_up(v, d, 64);
    if (lane >= d) v += o;
  }
  return v;
}

// Exclusive scan across a 256-thread block; returns the block total in *total.
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t* total) {
  __shared__ uint32_t wsum[kScanThreads / 64];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const uint32_t incl = wave_incl_scan(v);
  if (lane == 63) wsum[w] = incl;
  __syncthreads();
  uint32_t before = 0, all = 0;
#pragma unroll
  for (int i = 0; i < kScanThreads / 64; ++i) {
    if (i < w) before += wsum[i];
    all += wsum[i];
  }
  __syncthreads();
  *total = all;
  return before + incl - v;
}

__device__ __forceinline__ int64_t eff_len(int64_t n, const int32_t* n_dev) {
  if (n_dev == nullptr) return n;
  const int64_t m = *n_dev;
  return m < n ? m : n;
}

template <class F>
__global__ void __launch_bounds__(kScanThreads)
    scan_reduce_kernel(F f, int64_t n, const int32_t* n_dev, uint32_t* tile_sums) {
  const int64_t m = eff_len(n, n_dev);
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile;
  uint32_t s = 0;
#pragma unroll
  for (int it = 0; it < kScanItems; ++it) {
    const int64_t i = base + it * kScanThreads + threadIdx.x;
    if (i < m) s += f(i);
  }
  uint32_t total;
  block_excl_scan(s, &total);
  if (threadIdx.x == 0) tile_sums[blockIdx.x] = total;
}

// One block: exclusive scan of tile_sums[0..ntiles) in place; *total_out = sum.
__global__ void __launch_bounds__(1024)
    scan_tiles_kernel(uint32_t* tile_sums, int64_t ntiles, uint32_t* total_out);

template <class F>
__global__ void __launch_bounds__(kScanThreads)
    scan_write_kernel(F f, int64_t n, const int32_t* n_dev, const uint32_t* tile_prefix,
                      uint32_t* out) {
  const int64_t m = eff_len(n, n_dev);
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile + threadIdx.x * kScanItems;
  uint32_t v[kScanItems];
  uint32_t s = 0;
#pragma unroll
  for (int it = 0; it < kScanItems; ++it) {
    const int64_t i = base + it;
    v[it] = i < m ? f(i) : 0u;
    s += v[it];
  }
  uint32_t total;
  uint32_t run = block_excl_scan(s, &total) + tile_prefix[blockIdx.x];
#pragma unroll
  for (int it = 0; it < kScanItems; ++it) {
    const int64_t i = base + it;
    if (i < m) out[i] = run;
    run += v[it];
  }
}

// out[i] = sum_{j<i} f(j) for i < effective length; *total = sum of all.
// `tile_buf` needs scan_tiles(n) entries.
template <class F>
int exclusive_scan(F f, int64_t n, const int32_t* n_dev, uint32_t* out, uint32_t* total,
                   uint32_t* tile_buf, hipStream_t s) {
  const int64_t nt = scan_tiles(n);
  if (nt > 0x7fffffffll) return set_error(MX_EINVAL, "scan too long");
  const dim3 grid(static_cast<uint32_t>(nt));
  scan_reduce_kernel<F><<<grid, kScanThreads, 0, s>>>(f, n, n_dev, tile_buf);
  scan_tiles_kernel<<<1, 1024, 0, s>>>(tile_buf, nt, total);
  scan_write_kernel<F><<<grid, kScanThreads, 0, s>>>(f, n, n_dev, tile_buf, out);
  MX_LAUNCH_CHECK();
  return MX_OK;
}

}  // namespace mx
