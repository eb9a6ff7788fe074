// bounds_check_indices for gfx950: the step callers run before every TBE
// lookup so that out-of-range indices or offsets never reach a gather.
//
// Semantics: fbgemm_gpu bounds_check_indices (upstream
// src/split_embeddings_utils/, recalled), BoundsCheckMode FATAL=0,
// WARNING=1, IGNORE=2, NONE=3.  This build's contract:
//   * repaired offsets o'[i] = max_{j <= i} clamp(o[j], 0, N): in [0, N] and
//     non-decreasing, so no two bags overlap and no bag runs past the indices;
//   * every index of bag (t, b), i.e. positions [o'[t*B+b], o'[t*B+b+1]),
//     outside [0, rows_per_table[t]) is replaced by 0 (variable batch per
//     feature: bags B_offsets[t] .. B_offsets[t+1]-1 belong to table t);
//   * each repaired entry (offset or index) adds one to warning[0];
//   * FATAL repairs nothing and only counts (the host raises on a non-zero
//     count); NONE does nothing.
// Work: two launches, no zeroed state.  A tile kernel takes, one wave per
// tile, the maximum of the clamped offsets of every tile of `tile` bags.  Then
// a block owns `bpb` consecutive bags (32 to 256, by the mean bag length): it
// rebuilds o' for them exactly (the maximum over earlier tiles and over the
// earlier part of its own tile, then a block-wide max-scan), repairs its own
// offsets, and checks the indices of its bags -- one contiguous range of
// positions -- finding each position's bag by a binary search over the
// repaired offsets in LDS.  Only the owner writes an offset; a neighbour that
// reads it before or after the repair computes the same o' (the maximum of a
// prefix is unchanged when some of its entries are replaced by their own
// prefix maxima), so no block waits on another.
#include <mutex>

#include "mx_common.h"
#include "scan.h"

// Scratch of mx_bounds_check_indices_noalloc: the per-tile offset maxima (at
// most 1024 tiles for any batch), one copy per device, held until the process
// ends.  Host code never passes this name to a kernel (on the host it is a
// stand-in, not a device address): it uses the address hipGetSymbolAddress
// returns for the current device.
static __device__ __align__(256) uint32_t scratch[1024];

namespace mx {
namespace {

constexpr int kMaxBagsPerBlock = 256;
constexpr int kIdxPerThread = 4;  // index loads in flight per thread

template <typename I>
__device__ __forceinline__ uint32_t clamp_off(I v, int64_t N) {
  const int64_t x = static_cast<int64_t>(v);
  return static_cast<uint32_t>(x < 0 ? 0 : (x > N ? N : x));
}

__device__ __forceinline__ uint32_t umax(uint32_t a, uint32_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint32_t wave_max(uint32_t v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = umax(v, __shfl_xor(v, m, 64));
  return v;
}

template <typename I>
__global__ void __launch_bounds__(256)
    tile_max_kernel(const I* __restrict__ offsets, int64_t nbags, int64_t N, int64_t tile,
                    int64_t ntiles, uint32_t* __restrict__ tilemax) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (t >= ntiles) return;  // whole waves only; no block barrier below
  const int lane = threadIdx.x & 63;
  const int64_t e0 = t * tile;
  const int64_t e1 = e0 + tile < nbags ? e0 + tile : nbags;
  uint32_t m = 0;
#pragma unroll 4
  for (int64_t i = e0 + lane; i < e1; i += 64) m = umax(m, clamp_off(offsets[i], N));
  m = wave_max(m);
  if (lane == 0) tilemax[t] = m;
}

template <typename I>
__global__ void __launch_bounds__(256)
    bounds_main_kernel(const int64_t* __restrict__ rows, I* __restrict__ indices,
                       I* __restrict__ offsets, int64_t nbags, int64_t B,
                       const int32_t* __restrict__ B_offsets, int32_t T, int64_t N,
                       int32_t mode, unsigned long long* __restrict__ warning,
                       const uint32_t* __restrict__ tilemax, int64_t tile, int32_t bpb) {
  __shared__ uint32_t s_red[4];
  __shared__ uint32_t s_wmax[4];
  __shared__ uint32_t s_rep[kMaxBagsPerBlock + 1];
  __shared__ int64_t s_lim[kMaxBagsPerBlock];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t b0 = static_cast<int64_t>(blockIdx.x) * bpb;
  const int64_t b1 = b0 + bpb < nbags ? b0 + bpb : nbags;
  const int nb = static_cast<int>(b1 - b0);
  const bool fix = mode != MX_BOUNDS_FATAL;
  uint32_t nbad = 0;
  // Carry: max clamp(o[j]) over j < b0 -- whole tiles, then the rest of b0's tile.
  const int64_t tb = b0 / tile;
  uint32_t carry = 0;
  for (int64_t t = tid; t < tb; t += 256) carry = umax(carry, tilemax[t]);
  for (int64_t j = tb * tile + tid; j < b0; j += 256) carry = umax(carry, clamp_off(offsets[j], N));
  carry = wave_max(carry);
  if (lane == 0) s_red[w] = carry;
  // This thread's bag: its offset and its table's row count.
  const bool mine = tid < nb;
  const int64_t bag = b0 + tid;
  const I orig = mine ? offsets[bag] : I(0);
  if (mine) {
    int64_t t;
    if (B_offsets) {  // last table whose first bag is <= bag
      int32_t lo = 0, hi = T;
      while (hi - lo > 1) {
        const int32_t mid = lo + ((hi - lo) >> 1);
        if (B_offsets[mid] <= bag)
          lo = mid;
        else
          hi = mid;
      }
      t = lo;
    } else {
      t = bag / B;
    }
    s_lim[tid] = rows[t];
  }
  const uint32_t v = wave_incl_scan<MaxOp>(mine ? clamp_off(orig, N) : 0u);
  if (lane == 63) s_wmax[w] = v;
  __syncthreads();
  carry = umax(umax(s_red[0], s_red[1]), umax(s_red[2], s_red[3]));
  uint32_t before = carry;
  for (int k = 0; k < w; ++k) before = umax(before, s_wmax[k]);
  const uint32_t rep = umax(v, before);
  if (mine) {
    s_rep[tid] = rep;
    if (static_cast<int64_t>(orig) != static_cast<int64_t>(rep)) {
      ++nbad;
      if (fix) offsets[bag] = static_cast<I>(rep);
    }
  }
  if (tid == 0) {
    // o'[b1]: entry b1 is the next block's first offset (read either before
    // or after its owner repairs it: same o') or, in the last block, the
    // final offset, which this thread owns.
    const uint32_t all = umax(carry, umax(umax(s_wmax[0], s_wmax[1]), umax(s_wmax[2], s_wmax[3])));
    const I e = offsets[b1];
    const uint32_t r = umax(all, clamp_off(e, N));
    s_rep[nb] = r;
    if (b1 == nbags && static_cast<int64_t>(e) != static_cast<int64_t>(r)) {
      ++nbad;
      if (fix) offsets[b1] = static_cast<I>(r);
    }
  }
  __syncthreads();
  // Indices of the block's bags: positions [o'[b0], o'[b1]).
  const int64_t p0 = s_rep[0], p1 = s_rep[nb];
  for (int64_t base = p0; base < p1; base += 256 * kIdxPerThread) {
    I idx[kIdxPerThread];
#pragma unroll
    for (int k = 0; k < kIdxPerThread; ++k) {
      const int64_t l = base + k * 256 + tid;
      idx[k] = l < p1 ? indices[l] : I(0);
    }
#pragma unroll
    for (int k = 0; k < kIdxPerThread; ++k) {
      const int64_t l = base + k * 256 + tid;
      if (l >= p1) break;
      int lo = 0, hi = nb;  // s_rep[lo] <= l < s_rep[hi]
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (static_cast<int64_t>(s_rep[mid]) <= l)
          lo = mid;
        else
          hi = mid;
      }
      const int64_t x = static_cast<int64_t>(idx[k]);
      if (x < 0 || x >= s_lim[lo]) {
        ++nbad;
        if (fix) indices[l] = static_cast<I>(0);
      }
    }
  }
  unsigned long long total = nbad;
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) total += __shfl_xor(total, m, 64);
  if (lane == 0 && total) atomicAdd(warning, total);
}

struct BoundsWs {
  uint32_t* tilemax;
  int64_t tile;    // bags per tile: a power of two >= 256, so a block's bags share one tile
  int64_t ntiles;  // at most 1024 (bounded carry work per block)
  size_t bytes;
};

BoundsWs carve_bounds(uint8_t* base, int64_t nbags) {
  BoundsWs w{};
  int64_t tile = 256;
  while (ceil_div(nbags, tile) > 1024) tile *= 2;
  w.tile = tile;
  w.ntiles = ceil_div(nbags > 0 ? nbags : 1, tile);
  w.tilemax = reinterpret_cast<uint32_t*>(base);
  w.bytes = (static_cast<size_t>(w.ntiles) * 4 + 255) & ~size_t(255);
  return w;
}

template <typename I>
int run_bounds(const int64_t* rows, void* indices, void* offsets, int64_t nbags, int64_t B,
               const int32_t* B_offsets, int32_t T, int64_t N, int32_t mode,
               unsigned long long* warning, const BoundsWs& w, hipStream_t s) {
  // Bags per block: about one pass of index loads (1024 positions) per block
  // at the batch's mean pooling factor, between 32 and 256 bags.
  int32_t bpb = kMaxBagsPerBlock;
  while (bpb > 32 && bpb * N > 256 * kIdxPerThread * nbags) bpb >>= 1;
  tile_max_kernel<I><<<dim3(static_cast<uint32_t>(ceil_div(w.ntiles, 4))), 256, 0, s>>>(
      static_cast<const I*>(offsets), nbags, N, w.tile, w.ntiles, w.tilemax);
  MX_LAUNCH_CHECK();
  bounds_main_kernel<I><<<dim3(static_cast<uint32_t>(ceil_div(nbags, bpb))), 256, 0, s>>>(
      rows, static_cast<I*>(indices), static_cast<I*>(offsets), nbags, B, B_offsets, T, N, mode,
      warning, w.tilemax, w.tile, bpb);
  MX_LAUNCH_CHECK();
  return MX_OK;
}

}  // namespace
}  // namespace mx

using namespace mx;

extern "C" size_t mx_bounds_check_workspace_bytes(int32_t T, int64_t B) {
  if (T < 0 || B < 0) return 0;
  return carve_bounds(nullptr, static_cast<int64_t>(T) * B).bytes;
}

namespace {

int bounds_impl(const int64_t* rows_per_table, int32_t T, int64_t B, int64_t nbags,
                const int32_t* B_offsets, void* indices, void* offsets, int32_t index_bytes,
                int64_t N, int32_t mode, int64_t* warning, void* workspace,
                size_t workspace_bytes, void* stream) {
  MX_REQUIRE(T >= 0 && B >= 0 && N >= 0 && nbags >= 0, "negative size");
  MX_REQUIRE(index_bytes == 4 || index_bytes == 8, "indices must be int32 or int64");
  MX_REQUIRE(mode >= MX_BOUNDS_FATAL && mode <= MX_BOUNDS_NONE, "bounds_check_mode %d invalid",
             mode);
  if (mode == MX_BOUNDS_NONE || nbags == 0) return MX_OK;
  MX_REQUIRE(N < (int64_t(1) << 32), "N %lld above 2^32 indices", (long long)N);
  MX_REQUIRE(rows_per_table && offsets && warning && (indices || N == 0), "null pointer argument");
  MX_REQUIRE(ceil_div(nbags, 32) <= 0x7fffffffll, "too many bags");
  const BoundsWs w = carve_bounds(static_cast<uint8_t*>(workspace), nbags);
  if (workspace == nullptr || workspace_bytes < w.bytes)
    return set_error(MX_EWORKSPACE, "workspace of %zu bytes needed", w.bytes);
  auto* wc = reinterpret_cast<unsigned long long*>(warning);
  auto* s = as_stream(stream);
  return index_bytes == 8 ? run_bounds<int64_t>(rows_per_table, indices, offsets, nbags, B,
                                                B_offsets, T, N, mode, wc, w, s)
                          : run_bounds<int32_t>(rows_per_table, indices, offsets, nbags, B,
                                                B_offsets, T, N, mode, wc, w, s);
}

}  // namespace

extern "C" int mx_bounds_check_indices(const int64_t* rows_per_table, int32_t T, int64_t B,
                                       void* indices, void* offsets, int32_t index_bytes,
                                       int64_t N, int32_t mode, int64_t* warning,
                                       void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  return bounds_impl(rows_per_table, T, B, static_cast<int64_t>(T) * B, nullptr, indices,
                     offsets, index_bytes, N, mode, warning, workspace, workspace_bytes, stream);
}

namespace {

std::mutex g_scratch_mu;
void* g_scratch_dev[64] = {};

// Device address of `scratch` on the current device, looked up on the
// device's first call (with that device current) and kept.
int scratch_address(void** out) {
  int dev = 0;
  MX_HIP_CHECK(hipGetDevice(&dev));
  MX_REQUIRE(dev >= 0 && dev < 64, "device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_dev[dev] == nullptr) {
    void* p = nullptr;
    MX_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    MX_REQUIRE(p != nullptr, "no device address for the bounds-check scratch");
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return MX_OK;
}

}  // namespace

extern "C" int mx_bounds_check_indices_noalloc(const int64_t* rows_per_table, int32_t T,
                                               int64_t B, void* indices, void* offsets,
                                               int32_t index_bytes, int64_t N, int32_t mode,
                                               int64_t* warning, void* stream) {
  clear_error();
  MX_REQUIRE(T >= 0 && B >= 0, "negative size");
  const int64_t nbags = static_cast<int64_t>(T) * B;
  const size_t need = carve_bounds(nullptr, nbags).bytes;
  if (need > sizeof(scratch))
    return set_error(MX_EWORKSPACE,
                     "T*B = %lld bags need %zu bytes of scratch, above the %zu bytes this entry "
                     "point holds; use mx_bounds_check_indices with a workspace",
                     (long long)nbags, need, sizeof(scratch));
  void* ws = nullptr;
  if (int rc = scratch_address(&ws)) return rc;
  // Every tile maximum the main kernel reads is written by the tile kernel of
  // the same call first, so the scratch needs no clearing.
  return bounds_impl(rows_per_table, T, B, nbags, nullptr, indices, offsets, index_bytes, N,
                     mode, warning, ws, sizeof(scratch), stream);
}

extern "C" size_t mx_bounds_check_workspace_bytes_vbe(int64_t total_B) {
  if (total_B < 0) return 0;
  return carve_bounds(nullptr, total_B).bytes;
}

extern "C" int mx_bounds_check_indices_vbe(const int64_t* rows_per_table, int32_t T,
                                           int64_t total_B, const int32_t* B_offsets,
                                           void* indices, void* offsets, int32_t index_bytes,
                                           int64_t N, int32_t mode, int64_t* warning,
                                           void* workspace, size_t workspace_bytes,
                                           void* stream) {
  clear_error();
  MX_REQUIRE(T >= 1 && (total_B == 0 || B_offsets), "VBE needs B_offsets [T+1]");
  return bounds_impl(rows_per_table, T, 0, total_B, B_offsets, indices, offsets, index_bytes, N,
                     mode, warning, workspace, workspace_bytes, stream);
}
