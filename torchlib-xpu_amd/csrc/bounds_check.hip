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
// Work: one max-scan (decoupled look-back) builds o' in the workspace, then
// entry-parallel kernels compare/repair offsets and check every index against
// the table of the bag found by binary search over o'.  Thread i owns
// offsets[i] or indices[i], so repairs never race.
#include "mx_common.h"
#include "scan.h"

namespace mx {
namespace {

template <typename I>
struct ClampedOffset {
  const I* off;
  int64_t N;
  __device__ uint32_t operator()(int64_t i) const {
    const int64_t x = static_cast<int64_t>(off[i]);
    return static_cast<uint32_t>(x < 0 ? 0 : (x > N ? N : x));
  }
};

__device__ __forceinline__ void count_bad(uint32_t bad, unsigned long long* warning) {
  const unsigned long long nbad = __popcll(__ballot(bad));
  if ((threadIdx.x & 63) == 0 && nbad) atomicAdd(warning, nbad);
}

template <typename I>
__global__ void __launch_bounds__(256)
    fix_offsets_kernel(I* __restrict__ offsets, const uint32_t* __restrict__ rep, int64_t n_off,
                       int32_t mode, unsigned long long* __restrict__ warning) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  uint32_t bad = 0;
  if (i < n_off) {
    const int64_t r = rep[i];
    if (r != static_cast<int64_t>(offsets[i])) {
      bad = 1;
      if (mode != MX_BOUNDS_FATAL) offsets[i] = static_cast<I>(r);
    }
  }
  count_bad(bad, warning);
}

template <typename I>
__global__ void __launch_bounds__(256)
    check_indices_kernel(const int64_t* __restrict__ rows, I* __restrict__ indices,
                         const uint32_t* __restrict__ rep, int64_t nbags, int64_t B,
                         const int32_t* __restrict__ B_offsets, int32_t T, int64_t N,
                         int32_t mode, unsigned long long* __restrict__ warning) {
  const int64_t l = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  uint32_t bad = 0;
  if (l < N && l >= rep[0] && l < rep[nbags]) {  // positions no bag covers are never read
    int64_t lo = 0, hi = nbags;  // rep[lo] <= l < rep[hi]
    while (hi - lo > 1) {
      const int64_t mid = lo + ((hi - lo) >> 1);
      if (static_cast<int64_t>(rep[mid]) <= l)
        lo = mid;
      else
        hi = mid;
    }
    int64_t t;
    if (B_offsets) {  // last table whose first bag is <= lo
      int32_t tl = 0, th = T;
      while (th - tl > 1) {
        const int32_t mid = tl + ((th - tl) >> 1);
        if (B_offsets[mid] <= lo)
          tl = mid;
        else
          th = mid;
      }
      t = tl;
    } else {
      t = lo / B;
    }
    const int64_t idx = static_cast<int64_t>(indices[l]);
    if (idx < 0 || idx >= rows[t]) {
      bad = 1;
      if (mode != MX_BOUNDS_FATAL) indices[l] = static_cast<I>(0);
    }
  }
  count_bad(bad, warning);
}

struct BoundsWs {
  unsigned long long* state;
  int64_t state_words;
  uint32_t* rep;
  size_t bytes;
};

BoundsWs carve_bounds(uint8_t* base, int64_t n_off) {
  BoundsWs w{};
  w.state_words = scan_tiles(n_off) + 2;
  const size_t state_bytes = (static_cast<size_t>(w.state_words) * 8 + 255) & ~size_t(255);
  w.state = reinterpret_cast<unsigned long long*>(base);
  w.rep = reinterpret_cast<uint32_t*>(base ? base + state_bytes : nullptr);
  w.bytes = state_bytes + ((static_cast<size_t>(n_off) * 4 + 255) & ~size_t(255));
  return w;
}

template <typename I>
int run_bounds(const int64_t* rows, void* indices, void* offsets, int64_t nbags, int64_t B,
               const int32_t* B_offsets, int32_t T, int64_t N, int32_t mode,
               unsigned long long* warning, const BoundsWs& w, hipStream_t s) {
  const int64_t n_off = nbags + 1;
  zero_u64_kernel<<<1, 256, 0, s>>>(w.state, w.state_words);
  MX_LAUNCH_CHECK();
  const ScanState st{w.state, reinterpret_cast<unsigned int*>(w.state + w.state_words - 1)};
  if (int rc = prefix_scan<ClampedOffset<I>, MaxOp, true>(
          ClampedOffset<I>{static_cast<const I*>(offsets), N}, n_off, nullptr, w.rep, nullptr, st,
          s))
    return rc;
  if (N > 0) {
    check_indices_kernel<I><<<dim3(static_cast<uint32_t>(ceil_div(N, 256))), 256, 0, s>>>(
        rows, static_cast<I*>(indices), w.rep, nbags, B, B_offsets, T, N, mode, warning);
    MX_LAUNCH_CHECK();
  }
  fix_offsets_kernel<I><<<dim3(static_cast<uint32_t>(ceil_div(n_off, 256))), 256, 0, s>>>(
      static_cast<I*>(offsets), w.rep, n_off, mode, warning);
  MX_LAUNCH_CHECK();
  return MX_OK;
}

}  // namespace
}  // namespace mx

using namespace mx;

extern "C" size_t mx_bounds_check_workspace_bytes(int32_t T, int64_t B) {
  if (T < 0 || B < 0) return 0;
  return carve_bounds(nullptr, static_cast<int64_t>(T) * B + 1).bytes;
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
  MX_REQUIRE(ceil_div(N, 256) <= 0x7fffffffll && ceil_div(nbags + 1, 256) <= 0x7fffffffll,
             "too many indices or bags");
  const BoundsWs w = carve_bounds(static_cast<uint8_t*>(workspace), nbags + 1);
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

extern "C" size_t mx_bounds_check_workspace_bytes_vbe(int64_t total_B) {
  if (total_B < 0) return 0;
  return carve_bounds(nullptr, total_B + 1).bytes;
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
