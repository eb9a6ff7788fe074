// Device-wide prefix scan of 32-bit values produced by a functor, in one
// launch (decoupled look-back), for an associative operator (sum or max).
// The effective length may live on the device (`n_dev`, e.g. a run count),
// so no host synchronisation is needed; `n` is the host-side upper bound that
// sizes the grid.
#pragma once

#include "mx_common.h"

namespace mx {

// 3072-element tiles (2048: +2.4 us, 4096: +2.8 us on 668k) in blocks of 16
// waves with 3 elements per lane: more waves per SIMD hide the dependent
// loads (config 3's run-head scan: 10.8 us with 4 waves of 12, 9.4 with 8 of
// 6, 9.0 with 16 of 3).
constexpr int kScanThreads = 1024;
constexpr int kScanItems = 3;
constexpr int64_t kScanTile = kScanThreads * kScanItems;

inline int64_t scan_tiles(int64_t n) { return ceil_div(n > 0 ? n : 1, kScanTile); }

struct SumOp {
  static __device__ __forceinline__ uint32_t identity() { return 0u; }
  static __device__ __forceinline__ uint32_t apply(uint32_t a, uint32_t b) { return a + b; }
};

struct MaxOp {
  static __device__ __forceinline__ uint32_t identity() { return 0u; }
  static __device__ __forceinline__ uint32_t apply(uint32_t a, uint32_t b) { return a > b ? a : b; }
};

// Inclusive scan over the 64 lanes of a wave.
template <class Op = SumOp>
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t o = __shfl_up(v, d, 64);
    if (lane >= d) v = Op::apply(o, v);
  }
  return v;
}

// Exclusive scan across a block of kScanThreads threads; returns the block aggregate in *total.
template <class Op = SumOp>
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t* total) {
  __shared__ uint32_t wsum[kScanThreads / 64];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const uint32_t incl = wave_incl_scan<Op>(v);
  if (lane == 63) wsum[w] = incl;
  __syncthreads();
  uint32_t before = Op::identity(), all = Op::identity();
#pragma unroll
  for (int i = 0; i < kScanThreads / 64; ++i) {
    if (i < w) before = Op::apply(before, wsum[i]);
    all = Op::apply(all, wsum[i]);
  }
  __syncthreads();
  *total = all;
  // Exclusive value of this lane: the inclusive scan of the previous lane.
  const uint32_t prev = __shfl_up(incl, 1, 64);
  return lane == 0 ? before : Op::apply(before, prev);
}

__device__ __forceinline__ int64_t eff_len(int64_t n, const int32_t* n_dev) {
  if (n_dev == nullptr) return n;
  const int64_t m = *n_dev;
  return m < n ? m : n;
}

// Single-pass scan with decoupled look-back.  Tiles take a ticket in launch
// order, publish their aggregate, then walk back over predecessors' status
// words (aggregate or inclusive prefix, packed with the value in one 64-bit
// word) until an inclusive prefix is found.  A tile only waits on tiles that
// took earlier tickets, which are already running and publish their
// aggregate before they wait themselves, so every wait ends.  The status
// words and the ticket must be zero before the launch.
// A look-back that exhausts its spin bound (never expected: a predecessor
// holds an earlier ticket and publishes without waiting) marks the call as
// failed: `fail` is a word of the call's zeroed workspace that every later
// kernel of the call checks before it uses the results, and `mailbox`, when
// the caller registered one for the device, is a host-visible word through
// which the failure reaches the host.  Partial prefixes are never larger than
// the true ones, so the stores made before the check stay in bounds.
struct Faults {
  unsigned int* fail;
  unsigned int* mailbox;  // the device's MX_STATUS_WORDS host-visible words, may be null
  int spin_limit;         // > 0: spins before giving up; < 0: give up at once (test hook)
};

__device__ __forceinline__ void report_fault(const Faults& f) {
  __hip_atomic_store(f.fail, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (f.mailbox)
    __hip_atomic_store(f.mailbox + MX_STATUS_LOOKBACK, 1u, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_SYSTEM);
}

// True when a kernel of the call gave up.  Uniform across a block only when
// the word was set by an earlier launch; a kernel whose own tiles may set it
// reads it once per block (one thread, broadcast through LDS).
__device__ __forceinline__ bool call_failed(const unsigned int* fail) {
  return fail != nullptr &&
         __hip_atomic_load(fail, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u;
}

// One more spin of a bounded wait; false once the wait must give up.
__device__ __forceinline__ bool keep_waiting(int& spins, const Faults& f) {
  if (++spins > f.spin_limit) return false;
  __builtin_amdgcn_s_sleep(1);
  return true;
}

struct ScanState {
  unsigned long long* status;  // one word per tile
  unsigned int* ticket;        // [0] next tile
  Faults faults;
};

constexpr unsigned long long kScanFlagAgg = 1ull << 62;
constexpr unsigned long long kScanFlagIncl = 2ull << 62;
constexpr int kScanSpinLimit = 1 << 22;

// INCL = false: epi(i, op(f(0..i-1)), f(i)) (identity at 0); true: epi(i, op(f(0..i)), f(i)).
// epi.total(aggregate) runs once, in the last tile.  An epilogue is a
// functor with operator()(int64_t i, uint32_t scanned, uint32_t value) and
// total(uint32_t); `value` is f(i), so the epilogue need not recompute it.
template <class F, class Op, bool INCL, class Epi>
__global__ void __launch_bounds__(kScanThreads)
    scan_onepass_kernel(F f, int64_t n, const int32_t* n_dev, Epi epi, ScanState st,
                        int64_t ntiles) {
  (void)ntiles;
  __shared__ uint32_t s_tile, s_prefix;
  __shared__ bool s_gave_up, s_failed;
  // One thread reads the failure word and takes the ticket, so that every
  // wave of the block sees the same answer: another tile of this launch may
  // set the word while the block starts.  A block that finds the call failed
  // takes no ticket; every tile that took one publishes, so no tile waits on it.
  if (threadIdx.x == 0) {
    s_failed = call_failed(st.faults.fail);  // the input of this scan is not valid
    if (!s_failed) s_tile = atomicAdd(st.ticket, 1u);
    s_gave_up = false;
  }
  __syncthreads();
  if (s_failed) return;  // block-uniform
  const int64_t tile = s_tile;
  const int64_t m = eff_len(n, n_dev);
  // Tiles past the effective length hold only identities: they return at once
  // (later tiles are past it too, so nobody looks back at them) and the tile
  // holding element m-1 (tile 0 when m == 0) reports the total.
  const int64_t last = m > 0 ? (m - 1) / kScanTile : 0;
  if (tile > last) return;  // block-uniform
  const int64_t base = tile * kScanTile + threadIdx.x * kScanItems;
  uint32_t v[kScanItems];
  uint32_t agg = Op::identity();
#pragma unroll
  for (int it = 0; it < kScanItems; ++it) {
    const int64_t i = base + it;
    v[it] = i < m ? f(i) : Op::identity();
    agg = Op::apply(agg, v[it]);
  }
  uint32_t tile_total;
  const uint32_t excl = block_excl_scan<Op>(agg, &tile_total);
  if (threadIdx.x < 64) {  // wave 0 looks back 64 predecessors at a time
    const int lane = threadIdx.x;
    uint32_t prefix = Op::identity();
    if (tile == 0) {
      if (lane == 0)
        __hip_atomic_store(&st.status[0], kScanFlagIncl | tile_total, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    } else {
      if (lane == 0)
        __hip_atomic_store(&st.status[tile], kScanFlagAgg | tile_total, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      int64_t j = tile - 1;  // nearest predecessor not yet folded in
      int spins = 0;
      while (true) {
        if (st.faults.spin_limit < 0) {  // test hook: give up at once
          if (lane == 0) {
            report_fault(st.faults);
            s_gave_up = true;
          }
          break;
        }
        const int64_t idx = j - lane;
        const unsigned long long w =
            idx >= 0 ? __hip_atomic_load(&st.status[idx], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                     : (kScanFlagIncl | Op::identity());  // before tile 0
        const unsigned long long flag = w >> 62;
        if (__ballot(flag == 0) != 0ull) {  // some predecessor has not published yet
          if (!keep_waiting(spins, st.faults)) {  // never expected; keeps the wait bounded
            if (lane == 0) {
              report_fault(st.faults);
              s_gave_up = true;
            }
            break;
          }
          continue;
        }
        const unsigned long long incl = __ballot(flag == 2);
        // Fold lanes up to (and including) the nearest inclusive prefix.
        const int stop = incl ? __builtin_ctzll(incl) : 63;
        uint32_t x = lane <= stop ? static_cast<uint32_t>(w) : Op::identity();
#pragma unroll
        for (int mm = 32; mm >= 1; mm >>= 1) x = Op::apply(x, __shfl_xor(x, mm, 64));
        prefix = Op::apply(x, prefix);
        if (incl) break;
        j -= 64;
      }
      if (lane == 0)
        __hip_atomic_store(&st.status[tile], kScanFlagIncl | Op::apply(prefix, tile_total),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (lane == 0) {
      s_prefix = prefix;
      if (tile == last && !s_gave_up) epi.total(Op::apply(prefix, tile_total));
    }
  }
  __syncthreads();
  if (s_gave_up) return;  // block-uniform; later kernels see the failure
  uint32_t run = Op::apply(s_prefix, excl);
#pragma unroll
  for (int it = 0; it < kScanItems; ++it) {
    const int64_t i = base + it;
    if constexpr (INCL) run = Op::apply(run, v[it]);
    if (i < m) epi(i, run, v[it]);
    if constexpr (!INCL) run = Op::apply(run, v[it]);
  }
}

// Prefix scan of f over [0, effective length), results handed to `epi`.
// `st` must have scan_tiles(n) zeroed status words and a zeroed ticket.
template <class F, class Op = SumOp, bool INCL = false, class Epi>
int prefix_scan_epi(F f, int64_t n, const int32_t* n_dev, Epi epi, ScanState st,
                    hipStream_t s) {
  const int64_t nt = scan_tiles(n);
  if (nt > 0x7fffffffll) return set_error(MX_EINVAL, "scan too long");
  scan_onepass_kernel<F, Op, INCL, Epi><<<dim3(static_cast<uint32_t>(nt)), kScanThreads, 0, s>>>(
      f, n, n_dev, epi, st, nt);
  MX_LAUNCH_CHECK();
  return MX_OK;
}

// Fills p[0..n) with zeros (a kernel, not a memset, so callers can capture it).
__global__ void zero_u64_kernel(unsigned long long* p, int64_t n);

}  // namespace mx
