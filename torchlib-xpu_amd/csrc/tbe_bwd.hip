// TBE backward for gfx950: transpose_embedding_input (linearize, stable LSD
// radix sort of (key, info) pairs, run-length encoding) and the fused
// segment-reduce + exact rowwise-Adagrad update.
//
// Semantics: fbgemm_gpu transpose_embedding_input (upstream
// src/split_embeddings_utils/, recalled) and
// split_embedding_backward_codegen_rowwise_adagrad_unweighted_exact_cuda with
// the rowwise_adagrad update rule of upstream codegen/genscript/optimizers.py
// (recalled; textbook rowwise Adagrad):
//   h += mean_d(g_d^2);  m = lr / (sqrt(h) + eps);  w = c*w - m*g.
//
// Design:
//  * Keys fit 32 bits whenever total_hash_size_bits <= 32, so the sort moves
//    (u32 key, u32 info) pairs: ceil(bits/8) LSD passes of 8-bit digits.
//  * linearize: a block takes 1024 consecutive positions, finds the bag range
//    they span with two cooperative 128-ary searches, lets every non-empty
//    bag mark its first position in LDS and gives each position the latest
//    mark (a max-scan), so no per-position search.  The same kernel
//    accumulates the digit counts of every pass (LDS, then one atomic per bin
//    and block into its XCD's copy): per feature for a fixed batch of at most
//    kSegMaxT features (a global sort, when some key lies outside its table's
//    range, sums them), else for the whole batch.  Those counts start at
//    zero: an eager backward keeps them in a region of its stream that its
//    update launch clears for the next call; other calls keep them in the
//    workspace and clear them with one more kernel.
//  * One launch per pass ("onesweep"): a block of 16 waves ranks a 3072-key
//    tile (each wave 192 keys, 64 at a time, stable ranks from 8 ballots),
//    then thread d finds how many keys of digit d earlier tiles of its
//    segment (its feature's keys, or the whole batch) hold through a
//    decoupled look-back over per-(tile, digit) status words, and the tile
//    scatters.  Tiles take tickets in launch order, so every wait ends.
//  * Run-length encoding is a head-flag scan whose epilogue writes the run
//    keys and offsets.
//  * Each run (one distinct (t, i)) is reduced by one G-lane group, lanes
//    owning columns, occurrences added in sorted order.  Runs longer than
//    kLong are cut into kChunk-occurrence chunks reduced in parallel into a
//    workspace, then summed in chunk order.  No atomics on data: results are
//    deterministic.  Runs and chunks are split into one contiguous key range
//    per XCD, so an XCD re-reads only its tables' gradient columns, from its
//    own L2.
#include <map>
#include <memory>
#include <mutex>
#include <type_traits>
#include <utility>

#include "mx_common.h"
#include "scan.h"

namespace mx {

namespace {

constexpr int kRadixBits = 8;
constexpr int kRadix = 1 << kRadixBits;
constexpr int kMaxPasses = 4;
// The digit histograms are kept in one copy per XCD (a linearize block adds
// into the copy of the XCD it runs on, block i on XCD i % 8), so that the
// blocks' device-scope atomics spread over 8x more counters; a sort pass sums
// the copies of its digit.
constexpr int kHistCopies = 8;
constexpr int64_t kHistCopyWords = kMaxPasses * kRadix;
// 3072-key tiles: 218 tiles for config 3's 668k keys, one per CU.  A wave
// ranks its keys with one ballot per digit bit and one LDS count update per
// key, a chain of dependent latencies: 16 waves of 3 keys per lane (4 per
// SIMD) hide what 4 waves of 12 did not (load and rank 5.2 -> 2.2 us per
// tile, each pass 19.9 -> 17.2 us on config 3).  2048-key tiles lose ~2 us
// per pass; 4096-key tiles are no faster and 6144-key ones slower (the
// shorter look-back saves less than the longer ranking costs).
constexpr int kSweepWaves = 16;                                // waves per sort block
constexpr int kSweepThreads = 64 * kSweepWaves;
constexpr int kSweepItems = 3;                                 // keys per lane per pass
constexpr int64_t kSweepWaveKeys = 64 * kSweepItems;
constexpr int64_t kSweepTile = kSweepWaves * kSweepWaveKeys;  // keys per block
static_assert(kSweepThreads >= 256, "the first 256 threads own one digit each");
// 1024-position linearize blocks: 654 blocks on config 3, 2-3 per CU, whose
// dependent search and marking loads overlap (11.8 -> 10.5 us against 2048).
constexpr int kLinItems = 4;
// Segmented sort: at most this many features (one segment each); their digit
// counts are kept in one copy per XCD, like the batch's.
constexpr int kSegMaxT = 63;
constexpr int64_t kSegRow = static_cast<int64_t>(kHistCopies) * kMaxPasses * kRadix;  // per feature
constexpr int64_t kLinTile = 256 * kLinItems;         // positions per linearize block
// Runs longer than kLong are chunked.  A wave's four short runs last as long
// as the longest (two occurrences per round): 24 instead of 32 moves the
// 13-16-round runs to the chunk path (config 3: 161.1 -> 158.8 us; 12, 16 and
// 20 were within 1 us of it, 8 slower).
constexpr int kLong = 24;
constexpr int kChunk = 32;                            // occurrences per chunk
// One-pass scans per backward: run heads, chunk layout.
constexpr int kScanSlots = 2;
// Upper bound of the chunk count: sum over runs longer than kLong of
// ceil(len / kChunk) <= N / kChunk + (number of such runs).
int64_t max_chunks(int64_t N) { return N / kChunk + N / (kLong + 1) + 2; }

__device__ __forceinline__ uint32_t digit_mask(int bits, int p) {
  const int nb = bits - p * kRadixBits;
  return nb >= kRadixBits ? (kRadix - 1u) : ((1u << nb) - 1u);
}

// ---- segments -------------------------------------------------------------

// The sort's segments, one per feature of a batch with at most kSegMaxT
// features (a fixed batch, or a variable one whose B_off gives each feature's
// first bag), or per run of consecutive features with equal hsc (features that
// share one table).  When hsc does not decrease, hsc[T] <= 2^bits and every
// key of a segment lies in [its hsc, the next segment's hsc), all keys of a
// segment precede those of the next: sorting each segment's positions on its
// own gives the global order, each segment's tiles (segments start at tile
// boundaries) look back only over tiles of their own segment, and the chains
// are ~S times shorter.  Linearize checks hsc in every block: when it
// decreases (features sharing tables out of order) or hsc[T] > 2^bits, it
// counts the whole batch's digits and sets `bad` to kSegTables.  Otherwise it
// writes fpos and tprefix (per segment; entries S+1 .. T repeat the end),
// counts each segment's digits, and sets `bad` to kSegKeys if a key lies
// outside its table's range; the passes then sort globally, summing the
// per-segment counts.
constexpr unsigned int kSegKeys = 1u;    // a key outside its table's range
constexpr unsigned int kSegTables = 2u;  // hsc decreases, or exceeds 2^bits
struct SegSort {
  int64_t* fpos;         // [T + 1] first position of each segment
  int32_t* tprefix;      // [T + 1] first tile of each segment
  uint32_t* fhist;       // [T][kHistCopies][kMaxPasses][kRadix] per-segment digit counts (zeroed), a pass's row
  unsigned int* bad;     // zeroed; nonzero (kSegKeys or kSegTables): sort globally
  int32_t T;             // 0: no segments
  const int32_t* B_off;  // [T + 1] first bag of each feature (variable batch); null: t * B
};

// ---- linearize ------------------------------------------------------------

// A block takes kLinTile consecutive positions; wave w owns positions
// [w * kLinTile / 4, (w + 1) * kLinTile / 4), 64 consecutive ones per item.
constexpr int kLinWavePos = kLinTile / 4;

template <typename I>
__global__ void __launch_bounds__(256)
    linearize_kernel(const int64_t* __restrict__ hsc, const I* __restrict__ indices,
                     const I* __restrict__ offsets, int64_t nbags, int64_t B, int32_t nb,
                     const int32_t* __restrict__ b_t_map, int64_t N, int32_t bits,
                     int32_t passes, int64_t* __restrict__ linear_out,
                     uint32_t* __restrict__ keys, uint32_t* __restrict__ vals,
                     const float* __restrict__ iw, uint32_t* __restrict__ vals2,
                     uint32_t* __restrict__ ghist, unsigned long long* __restrict__ zero,
                     int64_t zero_words, SegSort seg) {
  __shared__ uint32_t s_mark[kLinTile];  // bag (relative to blo) starting at each position
  __shared__ uint32_t hf[2][kMaxPasses][kRadix];  // digit counts of the block's first two features
  __shared__ int s_bad;
  __shared__ int s_tables_ok;  // hsc does not decrease and fits the bits (per-segment counts)
  __shared__ int s_ngroups;    // segments: runs of features with equal hsc (one table)
  __shared__ int64_t s_hsc[kSegMaxT + 1];  // hsc of a batch of at most kSegMaxT features
  __shared__ int32_t s_boff[kSegMaxT + 1]; // first bag of each feature (variable batch)
  __shared__ int64_t s_gend[kSegMaxT];     // feature t's table end: hsc of the next segment
  __shared__ int s_gid[kSegMaxT];          // feature t's segment
  __shared__ int s_gfirst[kSegMaxT + 1];   // segment g's first feature; [S] = T
  __shared__ int64_t s_range[2][2];      // [half][lo, hi] of the cooperative searches
  __shared__ uint32_t s_cnt[2][2];       // [half][wave of the half]
  __shared__ uint32_t s_wmax[4];
  __shared__ uint32_t h[kMaxPasses][kRadix];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t l0 = static_cast<int64_t>(blockIdx.x) * kLinTile;
  const int64_t lend = l0 + kLinTile < N ? l0 + kLinTile : N;
  const int64_t pbase = l0 + w * kLinWavePos + lane;  // item it: pbase + it * 64
  // The later kernels' zeroed state, spread over the grid.
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < zero_words;
       i += static_cast<int64_t>(gridDim.x) * 256)
    zero[i] = 0ull;
  I idx[kLinItems];
#pragma unroll
  for (int it = 0; it < kLinItems; ++it) {  // in flight during the searches below
    const int64_t l = pbase + it * 64;
    idx[it] = l < lend ? indices[l] : I(0);
  }
  // Wave 0 loads hsc (at most kSegMaxT + 1 entries) now and stages it in LDS
  // after the searches, when it has arrived.
  const int64_t lane_hsc = seg.T > 0 && w == 0 && lane <= seg.T ? hsc[lane] : 0;
  const int32_t lane_boff = seg.B_off && w == 0 && lane <= seg.T ? seg.B_off[lane] : 0;
  // Last bag with offsets[bag] <= target (0 when none), for the block's first
  // (half 0) and last (half 1) position: 128-ary searches, one probe per
  // thread and round, so ceil(log128(nbags)) dependent loads instead of
  // log2(nbags).  Invariant: offsets[lo] <= target < offsets[hi] (hi = nbags:
  // past the end).
  {
    const int half = threadIdx.x >> 7, q = threadIdx.x & 127;
    const int64_t target = half == 0 ? l0 : lend - 1;
    if (q == 0) {
      s_range[half][0] = 0;
      s_range[half][1] = nbags;
    }
    __syncthreads();
    while (true) {
      const int64_t lo = s_range[0][0], hi = s_range[0][1];
      const int64_t lo1 = s_range[1][0], hi1 = s_range[1][1];
      if (hi - lo <= 1 && hi1 - lo1 <= 1) break;  // block-uniform
      const int64_t mylo = half == 0 ? lo : lo1, myhi = half == 0 ? hi : hi1;
      const int64_t stride = (myhi - mylo + 127) / 128;
      const int64_t pos = mylo + q * stride;
      // Probe q = 0 is lo itself (true by the invariant); probes past hi are false.
      const bool le = myhi - mylo > 1 && pos < myhi &&
                      (q == 0 || static_cast<int64_t>(offsets[pos]) <= target);
      const uint64_t bal = __ballot(le);
      if (lane == 0) s_cnt[half][w & 1] = __popcll(bal);
      __syncthreads();
      if (q == 0 && myhi - mylo > 1) {
        const int64_t c = s_cnt[half][0] + s_cnt[half][1];  // probes 0..c-1 are <= target
        const int64_t nlo = mylo + (c - 1) * stride;
        const int64_t nhi = mylo + c * stride;
        s_range[half][0] = nlo;
        s_range[half][1] = nhi < myhi ? nhi : myhi;
      }
      __syncthreads();
    }
  }
  const int64_t blo = s_range[0][0], bhi = s_range[1][0];
  if (seg.T > 0 && w == 0) {  // hsc into LDS; segments; does hsc not decrease?
    const int64_t next = __shfl(lane_hsc, lane + 1 < 64 ? lane + 1 : 63, 64);
    const int64_t prev = __shfl(lane_hsc, lane > 0 ? lane - 1 : 0, 64);
    if (lane <= seg.T) {
      s_hsc[lane] = lane_hsc;
      s_boff[lane] = lane_boff;
    }
    // In-range keys must also fit the sorted bits (a sort over fewer bits
    // orders keys by their low bits, across features).
    const bool fits = lane != seg.T || bits >= 62 || lane_hsc <= (int64_t(1) << bits);
    const bool all_up = __all((lane >= seg.T || lane_hsc <= next) && fits);
    // Consecutive features with equal hsc share a table: one segment, whose
    // keys end at the next segment's hsc (hsc[T] for the last).
    const bool start = lane < seg.T && (lane == 0 || lane_hsc != prev);
    const uint64_t sm = __ballot(start);
    const uint64_t upto = (2ull << lane) - 1ull;  // lanes 0..lane
    const uint64_t above = sm & ~upto;
    const int nxt = above ? __ffsll(static_cast<long long>(above)) - 1 : seg.T;
    const int64_t gend = __shfl(lane_hsc, nxt, 64);
    const int gid = __popcll(sm & upto) - 1;
    if (lane < seg.T) {
      s_gid[lane] = gid;
      s_gend[lane] = gend;
    }
    if (start) s_gfirst[gid] = lane;
    if (lane == 0) {
      s_tables_ok = all_up ? 1 : 0;
      s_ngroups = __popcll(sm);
      s_gfirst[__popcll(sm)] = seg.T;
    }
  }
  // Digit counts per feature when segments are possible (their sum gives the
  // whole batch's if a key turns out to lie outside its feature), else the
  // whole batch's.  Both count arrays start at zero: which one is used is
  // known after the next barrier, which also publishes s_hsc and s_tables_ok.
  for (int i = threadIdx.x; i < 2 * kMaxPasses * kRadix; i += 256) (&hf[0][0][0])[i] = 0u;
  for (int i = threadIdx.x; i < kMaxPasses * kRadix; i += 256) (&h[0][0])[i] = 0u;
  // The block's first feature: its first bag's (checked below for a variable
  // batch, whose bags need not match a feature's B_off range).
  int64_t t_lo = 0;
  if (seg.T > 0) {
    t_lo = seg.B_off ? (nb >= 32 ? 0 : static_cast<int64_t>(static_cast<uint32_t>(b_t_map[blo]) >> nb))
                     : blo / B;
    if (t_lo >= seg.T) t_lo = seg.T - 1;
  }
  if (threadIdx.x == 0) s_bad = 0;
  // Bag of every position without a search when the block spans few bags:
  // each non-empty bag marks its first position, and position l's bag is the
  // largest mark at or before l (an inclusive max-scan; bag ids grow with
  // position, and position l0 belongs to bag blo, mark 0).
  const bool marked = bhi - blo < 4 * kLinTile;  // block-uniform
  uint32_t rel[kLinItems];
  if (marked) {
    for (int i = threadIdx.x; i < kLinTile; i += 256) s_mark[i] = 0u;
    __syncthreads();
    for (int64_t b = blo + threadIdx.x; b <= bhi; b += 256) {
      const int64_t o0 = static_cast<int64_t>(offsets[b]);
      const int64_t o1 = static_cast<int64_t>(offsets[b + 1]);
      if (o1 > o0 && o0 >= l0 && o0 < lend) s_mark[o0 - l0] = static_cast<uint32_t>(b - blo);
    }
    __syncthreads();
    uint32_t wmax = 0u;
#pragma unroll
    for (int it = 0; it < kLinItems; ++it) {
      const uint32_t m = s_mark[w * kLinWavePos + it * 64 + lane];
      wmax = m > wmax ? m : wmax;
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
      const uint32_t o = __shfl_xor(wmax, d, 64);
      wmax = o > wmax ? o : wmax;
    }
    if (lane == 0) s_wmax[w] = wmax;
    __syncthreads();
    uint32_t carry = 0u;  // largest mark before this wave's positions
    for (int i = 0; i < w; ++i) carry = s_wmax[i] > carry ? s_wmax[i] : carry;
#pragma unroll
    for (int it = 0; it < kLinItems; ++it) {
      uint32_t v = wave_incl_scan<MaxOp>(s_mark[w * kLinWavePos + it * 64 + lane]);
      v = v > carry ? v : carry;
      rel[it] = v;
      carry = __shfl(v, 63, 64);
    }
  } else {
    // Many empty bags inside the block: per-position binary search.
#pragma unroll
    for (int it = 0; it < kLinItems; ++it) {
      const int64_t l = pbase + it * 64;
      int64_t lo = blo, hi = bhi + 1;  // offsets[hi] > l for every l of the block
      while (l < lend && hi - lo > 1) {
        const int64_t mid = lo + ((hi - lo) >> 1);
        if (static_cast<int64_t>(offsets[mid]) <= l)
          lo = mid;
        else
          hi = mid;
      }
      rel[it] = static_cast<uint32_t>(lo - blo);
    }
    __syncthreads();  // count arrays cleared
  }
  // Positions' keys and digit counts, compiled apart for per-feature counts
  // (PF) and the whole batch's, so that each keeps straight-line code.
  const bool pf = seg.T > 0 && s_tables_ok != 0;  // block-uniform
  auto tail = [&](auto pf_c) {
    constexpr bool PF = decltype(pf_c)::value;
#pragma unroll
    for (int it = 0; it < kLinItems; ++it) {
      const int64_t l = pbase + it * 64;
      if (l >= lend) continue;
      const int64_t bag = blo + rel[it];
      // Info word (t << nb) | b: computed for a fixed batch, given per bag (VBE).
      uint32_t info;
      int64_t t;
      if (b_t_map) {
        info = static_cast<uint32_t>(b_t_map[bag]);
        t = nb >= 32 ? 0 : static_cast<int64_t>(info >> nb);
      } else {
        t = bag / B;
        const int64_t b = bag - t * B;
        info = (nb >= 32 ? 0u : (static_cast<uint32_t>(t) << nb)) | static_cast<uint32_t>(b);
      }
      // A variable batch's segments take their positions from B_off, so each
      // bag must lie in its own feature's range of bags; else the sort is global.
      if (seg.B_off && (t >= seg.T || bag < s_boff[t] || bag >= s_boff[t + 1])) {
        s_bad = 1;
        if (t >= seg.T) t = seg.T - 1;  // in-bounds LDS reads
      }
      const int64_t key = (seg.T > 0 ? s_hsc[t] : hsc[t]) + static_cast<int64_t>(idx[it]);
      if (linear_out) linear_out[l] = key;
      const uint32_t k32 = static_cast<uint32_t>(key);
      keys[l] = k32;
      vals[l] = info;
      if (iw) vals2[l] = __float_as_uint(iw[l]);  // per-sample weight rides along the sort
      if constexpr (!PF) {
        for (int p = 0; p < passes; ++p)
          atomicAdd(&h[p][(k32 >> (p * kRadixBits)) & digit_mask(bits, p)], 1u);
      } else {
        const int64_t i64 = static_cast<int64_t>(idx[it]);
        const int gl = s_gid[t];
        const int tf = gl - s_gid[t_lo];  // relative to the block's first segment
        const int64_t rows_t = s_gend[t] - s_hsc[t];
        if (i64 < 0 || i64 >= rows_t) s_bad = 1;  // outside its table's range
        for (int p = 0; p < passes; ++p) {
          const uint32_t d = (k32 >> (p * kRadixBits)) & digit_mask(bits, p);
          if (tf == 0 || tf == 1)
            atomicAdd(&hf[tf][p][d], 1u);
          else  // a block over three or more segments (short ones): straight to memory
            atomicAdd(&seg.fhist[gl * kSegRow + (blockIdx.x % kHistCopies) * kHistCopyWords +
                                 p * kRadix + d], 1u);
        }
      }
    }
    __syncthreads();
    if constexpr (PF) {
      if (threadIdx.x == 0 && s_bad) *seg.bad = kSegKeys;
      const int nbins = passes * kRadix;
      const int rot = static_cast<int>(blockIdx.x * 97u % static_cast<uint32_t>(nbins));
      const int g_lo = s_gid[t_lo];
      for (int f = 0; f < 2 && g_lo + f < s_ngroups; ++f)
        for (int jj = threadIdx.x; jj < nbins; jj += 256) {
          const int j = jj + rot < nbins ? jj + rot : jj + rot - nbins;
          const uint32_t c = (&hf[f][0][0])[j];
          if (c)
            atomicAdd(&seg.fhist[(g_lo + f) * kSegRow + (blockIdx.x % kHistCopies) * kHistCopyWords + j],
                      c);
        }
      if (blockIdx.x == 0 && w == 0) {
        // Lane g <= S: segment g's first position (its first feature's); its
        // tile count; the segments' first tiles by a wave scan.  Entries S+1 .. T
        // repeat the end, so no tile falls in them.  The positions must not
        // decrease for the segments to be in key order (hsc does not: checked).
        const int T = seg.T, S = s_ngroups;
        int64_t fbag = seg.B_off ? static_cast<int64_t>(s_boff[s_gfirst[lane < S ? lane : S]])
                                 : static_cast<int64_t>(s_gfirst[lane < S ? lane : S]) * B;
        fbag = fbag < 0 ? 0 : (fbag > nbags ? nbags : fbag);  // a bad B_off fails the checks below
        const int64_t fp = lane <= S ? static_cast<int64_t>(offsets[fbag]) : N;
        const int64_t fnext = __shfl(fp, lane + 1 < 64 ? lane + 1 : 63, 64);
        const uint32_t nt = lane < S ? static_cast<uint32_t>(ceil_div(fnext - fp, kSweepTile)) : 0u;
        const uint32_t incl = wave_incl_scan<SumOp>(nt);
        // The segments must also cover exactly the positions [0, N).
        bool bad = (lane < S && fnext < fp) || (lane == 0 && fp != 0) || (lane == S && fp != N);
        if (lane <= T) seg.fpos[lane] = fp;
        if (lane < T) seg.tprefix[lane + 1] = static_cast<int32_t>(incl);
        if (lane == 0) seg.tprefix[0] = 0;
        if (__any(bad) && lane == 0) *seg.bad = kSegKeys;
      }
    } else {
      // Into this XCD's copy, each block starting at another bin so that blocks
      // finishing together do not queue on the same counters.
      uint32_t* gcopy = ghist + (blockIdx.x % kHistCopies) * kHistCopyWords;
      const int nbins = passes * kRadix;
      const int rot = static_cast<int>((blockIdx.x / kHistCopies) * 97u % static_cast<uint32_t>(nbins));
      for (int j = threadIdx.x; j < nbins; j += 256) {
        const int i = j + rot < nbins ? j + rot : j + rot - nbins;
        const uint32_t c = (&h[0][0])[i];
        if (c) atomicAdd(&gcopy[i], c);
      }
      // Features that share a table: no segments, the passes read these counts.
      if (seg.T > 0 && blockIdx.x == 0 && threadIdx.x == 0) *seg.bad = kSegTables;
    }
  };
  if (pf)
    tail(std::true_type{});
  else
    tail(std::false_type{});
}

// ---- radix sort: one launch per pass --------------------------------------

// A look-back status word: a flag in the top two bits (0 unpublished, 1 the
// tile's own count, 2 the inclusive prefix), the count below.  32-bit words
// (counts below 2^30) halve the uncached look-back traffic against 64-bit
// ones (config 3: 17.2 -> 16.4 us per pass); larger sorts use 64-bit words.
template <typename SW>
struct SweepWord {
  static constexpr int kFlagShift = 8 * static_cast<int>(sizeof(SW)) - 2;
  static constexpr SW kAgg = SW(1) << kFlagShift;
  static constexpr SW kIncl = SW(2) << kFlagShift;
  static constexpr SW kValue = kAgg - 1;
};

// status: [tiles][kRadix] zeroed words; ticket: zeroed next-tile counter.
// ghist: this pass's digit counts, kHistCopies copies kHistCopyWords apart.
// One tile of a pass, compiled apart for per-feature segments (kTileSeg), one
// global sort over the whole batch's digit counts (kTileGlobal) and one over
// the sum of the per-feature counts (kTileKeys), so that the global path keeps
// the code of a sort without segments (one body with both paths scheduled it
// ~2 us per call slower).
constexpr int kTileSeg = 0, kTileGlobal = 1, kTileKeys = 2;
// A tile in digit order, staged in LDS between its ranking and its stores,
// with the tile-local scan of its digit counts.
struct SweepStage {
  uint32_t k[kSweepTile];
  uint32_t v[kSweepTile];
  uint32_t v2[kSweepTile];
  uint32_t tstart[kRadix];     // a digit's first position in the tile's digit order
  uint32_t tsum[kRadix / 64];  // per-wave totals of the tile's digit counts
};
template <int MODE, bool LAST, typename SW>
__device__ __forceinline__ void sweep_tile(
    const uint32_t* __restrict__ keys, const uint32_t* __restrict__ vals,
    const uint32_t* __restrict__ vals2, int64_t n, int shift, int nbits,
    const uint32_t* __restrict__ ghist, SW* status, unsigned int* ticket, const Faults& faults,
    uint32_t* __restrict__ keys_out, int64_t* __restrict__ keys_out64,
    uint32_t* __restrict__ vals_out, uint32_t* __restrict__ vals2_out, const SegSort& seg,
    int64_t lane_fpos, int32_t lane_tp, unsigned int& s_tile, unsigned int& s_stop,
    uint32_t (&cnt)[kSweepWaves][kRadix], uint32_t (&s_base)[kRadix],
    uint32_t (&s_wsum)[kRadix / 64], SweepStage& stg) {
  const int w = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  // One thread reads the failure word and takes the ticket, so the whole
  // block agrees (a tile of this launch may set the word while the block
  // starts).  A block of a failed call takes no ticket: every tile that took
  // one publishes, so no tile waits on it.  s_stop is 1 from here on when the
  // block must not scatter (failed call, or a give-up in the digit phase).
  if (threadIdx.x == 0) {
    s_stop = call_failed(faults.fail) ? 1u : 0u;  // an earlier pass gave up: nothing valid to sort
    if (s_stop == 0u) s_tile = atomicAdd(ticket, 1u);
  }
  for (int i = threadIdx.x; i < kSweepWaves * kRadix; i += kSweepThreads) (&cnt[0][0])[i] = 0u;
  __syncthreads();
  if (s_stop != 0u) return;  // block-uniform
  const int64_t tile = s_tile;
  // The tile's positions [pbeg, pend) and the first tile of its look-back
  // chain: its feature's first tile (segments), or tile 0.  Tiles past the
  // last real tile return (nobody waits on them: their tickets are last).
  int64_t pbeg, pend, tile0 = 0, f = 0, fpos_f = 0;
  if constexpr (MODE == kTileSeg) {
    const int32_t tp_next = __shfl(lane_tp, lane + 1 < 64 ? lane + 1 : 63, 64);
    const bool mine = lane < seg.T && lane_tp <= tile && tile < tp_next;
    const uint64_t m = __ballot(mine);  // one feature at most (wave-uniform)
    if (m == 0ull) return;              // block-uniform: past every segment
    f = __ffsll(static_cast<long long>(m)) - 1;
    tile0 = __shfl(lane_tp, static_cast<int>(f), 64);
    fpos_f = __shfl(lane_fpos, static_cast<int>(f), 64);
    const int64_t fnext = __shfl(lane_fpos, static_cast<int>(f) + 1, 64);
    const int64_t fe = fnext < n ? fnext : n;  // fpos[T] == n (checked)
    pbeg = fpos_f + (tile - tile0) * kSweepTile;
    pend = pbeg + kSweepTile < fe ? pbeg + kSweepTile : fe;
  } else {
    pbeg = tile * kSweepTile;
    if (pbeg >= n) return;  // block-uniform
    pend = pbeg + kSweepTile < n ? pbeg + kSweepTile : n;
  }
  const int64_t i0 = pbeg + w * kSweepWaveKeys + lane;
  uint32_t k[kSweepItems], v[kSweepItems], v2[kSweepItems], rank[kSweepItems];
#pragma unroll
  for (int it = 0; it < kSweepItems; ++it) {
    const int64_t i = i0 + it * 64;
    const bool valid = i < pend;
    k[it] = valid ? keys[i] : 0u;
    v[it] = valid ? vals[i] : 0u;
    v2[it] = (valid && vals2) ? vals2[i] : 0u;
  }
  const uint32_t mask = (1u << nbits) - 1u;
  const uint64_t lt = (1ull << lane) - 1ull;
#pragma unroll
  for (int it = 0; it < kSweepItems; ++it) {
    const bool valid = i0 + it * 64 < pend;
    const uint32_t d = (k[it] >> shift) & mask;
    uint64_t peers = __ballot(valid);
    for (int bit = 0; bit < nbits; ++bit) {
      const bool set = (d >> bit) & 1u;
      const uint64_t bb = __ballot(set);
      peers &= set ? bb : ~bb;
    }
    const uint32_t before = cnt[w][d];
    rank[it] = before + static_cast<uint32_t>(__popcll(peers & lt));
    // The lowest lane of each digit group advances the wave's count after
    // every lane has read it (LDS operations of a wave are ordered).
    if (valid && (peers & lt) == 0ull) cnt[w][d] = before + static_cast<uint32_t>(__popcll(peers));
  }
  __syncthreads();
  // Digit phase: the first kRadix threads (whole waves) own one digit each;
  // the block's other waves only pass the barriers.
  const int d = threadIdx.x;
  const bool digit_wave = w < kRadix / 64;  // wave-uniform
  const bool used = digit_wave && d <= static_cast<int>(mask);  // same for every tile of the pass
  uint32_t total = 0u, incl = 0u, tincl = 0u, gcount = 0u;
  if (digit_wave) {
#pragma unroll
    for (int x = 0; x < kSweepWaves; ++x) {  // per-wave counts -> per-wave prefixes
      const uint32_t c = cnt[x][d];
      cnt[x][d] = total;
      total += c;
    }
    tincl = wave_incl_scan<SumOp>(total);  // the tile's digit counts: its local digit starts
    if (lane == 63) stg.tsum[w] = tincl;
    if constexpr (MODE == kTileSeg) {
      if (used)
#pragma unroll
        for (int x = 0; x < kHistCopies; ++x) gcount += seg.fhist[f * kSegRow + x * kHistCopyWords + d];
    } else if constexpr (MODE == kTileKeys) {
      // A key outside its feature's range (invalid input): linearize counted per
      // feature, the pass sorts globally over their sum.
      if (used)
#pragma unroll 4
        for (int t = 0; t < seg.T; ++t)
#pragma unroll
          for (int x = 0; x < kHistCopies; ++x) gcount += seg.fhist[t * kSegRow + x * kHistCopyWords + d];
    } else {
      if (used)
#pragma unroll
        for (int x = 0; x < kHistCopies; ++x) gcount += ghist[x * kHistCopyWords + d];
    }
    incl = wave_incl_scan<SumOp>(gcount);
    if (lane == 63) s_wsum[w] = incl;
  }
  __syncthreads();
  if (digit_wave) {
    // Exclusive scan of the pass's digit counts: the digit's global base.
    uint32_t goff = 0u;
#pragma unroll
    for (int i = 0; i < kRadix / 64; ++i)
      if (i < w) goff += s_wsum[i];
    const uint32_t prev = __shfl_up(incl, 1, 64);
    if (lane != 0) goff += prev;
    if constexpr (MODE == kTileSeg) goff += static_cast<uint32_t>(fpos_f);  // the segment's first position
    uint32_t tstart = tincl - total;  // the digit's first position in the tile's digit order
#pragma unroll
    for (int i = 0; i < kRadix / 64; ++i)
      if (i < w) tstart += stg.tsum[i];
    stg.tstart[d] = tstart;
    uint32_t prefix = 0u;
    // A digit no key of the segment (or batch) holds has no tile to publish
    // for or wait on (the last pass of a table-wide segment uses ~16 of its
    // digits).
    if (used && gcount != 0u) {
      using Word = SweepWord<SW>;
      SW* mine = status + tile * kRadix + d;
      if (tile == tile0) {
        __hip_atomic_store(mine, Word::kIncl | total, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      } else {
        __hip_atomic_store(mine, Word::kAgg | total, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // Look back kLookBack predecessors per round (independent loads), folding
        // them nearest first until an inclusive word; an unpublished word
        // (flag 0) ends the round and the next round resumes there.  Wider
        // rounds issue more uncached loads than they save in rounds (per pass
        // at 2048-key tiles: 8 +0.6 us, 16 +2.2, 32 +5.1; 2 is no faster).
        constexpr int kLookBack = 4;
        int64_t j = tile - 1;  // nearest predecessor not yet folded in
        int spins = 0;
        bool done = false;
        if (faults.spin_limit < 0) {  // test hook: give up at once
          report_fault(faults);
          s_stop = 1u;
          done = true;
        }
        while (!done) {
          SW x[kLookBack];
#pragma unroll
          for (int q = 0; q < kLookBack; ++q)
            x[q] = j - q >= tile0 ? __hip_atomic_load(status + (j - q) * kRadix + d,
                                                      __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                  : Word::kIncl;  // before the chain (never reached: its first tile is inclusive)
          int folded = 0;
#pragma unroll
          for (int q = 0; q < kLookBack; ++q) {
            if (done || folded < q) continue;  // stopped at an earlier predecessor of these loads
            const SW flag = x[q] >> Word::kFlagShift;
            if (flag == 0) continue;
            prefix += static_cast<uint32_t>(x[q] & Word::kValue);
            folded = q + 1;
            if (flag == 2) done = true;
          }
          j -= folded;
          if (!done && folded < kLookBack) {     // waiting on an unpublished predecessor
            if (!keep_waiting(spins, faults)) {  // never expected; keeps the wait bounded
              report_fault(faults);
              s_stop = 1u;
              break;
            }
          }
        }
        __hip_atomic_store(mine, Word::kIncl | (prefix + total), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    // Global position of the digit's keys, less their first position in the
    // tile's digit order (modulo 2^32).
    s_base[d] = goff + prefix - tstart;
  }
  __syncthreads();
  // A give-up published a partial prefix (so later tiles end their waits) and
  // the call is marked failed: the tile writes nothing.
  if (s_stop != 0u) return;  // block-uniform
  // The tile in digit order through LDS, then stored by consecutive threads:
  // the keys of one digit land at consecutive addresses, so a wave's store is
  // a few runs instead of 64 scattered words.
#pragma unroll
  for (int it = 0; it < kSweepItems; ++it) {
    if (i0 + it * 64 >= pend) continue;
    const uint32_t dd = (k[it] >> shift) & mask;
    const uint32_t local = stg.tstart[dd] + cnt[w][dd] + rank[it];  // below the tile's size
    stg.k[local] = k[it];
    stg.v[local] = v[it];
    if (vals2) stg.v2[local] = v2[it];
  }
  __syncthreads();
  const int64_t tile_n = pend - pbeg;
#pragma unroll
  for (int it = 0; it < kSweepItems; ++it) {
    const int64_t i = threadIdx.x + it * kSweepThreads;
    if (i >= tile_n) continue;
    const uint32_t kk = stg.k[i];
    const uint32_t pos = s_base[(kk >> shift) & mask] + static_cast<uint32_t>(i);
    if (pos >= n) continue;  // never; keeps stores in bounds whatever the counts
    if constexpr (LAST)
      keys_out64[pos] = static_cast<int64_t>(kk);
    else
      keys_out[pos] = kk;
    vals_out[pos] = stg.v[i];
    if (vals2) vals2_out[pos] = stg.v2[i];
  }
}

template <bool LAST, typename SW>
__global__ void __launch_bounds__(kSweepThreads)
    onesweep_kernel(const uint32_t* __restrict__ keys, const uint32_t* __restrict__ vals,
                    const uint32_t* __restrict__ vals2, int64_t n, int shift, int nbits,
                    const uint32_t* __restrict__ ghist, SW* status,
                    unsigned int* ticket, Faults faults, uint32_t* __restrict__ keys_out,
                    int64_t* __restrict__ keys_out64, uint32_t* __restrict__ vals_out,
                    uint32_t* __restrict__ vals2_out, SegSort seg) {
  __shared__ unsigned int s_tile, s_stop;
  __shared__ uint32_t cnt[kSweepWaves][kRadix];  // per-wave digit counts, then per-wave prefixes
  __shared__ uint32_t s_base[kRadix];
  __shared__ uint32_t s_wsum[kRadix / 64];
  __shared__ SweepStage stg;
  const int lane = threadIdx.x & 63;
  // The segment state loads while the tile takes its ticket (neither depends
  // on the other): why the passes sort globally (0: they do not), and lane
  // f <= T's feature first position and first tile.
  const unsigned int why = seg.T > 0 ? __hip_atomic_load(seg.bad, __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT)
                                     : kSegTables;
  int64_t lane_fpos = 0;
  int32_t lane_tp = 0;
  if (seg.T > 0 && lane <= seg.T) {
    lane_fpos = seg.fpos[lane];
    lane_tp = seg.tprefix[lane];
  }
  if (why == 0u)  // grid-uniform
    sweep_tile<kTileSeg, LAST, SW>(keys, vals, vals2, n, shift, nbits, ghist, status, ticket,
                                   faults, keys_out, keys_out64, vals_out, vals2_out, seg,
                                   lane_fpos, lane_tp, s_tile, s_stop, cnt, s_base, s_wsum, stg);
  else if (why == kSegKeys)
    sweep_tile<kTileKeys, LAST, SW>(keys, vals, vals2, n, shift, nbits, ghist, status, ticket,
                                    faults, keys_out, keys_out64, vals_out, vals2_out, seg,
                                    lane_fpos, lane_tp, s_tile, s_stop, cnt, s_base, s_wsum, stg);
  else
    sweep_tile<kTileGlobal, LAST, SW>(keys, vals, vals2, n, shift, nbits, ghist, status, ticket,
                                      faults, keys_out, keys_out64, vals_out, vals2_out, seg,
                                      lane_fpos, lane_tp, s_tile, s_stop, cnt, s_base, s_wsum, stg);
}

// One sort pass over a workspace whose status words are of type SW.
template <bool LAST, typename SW>
void sweep(dim3 grid, hipStream_t s, const uint32_t* keys, const uint32_t* vals,
           const uint32_t* vals2, int64_t n, int shift, int nbits, const uint32_t* ghist,
           unsigned long long* status, unsigned int* ticket, const Faults& f, uint32_t* keys_out,
           int64_t* keys_out64, uint32_t* vals_out, uint32_t* vals2_out, const SegSort& seg) {
  onesweep_kernel<LAST, SW><<<grid, kSweepThreads, 0, s>>>(
      keys, vals, vals2, n, shift, nbits, ghist, reinterpret_cast<SW*>(status), ticket, f,
      keys_out, keys_out64, vals_out, vals2_out, seg);
}

__global__ void copy_keys_kernel(const uint32_t* __restrict__ keys,
                                 const uint32_t* __restrict__ vals, int64_t n,
                                 int64_t* __restrict__ keys_out64, uint32_t* __restrict__ vals_out,
                                 const uint32_t* __restrict__ vals2,
                                 uint32_t* __restrict__ vals2_out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  keys_out64[i] = keys[i];
  vals_out[i] = vals[i];
  if (vals2) vals2_out[i] = vals2[i];
}

// Clears up to two int32 scalars (a kernel, not a memset, so the call can be
// captured in a graph).
__global__ void zero_two_kernel(int32_t* a, int32_t* b) {
  if (threadIdx.x == 0) {
    if (a) *a = 0;
    if (b) *b = 0;
  }
}

// ---- run-length encoding --------------------------------------------------

struct HeadFlag {
  const int64_t* keys;
  __device__ uint32_t operator()(int64_t i) const {
    return (i == 0 || keys[i] != keys[i - 1]) ? 1u : 0u;
  }
};

// Epilogue of the head-flag scan: element i with exclusive head count r
// starts run r when it is a head.
struct RleEpi {
  const int64_t* keys;
  int64_t n;
  int64_t* run_keys;
  int32_t* cum;
  uint32_t* num_runs;        // device count used by later kernels
  int32_t* num_runs_out;     // the op's int32 output, may be null
  __device__ void operator()(int64_t i, uint32_t r, uint32_t head) const {
    if (head) {
      run_keys[r] = keys[i];
      cum[r] = static_cast<int32_t>(i);
    }
  }
  __device__ void total(uint32_t t) const {
    *num_runs = t;
    if (num_runs_out) *num_runs_out = static_cast<int32_t>(t);
    cum[t] = static_cast<int32_t>(n);
  }
};

// run_lengths[r] = cum[r+1] - cum[r] for the num_runs runs; past them the
// arrays read as the complete cumsum of zero-padded lengths: run_lengths 0,
// cum N.  (Threads r >= m write cum[r+1] > m, threads r < m read cum[<= m]:
// no overlap.)  When a look-back of the call gave up, the runs were never
// counted: the outputs become an empty layout (no runs, lengths 0, cum 0).
__global__ void __launch_bounds__(256)
    run_lengths_kernel(int32_t* __restrict__ cum, const uint32_t* __restrict__ num_runs,
                       int64_t n, int32_t* __restrict__ lengths, int32_t* num_runs_out,
                       const unsigned int* fail) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (call_failed(fail)) {  // set before this launch: the same for every thread
    if (r == 0) {
      cum[0] = 0;
      if (num_runs_out) *num_runs_out = 0;
    }
    if (r < n) {
      lengths[r] = 0;
      cum[r + 1] = 0;
    }
    return;
  }
  const int64_t m = *num_runs;
  if (r >= n) return;
  if (r < m) {
    lengths[r] = cum[r + 1] - cum[r];
  } else {
    lengths[r] = 0;
    cum[r + 1] = static_cast<int32_t>(n);
  }
}

struct ChunkCount {
  const int32_t* cum;
  __device__ uint32_t operator()(int64_t r) const {
    const int32_t len = cum[r + 1] - cum[r];
    return len > kLong ? static_cast<uint32_t>((len + kChunk - 1) / kChunk) : 0u;
  }
};

// Chunk marks (a zeroed array over the chunks): chunk q0 + j of long run r,
// for j = 0, kMarkEvery, 2 kMarkEvery, ..., holds r + 1, with kRunStart set
// on the run's first chunk.  The owner of any chunk is the nearest mark at
// or before it, at most kMarkEvery - 1 chunks back: one round of loads.
constexpr int kMarkEvery = 16;
constexpr uint32_t kRunStart = 0x80000000u;

// Epilogue of the chunk-count scan: chunk_start[r] = first chunk of run r
// (runs of at most kLong occurrences own no chunk) and the chunk marks.
struct ChunkEpi {
  const int32_t* cum;
  uint32_t* chunk_start;
  uint32_t* chunk_mark;
  uint32_t* total_chunks;
  __device__ void operator()(int64_t r, uint32_t q0, uint32_t nq) const {
    chunk_start[r] = q0;
    for (uint32_t j = 0; j < nq; j += kMarkEvery)
      chunk_mark[q0 + j] = (static_cast<uint32_t>(r) + 1u) | (j == 0 ? kRunStart : 0u);
  }
  __device__ void total(uint32_t t) const { *total_chunks = t; }
};

// ---- workspace layout -----------------------------------------------------

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

int64_t sweep_tiles(int64_t n) { return ceil_div(n > 0 ? n : 1, kSweepTile); }
// Tiles of a pass, with room for segments: each of up to kSegMaxT segments
// starts at a tile boundary, so they need at most kSegMaxT more tiles.
int64_t sweep_status_tiles(int64_t n) { return sweep_tiles(n) + kSegMaxT; }
// Room per pass, in 8-byte words: the most status words a call can use (8-byte
// words, every segment tile), then 32 words holding the ticket.
int64_t sweep_pass_words(int64_t n) { return sweep_status_tiles(n) * kRadix + 32; }
constexpr size_t kSegHistBytes = static_cast<size_t>(kSegMaxT) * kSegRow * 4;
constexpr size_t kStatusBytes = 256;
constexpr size_t kHistBytes = (kHistCopies * kHistCopyWords * 4 + 255) & ~size_t(255);
// The words linearize adds into, which must be zero when it starts: the
// segment word, the digit histograms and the per-feature digit counts.
constexpr size_t kEarlyBytes = kStatusBytes + kHistBytes + kSegHistBytes;

struct SortWs {
  uint32_t* keys[2];
  uint32_t* vals[2];
  uint32_t* vals2[2];  // per-sample weights (weighted backward only)
  // Zeroed state, contiguous: the early words (segment word, digit
  // histograms, per-feature digit counts; kEarlyBytes), then the failure word,
  // the scan slots, the chunk marks and the sweep state (cleared by linearize).
  unsigned long long* zeroed;
  unsigned long long* late;
  unsigned int* fail;              // set when a look-back of the call gave up
  unsigned long long* scan_state;  // kScanSlots slots of scan_slot_words
  int64_t scan_slot_words;
  uint32_t* ghist;                 // [kHistCopies][kMaxPasses][kRadix]
  uint32_t* fhist;                 // [kSegMaxT][kHistCopies][kMaxPasses][kRadix] per-feature digit counts
  unsigned int* seg_bad;           // nonzero (kSegKeys, kSegTables): the passes sort globally
  int64_t* fpos;                   // [kSegMaxT + 1] (written by linearize)
  int32_t* tprefix;                // [kSegMaxT + 1] (written by linearize)
  uint32_t* chunk_mark;            // [max_chunks(N)] (backward only)
  unsigned long long* sweep;       // kMaxPasses x sweep_pass_words
  int64_t sweep_words;
  uint32_t* counters;  // [0] num_runs, [1] total chunks
  size_t bytes;
  int64_t early_words;  // early words the call used (set by run_transpose)
};

SortWs carve_sort(uint8_t* base, int64_t N) {
  SortWs w{};
  const int64_t n = N > 0 ? N : 1;
  const int64_t slot_words = scan_tiles(n + 1) + 2;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    uint8_t* p = base ? base + off : nullptr;
    off += align256(bytes);
    return p;
  };
  for (int i = 0; i < 2; ++i) {
    w.keys[i] = reinterpret_cast<uint32_t*>(take(n * 4));
    w.vals[i] = reinterpret_cast<uint32_t*>(take(n * 4));
    w.vals2[i] = reinterpret_cast<uint32_t*>(take(n * 4));
  }
  w.scan_slot_words = align256(slot_words * 8) / 8;
  w.sweep_words = sweep_pass_words(n);
  const size_t scan_bytes = kScanSlots * w.scan_slot_words * 8;
  const size_t mark_bytes = align256(static_cast<size_t>(max_chunks(n)) * 4);
  // Zeroed state: the early words (cleared before linearize, which adds into
  // the counts), then the failure word, the scans' and passes' look-back
  // state and the chunk marks (cleared by linearize itself).
  const size_t late0 = kEarlyBytes, scan0 = late0 + kStatusBytes, mark0 = scan0 + scan_bytes;
  uint8_t* z = take(mark0 + mark_bytes + kMaxPasses * w.sweep_words * 8);
  w.zeroed = reinterpret_cast<unsigned long long*>(z);
  w.seg_bad = reinterpret_cast<unsigned int*>(z);
  w.ghist = z ? reinterpret_cast<uint32_t*>(z + kStatusBytes) : nullptr;
  w.fhist = z ? reinterpret_cast<uint32_t*>(z + kStatusBytes + kHistBytes) : nullptr;
  w.late = z ? reinterpret_cast<unsigned long long*>(z + late0) : nullptr;
  w.fail = z ? reinterpret_cast<unsigned int*>(z + late0) : nullptr;
  w.scan_state = z ? reinterpret_cast<unsigned long long*>(z + scan0) : nullptr;
  w.chunk_mark = z ? reinterpret_cast<uint32_t*>(z + mark0) : nullptr;
  w.sweep = z ? reinterpret_cast<unsigned long long*>(z + mark0 + mark_bytes) : nullptr;
  w.fpos = reinterpret_cast<int64_t*>(take((kSegMaxT + 1) * 8));
  w.tprefix = reinterpret_cast<int32_t*>(take((kSegMaxT + 1) * 4));
  w.counters = reinterpret_cast<uint32_t*>(take(64));
  w.bytes = off;
  return w;
}

// Early words of a call: the segment word, the histograms, and the digit
// counts of `seg_features` features.
int64_t early_zeroed_words(const SortWs& w, int32_t seg_features) {
  return static_cast<int64_t>(reinterpret_cast<uint8_t*>(w.fhist) -
                              reinterpret_cast<uint8_t*>(w.zeroed)) / 8 +
         static_cast<int64_t>(seg_features) * kSegRow / 2;
}

// A call's sweep state per pass, in 8-byte words: `tiles` x kRadix status
// words of `word_bytes` each, then 32 words holding the ticket (a multiple of
// 256 bytes; at most the workspace's sweep_words).
int64_t call_pass_words(int64_t tiles, int word_bytes) {
  return align256(static_cast<size_t>(tiles) * kRadix * word_bytes) / 8 + 32;
}

// Words linearize clears for a sort of `passes` passes of `pass_words` each:
// the failure word, the scan state, the chunk marks and the sweep state of
// those passes (the rest of the workspace's sweep state is left alone).
int64_t late_zeroed_words(const SortWs& w, int passes, int64_t pass_words) {
  return static_cast<int64_t>(reinterpret_cast<uint8_t*>(w.sweep) -
                              reinterpret_cast<uint8_t*>(w.late)) / 8 +
         passes * pass_words;
}

// Where the call's look-backs report a give-up.
Faults call_faults(const SortWs& w) {
  return Faults{w.fail, status_mailbox(), lookback_spin_limit(kScanSpinLimit)};
}

// Scan-state slot i: status words, then the ticket in the last word.
ScanState scan_slot(const SortWs& w, int i) {
  unsigned long long* base = w.scan_state + i * w.scan_slot_words;
  return ScanState{base, reinterpret_cast<unsigned int*>(base + w.scan_slot_words - 1),
                   call_faults(w)};
}

struct TransposeOut {
  int64_t* linear;      // may be null
  int64_t* sorted;      // [N]
  int32_t* infos;       // [N]
  int64_t* run;         // [N]
  int32_t* run_lengths; // [N], may be null
  int32_t* num_runs;    // [1], may be null
  int32_t* cum;         // [N+1]
  float* weights_sorted;  // [N] per-sample weights in sorted order, or null
};

// Early words kept zero between calls.  Clearing a call's early words in its
// workspace is one more launch, ~4.5 us of kernel boundary per call.  An
// eager backward takes them instead from a region of its (device, stream)
// that is zero between calls: the call's last kernel clears what the call
// used, after the sort passes have read it, and the next call on the stream
// runs after that kernel.  A call holds `mu` while it submits its kernels, so
// that calls of two host threads on one stream do not interleave.  A region
// in an unknown state (new, or left by a call that stopped between its first
// launch and its last) is cleared by the next call before use.
struct ZeroedRegion {
  std::mutex mu;
  uint8_t* base = nullptr;  // kEarlyBytes, laid out like a workspace's early words
  bool dirty = true;
};

// The region of the current device and stream `s`, allocated on first use;
// null while `s` is being captured (a graph keeps clearing its workspace's
// early words itself), when the allocation fails, once a device holds
// kMaxStreamRegions regions (a caller that makes a new stream per call pays
// the clearing launch instead of 2 MB per stream), or while the test hook
// asks for workspace counters.  Regions live until the process ends.
constexpr int kMaxStreamRegions = 64;

ZeroedRegion* stream_region(hipStream_t s) {
  if (force_workspace_counters()) return nullptr;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  int dev = 0;
  if (hipStreamIsCapturing(s, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone ||
      hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  static std::mutex mu;
  static std::map<std::pair<int, hipStream_t>, std::unique_ptr<ZeroedRegion>> regions;
  static std::map<int, int> per_device;
  std::lock_guard<std::mutex> lock(mu);
  auto it = regions.find({dev, s});
  if (it != regions.end()) return it->second.get();
  if (per_device[dev] >= kMaxStreamRegions) return nullptr;
  void* p = nullptr;
  if (hipMalloc(&p, kEarlyBytes) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  auto r = std::make_unique<ZeroedRegion>();
  r->base = static_cast<uint8_t*>(p);
  ++per_device[dev];
  return (regions[{dev, s}] = std::move(r)).get();
}

// nbags = T * B bags of a fixed batch B, or (b_t_map non-null, VBE) the
// total bag count with each bag's info word given.  zr: the stream's zeroed
// region for the early words (held locked by the caller, whose last kernel
// clears w.early_words of it), or null: the workspace's, cleared here.
int run_transpose(const int64_t* hsc, int32_t T, int64_t B, int64_t nbags,
                  const int32_t* b_t_map, const int32_t* B_off, int32_t bits, int32_t nb, const void* indices,
                  const void* offsets, int32_t index_bytes, int64_t N, const float* iw,
                  const TransposeOut& o, SortWs& w, hipStream_t s, ZeroedRegion* zr) {
  // With per-sample weights the weights travel with the keys as a second payload.
  uint32_t* const v2[2] = {iw ? w.vals2[0] : nullptr, iw ? w.vals2[1] : nullptr};
  uint32_t* const v2_final = iw ? reinterpret_cast<uint32_t*>(o.weights_sorted) : nullptr;
  const dim3 g256(static_cast<uint32_t>(ceil_div(N, 256)));
  const int passes = (bits + kRadixBits - 1) / kRadixBits;
  if (zr) {  // the early words move to the region (same layout)
    const ptrdiff_t d = zr->base - reinterpret_cast<uint8_t*>(w.zeroed);
    w.zeroed = reinterpret_cast<unsigned long long*>(zr->base);
    w.seg_bad = reinterpret_cast<unsigned int*>(reinterpret_cast<uint8_t*>(w.seg_bad) + d);
    w.ghist = reinterpret_cast<uint32_t*>(reinterpret_cast<uint8_t*>(w.ghist) + d);
    w.fhist = reinterpret_cast<uint32_t*>(reinterpret_cast<uint8_t*>(w.fhist) + d);
  }
  // Segments (one per feature) for a batch of at most kSegMaxT features: a
  // fixed batch, or a variable one whose features' first bags are given.
  SegSort seg{};
  if ((b_t_map == nullptr || B_off != nullptr) && T >= 1 && T <= kSegMaxT && passes > 0)
    seg = SegSort{w.fpos, w.tprefix, w.fhist, w.seg_bad, T, b_t_map ? B_off : nullptr};
  w.early_words = early_zeroed_words(w, seg.T);
  if (zr == nullptr || zr->dirty) {  // the early words start at zero (a dirty region: all of them)
    const int64_t words = zr ? static_cast<int64_t>(kEarlyBytes / 8) : w.early_words;
    const int64_t blocks = ceil_div(words, 256);
    zero_u64_kernel<<<dim3(static_cast<uint32_t>(blocks < 2048 ? blocks : 2048)), 256, 0, s>>>(
        w.zeroed, words);
    MX_LAUNCH_CHECK();
  }
  if (zr) zr->dirty = true;  // until the caller's last kernel is launched
  const int64_t ntiles = sweep_tiles(N) + seg.T;  // segments start at tile boundaries
  if (ntiles > 0xffffffffll) return set_error(MX_EINVAL, "too many sort tiles");
  // Every count fits a 32-bit word's 30 bits.
  const bool w32 = N < (int64_t(1) << 30) && !force_wide_sort_words();
  const int64_t pass_words = call_pass_words(ntiles, w32 ? 4 : 8);
  // Linearize also clears the look-back state of the later kernels.
  const int64_t late_words = late_zeroed_words(w, passes, pass_words);
  const dim3 glin(static_cast<uint32_t>(ceil_div(N, kLinTile)));
  if (index_bytes == 8)
    linearize_kernel<int64_t><<<glin, 256, 0, s>>>(
        hsc, static_cast<const int64_t*>(indices), static_cast<const int64_t*>(offsets), nbags, B,
        nb, b_t_map, N, bits, passes, o.linear, w.keys[0], w.vals[0], iw, v2[0], w.ghist,
        w.late, late_words, seg);
  else
    linearize_kernel<int32_t><<<glin, 256, 0, s>>>(
        hsc, static_cast<const int32_t*>(indices), static_cast<const int32_t*>(offsets), nbags, B,
        nb, b_t_map, N, bits, passes, o.linear, w.keys[0], w.vals[0], iw, v2[0], w.ghist,
        w.late, late_words, seg);
  MX_LAUNCH_CHECK();

  const dim3 gsweep(static_cast<uint32_t>(ntiles));
  int cur = 0;
  if (passes == 0) {
    copy_keys_kernel<<<g256, 256, 0, s>>>(w.keys[0], w.vals[0], N, o.sorted,
                                          reinterpret_cast<uint32_t*>(o.infos), v2[0], v2_final);
    MX_LAUNCH_CHECK();
  }
  for (int p = 0; p < passes; ++p) {
    const int shift = p * kRadixBits;
    const int nbits = bits - shift < kRadixBits ? bits - shift : kRadixBits;
    unsigned long long* st = w.sweep + p * pass_words;
    unsigned int* ticket = reinterpret_cast<unsigned int*>(st + pass_words - 32);
    const uint32_t* gh = w.ghist + p * kRadix;
    SegSort segp = seg;  // this pass's row of the per-feature digit counts
    if (seg.T > 0) segp.fhist = seg.fhist + p * kRadix;
    const Faults f = call_faults(w);
    const bool last = p == passes - 1;
    const auto launch = last ? (w32 ? &sweep<true, uint32_t> : &sweep<true, unsigned long long>)
                             : (w32 ? &sweep<false, uint32_t> : &sweep<false, unsigned long long>);
    launch(gsweep, s, w.keys[cur], w.vals[cur], v2[cur], N, shift, nbits, gh, st, ticket, f,
           last ? nullptr : w.keys[cur ^ 1], last ? o.sorted : nullptr,
           last ? reinterpret_cast<uint32_t*>(o.infos) : w.vals[cur ^ 1],
           last ? v2_final : v2[cur ^ 1], segp);
    MX_LAUNCH_CHECK();
    cur ^= 1;
  }

  // Run-length encode the sorted keys.
  if (int rc = prefix_scan_epi(HeadFlag{o.sorted}, N, nullptr,
                               RleEpi{o.sorted, N, o.run, o.cum, &w.counters[0], o.num_runs},
                               scan_slot(w, 0), s))
    return rc;
  if (o.run_lengths) {
    run_lengths_kernel<<<g256, 256, 0, s>>>(o.cum, &w.counters[0], N, o.run_lengths,
                                            o.num_runs, w.fail);
    MX_LAUNCH_CHECK();
  }
  return MX_OK;
}

// ---- segment reduce + rowwise Adagrad -------------------------------------

constexpr int kMaxCachedTables = 512;  // table metadata kept in LDS up to this T

struct BwdArgs {
  void* W;  // fp32 or fp16 rows (the kernels' WT)
  const int64_t* w_off;
  const int32_t* D_off;
  const int64_t* hsc;
  const void* offsets;
  const float* grad;
  float* m1;
  const int64_t* m1_off;
  const int64_t* run;
  const int32_t* cum;
  const int32_t* infos;
  const float* iw_sorted;  // per-sample weights in sorted order, or null
  const int32_t* B_off;    // VBE: first bag of each table [T+1], or null (fixed batch)
  const int64_t* row_out;  // VBE: gradient row offset of each bag, or null
  const uint32_t* num_runs;
  const uint32_t* chunk_start;
  const uint32_t* chunk_mark;  // chunk marks (kMarkEvery), from the chunk-count scan
  const uint32_t* total_chunks;
  float* partial;
  const unsigned int* fail;  // set when a look-back of the call gave up: nothing is updated
  // The stream's zeroed region of the sort's early words, or null: the update
  // launch clears its first rezero_words words (the sort has read them).
  unsigned long long* rezero;
  int64_t rezero_words;
  int64_t B;
  int64_t total_D;
  int32_t T;
  int32_t max_D;
  int32_t nb;
  int32_t pooling;
  int32_t wd_mode;
  float lr;
  float eps;
  float wd;
  int32_t sr;     // fp16 weights: stochastic rounding instead of round-to-nearest-even
  // Random state of the stochastic rounding: (seed, offset) as values, or read
  // when the kernel runs from seed_dev / offset_dev (+ offset) -- the form a
  // graph-captured call carries, so each replay draws new bits.
  uint64_t seed;
  uint64_t offset;
  const int64_t* seed_dev;
  const int64_t* offset_dev;
};

// The call's 64-bit rounding key: seed ^ (offset * odd constant).
__device__ __forceinline__ uint64_t rounding_key(const BwdArgs& a) {
  const uint64_t seed = a.seed_dev ? static_cast<uint64_t>(*a.seed_dev) : a.seed;
  const uint64_t off = a.offset_dev ? static_cast<uint64_t>(*a.offset_dev) + a.offset : a.offset;
  return seed ^ (off * 0xD1B54A32D192ED03ull);
}

// Per-table metadata, staged in LDS when T is small enough.
struct TableMeta {
  int64_t hsc[kMaxCachedTables];
  int64_t w_off[kMaxCachedTables];
  int64_t m1_off[kMaxCachedTables];
  int32_t D_off[kMaxCachedTables + 1];
};

__device__ __forceinline__ void stage_meta(const BwdArgs& a, TableMeta& m) {
  if (a.T <= kMaxCachedTables) {
    for (int i = threadIdx.x; i <= a.T; i += blockDim.x) {
      m.D_off[i] = a.D_off[i];
      if (i < a.T) {
        m.hsc[i] = a.hsc[i];
        m.w_off[i] = a.w_off[i];
        m.m1_off[i] = a.m1_off[i];
      }
    }
  }
  __syncthreads();
}

struct MetaView {
  const BwdArgs& a;
  const TableMeta& m;
  bool cached;
  __device__ int64_t hsc(int64_t t) const { return cached ? m.hsc[t] : a.hsc[t]; }
  __device__ int64_t w_off(int64_t t) const { return cached ? m.w_off[t] : a.w_off[t]; }
  __device__ int64_t m1_off(int64_t t) const { return cached ? m.m1_off[t] : a.m1_off[t]; }
  __device__ int32_t D_off(int64_t t) const { return cached ? m.D_off[t] : a.D_off[t]; }
};

__device__ __forceinline__ void ld4(const float* p, float (&v)[4]) {
  const float4 x = *reinterpret_cast<const float4*>(p);
  v[0] = x.x;
  v[1] = x.y;
  v[2] = x.z;
  v[3] = x.w;
}

__device__ __forceinline__ void st4(float* p, const float (&v)[4]) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
}

// Work items [0, total) in sorted-key order, split into one contiguous range
// per XCD.  Blocks go to the XCDs round-robin (block i runs on XCD i % 8), so
// the blocks of one XCD walk one range of keys -- one range of tables -- and
// read only those tables' gradient columns, which then stay in that XCD's L2
// (each occurrence re-reads its bag's gradient row).  The grid is a multiple
// of 8.  A wave starts at `first` and steps by `step` while below `end`.
struct XcdRange {
  int64_t first, step, end;
};

template <int P>
__device__ __forceinline__ XcdRange xcd_range(int64_t total, int64_t bid, int64_t nblk) {
  constexpr int64_t kXcd = 8;
  const int64_t x = bid % kXcd, j = bid / kXcd, per = nblk / kXcd;
  const int64_t begin = total * x / kXcd;
  const int64_t wave = threadIdx.x >> 6;
  return {begin + (j * 4 + wave) * P, per * 4 * P, total * (x + 1) / kXcd};
}

__device__ __forceinline__ int64_t table_of(const BwdArgs& a, int32_t info) {
  return a.nb >= 32 ? 0 : static_cast<int64_t>(static_cast<uint32_t>(info) >> a.nb);
}

// Column chunk c of lane k (columns (c*G + k)*4 .. +4) lies inside a row of
// D floats.  A full-width instance -- every table's D is G*NCH*4 -- has no
// partial rows and drops the test at compile time (config 3: update launch
// 71.4 -> 62.3 us, chunk sums 17.1 -> 15.9 us).
template <bool FULL, int G>
__device__ __forceinline__ bool col_in(int c, int k, int32_t D) {
  return FULL || (c * G + k) * 4 < D;
}

// A plain instance serves the common call -- SUM pooling, no per-sample
// weights, a fixed batch, no weight decay -- with those options as
// constants, so every per-element test on them folds away (config 3: update
// launch 66.7 -> 62.6 us, chunk sums 16.0 -> 14.5 us).
template <bool PLAIN>
__device__ __forceinline__ void pin_options(BwdArgs& a) {
  if constexpr (PLAIN) {
    a.pooling = MX_POOL_SUM;
    a.iw_sorted = nullptr;
    a.B_off = nullptr;
    a.row_out = nullptr;
    a.wd_mode = 0;
  }
}

// Group-level (G lanes, lane k) sum of the (MEAN-scaled) gradient rows of
// occurrences [s0, s1) of table t, in order.  Lane k owns columns
// (c*G + k)*4 .. +4 for c < NCH.  Called with the whole group converged.
// `info0` is lane k's infos[s0 + k] (valid for k < s1 - s0), already loaded
// by the caller to find the table.
template <typename I, int G, int NCH, int U, bool FULL>
__device__ void group_sum_occurrences(const BwdArgs& a, const MetaView& mv, int32_t D,
                                      int64_t s0, int64_t s1, int g, int k, int32_t info0,
                                      float (&acc)[NCH][4]) {
  const uint32_t bmask = a.nb >= 32 ? 0xffffffffu : ((1u << a.nb) - 1u);
  int32_t info_cur = info0;
  for (int64_t base = s0; base < s1; base += G) {
    const int n = static_cast<int>(s1 - base < G ? s1 - base : G);
    // The next batch's infos load now, ahead of this batch's gradient rows.
    const int32_t info_next = base + G + k < s1 ? a.infos[base + G + k] : 0;
    int64_t my_row = 0;  // element offset of the occurrence's gradient row slice
    float my_s = 1.0f;   // MEAN: 1/L of the occurrence's bag
    float my_w = 1.0f;   // weighted: the occurrence's per-sample weight
    if (k < n) {
      const int32_t info = info_cur;
      const int64_t b = static_cast<int64_t>(static_cast<uint32_t>(info) & bmask);
      // The occurrence's own feature: features that share a table share its
      // rows (one run) but each has its own bags and gradient columns.
      const int64_t tj = table_of(a, info);
      const int64_t bag = a.B_off ? a.B_off[tj] + b : tj * a.B + b;
      // Full width: every feature's columns start at tj * G*NCH*4 (config 3:
      // chunk sums 14.5 -> 12.8 us against the table lookup).
      my_row = a.row_out ? a.row_out[bag] : b * a.total_D + (FULL ? tj * (G * NCH * 4) : mv.D_off(tj));
      if (a.pooling == MX_POOL_MEAN) {
        const I* off = static_cast<const I*>(a.offsets);
        const int64_t L = static_cast<int64_t>(off[bag + 1]) - static_cast<int64_t>(off[bag]);
        my_s = L > 0 ? 1.0f / static_cast<float>(L) : 0.0f;
      }
      if (a.iw_sorted) my_w = a.iw_sorted[base + k];
    }
    const bool mean = a.pooling == MX_POOL_MEAN, weighted = a.iw_sorted != nullptr;
    for (int j = 0; j < n; j += U) {
      float v[U][NCH][4];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (j + u < n) {
          const float* row = a.grad + __shfl(my_row, g * G + j + u, 64);
#pragma unroll
          for (int c = 0; c < NCH; ++c)
            if (col_in<FULL, G>(c, k, D)) ld4(row + (c * G + k) * 4, v[u][c]);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (j + u < n) {
          const float sc = __shfl(my_s, g * G + j + u, 64);
          const float wt = __shfl(my_w, g * G + j + u, 64);
#pragma unroll
          for (int c = 0; c < NCH; ++c)
            if (col_in<FULL, G>(c, k, D)) {
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                float x = v[u][c][e];
                if (mean) x = __fmul_rn(x, sc);
                if (weighted) x = __fmul_rn(x, wt);
                acc[c][e] += x;
              }
            }
        }
      }
    }
    info_cur = info_next;
  }
}

// ---- weight rows: fp32, or fp16 with round-to-nearest-even / stochastic
// rounding of the updated value ---------------------------------------------

__device__ __forceinline__ void ld_row4(const float* p, float (&v)[4]) { ld4(p, v); }

__device__ __forceinline__ void ld_row4(const __half* p, float (&v)[4]) {
  const uint2 x = *reinterpret_cast<const uint2*>(p);
  v[0] = __half2float(__ushort_as_half(static_cast<unsigned short>(x.x & 0xffffu)));
  v[1] = __half2float(__ushort_as_half(static_cast<unsigned short>(x.x >> 16)));
  v[2] = __half2float(__ushort_as_half(static_cast<unsigned short>(x.y & 0xffffu)));
  v[3] = __half2float(__ushort_as_half(static_cast<unsigned short>(x.y >> 16)));
}

// 32 random bits for element `elem` of a call seeded with `seed`: the
// splitmix64 output function (Steele, Lea, Flood 2014) of seed + elem * golden.
__device__ __forceinline__ uint32_t sr_bits(uint64_t seed, uint64_t elem) {
  uint64_t z = seed + elem * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  z ^= z >> 31;
  return static_cast<uint32_t>(z >> 32);
}

// Stochastic rounding to fp16: add to |x| a uniform amount below fp16's last
// place at x's binade (13 random bits in the fp32 mantissa positions fp16
// drops), then round toward zero, so x rounds up with probability equal to
// its distance from the lower neighbour.  The noise is the exact difference
// of two fp32 values of x's sign and exponent.
__device__ __forceinline__ __half round_half_sr(float x, uint32_t rnd) {
  const uint32_t signexp = __float_as_uint(x) & 0xff800000u;
  const float noise = __uint_as_float(signexp | (rnd >> 19)) - __uint_as_float(signexp);
  return __float2half_rz(x + noise);
}

__device__ __forceinline__ void st_row4(const BwdArgs&, uint64_t, float* p, int64_t,
                                        const float (&v)[4]) {
  st4(p, v);
}

// elem: index of p[0] in the weights buffer; key: the call's rounding key
// (together they key the random bits).
__device__ __forceinline__ void st_row4(const BwdArgs& a, uint64_t key, __half* p, int64_t elem,
                                        const float (&v)[4]) {
  __half h[4];
#pragma unroll
  for (int e = 0; e < 4; ++e)
    h[e] = a.sr ? round_half_sr(v[e], sr_bits(key, static_cast<uint64_t>(elem + e)))
                : __float2half_rn(v[e]);
  uint2 x;
  x.x = static_cast<uint32_t>(__half_as_ushort(h[0])) |
        (static_cast<uint32_t>(__half_as_ushort(h[1])) << 16);
  x.y = static_cast<uint32_t>(__half_as_ushort(h[2])) |
        (static_cast<uint32_t>(__half_as_ushort(h[3])) << 16);
  *reinterpret_cast<uint2*>(p) = x;
}

// Rowwise Adagrad on one row held by a G-lane group (lane k owns columns
// (c*G + k)*4 .. +4): h += mean(g^2), m = lr / (sqrt(h) + eps),
// w = fma(-m, g, c*w); lane 0 of the group writes h.  `row0` is the
// weights-buffer index of the row's first element.
template <int G, int NCH, bool FULL, typename WT>
__device__ __forceinline__ void adagrad_update(const BwdArgs& a, int32_t D, int k,
                                               const float (&gs)[NCH][4], const float (&w)[NCH][4],
                                               WT* wrow, int64_t row0, float* hp, float h0) {
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    if (!col_in<FULL, G>(c, k, D)) continue;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float ge = a.wd_mode == 1 ? __builtin_fmaf(a.wd, w[c][e], gs[c][e]) : gs[c][e];
      ss = __builtin_fmaf(ge, ge, ss);
    }
  }
#pragma unroll
  for (int m = G / 2; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);  // group tree, fixed order
  const float h = h0 + ss / static_cast<float>(D);
  const float mult = a.lr / (sqrtf(h) + a.eps);
  float corr = 1.0f;
  if (a.wd_mode == 1)
    corr = 1.0f - mult * a.wd;
  else if (a.wd_mode == 2)
    corr = 1.0f - a.lr * a.wd;
  const uint64_t key = a.sr ? rounding_key(a) : 0ull;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    if (!col_in<FULL, G>(c, k, D)) continue;
    float nw[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) nw[e] = __builtin_fmaf(-mult, gs[c][e], __fmul_rn(corr, w[c][e]));
    st_row4(a, key, wrow + (c * G + k) * 4, row0 + (c * G + k) * 4, nw);
  }
  if (k == 0) *hp = h;
}

// Pass B (long runs): a block owns the long runs whose first chunk lies in
// its kLongRange-chunk range (found by one parallel read of the chunk marks; at
// most kLongRange start in a range) and handles them one after another.  Per run, the 256/G groups sum the run's chunk
// partials round-robin (group j takes chunks j, j + 256/G, ...), the group
// vectors are combined in group order through LDS, and group 0 applies the
// update.
constexpr int kLongRange = 4;  // chunks per block range
constexpr int kLongBlocksPerCu = 2;  // long-run blocks of the runs launch, per CU

template <typename WT, int G, int NCH, int U, bool FULL>
__device__ __forceinline__ void long_run_body(const BwdArgs& a, const MetaView& mv, int64_t bid,
                                              int64_t nblk) {
  constexpr int NG = 256 / G;
  __shared__ float part[NG][G * NCH * 4];
  __shared__ uint32_t s_runs[kLongRange];
  __shared__ int s_nruns;
  const int grp = threadIdx.x / G, k = threadIdx.x % G;
  const int64_t total = *a.total_chunks;
  for (int64_t q0 = bid * kLongRange; q0 < total; q0 += nblk * kLongRange) {
    if (threadIdx.x < 64) {  // wave 0 lists the runs starting in the range, in order
      const int64_t q = q0 + threadIdx.x;
      const bool in = threadIdx.x < kLongRange && q < total;
      const uint32_t m = in ? a.chunk_mark[q] : 0u;
      const bool start = (m & kRunStart) != 0u;
      const uint64_t bal = __ballot(start);
      if (start) s_runs[__popcll(bal & ((1ull << threadIdx.x) - 1ull))] = (m & ~kRunStart) - 1u;
      if (threadIdx.x == 0) s_nruns = __popcll(bal);
    }
    __syncthreads();
    const int nr = s_nruns;
    for (int ri = 0; ri < nr; ++ri) {
      const uint32_t r = s_runs[ri];
      const int64_t s0 = a.cum[r];
      const int64_t s1 = a.cum[r + 1];
      const int64_t key = a.run[r];
      const int64_t qf = a.chunk_start[r];  // the run's first chunk
      const int64_t q1 = qf + (s1 - s0 + kChunk - 1) / kChunk;
      const int64_t t = table_of(a, a.infos[s0]);  // a feature of the run's table
      const int32_t D = FULL ? G * NCH * 4 : mv.D_off(t + 1) - mv.D_off(t);
      const int64_t idx = key - mv.hsc(t);
      const int64_t row0 = mv.w_off(t) + idx * D;
      WT* wrow = static_cast<WT*>(a.W) + row0;
      float* hp = a.m1 + mv.m1_off(t) + idx;
      float w[NCH][4];
      float h0 = 0.0f;
      if (grp == 0) {  // the row and its momentum load while the partials are summed
#pragma unroll
        for (int c = 0; c < NCH; ++c)
          if (col_in<FULL, G>(c, k, D)) ld_row4(wrow + (c * G + k) * 4, w[c]);
        h0 = *hp;
      }
      float gs[NCH][4];
#pragma unroll
      for (int c = 0; c < NCH; ++c)
#pragma unroll
        for (int e = 0; e < 4; ++e) gs[c][e] = 0.0f;
      for (int64_t qq = qf + grp; qq < q1; qq += NG * U) {
        float v[U][NCH][4];
#pragma unroll
        for (int u = 0; u < U; ++u)
          if (qq + u * NG < q1)
#pragma unroll
            for (int c = 0; c < NCH; ++c)
              if (col_in<FULL, G>(c, k, D)) ld4(a.partial + (qq + u * NG) * a.max_D + (c * G + k) * 4, v[u][c]);
#pragma unroll
        for (int u = 0; u < U; ++u)
          if (qq + u * NG < q1)
#pragma unroll
            for (int c = 0; c < NCH; ++c)
              if (col_in<FULL, G>(c, k, D))
#pragma unroll
                for (int e = 0; e < 4; ++e) gs[c][e] += v[u][c][e];
      }
#pragma unroll
      for (int c = 0; c < NCH; ++c)
#pragma unroll
        for (int e = 0; e < 4; ++e) part[grp][(c * G + k) * 4 + e] = gs[c][e];
      __syncthreads();
      if (grp == 0) {
#pragma unroll
        for (int c = 0; c < NCH; ++c)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float x = part[0][(c * G + k) * 4 + e];
            for (int j = 1; j < NG; ++j) x += part[j][(c * G + k) * 4 + e];
            gs[c][e] = x;
          }
        adagrad_update<G, NCH, FULL>(a, D, k, gs, w, wrow, row0, hp, h0);
      }
      __syncthreads();
    }
    __syncthreads();  // s_runs / s_nruns are rewritten for the next range
  }
}

// Pass A: one group per chunk of a long run -> partial sum in the workspace.
template <typename I, int G, int NCH, int U, bool FULL, bool PLAIN>
__global__ void __launch_bounds__(256) bwd_chunk_kernel(BwdArgs a) {
  pin_options<PLAIN>(a);
  if (call_failed(a.fail)) return;  // the run layout is not valid
  __shared__ TableMeta meta;
  stage_meta(a, meta);
  const MetaView mv{a, meta, a.T <= kMaxCachedTables};
  constexpr int P = 64 / G;
  const int lane = threadIdx.x & 63;
  const int g = lane / G, k = lane % G;
  const XcdRange xr = xcd_range<P>(*a.total_chunks, blockIdx.x, gridDim.x);
  for (int64_t qb = xr.first; qb < xr.end; qb += xr.step) {
    const int64_t q = qb + g;
    if (q >= xr.end) continue;
    // Owner: the nearest chunk mark at or before q (lane k < kMarkEvery reads
    // chunk q - k; the smallest k with a mark wins).
    static_assert(G >= kMarkEvery, "a group covers the mark spacing");
    const uint32_t m = k < kMarkEvery && q - k >= 0 ? a.chunk_mark[q - k] : 0u;
    uint64_t bal = __ballot(m != 0u);
    if constexpr (G < 64) bal = (bal >> (g * G)) & ((1ull << G) - 1ull);
    const int nearest = __ffsll(static_cast<long long>(bal)) - 1;  // always a mark within reach
    const int64_t r = static_cast<int64_t>((__shfl(m, g * G + nearest, 64) & ~kRunStart) - 1u);
    const int64_t s0 = a.cum[r] + (q - a.chunk_start[r]) * kChunk;
    const int64_t e0 = a.cum[r + 1];
    const int64_t s1 = s0 + kChunk < e0 ? s0 + kChunk : e0;
    const int32_t info0 = k < s1 - s0 ? a.infos[s0 + k] : 0;
    const int64_t t = table_of(a, __shfl(info0, g * G, 64));
    const int32_t D = FULL ? G * NCH * 4 : mv.D_off(t + 1) - mv.D_off(t);
    float acc[NCH][4];
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[c][e] = 0.0f;
    group_sum_occurrences<I, G, NCH, U, FULL>(a, mv, D, s0, s1, g, k, info0, acc);
    float* dst = a.partial + q * a.max_D;
#pragma unroll
    for (int c = 0; c < NCH; ++c)
      if (col_in<FULL, G>(c, k, D)) st4(dst + (c * G + k) * 4, acc[c]);
  }
}

// Pass B (runs of at most kLong occurrences): one G-lane group per run --
// gradient sum in sorted order, rowwise Adagrad, in-place update.  The
// table of a run comes from the first batch of infos, which is kept for the
// gradient sum.
template <typename I, typename WT, int G, int NCH, int U, bool FULL>
__device__ __forceinline__ void short_run_body(const BwdArgs& a, const MetaView& mv, int64_t bid,
                                               int64_t nblk) {
  constexpr int P = 64 / G;
  const int lane = threadIdx.x & 63;
  const int g = lane / G, k = lane % G;
  const XcdRange xr = xcd_range<P>(*a.num_runs, bid, nblk);
  for (int64_t r = xr.first + g; r < xr.end; r += xr.step) {
    const int64_t cs0 = a.cum[r];
    const int64_t cs1 = a.cum[r + 1];
    const int64_t ckey = a.run[r];
    if (cs1 - cs0 > kLong) continue;  // long runs: long_run_body
    const int32_t info0 = k < cs1 - cs0 ? a.infos[cs0 + k] : 0;
    const int64_t t = table_of(a, __shfl(info0, g * G, 64));
    const int32_t D = FULL ? G * NCH * 4 : mv.D_off(t + 1) - mv.D_off(t);
    const int64_t idx = ckey - mv.hsc(t);
    const int64_t row0 = mv.w_off(t) + idx * D;
    WT* wrow = static_cast<WT*>(a.W) + row0;
    float* hp = a.m1 + mv.m1_off(t) + idx;
    float w[NCH][4];
#pragma unroll
    for (int c = 0; c < NCH; ++c)
      if (col_in<FULL, G>(c, k, D)) ld_row4(wrow + (c * G + k) * 4, w[c]);
    const float h0 = *hp;
    float gs[NCH][4];
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e) gs[c][e] = 0.0f;
    group_sum_occurrences<I, G, NCH, U, FULL>(a, mv, D, cs0, cs1, g, k, info0, gs);
    adagrad_update<G, NCH, FULL>(a, D, k, gs, w, wrow, row0, hp, h0);
  }
}

// Both run classes in one launch: they update disjoint rows and momentum
// words and need nothing of each other.  The first `nlong` blocks (a multiple
// of 8, so that block i of the short-run part still runs on XCD i % 8) combine
// the long runs' chunk partials; the others sum and update the short runs.
// The long-run blocks are latency-bound and finish under the short-run
// blocks' row read-modify-writes (config 3: 164.7 us per backward against
// 175.5 with the long runs on a second stream, forked and joined around the
// update).  Rows of up to 2 float4 chunks per lane are held to 80 registers
// (6 waves per SIMD, the short-run part's own occupancy; a few long-run
// values spill): 5 waves per SIMD took 167.5 us.
template <int NCH>
constexpr int runs_waves() {
  return NCH <= 2 ? 6 : 1;
}

template <typename I, typename WT, int G, int NCH, int U, int GL, int NCHL, int UL, bool FULL,
          bool PLAIN>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(runs_waves<NCH>())))
    bwd_runs_kernel(BwdArgs a, int64_t nlong) {
  // The early words go back to zero for the stream's next call, also when
  // this call failed (every block passes here before it may return).
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < a.rezero_words;
       i += static_cast<int64_t>(gridDim.x) * 256)
    a.rezero[i] = 0ull;
  pin_options<PLAIN>(a);
  if (call_failed(a.fail)) return;  // the run layout is not valid
  __shared__ TableMeta meta;
  stage_meta(a, meta);
  const MetaView mv{a, meta, a.T <= kMaxCachedTables};
  if (static_cast<int64_t>(blockIdx.x) < nlong)
    long_run_body<WT, GL, NCHL, UL, FULL>(a, mv, blockIdx.x, nlong);
  else
    short_run_body<I, WT, G, NCH, U, FULL>(a, mv, blockIdx.x - nlong, gridDim.x - nlong);
}

// After the run encoding: the chunk layout of the long runs (chunk-count
// scan), their chunk partial sums, then both run classes in one launch.
template <typename I, typename WT, int G, int NCH, bool FULL, bool PLAIN>
int launch_bwd(const BwdArgs& a, SortWs& ws, uint32_t* chunk_start, int64_t N, hipStream_t s) {
  if (int rc = prefix_scan_epi(
          ChunkCount{a.cum}, N, reinterpret_cast<const int32_t*>(a.num_runs),
          ChunkEpi{a.cum, chunk_start, ws.chunk_mark, &ws.counters[1]}, scan_slot(ws, 1), s))
    return rc;
  constexpr int P = 64 / G;
  const int64_t cus = num_cus();
  const int64_t want = ceil_div(N, 4 * P);
  const int64_t nblk = want < 1 ? 1 : (want > cus * 16 ? cus * 16 : want);
  const int64_t ngrid = ceil_div(nblk, 8) * 8;  // whole rounds over the XCDs
  constexpr int UC = NCH <= 1 ? 8 : (NCH <= 2 ? 8 : 4);  // chunks are full: more in flight
  bwd_chunk_kernel<I, G, NCH, UC, FULL, PLAIN><<<dim3(static_cast<uint32_t>(ngrid)), 256, 0, s>>>(a);
  MX_LAUNCH_CHECK();
  // Long runs: twice the lanes per row where the row allows (more groups
  // summing partials per block; measured 15.1 -> 12.4 us on config 3).
  constexpr int GL = NCH >= 2 && G < 64 ? 2 * G : G;
  constexpr int NCHL = GL == 2 * G ? NCH / 2 : NCH;
  constexpr int U = NCH <= 1 ? 4 : 2;  // short runs: keep registers low
  const int64_t long_want = ceil_div(max_chunks(N), kLongRange);
  const int64_t long_cap = cus * kLongBlocksPerCu;
  const int64_t nlong = ceil_div(long_want < long_cap ? long_want : long_cap, 8) * 8;
  bwd_runs_kernel<I, WT, G, NCH, U, GL, NCHL, 4, FULL, PLAIN>
      <<<dim3(static_cast<uint32_t>(nlong + ngrid)), 256, 0, s>>>(a, nlong);
  MX_LAUNCH_CHECK();
  return MX_OK;
}

// Full-width instance when every table's D equals the row width of the
// chosen (G, NCH): total_D = T * max_D says so (no D exceeds max_D, and the
// D_offsets sum to total_D: a fixed batch's grad_output width, the recast
// sequence batch's T * D; a variable batch passes 0).  Plain instance for SUM
// pooling without weights or weight decay.
template <typename I, typename WT, int G, int NCH>
int launch_width(const BwdArgs& a, SortWs& ws, uint32_t* chunk_start, int64_t N, hipStream_t s) {
  constexpr int kWidth = G * NCH * 4;
  const bool full = a.max_D == kWidth && a.total_D == static_cast<int64_t>(a.T) * kWidth;
  const bool plain = a.pooling == MX_POOL_SUM && a.iw_sorted == nullptr && a.B_off == nullptr &&
                     a.wd_mode == 0;
  if (full)
    return plain ? launch_bwd<I, WT, G, NCH, true, true>(a, ws, chunk_start, N, s)
                 : launch_bwd<I, WT, G, NCH, true, false>(a, ws, chunk_start, N, s);
  return plain ? launch_bwd<I, WT, G, NCH, false, true>(a, ws, chunk_start, N, s)
               : launch_bwd<I, WT, G, NCH, false, false>(a, ws, chunk_start, N, s);
}

// Lanes per run (G) and float4 chunks per lane (NCH) from the widest table.
template <typename I, typename WT>
int dispatch_bwd(const BwdArgs& a, SortWs& ws, uint32_t* chunk_start, int64_t N, hipStream_t s) {
  if (a.max_D <= 64) return launch_width<I, WT, 16, 1>(a, ws, chunk_start, N, s);
  if (a.max_D <= 128) return launch_width<I, WT, 16, 2>(a, ws, chunk_start, N, s);
  if (a.max_D <= 256) return launch_width<I, WT, 32, 2>(a, ws, chunk_start, N, s);
  if (a.max_D <= 512) return launch_width<I, WT, 64, 2>(a, ws, chunk_start, N, s);
  return launch_width<I, WT, 64, 4>(a, ws, chunk_start, N, s);
}

struct BwdWs {
  SortWs sort;
  int64_t* sorted;
  int32_t* infos;
  int64_t* run;
  int32_t* cum;
  uint32_t* chunk_start;
  float* weights_sorted;
  float* partial;
  size_t bytes;
};


BwdWs carve_bwd(uint8_t* base, int64_t N, int32_t max_D) {
  BwdWs w{};
  w.sort = carve_sort(base, N);
  size_t off = w.sort.bytes;
  const int64_t n = N > 0 ? N : 1;
  auto take = [&](size_t bytes) {
    uint8_t* p = base ? base + off : nullptr;
    off += align256(bytes);
    return p;
  };
  w.sorted = reinterpret_cast<int64_t*>(take(n * 8));
  w.infos = reinterpret_cast<int32_t*>(take(n * 4));
  w.run = reinterpret_cast<int64_t*>(take(n * 8));
  w.cum = reinterpret_cast<int32_t*>(take((n + 1) * 4));
  w.chunk_start = reinterpret_cast<uint32_t*>(take((n + 1) * 4));
  w.weights_sorted = reinterpret_cast<float*>(take(n * 4));
  w.partial = reinterpret_cast<float*>(take(static_cast<size_t>(max_chunks(n)) * max_D * 4));
  w.bytes = off;
  return w;
}

}  // namespace
}  // namespace mx

using namespace mx;

extern "C" int32_t mx_tbe_info_B_num_bits(int32_t T, int64_t B) {
  if (T < 0 || B < 0) return -1;
  int tb = 0;
  while ((int64_t(1) << tb) < T) ++tb;  // bits for t in [0, T)
  int bb = 1;
  while ((int64_t(1) << bb) < B) ++bb;  // bits for b in [0, B)
  if (tb + bb > 32) return -1;
  // 26 bits for b (room for 64 tables) unless T or B need a different split.
  if (bb <= 26 && tb <= 6) return 26;
  return 32 - tb;
}

extern "C" size_t mx_tbe_transpose_workspace_bytes(int64_t N, int32_t total_hash_size_bits) {
  (void)total_hash_size_bits;
  return carve_sort(nullptr, N).bytes;
}

namespace {

// Batch layout of a call: a fixed batch B per table (all pointers null,
// nbags = T * B), or variable batch per feature (VBE): b_t_map [nbags] info
// word (t << info_B_num_bits) | b of each bag, and for the backward also
// B_offsets [T+1] (first bag of each table) and row_out [nbags] (gradient row
// offset of each bag).
struct Layout {
  int64_t nbags;
  const int32_t* B_offsets;
  const int64_t* row_out;
  const int32_t* b_t_map;
};

int check_common(int32_t T, int64_t B, const Layout& lay, int32_t bits, int32_t nb,
                 int32_t index_bytes, int64_t N) {
  MX_REQUIRE(T >= 0 && B >= 0 && N >= 0 && lay.nbags >= 0, "negative size");
  MX_REQUIRE(bits >= 0 && bits <= 32, "total_hash_size_bits %d not in [0, 32]", bits);
  MX_REQUIRE(index_bytes == 4 || index_bytes == 8, "indices must be int32 or int64");
  MX_REQUIRE(N < 0x7fffffffll, "N %lld too large for int32 run offsets", (long long)N);
  MX_REQUIRE(nb >= 1 && nb <= 32, "info_B_num_bits %d invalid", nb);
  MX_REQUIRE(B <= (int64_t(1) << nb), "B does not fit info_B_num_bits");
  MX_REQUIRE(N == 0 || (T > 0 && lay.nbags > 0), "%lld indices but no bags (T=%d, bags=%lld)",
             (long long)N, T, (long long)lay.nbags);
  return MX_OK;
}

int transpose_impl(const int64_t* hash_size_cumsum, int32_t T, int64_t B, const Layout& lay,
                   int32_t total_hash_size_bits, int32_t info_B_num_bits, const void* indices,
                   const void* offsets, int32_t index_bytes, int64_t N, int64_t* linear_indices,
                   int64_t* sorted_linear_indices, int32_t* infos_sorted,
                   int64_t* sorted_linear_indices_run, int32_t* run_lengths, int32_t* num_runs,
                   int32_t* cumulative_run_lengths, void* workspace, size_t workspace_bytes,
                   void* stream) {
  if (int rc = check_common(T, B, lay, total_hash_size_bits, info_B_num_bits, index_bytes, N))
    return rc;
  auto* s = as_stream(stream);
  if (N == 0) {  // no runs: num_runs = 0, cumulative_run_lengths = {0}
    if (num_runs || cumulative_run_lengths) {
      zero_two_kernel<<<1, 64, 0, s>>>(num_runs, cumulative_run_lengths);
      MX_LAUNCH_CHECK();
    }
    return MX_OK;
  }
  MX_REQUIRE(hash_size_cumsum && indices && offsets && sorted_linear_indices && infos_sorted &&
                 sorted_linear_indices_run && run_lengths && num_runs && cumulative_run_lengths,
             "null pointer argument");
  SortWs w = carve_sort(static_cast<uint8_t*>(workspace), N);
  if (workspace == nullptr || workspace_bytes < w.bytes)
    return set_error(MX_EWORKSPACE, "workspace of %zu bytes needed", w.bytes);
  TransposeOut o{linear_indices, sorted_linear_indices, infos_sorted, sorted_linear_indices_run,
                 run_lengths, num_runs, cumulative_run_lengths, nullptr};
  return run_transpose(hash_size_cumsum, T, B, lay.nbags, lay.b_t_map, lay.B_offsets,
                       total_hash_size_bits,
                       info_B_num_bits, indices, offsets, index_bytes, N, nullptr, o, w, s,
                       nullptr);
}

int backward_impl(void* weights, int32_t weights_ty, const int64_t* weights_offsets,
                  const int32_t* D_offsets, int32_t T, int64_t B, int32_t nb, const Layout& lay,
                  int32_t max_D, const int64_t* hash_size_cumsum, int32_t total_hash_size_bits,
                  const void* indices, const void* offsets, int32_t index_bytes, int64_t N,
                  int32_t pooling_mode, const float* indice_weights, const float* grad_output,
                  int64_t total_D, float* momentum1, const int64_t* momentum1_offsets,
                  float learning_rate, float eps, float weight_decay, int32_t weight_decay_mode,
                  int32_t stochastic_rounding, const mx_rng_state* rng, void* workspace,
                  size_t workspace_bytes, void* stream) {
  if (int rc = check_common(T, B, lay, total_hash_size_bits, nb, index_bytes, N)) return rc;
  MX_REQUIRE(max_D > 0 && max_D <= 1024 && max_D % 4 == 0,
             "max_D %d must be a multiple of 4 in [4, 1024]", max_D);
  MX_REQUIRE(pooling_mode == MX_POOL_SUM || pooling_mode == MX_POOL_MEAN,
             "pooling_mode %d not supported (SUM=0, MEAN=1)", pooling_mode);
  MX_REQUIRE(weight_decay_mode >= 0 && weight_decay_mode <= 2,
             "weight_decay_mode %d not supported (0 none, 1 L2, 2 decoupled)", weight_decay_mode);
  MX_REQUIRE(weights_ty == MX_SPARSE_FP32 || weights_ty == MX_SPARSE_FP16,
             "weights type %d not supported (FP32=0, FP16=1)", weights_ty);
  if (N == 0) return MX_OK;
  MX_REQUIRE(weights && weights_offsets && D_offsets && hash_size_cumsum && indices && offsets &&
                 grad_output && momentum1 && momentum1_offsets,
             "null pointer argument");
  BwdWs w = carve_bwd(static_cast<uint8_t*>(workspace), N, max_D);
  if (workspace == nullptr || workspace_bytes < w.bytes)
    return set_error(MX_EWORKSPACE, "workspace of %zu bytes needed", w.bytes);
  auto* s = as_stream(stream);
  TransposeOut o{nullptr, w.sorted, w.infos, w.run, nullptr, nullptr, w.cum,
                 indice_weights ? w.weights_sorted : nullptr};
  ZeroedRegion* zr = stream_region(s);
  std::unique_lock<std::mutex> zr_lock;
  if (zr) zr_lock = std::unique_lock<std::mutex>(zr->mu);
  if (int rc = run_transpose(hash_size_cumsum, T, B, lay.nbags, lay.b_t_map, lay.B_offsets,
                             total_hash_size_bits, nb, indices, offsets, index_bytes, N,
                             indice_weights, o, w.sort, s, zr))
    return rc;
  BwdArgs a;
  a.rezero = zr ? reinterpret_cast<unsigned long long*>(zr->base) : nullptr;
  a.rezero_words = zr ? w.sort.early_words : 0;
  a.W = weights;
  a.w_off = weights_offsets;
  a.D_off = D_offsets;
  a.hsc = hash_size_cumsum;
  a.offsets = offsets;
  a.grad = grad_output;
  a.m1 = momentum1;
  a.m1_off = momentum1_offsets;
  a.run = w.run;
  a.cum = w.cum;
  a.infos = w.infos;
  a.iw_sorted = indice_weights ? w.weights_sorted : nullptr;
  a.B_off = lay.b_t_map ? lay.B_offsets : nullptr;
  a.row_out = lay.b_t_map ? lay.row_out : nullptr;
  a.num_runs = &w.sort.counters[0];
  a.chunk_start = w.chunk_start;
  a.chunk_mark = w.sort.chunk_mark;
  a.T = T;
  a.total_chunks = &w.sort.counters[1];
  a.partial = w.partial;
  a.fail = w.sort.fail;
  a.B = B;
  a.total_D = total_D;
  a.max_D = max_D;
  a.nb = nb;
  a.pooling = pooling_mode;
  a.wd_mode = weight_decay_mode;
  a.lr = learning_rate;
  a.eps = eps;
  a.wd = weight_decay;
  a.sr = stochastic_rounding != 0 ? 1 : 0;
  MX_REQUIRE(!a.sr || rng != nullptr, "stochastic rounding needs a random state");
  a.seed = a.sr ? rng->seed : 0;
  a.offset = a.sr ? rng->offset : 0;
  a.seed_dev = a.sr ? rng->seed_dev : nullptr;
  a.offset_dev = a.sr ? rng->offset_dev : nullptr;
  int rc;
  if (weights_ty == MX_SPARSE_FP16)
    rc = index_bytes == 8 ? dispatch_bwd<int64_t, __half>(a, w.sort, w.chunk_start, N, s)
                          : dispatch_bwd<int32_t, __half>(a, w.sort, w.chunk_start, N, s);
  else
    rc = index_bytes == 8 ? dispatch_bwd<int64_t, float>(a, w.sort, w.chunk_start, N, s)
                          : dispatch_bwd<int32_t, float>(a, w.sort, w.chunk_start, N, s);
  if (zr && rc == MX_OK) zr->dirty = false;  // the update launch clears the region
  return rc;
}

}  // namespace

extern "C" int mx_tbe_transpose_embedding_input(
    const int64_t* hash_size_cumsum, int32_t T, int64_t B, int32_t total_hash_size_bits,
    int32_t info_B_num_bits, const void* indices, const void* offsets, int32_t index_bytes,
    int64_t N, int64_t* linear_indices, int64_t* sorted_linear_indices, int32_t* infos_sorted,
    int64_t* sorted_linear_indices_run, int32_t* run_lengths, int32_t* num_runs,
    int32_t* cumulative_run_lengths, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  const Layout lay{static_cast<int64_t>(T) * B, nullptr, nullptr, nullptr};
  return transpose_impl(hash_size_cumsum, T, B, lay, total_hash_size_bits, info_B_num_bits,
                        indices, offsets, index_bytes, N, linear_indices, sorted_linear_indices,
                        infos_sorted, sorted_linear_indices_run, run_lengths, num_runs,
                        cumulative_run_lengths, workspace, workspace_bytes, stream);
}

extern "C" int mx_tbe_transpose_embedding_input_vbe(
    const int64_t* hash_size_cumsum, int32_t T, int64_t total_B, const int32_t* vbe_b_t_map,
    int32_t total_hash_size_bits, int32_t info_B_num_bits, const void* indices,
    const void* offsets, int32_t index_bytes, int64_t N, int64_t* linear_indices,
    int64_t* sorted_linear_indices, int32_t* infos_sorted, int64_t* sorted_linear_indices_run,
    int32_t* run_lengths, int32_t* num_runs, int32_t* cumulative_run_lengths, void* workspace,
    size_t workspace_bytes, void* stream) {
  clear_error();
  MX_REQUIRE(total_B == 0 || vbe_b_t_map, "VBE needs the b_t map");
  // Sorting needs only each bag's info word.
  const Layout lay{total_B, nullptr, nullptr, vbe_b_t_map};
  return transpose_impl(hash_size_cumsum, T, 0, lay, total_hash_size_bits, info_B_num_bits,
                        indices, offsets, index_bytes, N, linear_indices, sorted_linear_indices,
                        infos_sorted, sorted_linear_indices_run, run_lengths, num_runs,
                        cumulative_run_lengths, workspace, workspace_bytes, stream);
}

extern "C" size_t mx_tbe_backward_workspace_bytes(int64_t N, int32_t total_hash_size_bits,
                                                  int32_t max_D) {
  (void)total_hash_size_bits;
  return carve_bwd(nullptr, N, max_D > 0 ? max_D : 1).bytes;
}

extern "C" int mx_tbe_backward_rowwise_adagrad(
    void* weights, int32_t weights_ty, const int64_t* weights_offsets, const int32_t* D_offsets,
    int32_t T, int64_t B, int32_t max_D, const int64_t* hash_size_cumsum, int32_t total_hash_size_bits,
    const void* indices, const void* offsets, int32_t index_bytes, int64_t N,
    int32_t pooling_mode, const float* indice_weights, const float* grad_output, int64_t total_D,
    float* momentum1, const int64_t* momentum1_offsets, float learning_rate, float eps,
    float weight_decay, int32_t weight_decay_mode, int32_t stochastic_rounding,
    const mx_rng_state* rng, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  const int32_t nb = mx_tbe_info_B_num_bits(T, B);
  MX_REQUIRE(nb > 0, "T=%d, B=%lld do not fit a 32-bit info word", T, (long long)B);
  const Layout lay{static_cast<int64_t>(T) * B, nullptr, nullptr, nullptr};
  return backward_impl(weights, weights_ty, weights_offsets, D_offsets, T, B, nb, lay, max_D,
                       hash_size_cumsum, total_hash_size_bits, indices, offsets, index_bytes, N,
                       pooling_mode, indice_weights, grad_output, total_D, momentum1,
                       momentum1_offsets, learning_rate, eps, weight_decay, weight_decay_mode,
                       stochastic_rounding, rng, workspace, workspace_bytes, stream);
}

extern "C" int mx_tbe_backward_rowwise_adagrad_vbe(
    void* weights, int32_t weights_ty, const int64_t* weights_offsets, const int32_t* D_offsets,
    int32_t T, int64_t max_B, int32_t max_D, const int64_t* hash_size_cumsum,
    int32_t total_hash_size_bits, const void* indices, const void* offsets, int32_t index_bytes,
    int64_t N, int32_t pooling_mode, const float* indice_weights, const float* grad_output,
    int64_t total_B, const int32_t* B_offsets, const int64_t* vbe_row_output_offsets,
    const int32_t* vbe_b_t_map, int32_t info_B_num_bits, float* momentum1,
    const int64_t* momentum1_offsets, float learning_rate, float eps, float weight_decay,
    int32_t weight_decay_mode, int32_t stochastic_rounding, const mx_rng_state* rng,
    void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  MX_REQUIRE(total_B == 0 || (B_offsets && vbe_row_output_offsets && vbe_b_t_map),
             "VBE needs B_offsets, row output offsets and the b_t map");
  const Layout lay{total_B, B_offsets, vbe_row_output_offsets, vbe_b_t_map};
  return backward_impl(weights, weights_ty, weights_offsets, D_offsets, T, max_B,
                       info_B_num_bits, lay, max_D, hash_size_cumsum, total_hash_size_bits,
                       indices, offsets, index_bytes, N, pooling_mode, indice_weights,
                       grad_output, 0, momentum1, momentum1_offsets, learning_rate, eps,
                       weight_decay, weight_decay_mode, stochastic_rounding, rng, workspace,
                       workspace_bytes, stream);
}

// ---- sequence lookups (PoolingMode NONE) -----------------------------------
//
// Semantics: fbgemm_gpu split_embedding_nobag_backward_codegen_rowwise_adagrad_
// unweighted_exact_cuda and transpose_embedding_input(nobag=True) (recalled):
// every position l of bag (t, b) is its own occurrence with its own gradient
// row grad_output[l, :] (all tables of width D); each distinct (t, i) sums the
// rows of its occurrences in sorted (position) order and takes the rowwise
// Adagrad step of the pooled backward.  The nobag transpose's info of a
// position is l * T + t (int64).
//
// Design: the batch is recast as a variable batch in which every position is
// a bag of length one: bag l has offsets l and l + 1, belongs to table t with
// b = l - offsets[t*B] (the b_t word (t << nb) | b), and its gradient row
// starts at l * D.  The sort, run encoding and update then run unchanged.
// Needs offsets[0] = 0 and offsets[T*B] = N, as upstream.
namespace mx {
namespace {

constexpr int kNobagMaxT = 1024;  // tables whose first positions fit LDS

template <typename I>
__global__ void __launch_bounds__(256)
    nobag_layout_kernel(const I* __restrict__ offsets, int32_t T, int64_t B, int64_t N,
                        int32_t D, int32_t nb, I* __restrict__ bag_offsets,
                        int32_t* __restrict__ b_t_map, int64_t* __restrict__ row_out,
                        int32_t* __restrict__ B_offsets, int32_t* __restrict__ D_offsets) {
  __shared__ int64_t s_pos[kNobagMaxT + 1];
  const bool lds = T <= kNobagMaxT;
  if (lds)
    for (int t = threadIdx.x; t <= T; t += 256) s_pos[t] = static_cast<int64_t>(offsets[t * B]);
  __syncthreads();
  if (blockIdx.x == 0) {
    for (int t = threadIdx.x; t <= T; t += 256) {
      if (B_offsets) B_offsets[t] = static_cast<int32_t>(offsets[t * B]);
      if (D_offsets) D_offsets[t] = t * D;
    }
    if (threadIdx.x == 0) bag_offsets[N] = static_cast<I>(N);
  }
  for (int64_t l = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; l < N;
       l += static_cast<int64_t>(gridDim.x) * 256) {
    int32_t lo = 0, hi = T;  // pos[lo] <= l < pos[hi] (lo = 0 or T - 1 outside every bag)
    while (hi - lo > 1) {
      const int32_t mid = lo + ((hi - lo) >> 1);
      const int64_t pm = lds ? s_pos[mid] : static_cast<int64_t>(offsets[mid * B]);
      if (pm <= l)
        lo = mid;
      else
        hi = mid;
    }
    const int64_t p = lds ? s_pos[lo] : static_cast<int64_t>(offsets[lo * B]);
    const int64_t b = l - p > 0 ? l - p : 0;
    bag_offsets[l] = static_cast<I>(l);
    b_t_map[l] = static_cast<int32_t>((nb >= 32 ? 0u : (static_cast<uint32_t>(lo) << nb)) |
                                      static_cast<uint32_t>(b));
    if (row_out) row_out[l] = l * D;
  }
}

// Sorted (t << nb) | b words of the recast batch -> the nobag infos l * T + t.
template <typename I>
__global__ void __launch_bounds__(256)
    nobag_infos_kernel(const int32_t* __restrict__ infos, const I* __restrict__ offsets,
                       int32_t T, int64_t B, int64_t N, int32_t nb, int64_t* __restrict__ out) {
  const uint32_t bmask = nb >= 32 ? 0xffffffffu : ((1u << nb) - 1u);
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < N;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const uint32_t w = static_cast<uint32_t>(infos[i]);
    const int64_t t = nb >= 32 ? 0 : static_cast<int64_t>(w >> nb);
    const int64_t l = static_cast<int64_t>(offsets[t * B]) + static_cast<int64_t>(w & bmask);
    out[i] = l * T + t;
  }
}

// The recast batch's arrays, after the backward's (or transpose's) workspace.
struct NobagWs {
  void* bag_offsets;  // [N + 1] of the index type
  int32_t* b_t_map;   // [N]
  int64_t* row_out;   // [N]
  int32_t* B_offsets; // [T + 1]
  int32_t* D_offsets; // [T + 1]
  int32_t* infos;     // [N] (transpose: the sorted b_t words)
  size_t bytes;
};

NobagWs carve_nobag(uint8_t* base, size_t off, int64_t N, int32_t T, int32_t index_bytes) {
  NobagWs w{};
  auto take = [&](size_t bytes) {
    uint8_t* p = base ? base + off : nullptr;
    off += align256(bytes);
    return p;
  };
  const int64_t n = N > 0 ? N : 1;
  w.bag_offsets = take(static_cast<size_t>(n + 1) * static_cast<size_t>(index_bytes));
  w.b_t_map = reinterpret_cast<int32_t*>(take(n * 4));
  w.row_out = reinterpret_cast<int64_t*>(take(n * 8));
  w.B_offsets = reinterpret_cast<int32_t*>(take(static_cast<size_t>(T + 1) * 4));
  w.D_offsets = reinterpret_cast<int32_t*>(take(static_cast<size_t>(T + 1) * 4));
  w.infos = reinterpret_cast<int32_t*>(take(n * 4));
  w.bytes = off;
  return w;
}

int launch_nobag_layout(const void* offsets, int32_t index_bytes, int32_t T, int64_t B,
                        int64_t N, int32_t D, int32_t nb, const NobagWs& w, bool backward,
                        hipStream_t s) {
  const int64_t want = ceil_div(N, 256);
  const int64_t cap = static_cast<int64_t>(num_cus()) * 8;
  const dim3 gd(static_cast<uint32_t>(want < 1 ? 1 : (want < cap ? want : cap)));
  if (index_bytes == 8)
    nobag_layout_kernel<int64_t><<<gd, 256, 0, s>>>(
        static_cast<const int64_t*>(offsets), T, B, N, D, nb,
        static_cast<int64_t*>(w.bag_offsets), w.b_t_map, backward ? w.row_out : nullptr,
        w.B_offsets, backward ? w.D_offsets : nullptr);
  else
    nobag_layout_kernel<int32_t><<<gd, 256, 0, s>>>(
        static_cast<const int32_t*>(offsets), T, B, N, D, nb,
        static_cast<int32_t*>(w.bag_offsets), w.b_t_map, backward ? w.row_out : nullptr,
        w.B_offsets, backward ? w.D_offsets : nullptr);
  MX_LAUNCH_CHECK();
  return MX_OK;
}

int check_nobag(int32_t T, int64_t B, int32_t D, int32_t index_bytes, int64_t N) {
  MX_REQUIRE(T >= 0 && B >= 0 && N >= 0, "negative T, B or N");
  MX_REQUIRE(D > 0 && D <= 1024 && D % 4 == 0, "D %d must be a multiple of 4 in [4, 1024]", D);
  MX_REQUIRE(index_bytes == 4 || index_bytes == 8, "indices must be int32 or int64");
  MX_REQUIRE(N < 0x7fffffffll, "N %lld too large for int32 positions", (long long)N);
  MX_REQUIRE(N == 0 || (T > 0 && B > 0), "%lld indices but no bags (T=%d, B=%lld)",
             (long long)N, T, (long long)B);
  return MX_OK;
}

}  // namespace
}  // namespace mx

extern "C" size_t mx_tbe_backward_nobag_workspace_bytes(int64_t N, int32_t T,
                                                        int32_t total_hash_size_bits, int32_t D) {
  (void)total_hash_size_bits;
  const size_t base = carve_bwd(nullptr, N, D > 0 ? D : 1).bytes;
  return carve_nobag(nullptr, base, N, T > 0 ? T : 0, 8).bytes;
}

extern "C" int mx_tbe_backward_rowwise_adagrad_nobag(
    void* weights, int32_t weights_ty, const int64_t* weights_offsets, int32_t T, int64_t B,
    int32_t D, const int64_t* hash_size_cumsum, int32_t total_hash_size_bits,
    const void* indices, const void* offsets, int32_t index_bytes, int64_t N,
    const float* grad_output, float* momentum1, const int64_t* momentum1_offsets,
    float learning_rate, float eps, float weight_decay, int32_t weight_decay_mode,
    int32_t stochastic_rounding, const mx_rng_state* rng, void* workspace,
    size_t workspace_bytes, void* stream) {
  clear_error();
  if (int rc = check_nobag(T, B, D, index_bytes, N)) return rc;
  if (N == 0) return MX_OK;
  MX_REQUIRE(offsets && workspace, "null pointer argument");
  const int32_t nb = mx_tbe_info_B_num_bits(T, N);
  MX_REQUIRE(nb > 0, "T=%d and N=%lld do not fit a 32-bit info word", T, (long long)N);
  const size_t base = carve_bwd(nullptr, N, D).bytes;
  const NobagWs nw = carve_nobag(static_cast<uint8_t*>(workspace), base, N, T, index_bytes);
  if (workspace_bytes < nw.bytes)
    return set_error(MX_EWORKSPACE, "workspace of %zu bytes needed", nw.bytes);
  auto* s = as_stream(stream);
  if (int rc = launch_nobag_layout(offsets, index_bytes, T, B, N, D, nb, nw, true, s)) return rc;
  const Layout lay{N, nw.B_offsets, nw.row_out, nw.b_t_map};
  // total_D = T * D: every table is D wide (the full-width instances apply).
  return backward_impl(weights, weights_ty, weights_offsets, nw.D_offsets, T, N, nb, lay, D,
                       hash_size_cumsum, total_hash_size_bits, indices, nw.bag_offsets,
                       index_bytes, N, MX_POOL_SUM, nullptr, grad_output,
                       static_cast<int64_t>(T) * D, momentum1,
                       momentum1_offsets, learning_rate, eps, weight_decay, weight_decay_mode,
                       stochastic_rounding, rng, workspace, base, stream);
}

extern "C" size_t mx_tbe_transpose_nobag_workspace_bytes(int64_t N, int32_t T,
                                                         int32_t total_hash_size_bits) {
  (void)total_hash_size_bits;
  return carve_nobag(nullptr, carve_sort(nullptr, N).bytes, N, T > 0 ? T : 0, 8).bytes;
}

extern "C" int mx_tbe_transpose_embedding_input_nobag(
    const int64_t* hash_size_cumsum, int32_t T, int64_t B, int32_t total_hash_size_bits,
    const void* indices, const void* offsets, int32_t index_bytes, int64_t N,
    int64_t* linear_indices, int64_t* sorted_linear_indices, int64_t* infos_sorted,
    int64_t* sorted_linear_indices_run, int32_t* run_lengths, int32_t* num_runs,
    int32_t* cumulative_run_lengths, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  MX_REQUIRE(T >= 0 && B >= 0 && N >= 0, "negative T, B or N");
  MX_REQUIRE(index_bytes == 4 || index_bytes == 8, "indices must be int32 or int64");
  MX_REQUIRE(N < 0x7fffffffll, "N %lld too large for int32 positions", (long long)N);
  const Layout empty{0, nullptr, nullptr, nullptr};
  if (N == 0)
    return transpose_impl(hash_size_cumsum, T, 0, empty, total_hash_size_bits, 26, indices,
                          offsets, index_bytes, 0, linear_indices, sorted_linear_indices,
                          nullptr, sorted_linear_indices_run, run_lengths, num_runs,
                          cumulative_run_lengths, workspace, workspace_bytes, stream);
  MX_REQUIRE(T > 0 && B > 0, "%lld indices but no bags (T=%d, B=%lld)", (long long)N, T,
             (long long)B);
  MX_REQUIRE(offsets && infos_sorted && workspace, "null pointer argument");
  const int32_t nb = mx_tbe_info_B_num_bits(T, N);
  MX_REQUIRE(nb > 0, "T=%d and N=%lld do not fit a 32-bit info word", T, (long long)N);
  const size_t base = carve_sort(nullptr, N).bytes;
  const NobagWs nw = carve_nobag(static_cast<uint8_t*>(workspace), base, N, T, index_bytes);
  if (workspace_bytes < nw.bytes)
    return set_error(MX_EWORKSPACE, "workspace of %zu bytes needed", nw.bytes);
  auto* s = as_stream(stream);
  if (int rc = launch_nobag_layout(offsets, index_bytes, T, B, N, 4, nb, nw, false, s)) return rc;
  const Layout lay{N, nw.B_offsets, nullptr, nw.b_t_map};  // B_offsets: per-feature sort segments
  if (int rc = transpose_impl(hash_size_cumsum, T, 0, lay, total_hash_size_bits, nb, indices,
                              nw.bag_offsets, index_bytes, N, linear_indices,
                              sorted_linear_indices, nw.infos, sorted_linear_indices_run,
                              run_lengths, num_runs, cumulative_run_lengths, workspace, base,
                              stream))
    return rc;
  const int64_t want = ceil_div(N, 256);
  const int64_t cap = static_cast<int64_t>(num_cus()) * 8;
  const dim3 gd(static_cast<uint32_t>(want < cap ? want : cap));
  if (index_bytes == 8)
    nobag_infos_kernel<int64_t><<<gd, 256, 0, s>>>(nw.infos, static_cast<const int64_t*>(offsets),
                                                   T, B, N, nb, infos_sorted);
  else
    nobag_infos_kernel<int32_t><<<gd, 256, 0, s>>>(nw.infos, static_cast<const int32_t*>(offsets),
                                                   T, B, N, nb, infos_sorted);
  MX_LAUNCH_CHECK();
  return MX_OK;
}
