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
//    (u32 key, u32 info) pairs: ceil(bits/8) passes of 8-bit digits.  A pass
//    is histogram -> one device-wide exclusive scan (digit-major) ->
//    scatter.  The unit of work is one wave and a 1024-key tile; inside a
//    tile keys are ranked 64 at a time with 8 ballots (peer mask of equal
//    digits), so the scatter is stable without block barriers.
//  * Run-length encoding is a head-flag scan.
//  * Each run (one distinct (t, i)) is reduced by one wave, lanes owning
//    columns, occurrences added in sorted order.  Runs longer than kLong are
//    cut into kChunk-occurrence chunks reduced in parallel into a workspace,
//    then summed in chunk order by the run's wave.  No atomics: results are
//    deterministic.
#include "mx_common.h"
#include "scan.h"

namespace mx {

namespace {

constexpr int kRadixBits = 8;
constexpr int kRadix = 1 << kRadixBits;
constexpr int kSortItems = 16;
constexpr int64_t kSortTile = 64 * kSortItems;  // keys per wave-tile
constexpr int kLong = 32;                       // runs longer than this are chunked
constexpr int kChunk = 32;                      // occurrences per chunk
// Scans per backward: one per radix pass (at most 4), run heads, chunk layout.
constexpr int kScanSlots = 6;

// ---- linearize ------------------------------------------------------------

template <typename I>
__global__ void __launch_bounds__(256)
    linearize_kernel(const int64_t* __restrict__ hsc, const I* __restrict__ indices,
                     const I* __restrict__ offsets, int64_t nbags, int64_t B, int32_t nb,
                     int64_t N, int64_t* __restrict__ linear_out, uint32_t* __restrict__ keys,
                     uint32_t* __restrict__ vals, const float* __restrict__ iw,
                     uint32_t* __restrict__ vals2) {
  const int64_t l = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (l >= N) return;
  // Bag owning position l: last bag with offsets[bag] <= l.
  int64_t lo = 0, hi = nbags;  // offsets[lo] <= l < offsets[hi]
  while (hi - lo > 1) {
    const int64_t mid = lo + ((hi - lo) >> 1);
    if (static_cast<int64_t>(offsets[mid]) <= l)
      lo = mid;
    else
      hi = mid;
  }
  const int64_t t = lo / B;
  const int64_t b = lo - t * B;
  const int64_t key = hsc[t] + static_cast<int64_t>(indices[l]);
  if (linear_out) linear_out[l] = key;
  keys[l] = static_cast<uint32_t>(key);
  vals[l] = (nb >= 32 ? 0u : (static_cast<uint32_t>(t) << nb)) | static_cast<uint32_t>(b);
  if (iw) vals2[l] = __float_as_uint(iw[l]);  // per-sample weight rides along the sort
}

// ---- radix sort -----------------------------------------------------------

__global__ void __launch_bounds__(256)
    radix_hist_kernel(const uint32_t* __restrict__ keys, int64_t n, int shift, int nbits,
                      uint32_t* __restrict__ hist, int64_t ntiles) {
  __shared__ uint32_t cnt[4][kRadix];
  const int w = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t tile = static_cast<int64_t>(blockIdx.x) * 4 + w;
  for (int d = lane; d < kRadix; d += 64) cnt[w][d] = 0;
  __syncthreads();
  const uint32_t mask = (1u << nbits) - 1u;
  if (tile < ntiles) {
#pragma unroll 4
    for (int it = 0; it < kSortItems; ++it) {
      const int64_t i = tile * kSortTile + it * 64 + lane;
      if (i < n) atomicAdd(&cnt[w][(keys[i] >> shift) & mask], 1u);
    }
  }
  __syncthreads();
  if (tile < ntiles)
    for (int d = lane; d < kRadix; d += 64) hist[d * ntiles + tile] = cnt[w][d];
}

struct LoadU32 {
  const uint32_t* p;
  __device__ uint32_t operator()(int64_t i) const { return p[i]; }
};

template <bool LAST>
__global__ void __launch_bounds__(256)
    radix_scatter_kernel(const uint32_t* __restrict__ keys, const uint32_t* __restrict__ vals,
                         int64_t n, int shift, int nbits, const uint32_t* __restrict__ hist_scan,
                         int64_t ntiles, uint32_t* __restrict__ keys_out,
                         int64_t* __restrict__ keys_out64, uint32_t* __restrict__ vals_out,
                         const uint32_t* __restrict__ vals2, uint32_t* __restrict__ vals2_out) {
  __shared__ uint32_t base[4][kRadix];
  const int w = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t tile = static_cast<int64_t>(blockIdx.x) * 4 + w;
  if (tile < ntiles)
    for (int d = lane; d < kRadix; d += 64) base[w][d] = hist_scan[d * ntiles + tile];
  __syncthreads();
  if (tile >= ntiles) return;
  const uint32_t mask = (1u << nbits) - 1u;
  const uint64_t lt = (1ull << lane) - 1ull;
  for (int it = 0; it < kSortItems; ++it) {
    const int64_t i = tile * kSortTile + it * 64 + lane;
    const bool valid = i < n;
    const uint32_t k = valid ? keys[i] : 0u;
    const uint32_t v = valid ? vals[i] : 0u;
    const uint32_t v2 = (valid && vals2) ? vals2[i] : 0u;
    const uint32_t d = (k >> shift) & mask;
    uint64_t peers = __ballot(valid);
    for (int bit = 0; bit < nbits; ++bit) {
      const bool set = (d >> bit) & 1u;
      const uint64_t bb = __ballot(set);
      peers &= set ? bb : ~bb;
    }
    const uint32_t rank = static_cast<uint32_t>(__popcll(peers & lt));
    const uint32_t pos = base[w][d] + rank;
    if (valid) {
      if constexpr (LAST)
        keys_out64[pos] = static_cast<int64_t>(k);
      else
        keys_out[pos] = k;
      vals_out[pos] = v;
      if (vals2) vals2_out[pos] = v2;
    }
    // The lowest lane of each digit group advances that digit's cursor after
    // every lane of the wave has read it above (LDS ops of a wave are ordered).
    if (valid && rank == 0) base[w][d] = pos + static_cast<uint32_t>(__popcll(peers));
  }
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

__global__ void __launch_bounds__(256)
    rle_write_kernel(const int64_t* __restrict__ keys, int64_t n,
                     const uint32_t* __restrict__ run_id, const uint32_t* __restrict__ num_runs,
                     int64_t* __restrict__ run_keys, int32_t* __restrict__ cum) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i == 0) cum[*num_runs] = static_cast<int32_t>(n);
  if (i >= n) return;
  if (i == 0 || keys[i] != keys[i - 1]) {
    const uint32_t r = run_id[i];
    run_keys[r] = keys[i];
    cum[r] = static_cast<int32_t>(i);
  }
}

__global__ void __launch_bounds__(256)
    run_lengths_kernel(const int32_t* __restrict__ cum, const uint32_t* __restrict__ num_runs,
                       int64_t n, int32_t* __restrict__ lengths, int32_t* __restrict__ num_runs_out) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t m = *num_runs;
  if (r == 0 && num_runs_out) *num_runs_out = static_cast<int32_t>(m);
  if (r >= m || r >= n) return;
  lengths[r] = cum[r + 1] - cum[r];
}

// chunk_run[q] = the run that owns chunk q (runs longer than kLong only).
__global__ void __launch_bounds__(256)
    chunk_map_kernel(const int32_t* __restrict__ cum, const uint32_t* __restrict__ num_runs,
                     const uint32_t* __restrict__ chunk_start, uint32_t* __restrict__ chunk_run,
                     int64_t n) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (r >= n || r >= static_cast<int64_t>(*num_runs)) return;
  const int32_t len = cum[r + 1] - cum[r];
  if (len <= kLong) return;
  const uint32_t q0 = chunk_start[r];
  const int32_t nq = (len + kChunk - 1) / kChunk;
  for (int32_t i = 0; i < nq; ++i) chunk_run[q0 + i] = static_cast<uint32_t>(r);
}

struct ChunkCount {
  const int32_t* cum;
  __device__ uint32_t operator()(int64_t r) const {
    const int32_t len = cum[r + 1] - cum[r];
    return len > kLong ? static_cast<uint32_t>((len + kChunk - 1) / kChunk) : 0u;
  }
};

// ---- workspace layout -----------------------------------------------------

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

struct SortWs {
  uint32_t* keys[2];
  uint32_t* vals[2];
  uint32_t* vals2[2];  // per-sample weights (weighted backward only)
  uint32_t* hist;
  unsigned long long* scan_state;  // kScanSlots slots of (tiles + 1) zeroed words
  int64_t scan_slot_words;
  uint32_t* run_id;
  uint32_t* counters;  // [0] num_runs, [1] total chunks
  size_t bytes;
};

SortWs carve_sort(uint8_t* base, int64_t N) {
  SortWs w{};
  const int64_t n = N > 0 ? N : 1;
  const int64_t ntiles = ceil_div(n, kSortTile);
  const int64_t hist_n = kRadix * ntiles;
  const int64_t slot_words = scan_tiles(hist_n > n + 1 ? hist_n : n + 1) + 2;
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
  w.hist = reinterpret_cast<uint32_t*>(take(hist_n * 4));
  w.scan_state = reinterpret_cast<unsigned long long*>(take(kScanSlots * slot_words * 8));
  w.scan_slot_words = slot_words;
  w.run_id = reinterpret_cast<uint32_t*>(take((n + 1) * 4));
  w.counters = reinterpret_cast<uint32_t*>(take(64));
  w.bytes = off;
  return w;
}

// Scan-state slot i: status words, then the ticket pair in the last word.
ScanState scan_slot(const SortWs& w, int i) {
  unsigned long long* base = w.scan_state + i * w.scan_slot_words;
  return ScanState{base, reinterpret_cast<unsigned int*>(base + w.scan_slot_words - 1)};
}

struct TransposeOut {
  int64_t* linear;      // may be null
  int64_t* sorted;      // [N]
  int32_t* infos;       // [N]
  int64_t* run;         // [N]
  int32_t* run_lengths; // [N]
  int32_t* num_runs;    // [1]
  int32_t* cum;         // [N+1]
  float* weights_sorted;  // [N] per-sample weights in sorted order, or null
};

int run_transpose(const int64_t* hsc, int32_t T, int64_t B, int32_t bits, int32_t nb,
                  const void* indices, const void* offsets, int32_t index_bytes, int64_t N,
                  const float* iw, const TransposeOut& o, SortWs& w, hipStream_t s) {
  // With per-sample weights the weights travel with the keys as a second payload.
  uint32_t* const v2[2] = {iw ? w.vals2[0] : nullptr, iw ? w.vals2[1] : nullptr};
  uint32_t* const v2_final = iw ? reinterpret_cast<uint32_t*>(o.weights_sorted) : nullptr;
  const int64_t nbags = static_cast<int64_t>(T) * B;
  const dim3 g256(static_cast<uint32_t>(ceil_div(N, 256)));
  {  // every scan's look-back state starts at zero (a kernel, not a memset)
    const int64_t words = kScanSlots * w.scan_slot_words;
    const int64_t blocks = ceil_div(words, 256);
    zero_u64_kernel<<<dim3(static_cast<uint32_t>(blocks < 1024 ? blocks : 1024)), 256, 0, s>>>(
        w.scan_state, words);
    MX_LAUNCH_CHECK();
  }
  if (index_bytes == 8)
    linearize_kernel<int64_t><<<g256, 256, 0, s>>>(
        hsc, static_cast<const int64_t*>(indices), static_cast<const int64_t*>(offsets), nbags, B,
        nb, N, o.linear, w.keys[0], w.vals[0], iw, v2[0]);
  else
    linearize_kernel<int32_t><<<g256, 256, 0, s>>>(
        hsc, static_cast<const int32_t*>(indices), static_cast<const int32_t*>(offsets), nbags, B,
        nb, N, o.linear, w.keys[0], w.vals[0], iw, v2[0]);
  MX_LAUNCH_CHECK();

  const int64_t ntiles = ceil_div(N, kSortTile);
  const dim3 gsort(static_cast<uint32_t>(ceil_div(ntiles, 4)));
  const int passes = (bits + kRadixBits - 1) / kRadixBits;
  int cur = 0;
  if (passes == 0) {
    copy_keys_kernel<<<g256, 256, 0, s>>>(w.keys[0], w.vals[0], N, o.sorted,
                                          reinterpret_cast<uint32_t*>(o.infos), v2[0], v2_final);
    MX_LAUNCH_CHECK();
  }
  for (int p = 0; p < passes; ++p) {
    const int shift = p * kRadixBits;
    const int nbits = bits - shift < kRadixBits ? bits - shift : kRadixBits;
    radix_hist_kernel<<<gsort, 256, 0, s>>>(w.keys[cur], N, shift, nbits, w.hist, ntiles);
    MX_LAUNCH_CHECK();
    if (int rc = exclusive_scan(LoadU32{w.hist}, kRadix * ntiles, nullptr, w.hist, nullptr,
                                scan_slot(w, p), s))
      return rc;
    const bool last = p == passes - 1;
    if (last) {
      radix_scatter_kernel<true><<<gsort, 256, 0, s>>>(
          w.keys[cur], w.vals[cur], N, shift, nbits, w.hist, ntiles, nullptr, o.sorted,
          reinterpret_cast<uint32_t*>(o.infos), v2[cur], v2_final);
    } else {
      radix_scatter_kernel<false><<<gsort, 256, 0, s>>>(
          w.keys[cur], w.vals[cur], N, shift, nbits, w.hist, ntiles, w.keys[cur ^ 1], nullptr,
          w.vals[cur ^ 1], v2[cur], v2[cur ^ 1]);
    }
    MX_LAUNCH_CHECK();
    cur ^= 1;
  }

  // Run-length encode the sorted keys.
  if (int rc = exclusive_scan(HeadFlag{o.sorted}, N, nullptr, w.run_id, &w.counters[0],
                              scan_slot(w, 4), s))
    return rc;
  rle_write_kernel<<<g256, 256, 0, s>>>(o.sorted, N, w.run_id, &w.counters[0], o.run, o.cum);
  MX_LAUNCH_CHECK();
  run_lengths_kernel<<<g256, 256, 0, s>>>(o.cum, &w.counters[0], N, o.run_lengths, o.num_runs);
  MX_LAUNCH_CHECK();
  return MX_OK;
}

// ---- segment reduce + rowwise Adagrad -------------------------------------

constexpr int kMaxCachedTables = 512;  // table metadata kept in LDS up to this T

struct BwdArgs {
  float* W;
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
  const uint32_t* num_runs;
  const uint32_t* chunk_start;
  const uint32_t* chunk_run;
  const uint32_t* total_chunks;
  float* partial;
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
};

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

__device__ __forceinline__ int64_t table_of(const BwdArgs& a, int32_t info) {
  return a.nb >= 32 ? 0 : static_cast<int64_t>(static_cast<uint32_t>(info) >> a.nb);
}

// Group-level (G lanes, lane k) sum of the (MEAN-scaled) gradient rows of
// occurrences [s0, s1) of table t, in order.  Lane k owns columns
// (c*G + k)*4 .. +4 for c < NCH.  Called with the whole group converged.
// `info0` is lane k's infos[s0 + k] (valid for k < s1 - s0), already loaded
// by the caller to find the table.
template <typename I, int G, int NCH, int U>
__device__ void group_sum_occurrences(const BwdArgs& a, int64_t t, int32_t D0, int32_t D,
                                      int64_t s0, int64_t s1, int g, int k, int32_t info0,
                                      float (&acc)[NCH][4]) {
  const uint32_t bmask = a.nb >= 32 ? 0xffffffffu : ((1u << a.nb) - 1u);
  for (int64_t base = s0; base < s1; base += G) {
    const int n = static_cast<int>(s1 - base < G ? s1 - base : G);
    int32_t my_b = 0;
    float my_s = 1.0f;  // MEAN: 1/L of the occurrence's bag
    float my_w = 1.0f;  // weighted: the occurrence's per-sample weight
    if (k < n) {
      const int32_t info = base == s0 ? info0 : a.infos[base + k];
      my_b = static_cast<int32_t>(static_cast<uint32_t>(info) & bmask);
      if (a.pooling == MX_POOL_MEAN) {
        const I* off = static_cast<const I*>(a.offsets);
        const int64_t bag = t * a.B + my_b;
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
          const int64_t b = __shfl(my_b, g * G + j + u, 64);
          const float* row = a.grad + b * a.total_D + D0;
#pragma unroll
          for (int c = 0; c < NCH; ++c)
            if ((c * G + k) * 4 < D) ld4(row + (c * G + k) * 4, v[u][c]);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (j + u < n) {
          const float sc = __shfl(my_s, g * G + j + u, 64);
          const float wt = __shfl(my_w, g * G + j + u, 64);
#pragma unroll
          for (int c = 0; c < NCH; ++c)
            if ((c * G + k) * 4 < D) {
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
  }
}

// Rowwise Adagrad on one row held by a G-lane group (lane k owns columns
// (c*G + k)*4 .. +4): h += mean(g^2), m = lr / (sqrt(h) + eps),
// w = fma(-m, g, c*w); lane 0 of the group writes h.
template <int G, int NCH>
__device__ __forceinline__ void adagrad_update(const BwdArgs& a, int32_t D, int k,
                                               const float (&gs)[NCH][4], const float (&w)[NCH][4],
                                               float* wrow, float* hp, float h0) {
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    if ((c * G + k) * 4 >= D) continue;
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
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    if ((c * G + k) * 4 >= D) continue;
    float nw[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) nw[e] = __builtin_fmaf(-mult, gs[c][e], __fmul_rn(corr, w[c][e]));
    st4(wrow + (c * G + k) * 4, nw);
  }
  if (k == 0) *hp = h;
}

// Pass B (long runs): one 256-thread block per run longer than kLong.  The
// 256/G groups sum the run's chunk partials round-robin (group j takes
// chunks j, j + 256/G, ...), the group vectors are combined in group order
// through LDS, and group 0 applies the update.
template <int G, int NCH, int U>
__global__ void __launch_bounds__(256) bwd_long_run_kernel(BwdArgs a) {
  __shared__ TableMeta meta;
  constexpr int NG = 256 / G;
  __shared__ float part[NG][G * NCH * 4];
  stage_meta(a, meta);
  const MetaView mv{a, meta, a.T <= kMaxCachedTables};
  const int grp = threadIdx.x / G, k = threadIdx.x % G;
  const int64_t total = *a.total_chunks;
  for (int64_t q = blockIdx.x; q < total; q += gridDim.x) {
    const uint32_t r = a.chunk_run[q];
    if (q > 0 && a.chunk_run[q - 1] == r) continue;  // not the run's first chunk (block-uniform)
    const int64_t s0 = a.cum[r];
    const int64_t s1 = a.cum[r + 1];
    const int64_t t = table_of(a, a.infos[s0]);
    const int32_t D0 = mv.D_off(t);
    const int32_t D = mv.D_off(t + 1) - D0;
    (void)D0;
    const int64_t q1 = q + (s1 - s0 + kChunk - 1) / kChunk;
    float gs[NCH][4];
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e) gs[c][e] = 0.0f;
    for (int64_t qq = q + grp; qq < q1; qq += NG * U) {
      float v[U][NCH][4];
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (qq + u * NG < q1)
#pragma unroll
          for (int c = 0; c < NCH; ++c)
            if ((c * G + k) * 4 < D) ld4(a.partial + (qq + u * NG) * a.max_D + (c * G + k) * 4, v[u][c]);
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (qq + u * NG < q1)
#pragma unroll
          for (int c = 0; c < NCH; ++c)
            if ((c * G + k) * 4 < D)
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
      const int64_t idx = a.run[r] - mv.hsc(t);
      float* wrow = a.W + mv.w_off(t) + idx * D;
      float* hp = a.m1 + mv.m1_off(t) + idx;
      float w[NCH][4];
#pragma unroll
      for (int c = 0; c < NCH; ++c)
        if ((c * G + k) * 4 < D) ld4(wrow + (c * G + k) * 4, w[c]);
      adagrad_update<G, NCH>(a, D, k, gs, w, wrow, hp, *hp);
    }
    __syncthreads();
  }
}

// Pass A: one group per chunk of a long run -> partial sum in the workspace.
template <typename I, int G, int NCH, int U>
__global__ void __launch_bounds__(256) bwd_chunk_kernel(BwdArgs a) {
  __shared__ TableMeta meta;
  stage_meta(a, meta);
  const MetaView mv{a, meta, a.T <= kMaxCachedTables};
  constexpr int P = 64 / G;
  const int lane = threadIdx.x & 63;
  const int g = lane / G, k = lane % G;
  const int64_t wave = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t nwaves = static_cast<int64_t>(gridDim.x) * 4;
  const int64_t total = *a.total_chunks;
  for (int64_t qb = wave * P; qb < total; qb += nwaves * P) {
    const int64_t q = qb + g;
    if (q >= total) continue;
    const int64_t r = a.chunk_run[q];
    const int64_t s0 = a.cum[r] + (q - a.chunk_start[r]) * kChunk;
    const int64_t e0 = a.cum[r + 1];
    const int64_t s1 = s0 + kChunk < e0 ? s0 + kChunk : e0;
    const int32_t info0 = k < s1 - s0 ? a.infos[s0 + k] : 0;
    const int64_t t = table_of(a, __shfl(info0, g * G, 64));
    const int32_t D0 = mv.D_off(t);
    const int32_t D = mv.D_off(t + 1) - D0;
    float acc[NCH][4];
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[c][e] = 0.0f;
    group_sum_occurrences<I, G, NCH, U>(a, t, D0, D, s0, s1, g, k, info0, acc);
    float* dst = a.partial + q * a.max_D;
#pragma unroll
    for (int c = 0; c < NCH; ++c)
      if ((c * G + k) * 4 < D) st4(dst + (c * G + k) * 4, acc[c]);
  }
}

// Pass B (runs of at most kLong occurrences): one G-lane group per run --
// gradient sum in sorted order, rowwise Adagrad, in-place update.  The
// table of a run comes from the first batch of infos, which is kept for the
// gradient sum.
template <typename I, int G, int NCH, int U>
__global__ void __launch_bounds__(256) bwd_update_kernel(BwdArgs a) {
  __shared__ TableMeta meta;
  stage_meta(a, meta);
  const MetaView mv{a, meta, a.T <= kMaxCachedTables};
  constexpr int P = 64 / G;
  const int lane = threadIdx.x & 63;
  const int g = lane / G, k = lane % G;
  const int64_t wave = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 4 * P;
  const int64_t nruns = *a.num_runs;
  for (int64_t r = wave * P + g; r < nruns; r += stride) {
    const int64_t cs0 = a.cum[r];
    const int64_t cs1 = a.cum[r + 1];
    const int64_t ckey = a.run[r];
    if (cs1 - cs0 > kLong) continue;  // long runs: bwd_long_run_kernel
    const int32_t info0 = k < cs1 - cs0 ? a.infos[cs0 + k] : 0;
    const int64_t t = table_of(a, __shfl(info0, g * G, 64));
    const int32_t D0 = mv.D_off(t);
    const int32_t D = mv.D_off(t + 1) - D0;
    const int64_t idx = ckey - mv.hsc(t);
    float* wrow = a.W + mv.w_off(t) + idx * D;
    float* hp = a.m1 + mv.m1_off(t) + idx;
    float w[NCH][4];
#pragma unroll
    for (int c = 0; c < NCH; ++c)
      if ((c * G + k) * 4 < D) ld4(wrow + (c * G + k) * 4, w[c]);
    const float h0 = *hp;
    float gs[NCH][4];
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e) gs[c][e] = 0.0f;
    group_sum_occurrences<I, G, NCH, U>(a, t, D0, D, cs0, cs1, g, k, info0, gs);
    adagrad_update<G, NCH>(a, D, k, gs, w, wrow, hp, h0);
  }
}

template <typename I, int G, int NCH>
int launch_bwd(const BwdArgs& a, int64_t N, hipStream_t s) {
  constexpr int U = NCH <= 1 ? 4 : 2;   // runs are short: keep registers low
  constexpr int UC = NCH <= 1 ? 8 : (NCH <= 2 ? 8 : 4);  // chunks are full: more in flight
  constexpr int P = 64 / G;
  const int64_t want = ceil_div(N, 4 * P);
  const int64_t cap = static_cast<int64_t>(num_cus()) * 16;
  const dim3 grid(static_cast<uint32_t>(want < 1 ? 1 : (want > cap ? cap : want)));
  bwd_chunk_kernel<I, G, NCH, UC><<<grid, 256, 0, s>>>(a);
  MX_LAUNCH_CHECK();
  const int64_t long_cap = static_cast<int64_t>(num_cus()) * 4;
  const int64_t long_want = ceil_div(N, kChunk);
  bwd_long_run_kernel<G, NCH, 4><<<dim3(static_cast<uint32_t>(long_want < long_cap ? (long_want < 1 ? 1 : long_want) : long_cap)), 256, 0, s>>>(a);
  MX_LAUNCH_CHECK();
  bwd_update_kernel<I, G, NCH, U><<<grid, 256, 0, s>>>(a);
  MX_LAUNCH_CHECK();
  return MX_OK;
}

// Lanes per run (G) and float4 chunks per lane (NCH) from the widest table.
template <typename I>
int dispatch_bwd(const BwdArgs& a, int64_t N, hipStream_t s) {
  if (a.max_D <= 64) return launch_bwd<I, 16, 1>(a, N, s);
  if (a.max_D <= 128) return launch_bwd<I, 16, 2>(a, N, s);
  if (a.max_D <= 256) return launch_bwd<I, 32, 2>(a, N, s);
  if (a.max_D <= 512) return launch_bwd<I, 64, 2>(a, N, s);
  return launch_bwd<I, 64, 4>(a, N, s);
}

struct BwdWs {
  SortWs sort;
  int64_t* sorted;
  int32_t* infos;
  int64_t* run;
  int32_t* run_lengths;
  int32_t* num_runs;
  int32_t* cum;
  uint32_t* chunk_start;
  uint32_t* chunk_run;
  float* weights_sorted;
  float* partial;
  size_t bytes;
};

int64_t max_chunks(int64_t N) { return N / kChunk + N / (kLong + 1) + 2; }  // >= sum of ceil(len/kChunk)

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
  w.run_lengths = reinterpret_cast<int32_t*>(take(n * 4));
  w.num_runs = reinterpret_cast<int32_t*>(take(4));
  w.cum = reinterpret_cast<int32_t*>(take((n + 1) * 4));
  w.chunk_start = reinterpret_cast<uint32_t*>(take((n + 1) * 4));
  w.chunk_run = reinterpret_cast<uint32_t*>(take(static_cast<size_t>(max_chunks(n)) * 4));
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

static int check_common(int32_t T, int64_t B, int32_t bits, int32_t nb, int32_t index_bytes,
                        int64_t N) {
  MX_REQUIRE(T >= 0 && B >= 0 && N >= 0, "negative size");
  MX_REQUIRE(bits >= 0 && bits <= 32, "total_hash_size_bits %d not in [0, 32]", bits);
  MX_REQUIRE(index_bytes == 4 || index_bytes == 8, "indices must be int32 or int64");
  MX_REQUIRE(N < 0x7fffffffll, "N %lld too large for int32 run offsets", (long long)N);
  MX_REQUIRE(nb >= 1 && nb <= 32, "info_B_num_bits %d invalid", nb);
  MX_REQUIRE(B <= (int64_t(1) << nb), "B does not fit info_B_num_bits");
  return MX_OK;
}

extern "C" int mx_tbe_transpose_embedding_input(
    const int64_t* hash_size_cumsum, int32_t T, int64_t B, int32_t total_hash_size_bits,
    int32_t info_B_num_bits, const void* indices, const void* offsets, int32_t index_bytes,
    int64_t N, int64_t* linear_indices, int64_t* sorted_linear_indices, int32_t* infos_sorted,
    int64_t* sorted_linear_indices_run, int32_t* run_lengths, int32_t* num_runs,
    int32_t* cumulative_run_lengths, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  if (int rc = check_common(T, B, total_hash_size_bits, info_B_num_bits, index_bytes, N)) return rc;
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
  return run_transpose(hash_size_cumsum, T, B, total_hash_size_bits, info_B_num_bits, indices,
                       offsets, index_bytes, N, nullptr, o, w, s);
}

extern "C" size_t mx_tbe_backward_workspace_bytes(int64_t N, int32_t total_hash_size_bits,
                                                  int32_t max_D) {
  (void)total_hash_size_bits;
  return carve_bwd(nullptr, N, max_D > 0 ? max_D : 1).bytes;
}

extern "C" int mx_tbe_backward_rowwise_adagrad(
    float* weights, const int64_t* weights_offsets, const int32_t* D_offsets, int32_t T,
    int64_t B, int32_t max_D, const int64_t* hash_size_cumsum, int32_t total_hash_size_bits,
    const void* indices, const void* offsets, int32_t index_bytes, int64_t N,
    int32_t pooling_mode, const float* indice_weights, const float* grad_output, int64_t total_D,
    float* momentum1, const int64_t* momentum1_offsets, float learning_rate, float eps,
    float weight_decay, int32_t weight_decay_mode, void* workspace, size_t workspace_bytes,
    void* stream) {
  clear_error();
  const int32_t nb = mx_tbe_info_B_num_bits(T, B);
  MX_REQUIRE(nb > 0, "T=%d, B=%lld do not fit a 32-bit info word", T, (long long)B);
  if (int rc = check_common(T, B, total_hash_size_bits, nb, index_bytes, N)) return rc;
  MX_REQUIRE(max_D > 0 && max_D <= 1024 && max_D % 4 == 0,
             "max_D %d must be a multiple of 4 in [4, 1024]", max_D);
  MX_REQUIRE(pooling_mode == MX_POOL_SUM || pooling_mode == MX_POOL_MEAN,
             "pooling_mode %d not supported (SUM=0, MEAN=1)", pooling_mode);
  MX_REQUIRE(weight_decay_mode >= 0 && weight_decay_mode <= 2,
             "weight_decay_mode %d not supported (0 none, 1 L2, 2 decoupled)", weight_decay_mode);
  if (N == 0) return MX_OK;
  MX_REQUIRE(weights && weights_offsets && D_offsets && hash_size_cumsum && indices && offsets &&
                 grad_output && momentum1 && momentum1_offsets,
             "null pointer argument");
  BwdWs w = carve_bwd(static_cast<uint8_t*>(workspace), N, max_D);
  if (workspace == nullptr || workspace_bytes < w.bytes)
    return set_error(MX_EWORKSPACE, "workspace of %zu bytes needed", w.bytes);
  auto* s = as_stream(stream);
  TransposeOut o{nullptr, w.sorted, w.infos, w.run, w.run_lengths, w.num_runs, w.cum,
                 indice_weights ? w.weights_sorted : nullptr};
  if (int rc = run_transpose(hash_size_cumsum, T, B, total_hash_size_bits, nb, indices, offsets,
                             index_bytes, N, indice_weights, o, w.sort, s))
    return rc;
  // Chunk layout of long runs.
  if (int rc = exclusive_scan(ChunkCount{w.cum}, N, w.num_runs, w.chunk_start,
                              &w.sort.counters[1], scan_slot(w.sort, 5), s))
    return rc;
  chunk_map_kernel<<<dim3(static_cast<uint32_t>(ceil_div(N, 256))), 256, 0, s>>>(
      w.cum, &w.sort.counters[0], w.chunk_start, w.chunk_run, N);
  MX_LAUNCH_CHECK();
  BwdArgs a;
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
  a.num_runs = &w.sort.counters[0];
  a.chunk_start = w.chunk_start;
  a.chunk_run = w.chunk_run;
  a.T = T;
  a.total_chunks = &w.sort.counters[1];
  a.partial = w.partial;
  a.B = B;
  a.total_D = total_D;
  a.max_D = max_D;
  a.nb = nb;
  a.pooling = pooling_mode;
  a.wd_mode = weight_decay_mode;
  a.lr = learning_rate;
  a.eps = eps;
  a.wd = weight_decay;
  return index_bytes == 8 ? dispatch_bwd<int64_t>(a, N, s) : dispatch_bwd<int32_t>(a, N, s);
}
