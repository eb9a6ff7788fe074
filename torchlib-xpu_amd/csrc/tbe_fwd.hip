// Table-batched embedding (TBE) training forward, fp32 or fp16 weights, gfx950.
//
// Semantics: fbgemm_gpu split_embedding_codegen_forward_{unweighted,weighted}
// (upstream codegen/training/forward/, recalled), i.e. the pooled SpMDM of
// torch/include/fbgemm/FbgemmEmbedding.h:26-39 applied per table:
//   out[b, D_off[t] + d] = sum_{l in bag(t,b)} W_t[idx[l], d]   (SUM)
//   MEAN multiplies the sum by 1/L for L > 0; an empty bag gives 0.
// fp16 weight rows are widened to fp32 element by element before the sum.
//
// Design: G lanes per bag (G = 32 for D <= 128: two bags per wave64).  Lane
// k owns 4*NCH columns, so a group reads a whole row with one coalesced
// float4 load per lane and every column is accumulated in index order -- the
// sum is bit-identical to a sequential CPU loop.  A bag's indices are fetched
// G at a time with one coalesced load and handed out with ds_bpermute; U rows
// are loaded before any is accumulated (D=128: 8 x 512 B in flight per bag).
// A batch of U loads has no branch between its loads (rows past the bag's end
// are clamped to its last row and their sums dropped by a select), so the
// compiler issues all U before the first wait.  When every bag of a wave is
// in one table and that table fits 4 GiB, rows are read through one buffer
// descriptor of the table with 32-bit byte offsets (no 64-bit address per
// row); otherwise through 64-bit pointers.
// Blocks are remapped so that each XCD works on a contiguous range of bags
// (t-major), keeping one table's hot rows in one XCD's L2 (measured: 27.8 us
// vs 31.0 us without the remap on config 2).  With several bags per wave, a
// block ranks its bags by length and gives bags of similar length to one
// wave (config 2: 36.7 -> 35.9 us cold, 34.1 -> 33.3 us over rotating
// batches).
#include "mx_common.h"

namespace mx {
namespace {

template <int VEC>
struct VecF;
template <>
struct VecF<1> {
  using T = float;
};
template <>
struct VecF<2> {
  using T = float2;
};
template <>
struct VecF<4> {
  using T = float4;
};

template <int VEC>
__device__ __forceinline__ void load_vec(const float* p, float (&v)[VEC]) {
  using T = typename VecF<VEC>::T;
  const T x = *reinterpret_cast<const T*>(p);
  if constexpr (VEC == 1) {
    v[0] = x;
  } else if constexpr (VEC == 2) {
    v[0] = x.x;
    v[1] = x.y;
  } else {
    v[0] = x.x;
    v[1] = x.y;
    v[2] = x.z;
    v[3] = x.w;
  }
}

// Four consecutive weights of a row as fp32 (16 B of fp32 or 8 B of fp16).
__device__ __forceinline__ void load_row4(const float* p, float (&v)[4]) { load_vec<4>(p, v); }

__device__ __forceinline__ void load_row4(const __half* p, float (&v)[4]) {
  const uint2 x = *reinterpret_cast<const uint2*>(p);
  v[0] = __half2float(__ushort_as_half(static_cast<unsigned short>(x.x & 0xffffu)));
  v[1] = __half2float(__ushort_as_half(static_cast<unsigned short>(x.x >> 16)));
  v[2] = __half2float(__ushort_as_half(static_cast<unsigned short>(x.y & 0xffffu)));
  v[3] = __half2float(__ushort_as_half(static_cast<unsigned short>(x.y >> 16)));
}

constexpr int kWavesPerBlock = 4;

}  // namespace

// Where bag i of the flattened (t, b) bag space lives: fixed batch (t = i / B,
// output row b of stride total_D) or variable batch per feature ("VBE": the
// bag's (t << nb) | b word and its output element offset, both per bag).
struct BagMap {
  int64_t B;
  int64_t total_D;
  const int32_t* b_t_map;  // VBE only
  const int64_t* row_out;  // VBE only
  int32_t nb;              // VBE only
  __device__ __forceinline__ void locate(int64_t bag, int64_t& t, int64_t& b) const {
    if (b_t_map) {
      const uint32_t info = static_cast<uint32_t>(b_t_map[bag]);
      t = nb >= 32 ? 0 : static_cast<int64_t>(info >> nb);
      b = static_cast<int64_t>(nb >= 32 ? info : (info & ((1u << nb) - 1u)));
    } else {
      t = bag / B;
      b = bag - t * B;
    }
  }
  // First element of the bag's output (and gradient) row.
  __device__ __forceinline__ int64_t out_base(int64_t bag, int64_t b, int32_t D0) const {
    return row_out ? row_out[bag] : b * total_D + D0;
  }
};

namespace {

// A buffer descriptor of a wave-uniform table base: stride 0 and the whole
// 32-bit offset range (callers keep every offset below 2^32), gfx9 format word.
template <typename WT>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t table_rsrc(const WT* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<WT*>(base), 0, 0xffffffff, 0x00020000);
}

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));

// Four consecutive weights at byte `off` of the table as fp32.
__device__ __forceinline__ void buf_row4(__amdgpu_buffer_rsrc_t r, uint32_t off, const float*,
                                         float (&v)[4]) {
  const i32x4 x = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
  v[0] = __int_as_float(x.x);
  v[1] = __int_as_float(x.y);
  v[2] = __int_as_float(x.z);
  v[3] = __int_as_float(x.w);
}

__device__ __forceinline__ void buf_row4(__amdgpu_buffer_rsrc_t r, uint32_t off, const __half*,
                                         float (&v)[4]) {
  const i32x2 x = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
  v[0] = __half2float(__ushort_as_half(static_cast<unsigned short>(x.x & 0xffff)));
  v[1] = __half2float(__ushort_as_half(static_cast<unsigned short>(static_cast<uint32_t>(x.x) >> 16)));
  v[2] = __half2float(__ushort_as_half(static_cast<unsigned short>(x.y & 0xffff)));
  v[3] = __half2float(__ushort_as_half(static_cast<unsigned short>(static_cast<uint32_t>(x.y) >> 16)));
}

// Adds the n rows of one batch of a bag to the group's accumulators, U rows
// in flight per lane.  Lane j of the group holds row j's location: its byte
// offset in the wave's table (BUF: buffer loads off one descriptor, a 32-bit
// offset per lane) or its element offset (64-bit global addresses).  The loop
// body has no branch: every one of the U loads is issued (slots past the
// batch re-read its last row, from cache) and the sums take only the rows of
// the batch, through a select, so each column still adds exactly its rows in
// index order.  Straight-line code lets the compiler keep the U loads in
// flight together instead of waiting on each one.
template <bool BUF, typename WT, int G, int NCH, int U, bool WEIGHTED>
__device__ __forceinline__ void pool_batch(uint64_t my_off, float my_w, int n, int g,
                                           const WT* const (&lane_col)[NCH],
                                           __amdgpu_buffer_rsrc_t rsrc,
                                           const uint32_t (&lane_byte)[NCH],
                                           float (&acc)[NCH][4]) {
  for (int j = 0; j < n; j += U) {
    float v[U][NCH][4];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int r = j + u < n ? j + u : n - 1;
      if constexpr (BUF) {
        const uint32_t off = __shfl(static_cast<uint32_t>(my_off), g * G + r, 64);
#pragma unroll
        for (int c = 0; c < NCH; ++c) buf_row4(rsrc, off + lane_byte[c], lane_col[c], v[u][c]);
      } else {
        const uint64_t off = __shfl(my_off, g * G + r, 64);
#pragma unroll
        for (int c = 0; c < NCH; ++c) load_row4(lane_col[c] + off, v[u][c]);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool take = j + u < n;
      float wgt = 1.0f;
      if constexpr (WEIGHTED) wgt = __shfl(my_w, g * G + (take ? j + u : n - 1), 64);
#pragma unroll
      for (int c = 0; c < NCH; ++c)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float x;
          if constexpr (WEIGHTED)
            x = __builtin_fmaf(wgt, v[u][c][e], acc[c][e]);
          else
            x = acc[c][e] + v[u][c][e];
          acc[c][e] = take ? x : acc[c][e];
        }
    }
  }
}

// Waves per SIMD an instance is compiled for: 8 (a 64-register budget) where
// that fits without spilling -- one float4 chunk per lane, unweighted, int64
// indices -- so that 16k waves of a D=128 batch run in 2 rounds instead of
// 2.3; the compiler's own choice elsewhere.
template <typename I, int NCH, bool WEIGHTED>
constexpr int fwd_waves() {
  return (NCH == 1 && !WEIGHTED && sizeof(I) == 8) ? 8 : 1;
}

// A wave serves 64/G bags at once, G lanes per bag, lane k owning columns
// (c*G + k)*4 .. +4 (float4 loads: a D=128 row is one 512 B access of 32
// lanes).  Several bags per wave keep several independent offsets -> indices
// -> rows chains in flight; each column is still summed in index order.
template <typename I, typename WT, int G, int NCH, int U, bool WEIGHTED, bool OUT_F16>
__global__ void __launch_bounds__(256)
    __attribute__((amdgpu_waves_per_eu(fwd_waves<I, NCH, WEIGHTED>())))
    tbe_fwd_group_kernel(const WT* __restrict__ W, const int64_t* __restrict__ w_off,
                         const int32_t* __restrict__ D_off, BagMap bm,
                         const I* __restrict__ indices, const I* __restrict__ offsets,
                         int32_t pooling, const float* __restrict__ iw, void* __restrict__ out,
                         int64_t nbags) {
  constexpr int P = 64 / G;
  const int64_t lb = xcd_remap(blockIdx.x, gridDim.x);
  const int lane = threadIdx.x & 63;
  const int g = lane / G, k = lane % G;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int64_t bag, start = 0, end = 0;
  if constexpr (P > 1) {
    // A wave lasts as long as its longest bag: the block ranks its BPB bags
    // by length (longest first, ties by position) and wave w takes ranks
    // [w*P, w*P + P), so bags of similar length share a wave.  Each bag
    // still writes its own output row.
    constexpr int BPB = kWavesPerBlock * P;
    __shared__ int64_t s_start[BPB], s_end[BPB];
    __shared__ int32_t s_bag[BPB];
    const int64_t bag0 = lb * BPB;
    if (threadIdx.x < BPB) {
      const int64_t bb = bag0 + threadIdx.x;
      int64_t st = 0, en = -1;  // slots past the batch rank last
      if (bb < nbags) {
        st = static_cast<int64_t>(offsets[bb]);
        en = static_cast<int64_t>(offsets[bb + 1]);
      }
      s_start[threadIdx.x] = st;
      s_end[threadIdx.x] = en;
    }
    __syncthreads();
    if (threadIdx.x < BPB) {
      const int i = threadIdx.x;
      const int64_t li = s_end[i] - s_start[i];
      int rank = 0;
#pragma unroll
      for (int j = 0; j < BPB; ++j) {
        const int64_t lj = s_end[j] - s_start[j];
        rank += (lj > li || (lj == li && j < i)) ? 1 : 0;
      }
      s_bag[rank] = i;
    }
    __syncthreads();
    const int i = s_bag[wave * P + g];
    bag = bag0 + i;
    start = s_start[i];
    end = s_end[i];
  } else {
    bag = lb * kWavesPerBlock + wave;
    if (bag < nbags) {
      start = static_cast<int64_t>(offsets[bag]);
      end = static_cast<int64_t>(offsets[bag + 1]);
    }
  }
  if (bag >= nbags) return;  // whole group (idle slots rank last)
  int64_t t, b;
  bm.locate(bag, t, b);
  const int32_t D0 = D_off[t];
  const int32_t D = D_off[t + 1] - D0;
  const WT* __restrict__ Wt = W + w_off[t];
  // When the wave's bags share one table (a fixed batch of even B, or most
  // waves of any batch), its rows are read through one buffer descriptor.
  const int64_t tw = readlane_i64(t, __builtin_amdgcn_readfirstlane(lane));
  const bool one_table = __all(t == tw);  // wave-uniform
  const __amdgpu_buffer_rsrc_t rsrc = table_rsrc(W + w_off[tw]);

  float acc[NCH][4];
#pragma unroll
  for (int c = 0; c < NCH; ++c)
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[c][e] = 0.0f;
  bool active[NCH];
  const WT* lane_col[NCH];   // this lane's first column of each chunk, row 0
  uint32_t lane_byte[NCH];   // the same as a byte offset in the table
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    active[c] = (c * G + k) * 4 < D;
    // A chunk past the row's end reads the row's first columns instead (never
    // stored), so that no load sits behind a branch.
    const int col = active[c] ? (c * G + k) * 4 : 0;
    lane_col[c] = Wt + col;
    lane_byte[c] = static_cast<uint32_t>(col * sizeof(WT));
  }

  // The group's indices come G at a time, one batch ahead of its rows, so a
  // bag longer than G does not wait for its next batch of indices.
  I nxt_idx = start + k < end ? indices[start + k] : I(0);
  float nxt_w = 0.0f;
  if constexpr (WEIGHTED) nxt_w = start + k < end ? iw[start + k] : 0.0f;
  for (int64_t base = start; base < end; base += G) {
    const int n = static_cast<int>(end - base < G ? end - base : G);
    const I cur_idx = nxt_idx;
    [[maybe_unused]] const float my_w = nxt_w;
    if (base + G + k < end) {
      nxt_idx = indices[base + G + k];
      if constexpr (WEIGHTED) nxt_w = iw[base + G + k];
    }
    // The lane that loads an index also turns it into the row's offset,
    // once, instead of every lane of the group per row: in bytes for buffer
    // loads when every row of the batch ends below 4 GiB into its table (one
    // 32-bit word per row between lanes, one 32-bit add per load), else in
    // elements for 64-bit addresses.
    const uint64_t my_elem = k < n ? static_cast<uint64_t>(cur_idx) * static_cast<uint64_t>(D) : 0;
    const uint64_t my_end = (my_elem + static_cast<uint64_t>(D)) * sizeof(WT);
    if (one_table && __all(my_end <= 0xffffffffull))  // wave-uniform
      pool_batch<true, WT, G, NCH, U, WEIGHTED>(my_elem * sizeof(WT), my_w, n, g, lane_col, rsrc,
                                               lane_byte, acc);
    else  // a wave over two tables, or a table past 4 GiB: half the rows in flight
      pool_batch<false, WT, G, NCH, (U > 1 ? U / 2 : 1), WEIGHTED>(my_elem, my_w, n, g, lane_col,
                                                                 rsrc, lane_byte, acc);
  }
  const int64_t L = end - start;
  if (pooling == MX_POOL_MEAN && L > 0) {
    const float inv = 1.0f / static_cast<float>(L);
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[c][e] *= inv;
  }
  const int64_t obase = bm.out_base(bag, b, D0);
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    if (!active[c]) continue;
    const int64_t col = obase + (c * G + k) * 4;
    if constexpr (OUT_F16) {
      __half* o = reinterpret_cast<__half*>(out) + col;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = __float2half_rn(acc[c][e]);
    } else {
      *reinterpret_cast<float4*>(reinterpret_cast<float*>(out) + col) =
          make_float4(acc[c][0], acc[c][1], acc[c][2], acc[c][3]);
    }
  }
}

// Gradient of the per-sample weights of a weighted lookup:
//   grad_iw[l] = sum_d grad_output[b, D_off[t] + d] * W_t[idx[l], d]
// (MEAN: times 1/L), 0 for tables whose feature_requires_grad entry is 0.
// Same G-lane-per-bag mapping as the forward; the bag's gradient slice stays
// in registers, each row's dot product is reduced over the group in a fixed
// xor-tree order.
template <typename I, typename WT, int G, int NCH, int U>
__global__ void __launch_bounds__(256)
    grad_indice_weights_kernel(const float* __restrict__ grad, BagMap bm,
                               const WT* __restrict__ W, const int64_t* __restrict__ w_off,
                               const int32_t* __restrict__ D_off,
                               const I* __restrict__ indices, const I* __restrict__ offsets,
                               int32_t pooling, const int32_t* __restrict__ frg,
                               float* __restrict__ out, int64_t nbags) {
  constexpr int P = 64 / G;
  const int64_t lb = xcd_remap(blockIdx.x, gridDim.x);
  const int lane = threadIdx.x & 63;
  const int g = lane / G, k = lane % G;
  const int64_t bag = (lb * kWavesPerBlock + (threadIdx.x >> 6)) * P + g;
  if (bag >= nbags) return;  // whole group
  int64_t t, b;
  bm.locate(bag, t, b);
  const int64_t start = static_cast<int64_t>(offsets[bag]);
  const int64_t end = static_cast<int64_t>(offsets[bag + 1]);
  if (frg != nullptr && frg[t] == 0) {
    for (int64_t l = start + k; l < end; l += G) out[l] = 0.0f;
    return;
  }
  const int32_t D0 = D_off[t];
  const int32_t D = D_off[t + 1] - D0;
  const WT* __restrict__ Wt = W + w_off[t];
  bool active[NCH];
  float gv[NCH][4];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    active[c] = (c * G + k) * 4 < D;
    if (active[c])
      load_vec<4>(grad + bm.out_base(bag, b, D0) + (c * G + k) * 4, gv[c]);
    else
      gv[c][0] = gv[c][1] = gv[c][2] = gv[c][3] = 0.0f;
  }
  const int64_t L = end - start;
  const float inv = (pooling == MX_POOL_MEAN && L > 0) ? 1.0f / static_cast<float>(L) : 1.0f;
  for (int64_t base = start; base < end; base += G) {
    const int n = static_cast<int>(end - base < G ? end - base : G);
    const int64_t my_idx = k < n ? static_cast<int64_t>(indices[base + k]) : 0;
    for (int j = 0; j < n; j += U) {
      float v[U][NCH][4];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (j + u < n) {
          const int64_t r = __shfl(my_idx, g * G + j + u, 64);
#pragma unroll
          for (int c = 0; c < NCH; ++c)
            if (active[c]) load_row4(Wt + r * D + (c * G + k) * 4, v[u][c]);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (j + u < n) {
          float dot = 0.0f;
#pragma unroll
          for (int c = 0; c < NCH; ++c)
            if (active[c])
#pragma unroll
              for (int e = 0; e < 4; ++e) dot = __builtin_fmaf(gv[c][e], v[u][c][e], dot);
#pragma unroll
          for (int m = G / 2; m >= 1; m >>= 1) dot += __shfl_xor(dot, m, 64);
          if (k == 0) out[base + j + u] = pooling == MX_POOL_MEAN ? __fmul_rn(dot, inv) : dot;
        }
      }
    }
  }
}

template <typename I, typename WT, int G, int NCH, bool WEIGHTED, bool OUT_F16>
void launch_fwd_group(hipStream_t s, const WT* W, const int64_t* w_off, const int32_t* D_off,
                      const BagMap& bm, const void* idx, const void* off, int32_t pooling,
                      const float* iw, void* out, int64_t nbags) {
  constexpr int U = NCH <= 1 ? 8 : (NCH <= 2 ? 4 : 2);  // rows in flight per lane
  constexpr int P = 64 / G;
  const int64_t grid = ceil_div(nbags, kWavesPerBlock * P);
  tbe_fwd_group_kernel<I, WT, G, NCH, U, WEIGHTED, OUT_F16><<<dim3(static_cast<uint32_t>(grid)), 256, 0, s>>>(
      W, w_off, D_off, bm, static_cast<const I*>(idx), static_cast<const I*>(off), pooling, iw, out,
      nbags);
}

template <typename I, typename WT, bool WEIGHTED, bool OUT_F16>
int dispatch_fwd(hipStream_t s, int32_t max_D, const WT* W, const int64_t* w_off,
                 const int32_t* D_off, const BagMap& bm, const void* idx, const void* off,
                 int32_t pooling, const float* iw, void* out, int64_t nbags) {
#define MX_FWD_G(G, NCH) \
  launch_fwd_group<I, WT, G, NCH, WEIGHTED, OUT_F16>(s, W, w_off, D_off, bm, idx, off, pooling, iw, out, nbags)
  if (max_D <= 64)
    MX_FWD_G(16, 1);  // 4 bags per wave
  else if (max_D <= 128)
    MX_FWD_G(32, 1);  // 2 bags per wave, one D=128 row per 32 lanes x 16 B
  else if (max_D <= 256)
    MX_FWD_G(64, 1);
  else if (max_D <= 512)
    MX_FWD_G(64, 2);
  else
    MX_FWD_G(64, 4);
#undef MX_FWD_G
  return MX_OK;
}

// ---- sequence lookups (PoolingMode NONE) -----------------------------------
//
// Semantics: fbgemm_gpu split_embedding_nobag_codegen_forward_unweighted_cuda
// (recalled): every table has the same D and position l of bag (t, b) writes
// its own row, out[l, :] = W_t[indices[l], :] (fp16 rows widened to fp32).
// Positions outside every bag (before offsets[0] or from offsets[T*B] on) are
// written as zeros.
//
// Design: a gather over positions, not bags, so no wave waits on a long bag.
// G lanes per position, lane k one float4 chunk per row; a group takes G
// consecutive positions at a time (one coalesced index load), each lane finds
// its own position's table by a binary search over the tables' first
// positions offsets[t*B] staged in LDS, and the group then copies U rows at a
// time (all U loads before the first store).  Blocks are remapped so that each
// XCD copies a contiguous range of positions (t-major, so mostly its own
// tables' hot rows).
constexpr int kNobagMaxT = 1024;  // tables whose first positions fit LDS; more: searched in memory

template <typename I>
__device__ __forceinline__ int32_t nobag_table(const int64_t* s_pos, bool lds, const I* offsets,
                                               int64_t B, int32_t T, int64_t l) {
  int32_t lo = 0, hi = T;  // pos[lo] <= l < pos[hi]
  while (hi - lo > 1) {
    const int32_t mid = lo + ((hi - lo) >> 1);
    const int64_t pm = lds ? s_pos[mid] : static_cast<int64_t>(offsets[mid * B]);
    if (pm <= l)
      lo = mid;
    else
      hi = mid;
  }
  return lo;
}

template <typename I, typename WT, int G, int NCH, int U, bool OUT_F16>
__global__ void __launch_bounds__(256)
    tbe_fwd_nobag_kernel(const WT* __restrict__ W, const int64_t* __restrict__ w_off,
                         const I* __restrict__ indices, const I* __restrict__ offsets, int32_t T,
                         int64_t B, int32_t D, int64_t N, void* __restrict__ out) {
  __shared__ int64_t s_pos[kNobagMaxT + 1];
  const bool lds = T <= kNobagMaxT;
  if (lds)
    for (int t = threadIdx.x; t <= T; t += 256) s_pos[t] = static_cast<int64_t>(offsets[t * B]);
  __syncthreads();
  const int64_t p0 = lds ? s_pos[0] : static_cast<int64_t>(offsets[0]);
  const int64_t p1 = lds ? s_pos[T] : static_cast<int64_t>(offsets[static_cast<int64_t>(T) * B]);
  constexpr int NG = 256 / G;  // groups per block
  const int lane = threadIdx.x & 63;
  const int g = lane / G, k = lane % G;
  const int64_t lb = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t step = static_cast<int64_t>(gridDim.x) * NG * G;
  for (int64_t base = (lb * NG + threadIdx.x / G) * G; base < N; base += step) {
    const int64_t l = base + k;
    int64_t my_row = -1;  // element offset of position l's row; -1: zeros
    if (l < N && l >= p0 && l < p1) {
      const int32_t t = nobag_table(s_pos, lds, offsets, B, T, l);
      my_row = w_off[t] + static_cast<int64_t>(indices[l]) * D;
    }
    const int n = static_cast<int>(N - base < G ? N - base : G);
    for (int j = 0; j < n; j += U) {
      float v[U][NCH][4];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int r = j + u < n ? j + u : n - 1;
        const int64_t off = __shfl(my_row, g * G + r, 64);
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
          const int col = (c * G + k) * 4;
          if (col < D && off >= 0)
            load_row4(W + off + col, v[u][c]);
          else
            v[u][c][0] = v[u][c][1] = v[u][c][2] = v[u][c][3] = 0.0f;
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (j + u >= n) continue;
        const int64_t o = (base + j + u) * D;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
          const int col = (c * G + k) * 4;
          if (col >= D) continue;
          if constexpr (OUT_F16) {
            __half2 h[2] = {__floats2half2_rn(v[u][c][0], v[u][c][1]),
                            __floats2half2_rn(v[u][c][2], v[u][c][3])};
            *reinterpret_cast<uint2*>(static_cast<__half*>(out) + o + col) =
                *reinterpret_cast<const uint2*>(h);
          } else {
            *reinterpret_cast<float4*>(static_cast<float*>(out) + o + col) =
                make_float4(v[u][c][0], v[u][c][1], v[u][c][2], v[u][c][3]);
          }
        }
      }
    }
  }
}

template <typename I, typename WT, int G, int NCH, bool OUT_F16>
void launch_nobag(hipStream_t s, const WT* W, const int64_t* w_off, const void* idx,
                  const void* off, int32_t T, int64_t B, int32_t D, int64_t N, void* out) {
  constexpr int U = NCH <= 1 ? 8 : (NCH <= 2 ? 4 : 2);
  const int64_t want = ceil_div(N, 256);  // 256 positions per block and round
  const int64_t cap = static_cast<int64_t>(num_cus()) * 16;
  const int64_t grid = want < cap ? want : cap;
  tbe_fwd_nobag_kernel<I, WT, G, NCH, U, OUT_F16><<<dim3(static_cast<uint32_t>(grid)), 256, 0, s>>>(
      W, w_off, static_cast<const I*>(idx), static_cast<const I*>(off), T, B, D, N, out);
}

template <typename I, typename WT, bool OUT_F16>
void dispatch_nobag(hipStream_t s, const WT* W, const int64_t* w_off, const void* idx,
                    const void* off, int32_t T, int64_t B, int32_t D, int64_t N, void* out) {
#define MX_NOBAG_G(G, NCH) launch_nobag<I, WT, G, NCH, OUT_F16>(s, W, w_off, idx, off, T, B, D, N, out)
  if (D <= 64)
    MX_NOBAG_G(16, 1);
  else if (D <= 128)
    MX_NOBAG_G(32, 1);
  else if (D <= 256)
    MX_NOBAG_G(64, 1);
  else if (D <= 512)
    MX_NOBAG_G(64, 2);
  else
    MX_NOBAG_G(64, 4);
#undef MX_NOBAG_G
}

}  // namespace
}  // namespace mx

using namespace mx;

namespace {

int tbe_forward_impl(const void* weights, int32_t weights_ty, const int64_t* weights_offsets,
                     const int32_t* D_offsets, int32_t T, int64_t nbags, int32_t max_D,
                     const void* indices, const void* offsets, int32_t index_bytes,
                     int32_t pooling_mode, const float* indice_weights, void* out,
                     int32_t out_dtype, const BagMap& bm, bool has_output, void* stream) {
  MX_REQUIRE(T >= 0 && nbags >= 0, "negative T or bag count");
  MX_REQUIRE(max_D >= 0 && max_D <= 1024 && max_D % 4 == 0,
             "max_D %d must be a multiple of 4 in [0, 1024]", max_D);
  MX_REQUIRE(index_bytes == 4 || index_bytes == 8, "indices must be int32 or int64");
  MX_REQUIRE(pooling_mode == MX_POOL_SUM || pooling_mode == MX_POOL_MEAN,
             "pooling_mode %d not supported (SUM=0, MEAN=1)", pooling_mode);
  MX_REQUIRE(out_dtype == MX_SPARSE_FP32 || out_dtype == MX_SPARSE_FP16,
             "output_dtype %d not supported (FP32=0, FP16=1)", out_dtype);
  MX_REQUIRE(weights_ty == MX_SPARSE_FP32 || weights_ty == MX_SPARSE_FP16,
             "weights type %d not supported (FP32=0, FP16=1)", weights_ty);
  if (nbags == 0 || !has_output) return MX_OK;
  MX_REQUIRE(weights && weights_offsets && D_offsets && offsets && out, "null pointer argument");
  MX_REQUIRE(ceil_div(nbags, kWavesPerBlock) <= 0x7fffffffll, "too many bags");
  auto* s = as_stream(stream);
  const bool w = indice_weights != nullptr;
  const bool h = out_dtype == MX_SPARSE_FP16;
#define MX_ARGS(WT) s, max_D, static_cast<const WT*>(weights), weights_offsets, D_offsets, bm, \
                indices, offsets, pooling_mode, indice_weights, out, nbags
#define MX_FWD_W(I, WT)                                                                          \
  if (w)                                                                                         \
    h ? dispatch_fwd<I, WT, true, true>(MX_ARGS(WT)) : dispatch_fwd<I, WT, true, false>(MX_ARGS(WT)); \
  else                                                                                           \
    h ? dispatch_fwd<I, WT, false, true>(MX_ARGS(WT)) : dispatch_fwd<I, WT, false, false>(MX_ARGS(WT));
  const bool w16 = weights_ty == MX_SPARSE_FP16;
  if (index_bytes == 8) {
    if (w16) {
      MX_FWD_W(int64_t, __half)
    } else {
      MX_FWD_W(int64_t, float)
    }
  } else {
    if (w16) {
      MX_FWD_W(int32_t, __half)
    } else {
      MX_FWD_W(int32_t, float)
    }
  }
#undef MX_FWD_W
#undef MX_ARGS
  MX_LAUNCH_CHECK();
  return MX_OK;
}

}  // namespace

extern "C" int mx_tbe_forward(const void* weights, int32_t weights_ty,
                              const int64_t* weights_offsets, const int32_t* D_offsets, int32_t T,
                              int64_t B, int32_t max_D, const void* indices, const void* offsets,
                              int32_t index_bytes, int32_t pooling_mode,
                              const float* indice_weights, void* out, int32_t out_dtype,
                              int64_t total_D, void* stream) {
  clear_error();
  MX_REQUIRE(T >= 0 && B >= 0, "negative T or B");
  const BagMap bm{B, total_D, nullptr, nullptr, 0};
  return tbe_forward_impl(weights, weights_ty, weights_offsets, D_offsets, T,
                          static_cast<int64_t>(T) * B, max_D, indices, offsets, index_bytes,
                          pooling_mode, indice_weights, out, out_dtype, bm, total_D > 0, stream);
}

extern "C" int mx_tbe_forward_vbe(const void* weights, int32_t weights_ty,
                                  const int64_t* weights_offsets, const int32_t* D_offsets,
                                  int32_t T, int64_t total_B, int32_t max_D, const void* indices,
                                  const void* offsets, int32_t index_bytes, int32_t pooling_mode,
                                  const float* indice_weights, const int64_t* vbe_row_output_offsets,
                                  const int32_t* vbe_b_t_map, int32_t info_B_num_bits, void* out,
                                  int32_t out_dtype, void* stream) {
  clear_error();
  MX_REQUIRE(info_B_num_bits >= 1 && info_B_num_bits <= 32, "info_B_num_bits %d invalid",
             info_B_num_bits);
  MX_REQUIRE(total_B == 0 || (vbe_row_output_offsets && vbe_b_t_map),
             "VBE metadata (row output offsets, b_t map) required");
  const BagMap bm{0, 0, vbe_b_t_map, vbe_row_output_offsets, info_B_num_bits};
  return tbe_forward_impl(weights, weights_ty, weights_offsets, D_offsets, T, total_B, max_D,
                          indices, offsets, index_bytes, pooling_mode, indice_weights, out,
                          out_dtype, bm, true, stream);
}

extern "C" int mx_tbe_forward_nobag(const void* weights, int32_t weights_ty,
                                    const int64_t* weights_offsets, int32_t T, int64_t B,
                                    int32_t D, const void* indices, const void* offsets,
                                    int32_t index_bytes, int64_t N, void* out, int32_t out_dtype,
                                    void* stream) {
  clear_error();
  MX_REQUIRE(T >= 0 && B >= 0 && N >= 0, "negative T, B or N");
  MX_REQUIRE(D > 0 && D <= 1024 && D % 4 == 0, "D %d must be a multiple of 4 in [4, 1024]", D);
  MX_REQUIRE(index_bytes == 4 || index_bytes == 8, "indices must be int32 or int64");
  MX_REQUIRE(out_dtype == MX_SPARSE_FP32 || out_dtype == MX_SPARSE_FP16,
             "output_dtype %d not supported (FP32=0, FP16=1)", out_dtype);
  MX_REQUIRE(weights_ty == MX_SPARSE_FP32 || weights_ty == MX_SPARSE_FP16,
             "weights type %d not supported (FP32=0, FP16=1)", weights_ty);
  if (N == 0) return MX_OK;
  MX_REQUIRE(T > 0 && B > 0, "%lld indices but no bags (T=%d, B=%lld)", (long long)N, T,
             (long long)B);
  MX_REQUIRE(weights && weights_offsets && indices && offsets && out, "null pointer argument");
  auto* s = as_stream(stream);
  const bool h = out_dtype == MX_SPARSE_FP16;
#define MX_NB(I, WT)                                                                          \
  (h ? dispatch_nobag<I, WT, true>(s, static_cast<const WT*>(weights), weights_offsets,       \
                                   indices, offsets, T, B, D, N, out)                          \
     : dispatch_nobag<I, WT, false>(s, static_cast<const WT*>(weights), weights_offsets,      \
                                    indices, offsets, T, B, D, N, out))
  const bool w16 = weights_ty == MX_SPARSE_FP16;
  if (index_bytes == 8) {
    if (w16)
      MX_NB(int64_t, __half);
    else
      MX_NB(int64_t, float);
  } else {
    if (w16)
      MX_NB(int32_t, __half);
    else
      MX_NB(int32_t, float);
  }
#undef MX_NB
  MX_LAUNCH_CHECK();
  return MX_OK;
}

namespace {

int grad_indice_weights_impl(const float* grad_output, const BagMap& bm, const void* weights,
                             int32_t weights_ty, const int64_t* weights_offsets,
                             const int32_t* D_offsets, int32_t T, int64_t nbags, int32_t max_D,
                             const void* indices, const void* offsets, int32_t index_bytes,
                             int32_t pooling_mode, const int32_t* feature_requires_grad,
                             float* grad_indice_weights, void* stream) {
  MX_REQUIRE(T >= 0 && nbags >= 0, "negative T or bag count");
  MX_REQUIRE(max_D >= 0 && max_D <= 1024 && max_D % 4 == 0,
             "max_D %d must be a multiple of 4 in [0, 1024]", max_D);
  MX_REQUIRE(index_bytes == 4 || index_bytes == 8, "indices must be int32 or int64");
  MX_REQUIRE(pooling_mode == MX_POOL_SUM || pooling_mode == MX_POOL_MEAN,
             "pooling_mode %d not supported (SUM=0, MEAN=1)", pooling_mode);
  MX_REQUIRE(weights_ty == MX_SPARSE_FP32 || weights_ty == MX_SPARSE_FP16,
             "weights type %d not supported (FP32=0, FP16=1)", weights_ty);
  if (nbags == 0) return MX_OK;
  MX_REQUIRE(grad_output && weights && weights_offsets && D_offsets && offsets &&
                 grad_indice_weights,
             "null pointer argument");
  auto* s = as_stream(stream);
#define MX_GIW(I, G, NCH, U)                                                                   \
  do {                                                                                         \
    if (weights_ty == MX_SPARSE_FP16)                                                          \
      MX_GIW_T(I, __half, G, NCH, U);                                                          \
    else                                                                                       \
      MX_GIW_T(I, float, G, NCH, U);                                                           \
  } while (0)
#define MX_GIW_T(I, WT, G, NCH, U)                                                             \
  grad_indice_weights_kernel<I, WT, G, NCH, U><<<dim3(static_cast<uint32_t>(                  \
                                               ceil_div(nbags, kWavesPerBlock * (64 / G)))),   \
                                           256, 0, s>>>(                                      \
      grad_output, bm, static_cast<const WT*>(weights), weights_offsets, D_offsets,            \
      static_cast<const I*>(indices), static_cast<const I*>(offsets), pooling_mode,            \
      feature_requires_grad, grad_indice_weights, nbags)
#define MX_GIW_D(I)                 \
  if (max_D <= 64)                  \
    MX_GIW(I, 16, 1, 8);            \
  else if (max_D <= 128)            \
    MX_GIW(I, 32, 1, 8);            \
  else if (max_D <= 256)            \
    MX_GIW(I, 64, 1, 8);            \
  else if (max_D <= 512)            \
    MX_GIW(I, 64, 2, 4);            \
  else                              \
    MX_GIW(I, 64, 4, 2);
  if (index_bytes == 8) {
    MX_GIW_D(int64_t)
  } else {
    MX_GIW_D(int32_t)
  }
#undef MX_GIW_D
#undef MX_GIW
#undef MX_GIW_T
  MX_LAUNCH_CHECK();
  return MX_OK;
}

}  // namespace

extern "C" int mx_tbe_grad_indice_weights(const float* grad_output, int64_t total_D,
                                          const void* weights, int32_t weights_ty,
                                          const int64_t* weights_offsets,
                                          const int32_t* D_offsets, int32_t T, int64_t B,
                                          int32_t max_D, const void* indices, const void* offsets,
                                          int32_t index_bytes, int32_t pooling_mode,
                                          const int32_t* feature_requires_grad,
                                          float* grad_indice_weights, void* stream) {
  clear_error();
  MX_REQUIRE(T >= 0 && B >= 0, "negative T or B");
  const BagMap bm{B, total_D, nullptr, nullptr, 0};
  return grad_indice_weights_impl(grad_output, bm, weights, weights_ty, weights_offsets,
                                  D_offsets, T, static_cast<int64_t>(T) * B, max_D, indices,
                                  offsets, index_bytes, pooling_mode, feature_requires_grad,
                                  grad_indice_weights, stream);
}

extern "C" int mx_tbe_grad_indice_weights_vbe(
    const float* grad_output, const void* weights, int32_t weights_ty,
    const int64_t* weights_offsets, const int32_t* D_offsets, int32_t T, int64_t total_B,
    int32_t max_D, const void* indices, const void* offsets, int32_t index_bytes,
    int32_t pooling_mode, const int64_t* vbe_row_output_offsets, const int32_t* vbe_b_t_map,
    int32_t info_B_num_bits, const int32_t* feature_requires_grad, float* grad_indice_weights,
    void* stream) {
  clear_error();
  MX_REQUIRE(info_B_num_bits >= 1 && info_B_num_bits <= 32, "info_B_num_bits %d invalid",
             info_B_num_bits);
  MX_REQUIRE(total_B == 0 || (vbe_row_output_offsets && vbe_b_t_map),
             "VBE metadata (row output offsets, b_t map) required");
  const BagMap bm{0, 0, vbe_b_t_map, vbe_row_output_offsets, info_B_num_bits};
  return grad_indice_weights_impl(grad_output, bm, weights, weights_ty, weights_offsets,
                                  D_offsets, T, total_B, max_D, indices, offsets, index_bytes,
                                  pooling_mode, feature_requires_grad, grad_indice_weights,
                                  stream);
}
