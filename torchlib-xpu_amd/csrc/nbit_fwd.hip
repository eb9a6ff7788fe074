// Quantized ("nbit") TBE inference forward for gfx950: FP32, FP16, INT8,
// INT4, INT2 and FP8 (hfp8) tables, one launch per type present; fp32, fp16
// or bf16 output.
//
// Semantics: fbgemm_gpu int_nbit_split_embedding_codegen_lookup_function
// (upstream codegen/inference/, recalled).  Row layout is the TBE layout of
// torch/include/fbgemm/FbgemmEmbedding.h:88-92,144-149 (scale_bias_last =
// false): an fp16 scale and an fp16 bias at the front of each INT8/INT4/INT2
// row, then the codes, the even element of each INT4 byte in the low
// nibble; value = scale * q + bias in fp32.  Rows are padded to
// row_alignment bytes.
//
// Design: a wave serves P = 64/G bags of one table at once; each group of G
// lanes walks its own bag's rows in index order, lane k owning columns
// [k*CPL, (k+1)*CPL) with CPL = D/G.  A lane reads its CPL codes with one
// wide load (INT8 D=128: 16 B), the row's qparams with one dword load, and
// dequantizes in registers as acc += scale*q, keeping sum(bias) apart, so
// each code costs one byte-selecting convert (plus a mask per word of INT4 or
// INT2 codes) and one FMA, an fp16 element one mixed-precision FMA, and no
// cross-lane reduction is needed.  The G indices of a batch are fetched with one coalesced load by
// the group and handed out with ds_bpermute.  Tables of every type share the
// launch; the type/width switch is wave-uniform.
#include <type_traits>

#include "mx_common.h"

namespace mx {
namespace {

// Bytes of row data each lane keeps in flight (sets the rows loaded before
// any is accumulated).
constexpr int kInflightBytes = 96;

struct NbitArgs {
  const uint8_t* W;
  const int64_t* w_off;
  const uint8_t* tys;
  const int32_t* D_off;
  const void* idx;
  const void* off;
  const float* iw;
  void* out;
  int64_t B;
  int64_t Bp;  // B rounded up to bags-per-block
  int64_t total_D;
  int64_t nwaves;
  int32_t T;
  int32_t pooling;
  int32_t row_align;
  int32_t out_kind;        // output element: 0 fp32, 1 fp16, 2 bf16
  int32_t served;          // bit ty set: the call launches type ty
  Hfp8 fp8;                // FP8 tables' format (when served)
  uint32_t nchk;           // trailing blocks that check the tables (T in the first launch, else 0)
  unsigned int* mailbox;   // host-visible status words of the device, may be null
};

// A table the call can serve: its type has a launch, its D is not negative,
// and its codes fill whole bytes (INT4: D even, INT2: D a multiple of 4; the
// row holds D*bits/8 code bytes, rounded down).
template <int TY>
__device__ __forceinline__ bool whole_bytes(int32_t D) {
  if constexpr (TY == MX_SPARSE_INT4) return (D & 1) == 0;
  if constexpr (TY == MX_SPARSE_INT2) return (D & 3) == 0;
  return true;
}

__device__ __host__ __forceinline__ int64_t row_bytes_of(int32_t ty, int32_t D, int32_t align) {
  int64_t u;
  switch (ty) {
    case MX_SPARSE_FP32: u = 4ll * D; break;
    case MX_SPARSE_FP16: u = 2ll * D; break;
    case MX_SPARSE_INT8: u = D + 4ll; break;
    case MX_SPARSE_INT4: u = D / 2 + 4ll; break;
    case MX_SPARSE_INT2: u = D / 4 + 4ll; break;
    case MX_SPARSE_FP8: u = D; break;
    default: return -1;
  }
  if (align > 1) u = (u + align - 1) / align * align;
  return u;
}

// Rows start at 4-byte boundaries (the kernels read codes and qparams in
// 4-byte words): the table's first byte and its row stride are multiples of 4.
__device__ __host__ __forceinline__ bool rows_aligned(int64_t w_off, int64_t stride) {
  return ((w_off | stride) & 3) == 0;
}

__device__ __forceinline__ bool table_ok(int32_t ty, int32_t D, int32_t served, int64_t w_off,
                                         int32_t align) {
  if (ty < 0 || ty > MX_SPARSE_FP8 || ty == MX_SPARSE_BF16 || ((served >> ty) & 1) == 0 || D < 0)
    return false;
  if (!rows_aligned(w_off, row_bytes_of(ty, D, align))) return false;
  if (ty == MX_SPARSE_INT4) return whole_bytes<MX_SPARSE_INT4>(D);
  if (ty == MX_SPARSE_INT2) return whole_bytes<MX_SPARSE_INT2>(D);
  return true;
}

template <int TY>
struct TyInfo;
template <>
struct TyInfo<MX_SPARSE_FP32> {
  static constexpr int kBits = 32;
  static constexpr bool kQ = false;
};
template <>
struct TyInfo<MX_SPARSE_FP16> {
  static constexpr int kBits = 16;
  static constexpr bool kQ = false;
};
template <>
struct TyInfo<MX_SPARSE_INT8> {
  static constexpr int kBits = 8;
  static constexpr bool kQ = true;
};
template <>
struct TyInfo<MX_SPARSE_INT4> {
  static constexpr int kBits = 4;
  static constexpr bool kQ = true;
};
template <>
struct TyInfo<MX_SPARSE_INT2> {
  static constexpr int kBits = 2;
  static constexpr bool kQ = true;
};
template <>
struct TyInfo<MX_SPARSE_FP8> {
  static constexpr int kBits = 8;
  static constexpr bool kQ = false;
};

typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x2a4 __attribute__((ext_vector_type(2), aligned(4)));

// Loads BPL bytes (a power of two) starting at p into 32-bit words.
template <int BPL>
__device__ __forceinline__ void load_codes(const uint8_t* p, uint32_t (&w)[BPL >= 4 ? BPL / 4 : 1]) {
  if constexpr (BPL == 1) {
    w[0] = *p;
  } else if constexpr (BPL == 2) {
    w[0] = *reinterpret_cast<const uint16_t*>(p);
  } else if constexpr (BPL == 4) {
    w[0] = *reinterpret_cast<const uint32_t*>(p);
  } else if constexpr (BPL == 8) {
    const u32x2a4 v = *reinterpret_cast<const u32x2a4*>(p);
    w[0] = v.x;
    w[1] = v.y;
  } else {
#pragma unroll
    for (int q = 0; q < BPL / 16; ++q) {
      const u32x4a4 v = *reinterpret_cast<const u32x4a4*>(p + 16 * q);
      w[4 * q + 0] = v.x;
      w[4 * q + 1] = v.y;
      w[4 * q + 2] = v.z;
      w[4 * q + 3] = v.w;
    }
  }
}

// Element e of the lane's chunk as fp32 (the raw code for integer types).
template <int TY, int BPL>
__device__ __forceinline__ float elem(const uint32_t (&w)[BPL >= 4 ? BPL / 4 : 1], int e) {
  constexpr int bits = TyInfo<TY>::kBits;
  const int bit = e * bits;
  const uint32_t word = w[bit >> 5];
  const int sh = bit & 31;
  if constexpr (TY == MX_SPARSE_FP32) {
    return __uint_as_float(word);
  } else if constexpr (TY == MX_SPARSE_FP16) {
    const uint16_t h = static_cast<uint16_t>(word >> sh);
    return __half2float(__ushort_as_half(h));
  } else {
    return static_cast<float>((word >> sh) & ((1u << bits) - 1u));
  }
}

// fp32 of byte N of x: v_cvt_f32_ubyteN selects the byte itself, so a code
// costs one instruction (the compiler emits a bit-field extract and
// v_cvt_f32_ubyte0 for the shift-and-mask form).
template <int N>
__device__ __forceinline__ float ubyte_f32(uint32_t x) {
  float f;
  if constexpr (N == 0)
    asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(f) : "v"(x));
  else if constexpr (N == 1)
    asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(f) : "v"(x));
  else if constexpr (N == 2)
    asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(f) : "v"(x));
  else
    asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(f) : "v"(x));
  return f;
}

// The 32/bits codes of one little-endian word as fp32, in element order: for
// INT4 the low and high nibbles of each byte are masked into two words
// (0x0F0F0F0F), for INT2 the four 2-bit fields into four, and each byte is
// then converted directly.  Exact: every code is a small integer.
template <int BITS>
__device__ __forceinline__ void decode_word(uint32_t w, float (&f)[32 / BITS]) {
  if constexpr (BITS == 8) {
    f[0] = ubyte_f32<0>(w);
    f[1] = ubyte_f32<1>(w);
    f[2] = ubyte_f32<2>(w);
    f[3] = ubyte_f32<3>(w);
  } else {
    constexpr int K = 8 / BITS;  // codes per byte
    constexpr uint32_t m = BITS == 4 ? 0x0F0F0F0Fu : 0x03030303u;
#pragma unroll
    for (int j = 0; j < K; ++j) {
      const uint32_t p = (w >> (j * BITS)) & m;  // field j of every byte
      f[0 * K + j] = ubyte_f32<0>(p);
      f[1 * K + j] = ubyte_f32<1>(p);
      f[2 * K + j] = ubyte_f32<2>(p);
      f[3 * K + j] = ubyte_f32<3>(p);
    }
  }
}

// acc + m * (fp16 half H of w), one v_fma_mix_f32 (the half converts inside
// the FMA, rounded once as fma(float(h), m, acc)).
template <int H>
__device__ __forceinline__ float fma_half(uint32_t w, float m, float acc) {
  float r;
  if constexpr (H == 0)
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(w), "v"(m), "v"(acc));
  else
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
        : "=v"(r)
        : "v"(w), "v"(m), "v"(acc));
  return r;
}

template <typename I>
__device__ __forceinline__ int64_t idx_at(const void* p, int64_t i) {
  return static_cast<int64_t>(reinterpret_cast<const I*>(p)[i]);
}

// A 16-bit output element: fp16 rounded to nearest even, or bf16 as FBGEMM's
// CPU kernels write it (the top half of the fp32 bits after adding 0x8000:
// to nearest, ties away from zero; NaN stays a quiet NaN).
__device__ __forceinline__ uint16_t out16(float v, int32_t kind) {
  if (kind == 1) return __half_as_ushort(__float2half_rn(v));
  const uint32_t x = __float_as_uint(v);
  if ((x & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((x >> 16) | 0x40u);
  return static_cast<uint16_t>((x + 0x8000u) >> 16);
}

__device__ __forceinline__ void store_out(const NbitArgs& a, int64_t col_base, int ncols,
                                          const float* v) {
  if (a.out_kind != 0) {
    uint16_t* o = reinterpret_cast<uint16_t*>(a.out) + col_base;
    for (int e = 0; e < ncols; ++e) o[e] = out16(v[e], a.out_kind);
  } else {
    float* o = reinterpret_cast<float*>(a.out) + col_base;
    for (int e = 0; e < ncols; ++e) o[e] = v[e];
  }
}

// Fast path: CPL columns per lane, CPL*bits a multiple of 8.  A lane's BPL
// code bytes are NCHK chunks of CH <= 16 bytes, interleaved across the group:
// chunk q of lane k is bytes (q*G + k)*CH of the row's codes.  Each load
// instruction then covers one contiguous G*CH-byte span of every row (one
// 128-byte line for G*CH = 128) instead of touching every line of a wide row
// with a few lanes each, which multiplied the texture path's tag lookups.
template <typename I, int G, int TY, int CPL>
__device__ void bag_fast(const NbitArgs& a, const uint8_t* __restrict__ Wt, int64_t stride,
                         int64_t start, int64_t end, int64_t out_col, int g, int k) {
  constexpr int BITS = TyInfo<TY>::kBits;
  constexpr bool Q = TyInfo<TY>::kQ;
  constexpr int BPL = CPL * BITS / 8;
  constexpr int NW = BPL >= 4 ? BPL / 4 : 1;
  constexpr int CH = BPL < 16 ? BPL : 16;  // bytes per chunk (one load)
  constexpr int NCHK = BPL / CH;           // chunks per lane
  constexpr int CPC = CPL / NCHK;          // columns per chunk
  constexpr int WPC = NW / NCHK;           // code words per chunk
  constexpr int U0 = kInflightBytes / (BPL + (Q ? 4 : 0));
  constexpr int U = U0 < 1 ? 1 : (U0 > 8 ? 8 : U0);
  const int64_t lane_off = (Q ? 4 : 0) + static_cast<int64_t>(k) * CH;

  float acc[CPL];
#pragma unroll
  for (int e = 0; e < CPL; ++e) acc[e] = 0.0f;
  float bsum = 0.0f;
  const bool weighted = a.iw != nullptr;

  // Row numbers travel between lanes as one 32-bit word when the indices are
  // int32 (one ds_bpermute and one 32x32->64 multiply-add per row); a row is
  // under 2^32 bytes.
  using R = std::conditional_t<sizeof(I) == 4, uint32_t, int64_t>;
  const uint32_t stride32 = static_cast<uint32_t>(stride);
  // The group's indices come G at a time, one batch ahead of its rows, so a
  // bag longer than G does not wait for its next batch of indices (config 5:
  // 1,181 -> 1,144 us per call; config 4: 423.6 -> 421.6 us).  Batches of 2G
  // indices where the in-flight budget holds 2G narrow rows measured no
  // further gain (1,142.6 us); 128 or 160 bytes in flight per lane instead of
  // 96: 1,217 and 1,371 us.
  R nxt_idx = start + k < end ? static_cast<R>(reinterpret_cast<const I*>(a.idx)[start + k]) : R(0);
  float nxt_w = (weighted && start + k < end) ? a.iw[start + k] : 1.0f;
  for (int64_t base = start; base < end; base += G) {
    const int n = static_cast<int>(end - base < G ? end - base : G);
    const R my_idx = nxt_idx;
    const float my_w = nxt_w;
    if (base + G + k < end) {
      nxt_idx = static_cast<R>(reinterpret_cast<const I*>(a.idx)[base + G + k]);
      if (weighted) nxt_w = a.iw[base + G + k];
    }
    for (int j = 0; j < n; j += U) {
      uint32_t codes[U][NW];
      uint32_t qp[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        // Lanes past the batch (j + u >= n) hold row 0 and go unused.
        const R r = __shfl(my_idx, g * G + j + u, 64);
        if (j + u < n) {
          const uint8_t* row = Wt + static_cast<uint64_t>(r) * stride32;
#pragma unroll
          for (int q = 0; q < NCHK; ++q)
            load_codes<CH>(row + lane_off + q * G * CH,
                           *reinterpret_cast<uint32_t(*)[WPC]>(&codes[u][q * WPC]));
          if constexpr (Q) qp[u] = *reinterpret_cast<const uint32_t*>(row);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float wgt = __shfl(my_w, g * G + j + u, 64);
        if (j + u < n) {
          if constexpr (Q) {
            float scale = __half2float(__ushort_as_half(static_cast<uint16_t>(qp[u] & 0xffffu)));
            float bias = __half2float(__ushort_as_half(static_cast<uint16_t>(qp[u] >> 16)));
            if (weighted) {
              scale *= wgt;
              bias *= wgt;
            }
            bsum += bias;
            constexpr int EPW = 32 / BITS;  // codes per word
#pragma unroll
            for (int q = 0; q < NW; ++q) {
              float f[EPW];
              decode_word<BITS>(codes[u][q], f);
#pragma unroll
              for (int j = 0; j < EPW; ++j)
                if (q * EPW + j < CPL) acc[q * EPW + j] = __builtin_fmaf(scale, f[j], acc[q * EPW + j]);
            }
          } else if constexpr (TY == MX_SPARSE_FP8) {
#pragma unroll
            for (int e = 0; e < CPL; ++e) {
              const float v = a.fp8.decode((codes[u][e >> 2] >> ((e & 3) * 8)) & 0xffu);
              acc[e] = weighted ? __builtin_fmaf(wgt, v, acc[e]) : acc[e] + v;
            }
          } else if constexpr (TY == MX_SPARSE_FP16) {
            // acc += w * h with the fp16 converted inside the FMA (w = 1
            // unweighted: exactly acc + float(h)).
            const float m = weighted ? wgt : 1.0f;
#pragma unroll
            for (int e = 0; e < CPL; e += 2) {
              acc[e] = fma_half<0>(codes[u][e / 2], m, acc[e]);
              if (e + 1 < CPL) acc[e + 1] = fma_half<1>(codes[u][e / 2], m, acc[e + 1]);
            }
          } else {
            if (weighted) {
#pragma unroll
              for (int e = 0; e < CPL; ++e)
                acc[e] = __builtin_fmaf(wgt, elem<TY, BPL>(codes[u], e), acc[e]);
            } else {
#pragma unroll
              for (int e = 0; e < CPL; ++e) acc[e] += elem<TY, BPL>(codes[u], e);
            }
          }
        }
      }
    }
  }
  const int64_t L = end - start;
  const float inv = (a.pooling == MX_POOL_MEAN && L > 0) ? 1.0f / static_cast<float>(L) : 1.0f;
  float res[CPL];
#pragma unroll
  for (int e = 0; e < CPL; ++e) res[e] = (acc[e] + bsum) * inv;
  if (L == 0) {
#pragma unroll
    for (int e = 0; e < CPL; ++e) res[e] = 0.0f;
  }
  // Element e of the lane is column (q*G + k)*CPC + j of the table, e = q*CPC + j.
  const int64_t col = out_col + static_cast<int64_t>(k) * CPC;
  if (a.out_kind != 0) {
    uint16_t h[CPL];
    if (a.out_kind == 1) {  // the conversion loops apart, so each stays straight-line
#pragma unroll
      for (int e = 0; e < CPL; ++e) h[e] = __half_as_ushort(__float2half_rn(res[e]));
    } else {
#pragma unroll
      for (int e = 0; e < CPL; ++e) h[e] = out16(res[e], 2);
    }
#pragma unroll
    for (int q = 0; q < NCHK; ++q) {
      uint16_t* o = reinterpret_cast<uint16_t*>(a.out) + col + q * G * CPC;
      const uint16_t* hq = h + q * CPC;
      if constexpr (CPC % 8 == 0) {
#pragma unroll
        for (int v = 0; v < CPC / 8; ++v)
          *reinterpret_cast<uint4*>(o + 8 * v) = *reinterpret_cast<const uint4*>(hq + 8 * v);
      } else if constexpr (CPC == 4) {
        *reinterpret_cast<uint2*>(o) = *reinterpret_cast<const uint2*>(hq);
      } else {
#pragma unroll
        for (int e = 0; e < CPC; ++e) o[e] = hq[e];
      }
    }
  } else {
#pragma unroll
    for (int q = 0; q < NCHK; ++q) {
      float* o = reinterpret_cast<float*>(a.out) + col + q * G * CPC;
      const float* rq = res + q * CPC;
      if constexpr (CPC % 4 == 0) {
#pragma unroll
        for (int v = 0; v < CPC / 4; ++v)
          *reinterpret_cast<float4*>(o + 4 * v) =
              make_float4(rq[4 * v], rq[4 * v + 1], rq[4 * v + 2], rq[4 * v + 3]);
      } else {
#pragma unroll
        for (int e = 0; e < CPC; ++e) o[e] = rq[e];
      }
    }
  }
}

// Any D: lanes own 8-column blocks, one block sweep per pass over the bag.
template <typename I, int G>
__device__ void bag_generic(const NbitArgs& a, int32_t ty, int32_t D,
                            const uint8_t* __restrict__ Wt, int64_t stride, int64_t start,
                            int64_t end, int64_t out_col, int k) {
  const int bits = ty == MX_SPARSE_FP32 ? 32 : ty == MX_SPARSE_FP16 ? 16
                 : (ty == MX_SPARSE_INT8 || ty == MX_SPARSE_FP8) ? 8 : ty == MX_SPARSE_INT4 ? 4 : 2;
  const bool q = ty == MX_SPARSE_INT8 || ty == MX_SPARSE_INT4 || ty == MX_SPARSE_INT2;
  const int64_t L = end - start;
  const float inv = (a.pooling == MX_POOL_MEAN && L > 0) ? 1.0f / static_cast<float>(L) : 1.0f;
  for (int cb = k * 8; cb < D; cb += G * 8) {
    const int nc = D - cb < 8 ? D - cb : 8;
    float acc[8];
    for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
    float bsum = 0.0f;
    for (int64_t l = start; l < end; ++l) {
      const int64_t r = idx_at<I>(a.idx, l);
      const float wgt = a.iw ? a.iw[l] : 1.0f;
      const uint8_t* row = Wt + r * stride;
      float scale = 1.0f;
      if (q) {
        const uint32_t qp = *reinterpret_cast<const uint32_t*>(row);
        scale = __half2float(__ushort_as_half(static_cast<uint16_t>(qp & 0xffffu))) * wgt;
        bsum += __half2float(__ushort_as_half(static_cast<uint16_t>(qp >> 16))) * wgt;
        row += 4;
      }
      for (int e = 0; e < nc; ++e) {
        const int c = cb + e;
        float v;
        if (bits == 32) {
          v = reinterpret_cast<const float*>(row)[c];
        } else if (ty == MX_SPARSE_FP8) {
          v = a.fp8.decode(row[c]);
        } else if (bits == 16) {
          v = __half2float(__ushort_as_half(reinterpret_cast<const uint16_t*>(row)[c]));
        } else {
          const int bit = c * bits;
          v = static_cast<float>((row[bit >> 3] >> (bit & 7)) & ((1 << bits) - 1));
        }
        acc[e] = q ? __builtin_fmaf(scale, v, acc[e]) : __builtin_fmaf(wgt, v, acc[e]);
      }
    }
    float res[8];
    for (int e = 0; e < 8; ++e) res[e] = L > 0 ? (acc[e] + bsum) * inv : 0.0f;
    store_out(a, out_col + cb, nc, res);
  }
}

template <typename I, int G, int MAXCPL, int TY>
__device__ __forceinline__ void dispatch_cpl(const NbitArgs& a, int32_t D,
                                             const uint8_t* __restrict__ Wt, int64_t stride,
                                             int64_t start, int64_t end, int64_t out_col, int g,
                                             int k) {
  constexpr int BITS = TyInfo<TY>::kBits;
  const int cpl = D / G;
  if (cpl * G == D) {
    switch (cpl) {
#define MX_CPL(C)                                                                  \
  case C:                                                                          \
    if constexpr ((C * BITS) % 8 == 0 && C * BITS <= 512 && C <= MAXCPL) {         \
      bag_fast<I, G, TY, C>(a, Wt, stride, start, end, out_col, g, k);             \
      return;                                                                      \
    }                                                                              \
    break;
      MX_CPL(2)
      MX_CPL(4)
      MX_CPL(8)
      MX_CPL(16)
      MX_CPL(32)
#undef MX_CPL
      default: break;
    }
  }
  bag_generic<I, G>(a, TY, D, Wt, stride, start, end, out_col, k);
}

// Waves per block: a block ranks its waves x 64/G bags by length.
constexpr int kWpb = 4;
constexpr int kBlockThreads = 64 * kWpb;

// MAXCPL bounds the columns per lane compiled into this instance: the kernel's
// register budget is set by its widest path, so a launch whose tables are all
// narrow (max D <= 16*G) runs an instance without the 32-column paths.
// One launch per table type present: the instance holds only that type's
// paths (fewer registers, higher occupancy); waves whose table has another
// type return at once.

// Table t's type byte: the scalar unit loads dwords, so the aligned dword
// holding it is read (its four bytes share one page, so the read stays in
// mapped memory even for the last byte of the array).
__device__ __forceinline__ int32_t table_type(const uint8_t* tys, int64_t t) {
  const uintptr_t addr = reinterpret_cast<uintptr_t>(tys) + static_cast<uintptr_t>(t);
  const uint32_t w = load_scalar(reinterpret_cast<const uint32_t*>(addr & ~uintptr_t(3)));
  return static_cast<int32_t>((w >> (8 * (addr & 3))) & 0xffu);
}

// Run by one block per table, appended to the call's first launch: a table
// no launch of the call serves (a type byte outside the served types, or
// codes that do not fill whole bytes) gets its columns of every bag written
// as zeros, and the call reports it through the device's status words.
__device__ __forceinline__ void check_table(const NbitArgs& a, int64_t t, int32_t ty) {
  const int32_t D0 = load_scalar(a.D_off + t);
  const int32_t D = load_scalar(a.D_off + t + 1) - D0;
  if (table_ok(ty, D, a.served, load_scalar(a.w_off + t), a.row_align)) return;
  const int64_t c0 = D0 < 0 ? 0 : D0;
  const int64_t c1 = static_cast<int64_t>(D0) + (D > 0 ? D : 0);
  const int64_t nc = (c1 < a.total_D ? c1 : a.total_D) - c0;
  for (int64_t b = 0; b < a.B; ++b)
    for (int64_t c = threadIdx.x; c < nc; c += blockDim.x) {
      const int64_t o = b * a.total_D + c0 + c;
      if (a.out_kind != 0)
        reinterpret_cast<uint16_t*>(a.out)[o] = 0u;  // +0 in fp16 and bf16
      else
        reinterpret_cast<float*>(a.out)[o] = 0.0f;
    }
  if (threadIdx.x == 0 && a.mailbox)
    __hip_atomic_store(a.mailbox + MX_STATUS_NBIT_TABLE, 1u, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_SYSTEM);
}

template <typename I, int G, int MAXCPL, int TY>
__device__ __forceinline__ void nbit_fwd_body(const NbitArgs& a) {
  constexpr int P = 64 / G;           // bags per wave
  constexpr int BPB = kWpb * P;       // bags per block, all of one table
  // Hardware block order (round-robin over the XCDs): tables of different
  // types interleave on every XCD, so no XCD is left with only the slow ones.
  // Half of a two-type launch's blocks find another type and leave: their
  // table comes from a 32-bit division and its type from a scalar load, so
  // they hold their slot for a few hundred cycles.
  const uint32_t bpt = static_cast<uint32_t>(a.Bp / BPB);  // blocks per table
  const uint32_t tu = blockIdx.x / bpt;
  if (tu >= static_cast<uint32_t>(a.T)) {  // block-uniform
    // The call's first launch ends with nchk = T blocks, one per table, that
    // check the tables.  Config 5 per call, against no check: +2.5 us with
    // the blocks here, +9.5 us with them first in the grid (every block then
    // tests its index against nchk) or with the checks made by blocks that
    // leave at the type test below (half the blocks of a two-type launch).
    const int64_t tc = static_cast<int64_t>(blockIdx.x) - static_cast<int64_t>(a.T) * bpt;
    if (tc < a.nchk) check_table(a, tc, table_type(a.tys, tc));
    return;
  }
  const int64_t t = tu;
  const int32_t ty = table_type(a.tys, t);
  if (ty != TY) return;  // block-uniform
  const int64_t b0 = static_cast<int64_t>(blockIdx.x - tu * bpt) * BPB;
  // A wave lasts as long as its longest bag: the block ranks its BPB bags by
  // length (longest first, ties by position) and wave w takes ranks
  // [w*P, w*P + P), so bags of similar length share a wave.  Each bag still
  // writes its own output row.
  static_assert(BPB <= kBlockThreads, "one thread per bag ranks the block's bags");
  __shared__ int64_t s_start[BPB], s_end[BPB];
  __shared__ int s_bag[BPB];
  if (threadIdx.x < BPB) {
    const int64_t b = b0 + threadIdx.x;
    int64_t start = 0, end = -1;  // slots past the batch rank last
    if (b < a.B) {
      start = idx_at<I>(a.off, t * a.B + b);
      end = idx_at<I>(a.off, t * a.B + b + 1);
    }
    s_start[threadIdx.x] = start;
    s_end[threadIdx.x] = end;
  }
  __syncthreads();
  if (threadIdx.x < BPB) {
    const int i = threadIdx.x;
    const int64_t li = s_end[i] - s_start[i];
    int rank = 0;
    for (int j = 0; j < BPB; ++j) {
      const int64_t lj = s_end[j] - s_start[j];
      rank += (lj > li || (lj == li && j < i)) ? 1 : 0;
    }
    s_bag[rank] = i;
  }
  __syncthreads();
  const int32_t D0 = load_scalar(a.D_off + t);
  const int32_t D = load_scalar(a.D_off + t + 1) - D0;
  const int64_t stride = row_bytes_of(ty, D, a.row_align);
  const int64_t wo = load_scalar(a.w_off + t);
  // A table whose codes leave a partial byte, or whose rows do not start at
  // 4-byte boundaries, is left to the check blocks.
  if (!whole_bytes<TY>(D) || !rows_aligned(wo, stride)) return;  // block-uniform
  const int lane = threadIdx.x & 63;
  const int g = lane / G;
  const int k = lane % G;
  const uint8_t* __restrict__ Wt = a.W + wo;
  const int i = s_bag[(threadIdx.x >> 6) * P + g];
  const int64_t b = b0 + i;
  if (b >= a.B) return;  // whole group idle (idle slots rank last); its lanes stay converged
  dispatch_cpl<I, G, MAXCPL, TY>(a, D, Wt, stride, s_start[i], s_end[i], b * a.total_D + D0, g, k);
}

// The check blocks alone, for a call that launches no type.
__global__ void __launch_bounds__(kBlockThreads) nbit_check_kernel(NbitArgs a) {
  check_table(a, blockIdx.x, table_type(a.tys, blockIdx.x));
}

template <typename I, int G, int MAXCPL, int TY>
__global__ void __launch_bounds__(kBlockThreads) nbit_fwd_kernel(NbitArgs a) {
  nbit_fwd_body<I, G, MAXCPL, TY>(a);
}

// INT4 tables: the same body held to 96 registers for 5 waves per SIMD
// (config 5's INT4 launch: 684 against 734 us at 4 waves; the other types
// either fit already or would spill).
template <typename I, int G, int MAXCPL, int TY>
__global__ void __launch_bounds__(kBlockThreads) __attribute__((amdgpu_waves_per_eu(5)))
    nbit_fwd_kernel_w5(NbitArgs a) {
  nbit_fwd_body<I, G, MAXCPL, TY>(a);
}

template <int G, int MAXCPL, int TY>
int launch_nbit(NbitArgs a, int32_t index_bytes, hipStream_t s) {
  constexpr int BPB = kWpb * (64 / G);  // bags per block
  a.Bp = ceil_div(a.B, BPB) * BPB;      // every block within one table
  a.nwaves = static_cast<int64_t>(a.T) * (a.Bp / BPB) * kWpb;
  const int64_t grid = ceil_div(a.nwaves, kWpb) + a.nchk;  // + the check blocks
  MX_REQUIRE(grid <= 0x7fffffffll, "too many bags");
  const dim3 gd(static_cast<uint32_t>(grid));
  if constexpr (TY == MX_SPARSE_INT4) {
    if (index_bytes == 8)
      nbit_fwd_kernel_w5<int64_t, G, MAXCPL, TY><<<gd, kBlockThreads, 0, s>>>(a);
    else
      nbit_fwd_kernel_w5<int32_t, G, MAXCPL, TY><<<gd, kBlockThreads, 0, s>>>(a);
  } else {
    if (index_bytes == 8)
      nbit_fwd_kernel<int64_t, G, MAXCPL, TY><<<gd, kBlockThreads, 0, s>>>(a);
    else
      nbit_fwd_kernel<int32_t, G, MAXCPL, TY><<<gd, kBlockThreads, 0, s>>>(a);
  }
  MX_LAUNCH_CHECK();
  return MX_OK;
}

// Lanes per bag and widest compiled path from the type's largest D.
template <int TY>
int launch_type(const NbitArgs& a, int32_t max_D, int32_t index_bytes, hipStream_t s) {
  if (max_D <= 0) return MX_OK;
  if (max_D <= 128) return launch_nbit<8, 16, TY>(a, index_bytes, s);
  if (max_D <= 256) return launch_nbit<8, 32, TY>(a, index_bytes, s);
  if (max_D <= 512) return launch_nbit<16, 32, TY>(a, index_bytes, s);
  return launch_nbit<32, 32, TY>(a, index_bytes, s);
}

// ---- sequence lookups (PoolingMode NONE) -----------------------------------
//
// Semantics: fbgemm_gpu int_nbit_split_embedding_nobag_codegen_forward_
// unweighted_cuda (recalled): every table has the same D (the largest max_*_D)
// and position l writes its own dequantized row, out[l, :].  An INT8/INT4/INT2
// element is fma(scale, q, bias) in fp32 (one rounding, as FBGEMM's CPU kernels
// dequantize the first row of a bag); FP32, FP16 and FP8 elements are the row's
// values themselves.  Then the output rounding of the pooled lookup.
//
// Design: a gather over positions, one launch per type present: G = 16 lanes
// per position, lane k the 8-element blocks k, k + 16, ... of the row; a group
// takes 16 consecutive positions (one coalesced index load), each lane finds
// its position's table by a binary search over the tables' first positions in
// LDS, and positions of another type's tables are left to that type's launch.
// U rows are loaded before the first is stored.  Tables the call cannot serve
// (unlaunched type, partial code bytes, misaligned rows, D other than the
// call's) and positions outside every bag are written as zeros by the check
// launch, which reports such tables through the status words.
constexpr int kNobagMaxT = 1024;
constexpr int kNobagG = 16;
constexpr int kNobagU = 4;

// Table of position l: the last t with offsets[t*B] <= l.
template <typename I>
__device__ __forceinline__ int32_t nobag_table(const int64_t* s_pos, bool lds, const NbitArgs& a,
                                               int64_t l) {
  int32_t lo = 0, hi = a.T;
  while (hi - lo > 1) {
    const int32_t mid = lo + ((hi - lo) >> 1);
    const int64_t pm = lds ? s_pos[mid] : idx_at<I>(a.off, mid * a.B);
    if (pm <= l)
      lo = mid;
    else
      hi = mid;
  }
  return lo;
}

template <typename I>
__device__ __forceinline__ void stage_positions(const NbitArgs& a, int64_t* s_pos, bool lds) {
  if (lds)
    for (int t = threadIdx.x; t <= a.T; t += blockDim.x) s_pos[t] = idx_at<I>(a.off, t * a.B);
  __syncthreads();
}

// Bytes [o, o + n) of a row (n <= 32, o at the element block's start) into
// little-endian words: whole words when the block's bytes are whole words at
// 4-byte alignment (rows start 4-aligned), else byte by byte.
template <int NB>
__device__ __forceinline__ void load_block(const uint8_t* p, int n, uint32_t (&w)[8]) {
  if (n == NB && (NB % 4 == 0)) {
#pragma unroll
    for (int q = 0; q < NB / 4; ++q) w[q] = reinterpret_cast<const uint32_t*>(p)[q];
  } else if (n == NB && NB == 2) {
    w[0] = *reinterpret_cast<const uint16_t*>(p);
  } else {
#pragma unroll
    for (int q = 0; q < 8; ++q) w[q] = 0u;
    for (int i = 0; i < n; ++i) w[i >> 2] |= static_cast<uint32_t>(p[i]) << ((i & 3) * 8);
  }
}

// Element e of a block of TY codes (the raw code for integer types).
template <int TY>
__device__ __forceinline__ float block_elem(const NbitArgs& a, const uint32_t (&w)[8], int e) {
  constexpr int bits = TyInfo<TY>::kBits;
  const int bit = e * bits;
  const uint32_t word = w[bit >> 5];
  const int sh = bit & 31;
  if constexpr (TY == MX_SPARSE_FP32) return __uint_as_float(word);
  if constexpr (TY == MX_SPARSE_FP16)
    return __half2float(__ushort_as_half(static_cast<uint16_t>(word >> sh)));
  if constexpr (TY == MX_SPARSE_FP8) return a.fp8.decode((word >> sh) & 0xffu);
  return static_cast<float>((word >> sh) & ((1u << bits) - 1u));
}

template <typename I, int TY>
__global__ void __launch_bounds__(256) nbit_nobag_kernel(NbitArgs a, int32_t D, int64_t N) {
  constexpr int G = kNobagG, U = kNobagU, NG = 256 / G;
  constexpr int BITS = TyInfo<TY>::kBits;
  constexpr bool Q = TyInfo<TY>::kQ;
  constexpr int NB = 8 * BITS / 8;  // bytes of a full 8-element block
  __shared__ int64_t s_pos[kNobagMaxT + 1];
  const bool lds = a.T <= kNobagMaxT;
  stage_positions<I>(a, s_pos, lds);
  const int64_t p0 = lds ? s_pos[0] : idx_at<I>(a.off, 0);
  const int64_t p1 = lds ? s_pos[a.T] : idx_at<I>(a.off, static_cast<int64_t>(a.T) * a.B);
  const int lane = threadIdx.x & 63;
  const int g = lane / G, k = lane % G;
  const int64_t lb = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t step = static_cast<int64_t>(gridDim.x) * NG * G;
  for (int64_t base = (lb * NG + threadIdx.x / G) * G; base < N; base += step) {
    const int64_t l = base + k;
    int64_t my_row = -1;  // byte offset of l's row in the weights; -1: not this launch's
    if (l < N && l >= p0 && l < p1) {
      const int32_t t = nobag_table<I>(s_pos, lds, a, l);
      const int32_t Dt = a.D_off[t + 1] - a.D_off[t];
      const int64_t wo = a.w_off[t];
      if (static_cast<int32_t>(a.tys[t]) == TY && Dt == D &&
          table_ok(TY, Dt, a.served, wo, a.row_align))
        my_row = wo + idx_at<I>(a.idx, l) * row_bytes_of(TY, Dt, a.row_align);
    }
    const int n = static_cast<int>(N - base < G ? N - base : G);
    for (int j = 0; j < n; j += U) {
      int64_t roff[U];
#pragma unroll
      for (int u = 0; u < U; ++u) roff[u] = __shfl(my_row, g * G + (j + u < n ? j + u : n - 1), 64);
      for (int cb = k * 8; cb < D; cb += G * 8) {
        const int nc = D - cb < 8 ? D - cb : 8;
        const int nbytes = nc * BITS / 8;
        uint32_t w[U][8];
        uint32_t qp[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          qp[u] = 0u;
          if (j + u < n && roff[u] >= 0) {
            const uint8_t* row = a.W + roff[u];
            load_block<NB>(row + (Q ? 4 : 0) + cb * BITS / 8, nbytes, w[u]);
            if constexpr (Q) qp[u] = *reinterpret_cast<const uint32_t*>(row);
          }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          if (j + u >= n || roff[u] < 0) continue;
          float v[8];
          const float scale = __half2float(__ushort_as_half(static_cast<uint16_t>(qp[u] & 0xffffu)));
          const float bias = __half2float(__ushort_as_half(static_cast<uint16_t>(qp[u] >> 16)));
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float x = block_elem<TY>(a, w[u], e);
            v[e] = Q ? __builtin_fmaf(scale, x, bias) : x;
          }
          store_out(a, (base + j + u) * D + cb, nc, v);
        }
      }
    }
  }
}

// One block per table zeroes the positions of a table the call cannot serve
// and reports it; block T zeroes the positions outside every bag.
template <typename I>
__global__ void __launch_bounds__(256) nbit_nobag_check_kernel(NbitArgs a, int32_t D, int64_t N) {
  const int64_t t = blockIdx.x;
  int64_t lo, hi, lo2 = 0, hi2 = 0;
  if (t < a.T) {
    const int32_t Dt = a.D_off[t + 1] - a.D_off[t];
    if (Dt == D && table_ok(a.tys[t], Dt, a.served, a.w_off[t], a.row_align)) return;
    lo = idx_at<I>(a.off, t * a.B);
    hi = idx_at<I>(a.off, (t + 1) * a.B);
    if (threadIdx.x == 0 && a.mailbox)
      __hip_atomic_store(a.mailbox + MX_STATUS_NBIT_TABLE, 1u, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_SYSTEM);
  } else {
    lo = 0;
    hi = idx_at<I>(a.off, 0);
    lo2 = idx_at<I>(a.off, static_cast<int64_t>(a.T) * a.B);
    hi2 = N;
  }
  for (int r = 0; r < 2; ++r) {
    int64_t s0 = r == 0 ? lo : lo2, s1 = r == 0 ? hi : hi2;
    s0 = s0 < 0 ? 0 : s0;
    s1 = s1 > N ? N : s1;
    for (int64_t i = s0 * D + threadIdx.x; i < s1 * D; i += blockDim.x) {
      if (a.out_kind != 0)
        reinterpret_cast<uint16_t*>(a.out)[i] = 0u;
      else
        reinterpret_cast<float*>(a.out)[i] = 0.0f;
    }
  }
}

template <int TY>
int launch_nobag_type(const NbitArgs& a, int32_t max_D, int32_t D, int64_t N,
                      int32_t index_bytes, hipStream_t s) {
  if (max_D <= 0) return MX_OK;
  const int64_t want = ceil_div(N, 256);  // 256 positions per block and round
  const int64_t cap = static_cast<int64_t>(num_cus()) * 16;
  const dim3 gd(static_cast<uint32_t>(want < cap ? want : cap));
  if (index_bytes == 8)
    nbit_nobag_kernel<int64_t, TY><<<gd, 256, 0, s>>>(a, D, N);
  else
    nbit_nobag_kernel<int32_t, TY><<<gd, 256, 0, s>>>(a, D, N);
  MX_LAUNCH_CHECK();
  return MX_OK;
}

}  // namespace
}  // namespace mx

using namespace mx;

extern "C" int64_t mx_nbit_row_bytes(int32_t ty, int32_t D, int32_t row_alignment) {
  if (D < 0) return -1;
  return row_bytes_of(ty, D, row_alignment);
}

extern "C" int mx_nbit_forward(const uint8_t* dev_weights, const int64_t* weights_offsets,
                               const uint8_t* weights_tys, const int32_t* D_offsets, int32_t T,
                               int64_t B, int32_t max_int2_D, int32_t max_int4_D,
                               int32_t max_int8_D, int32_t max_float16_D, int32_t max_float32_D,
                               const void* indices, const void* offsets, int32_t index_bytes,
                               int32_t pooling_mode, const float* indice_weights,
                               int32_t output_dtype, int32_t row_alignment,
                               int32_t max_float8_D, int32_t fp8_exponent_bits,
                               int32_t fp8_exponent_bias, void* out, int64_t total_D,
                               void* stream) {
  clear_error();
  MX_REQUIRE(T >= 0 && B >= 0, "negative T or B");
  MX_REQUIRE(index_bytes == 4 || index_bytes == 8, "indices must be int32 or int64");
  MX_REQUIRE(pooling_mode == MX_POOL_SUM || pooling_mode == MX_POOL_MEAN,
             "pooling_mode %d not supported (SUM=0, MEAN=1)", pooling_mode);
  MX_REQUIRE(output_dtype == MX_SPARSE_FP32 || output_dtype == MX_SPARSE_FP16 ||
                 output_dtype == MX_SPARSE_BF16,
             "output_dtype %d not supported (FP32=0, FP16=1, BF16=5)", output_dtype);
  MX_REQUIRE(row_alignment >= 1, "row_alignment must be positive");
  int32_t max_D = 0;
  for (int32_t d :
       {max_int2_D, max_int4_D, max_int8_D, max_float16_D, max_float32_D, max_float8_D}) {
    MX_REQUIRE(d >= 0, "negative max_D");
    if (d > max_D) max_D = d;
  }
  MX_REQUIRE(max_D <= 1024, "max D %d above 1024", max_D);
  // Codes fill whole bytes of a row (its size is D*bits/8 + 4 rounded down).
  MX_REQUIRE(max_int4_D % 2 == 0 && max_int2_D % 4 == 0,
             "INT4 D must be even and INT2 D a multiple of 4 (max_int4_D %d, max_int2_D %d)",
             max_int4_D, max_int2_D);
  MX_REQUIRE(max_float8_D == 0 || hfp8_format_ok(fp8_exponent_bits, fp8_exponent_bias),
             "FP8 tables need 1 <= fp8_exponent_bits <= 7 and 0 <= fp8_exponent_bias <= 120 "
             "(got %d, %d)", fp8_exponent_bits, fp8_exponent_bias);
  if (static_cast<int64_t>(T) * B == 0 || total_D == 0) return MX_OK;
  MX_REQUIRE(dev_weights && weights_offsets && weights_tys && D_offsets && offsets && out,
             "null pointer argument");
  NbitArgs a;
  a.W = dev_weights;
  a.w_off = weights_offsets;
  a.tys = weights_tys;
  a.D_off = D_offsets;
  a.idx = indices;
  a.off = offsets;
  a.iw = indice_weights;
  a.out = out;
  a.B = B;
  a.Bp = 0;
  a.total_D = total_D;
  a.nwaves = 0;
  a.T = T;
  a.pooling = pooling_mode;
  a.row_align = row_alignment;
  a.out_kind = output_dtype == MX_SPARSE_FP16 ? 1 : (output_dtype == MX_SPARSE_BF16 ? 2 : 0);
  a.served = (max_int8_D > 0 ? 1 << MX_SPARSE_INT8 : 0) | (max_int4_D > 0 ? 1 << MX_SPARSE_INT4 : 0) |
             (max_int2_D > 0 ? 1 << MX_SPARSE_INT2 : 0) |
             (max_float16_D > 0 ? 1 << MX_SPARSE_FP16 : 0) |
             (max_float32_D > 0 ? 1 << MX_SPARSE_FP32 : 0) |
             (max_float8_D > 0 ? 1 << MX_SPARSE_FP8 : 0);
  a.fp8 = max_float8_D > 0 ? Hfp8::make(fp8_exponent_bits, fp8_exponent_bias) : Hfp8::make(4, 7);
  a.nchk = static_cast<uint32_t>(T);  // the first launch checks the tables
  a.mailbox = status_mailbox();
  auto* s = as_stream(stream);
  // Tables of a type whose max_*_D is 0 are not served (the upstream contract:
  // the maxima describe the tables); the first launch's check blocks zero their
  // columns and report them, and so they do for INT4/INT2 tables whose D
  // leaves a partial byte.  With no type to launch, the check blocks run alone.
  if (a.served == 0) {
    nbit_check_kernel<<<dim3(static_cast<uint32_t>(T)), kBlockThreads, 0, s>>>(a);
    MX_LAUNCH_CHECK();
    return MX_OK;
  }
  if (int rc = launch_type<MX_SPARSE_INT8>(a, max_int8_D, index_bytes, s)) return rc;
  if (max_int8_D > 0) a.nchk = 0;
  if (int rc = launch_type<MX_SPARSE_INT4>(a, max_int4_D, index_bytes, s)) return rc;
  if (max_int4_D > 0) a.nchk = 0;
  if (int rc = launch_type<MX_SPARSE_INT2>(a, max_int2_D, index_bytes, s)) return rc;
  if (max_int2_D > 0) a.nchk = 0;
  if (int rc = launch_type<MX_SPARSE_FP16>(a, max_float16_D, index_bytes, s)) return rc;
  if (max_float16_D > 0) a.nchk = 0;
  if (int rc = launch_type<MX_SPARSE_FP8>(a, max_float8_D, index_bytes, s)) return rc;
  if (max_float8_D > 0) a.nchk = 0;
  return launch_type<MX_SPARSE_FP32>(a, max_float32_D, index_bytes, s);
}

extern "C" int mx_nbit_forward_nobag(const uint8_t* dev_weights, const int64_t* weights_offsets,
                                     const uint8_t* weights_tys, const int32_t* D_offsets,
                                     int32_t T, int64_t B, int32_t max_int2_D, int32_t max_int4_D,
                                     int32_t max_int8_D, int32_t max_float16_D,
                                     int32_t max_float32_D, const void* indices,
                                     const void* offsets, int32_t index_bytes, int64_t N,
                                     int32_t output_dtype, int32_t row_alignment,
                                     int32_t max_float8_D, int32_t fp8_exponent_bits,
                                     int32_t fp8_exponent_bias, void* out, void* stream) {
  clear_error();
  MX_REQUIRE(T >= 0 && B >= 0 && N >= 0, "negative T, B or N");
  MX_REQUIRE(index_bytes == 4 || index_bytes == 8, "indices must be int32 or int64");
  MX_REQUIRE(output_dtype == MX_SPARSE_FP32 || output_dtype == MX_SPARSE_FP16 ||
                 output_dtype == MX_SPARSE_BF16,
             "output_dtype %d not supported (FP32=0, FP16=1, BF16=5)", output_dtype);
  MX_REQUIRE(row_alignment >= 1, "row_alignment must be positive");
  int32_t D = 0;
  for (int32_t d :
       {max_int2_D, max_int4_D, max_int8_D, max_float16_D, max_float32_D, max_float8_D}) {
    MX_REQUIRE(d >= 0, "negative max_D");
    if (d > D) D = d;
  }
  MX_REQUIRE(D <= 1024, "max D %d above 1024", D);
  MX_REQUIRE(max_int4_D % 2 == 0 && max_int2_D % 4 == 0,
             "INT4 D must be even and INT2 D a multiple of 4 (max_int4_D %d, max_int2_D %d)",
             max_int4_D, max_int2_D);
  MX_REQUIRE(max_float8_D == 0 || hfp8_format_ok(fp8_exponent_bits, fp8_exponent_bias),
             "FP8 tables need 1 <= fp8_exponent_bits <= 7 and 0 <= fp8_exponent_bias <= 120 "
             "(got %d, %d)", fp8_exponent_bits, fp8_exponent_bias);
  if (N == 0 || D == 0) return MX_OK;
  MX_REQUIRE(T > 0 && B > 0, "%lld indices but no bags (T=%d, B=%lld)", (long long)N, T,
             (long long)B);
  MX_REQUIRE(dev_weights && weights_offsets && weights_tys && D_offsets && indices && offsets &&
                 out,
             "null pointer argument");
  NbitArgs a{};
  a.W = dev_weights;
  a.w_off = weights_offsets;
  a.tys = weights_tys;
  a.D_off = D_offsets;
  a.idx = indices;
  a.off = offsets;
  a.iw = nullptr;
  a.out = out;
  a.B = B;
  a.total_D = D;
  a.T = T;
  a.pooling = MX_POOL_NONE;
  a.row_align = row_alignment;
  a.out_kind = output_dtype == MX_SPARSE_FP16 ? 1 : (output_dtype == MX_SPARSE_BF16 ? 2 : 0);
  a.served = (max_int8_D > 0 ? 1 << MX_SPARSE_INT8 : 0) | (max_int4_D > 0 ? 1 << MX_SPARSE_INT4 : 0) |
             (max_int2_D > 0 ? 1 << MX_SPARSE_INT2 : 0) |
             (max_float16_D > 0 ? 1 << MX_SPARSE_FP16 : 0) |
             (max_float32_D > 0 ? 1 << MX_SPARSE_FP32 : 0) |
             (max_float8_D > 0 ? 1 << MX_SPARSE_FP8 : 0);
  a.fp8 = max_float8_D > 0 ? Hfp8::make(fp8_exponent_bits, fp8_exponent_bias) : Hfp8::make(4, 7);
  a.nchk = 0;
  a.mailbox = status_mailbox();
  auto* s = as_stream(stream);
  const dim3 cg(static_cast<uint32_t>(T) + 1);
  if (index_bytes == 8)
    nbit_nobag_check_kernel<int64_t><<<cg, 256, 0, s>>>(a, D, N);
  else
    nbit_nobag_check_kernel<int32_t><<<cg, 256, 0, s>>>(a, D, N);
  MX_LAUNCH_CHECK();
  if (int rc = launch_nobag_type<MX_SPARSE_INT8>(a, max_int8_D, D, N, index_bytes, s)) return rc;
  if (int rc = launch_nobag_type<MX_SPARSE_INT4>(a, max_int4_D, D, N, index_bytes, s)) return rc;
  if (int rc = launch_nobag_type<MX_SPARSE_INT2>(a, max_int2_D, D, N, index_bytes, s)) return rc;
  if (int rc = launch_nobag_type<MX_SPARSE_FP16>(a, max_float16_D, D, N, index_bytes, s)) return rc;
  if (int rc = launch_nobag_type<MX_SPARSE_FP8>(a, max_float8_D, D, N, index_bytes, s)) return rc;
  return launch_nobag_type<MX_SPARSE_FP32>(a, max_float32_D, D, N, index_bytes, s);
}
