// Rowwise quantization codecs for gfx950: the formats the nbit lookup reads.
//
// Semantics: fbgemm_gpu FloatToFused8BitRowwiseQuantized /
// Fused8BitRowwiseQuantizedToFloat and FloatToFusedNBitRowwiseQuantizedSBHalf
// / FusedNBitRowwiseQuantizedSBHalfToFloat (upstream src/quantize_ops/,
// recalled), i.e. FBGEMM's FloatOrHalfToFused8BitRowwiseQuantizedSBFloat and
// FloatOrHalfToFusedNBitRowwiseQuantizedSBHalf (torch/include/fbgemm/
// QuantUtils.h declares them; torch's quantized::embedding_bag_{byte,4bit,
// 2bit}_prepack call them):
//   8-bit:  per row min m, max M; scale = (M - m) / 255, bias = m,
//           q = rint((x - m) * (255 / (M - m + 1e-8))); row = codes, fp32
//           scale, fp32 bias (D + 8 bytes).
//   N-bit:  bias = half(m); scale = half((M - bias) / (2^b - 1)) (1 if the
//           range is 0 or the scale underflows); q = clamp(rint((x - bias) *
//           (1 / scale)), 0, 2^b - 1), packed low bits first; row = codes,
//           fp16 scale, fp16 bias (ceil(D*b/8) + 4 bytes).
//   dequantize: x = q * scale + bias (one fma).
//
// One wave per row: the row is read twice (min/max, then codes; the second
// read hits L2), codes are written as consecutive bytes by consecutive lanes.
#include "mx_common.h"

namespace mx {
namespace {

template <typename T>
__device__ __forceinline__ float to_f32(T v);
template <>
__device__ __forceinline__ float to_f32<float>(float v) {
  return v;
}
template <>
__device__ __forceinline__ float to_f32<__half>(__half v) {
  return __half2float(v);
}

__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fminf(v, __shfl_xor(v, m, 64));
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

template <typename T>
__device__ __forceinline__ void row_min_max(const T* __restrict__ x, int64_t D, int lane, float* mn,
                                            float* mx_) {
  float lo = INFINITY, hi = -INFINITY;
  for (int64_t j = lane; j < D; j += 64) {
    const float v = to_f32(x[j]);
    lo = fminf(lo, v);
    hi = fmaxf(hi, v);
  }
  *mn = wave_min(lo);
  *mx_ = wave_max(hi);
}

template <typename T>
__global__ void __launch_bounds__(256)
    quantize_8bit_kernel(const T* __restrict__ in, int64_t rows, int64_t D,
                         uint8_t* __restrict__ out) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int lane = threadIdx.x & 63;
  const T* x = in + r * D;
  uint8_t* o = out + r * (D + 8);
  float mn, mxv;
  row_min_max(x, D, lane, &mn, &mxv);
  const float range = mxv - mn;
  const float scale = range / 255.0f;
  const float inv = 255.0f / (range + 1e-8f);
  for (int64_t j = lane; j < D; j += 64) {
    const float q = __builtin_rintf(__fmul_rn(to_f32(x[j]) - mn, inv));
    o[j] = static_cast<uint8_t>(q);
  }
  if (lane == 0) {
    float* sb = reinterpret_cast<float*>(o + D);  // D + 8 byte rows: 4-byte aligned when D % 4 == 0
    __builtin_memcpy(o + D, &scale, 4);
    __builtin_memcpy(o + D + 4, &mn, 4);
    (void)sb;
  }
}

__global__ void __launch_bounds__(256)
    dequantize_8bit_kernel(const uint8_t* __restrict__ in, int64_t rows, int64_t D,
                           void* __restrict__ out, int32_t out_f16) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int lane = threadIdx.x & 63;
  const uint8_t* x = in + r * (D + 8);
  float scale, bias;
  __builtin_memcpy(&scale, x + D, 4);
  __builtin_memcpy(&bias, x + D + 4, 4);
  for (int64_t j = lane; j < D; j += 64) {
    const float v = __builtin_fmaf(static_cast<float>(x[j]), scale, bias);
    if (out_f16)
      reinterpret_cast<__half*>(out)[r * D + j] = __float2half_rn(v);
    else
      reinterpret_cast<float*>(out)[r * D + j] = v;
  }
}

__device__ __forceinline__ float round_to_half(float v) { return __half2float(__float2half_rn(v)); }

template <typename T>
__global__ void __launch_bounds__(256)
    quantize_nbit_kernel(const T* __restrict__ in, int64_t rows, int64_t D, int32_t bits,
                         uint8_t* __restrict__ out) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int lane = threadIdx.x & 63;
  const int per_byte = 8 / bits;
  const int64_t nbytes = (D + per_byte - 1) / per_byte;
  const T* x = in + r * D;
  uint8_t* o = out + r * (nbytes + 4);
  float mn, mxv;
  row_min_max(x, D, lane, &mn, &mxv);
  const float bias = round_to_half(mn);
  const float range = mxv - bias;
  const int qmax = (1 << bits) - 1;
  float scale = range == 0.0f ? 1.0f : range / static_cast<float>(qmax);
  scale = round_to_half(scale);
  if (scale == 0.0f) scale = 1.0f;  // underflow in fp16
  float inv = 1.0f / scale;
  if (__builtin_isinf(inv)) {
    scale = 1.0f;
    inv = 1.0f;
  }
  for (int64_t p = lane; p < nbytes; p += 64) {
    uint32_t byte = 0;
    for (int e = 0; e < per_byte; ++e) {
      const int64_t j = p * per_byte + e;
      if (j >= D) break;
      float q = __builtin_rintf(__fmul_rn(to_f32(x[j]) - bias, inv));
      q = q < 0.0f ? 0.0f : (q > static_cast<float>(qmax) ? static_cast<float>(qmax) : q);
      byte |= static_cast<uint32_t>(q) << (e * bits);
    }
    o[p] = static_cast<uint8_t>(byte);
  }
  if (lane == 0) {
    const __half hs = __float2half_rn(scale), hb = __float2half_rn(bias);
    __builtin_memcpy(o + nbytes, &hs, 2);
    __builtin_memcpy(o + nbytes + 2, &hb, 2);
  }
}

__global__ void __launch_bounds__(256)
    dequantize_nbit_kernel(const uint8_t* __restrict__ in, int64_t rows, int64_t D, int32_t bits,
                           void* __restrict__ out, int32_t out_f16) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int lane = threadIdx.x & 63;
  const int per_byte = 8 / bits;
  const int64_t nbytes = (D + per_byte - 1) / per_byte;
  const uint8_t* x = in + r * (nbytes + 4);
  __half hs, hb;
  __builtin_memcpy(&hs, x + nbytes, 2);
  __builtin_memcpy(&hb, x + nbytes + 2, 2);
  const float scale = __half2float(hs), bias = __half2float(hb);
  const uint32_t mask = (1u << bits) - 1u;
  for (int64_t j = lane; j < D; j += 64) {
    const uint32_t q = (x[j / per_byte] >> ((j % per_byte) * bits)) & mask;
    const float v = __builtin_fmaf(static_cast<float>(q), scale, bias);
    if (out_f16)
      reinterpret_cast<__half*>(out)[r * D + j] = __float2half_rn(v);
    else
      reinterpret_cast<float*>(out)[r * D + j] = v;
  }
}

dim3 rows_grid(int64_t rows) { return dim3(static_cast<uint32_t>(ceil_div(rows, 4))); }

// hfp8 codecs: elementwise, grid-stride.
__global__ void __launch_bounds__(256)
    float_to_hfp8_kernel(const float* __restrict__ in, int64_t n, Hfp8 f, float clamp,
                         uint8_t* __restrict__ out) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * 256)
    out[i] = static_cast<uint8_t>(f.encode(in[i], clamp));
}

__global__ void __launch_bounds__(256)
    hfp8_to_float_kernel(const uint8_t* __restrict__ in, int64_t n, Hfp8 f,
                         float* __restrict__ out) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * 256)
    out[i] = f.decode(in[i]);
}

dim3 elementwise_grid(int64_t n) {
  const int64_t b = ceil_div(n, 256);
  return dim3(static_cast<uint32_t>(b < 8192 ? b : 8192));
}

}  // namespace
}  // namespace mx

using namespace mx;

extern "C" int mx_float_to_hfp8(const float* in, int64_t n, int32_t ebits, int32_t exponent_bias,
                                float max_pos, uint8_t* out, void* stream) {
  clear_error();
  MX_REQUIRE(n >= 0, "negative size");
  MX_REQUIRE(hfp8_format_ok(ebits, exponent_bias),
             "hfp8 needs 1 <= ebits <= 7 and 0 <= exponent_bias <= 120 (got %d, %d)", ebits,
             exponent_bias);
  MX_REQUIRE(max_pos > 0.0f, "max_pos must be positive");
  if (n == 0) return MX_OK;
  MX_REQUIRE(in && out, "null pointer argument");
  const Hfp8 f = Hfp8::make(ebits, exponent_bias);
  float_to_hfp8_kernel<<<elementwise_grid(n), 256, 0, as_stream(stream)>>>(
      in, n, f, max_pos < f.max_code ? max_pos : f.max_code, out);
  MX_LAUNCH_CHECK();
  return MX_OK;
}

extern "C" int mx_hfp8_to_float(const uint8_t* in, int64_t n, int32_t ebits,
                                int32_t exponent_bias, float* out, void* stream) {
  clear_error();
  MX_REQUIRE(n >= 0, "negative size");
  MX_REQUIRE(hfp8_format_ok(ebits, exponent_bias),
             "hfp8 needs 1 <= ebits <= 7 and 0 <= exponent_bias <= 120 (got %d, %d)", ebits,
             exponent_bias);
  if (n == 0) return MX_OK;
  MX_REQUIRE(in && out, "null pointer argument");
  hfp8_to_float_kernel<<<elementwise_grid(n), 256, 0, as_stream(stream)>>>(
      in, n, Hfp8::make(ebits, exponent_bias), out);
  MX_LAUNCH_CHECK();
  return MX_OK;
}

extern "C" int mx_quantize_fused8bit_rowwise(const void* in, int32_t in_dtype, int64_t rows,
                                             int64_t D, uint8_t* out, void* stream) {
  clear_error();
  MX_REQUIRE(rows >= 0 && D >= 0, "negative size");
  MX_REQUIRE(in_dtype == MX_DTYPE_F32 || in_dtype == MX_DTYPE_F16, "input must be fp32 or fp16");
  MX_REQUIRE(ceil_div(rows, 4) <= 0x7fffffffll, "too many rows");
  if (rows == 0) return MX_OK;
  MX_REQUIRE(in && out, "null pointer argument");
  auto* s = as_stream(stream);
  if (in_dtype == MX_DTYPE_F32)
    quantize_8bit_kernel<float><<<rows_grid(rows), 256, 0, s>>>(static_cast<const float*>(in), rows, D, out);
  else
    quantize_8bit_kernel<__half><<<rows_grid(rows), 256, 0, s>>>(static_cast<const __half*>(in), rows, D, out);
  MX_LAUNCH_CHECK();
  return MX_OK;
}

extern "C" int mx_dequantize_fused8bit_rowwise(const uint8_t* in, int64_t rows, int64_t D,
                                               void* out, int32_t out_dtype, void* stream) {
  clear_error();
  MX_REQUIRE(rows >= 0 && D >= 0, "negative size");
  MX_REQUIRE(out_dtype == MX_DTYPE_F32 || out_dtype == MX_DTYPE_F16, "output must be fp32 or fp16");
  MX_REQUIRE(ceil_div(rows, 4) <= 0x7fffffffll, "too many rows");
  if (rows == 0 || D == 0) return MX_OK;
  MX_REQUIRE(in && out, "null pointer argument");
  dequantize_8bit_kernel<<<rows_grid(rows), 256, 0, as_stream(stream)>>>(
      in, rows, D, out, out_dtype == MX_DTYPE_F16);
  MX_LAUNCH_CHECK();
  return MX_OK;
}

extern "C" int mx_quantize_fused_nbit_rowwise(const void* in, int32_t in_dtype, int64_t rows,
                                              int64_t D, int32_t bit_rate, uint8_t* out,
                                              void* stream) {
  clear_error();
  MX_REQUIRE(rows >= 0 && D >= 0, "negative size");
  MX_REQUIRE(bit_rate == 2 || bit_rate == 4 || bit_rate == 8, "bit_rate must be 2, 4 or 8");
  MX_REQUIRE(in_dtype == MX_DTYPE_F32 || in_dtype == MX_DTYPE_F16, "input must be fp32 or fp16");
  MX_REQUIRE(ceil_div(rows, 4) <= 0x7fffffffll, "too many rows");
  if (rows == 0) return MX_OK;
  MX_REQUIRE(in && out, "null pointer argument");
  auto* s = as_stream(stream);
  if (in_dtype == MX_DTYPE_F32)
    quantize_nbit_kernel<float><<<rows_grid(rows), 256, 0, s>>>(static_cast<const float*>(in), rows, D, bit_rate, out);
  else
    quantize_nbit_kernel<__half><<<rows_grid(rows), 256, 0, s>>>(static_cast<const __half*>(in), rows, D, bit_rate, out);
  MX_LAUNCH_CHECK();
  return MX_OK;
}

extern "C" int mx_dequantize_fused_nbit_rowwise(const uint8_t* in, int64_t rows, int64_t D,
                                                int32_t bit_rate, void* out, int32_t out_dtype,
                                                void* stream) {
  clear_error();
  MX_REQUIRE(rows >= 0 && D >= 0, "negative size");
  MX_REQUIRE(bit_rate == 2 || bit_rate == 4 || bit_rate == 8, "bit_rate must be 2, 4 or 8");
  MX_REQUIRE(out_dtype == MX_DTYPE_F32 || out_dtype == MX_DTYPE_F16, "output must be fp32 or fp16");
  MX_REQUIRE(ceil_div(rows, 4) <= 0x7fffffffll, "too many rows");
  if (rows == 0 || D == 0) return MX_OK;
  MX_REQUIRE(in && out, "null pointer argument");
  dequantize_nbit_kernel<<<rows_grid(rows), 256, 0, as_stream(stream)>>>(
      in, rows, D, bit_rate, out, out_dtype == MX_DTYPE_F16);
  MX_LAUNCH_CHECK();
  return MX_OK;
}
