// Shared helpers of the gfx950 kernels: status handling, launch geometry and
// small wave64 utilities.  Device code is written for CDNA4 only (wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>

#include "mx_fbgemm.h"

namespace mx {

constexpr int kWave = 64;

// Records the message of a failing call for mx_last_error(); returns `code`.
int set_error(int code, const char* fmt, ...);
void clear_error();

// Number of compute units of the current device (cached per device).
int num_cus();

// Host-visible status words registered for the current device
// (mx_set_status_mailbox, MX_STATUS_WORDS of them), or null: a look-back that
// gives up stores 1 into word MX_STATUS_LOOKBACK, an nbit lookup that meets a
// table it cannot serve into word MX_STATUS_NBIT_TABLE.
unsigned int* status_mailbox();
// Spin bound of the look-back waits: `dflt`, or -1 while the test hook that
// makes every look-back give up at once is on.
int lookback_spin_limit(int dflt);
// Test hook (mx_test_force_wide_sort_words): sort with 64-bit look-back words.
bool force_wide_sort_words();
// Test hook (mx_test_force_workspace_counters): eager backward calls clear
// their sort counters in the workspace, as captured calls do.
bool force_workspace_counters();

#define MX_REQUIRE(cond, ...)                                   \
  do {                                                          \
    if (!(cond)) return ::mx::set_error(MX_EINVAL, __VA_ARGS__); \
  } while (0)

#define MX_HIP_CHECK(expr)                                                              \
  do {                                                                                  \
    hipError_t mx_err_ = (expr);                                                        \
    if (mx_err_ != hipSuccess)                                                          \
      return ::mx::set_error(MX_EHIP, "%s failed: %s", #expr, hipGetErrorString(mx_err_)); \
  } while (0)

#define MX_LAUNCH_CHECK() MX_HIP_CHECK(hipGetLastError())

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Remaps a linear block id so that each of the 8 XCDs (which receive blocks
// round-robin) works on one contiguous eighth of the logical range.  Blocks
// that touch the same table then share one XCD's L2.
__device__ __forceinline__ int64_t xcd_remap(int64_t bid, int64_t nblocks) {
  constexpr int64_t kXcd = 8;
  const int64_t per = nblocks / kXcd;        // full rounds
  const int64_t full = per * kXcd;           // blocks covered by full rounds
  if (bid >= full) return bid;               // ragged tail keeps its id
  return (bid % kXcd) * per + bid / kXcd;
}

// Block-uniform load through the scalar data cache: the pointer is read as
// constant address space (s_load), valid for memory no thread of the kernel
// writes (data an earlier kernel wrote is seen: a dispatch invalidates the
// scalar cache).
template <typename T>
__device__ __forceinline__ T load_scalar(const T* p) {
  using CT = const __attribute__((address_space(4))) T;
  return *(CT*)(p);  // generic -> constant address space
}

template <typename T>
__device__ __forceinline__ T wave_bcast(T v, int lane) {
  return __shfl(v, lane, kWave);
}

// Scalar (SGPR) copy of lane `lane`'s 32-bit value; `lane` must be uniform.
__device__ __forceinline__ int32_t readlane_i32(int32_t v, int lane) {
  return __builtin_amdgcn_readlane(v, lane);
}
__device__ __forceinline__ int64_t readlane_i64(int64_t v, int lane) {
  const uint32_t lo = __builtin_amdgcn_readlane(static_cast<int32_t>(v & 0xffffffffll), lane);
  const uint32_t hi = __builtin_amdgcn_readlane(static_cast<int32_t>(v >> 32), lane);
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

__device__ __forceinline__ int lane_id() { return __lane_id(); }

// Sum over all 64 lanes (tree order fixed: deterministic).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}

template <typename I>
__device__ __forceinline__ int64_t ld_index(const void* p, int64_t i) {
  return static_cast<int64_t>(reinterpret_cast<const I*>(p)[i]);
}

// hfp8: the 8-bit float of fbgemm's FP8 TBE tables and HFP8 codecs (FBGEMM's
// Float8ToFloat_ref / FloatToFloat8_ref, torch/include/fbgemm/
// FbgemmConvert.h:181-200): a sign bit, `ebits` exponent bits and
// m = 7 - ebits mantissa bits, exponent bias `bias`; a code of exponent field
// E > 0 is 2^(E - bias) (1 + M / 2^m), of E = 0 the subnormal M 2^(1 - bias - m).
// With 1 <= ebits <= 7 and 0 <= bias <= 120 every code is a normal fp32
// number or zero, so decoding is exact and denormal-free.
inline bool hfp8_format_ok(int ebits, int bias) {
  return ebits >= 1 && ebits <= 7 && bias >= 0 && bias <= 120;
}

struct Hfp8 {
  int32_t m;        // mantissa bits
  int32_t bias;
  int32_t exp_off;  // 127 - bias: added to a code's exponent field gives fp32's
  float sub_scale;  // 2^(1 - bias - m), the subnormal quantum
  float sub_inv;    // 2^(bias + m - 1)
  float min_normal; // 2^(1 - bias)
  float max_code;   // the largest magnitude (every exponent field a number)

  static Hfp8 make(int ebits, int bias) {
    Hfp8 f;
    f.m = 7 - ebits;
    f.bias = bias;
    f.exp_off = 127 - bias;
    f.sub_scale = ldexpf(1.0f, 1 - bias - f.m);
    f.sub_inv = ldexpf(1.0f, bias + f.m - 1);
    f.min_normal = ldexpf(1.0f, 1 - bias);
    f.max_code = ldexpf(2.0f - ldexpf(1.0f, -f.m), (1 << ebits) - 1 - bias);
    return f;
  }

  // Code c (0..255) as fp32: a nonzero exponent field is built directly as
  // fp32 bits (the magnitude bits under fp32's exponent field, rebased), a
  // zero one as M times the quantum; the sign bit last (0x80 is -0).
  __device__ __forceinline__ float decode(uint32_t c) const {
    const uint32_t mag = c & 0x7fu;
    const float normal =
        __uint_as_float((mag << (23 - m)) + (static_cast<uint32_t>(exp_off) << 23));
    const float v = (mag >> m) != 0u ? normal : static_cast<float>(mag) * sub_scale;
    return __uint_as_float(__float_as_uint(v) | ((c & 0x80u) << 24));
  }

  // The code nearest to x (ties to even) after |x| is clamped to `clamp`
  // (at most max_code): below min_normal on the subnormal grid, else on the
  // grid of x's binade, a round-up into the next binade carrying into the
  // exponent field.  NaN encodes as the clamp.
  __device__ __forceinline__ uint32_t encode(float x, float clamp) const {
    const uint32_t s = (__float_as_uint(x) >> 24) & 0x80u;
    const float a = fminf(fabsf(x), clamp);
    if (a < min_normal) return s | static_cast<uint32_t>(rintf(a * sub_inv));
    const int be = static_cast<int>((__float_as_uint(a) >> 23) & 0xffu) - 127;
    const uint32_t k = static_cast<uint32_t>(rintf(ldexpf(a, m - be)));  // 2^m .. 2^(m+1)
    uint32_t e = static_cast<uint32_t>(be + bias), mant = k - (1u << m);
    if (mant == (1u << m)) {
      e += 1u;
      mant = 0u;
    }
    return s | (e << m) | mant;
  }
};

}  // namespace mx
