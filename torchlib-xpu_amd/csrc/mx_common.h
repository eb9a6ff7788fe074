// Shared helpers of the gfx950 kernels: status handling, launch geometry and
// small wave64 utilities.  Device code is written for CDNA4 only (wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

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

}  // namespace mx
