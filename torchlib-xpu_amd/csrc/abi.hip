// Status reporting and device queries shared by every entry point.
#include <atomic>
#include <mutex>
#include <string>

#include "mx_common.h"
#include "scan.h"

namespace mx {

namespace {
thread_local std::string g_last_error;
}

int set_error(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

void clear_error() { g_last_error.clear(); }

int num_cus() {
  static std::mutex mu;
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

namespace {
std::mutex g_mailbox_mu;
unsigned int* g_mailbox[64] = {};
std::atomic<int> g_force_giveup{0};
std::atomic<int> g_force_wide{0};
std::atomic<int> g_force_ws_counters{0};
}  // namespace

unsigned int* status_mailbox() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  std::lock_guard<std::mutex> lock(g_mailbox_mu);
  return g_mailbox[dev];
}

int lookback_spin_limit(int dflt) { return g_force_giveup.load() ? -1 : dflt; }

bool force_wide_sort_words() { return g_force_wide.load() != 0; }

bool force_workspace_counters() { return g_force_ws_counters.load() != 0; }

__global__ void zero_u64_kernel(unsigned long long* p, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    p[i] = 0ull;
}

}  // namespace mx

extern "C" int mx_version(void) { return MX_FBGEMM_VERSION; }

extern "C" const char* mx_last_error(void) { return mx::g_last_error.c_str(); }

extern "C" int mx_set_status_mailbox(unsigned int* host_words) {
  mx::clear_error();
  int dev = 0;
  MX_HIP_CHECK(hipGetDevice(&dev));
  MX_REQUIRE(dev >= 0 && dev < 64, "device %d out of range", dev);
  std::lock_guard<std::mutex> lock(mx::g_mailbox_mu);
  mx::g_mailbox[dev] = host_words;
  return MX_OK;
}

extern "C" int mx_test_force_lookback_giveup(int enable) {
  mx::g_force_giveup.store(enable != 0 ? 1 : 0);
  return MX_OK;
}

extern "C" int mx_test_force_wide_sort_words(int enable) {
  mx::g_force_wide.store(enable != 0 ? 1 : 0);
  return MX_OK;
}

extern "C" int mx_test_force_workspace_counters(int enable) {
  mx::g_force_ws_counters.store(enable != 0 ? 1 : 0);
  return MX_OK;
}
