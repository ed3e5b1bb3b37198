// C-ABI plumbing shared by every entry point: thread-local error text, the
// launch-status check, and the per-device launch-fact cache.
#include <stdarg.h>

#include <map>
#include <mutex>
#include <utility>

#include "common.h"

namespace moe {

namespace {
thread_local char g_last_error[512] = "";
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return MOE_ERR_LAUNCH;
  }
  return MOE_OK;
}

// The library's only global state: facts about a device (compute units) and
// about a kernel on a device (resident blocks per CU), each computed once per
// device under one mutex.  Entries are keyed by device so that a process
// driving several GPUs, or several threads on different streams, reads the
// values of the device it launches on.
namespace {
std::mutex g_cache_mutex;
std::map<int, int> g_cus;                               // device -> compute units
std::map<std::pair<int, const void*>, int> g_occupancy;  // (device, kernel) -> blocks per CU
}  // namespace

int current_device() {
  int dev = 0;
  return hipGetDevice(&dev) == hipSuccess ? dev : 0;
}

int device_cus(int dev) {
  std::lock_guard<std::mutex> lock(g_cache_mutex);
  auto it = g_cus.find(dev);
  if (it != g_cus.end()) return it->second;
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
  g_cus.emplace(dev, n);
  return n;
}

int cached_blocks_per_cu(int dev, const void* kernel, int threads, int lds_bytes) {
  std::lock_guard<std::mutex> lock(g_cache_mutex);
  const auto key = std::make_pair(dev, kernel);
  auto it = g_occupancy.find(key);
  if (it != g_occupancy.end()) return it->second;
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, threads, lds_bytes) != hipSuccess) {
    (void)hipGetLastError();  // a failed query must not surface as the next launch's error
    n = 1;
  }
  if (n <= 0) n = 1;
  g_occupancy.emplace(key, n);
  return n;
}

}  // namespace moe

extern "C" const char* moe_last_error(void) { return moe::g_last_error; }

extern "C" int moe_abi_version(void) { return 4; }
