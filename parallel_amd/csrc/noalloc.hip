// moe_permute_fwd_noalloc: the routing permutation of moe_permute_fwd for
// callers that cannot allocate device memory (code under HIP graph capture,
// tight serving loops, harnesses that forbid it).  The per-chunk histogram
// lives in a fixed device array instead of a caller workspace.
#include <mutex>

#include "common.h"

namespace {

// 1 MiB: room for the histogram of 2032 chunks of 512 routes at 128 buckets
// (just over a million routes); in general 1 MiB / (4 (num_buckets + 1))
// chunks.  Each GPU the library runs on holds its own copy until the process
// ends.  In host code `scratch` names a host-side stand-in, never device
// memory: the device address of the current device's copy comes from
// hipGetSymbolAddress, looked up once per device.
constexpr size_t kScratchBytes = size_t(1) << 20;
constexpr int kMaxScratchDevices = 64;

std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxScratchDevices] = {};  // device -> address of its copy (a fixed table: no allocation)

}  // namespace

static __device__ __align__(256) int32_t scratch[kScratchBytes / sizeof(int32_t)];

namespace {

int scratch_of_current_device(void** out) {
  const int dev = moe::current_device();
  MOE_REQUIRE(dev >= 0 && dev < kMaxScratchDevices, MOE_ERR_UNSUPPORTED,
              "moe_permute_fwd_noalloc: device %d is beyond the %d devices it keeps scratch for", dev,
              kMaxScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      (void)hipGetLastError();
      moe::set_error("moe_permute_fwd_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                     hipGetErrorString(e));
      return MOE_ERR_LAUNCH;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MOE_OK;
}

}  // namespace

extern "C" int moe_permute_fwd_noalloc(const void* hidden, int64_t T, int64_t H, const int64_t* ids, int64_t k,
                                       int64_t divisor, int64_t num_buckets, void* permuted, int32_t* perm,
                                       int32_t* pos_of_slot, int32_t* counts, int32_t* offsets, void* stream) {
  MOE_REQUIRE(T >= 0 && k >= 1 && k <= 16 && T * k < (1ll << 31) && num_buckets >= 1, MOE_ERR_INVALID,
              "moe_permute_fwd_noalloc: bad T=%lld k=%lld num_buckets=%lld", (long long)T, (long long)k,
              (long long)num_buckets);
  const size_t need = moe_permute_workspace_bytes(T * k, num_buckets);
  MOE_REQUIRE(need <= kScratchBytes, MOE_ERR_UNSUPPORTED,
              "moe_permute_fwd_noalloc: %lld routes over %lld buckets need %zu bytes of scratch, more than its "
              "fixed %zu; use moe_permute_fwd with a workspace",
              (long long)(T * k), (long long)num_buckets, need, kScratchBytes);
  void* ws = nullptr;
  const int rc = scratch_of_current_device(&ws);
  if (rc) return rc;
  // The count kernel stores every histogram entry that the scatter kernel
  // reads, so nothing in the scratch has to start at zero.
  return moe::permute_fwd_run(hidden, T, H, ids, k, divisor, num_buckets, permuted, perm, pos_of_slot, counts,
                              offsets, ws, kScratchBytes, stream);
}
