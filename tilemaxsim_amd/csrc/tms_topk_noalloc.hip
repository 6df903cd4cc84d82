// tms_topk_noalloc: the row-wise top-k of tms_topk with its intermediate keys in a fixed
// device array instead of a caller workspace. This translation unit holds the array and
// the entry point and no kernels (the levels run from tms_topk.hip's code object through
// topk_run), so the array sits in a code object of its own: under HIP's deferred module
// loading (the ROCm default) a GPU reserves it when tms_topk_noalloc first runs there,
// and callers of tms_topk alone never do.
#include <atomic>
#include <mutex>

#include "tms_common.h"
#include "tms_topk_host.h"

namespace tms {

// The tournament's intermediate keys (each GPU holds its own copy until the process
// ends). 32 MiB covers top-100 over (64, 1M) scores (12.9 MB) and (32, 5M) (32.0 MB).
constexpr int64_t kTopkScratchBytes = TMS_TOPK_SCRATCH_BYTES;
static __device__ __align__(256) uint64_t scratch[kTopkScratchBytes / 8];
constexpr int kMaxScratchDevices = 64;
static std::atomic<void*> g_scratch[kMaxScratchDevices];
static std::mutex g_scratch_mu;

// Device address of this GPU's copy of `scratch`, looked up once per device (with that
// device current) and cached; host code never passes the array's own name to a kernel.
static int scratch_address(const char* fn, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(TMS_ERR_HIP, "%s: hipGetDevice failed: %s", fn, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(TMS_ERR_UNSUPPORTED, "%s: device %d is beyond the %d devices the library tracks", fn, dev,
                kMaxScratchDevices);
  void* p = g_scratch[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || p == nullptr)
        return fail(TMS_ERR_HIP, "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", fn, dev,
                    hipGetErrorString(e));
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return TMS_OK;
}

}  // namespace tms

using namespace tms;

extern "C" int tms_topk_noalloc(const float* scores, int64_t nrows, int64_t n, int64_t k, float* out_values,
                                int64_t* out_indices, void* stream) {
  const char* fn = "tms_topk_noalloc";
  int rc = topk_checks(fn, scores, nrows, n, k, out_values, out_indices);
  if (rc != TMS_OK || nrows == 0 || k == 0) return rc;
  const int64_t need = topk_workspace_bytes(nrows, n, (int)k);
  if (need > kTopkScratchBytes)
    return fail(TMS_ERR_UNSUPPORTED,
                "%s: %lld rows of %lld scores at k=%lld need %lld bytes of scratch, above the library's fixed %lld "
                "(split the rows over several calls, or use tms_topk with a workspace)",
                fn, (long long)nrows, (long long)n, (long long)k, (long long)need, (long long)kTopkScratchBytes);
  void* ws = nullptr;
  if (need > 0) {
    rc = scratch_address(fn, &ws);
    if (rc != TMS_OK) return rc;
  }
  return topk_run(scores, nrows, n, k, ws, out_values, out_indices, (hipStream_t)stream);
}
