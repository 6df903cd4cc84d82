// Row-wise top-k: host entry points (tms_topk, tms_topk_workspace_size, tms_topk_noalloc);
// the selection kernel is in tms_topk_kernel.h.
#include <string.h>

#include <atomic>
#include <mutex>

#include "tms_topk_kernel.h"

namespace tms {

static int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Keys per row after each level, starting from n; stops when a row fits one chunk.
static int64_t level_sizes(int64_t n, int k, int64_t* sizes, int max_levels) {
  int64_t lv = 0;
  while (n > kChunk && lv < max_levels) {
    n = ceil_div(n, kChunk) * k;
    sizes[lv++] = n;
  }
  return lv;
}

static int64_t workspace_bytes(int64_t nrows, int64_t n, int k) {
  int64_t sizes[64];
  const int64_t lv = level_sizes(n, k, sizes, 64);
  int64_t a = 0, b = 0;  // ping-pong buffers: even levels in a, odd in b
  for (int64_t i = 0; i < lv; i++) {
    if (i % 2 == 0) a = sizes[i] > a ? sizes[i] : a;
    else b = sizes[i] > b ? sizes[i] : b;
  }
  return (a + b) * nrows * (int64_t)sizeof(uint64_t);
}

// Scratch of tms_topk_noalloc: the tournament's intermediate keys, in a fixed device array
// (each GPU the library runs on holds its own copy until the process ends). 32 MiB covers
// top-100 over (64, 1M) scores (12.9 MB) and (32, 5M) (32.0 MB).
constexpr int64_t kTopkScratchBytes = TMS_TOPK_SCRATCH_BYTES;
static __device__ __align__(256) uint64_t scratch[kTopkScratchBytes / 8];
constexpr int kMaxScratchDevices = 64;
static std::atomic<void*> g_scratch[kMaxScratchDevices];
static std::mutex g_scratch_mu;

static int topk_checks(const char* fn, const float* scores, int64_t nrows, int64_t n, int64_t k,
                       const float* out_values, const int64_t* out_indices);
static int topk_run(const float* scores, int64_t nrows, int64_t n, int64_t k, void* workspace, float* out_values,
                    int64_t* out_indices, hipStream_t st);
static int scratch_address(const char* fn, void** out);

}  // namespace tms

using namespace tms;

extern "C" {

int64_t tms_topk_workspace_size(int64_t nrows, int64_t n, int64_t k) {
  if (nrows <= 0 || n <= 0 || k <= 0 || k > kMaxK || k > n) return 0;
  return workspace_bytes(nrows, n, (int)k);
}

int tms_topk(const float* scores, int64_t nrows, int64_t n, int64_t k, void* workspace, int64_t workspace_bytes_,
             float* out_values, int64_t* out_indices, void* stream) {
  const char* fn = "tms_topk";
  int rc = topk_checks(fn, scores, nrows, n, k, out_values, out_indices);
  if (rc != TMS_OK || nrows == 0 || k == 0) return rc;
  const int64_t need = workspace_bytes(nrows, n, (int)k);
  if (need > 0 && (!workspace || workspace_bytes_ < need))
    return fail(TMS_ERR_INVALID, "%s: workspace of %lld bytes needed, got %lld", fn, (long long)need,
                (long long)workspace_bytes_);
  return topk_run(scores, nrows, n, k, workspace, out_values, out_indices, (hipStream_t)stream);
}

int tms_topk_noalloc(const float* scores, int64_t nrows, int64_t n, int64_t k, float* out_values,
                     int64_t* out_indices, void* stream) {
  const char* fn = "tms_topk_noalloc";
  int rc = topk_checks(fn, scores, nrows, n, k, out_values, out_indices);
  if (rc != TMS_OK || nrows == 0 || k == 0) return rc;
  const int64_t need = workspace_bytes(nrows, n, (int)k);
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

}  // extern "C"

namespace tms {

static int topk_checks(const char* fn, const float* scores, int64_t nrows, int64_t n, int64_t k,
                       const float* out_values, const int64_t* out_indices) {
  if (nrows < 0 || n < 0 || k < 0) return fail(TMS_ERR_INVALID, "%s: negative size", fn);
  if (k > n) return fail(TMS_ERR_INVALID, "%s: k=%lld exceeds the row length %lld", fn, (long long)k, (long long)n);
  if (k > kMaxK) return fail(TMS_ERR_UNSUPPORTED, "%s: k=%lld > %d is not supported", fn, (long long)k, kMaxK);
  if (n > 0xffffffffLL) return fail(TMS_ERR_UNSUPPORTED, "%s: rows longer than 2^32 - 1 are not supported", fn);
  if (nrows > 65535) return fail(TMS_ERR_UNSUPPORTED, "%s: more than 65535 rows per call", fn);
  if (nrows == 0 || k == 0) return TMS_OK;
  if (!scores || !out_values || !out_indices) return fail(TMS_ERR_INVALID, "%s: NULL pointer", fn);
  return TMS_OK;
}

// The levels of one call; `workspace` holds workspace_bytes(nrows, n, k) bytes.
static int topk_run(const float* scores, int64_t nrows, int64_t n, int64_t k, void* workspace, float* out_values,
                    int64_t* out_indices, hipStream_t st) {
  int64_t sizes[64];
  const int64_t lv = level_sizes(n, (int)k, sizes, 64);
  int64_t amax = 0;
  for (int64_t i = 0; i < lv; i += 2) amax = sizes[i] > amax ? sizes[i] : amax;
  uint64_t* bufs[2] = {(uint64_t*)workspace, (uint64_t*)workspace + amax * nrows};
  int64_t strides[2] = {amax, 0};
  for (int64_t i = 1; i < lv; i += 2) strides[1] = sizes[i] > strides[1] ? sizes[i] : strides[1];

  const dim3 last_block(kLastThreads), level_block(kLevelThreads);
  if (lv == 0) {
    if (n <= kShortRow)
      hipLaunchKernelGGL((topk_level_kernel<true, true, kShortThreads, kShortRow>), dim3(1, (unsigned)nrows),
                         dim3(kShortThreads), 0, st, scores, n, nullptr, n, n, nullptr, 0, out_values, out_indices,
                         (int)k);
    else
      hipLaunchKernelGGL((topk_level_kernel<true, true, kLastThreads>), dim3(1, (unsigned)nrows), last_block, 0, st,
                         scores, n, nullptr, n, n, nullptr, 0, out_values, out_indices, (int)k);
    return check_launch("topk_level_kernel");
  }
  // level 0: scores -> keys
  hipLaunchKernelGGL((topk_level_kernel<true, false, kLevelThreads>), dim3((unsigned)ceil_div(n, kChunk), (unsigned)nrows),
                     level_block, 0, st, scores, n, nullptr, n, n, bufs[0], strides[0], nullptr, nullptr, (int)k);
  int rc = check_launch("topk_level_kernel");
  if (rc) return rc;
  for (int64_t i = 1; i <= lv; i++) {
    const int64_t n_in = sizes[i - 1];
    const uint64_t* in = bufs[(i - 1) % 2];
    const int64_t in_stride = strides[(i - 1) % 2];
    if (i == lv && n_in <= kShortRow) {
      hipLaunchKernelGGL((topk_level_kernel<false, true, kShortThreads, kShortRow>), dim3(1, (unsigned)nrows),
                         dim3(kShortThreads), 0, st, scores, n, in, n_in, in_stride, nullptr, 0, out_values,
                         out_indices, (int)k);
    } else if (i == lv) {
      hipLaunchKernelGGL((topk_level_kernel<false, true, kLastThreads>), dim3(1, (unsigned)nrows), last_block, 0, st,
                         scores, n, in, n_in, in_stride, nullptr, 0, out_values, out_indices, (int)k);
    } else {
      hipLaunchKernelGGL((topk_level_kernel<false, false, kLevelThreads>),
                         dim3((unsigned)ceil_div(n_in, kChunk), (unsigned)nrows), level_block, 0, st, scores, n, in,
                         n_in, in_stride, bufs[i % 2], strides[i % 2], nullptr, nullptr, (int)k);
    }
    rc = check_launch("topk_level_kernel");
    if (rc) return rc;
  }
  return TMS_OK;
}

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
