// Row-wise top-k: host entry points tms_topk and tms_topk_workspace_size, and the level
// launches that tms_topk_noalloc (tms_topk_noalloc.hip) shares; the selection kernel is in
// tms_topk_kernel.h.
#include <string.h>

#include "tms_topk_host.h"
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

int64_t topk_workspace_bytes(int64_t nrows, int64_t n, int k) {
  int64_t sizes[64];
  const int64_t lv = level_sizes(n, k, sizes, 64);
  int64_t a = 0, b = 0;  // ping-pong buffers: even levels in a, odd in b
  for (int64_t i = 0; i < lv; i++) {
    if (i % 2 == 0) a = sizes[i] > a ? sizes[i] : a;
    else b = sizes[i] > b ? sizes[i] : b;
  }
  return (a + b) * nrows * (int64_t)sizeof(uint64_t);
}

}  // namespace tms

using namespace tms;

extern "C" {

int64_t tms_topk_workspace_size(int64_t nrows, int64_t n, int64_t k) {
  if (nrows <= 0 || n <= 0 || k <= 0 || k > kMaxK || k > n) return 0;
  return topk_workspace_bytes(nrows, n, (int)k);
}

int tms_topk(const float* scores, int64_t nrows, int64_t n, int64_t k, void* workspace, int64_t workspace_bytes_,
             float* out_values, int64_t* out_indices, void* stream) {
  const char* fn = "tms_topk";
  int rc = topk_checks(fn, scores, nrows, n, k, out_values, out_indices);
  if (rc != TMS_OK || nrows == 0 || k == 0) return rc;
  const int64_t need = topk_workspace_bytes(nrows, n, (int)k);
  if (need > 0 && (!workspace || workspace_bytes_ < need))
    return fail(TMS_ERR_INVALID, "%s: workspace of %lld bytes needed, got %lld", fn, (long long)need,
                (long long)workspace_bytes_);
  return topk_run(scores, nrows, n, k, workspace, out_values, out_indices, (hipStream_t)stream);
}

}  // extern "C"

namespace tms {

int topk_checks(const char* fn, const float* scores, int64_t nrows, int64_t n, int64_t k, const float* out_values,
                const int64_t* out_indices) {
  if (nrows < 0 || n < 0 || k < 0) return fail(TMS_ERR_INVALID, "%s: negative size", fn);
  if (k > n) return fail(TMS_ERR_INVALID, "%s: k=%lld exceeds the row length %lld", fn, (long long)k, (long long)n);
  if (k > kMaxK) return fail(TMS_ERR_UNSUPPORTED, "%s: k=%lld > %d is not supported", fn, (long long)k, kMaxK);
  if (n > 0xffffffffLL) return fail(TMS_ERR_UNSUPPORTED, "%s: rows longer than 2^32 - 1 are not supported", fn);
  if (nrows > 65535) return fail(TMS_ERR_UNSUPPORTED, "%s: more than 65535 rows per call", fn);
  if (nrows == 0 || k == 0) return TMS_OK;
  if (!scores || !out_values || !out_indices) return fail(TMS_ERR_INVALID, "%s: NULL pointer", fn);
  return TMS_OK;
}

// The levels of one call; `workspace` holds topk_workspace_bytes(nrows, n, k) bytes.
int topk_run(const float* scores, int64_t nrows, int64_t n, int64_t k, void* workspace, float* out_values,
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

}  // namespace tms
