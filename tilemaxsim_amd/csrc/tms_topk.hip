// Row-wise top-k of an fp32 score matrix (nrows, n) -> values (nrows, k) descending and
// int64 indices, the per-query top-100 the reference takes with torch.topk after scoring
// (src/cycle3_experiments.py:215).
//
// Each element becomes a 64-bit key: an order-preserving image of the float bits in the
// high word (NaN above +inf, as torch orders it) and the inverted index in the low word,
// so descending key order is "value descending, then index ascending" -- deterministic,
// and compared as integers (no float NaN semantics involved).
//
// Tournament: a workgroup sorts a chunk of kChunk keys in LDS (bitonic network) and keeps
// its best k; each level shrinks a row by kChunk / k until one chunk holds it, whose sorted
// head is the answer. Intermediate keys live in a caller-provided workspace.
#include <string.h>

#include "tms_common.h"

namespace tms {

constexpr int kChunk = 4096;  // keys sorted per workgroup (32 KiB of LDS)
constexpr int kTopkThreads = 256;
constexpr int kMaxK = kChunk / 4;

__device__ __forceinline__ uint32_t order_key(float f) {
  const uint32_t b = __builtin_bit_cast(uint32_t, f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key_value(uint32_t k) {
  const uint32_t b = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __builtin_bit_cast(float, b);
}

// FIRST: input is fp32 scores (row stride in_stride), indices are positions in the row.
// Otherwise input is keys. LAST: write (value, index) pairs; otherwise write the best k keys.
template <bool FIRST, bool LAST>
__global__ void __launch_bounds__(kTopkThreads) topk_level_kernel(const float* __restrict__ vals,
                                                                  const uint64_t* __restrict__ keys_in, int64_t n_in,
                                                                  int64_t in_stride, uint64_t* __restrict__ keys_out,
                                                                  int64_t out_stride, float* __restrict__ out_vals,
                                                                  int64_t* __restrict__ out_idx, int k) {
  __shared__ uint64_t s[kChunk];
  const int64_t row = blockIdx.y;
  const int64_t c0 = (int64_t)blockIdx.x * kChunk;
  for (int i = threadIdx.x; i < kChunk; i += kTopkThreads) {
    const int64_t p = c0 + i;
    uint64_t key = 0;  // below every real element
    if (p < n_in) {
      if constexpr (FIRST) {
        key = ((uint64_t)order_key(vals[row * in_stride + p]) << 32) | (uint64_t)(0xffffffffu - (uint32_t)p);
      } else {
        key = keys_in[row * in_stride + p];
      }
    }
    s[i] = key;
  }
  __syncthreads();
  // bitonic sort, descending
  for (int size = 2; size <= kChunk; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < kChunk / 2; i += kTopkThreads) {
        const int pos = 2 * i - (i & (stride - 1));
        const int partner = pos + stride;
        const bool desc = (pos & size) == 0;
        const uint64_t a = s[pos], b = s[partner];
        if ((a < b) == desc) {
          s[pos] = b;
          s[partner] = a;
        }
      }
      __syncthreads();
    }
  }
  for (int i = threadIdx.x; i < k; i += kTopkThreads) {
    const uint64_t key = s[i];
    if constexpr (LAST) {
      out_vals[row * k + i] = key_value((uint32_t)(key >> 32));
      out_idx[row * k + i] = (int64_t)(0xffffffffu - (uint32_t)key);
    } else {
      keys_out[row * out_stride + (int64_t)blockIdx.x * k + i] = key;
    }
  }
}

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
  if (nrows < 0 || n < 0 || k < 0) return fail(TMS_ERR_INVALID, "%s: negative size", fn);
  if (k > n) return fail(TMS_ERR_INVALID, "%s: k=%lld exceeds the row length %lld", fn, (long long)k, (long long)n);
  if (k > kMaxK) return fail(TMS_ERR_UNSUPPORTED, "%s: k=%lld > %d is not supported", fn, (long long)k, kMaxK);
  if (n > 0xffffffffLL) return fail(TMS_ERR_UNSUPPORTED, "%s: rows longer than 2^32 - 1 are not supported", fn);
  if (nrows > 65535) return fail(TMS_ERR_UNSUPPORTED, "%s: more than 65535 rows per call", fn);
  if (nrows == 0 || k == 0) return TMS_OK;
  if (!scores || !out_values || !out_indices) return fail(TMS_ERR_INVALID, "%s: NULL pointer", fn);
  const int64_t need = workspace_bytes(nrows, n, (int)k);
  if (need > 0 && (!workspace || workspace_bytes_ < need))
    return fail(TMS_ERR_INVALID, "%s: workspace of %lld bytes needed, got %lld", fn, (long long)need,
                (long long)workspace_bytes_);
  hipStream_t st = (hipStream_t)stream;
  int64_t sizes[64];
  const int64_t lv = level_sizes(n, (int)k, sizes, 64);
  int64_t amax = 0;
  for (int64_t i = 0; i < lv; i += 2) amax = sizes[i] > amax ? sizes[i] : amax;
  uint64_t* bufs[2] = {(uint64_t*)workspace, (uint64_t*)workspace + amax * nrows};
  int64_t strides[2] = {amax, 0};
  for (int64_t i = 1; i < lv; i += 2) strides[1] = sizes[i] > strides[1] ? sizes[i] : strides[1];

  const dim3 block(kTopkThreads);
  if (lv == 0) {
    hipLaunchKernelGGL((topk_level_kernel<true, true>), dim3(1, (unsigned)nrows), block, 0, st, scores, nullptr, n, n,
                       nullptr, 0, out_values, out_indices, (int)k);
    return check_launch("topk_level_kernel");
  }
  // level 0: scores -> keys
  hipLaunchKernelGGL((topk_level_kernel<true, false>), dim3((unsigned)ceil_div(n, kChunk), (unsigned)nrows), block, 0,
                     st, scores, nullptr, n, n, bufs[0], strides[0], nullptr, nullptr, (int)k);
  int rc = check_launch("topk_level_kernel");
  if (rc) return rc;
  for (int64_t i = 1; i <= lv; i++) {
    const int64_t n_in = sizes[i - 1];
    const uint64_t* in = bufs[(i - 1) % 2];
    const int64_t in_stride = strides[(i - 1) % 2];
    if (i == lv) {
      hipLaunchKernelGGL((topk_level_kernel<false, true>), dim3(1, (unsigned)nrows), block, 0, st, nullptr, in, n_in,
                         in_stride, nullptr, 0, out_values, out_indices, (int)k);
    } else {
      hipLaunchKernelGGL((topk_level_kernel<false, false>), dim3((unsigned)ceil_div(n_in, kChunk), (unsigned)nrows),
                         block, 0, st, nullptr, in, n_in, in_stride, bufs[i % 2], strides[i % 2], nullptr, nullptr,
                         (int)k);
    }
    rc = check_launch("topk_level_kernel");
    if (rc) return rc;
  }
  return TMS_OK;
}

}  // extern "C"
