// Row-wise top-k of an fp32 score matrix (nrows, n) -> values (nrows, k) descending and
// int64 indices, the per-query top-100 the reference takes with torch.topk after scoring
// (src/cycle3_experiments.py:215).
//
// Each element becomes a 64-bit key: an order-preserving image of the float bits in the
// high word (NaN above +inf, as torch orders it) and the inverted index in the low word,
// so descending key order is "value descending, then index ascending" -- deterministic,
// and compared as integers (no float NaN semantics involved).
//
// Tournament: a workgroup selects the best k of a chunk of kChunk keys and each level
// shrinks a row by kChunk / k until one chunk holds it; the last level sorts its k keys.
// Intermediate keys live in a caller-provided workspace. Selection is a radix select on
// the 64-bit keys held in registers (16 per thread): one 256-bin LDS histogram per 8-bit
// digit, from the top, narrowed to the keys that share the digits fixed so far, until
// the k-th largest key is known or a whole bin is needed (usually 3-4 passes).
#include <string.h>

#include <atomic>
#include <mutex>

#include "tms_common.h"

namespace tms {

constexpr int kChunk = 4096;  // keys sorted per workgroup (32 KiB of LDS)
constexpr int kTopkThreads = 256;
constexpr int kMaxK = kChunk / 4;

// Order-preserving image of a float's bits. -0.0 is taken as +0.0 (they compare equal,
// so they tie and go by index) and every NaN as the positive quiet NaN, so that a NaN
// with its sign bit set (x86's default NaN, or a negated one) still ranks above +inf.
__device__ __forceinline__ uint32_t order_key(float f) {
  uint32_t b = __builtin_bit_cast(uint32_t, f);
  b = (b == 0x80000000u) ? 0u : b;
  b = ((b & 0x7fffffffu) > 0x7f800000u) ? 0x7fc00000u : b;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// FIRST: input is fp32 scores (row stride in_stride), indices are positions in the row.
// Otherwise input is keys. LAST: write (value, index) pairs in descending order;
// otherwise write the best k keys of the chunk, in no particular order.
constexpr int kPerThread = kChunk / kTopkThreads;  // 16 keys per thread
static_assert(kTopkThreads == 256, "one histogram bin per thread; wave 0 scans four bins per lane");

// The values written by the LAST level are read back from the scores (vals, row stride
// val_stride) at the selected indices, so they keep the input's bits (-0.0, NaN payloads).
template <bool FIRST, bool LAST>
__global__ void __launch_bounds__(kTopkThreads) topk_level_kernel(const float* __restrict__ vals, int64_t val_stride,
                                                                  const uint64_t* __restrict__ keys_in, int64_t n_in,
                                                                  int64_t in_stride, uint64_t* __restrict__ keys_out,
                                                                  int64_t out_stride, float* __restrict__ out_vals,
                                                                  int64_t* __restrict__ out_idx, int k) {
  __shared__ uint32_t hist[256];
  __shared__ uint32_t pick[3];  // digit, keys above its bin, keys in its bin
  __shared__ uint32_t n_gt, n_eq;
  __shared__ uint64_t sel[LAST ? kMaxK : 1];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int64_t row = blockIdx.y;
  const int64_t c0 = (int64_t)blockIdx.x * kChunk;
  uint64_t key[kPerThread];
#pragma unroll
  for (int e = 0; e < kPerThread; e++) {
    const int64_t p = c0 + e * kTopkThreads + tid;
    key[e] = 0;  // below every real element
    if (p < n_in) {
      if constexpr (FIRST) {
        key[e] = ((uint64_t)order_key(vals[row * val_stride + p]) << 32) | (uint64_t)(0xffffffffu - (uint32_t)p);
      } else {
        key[e] = keys_in[row * in_stride + p];
      }
    }
  }

  // Radix select. After a pass, `prefix` holds the digits fixed so far and `need` the
  // number of keys still to take among the keys that share them.
  uint64_t prefix = 0;
  uint32_t need = (uint32_t)k;
  int shift = 64;
  bool whole_bin = false;  // the selection is every key >= prefix << shift
  while (shift > 0) {
    shift -= 8;
    hist[tid] = 0u;
    __syncthreads();
#pragma unroll
    for (int e = 0; e < kPerThread; e++)
      if (shift == 56 || (key[e] >> (shift + 8)) == prefix) atomicAdd(&hist[(uint32_t)(key[e] >> shift) & 255u], 1u);
    __syncthreads();
    if (wid == 0) {  // lane l scans bins 255 - 4l .. 252 - 4l, high to low
      uint32_t c[4];
#pragma unroll
      for (int j = 0; j < 4; j++) c[j] = hist[255 - 4 * lane - j];
      const uint32_t own = c[0] + c[1] + c[2] + c[3];
      uint32_t incl = own;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = __shfl_up(incl, o);
        if (lane >= o) incl += y;
      }
      const uint32_t excl = incl - own;
      if (excl < need && need <= incl) {  // exactly one lane: the need-th key is in its bins
        uint32_t above = excl;
        int j = 0;
        while (above + c[j] < need) above += c[j++];
        pick[0] = (uint32_t)(255 - 4 * lane - j);
        pick[1] = above;
        pick[2] = c[j];
      }
    }
    __syncthreads();
    const uint32_t d = pick[0], above = pick[1], cnt = pick[2];
    need -= above;
    prefix = (prefix << 8) | d;
    if (cnt == need && prefix != 0) {  // the whole bin is needed (keys are unique but padding)
      whole_bin = true;
      break;
    }
  }
  // Selection: every key > T, then `need` keys equal to T (only padding keys repeat).
  const uint64_t T = whole_bin ? (prefix << shift) - 1 : prefix;
  const uint32_t need_eq = whole_bin ? 0u : need;
  if (tid == 0) {
    n_gt = 0u;
    n_eq = 0u;
  }
  __syncthreads();
  auto put = [&](uint32_t pos, uint64_t kv) {
    if constexpr (LAST) sel[pos] = kv;
    else keys_out[row * out_stride + (int64_t)blockIdx.x * k + pos] = kv;
  };
#pragma unroll
  for (int e = 0; e < kPerThread; e++) {
    if (key[e] > T) {
      const uint32_t pos = atomicAdd(&n_gt, 1u);
      if (pos < (uint32_t)k - need_eq) put(pos, key[e]);  // always true; bounds every write
    } else if (key[e] == T && need_eq > 0u) {
      const uint32_t j = atomicAdd(&n_eq, 1u);
      if (j < need_eq) put((uint32_t)k - need_eq + j, key[e]);
    }
  }
  if constexpr (LAST) {
    int P = 1;  // bitonic sort of the k survivors, padded to a power of two
    while (P < k) P <<= 1;
    for (int i = k + tid; i < P; i += kTopkThreads) sel[i] = 0;
    __syncthreads();
    for (int size = 2; size <= P; size <<= 1) {
      for (int stride = size >> 1; stride > 0; stride >>= 1) {
        for (int i = tid; i < P / 2; i += kTopkThreads) {
          const int pos = 2 * i - (i & (stride - 1));
          const int partner = pos + stride;
          const bool desc = (pos & size) == 0;
          const uint64_t a = sel[pos], b = sel[partner];
          if ((a < b) == desc) {
            sel[pos] = b;
            sel[partner] = a;
          }
        }
        __syncthreads();
      }
    }
    for (int i = tid; i < k; i += kTopkThreads) {
      const int64_t idx = (int64_t)(0xffffffffu - (uint32_t)sel[i]);
      // a selected key is always a real element (k <= n); the clamp only bounds the read
      out_vals[row * k + i] = vals[row * val_stride + (idx < val_stride ? idx : val_stride - 1)];
      out_idx[row * k + i] = idx;
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

  const dim3 block(kTopkThreads);
  if (lv == 0) {
    hipLaunchKernelGGL((topk_level_kernel<true, true>), dim3(1, (unsigned)nrows), block, 0, st, scores, n, nullptr, n,
                       n, nullptr, 0, out_values, out_indices, (int)k);
    return check_launch("topk_level_kernel");
  }
  // level 0: scores -> keys
  hipLaunchKernelGGL((topk_level_kernel<true, false>), dim3((unsigned)ceil_div(n, kChunk), (unsigned)nrows), block, 0,
                     st, scores, n, nullptr, n, n, bufs[0], strides[0], nullptr, nullptr, (int)k);
  int rc = check_launch("topk_level_kernel");
  if (rc) return rc;
  for (int64_t i = 1; i <= lv; i++) {
    const int64_t n_in = sizes[i - 1];
    const uint64_t* in = bufs[(i - 1) % 2];
    const int64_t in_stride = strides[(i - 1) % 2];
    if (i == lv) {
      hipLaunchKernelGGL((topk_level_kernel<false, true>), dim3(1, (unsigned)nrows), block, 0, st, scores, n, in,
                         n_in, in_stride, nullptr, 0, out_values, out_indices, (int)k);
    } else {
      hipLaunchKernelGGL((topk_level_kernel<false, false>), dim3((unsigned)ceil_div(n_in, kChunk), (unsigned)nrows),
                         block, 0, st, scores, n, in, n_in, in_stride, bufs[i % 2], strides[i % 2], nullptr,
                         nullptr, (int)k);
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
