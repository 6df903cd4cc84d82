// Read-only streaming probe: the rate at which this part delivers a large buffer to a
// kernel that only reads it (no arithmetic and no writes beyond one word per lane). It
// is the ceiling the document-streaming kernels are measured against, and it runs from
// `bench.py --config readprobe`. Not part of the scoring path; no reference counterpart.
//
// Persistent grid (8 workgroups of 4 waves per CU) striding over 8 KiB chunks, each
// wave-iteration 8 independent 16-byte loads per lane (64 lanes x 16 B x 8 contiguous);
// the workgroups dispatched to one XCD (blockIdx % 8) take a contiguous range of block
// ids, which was the fastest of the mappings tried (contiguous runs per wave, grid-stride
// at 1x and 2x the resident grid, 4 / 8 / 16 KiB per iteration: 6.10-6.30 TB/s over a
// 46 GB buffer).
#include "tms_common.h"

namespace tms {

constexpr int kProbeDepth = 8;                          // 16-byte loads in flight per lane
constexpr int64_t kProbeChunk = 64 * 16 * kProbeDepth;  // bytes per wave-iteration
constexpr int kProbeGrid = 256 * 8;                     // workgroups (a multiple of 8)
static_assert((int64_t)kProbeGrid * 256 == TMS_READ_PROBE_SINK_WORDS, "one sink word per thread");

__global__ void __launch_bounds__(256) read_probe_kernel(const uint8_t* __restrict__ base, int64_t nchunks,
                                                         uint32_t* __restrict__ sink) {
  const int lane = threadIdx.x & 63;
  const int64_t nb = gridDim.x;
  const int64_t blk = (int64_t)(blockIdx.x % 8) * (nb / 8) + blockIdx.x / 8;
  const int64_t wave = blk * 4 + (threadIdx.x >> 6);
  const int64_t nwaves = nb * 4;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (int64_t c = wave; c < nchunks; c += nwaves) {
    const uint8_t* p = base + c * kProbeChunk + lane * 16;  // < (c + 1) * kProbeChunk
    u32x4 v[kProbeDepth];
#pragma unroll
    for (int j = 0; j < kProbeDepth; j++) v[j] = *(const u32x4*)(p + j * 1024);
#pragma unroll
    for (int j = 0; j < kProbeDepth; j++) acc ^= v[j];
  }
  sink[wave * 64 + lane] = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
}

}  // namespace tms

using namespace tms;

extern "C" int tms_read_probe(const void* buf, int64_t bytes, uint32_t* sink, int64_t sink_words, void* stream) {
  const char* fn = "tms_read_probe";
  if (bytes < 0 || bytes % kProbeChunk != 0)
    return fail(TMS_ERR_INVALID, "%s: bytes=%lld must be a non-negative multiple of %lld", fn, (long long)bytes,
                (long long)kProbeChunk);
  if (!sink || sink_words < TMS_READ_PROBE_SINK_WORDS)
    return fail(TMS_ERR_INVALID, "%s: the sink needs %d words", fn, TMS_READ_PROBE_SINK_WORDS);
  if (bytes > 0 && !buf) return fail(TMS_ERR_INVALID, "%s: buf is NULL", fn);
  hipLaunchKernelGGL(read_probe_kernel, dim3(kProbeGrid), dim3(256), 0, (hipStream_t)stream, (const uint8_t*)buf,
                     bytes / kProbeChunk, sink);
  return check_launch("read_probe_kernel");
}
