// Read-only streaming probe: the rate at which this part delivers a large buffer to a
// kernel that only reads it (no arithmetic and no writes beyond one word per lane). It
// is the ceiling the document-streaming kernels are measured against, and it runs from
// `bench.py --config readprobe`. Not part of the scoring path; no reference counterpart.
//
// Persistent grid (8 workgroups of 4 waves per CU) striding over 8 KiB chunks, each
// wave-iteration 8 independent 16-byte loads per lane (64 lanes x 16 B x 8 contiguous,
// non-temporal: each load covers whole 128-byte lines);
// the workgroups dispatched to one XCD (blockIdx % 8) take a contiguous range of block
// ids. With plain loads this was the fastest of the mappings tried (contiguous runs per
// wave, grid-stride at 1x and 2x the resident grid, 4 / 8 / 16 KiB per iteration:
// 6.10-6.30 TB/s over a 46 GB buffer); with non-temporal loads every such shape, and a
// one-shot grid of one chunk per wave, reads 6.9-7.1 TB/s.
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
    for (int j = 0; j < kProbeDepth; j++) v[j] = ld_stream<u32x4, true>(p + j * 1024);  // whole lines
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

// ---------------------------------------------------------------------------------
// LDS gather probe: the cost of one ds_read_b128 wave-instruction for a lane -> address
// pattern over a 128 KiB LDS buffer (one 16-wave workgroup per CU, every offset masked
// into the buffer), and patterns 0 to 3 again (4 to 7) at the PQ kernel's occupancy and
// footprint: two 8-wave workgroups per CU, each over its own 64 KiB buffer (a codebook's
// size). It backs the PQ kernel's floor: its codebook gathers are pattern 1 (5). Not
// part of the scoring path; no reference counterpart. A wave-instruction is served in
// four passes of 16 lanes, the lanes that share lane bit 5 and the parity of lane bits
// 2-4 (patterns 10 and 11 tell this apart from passes of 16 consecutive lanes); a pass
// costs the largest number of distinct rows it puts on one 16-byte bank group.
//   0: lane l -> bank group l % 16, random 256-byte rows: conflict-free;
//   1: the PQ gather: the 16 lanes of an MFMA lane group read random 16-byte rows of one
//      4 KiB subspace block (bank group = row % 16, random);
//   2: the 16 lanes of a lane group all read one bank group at random rows;
//   3: lane l -> bank group (l / 4) % 16 at random rows: every bank group gets exactly
//      four lanes of the wave, and four lanes of every pass share one;
//   10: lane l -> bank group l % 8 + 8 * (bit 4 of l): conflict-free by the pass rule,
//       two lanes per bank group in every pass of 16 consecutive lanes;
//   11: lane l -> bank group l % 8 + 8 * (parity of bits 2-4 of l): two lanes per bank
//       group in every pass by the rule, conflict-free in passes of 16 consecutive lanes.
// Patterns 8 and 9 run patterns 1 and 0 at the PQ kernel's shape with the PQ kernel's
// matrix work beside the gathers (two MFMAs per gathered fragment, random fp16 data):
// the gather rate this part holds under that mix, with no HBM traffic.
namespace tms {

constexpr int kLdsProbeUnits = 8192;  // 16-byte units (128 KiB)
constexpr int kLdsProbeOffs = 16;     // offsets per lane, cycled
constexpr int kLdsProbeIters = 4096;

__device__ __forceinline__ uint32_t probe_hash(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

// fp16 bits of a value in +-[0.5, 1) with random sign and mantissa, two per word
__device__ __forceinline__ uint32_t probe_halves(uint32_t h) {
  return (h & 0x83ff83ffu) | 0x38003800u;
}

// NT threads a workgroup over UNITS 16-byte units of LDS; waves are numbered across the
// grid (blockIdx.x * NT / 64 + wave), so every launch shape has TMS_LDS_PROBE_WAVES waves.
// MIX: the LDS holds random fp16 values, and every gathered fragment feeds two
// v_mfma_f32_16x16x32_f16 against random fp16 fragments held in registers (the PQ
// kernel's 64 MFMAs per 32 gathers, on data of the same kind), eight accumulators per wave.
template <int NT, int UNITS, bool MIX>
__global__ void __launch_bounds__(NT) lds_probe_kernel(int pattern, int64_t* __restrict__ cycles,
                                                       uint32_t* __restrict__ sink) {
  extern __shared__ u32x4 probe_lds[];
  for (int i = threadIdx.x; i < UNITS; i += NT) {
    if constexpr (MIX)
      probe_lds[i] = u32x4{probe_halves(probe_hash(4u * i)), probe_halves(probe_hash(4u * i + 1u)),
                           probe_halves(probe_hash(4u * i + 2u)), probe_halves(probe_hash(4u * i + 3u))};
    else
      probe_lds[i] = u32x4{(uint32_t)i, 1u, 2u, 3u};
  }
  constexpr int kWaves = NT / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int gw = blockIdx.x * kWaves + wave;  // < TMS_LDS_PROBE_WAVES
  uint32_t o[kLdsProbeOffs];
#pragma unroll
  for (int j = 0; j < kLdsProbeOffs; j++) {
    const uint32_t h = probe_hash((uint32_t)((gw * 64 + lane) * kLdsProbeOffs + j));
    uint32_t u;
    if (pattern == 0) u = (h % 512u) * 16u + (uint32_t)(lane & 15);
    else if (pattern == 1) u = (uint32_t)((j + 4 * (lane >> 4)) & 15) * 256u + (h % 256u);
    else if (pattern == 2) u = (h % 512u) * 16u + (uint32_t)(lane >> 4);
    else if (pattern == 3) u = (h % 512u) * 16u + (uint32_t)((lane >> 2) & 15);
    else if (pattern == 4) u = (h % 512u) * 16u + (uint32_t)((lane & 7) + 8 * ((lane >> 4) & 1));
    else u = (h % 512u) * 16u + (uint32_t)((lane & 7) + 8 * (((lane >> 2) ^ (lane >> 3) ^ (lane >> 4)) & 1));
    o[j] = u & (UNITS - 1);
  }
  __syncthreads();
  u32x4 acc = {0u, 0u, 0u, 0u};
  f32x4 macc[MIX ? 8 : 1];
  u32x4 qb[MIX ? 2 : 1];
  if constexpr (MIX) {
#pragma unroll
    for (int i = 0; i < 8; i++) macc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const uint32_t s0 = (uint32_t)(gw * 64 + lane) * 8u + 4u * h;
      qb[h] = u32x4{probe_halves(probe_hash(s0)), probe_halves(probe_hash(s0 + 1u)), probe_halves(probe_hash(s0 + 2u)),
                    probe_halves(probe_hash(s0 + 3u))};
    }
  }
  const uint64_t t0 = __builtin_readcyclecounter();
  for (int it = 0; it < kLdsProbeIters; it++) {
#pragma unroll
    for (int j = 0; j < kLdsProbeOffs; j++) {
      if constexpr (MIX) {
        const u32x4 f = probe_lds[o[j]];
        macc[2 * (j & 3)] = mfma16x16x32<TMS_DTYPE_F16>(f, qb[0], macc[2 * (j & 3)]);
        macc[2 * (j & 3) + 1] = mfma16x16x32<TMS_DTYPE_F16>(f, qb[1], macc[2 * (j & 3) + 1]);
      } else {
        acc ^= probe_lds[o[j]];
      }
    }
#pragma unroll
    for (int j = 0; j < kLdsProbeOffs; j++) asm volatile("" : "+v"(o[j]));  // keeps the loads in the loop
  }
  const uint64_t t1 = __builtin_readcyclecounter();
  if (lane == 0) cycles[gw] = (int64_t)(t1 - t0);
  if constexpr (MIX) {
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) sum += macc[i][0] + macc[i][1] + macc[i][2] + macc[i][3];
    acc[0] = __builtin_bit_cast(uint32_t, sum);
  }
  sink[gw * 64 + lane] = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
}

}  // namespace tms

extern "C" int tms_lds_probe(int pattern, int64_t* cycles, int64_t cycle_words, uint32_t* sink, int64_t sink_words,
                             void* stream) {
  const char* fn = "tms_lds_probe";
  if (pattern < 0 || pattern > 11) return fail(TMS_ERR_INVALID, "%s: pattern=%d must be 0 to 11", fn, pattern);
  if (!cycles || cycle_words < TMS_LDS_PROBE_WAVES)
    return fail(TMS_ERR_INVALID, "%s: cycles needs %d words", fn, TMS_LDS_PROBE_WAVES);
  if (!sink || sink_words < TMS_LDS_PROBE_WAVES * 64)
    return fail(TMS_ERR_INVALID, "%s: the sink needs %d words", fn, TMS_LDS_PROBE_WAVES * 64);
  if (pattern < 4 || pattern >= 10)  // one 16-wave workgroup per CU over 128 KiB
    hipLaunchKernelGGL((lds_probe_kernel<1024, kLdsProbeUnits, false>), dim3(TMS_LDS_PROBE_WAVES / 16), dim3(1024),
                       kLdsProbeUnits * 16, (hipStream_t)stream, pattern < 4 ? pattern : pattern - 6, cycles, sink);
  else if (pattern < 8)  // the PQ kernel's shape: two 8-wave workgroups per CU, 64 KiB each
    hipLaunchKernelGGL((lds_probe_kernel<512, kLdsProbeUnits / 2, false>), dim3(TMS_LDS_PROBE_WAVES / 8), dim3(512),
                       kLdsProbeUnits * 8, (hipStream_t)stream, pattern - 4, cycles, sink);
  else  // 8: the PQ gather (1), 9: conflict-free (0), each with two MFMAs per gathered fragment
    hipLaunchKernelGGL((lds_probe_kernel<512, kLdsProbeUnits / 2, true>), dim3(TMS_LDS_PROBE_WAVES / 8), dim3(512),
                       kLdsProbeUnits * 8, (hipStream_t)stream, pattern == 8 ? 1 : 0, cycles, sink);
  return check_launch("lds_probe_kernel");
}

// ---------------------------------------------------------------------------------
// MFMA probe: the sustained rate of v_mfma_f32_16x16x32_f16 with operands in registers
// and nothing else to do, on the operand values the caller passes (random fp16 in
// `bench.py --config mfmaprobe`: the switching activity of real data sets the clock this
// part holds). Two 4-wave workgroups per CU (2 waves per SIMD, as the shared-tile
// kernels run), eight independent accumulators per wave. It is the practical MFMA
// ceiling the batched kernels are read against. Not part of the scoring path; no
// reference counterpart.
namespace tms {

constexpr int kMfmaProbeIters = 20000;

__global__ void __launch_bounds__(256) mfma_probe_kernel(const u32x4* __restrict__ ops, float* __restrict__ sink) {
  const u32x4 a = ops[threadIdx.x], b = ops[256 + threadIdx.x];
  f32x4 acc[8];
#pragma unroll
  for (int i = 0; i < 8; i++) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < kMfmaProbeIters; it++) {
#pragma unroll
    for (int i = 0; i < 8; i++) acc[i] = mfma16x16x32<TMS_DTYPE_F16>(a, b, acc[i]);
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 8; i++) s += acc[i][0] + acc[i][1] + acc[i][2] + acc[i][3];
  sink[blockIdx.x * 256 + threadIdx.x] = s;
}

}  // namespace tms

extern "C" int tms_mfma_probe(const void* ops, float* sink, int64_t sink_words, int64_t* flops, void* stream) {
  const char* fn = "tms_mfma_probe";
  const int grid = 256 * 2;
  if (!ops || !sink || !flops) return fail(TMS_ERR_INVALID, "%s: NULL pointer", fn);
  if (sink_words < (int64_t)grid * 256) return fail(TMS_ERR_INVALID, "%s: the sink needs %d words", fn, grid * 256);
  *flops = (int64_t)grid * 4 * kMfmaProbeIters * 8 * (16 * 16 * 32 * 2);
  hipLaunchKernelGGL(mfma_probe_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, (const u32x4*)ops, sink);
  return check_launch("mfma_probe_kernel");
}
