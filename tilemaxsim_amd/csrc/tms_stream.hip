// Fixed-length dense MaxSim, d <= 128, query fragments in VGPRs: the streaming kernel
// with a control-flow shape the compiler's memory-counter tracking follows exactly.
//
// The general kernel (tms_dense.hip) walks documents with a cursor whose branches make
// the compiler drain every outstanding load before each tile. Here:
//  * documents are fixed length, so a wave's tiles are a flat sequence; each document
//    is padded to a multiple of R = PFD + 1 tiles with clamped duplicates of its last
//    token (a duplicate cannot change a max), so every document starts at ring slot 0;
//  * the inner loop body is straight-line and unrolled R times: it issues the loads of
//    tile g + PFD (index clamped to the last tile, so the count never varies) and scores
//    tile g from the ring; the per-document reduction sits between inner loops;
//  * scores are staged in registers (lane i holds document i of the wave's run) and
//    stored once, coalesced, after the loop.
// Every wave streams its own documents with the same (one or two) query blocks. Batched
// queries use batched_maxsim_kernel below, whose workgroups share tiles through LDS.
//
// Semantics as tms_dense.hip: fp32 accumulation, query rows past nq contribute 0, an
// empty document scores -inf.
#include "tms_common.h"

namespace tms {

struct StreamArgs {
  const uint8_t* Q;  // (nQ * nq, d)
  const uint8_t* D;  // (B, nd, d)
  float* out;        // (nQ, B)
  int64_t B, nd;
  int32_t nq, nbq;   // tokens per query, 32-token blocks per query
  int32_t blk0;      // first global query block of this launch
  int32_t blk_end;   // one past the last block of this launch
  int32_t nblk;      // blocks per wave
  int32_t d;         // 32 * KS
  int32_t docs_per_wave;  // documents per wave (per workgroup in the batched kernel); <= 64
};

template <int DT, int KS, int NB, int PFD>
__global__ void __launch_bounds__(256, 1) stream_maxsim_kernel(StreamArgs a) {
  constexpr int R = PFD + 1;
  const int lane = threadIdx.x & 63;
  const int r = lane & 15, g = lane >> 4;
  const int wid = threadIdx.x >> 6;
  const float NEG_INF = -__builtin_inff();

  const int my_blk0 = a.blk0;
  int my_nblk = a.blk_end - my_blk0;
  if (my_nblk > a.nblk) my_nblk = a.nblk;
  if (my_nblk <= 0) return;

  const int64_t unit = (int64_t)blockIdx.x * 4 + wid;
  const int64_t b_begin = unit * a.docs_per_wave;
  if (b_begin >= a.B) return;
  const int64_t b_end = (b_begin + a.docs_per_wave < a.B) ? b_begin + a.docs_per_wave : a.B;
  const int64_t ndocs = b_end - b_begin;

  // query fragments: block j, half h, step s -> token 16h + r of the block, chunk 4s + g
  auto q_valid = [&](int j, int h, int64_t& row) -> bool {
    const int jb = my_blk0 + j;
    const int qi = jb / a.nbq;
    const int tok = (jb - qi * a.nbq) * 32 + 16 * h + r;
    row = (int64_t)qi * a.nq + tok;
    return j < my_nblk && tok < a.nq;
  };
  u32x4 qf[NB][KS][2];
#pragma unroll
  for (int j = 0; j < NB; j++)
#pragma unroll
    for (int h = 0; h < 2; h++) {
      int64_t row;
      const bool v = q_valid(j, h, row);
#pragma unroll
      for (int s = 0; s < KS; s++)
        qf[j][s][h] = v ? *(const u32x4*)(a.Q + (row * a.d + 8 * (4 * s + g)) * 2) : u32x4{0u, 0u, 0u, 0u};
    }

  float pend[NB];
#pragma unroll
  for (int j = 0; j < NB; j++) pend[j] = NEG_INF;

  if (a.nd > 0) {
    const int64_t tiles = (a.nd + 15) / 16;
    const int64_t tpd = (tiles + R - 1) / R * R;  // tiles per document, padded to a multiple of R
    const int64_t total = ndocs * tpd;
    const int64_t row_bytes = (int64_t)a.d * 2;
    const uint8_t* base = a.D + b_begin * a.nd * row_bytes + (int64_t)(8 * g) * 2;

    // Address of this lane's token row for tile (doc offset dd, tile t).
    auto tile_ptr = [&](int64_t dd, int64_t t) -> const uint8_t* {
      int64_t tok = t * 16 + r;
      if (tok > a.nd - 1) tok = a.nd - 1;
      return base + (dd * a.nd + tok) * row_bytes;
    };
    // Prefetch cursor: tile index pf = pd * tpd + pt, saturating at the last tile (the
    // prefetches past the end re-read it, L1-resident, so each iteration issues KS loads).
    int64_t pd = 0, pt = 0, pf = 0;
    auto pf_next = [&]() {
      const bool more = pf < total - 1;
      pf += more ? 1 : 0;
      pt += more ? 1 : 0;
      const bool wrap = pt == tpd;
      pt = wrap ? 0 : pt;
      pd += wrap ? 1 : 0;
    };

    u32x4 ring[R][KS];
    auto load = [&](u32x4 (&buf)[KS]) {
      const uint8_t* p = tile_ptr(pd, pt);
#pragma unroll
      for (int s = 0; s < KS; s++) buf[s] = *(const u32x4*)(p + 64 * s);
    };
#pragma unroll
    for (int k = 0; k < PFD; k++) {
      load(ring[k]);
      pf_next();
    }

    float rmax[NB][2];
    auto score = [&](const u32x4 (&buf)[KS]) {
      f32x4 acc[NB][2];
#pragma unroll
      for (int j = 0; j < NB; j++) acc[j][0] = acc[j][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; s++)
#pragma unroll
        for (int j = 0; j < NB; j++)
#pragma unroll
          for (int h = 0; h < 2; h++) acc[j][h] = mfma16x16x32<DT>(buf[s], qf[j][s][h], acc[j][h]);
#pragma unroll
      for (int j = 0; j < NB; j++)
#pragma unroll
        for (int h = 0; h < 2; h++)
          rmax[j][h] = fmaxf(rmax[j][h], fmaxf(fmaxf(acc[j][h][0], acc[j][h][1]), fmaxf(acc[j][h][2], acc[j][h][3])));
    };

    for (int64_t dd = 0; dd < ndocs; dd++) {
#pragma unroll
      for (int j = 0; j < NB; j++) rmax[j][0] = rmax[j][1] = NEG_INF;
      for (int64_t t = 0; t < tpd; t += R) {
#pragma unroll
        for (int k = 0; k < R; k++) {
          load(ring[(k + PFD) % R]);
          pf_next();
          score(ring[k]);
        }
      }
      // document done: max over the 64 rows of each column, sum over query tokens
      float blk[NB];
#pragma unroll
      for (int j = 0; j < NB; j++) {
        float s = 0.f;
#pragma unroll
        for (int h = 0; h < 2; h++) {
          float m = rmax[j][h];
          m = fmaxf(m, __shfl_xor(m, 16));
          m = fmaxf(m, __shfl_xor(m, 32));
          int64_t row;
          s += q_valid(j, h, row) ? m : 0.f;
        }
        s += __shfl_xor(s, 8);
        s += __shfl_xor(s, 4);
        s += __shfl_xor(s, 2);
        s += __shfl_xor(s, 1);
        blk[j] = s;
      }
      const bool mine = lane == (int)dd;
#pragma unroll
      for (int j = 0; j < NB; j++) pend[j] = mine ? blk[j] : pend[j];
    }
  }

  // coalesced store: lane i writes document b_begin + i, per query (blocks of one query
  // summed in order; a query that began in an earlier launch accumulates)
  if (lane < ndocs) {
    const int64_t b = b_begin + lane;
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < NB; j++) {
      if (j >= my_nblk) break;
      const int jb = my_blk0 + j;
      const int qi = jb / a.nbq;
      s += pend[j];
      if (j == my_nblk - 1 || (jb + 1) / a.nbq != qi) {
        float* o = a.out + (int64_t)qi * a.B + b;
        *o = (qi * a.nbq < my_blk0) ? *o + s : s;
        s = 0.f;
      }
    }
  }
}

template <int K>
struct RingSlotS {
  static constexpr int value = K;
};

// Batched queries, tiles shared through LDS. The eight waves of a workgroup (one per CU,
// two per SIMD) stream the same documents; wave w holds a.nblk query blocks (whole
// queries) in VGPRs, so one pass over D serves up to 8 * a.nblk blocks. Each 16-token
// tile is loaded from memory once per workgroup: wave w < KS loads k-step w (lane
// (r, g): chunk 4 w + g of token r, the MFMA A-operand layout) and stores it to a
// three-slot LDS ring; after a barrier every wave reads the tile's KS k-steps from LDS.
// A loading wave keeps one 16-byte load per lane in flight per tile, PFD tiles ahead.
// The barriers fence LDS only, so they never wait for the loads in flight. The MFMA
// cluster of each tile runs at raised wave priority, so a wave that has its operands
// keeps the matrix pipe fed ahead of the other wave's bookkeeping.
template <int DT, int KS, int NB, int PFD>
__global__ void __launch_bounds__(512, 1) batched_maxsim_kernel(StreamArgs a) {
  static_assert(PFD >= 2, "tile i+1 is stored to LDS after tile i+PFD's load is issued");
  static_assert(PFD <= 6 && PFD % 2 == 0, "the step loop is unrolled PFD (even, <= 6) times");
  constexpr int NS = 3;  // LDS ring slots (two would do: a slot is rewritten only after a barrier that follows its last read)
  __shared__ u32x4 ring[NS][4][64];
  const int lane = threadIdx.x & 63;
  const int r = lane & 15, g = lane >> 4;
  const int wid = threadIdx.x >> 6;
  const float NEG_INF = -__builtin_inff();

  // A wave with no query block still loads its share of every tile.
  const int my_blk0 = a.blk0 + wid * a.nblk;
  int my_nblk = a.blk_end - my_blk0;
  if (my_nblk > a.nblk) my_nblk = a.nblk;

  const int64_t b_begin = (int64_t)blockIdx.x * a.docs_per_wave;
  if (b_begin >= a.B) return;  // whole workgroup
  const int64_t b_end = (b_begin + a.docs_per_wave < a.B) ? b_begin + a.docs_per_wave : a.B;
  const int64_t ndocs = b_end - b_begin;

  auto q_valid = [&](int j, int h, int64_t& row) -> bool {
    const int jb = my_blk0 + j;
    const int qi = jb / a.nbq;
    const int tok = (jb - qi * a.nbq) * 32 + 16 * h + r;
    row = (int64_t)qi * a.nq + tok;
    return j < my_nblk && tok < a.nq;
  };
  u32x4 qf[NB][KS][2];
#pragma unroll
  for (int j = 0; j < NB; j++)
#pragma unroll
    for (int h = 0; h < 2; h++) {
      int64_t row;
      const bool v = q_valid(j, h, row);
#pragma unroll
      for (int s = 0; s < KS; s++)
        qf[j][s][h] = v ? *(const u32x4*)(a.Q + (row * a.d + 8 * (4 * s + g)) * 2) : u32x4{0u, 0u, 0u, 0u};
    }

  bool qv[NB][2];  // query row 16 h + r of block j exists
#pragma unroll
  for (int j = 0; j < NB; j++)
#pragma unroll
    for (int h = 0; h < 2; h++) {
      int64_t row;
      qv[j][h] = q_valid(j, h, row);
    }
  float pend[NB];
#pragma unroll
  for (int j = 0; j < NB; j++) pend[j] = NEG_INF;

  if (a.nd > 0) {
    const int64_t tpd = (a.nd + 15) / 16;  // tiles per document
    const int64_t total = ndocs * tpd;
    const int64_t row_bytes = (int64_t)a.d * 2;
    const bool loader = wid < KS;          // d < 128 has fewer k-steps than waves
    const int ks = loader ? wid : 0;
    const uint8_t* base = a.D + b_begin * a.nd * row_bytes + (int64_t)(4 * ks + g) * 16;

    // load cursor (tile pd * tpd + pt), saturating at the last tile
    int64_t pd = 0, pt = 0, pf = 0;
    auto load_next = [&]() -> u32x4 {
      int64_t tok = pt * 16 + r;
      if (tok > a.nd - 1) tok = a.nd - 1;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (loader) v = *(const u32x4*)(base + (pd * a.nd + tok) * row_bytes);
      const bool more = pf < total - 1;
      pf += more ? 1 : 0;
      pt += more ? 1 : 0;
      const bool wrap = pt == tpd;
      pt = wrap ? 0 : pt;
      pd += wrap ? 1 : 0;
      return v;
    };

    u32x4 stg[PFD];
#pragma unroll
    for (int k = 0; k < PFD; k++) stg[k] = load_next();
    if (loader) ring[0][ks][lane] = stg[0];
    auto sync = [&]() {  // LDS-only fence: the loads in flight are not waited for
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    };
    // Fragments of the tile being scored and of the next one: after the barrier of step i
    // the tile i+1 fragments are read, and tile i's MFMAs hide that LDS latency.
    u32x4 frag[2][KS];
    sync();
#pragma unroll
    for (int s = 0; s < KS; s++) frag[0][s] = ring[0][s][lane];

    float rmax[NB][2];
#pragma unroll
    for (int j = 0; j < NB; j++) rmax[j][0] = rmax[j][1] = NEG_INF;
    int64_t i = 0, cd = 0, ct = 0;  // tile being scored: document cd, tile ct
    auto step = [&](auto slot) -> bool {
      constexpr int k = decltype(slot)::value;  // tile i's load was stg[k]
      constexpr int f = k & 1;                   // tile i's fragments are frag[f] (PFD is even)
      stg[k] = load_next();                      // tile i + PFD
      if (loader && i + 1 < total) ring[(i + 1) % NS][ks][lane] = stg[(k + 1) % PFD];
      sync();
#pragma unroll
      for (int s = 0; s < KS; s++) frag[f ^ 1][s] = ring[(i + 1) % NS][s][lane];  // tile i+1 (unused past the end)
      const u32x4(&t)[KS] = frag[f];
      f32x4 acc[NB][2];
#pragma unroll
      for (int j = 0; j < NB; j++) acc[j][0] = acc[j][1] = f32x4{0.f, 0.f, 0.f, 0.f};
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int s = 0; s < KS; s++)
#pragma unroll
        for (int j = 0; j < NB; j++)
#pragma unroll
          for (int h = 0; h < 2; h++) acc[j][h] = mfma16x16x32<DT>(t[s], qf[j][s][h], acc[j][h]);
      __builtin_amdgcn_s_setprio(0);
#pragma unroll
      for (int j = 0; j < NB; j++)
#pragma unroll
        for (int h = 0; h < 2; h++)  // two v_max3 per fragment
          rmax[j][h] = fmaxf(fmaxf(fmaxf(fmaxf(rmax[j][h], acc[j][h][0]), acc[j][h][1]), acc[j][h][2]), acc[j][h][3]);
      if (++ct == tpd) {  // document cd done: max over rows, sum over query tokens
#pragma unroll
        for (int j = 0; j < NB; j++) {
          float s = (qv[j][0] ? cross_row_max(rmax[j][0]) : 0.f) + (qv[j][1] ? cross_row_max(rmax[j][1]) : 0.f);
          rmax[j][0] = rmax[j][1] = NEG_INF;
          s = row_sum16(s);
          pend[j] = lane == (int)cd ? s : pend[j];
        }
        ct = 0;
        cd++;
      }
      return ++i == total;
    };
    bool done = false;
    while (!done) {
      done = step(RingSlotS<0>{});
      if (!done && PFD > 1) done = step(RingSlotS<1 % PFD>{});
      if (!done && PFD > 2) done = step(RingSlotS<2 % PFD>{});
      if (!done && PFD > 3) done = step(RingSlotS<3 % PFD>{});
      if (!done && PFD > 4) done = step(RingSlotS<4 % PFD>{});
      if (!done && PFD > 5) done = step(RingSlotS<5 % PFD>{});
    }
  }

  if (my_nblk <= 0) return;
  // coalesced store: lane i writes document b_begin + i, per query (blocks of one query
  // summed in order; a query that began in an earlier launch accumulates)
  if (lane < ndocs) {
    const int64_t b = b_begin + lane;
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < NB; j++) {
      if (j >= my_nblk) break;
      const int jb = my_blk0 + j;
      const int qi = jb / a.nbq;
      s += pend[j];
      if (j == my_nblk - 1 || (jb + 1) / a.nbq != qi) {
        float* o = a.out + (int64_t)qi * a.B + b;
        *o = (qi * a.nbq < my_blk0) ? *o + s : s;
        s = 0.f;
      }
    }
  }
}

#ifndef TMS_STREAM_PFD
#define TMS_STREAM_PFD 2  // tiles in flight ahead of the one being scored (single-query path)
#endif
#ifndef TMS_STREAM_TOKENS_PER_WAVE
#define TMS_STREAM_TOKENS_PER_WAVE 192
#endif

template <int DT, int KS, int NB>
static int stream_launch(const StreamArgs& a, int64_t grid, hipStream_t st) {
  hipLaunchKernelGGL((stream_maxsim_kernel<DT, KS, NB, TMS_STREAM_PFD>), dim3((unsigned)grid), dim3(256), 0, st, a);
  return check_launch("stream_maxsim_kernel");
}

#ifndef TMS_BATCHED_PFD
#define TMS_BATCHED_PFD 4  // tiles in flight per workgroup in the batched kernel
#endif
#define TMS_BATCHED_WAVES 8
template <int DT, int KS, int NB>
static int batched_launch(const StreamArgs& a, int64_t grid, hipStream_t st) {
  hipLaunchKernelGGL((batched_maxsim_kernel<DT, KS, NB, TMS_BATCHED_PFD>), dim3((unsigned)grid), dim3(64 * TMS_BATCHED_WAVES), 0,
                     st, a);
  return check_launch("batched_maxsim_kernel");
}
template <int DT, int NB>
static int batched_ks(const StreamArgs& a, int64_t grid, hipStream_t st) {
  switch (a.d / 32) {
    case 1: return batched_launch<DT, 1, NB>(a, grid, st);
    case 2: return batched_launch<DT, 2, NB>(a, grid, st);
    case 3: return batched_launch<DT, 3, NB>(a, grid, st);
    default: return batched_launch<DT, 4, NB>(a, grid, st);
  }
}
// Query blocks held in VGPRs per wave in the batched-query path: 1, 2 or kMaxBlocksPerWave.
constexpr int kMaxBlocksPerWave = 4;
template <int DT>
static int batched_nb(int nb, const StreamArgs& a, int64_t grid, hipStream_t st) {
  switch (nb) {
    case 1: return batched_ks<DT, 1>(a, grid, st);
    case 2: return batched_ks<DT, 2>(a, grid, st);
    default: return batched_ks<DT, kMaxBlocksPerWave>(a, grid, st);
  }
}

template <int DT, int NB>
static int stream_ks(const StreamArgs& a, int64_t grid, hipStream_t st) {
  switch (a.d / 32) {
    case 1: return stream_launch<DT, 1, NB>(a, grid, st);
    case 2: return stream_launch<DT, 2, NB>(a, grid, st);
    case 3: return stream_launch<DT, 3, NB>(a, grid, st);
    default: return stream_launch<DT, 4, NB>(a, grid, st);
  }
}

// Entry used by tms_dense.hip for fixed-length documents with d in {32, 64, 96, 128},
// 16-byte aligned Q and D. nQ queries of nq tokens; out is (nQ, B).
int run_stream(const void* Q, int64_t nQ, int64_t nq, int64_t d, const void* D, int64_t B, int64_t nd, int dtype,
               float* out, hipStream_t st) {
  StreamArgs a;
  a.Q = (const uint8_t*)Q;
  a.D = (const uint8_t*)D;
  a.out = out;
  a.B = B;
  a.nd = nd;
  a.nq = (int32_t)nq;
  a.nbq = (int32_t)((nq + 31) / 32);
  a.d = (int32_t)d;
  const int64_t nblocks = nQ * (int64_t)a.nbq;
  const bool split = a.nbq <= kMaxBlocksPerWave && nblocks >= 4;
  if (split) {
    // Blocks per wave: the smallest of 1, 2, 4 whose launch covers every block in one
    // pass (a wave computes all of its slots, used or not), else 4. A wave holds whole
    // queries, so a query's blocks never span waves or launches.
    int nb = kMaxBlocksPerWave;
    for (int c = 1; c < kMaxBlocksPerWave; c *= 2)
      if (c >= a.nbq && nblocks <= (int64_t)TMS_BATCHED_WAVES * ((c / a.nbq) * a.nbq)) {
        nb = c;
        break;
      }
    const int per_wave = (nb / a.nbq) * a.nbq;
    int64_t dpw = nd > 0 ? 4096 / nd : 64;  // long streams: each wave loads up to 32 KB of queries
    if (dpw < 1) dpw = 1;
    if (dpw > 64) dpw = 64;
    const int64_t min_wgs = (int64_t)256 * 4;  // one workgroup per CU, four rounds
    if (dpw > 1 && B / dpw < min_wgs) dpw = B / min_wgs > 0 ? B / min_wgs : 1;
    a.docs_per_wave = (int32_t)dpw;
    a.nblk = per_wave;
    const int64_t grid = (B + dpw - 1) / dpw;
    const int64_t per_launch = (int64_t)TMS_BATCHED_WAVES * per_wave;
    for (int64_t b0 = 0; b0 < nblocks; b0 += per_launch) {
      a.blk0 = (int32_t)b0;
      a.blk_end = (int32_t)(nblocks - b0 < per_launch ? nblocks : b0 + per_launch);
      const int rc = dtype == TMS_DTYPE_F16 ? batched_nb<TMS_DTYPE_F16>(nb, a, grid, st)
                                            : batched_nb<TMS_DTYPE_BF16>(nb, a, grid, st);
      if (rc) return rc;
    }
    return TMS_OK;
  }
  int64_t dpw = nd > 0 ? TMS_STREAM_TOKENS_PER_WAVE / nd : 1;
  const int64_t min_waves = (int64_t)256 * 16 * 2;
  if (dpw > 1 && B / dpw < min_waves) dpw = B / min_waves;
  if (dpw < 1) dpw = 1;
  if (dpw > 64) dpw = 64;
  a.docs_per_wave = (int32_t)dpw;
  const int64_t waves = (B + dpw - 1) / dpw;
  const int64_t grid = (waves + 3) / 4;
  for (int64_t b0 = 0; b0 < nblocks; b0 += 2) {  // two query blocks per pass over D
    a.blk0 = (int32_t)b0;
    a.blk_end = (int32_t)(nblocks - b0 < 2 ? nblocks : b0 + 2);
    a.nblk = a.blk_end - a.blk0;
    int rc;
    if (a.nblk == 2) {
      rc = dtype == TMS_DTYPE_F16 ? stream_ks<TMS_DTYPE_F16, 2>(a, grid, st)
                                  : stream_ks<TMS_DTYPE_BF16, 2>(a, grid, st);
    } else {
      rc = dtype == TMS_DTYPE_F16 ? stream_ks<TMS_DTYPE_F16, 1>(a, grid, st)
                                  : stream_ks<TMS_DTYPE_BF16, 1>(a, grid, st);
    }
    if (rc) return rc;
  }
  return TMS_OK;
}

}  // namespace tms
