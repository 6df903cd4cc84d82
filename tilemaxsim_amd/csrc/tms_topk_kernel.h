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
// shrinks a row by kChunk / k until one chunk holds it; the last level sorts its k keys
// (a last level of at most kShortRow keys runs a chunk of that size over four waves).
// Intermediate keys live in a caller-provided workspace. Levels that pass keys on first
// drop the keys below a bound on the chunk's k-th key taken from the threads' maxima
// (at k <= kFilterMaxK) and select among the survivors. Selection is a radix select on
// the 64-bit keys held in registers (4 or 16 per thread): one 256-bin LDS histogram per 8-bit
// digit, from the highest bit at which the chunk's real keys differ, narrowed to the
// keys that share the digits fixed so far, until the k-th largest key is known or a
// whole bin is needed (two or three passes for rows of similar scores). Padding keys are
// all 0 and a chunk's keys often share a digit, so the histogram updates would pile onto
// a few bins: each thread adds a run of equal bins with one atomic, and each wave counts
// into its own copy of the histogram.
#pragma once
#include "tms_common.h"

namespace tms {

constexpr int kChunk = 4096;  // keys sorted per workgroup (32 KiB of LDS)
// Threads per workgroup: a level that shrinks many chunks at once runs 4 waves per chunk
// (16 keys per thread); the last level, one chunk per row and nothing else running
// beside it, runs 16 waves (4 keys per thread, four waves per SIMD to overlap its serial
// steps). Measured on MaxSim-like and Gaussian rows, each is the faster of the two for
// its level.
constexpr int kLevelThreads = 256;
constexpr int kLastThreads = 1024;
constexpr int kMaxK = kChunk / 4;
// Rows (or last levels) of at most kShortRow keys: one chunk of that size over four
// waves, one per SIMD, so the serial steps (scans, reductions) are not repeated by four
// waves on every SIMD.
constexpr int kShortRow = 1024;
constexpr int kShortThreads = 256;
constexpr int kRankSortMaxK = 256;  // the last level orders up to this many keys by rank, more by a bitonic sort
// Levels that pass k keys on, at k <= kFilterMaxK, first drop the keys below a bound on
// the chunk's k-th key and select among the rest, gathered in LDS, when at most
// kCandCap of them remain.
constexpr int kFilterMaxK = 128;
constexpr int kCandCap = 1024;

// Order-preserving image of a float's bits, never 0 (0 is the padding key). Positive
// values map to b | 2^31 and negative ones to -b (mod 2^32), so -0.0 lands on +0.0's key
// (they compare equal, so they tie and go by index); every NaN, either sign, maps to the
// top key, above +inf, as torch ranks NaN.
__device__ __forceinline__ uint32_t order_key(float f) {
  const uint32_t b = __builtin_bit_cast(uint32_t, f);
  const uint32_t o = (int32_t)b < 0 ? 0u - b : (b | 0x80000000u);
  return (b & 0x7fffffffu) > 0x7f800000u ? 0xffffffffu : o;
}

// FIRST: input is fp32 scores (row stride in_stride), indices are positions in the row.
// Otherwise input is keys. LAST: write (value, index) pairs in descending order;
// otherwise write the best k keys of the chunk, in no particular order.
constexpr int kHistCopies = 4;  // wave w counts into copy w % 4; wave 0 scans four bins per lane

// Cross-lane steps without the LDS: DPP within 16-lane rows, row swaps across them.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, true);
}
template <int CTRL>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
  return ((uint64_t)dpp_u32<CTRL>((uint32_t)(v >> 32)) << 32) | dpp_u32<CTRL>((uint32_t)v);
}
// The value of lane l ^ 32 (permlane32_swap) or of the other row of the pair (row ^ 1,
// permlane16_swap), for a value every lane holds.
__device__ __forceinline__ uint32_t swap32_u32(uint32_t v, int lane) {
  const auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return lane < 32 ? (uint32_t)p[1] : (uint32_t)p[0];
}
__device__ __forceinline__ uint32_t swap16_u32(uint32_t v, int lane) {
  const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return ((lane >> 4) & 1) ? (uint32_t)p[0] : (uint32_t)p[1];
}
__device__ __forceinline__ uint64_t swap32_u64(uint64_t v, int lane) {
  return ((uint64_t)swap32_u32((uint32_t)(v >> 32), lane) << 32) | swap32_u32((uint32_t)v, lane);
}
__device__ __forceinline__ uint64_t swap16_u64(uint64_t v, int lane) {
  return ((uint64_t)swap16_u32((uint32_t)(v >> 32), lane) << 32) | swap16_u32((uint32_t)v, lane);
}
// Wave-wide min and max of 64-bit values and sum of counts; every lane gets the result.
__device__ __forceinline__ void wave_minmax(uint64_t& lo, uint64_t& hi, uint32_t& n, int lane) {
  auto step = [&](uint64_t l2, uint64_t h2, uint32_t n2) {
    lo = l2 < lo ? l2 : lo;
    hi = h2 > hi ? h2 : hi;
    n += n2;
  };
  step(dpp_u64<0xB1>(lo), dpp_u64<0xB1>(hi), dpp_u32<0xB1>(n));     // quad_perm [1,0,3,2]
  step(dpp_u64<0x4E>(lo), dpp_u64<0x4E>(hi), dpp_u32<0x4E>(n));     // quad_perm [2,3,0,1]
  step(dpp_u64<0x141>(lo), dpp_u64<0x141>(hi), dpp_u32<0x141>(n));  // row_half_mirror
  step(dpp_u64<0x140>(lo), dpp_u64<0x140>(hi), dpp_u32<0x140>(n));  // row_mirror
  step(swap16_u64(lo, lane), swap16_u64(hi, lane), swap16_u32(n, lane));
  step(swap32_u64(lo, lane), swap32_u64(hi, lane), swap32_u32(n, lane));
}
// Wave-wide maximum of a 32-bit value; every lane gets it.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x, int lane) {
  auto mx = [](uint32_t a, uint32_t b) { return a > b ? a : b; };
  x = mx(x, dpp_u32<0xB1>(x));   // quad_perm [1,0,3,2]
  x = mx(x, dpp_u32<0x4E>(x));   // quad_perm [2,3,0,1]
  x = mx(x, dpp_u32<0x141>(x));  // row_half_mirror
  x = mx(x, dpp_u32<0x140>(x));  // row_mirror
  x = mx(x, swap16_u32(x, lane));
  return mx(x, swap32_u32(x, lane));
}
// Inclusive prefix sum over the 64 lanes (lane order): row shifts, then row broadcasts.
__device__ __forceinline__ uint32_t wave_inclusive_sum(uint32_t x) {
  x += dpp_u32<0x111>(x);  // row_shr:1
  x += dpp_u32<0x112>(x);  // row_shr:2
  x += dpp_u32<0x114>(x);  // row_shr:4
  x += dpp_u32<0x118>(x);  // row_shr:8
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x142, 0xa, 0xf, false);  // row_bcast:15 into rows 1, 3
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x143, 0xc, 0xf, false);  // row_bcast:31 into rows 2, 3
  return x;
}

// One workgroup of NT threads selects the best k keys of chunk `chunk` of row `row`. The
// values written by the LAST level are read back from the scores (vals, row stride
// val_stride) at the selected indices, so they keep the input's bits (-0.0, NaN payloads).
// Every thread of the workgroup calls it (it synchronises the workgroup).
template <bool FIRST, bool LAST, int NT, int CH = kChunk>
__device__ __forceinline__ void topk_chunk(const float* __restrict__ vals, int64_t val_stride,
                                           const uint64_t* __restrict__ keys_in, int64_t n_in, int64_t in_stride,
                                           uint64_t* __restrict__ keys_out, int64_t out_stride,
                                           float* __restrict__ out_vals, int64_t* __restrict__ out_idx, int k,
                                           int64_t row, int64_t chunk) {
  constexpr int kPerThread = CH / NT;
  constexpr int kTopkWaves = NT / 64;
  static_assert(NT % 256 == 0 && NT <= kHistCopies * 256, "histogram clearing and the per-wave copies");
  static_assert(kTopkWaves <= 64, "one lane per wave in the cross-wave reduction");
  // Three histogram buffers: pass p counts into buffer p % 3, and buffer (p + 2) % 3 is
  // cleared after pass p's barrier, when no wave can still be scanning it (its last
  // scan, in pass p - 1, ended before that barrier) -- one barrier per pass.
  __shared__ uint32_t hist[3][kHistCopies][256];
  __shared__ uint32_t n_gt, n_eq, n_cand;
  __shared__ uint64_t cand[LAST ? 1 : kCandCap];
  __shared__ uint32_t red_t[kTopkWaves], red_m[kTopkWaves];
  __shared__ uint64_t sel[LAST ? kMaxK : 1];
  // FIRST && LAST (a row that fits one chunk): the selected scores' own bits, kept from
  // the loads so the output needs no second read of the scores.
  __shared__ uint32_t sel_bits[(FIRST && LAST) ? kMaxK : 1];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int64_t c0 = chunk * CH;
  // All loads are issued before any key is formed (one memory round trip, not one per
  // element). A chunk inside the row reads from one uniform base at 32-bit offsets and
  // every key is real; in the row's last chunk, positions past the row read its last
  // element and become padding.
  uint64_t key[kPerThread];
  float v[kPerThread];
  const bool inside = c0 + CH <= n_in;  // uniform
  if constexpr (FIRST) {
    if (inside) {
      const float* __restrict__ base = vals + row * val_stride + c0;
#pragma unroll
      for (int e = 0; e < kPerThread; e++) v[e] = base[e * NT + tid];
      const uint32_t inv = 0xffffffffu - (uint32_t)c0 - (uint32_t)tid;  // inverted index of element 0
#pragma unroll
      for (int e = 0; e < kPerThread; e++)
        key[e] = ((uint64_t)order_key(v[e]) << 32) | (uint64_t)(inv - (uint32_t)(e * NT));
    } else {
#pragma unroll
      for (int e = 0; e < kPerThread; e++) {
        const int64_t p = c0 + e * NT + tid;
        v[e] = vals[row * val_stride + (p < n_in ? p : n_in - 1)];
      }
#pragma unroll
      for (int e = 0; e < kPerThread; e++) {
        const int64_t p = c0 + e * NT + tid;
        key[e] = p < n_in ? ((uint64_t)order_key(v[e]) << 32) | (uint64_t)(0xffffffffu - (uint32_t)p)
                          : 0ull;  // below every real element
      }
    }
  } else {
    if (inside) {
      const uint64_t* __restrict__ base = keys_in + row * in_stride + c0;
#pragma unroll
      for (int e = 0; e < kPerThread; e++) key[e] = base[e * NT + tid];
    } else {
#pragma unroll
      for (int e = 0; e < kPerThread; e++) {
        const int64_t p = c0 + e * NT + tid;
        key[e] = keys_in[row * in_stride + (p < n_in ? p : n_in - 1)];
      }
#pragma unroll
      for (int e = 0; e < kPerThread; e++) {
        const int64_t p = c0 + e * NT + tid;
        key[e] = p < n_in ? key[e] : 0ull;
      }
    }
  }

  // The last level's ordering: each of the m distinct keys in sel[0, m) counts the keys
  // above it among sel[0, m8) (m rounded up to a multiple of 8; slots [m, m8 + kRankPad)
  // hold 0, below every real key), and a key of rank < k is written at its rank. S = 8, 4 or 2
  // lanes share a key when the threads allow: lane part p counts among slots
  // [p * m8 / S, (p + 1) * m8 / S), and DPP steps add the S counts.
  constexpr int kRankPad = 48;  // zero slots past m8 that the one-lane-per-key loop may read
  static_assert(kRankSortMaxK + kRankPad <= kMaxK, "the rank step's read ahead stays inside sel");
  auto rank_out = [&](int m, int m8) {
    const int lg = m * 8 <= NT ? 3 : (m * 4 <= NT ? 2 : (m * 2 <= NT ? 1 : 0));
    const int S = 1 << lg;
    const int per = m8 >> lg;
    for (int t = tid; t < (S > 1 ? S * m8 : m); t += NT) {
      const int i = t >> lg;
      const uint64_t me = sel[i];
      const int j0 = (t & (S - 1)) * per;
      uint32_t rank = 0u;
      int j = j0;
      const int end = j0 + per;
      if (S == 1) {
        // One lane per key, the whole range [0, m8) in steps of 32 with the next 16 keys
        // read ahead, so the LDS latency hides behind the compares (one wave per SIMD has
        // nothing else to run meanwhile). No exit between a read and its use, so the
        // compiler keeps the reads ahead. Reads run up to 40 slots past m8 and counts up
        // to 24, into slots that hold 0 (set with the keys): a 0 key is above nothing.
        uint64_t xa[16], xb[16];
        auto load16 = [&](uint64_t(&x)[16], int at) {
#pragma unroll
          for (int q = 0; q < 16; q++) x[q] = sel[at + q];
        };
        auto count16 = [&](const uint64_t(&x)[16]) {
#pragma unroll
          for (int q = 0; q < 16; q++) rank += x[q] > me ? 1u : 0u;
        };
        load16(xa, 0);
        for (j = 0; j < m8; j += 32) {
          load16(xb, j + 16);
          count16(xa);
          load16(xa, j + 32);
          count16(xb);
        }
        j = end;
      }
      for (; j + 8 <= end; j += 8) {  // eight reads in flight per step
        uint64_t x[8];
#pragma unroll
        for (int q = 0; q < 8; q++) x[q] = sel[j + q];
#pragma unroll
        for (int q = 0; q < 8; q++) rank += x[q] > me ? 1u : 0u;
      }
      for (; j < end; j++) rank += sel[j] > me ? 1u : 0u;
      if (S > 1) {
        rank += dpp_u32<0xB1>(rank);                 // quad_perm [1,0,3,2]: pairs
        if (S > 2) rank += dpp_u32<0x4E>(rank);      // quad_perm [2,3,0,1]: quads
        if (S > 4) rank += dpp_u32<0x141>(rank);     // row_half_mirror: the other quad of the eight
        if ((t & (S - 1)) != 0) continue;
      }
      if (i >= m || rank >= (uint32_t)k) continue;
      const int64_t idx = (int64_t)(0xffffffffu - (uint32_t)me);
      if constexpr (FIRST) out_vals[row * k + rank] = __builtin_bit_cast(float, sel_bits[i]);
      else out_vals[row * k + rank] = vals[row * val_stride + (idx < val_stride ? idx : val_stride - 1)];
      out_idx[row * k + rank] = idx;
    }
  };

  if constexpr (FIRST && LAST) {
    // A row of at most NT scores holds one key per thread (element tid), all real and
    // distinct (the index is in the low word): the top k are the keys of rank < k, with
    // no radix passes. n^2 / S compares per lane; at n = 256 about a quarter of the
    // passes' time.
    if (n_in <= NT && n_in <= kRankSortMaxK) {
      const int m8 = ((int)n_in + 7) & ~7;
      for (int t = tid; t < kRankSortMaxK + kRankPad; t += NT) sel[t] = t == tid ? key[0] : 0ull;  // 0 past the row
      if (tid < m8) sel_bits[tid] = __builtin_bit_cast(uint32_t, v[0]);
      __syncthreads();
      rank_out((int)n_in, m8);
      return;
    }
  }

  // Set-up that the first barrier below orders before its use: the first two histogram
  // buffers, the slot counters, and (last level) the padding slots of the rank sort.
  for (int i = tid; i < 2 * kHistCopies * 256; i += NT) (&hist[0][0][0])[i] = 0u;
  if (tid == 0) {
    n_gt = 0u;
    n_eq = 0u;
    n_cand = 0u;
  }
  if constexpr (LAST) {
    const int k8 = (k + 7) & ~7;
    if (k <= kRankSortMaxK)
      for (int t = k + tid; t < k8 + kRankPad; t += NT) sel[t] = 0ull;
  }
  auto below = [&](uint64_t m) -> uint32_t {  // set bits of m in lanes below this one
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
  };

  // The selection below runs over key[0, E); key[E, kPerThread) are 0 (padding). After
  // the pre-filter, the candidates' high words lie in [fT, fM].
  int E = kPerThread;
  bool filtered = false;
  uint32_t fT = 0u, fM = 0u;
  if constexpr (!LAST) {
    // Pre-filter. Wave w finds T_w, the j-th largest of its 64 threads' maximum high words
    // (j = ceil(k / waves); padding counts as 0). Each of those j threads holds a key whose
    // high word is >= T_w, so the chunk has at least waves * j >= k keys whose high word
    // is >= T = min_w T_w, and every key below T is below all of them: the top k lie among
    // the keys with high word >= T. On continuous scores they are a few k; they are
    // gathered in LDS and selected from there, at most kCandCap / NT per thread. T = 0
    // (fewer than j real keys in some wave) or more than kCandCap candidates (ties at the
    // bound) keep the registers and the full selection.
    if (k <= kFilterMaxK) {
      static_assert(kFilterMaxK <= 64 * kTopkWaves, "j <= 64: the bound is taken within each wave");
      static_assert(kCandCap % NT == 0 && kCandCap / NT <= kPerThread, "candidates per thread");
      uint32_t tm = 0u;
#pragma unroll
      for (int e = 0; e < kPerThread; e++) {
        const uint32_t h = (uint32_t)(key[e] >> 32);
        tm = h > tm ? h : tm;
      }
      // the j-th largest of the wave's tm, one bit at a time from the top: the largest t
      // that at least j lanes reach
      const uint32_t j = (uint32_t)((k + kTopkWaves - 1) / kTopkWaves);
      uint32_t t = 0u;
#pragma unroll
      for (int b = 31; b >= 0; b--) {
        const uint32_t c = t | (1u << b);
        t = (uint32_t)__popcll(__ballot(tm >= c)) >= j ? c : t;
      }
      const uint32_t wm = wave_max_u32(tm, lane);
      if (lane == 0) {
        red_t[wid] = t;
        red_m[wid] = wm;
      }
      __syncthreads();
      uint32_t T = red_t[0], M = red_m[0];
#pragma unroll
      for (int w = 1; w < kTopkWaves; w++) {
        T = red_t[w] < T ? red_t[w] : T;
        M = red_m[w] > M ? red_m[w] : M;
      }
      if (T != 0u) {  // uniform
        uint64_t mc[kPerThread];
        uint32_t wave_n = 0u;
#pragma unroll
        for (int e = 0; e < kPerThread; e++) {
          mc[e] = __ballot((uint32_t)(key[e] >> 32) >= T);
          wave_n += (uint32_t)__popcll(mc[e]);
        }
        uint32_t base = 0u;
        if (lane == 0) base = atomicAdd(&n_cand, wave_n);
        base = (uint32_t)__builtin_amdgcn_readlane((int)base, 0);
#pragma unroll
        for (int e = 0; e < kPerThread; e++) {
          const uint32_t pos = base + below(mc[e]);
          if ((uint32_t)(key[e] >> 32) >= T && pos < (uint32_t)kCandCap) cand[pos] = key[e];
          base += (uint32_t)__popcll(mc[e]);
        }
        __syncthreads();
        const uint32_t nc = (uint32_t)__builtin_amdgcn_readfirstlane((int)n_cand);
        if (nc <= (uint32_t)kCandCap) {
          filtered = true;
          fT = T;
          fM = M;
          E = (int)((nc + NT - 1) / NT);
#pragma unroll
          for (int e = 0; e < kPerThread; e++) {
            const uint32_t p = (uint32_t)(e * NT + tid);
            key[e] = (e < kCandCap / NT && p < nc) ? cand[e < kCandCap / NT ? p : 0] : 0ull;
          }
        }
      }
    }
  }

  // Where the real keys differ: the radix passes start below the bits that every real
  // key shares (scores in one binade share sign, exponent and the top mantissa bits), so
  // a row of similar scores takes two or three passes instead of up to eight. Padding
  // keys (0) are not real; a chunk with fewer than k real keys starts from the top.
  __shared__ uint64_t red_lo[kTopkWaves], red_hi[kTopkWaves];
  __shared__ uint32_t red_n[kTopkWaves];
  uint64_t prefix = 0;  // the key bits fixed so far: candidates have key >> shift == prefix
  int shift = 64;
  if (filtered) {
    // At least k candidates, all with high words in [fT, fM]: they share the bits above
    // the highest bit at which fT and fM differ (all 32 if they are equal).
    const uint32_t diff = fT ^ fM;
    shift = diff == 0u ? 32 : 64 - __builtin_clz(diff);
    prefix = shift == 64 ? 0ull : ((uint64_t)fM << 32) >> shift;
  } else {
    uint64_t lo = ~0ull, hi = 0ull;
    uint32_t nr = 0u;
#pragma unroll
    for (int e = 0; e < kPerThread; e++) {
      if (e < E && key[e] != 0ull) {
        lo = key[e] < lo ? key[e] : lo;
        hi = key[e] > hi ? key[e] : hi;
        nr++;
      }
    }
    wave_minmax(lo, hi, nr, lane);
    if (lane == 0) {
      red_lo[wid] = lo;
      red_hi[wid] = hi;
      red_n[wid] = nr;
    }
    __syncthreads();
    // lane w brings wave w's partial results; every lane gets the chunk's
    lo = lane < kTopkWaves ? red_lo[lane] : ~0ull;
    hi = lane < kTopkWaves ? red_hi[lane] : 0ull;
    nr = lane < kTopkWaves ? red_n[lane] : 0u;
    wave_minmax(lo, hi, nr, lane);
    if (nr >= (uint32_t)k) {
      const uint64_t diff = hi ^ lo;
      shift = diff == 0ull ? 0 : 64 - __builtin_clzll(diff);
      prefix = shift == 64 ? 0ull : hi >> shift;
    }
  }

  // Radix select, 8-bit digits (narrower for the last one). After a pass, `need` is the
  // number of keys still to take among the keys that share the prefix.
  uint32_t need = (uint32_t)k;
  bool whole_bin = false;  // the selection is every key >= prefix << shift
  for (int pass = 0; shift > 0; pass++) {
    const int w = shift < 8 ? shift : 8;
    shift -= w;
    uint32_t(&hb)[kHistCopies][256] = hist[pass % 3];
    {
      uint32_t run_bin = 0u, run_n = 0u;  // a run of this thread's keys in one bin
      auto count = [&](uint32_t bin) {
        if (run_n != 0u && bin != run_bin) {
          atomicAdd(&hb[wid % kHistCopies][run_bin], run_n);
          run_n = 0u;
        }
        run_bin = bin;
        run_n++;
      };
      if (shift >= 32) {
        // The digit lies in the high word (the score's order bits, where rows of distinct
        // scores are decided): 32-bit shifts and one bit-field extract per key instead of
        // 64-bit shifts. top = shift + w - 32 <= 32; top == 32 is the first pass from the
        // top, which every key takes.
        const uint32_t sh = (uint32_t)(shift - 32), top = sh + (uint32_t)w, pre = (uint32_t)prefix;
#pragma unroll
        for (int e = 0; e < kPerThread; e++) {
          if (e >= E) break;
          const uint32_t hi = (uint32_t)(key[e] >> 32);
          if (top == 32u || (hi >> top) == pre) count(__builtin_amdgcn_ubfe(hi, sh, (uint32_t)w));
        }
      } else {
#pragma unroll
        for (int e = 0; e < kPerThread; e++) {
          if (e >= E) break;
          if (shift + w == 64 || (key[e] >> (shift + w)) == prefix)
            count((uint32_t)(key[e] >> shift) & ((1u << w) - 1u));
        }
      }
      if (run_n != 0u) atomicAdd(&hb[wid % kHistCopies][run_bin], run_n);
    }
    __syncthreads();
    for (int i = tid; i < kHistCopies * 256; i += NT) (&hist[(pass + 2) % 3][0][0])[i] = 0u;
    // Every wave scans the histogram itself (lane l: bins 255 - 4l .. 252 - 4l, high to
    // low) and finds the bin that holds the need-th key.
    uint32_t c[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int bin = 255 - 4 * lane - j;
      c[j] = hb[0][bin] + hb[1][bin] + hb[2][bin] + hb[3][bin];
    }
    const uint32_t own = c[0] + c[1] + c[2] + c[3];
    const uint32_t incl = wave_inclusive_sum(own);
    const uint32_t excl = incl - own;
    const bool mine = excl < need && need <= incl;  // exactly one lane
    uint32_t above = excl, j = 0;
    if (mine)
      while (above + c[j] < need) above += c[j++];
    const uint32_t cj = c[0] * (j == 0) + c[1] * (j == 1) + c[2] * (j == 2) + c[3] * (j == 3);
    const int src = (int)__builtin_ctzll(__ballot(mine)) & 63;
    const uint32_t d = (uint32_t)__builtin_amdgcn_readlane((int)(255 - 4 * lane - j), src);
    const uint32_t cnt = (uint32_t)__builtin_amdgcn_readlane((int)cj, src);
    above = (uint32_t)__builtin_amdgcn_readlane((int)above, src);
    need -= above;
    prefix = (prefix << w) | d;
    if (cnt == need && prefix != 0) {  // the whole bin is needed (keys are unique but padding)
      whole_bin = true;
      break;
    }
  }
  // Selection: every key > T, then `need` keys equal to T (only padding keys repeat).
  // Each wave reserves its slots with one atomic per 64 keys (ballot and lane count).
  const uint64_t T = whole_bin ? (prefix << shift) - 1 : prefix;
  const uint32_t need_eq = whole_bin ? 0u : need;
  auto put = [&](uint32_t pos, uint64_t kv, int e) {
    if constexpr (FIRST && LAST) sel_bits[pos] = __builtin_bit_cast(uint32_t, v[e]);
    if constexpr (LAST) sel[pos] = kv;
    else keys_out[row * out_stride + chunk * k + pos] = kv;
  };
  // The wave's selected keys in element order: ballots first, then one atomic per wave
  // for all of them (and one for the keys equal to T, which only padding can need).
  uint64_t mg[kPerThread];
  uint32_t wave_gt = 0u, wave_eq = 0u;
  uint64_t any_eq = 0ull;
#pragma unroll
  for (int e = 0; e < kPerThread; e++) {
    mg[e] = 0ull;
    if (e >= E) continue;
    mg[e] = __ballot(key[e] > T);
    wave_gt += (uint32_t)__popcll(mg[e]);
    if (need_eq > 0u) {
      const uint64_t me = __ballot(key[e] == T);
      any_eq |= me;
      wave_eq += (uint32_t)__popcll(me);
    }
  }
  uint32_t base_gt = 0u, base_eq = 0u;
  if (lane == 0 && wave_gt > 0u) base_gt = atomicAdd(&n_gt, wave_gt);
  if (lane == 0 && wave_eq > 0u) base_eq = atomicAdd(&n_eq, wave_eq);
  base_gt = (uint32_t)__builtin_amdgcn_readlane((int)base_gt, 0);
  base_eq = (uint32_t)__builtin_amdgcn_readlane((int)base_eq, 0);
#pragma unroll
  for (int e = 0; e < kPerThread; e++) {
    if (e >= E) break;
    if (mg[e] != 0ull) {
      const uint32_t pos = base_gt + below(mg[e]);
      if (key[e] > T && pos < (uint32_t)k - need_eq) put(pos, key[e], e);  // always below; bounds every write
      base_gt += (uint32_t)__popcll(mg[e]);
    }
    if (any_eq != 0ull) {
      const uint64_t me = __ballot(key[e] == T);
      const uint32_t j = base_eq + below(me);
      if (key[e] == T && j < need_eq) put((uint32_t)k - need_eq + j, key[e], e);
      base_eq += (uint32_t)__popcll(me);
    }
  }
  if constexpr (LAST) {
    __syncthreads();
    if (k <= kRankSortMaxK) {  // every selected key is real, so all are distinct: rank = keys above it
      rank_out(k, (k + 7) & ~7);  // the slots past k hold 0 (set at the start)
      return;
    }
    int P = 1;  // bitonic sort of the k survivors, padded to a power of two
    while (P < k) P <<= 1;
    for (int i = k + tid; i < P; i += NT) sel[i] = 0;
    __syncthreads();
    for (int size = 2; size <= P; size <<= 1) {
      for (int stride = size >> 1; stride > 0; stride >>= 1) {
        for (int i = tid; i < P / 2; i += NT) {
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
    for (int i = tid; i < k; i += NT) {
      const int64_t idx = (int64_t)(0xffffffffu - (uint32_t)sel[i]);
      // a selected key is always a real element (k <= n); the clamp only bounds the read
      out_vals[row * k + i] = vals[row * val_stride + (idx < val_stride ? idx : val_stride - 1)];
      out_idx[row * k + i] = idx;
    }
  }
}

template <bool FIRST, bool LAST, int NT, int CH = kChunk>
__global__ void __launch_bounds__(NT) topk_level_kernel(const float* __restrict__ vals, int64_t val_stride,
                                                        const uint64_t* __restrict__ keys_in, int64_t n_in,
                                                        int64_t in_stride, uint64_t* __restrict__ keys_out,
                                                        int64_t out_stride, float* __restrict__ out_vals,
                                                        int64_t* __restrict__ out_idx, int k) {
  topk_chunk<FIRST, LAST, NT, CH>(vals, val_stride, keys_in, n_in, in_stride, keys_out, out_stride, out_vals, out_idx, k,
                                  blockIdx.y, blockIdx.x);
}

}  // namespace tms
