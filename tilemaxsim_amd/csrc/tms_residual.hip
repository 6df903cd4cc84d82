// Residual-compressed documents (the ColBERTv2 codec of colbert-ai 0.2.22, the ColBERT
// release the reference's PLAID drop-in runs against, src/plaid_integration_benchmark.py:23):
// decompression, and MaxSim decoded in registers.
//
// Format. Token t of the index is a centroid id codes[t] (int32) and a residual row of
// rb = d * nbits / 8 bytes: for every dimension j, bits 0..nbits-1 of its bucket index
// (least significant first) enter one bit stream, dimension after dimension, and the
// stream fills each byte from its most significant bit. The codec decodes
//   v = fp16(centroid[code] + weight[bucket])   (half arithmetic, per dimension)
//   x = v / fp16(|v|)                            (|v| accumulated in fp32)
// and PLAID scores the decoded documents with MaxSim.
//
// Decoding on gfx950:
//  * a byte of residual covers 8 / nbits dimensions; a 256-entry table in LDS (built by
//    each workgroup from the 2^nbits weights) maps a byte to the fp16 weights of its
//    dimensions, so an 8-dimension chunk takes nbits table reads (16 bytes in all);
//  * the centroid chunk is gathered straight into the MFMA A-operand registers of the
//    lane that owns the chunk (lane (r, g) owns chunk 4s + g of token r at k-step s, as in
//    the dense kernels); v = centroid + weight is one v_pk_add_f16 per 2 dimensions;
//  * |v|^2 is v_dot2_f32_f16 over the lane's dimensions plus two cross-lane adds.
//
// tms_residual_decompress writes x exactly as the codec computes it (fp32 division of
// fp16 values, rounded to fp16). The fused MaxSim kernel instead multiplies each token's
// dot products <q, v> by 1 / fp16(|v|) before the max, which is the same score without
// rounding x to fp16 first (differences ~1e-4 relative on unit-norm data).
#include <string.h>

#include "tms_common.h"

namespace tms {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;  // the single-query and decompression kernels' workgroup; the byte table's entries

// Reinterpret a dword as two halves and back. The argument is taken by value: with the
// ROCm 7.2 clang, __builtin_bit_cast applied directly to a subscripted ext-vector element
// (bit_cast(T, vec[i])) reads element 0 whatever i is, so element values must pass
// through a scalar first.
__device__ __forceinline__ f16x2 as_f16x2(uint32_t x) { return __builtin_bit_cast(f16x2, x); }
__device__ __forceinline__ uint32_t as_u32(f16x2 x) { return __builtin_bit_cast(uint32_t, x); }

struct ResArgs {
  const uint8_t* Q;          // (nq, d) fp16
  const uint8_t* centroids;  // (ncent, d) fp16
  const int32_t* codes;      // (T)
  const uint8_t* residuals;  // (T, rb)
  const int64_t* offsets;    // (ndocs + 1): document p is index rows [offsets[p], offsets[p+1])
  const int64_t* pids;       // (B) documents to score, or null for 0 .. B-1
  const uint16_t* weights;   // (2^nbits) fp16 bucket weights
  float* out;                // (B) scores, or (T, d) fp16 for the decompression kernel
  int64_t B, ndocs, T, ncent, pad_len;
  int32_t nq, nbq, blk0, d, rb, docs_per_wave;
  int32_t nblk, blk_end;  // batched kernel: blocks per wave, one past the launch's last block
  int32_t wpd;            // fused kernel: waves per document (1: each wave walks whole documents)
};

// Byte -> fp16 weights of its 8 / NBITS dimensions, in dimension order. The table is
// written and read only through __builtin_memcpy (byte-typed accesses), so no access
// to it depends on type-based alias rules.
template <int NBITS>
__device__ void build_lut(uint8_t* lut, const uint16_t* weights) {
  constexpr int kPerByte = 8 / NBITS;
  constexpr uint32_t kMask = (1u << NBITS) - 1u;
  for (int byte = threadIdx.x; byte < 256; byte += kThreads) {
    uint16_t e[kPerByte];
#pragma unroll
    for (int k = 0; k < kPerByte; k++) {
      // dimension k's bits sit at byte bits 7 - (k*NBITS + j), j = 0 .. NBITS-1
      uint32_t bucket = 0;
#pragma unroll
      for (int j = 0; j < NBITS; j++) bucket |= ((byte >> (7 - (k * NBITS + j))) & 1u) << j;
      e[k] = weights[bucket & kMask];
    }
    __builtin_memcpy(lut + byte * 2 * kPerByte, e, sizeof(e));
  }
}

// The NBITS residual bytes of one 8-dimension chunk (little-endian in a u32).
template <int NBITS>
__device__ __forceinline__ uint32_t load_res(const uint8_t* row, int chunk) {
  if constexpr (NBITS == 1) return row[chunk];
  else if constexpr (NBITS == 2) return *(const uint16_t*)(row + 2 * chunk);
  else return *(const uint32_t*)(row + 4 * chunk);
}

// The residual bytes of chunks c0 .. c0+KS-1 of one token (NBITS bytes per chunk, KS*NBITS
// contiguous bytes), one u32 per chunk as load_res returns it. WIDE: one load of the whole
// run, which needs KS*NBITS to be 1, 2, 4, 8 or 16 and the run aligned to its size (the
// host checks the pointer; rows are 4*KS*NBITS bytes, so every run is then aligned).
template <int NBITS, int KS, bool WIDE>
__device__ __forceinline__ void load_res_run(const uint8_t* row, int c0, uint32_t (&rr)[KS]) {
  constexpr int TB = NBITS * KS;
  if constexpr (WIDE) {
    const uint8_t* p = row + TB * (c0 / KS);
    if constexpr (TB == 16) {
      const uint4 v = *(const uint4*)p;
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int s = 0; s < KS; s++) rr[s] = w[s];  // NBITS = 4, KS = 4
    } else if constexpr (TB == 8) {
      const uint2 v = *(const uint2*)p;
      const uint64_t x = ((uint64_t)v.y << 32) | v.x;
#pragma unroll
      for (int s = 0; s < KS; s++) rr[s] = (uint32_t)(x >> (8 * NBITS * s)) & (uint32_t)((1ull << (8 * NBITS)) - 1);
    } else if constexpr (TB == 4) {
      const uint32_t x = *(const uint32_t*)p;
      if constexpr (NBITS == 4) {
        rr[0] = x;  // KS = 1
      } else {
#pragma unroll
        for (int s = 0; s < KS; s++) rr[s] = (x >> (8 * NBITS * s)) & ((1u << (8 * NBITS)) - 1u);
      }
    } else if constexpr (TB == 2) {
      const uint32_t x = *(const uint16_t*)p;
      if constexpr (NBITS == 2) {
        rr[0] = x;  // KS = 1
      } else {
#pragma unroll
        for (int s = 0; s < KS; s++) rr[s] = (x >> (8 * s)) & 0xffu;
      }
    } else {
      static_assert(TB == 1, "WIDE needs a power-of-two run of at most 16 bytes");
      rr[0] = *p;
    }
  } else {
#pragma unroll
    for (int s = 0; s < KS; s++) rr[s] = load_res<NBITS>(row, c0 + s);
  }
}
template <int NBITS, int KS>
constexpr bool res_run_pow2() {
  constexpr int TB = NBITS * KS;
  return TB == 1 || TB == 2 || TB == 4 || TB == 8 || TB == 16;
}

// fp16 weights of the chunk's 8 dimensions from the LDS table.
template <int NBITS>
__device__ __forceinline__ u32x4 chunk_weights(const uint8_t* lut, uint32_t rw) {
  uint32_t w[4];
  if constexpr (NBITS == 1) {
    __builtin_memcpy(w, lut + (rw & 0xffu) * 16, 16);
  } else if constexpr (NBITS == 2) {
    __builtin_memcpy(w, lut + (rw & 0xffu) * 8, 8);
    __builtin_memcpy(w + 2, lut + ((rw >> 8) & 0xffu) * 8, 8);
  } else {
#pragma unroll
    for (int i = 0; i < 4; i++) __builtin_memcpy(w + i, lut + ((rw >> (8 * i)) & 0xffu) * 4, 4);
  }
  return u32x4{w[0], w[1], w[2], w[3]};
}

// v = fp16(c + w) for 8 dimensions; n2 += sum v^2 in fp32.
__device__ __forceinline__ u32x4 add_chunk(u32x4 c, u32x4 w, float& n2) {
  u32x4 v;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t ci = c[i], wi = w[i];
    const f16x2 s = as_f16x2(ci) + as_f16x2(wi);
    n2 = __builtin_amdgcn_fdot2(s, s, n2, false);
    v[i] = as_u32(s);
  }
  return v;
}

// 1 / fp16(sqrt(n2)): the codec's half-precision norm (clamped at the smallest fp16 > 0).
__device__ __forceinline__ float inv_norm(float n2) {
  float n = (float)(_Float16)sqrtf(n2);
  return 1.0f / fmaxf(n, 5.9604645e-8f);
}

template <int K>
struct RingSlot {
  static constexpr int value = K;
};
bool rerank_fits(int64_t B, int64_t tokens_per_doc);  // tms_rerank.hip

#ifndef TMS_RES_SPLIT_WAVES
#define TMS_RES_SPLIT_WAVES 3072  // waves a split call may launch: three per SIMD
#endif
#ifndef TMS_RES1_RING
#define TMS_RES1_RING 3  // ring slots of the single-query fused kernel (3..8)
#endif
static_assert(TMS_RES1_RING >= 3 && TMS_RES1_RING <= 8, "the fused kernel's step loop is unrolled up to 8 times");

// ---------------------------------------------------------------------------------
// Fused MaxSim. One wave streams whole documents; a tile is 16 * NSUB tokens x d. For
// small calls (a.wpd > 1) the four waves of a workgroup split documents instead: part p
// of a document scores its tiles p, p + wpd, p + 2 wpd, ..., the parts' per-column
// maxima meet in LDS and part 0 sums them (in the same order, so the bits are those of
// the one-wave walk).
// With a ring of NS tiles, centroid ids are read NS tiles ahead and the centroid chunks
// and residual bytes NS - 1 tiles ahead of the tile being decoded and scored.
// QLDS: the query fragments sit in LDS (shared by the workgroup's four waves) instead of
// 8 * KS VGPRs per lane, which buys occupancy.
// Lane (r, g) owns chunks KS*g .. KS*g + KS-1 of token r, contiguous dimensions, so its
// residual bytes are one contiguous run: with WIDE they arrive in one load per token
// instead of one per chunk. Each vector-memory instruction costs about as much as a
// centroid gather, so this is what the gather rate depends on.
template <int KS, int NBITS, int NSUB, bool QLDS, bool WIDE, bool SPLIT>
__global__ void __launch_bounds__(256) residual_maxsim_kernel(ResArgs a) {
  constexpr int TT = 16 * NSUB;
  __shared__ __attribute__((aligned(16))) uint8_t lut[4096];
  __shared__ u32x4 qsh[QLDS ? KS * 2 * 64 : 1];
  build_lut<NBITS>(lut, a.weights);
  if constexpr (QLDS) {
    // fragment (s, h) of lane l: query token 32 blk0 + 16 h + l % 16, chunk KS (l / 16) + s
    for (int f = threadIdx.x; f < KS * 2 * 64; f += kThreads) {
      const int l = f & 63, h = (f >> 6) & 1, s = f >> 7;
      const int tok = a.blk0 * 32 + 16 * h + (l & 15);
      const int64_t row = tok < a.nq ? tok : a.nq - 1;
      const u32x4 v = *(const u32x4*)(a.Q + (row * a.d + 8 * (KS * (l >> 4) + s)) * 2);
      qsh[f] = tok < a.nq ? v : u32x4{0u, 0u, 0u, 0u};
    }
  }
  __syncthreads();

  const int lane = threadIdx.x & 63;
  const int r = lane & 15, g = lane >> 4;
  const int wid = threadIdx.x >> 6;
  const int wpd = SPLIT ? a.wpd : 1;  // 2 or 4 when SPLIT
  const int part = wid % wpd;  // 0 when each wave walks whole documents
  // wave-uniform, so the document walk below runs on the scalar unit
  const int64_t wave = (int64_t)blockIdx.x * (kThreads / 64) + wid;
  const int64_t b_begin =
      wave_uniform(SPLIT ? (int64_t)blockIdx.x * (kThreads / 64 / wpd) + wid / wpd : wave * a.docs_per_wave);
  const int64_t b_end =
      b_begin >= a.B ? b_begin : ((b_begin + a.docs_per_wave < a.B) ? b_begin + a.docs_per_wave : a.B);
  const float NEG_INF = -__builtin_inff();
  __shared__ float red[SPLIT ? kThreads / 64 : 1][2][16];  // each part's per-column maxima
  if (SPLIT && g == 0) red[wid][0][r] = red[wid][1][r] = NEG_INF;
  if (!SPLIT && b_begin >= a.B) return;  // (parts of a split document meet at a barrier)

  // query block a.blk0: query tokens 32 * blk0 + 16 h + r
  u32x4 qf[QLDS ? 1 : KS][2];
  bool qvalid[2];
#pragma unroll
  for (int h = 0; h < 2; h++) {
    const int tok = a.blk0 * 32 + 16 * h + r;
    qvalid[h] = tok < a.nq;
    if constexpr (!QLDS) {
      const int64_t row = qvalid[h] ? tok : a.nq - 1;  // loaded unconditionally, zeroed below
#pragma unroll
      for (int s = 0; s < KS; s++) {
        const u32x4 v = *(const u32x4*)(a.Q + (row * a.d + 8 * (KS * g + s)) * 2);
        qf[s][h] = qvalid[h] ? v : u32x4{0u, 0u, 0u, 0u};
      }
    }
  }
  auto qfrag = [&](int s, int h) -> u32x4 {
    if constexpr (QLDS) {
      // the empty asm hides the index from the optimiser, which would otherwise hoist
      // these loop-invariant reads into registers and undo the point of QLDS
      uint32_t idx = (uint32_t)((s * 2 + h) * 64 + lane);
      asm volatile("" : "+v"(idx));
      return qsh[idx];
    } else {
      return qf[s][h];
    }
  };

  // ---- documents ---------------------------------------------------------------
  // A cursor is a tile position: document position b in [b_begin, b_end), its first
  // index row, its length (< 2^31 tokens) and the tile's first token. All of it is
  // wave-uniform and lives in scalar registers.
  struct Cur {
    int64_t b, base;
    int32_t len, t0;
  };
  // The wave's documents (at most 64) are read once, lane j holding document
  // b_begin + j: base row and length (-1 for an invalid pid or offsets). The walk
  // below takes them with readlane, so crossing a document never waits for memory.
  int64_t dbase = 0;
  int32_t dlen = -1;
  if (b_begin + lane < b_end) {
    const int64_t p = a.pids ? a.pids[b_begin + lane] : b_begin + lane;
    if (p >= 0 && p < a.ndocs) {
      const int64_t s0 = a.offsets[p], e0 = a.offsets[p + 1];
      if (s0 >= 0 && e0 >= s0 && e0 <= a.T && e0 - s0 <= 0x7fffffff) {
        dbase = s0;
        dlen = (int32_t)(e0 - s0);
      }
    }
  }
  auto bounds = [&](int64_t b, int64_t& base) -> int64_t {
    const int j = (int)(b - b_begin);
    const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)dbase, j);
    const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)((uint64_t)dbase >> 32), j);
    base = (int64_t)(((uint64_t)hi << 32) | lo);
    return __builtin_amdgcn_readlane(dlen, j);
  };
  const bool first_blk = a.blk0 == 0;
  auto write = [&](int64_t b, float v) {
    if (lane == 0) {
      float* o = a.out + b;
      *o = first_blk ? v : *o + v;
    }
  };
  // Move to the first document at or after b with a token, scoring the empty (or
  // invalid) ones on the way. Past the last document the cursor keeps its last tile's
  // rows, so prefetches through it stay in bounds.
  auto seek = [&](Cur& c, int64_t b) {
    for (; b < b_end; b++) {
      int64_t base = 0;
      const int64_t len = bounds(b, base);
      if (len > 0) {
        c.b = b;
        c.base = base;
        c.len = (int32_t)len;
        c.t0 = part * TT;
        if (SPLIT && c.t0 >= c.len) c.b = b_end;  // a part with no tile of the (single) document
        return;
      }
      if (SPLIT && part != 0) {  // a document part: part 0 writes the score
      } else if (len < 0) {  // invalid pid or offsets: NaN, written as an integer by every launch
        if (lane == 0) store_nan_score(a.out + b);
      } else {
        write(b, a.pad_len > 0 ? 0.f : NEG_INF);
      }
    }
    c.b = b_end;
  };
  auto advance = [&](Cur& c) {
    if (c.b >= b_end) return;
    c.t0 += TT * wpd;
    if (c.t0 >= c.len) seek(c, c.b + 1);
  };
  auto row_of = [&](const Cur& c, int sub) -> int64_t {
    int32_t t = c.t0 + 16 * sub + r;
    if (t > c.len - 1) t = c.len - 1;
    return c.base + t;
  };

  // ---- pipeline state ------------------------------------------------------------
  struct Body {
    u32x4 cen[NSUB][KS];     // centroid chunks
    uint32_t res[NSUB][KS];  // residual bytes of the chunks
  };
  auto load_codes = [&](int32_t (&cd)[NSUB], const Cur& c) {
#pragma unroll
    for (int sub = 0; sub < NSUB; sub++) cd[sub] = a.codes[row_of(c, sub)];
  };
  auto load_body = [&](const int32_t (&cd)[NSUB], const Cur& c, Body& bd) {
#pragma unroll
    for (int sub = 0; sub < NSUB; sub++) {
      int64_t code = cd[sub];
      code = code < 0 ? 0 : (code >= a.ncent ? a.ncent - 1 : code);
      const uint8_t* crow = a.centroids + code * a.d * 2;
      const uint8_t* rrow = a.residuals + row_of(c, sub) * a.rb;
#pragma unroll
      for (int s = 0; s < KS; s++) bd.cen[sub][s] = *(const u32x4*)(crow + 16 * (KS * g + s));
      load_res_run<NBITS, KS, WIDE>(rrow, KS * g, bd.res[sub]);
    }
  };

  float rmax[2] = {NEG_INF, NEG_INF};
  auto finish = [&](int64_t b, int32_t len) {
    if constexpr (SPLIT) {  // the part's maxima go to LDS; part 0 combines them after the walk
#pragma unroll
      for (int h = 0; h < 2; h++) {
        float m = rmax[h];
        m = fmaxf(m, __shfl_xor(m, 16));
        m = fmaxf(m, __shfl_xor(m, 32));
        if (g == 0) red[wid][h][r] = m;
        rmax[h] = NEG_INF;
      }
      return;
    }
    const bool padded = len < a.pad_len;
    float s = 0.f;
#pragma unroll
    for (int h = 0; h < 2; h++) {
      float m = rmax[h];
      m = fmaxf(m, __shfl_xor(m, 16));
      m = fmaxf(m, __shfl_xor(m, 32));
      if (padded) m = fmaxf(m, 0.f);
      s += qvalid[h] ? m : 0.f;
      rmax[h] = NEG_INF;
    }
    s += __shfl_xor(s, 8);
    s += __shfl_xor(s, 4);
    s += __shfl_xor(s, 2);
    s += __shfl_xor(s, 1);
    write(b, s);
  };

  auto compute = [&](const Cur& c, const Body& bd) {
#pragma unroll
    for (int sub = 0; sub < NSUB; sub++) {
      float n2 = 0.f;
      f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
      for (int s = 0; s < KS; s++) {
        const u32x4 v = add_chunk(bd.cen[sub][s], chunk_weights<NBITS>(lut, bd.res[sub][s]), n2);
        acc[0] = mfma16x16x32<TMS_DTYPE_F16>(v, qfrag(s, 0), acc[0]);
        acc[1] = mfma16x16x32<TMS_DTYPE_F16>(v, qfrag(s, 1), acc[1]);
      }
      n2 += __shfl_xor(n2, 16);
      n2 += __shfl_xor(n2, 32);
      const float inv = inv_norm(n2);  // of token r (every g holds it)
      // accumulator rows are tokens 4 g + i
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float sc = __shfl(inv, 4 * g + i);
        rmax[0] = fmaxf(rmax[0], acc[0][i] * sc);
        rmax[1] = fmaxf(rmax[1], acc[1][i] * sc);
      }
    }
    if (c.t0 + TT * wpd >= c.len) finish(c.b, c.len);  // the last tile of this wave's share
  };

  // A ring of NS tiles. While tile i is scored, the bodies of tiles i+1 .. i+NS-1 and
  // the ids of tile i+NS are in flight. Each step issues the ids of tile i+NS before
  // the body of tile i+NS-1, so waiting for the ids of tile i+NS-1 (issued a step
  // earlier, before the body of tile i+NS-2) never waits for the later loads. One
  // cursor walks ahead (and scores empty documents as it passes them); the ring keeps
  // its positions. The step is unrolled NS times, so every ring slot is a compile-time
  // register.
  constexpr int NS = TMS_RES1_RING;
  // The walk is a lambda so that its early exits still reach the parts' barrier below.
  [&]() {
  Body bd[NS];
  int32_t ids[NS][NSUB];
  Cur cr[NS];
  Cur walk;
  seek(walk, b_begin);
  if (walk.b >= b_end) return;
#pragma unroll
  for (int k = 0; k < NS; k++) {
    cr[k] = walk;
    load_codes(ids[k], walk);
    advance(walk);
  }
#pragma unroll
  for (int k = 0; k < NS - 1; k++) load_body(ids[k], cr[k], bd[k]);
  auto step = [&](auto slot) -> bool {
    constexpr int k = decltype(slot)::value % NS;  // tile i sits in ring slot k
    constexpr int kb = (k + NS - 1) % NS;          // the slot tile i-1 left: tile i+NS-1
    const Cur c = cr[k];
    cr[k] = walk;                                  // tile i+NS
    advance(walk);
    load_codes(ids[k], cr[k]);
    load_body(ids[kb], cr[kb], bd[kb]);            // tile i+NS-1
    compute(c, bd[k]);                             // tile i
    return cr[(k + 1) % NS].b >= b_end;            // tile i+1 exists?
  };
  while (true) {
    if (step(RingSlot<0>{})) return;
    if (step(RingSlot<1>{})) return;
    if (step(RingSlot<2>{})) return;
    if constexpr (NS > 3) {
      if (step(RingSlot<3>{})) return;
    }
    if constexpr (NS > 4) {
      if (step(RingSlot<4>{})) return;
    }
    if constexpr (NS > 5) {
      if (step(RingSlot<5>{})) return;
    }
    if constexpr (NS > 6) {
      if (step(RingSlot<6>{})) return;
    }
    if constexpr (NS > 7) {
      if (step(RingSlot<7>{})) return;
    }
  }
  }();

  if constexpr (SPLIT) {  // one document per wave group: part 0 combines the parts and writes
    __syncthreads();
    const int32_t len0 = __builtin_amdgcn_readlane(dlen, 0);  // lane 0 holds document b_begin
    if (part == 0 && b_begin < b_end && len0 > 0) {
      const bool padded = len0 < a.pad_len;
      float s = 0.f;
#pragma unroll
      for (int h = 0; h < 2; h++) {
        float m = red[wid][h][r];
        for (int p = 1; p < wpd; p++) m = fmaxf(m, red[wid + p][h][r]);
        if (padded) m = fmaxf(m, 0.f);
        s += qvalid[h] ? m : 0.f;
      }
      s += __shfl_xor(s, 8);
      s += __shfl_xor(s, 4);
      s += __shfl_xor(s, 2);
      s += __shfl_xor(s, 1);
      write(b_begin, s);
    }
  }
}

// ---------------------------------------------------------------------------------
// Batched queries over residual-compressed documents. One workgroup of eight waves per
// CU walks a run of documents in 16-token tiles, every wave the same tiles. A tile is
// decoded once: wave w < KS decodes k-step w (lane (r, g): chunk 4 w + g of token r, the
// MFMA A-operand layout), the KS partial |v|^2 of each token meet in LDS, and the
// normalised x = fp16(v * (1 / fp16(|v|))) goes to an LDS ring from which all eight
// waves score the tile against the query blocks they hold, as the dense batched kernel
// does. Step i opens with one LDS-only barrier and then: reads tile i+1's fragments;
// (decoding waves) issues the ids of tile i+7 and the centroid chunks / residual bytes of
// tile i+5, normalises tile i+2 into the ring (its partial norms visible since the
// barrier) and decodes tile i+3 (its partial norms to LDS); scores tile i. The decoding
// work precedes the wave's own MFMAs, so it overlaps the MFMAs of the scoring-only wave
// that shares its SIMD instead of stalling the barrier after them.
constexpr int kResBatchedWaves = 8;

template <int KS, int NBITS, int NB>
__global__ void __launch_bounds__(64 * kResBatchedWaves, 1) residual_batched_kernel(ResArgs a) {
  constexpr int NS = 3;  // slots of every pipeline buffer: x tiles, partial norms, bodies, ids
  __shared__ __attribute__((aligned(16))) uint8_t lut[4096];
  __shared__ u32x4 ring[NS][4][64];
  __shared__ f32x4 nrm[NS][16];  // partial |v|^2 of token r from decoding wave w, at [slot][r][w]
  build_lut<NBITS>(lut, a.weights);

  const int lane = threadIdx.x & 63;
  const int r = lane & 15, g = lane >> 4;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // scalar: `decoder` branches stay uniform
  const bool decoder = wid < KS;
  const float NEG_INF = -__builtin_inff();

  const int64_t b_begin = wave_uniform((int64_t)blockIdx.x * a.docs_per_wave);
  const int64_t b_end = (b_begin + a.docs_per_wave < a.B) ? b_begin + a.docs_per_wave : a.B;
  const int64_t ndocs = b_end - b_begin;  // >= 1: the host launches no empty workgroup

  // Query blocks: wave w holds blocks blk0 + w * nblk + j (whole queries).
  const int my_blk0 = a.blk0 + wid * a.nblk;
  int my_nblk = a.blk_end - my_blk0;  // <= 0 for a wave with no query
  if (my_nblk > a.nblk) my_nblk = a.nblk;
  u32x4 qf[NB][KS][2];
  bool qv[NB][2];
#pragma unroll
  for (int j = 0; j < NB; j++)
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const int jb = my_blk0 + j;
      const int qi = jb / a.nbq;
      const int tok = (jb - qi * a.nbq) * 32 + 16 * h + r;
      qv[j][h] = j < my_nblk && tok < a.nq;
      const int64_t row = qv[j][h] ? (int64_t)qi * a.nq + tok : 0;
#pragma unroll
      for (int s = 0; s < KS; s++) {
        const u32x4 v = *(const u32x4*)(a.Q + (row * a.d + 8 * (4 * s + g)) * 2);
        qf[j][s][h] = qv[j][h] ? v : u32x4{0u, 0u, 0u, 0u};
      }
    }

  // The workgroup's documents (at most 64): lane j holds document b_begin + j's first
  // index row and length (-1 for an invalid pid or offsets).
  int64_t dbase = 0;
  int32_t dlen = -1;
  if (lane < ndocs) {
    const int64_t p = a.pids ? a.pids[b_begin + lane] : b_begin + lane;
    if (p >= 0 && p < a.ndocs) {
      const int64_t s0 = a.offsets[p], e0 = a.offsets[p + 1];
      if (s0 >= 0 && e0 >= s0 && e0 <= a.T && e0 - s0 <= 0x7fffffff) {
        dbase = s0;
        dlen = (int32_t)(e0 - s0);
      }
    }
  }
  // Per-document scores of the wave's blocks: lane j holds document b_begin + j.
  float pend[NB];
#pragma unroll
  for (int j = 0; j < NB; j++) pend[j] = NEG_INF;

  struct Cur {
    int64_t b, base;
    int32_t len, t0;
  };
  auto bounds = [&](int64_t b, int64_t& base) -> int32_t {
    const int j = (int)(b - b_begin);
    const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)dbase, j);
    const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)((uint64_t)dbase >> 32), j);
    base = (int64_t)(((uint64_t)hi << 32) | lo);
    return __builtin_amdgcn_readlane(dlen, j);
  };
  // Move to the first document at or after b with a token. With `record`, the empty or
  // invalid documents passed on the way get their scores. Past the last document the
  // cursor keeps its last tile's rows, so loads through it stay in bounds.
  auto seek = [&](Cur& c, int64_t b, bool record) {
    for (; b < b_end; b++) {
      int64_t base = 0;
      const int32_t len = bounds(b, base);
      if (len > 0) {
        c.b = b;
        c.base = base;
        c.len = len;
        c.t0 = 0;
        return;
      }
      if (record) {  // invalid pid or offsets (len < 0): the final store writes NaN for the lane
        const float v = a.pad_len > 0 ? 0.f : NEG_INF;
#pragma unroll
        for (int j = 0; j < NB; j++) pend[j] = lane == (int)(b - b_begin) ? v : pend[j];
      }
    }
    c.b = b_end;
  };
  auto advance = [&](Cur& c, bool record) {
    if (c.b >= b_end) return;
    c.t0 += 16;
    if (c.t0 >= c.len) seek(c, c.b + 1, record);
  };
  auto row_of = [&](const Cur& c) -> int64_t {
    int32_t t = c.t0 + r;
    if (t > c.len - 1) t = c.len - 1;
    return c.base + t;
  };

  Cur wc, wb, wi;  // scoring (tile i), body loads (tile i+4), id loads (tile i+6)
  wc.b = b_end;
  wc.base = 0;
  wc.len = 1;
  wc.t0 = 0;
  seek(wc, b_begin, true);

  // The pipeline, instantiated twice: decoding waves (loads, decode, ring writes) and
  // scoring-only waves, so each copy's loads are straight-line code whose outstanding
  // count the compiler tracks exactly (a load under a branch would make it wait for all).
  auto pipeline = [&](auto dec_tag) {
    constexpr bool DEC = decltype(dec_tag)::value == 1;
    wb = wc;
    wi = wc;
    __syncthreads();  // the byte table is built

    struct Body {
      u32x4 cen;
      uint32_t res;
    };
    int32_t ids[NS];
    Body bd[NS];
    u32x4 vkeep = {0u, 0u, 0u, 0u};
    const int chunk = 4 * (DEC ? wid : 0) + g;
    auto load_ids = [&](int32_t& id) {
      if constexpr (DEC) id = a.codes[row_of(wi)];
      advance(wi, false);
    };
    auto load_body = [&](const int32_t id, Body& bo) {
      if constexpr (DEC) {
        int64_t code = id;
        code = code < 0 ? 0 : (code >= a.ncent ? a.ncent - 1 : code);
        bo.cen = *(const u32x4*)(a.centroids + code * a.d * 2 + 16 * chunk);
        bo.res = load_res<NBITS>(a.residuals + row_of(wb) * a.rb, chunk);
      }
      advance(wb, false);
    };
    auto decode = [&](const Body& bo, int slot) {
      if constexpr (DEC) {
        float n2 = 0.f;
        vkeep = add_chunk(bo.cen, chunk_weights<NBITS>(lut, bo.res), n2);
        n2 = cross_row_sum(n2);  // over the wave's 32 dimensions of token r
        if (g == 0) nrm[slot][r][wid] = n2;
      }
    };
    auto normalise = [&](int slot) {
      if constexpr (DEC) {
        const f32x4 p = nrm[slot][r];
        float n2 = p[0];
#pragma unroll
        for (int w = 1; w < KS; w++) n2 += p[w];
        const float inv = inv_norm(n2);
        u32x4 x;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const uint32_t vi = vkeep[i];
          const f16x2 v2 = as_f16x2(vi);
          f16x2 q;
          q.x = (_Float16)((float)v2.x * inv);
          q.y = (_Float16)((float)v2.y * inv);
          x[i] = as_u32(q);
        }
        ring[slot][wid][lane] = x;
      }
    };
    auto sync = [&]() {  // LDS-only fence: the loads in flight are not waited for
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    };

    // Schedule, for tile t: ids loaded at step t-7, centroid chunk and residual bytes at
    // t-5, decoded at t-3 (partial norms to LDS), normalised at t-2 (into the ring),
    // fragments read at t-1, scored at t; tile t sits in slot t % 3 of every buffer. Step
    // i opens with the barrier, and a decoding wave then normalises tile i+2 and decodes
    // tile i+3 before issuing its MFMAs for tile i, so that work overlaps the MFMAs of the
    // scoring-only wave on its SIMD.
    // prologue: ends with tile 0's fragments read, tile 1 normalised, tile 2 decoded, the
    // bodies of tiles 3 and 4 and the ids of tiles 5 and 6 in flight
    load_ids(ids[0]);  // tiles 0, 1, 2
    load_ids(ids[1]);
    load_ids(ids[2]);
    load_body(ids[0], bd[0]);  // tiles 0, 1, 2
    load_body(ids[1], bd[1]);
    load_body(ids[2], bd[2]);
    load_ids(ids[0]);  // tiles 3, 4
    load_ids(ids[1]);
    decode(bd[0], 0);  // tile 0
    sync();
    normalise(0);
    load_body(ids[0], bd[0]);  // tile 3
    load_ids(ids[2]);          // tile 5
    decode(bd[1], 1);          // tile 1
    sync();
    normalise(1);
    u32x4 frag[2][KS];
#pragma unroll
    for (int s = 0; s < KS; s++) frag[0][s] = ring[0][s][lane];  // tile 0
    load_body(ids[1], bd[1]);  // tile 4
    load_ids(ids[0]);          // tile 6
    decode(bd[2], 2);          // tile 2

    float rmax[NB][2];
#pragma unroll
    for (int j = 0; j < NB; j++) rmax[j][0] = rmax[j][1] = NEG_INF;
    DocEnd<NB, false> doc_end;
    {
      const float no_scale[1][2] = {{1.f, 1.f}};
      doc_end.init(qv, no_scale, lane);
    }
    auto finish = [&]() {  // the document of wc ends with this tile
      doc_end.finish(rmax, wc.len < a.pad_len, lane, (int)(wc.b - b_begin), pend);
    };
    auto step = [&](auto slot) -> bool {
      constexpr int i = decltype(slot)::value;  // step index mod 6
      constexpr int k0 = i % NS, k1 = (i + 1) % NS, k2 = (i + 2) % NS;
      constexpr int f = i & 1;
      sync();
#pragma unroll
      for (int s = 0; s < KS; s++) frag[f ^ 1][s] = ring[k1][s][lane];  // tile i+1
      load_ids(ids[k1]);           // tile i+7 (the slot of tile i+4, whose body is loaded)
      load_body(ids[k2], bd[k2]);  // tile i+5 (the slot of tile i+2, decoded)
      normalise(k2);               // tile i+2
      decode(bd[k0], k0);          // tile i+3
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
          for (int h = 0; h < 2; h++) acc[j][h] = mfma16x16x32<TMS_DTYPE_F16>(t[s], qf[j][s][h], acc[j][h]);
      __builtin_amdgcn_s_setprio(0);
#pragma unroll
      for (int j = 0; j < NB; j++)
#pragma unroll
        for (int h = 0; h < 2; h++)
          rmax[j][h] = fmaxf(fmaxf(fmaxf(fmaxf(rmax[j][h], acc[j][h][0]), acc[j][h][1]), acc[j][h][2]), acc[j][h][3]);
      if (wc.t0 + 16 >= wc.len) finish();
      advance(wc, true);
      return wc.b >= b_end;
    };
    while (true) {
      if (step(RingSlot<0>{})) break;
      if (step(RingSlot<1>{})) break;
      if (step(RingSlot<2>{})) break;
      if (step(RingSlot<3>{})) break;
      if (step(RingSlot<4>{})) break;
      if (step(RingSlot<5>{})) break;
    }
  };
  if (wc.b < b_end) {
    if (decoder) pipeline(RingSlot<1>{});
    else pipeline(RingSlot<0>{});
  }

  // coalesced store: lane i writes document b_begin + i for each of the wave's queries
  if (my_nblk > 0 && lane < ndocs) {
    const int64_t b = b_begin + lane;
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < NB; j++) {
      if (j >= my_nblk) break;
      const int jb = my_blk0 + j;
      const int qi = jb / a.nbq;
      s += pend[j];
      if (j == my_nblk - 1 || (jb + 1) / a.nbq != qi) {  // the query's last block
        float* o = a.out + (int64_t)qi * a.B + b;
        if (dlen < 0) store_nan_score(o);  // invalid pid or offsets
        else *o = s;
        s = 0.f;
      }
    }
  }
}

// ---------------------------------------------------------------------------------
// Decompression: 16 lanes per token (lane k owns dimensions 8k .. 8k+7), four tokens
// per wave. Writes x = fp16(v / fp16(|v|)) with fp32 division, as the codec computes.
template <int NBITS>
__global__ void __launch_bounds__(256) residual_decompress_kernel(ResArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t lut[4096];
  build_lut<NBITS>(lut, a.weights);
  __syncthreads();
  const int k = threadIdx.x & 15;
  const int64_t t = (int64_t)blockIdx.x * (blockDim.x >> 4) + (threadIdx.x >> 4);
  const bool live = t < a.T && 8 * k < a.d;
  const int64_t tt = t < a.T ? t : a.T - 1;
  int64_t code = a.codes[tt];
  code = code < 0 ? 0 : (code >= a.ncent ? a.ncent - 1 : code);
  const int kk = 8 * k < a.d ? k : 0;
  const u32x4 c = *(const u32x4*)(a.centroids + (code * a.d + 8 * kk) * 2);
  const uint32_t rw = load_res<NBITS>(a.residuals + tt * a.rb, kk);
  float n2 = 0.f;
  const u32x4 v = add_chunk(c, chunk_weights<NBITS>(lut, rw), n2);
  if (!live) n2 = 0.f;
  n2 += __shfl_xor(n2, 1);
  n2 += __shfl_xor(n2, 2);
  n2 += __shfl_xor(n2, 4);
  n2 += __shfl_xor(n2, 8);
  float n = (float)(_Float16)sqrtf(n2);
  n = fmaxf(n, 5.9604645e-8f);
  u32x4 x;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t vi = v[i];
    const f16x2 p = as_f16x2(vi);
    f16x2 q;
    q.x = (_Float16)((float)p.x / n);
    q.y = (_Float16)((float)p.y / n);
    x[i] = as_u32(q);
  }
  if (live) *(u32x4*)((uint8_t*)a.out + (t * a.d + 8 * k) * 2) = x;
}

__global__ void residual_fill_kernel(float* out, int64_t n, float v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = v;
}

// ---------------------------------------------------------------------------------
// host side
#ifndef TMS_RES_TOKENS_PER_WAVE
#define TMS_RES_TOKENS_PER_WAVE 768  // document tokens one wave streams (rounded to whole documents)
#endif
static int check_format(const char* fn, int64_t d, int nbits, int64_t ncent, const void* centroids,
                        const void* weights) {
  if (nbits != 1 && nbits != 2 && nbits != 4)
    return fail(TMS_ERR_UNSUPPORTED, "%s: nbits=%d (supported: 1, 2, 4)", fn, nbits);
  if (d <= 0 || d > 128 || d % 32 != 0)
    return fail(TMS_ERR_UNSUPPORTED, "%s: d=%lld (supported: 32, 64, 96, 128)", fn, (long long)d);
  if (ncent <= 0) return fail(TMS_ERR_INVALID, "%s: no centroids", fn);
  if (!centroids || !weights) return fail(TMS_ERR_INVALID, "%s: centroids / bucket_weights is NULL", fn);
  if (((uintptr_t)centroids & 15) != 0) return fail(TMS_ERR_INVALID, "%s: centroids must be 16-byte aligned", fn);
  return TMS_OK;
}

#ifndef TMS_RES_QLDS
#define TMS_RES_QLDS 1  // query fragments in LDS
#endif
#ifndef TMS_RES_BATCHED_TOKENS
#define TMS_RES_BATCHED_TOKENS 4096  // document tokens one batched workgroup walks (whole documents)
#endif
// One residual load per token when the lane's run of KS*nbits bytes is a power of two and
// the residuals pointer is aligned to it (rows are 4*KS*nbits bytes, so every run is).
template <int KS, int NBITS, bool SPLIT>
static void launch_fused_split(const ResArgs& a, int64_t grid, hipStream_t st) {
  constexpr int kNSub = 1;
  constexpr bool kQlds = TMS_RES_QLDS;
  constexpr int TB = NBITS * KS;
  if constexpr (res_run_pow2<NBITS, KS>()) {
    if (((uintptr_t)a.residuals % TB) == 0) {
      hipLaunchKernelGGL((residual_maxsim_kernel<KS, NBITS, kNSub, kQlds, true, SPLIT>), dim3((unsigned)grid),
                         dim3(256), 0, st, a);
      return;
    }
  }
  hipLaunchKernelGGL((residual_maxsim_kernel<KS, NBITS, kNSub, kQlds, false, SPLIT>), dim3((unsigned)grid), dim3(256),
                     0, st, a);
}
template <int KS, int NBITS>
static void launch_fused_nbits(const ResArgs& a, int64_t grid, hipStream_t st) {
  if (a.wpd > 1) launch_fused_split<KS, NBITS, true>(a, grid, st);
  else launch_fused_split<KS, NBITS, false>(a, grid, st);
}
template <int KS>
static int launch_fused_ks(const ResArgs& a, int nbits, int64_t grid, hipStream_t st) {
  if (nbits == 1) launch_fused_nbits<KS, 1>(a, grid, st);
  else if (nbits == 2) launch_fused_nbits<KS, 2>(a, grid, st);
  else launch_fused_nbits<KS, 4>(a, grid, st);
  return check_launch("residual_maxsim_kernel");
}

template <int KS, int NB>
static int launch_batched_nb(const ResArgs& a, int nbits, int64_t grid, hipStream_t st) {
  const dim3 blk(64 * kResBatchedWaves);
  if (nbits == 1) hipLaunchKernelGGL((residual_batched_kernel<KS, 1, NB>), dim3((unsigned)grid), blk, 0, st, a);
  else if (nbits == 2) hipLaunchKernelGGL((residual_batched_kernel<KS, 2, NB>), dim3((unsigned)grid), blk, 0, st, a);
  else hipLaunchKernelGGL((residual_batched_kernel<KS, 4, NB>), dim3((unsigned)grid), blk, 0, st, a);
  return check_launch("residual_batched_kernel");
}
constexpr int kResMaxBlocksPerWave = 4;
template <int KS>
static int launch_batched_ks(const ResArgs& a, int nbits, int nb, int64_t grid, hipStream_t st) {
  switch (nb) {
    case 1: return launch_batched_nb<KS, 1>(a, nbits, grid, st);
    case 2: return launch_batched_nb<KS, 2>(a, nbits, grid, st);
    default: return launch_batched_nb<KS, kResMaxBlocksPerWave>(a, nbits, grid, st);
  }
}

// Arguments shared by the two MaxSim entry points; returns TMS_OK with `a` filled, or an
// error (or a negative value: nothing to launch, scores already written or none asked).
static int prep_maxsim(const char* fn, const void* Q, int64_t nQ, int64_t nq, int64_t d, const void* centroids,
                       int64_t ncent, const void* bucket_weights, int nbits, const int32_t* codes,
                       const uint8_t* residuals, int64_t total_tokens, const int64_t* offsets, int64_t ndocs,
                       const int64_t* pids, int64_t B, int64_t pad_len, float* out, hipStream_t st, ResArgs& a) {
  if (nQ < 0 || nq < 0 || d < 0 || ncent < 0 || total_tokens < 0 || ndocs < 0 || B < 0 || pad_len < 0)
    return fail(TMS_ERR_INVALID, "%s: negative size", fn);
  int rc = check_format(fn, d, nbits, ncent, centroids, bucket_weights);
  if (rc) return rc;
  if (B == 0 || nQ == 0) return -1;
  if (!out) return fail(TMS_ERR_INVALID, "%s: out is NULL", fn);
  if (!pids && B > ndocs) return fail(TMS_ERR_INVALID, "%s: B=%lld > ndocs=%lld without pids", fn, (long long)B,
                                      (long long)ndocs);
  if (!offsets) return fail(TMS_ERR_INVALID, "%s: offsets is NULL", fn);
  if (nq == 0) {
    const int64_t n = nQ * B;
    hipLaunchKernelGGL(residual_fill_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, out, n, 0.f);
    rc = check_launch("residual_fill_kernel");
    return rc ? rc : -1;
  }
  if (!Q) return fail(TMS_ERR_INVALID, "%s: Q is NULL", fn);
  if (total_tokens > 0 && (!codes || !residuals)) return fail(TMS_ERR_INVALID, "%s: codes / residuals is NULL", fn);
  if (((uintptr_t)Q & 15) != 0) return fail(TMS_ERR_INVALID, "%s: Q must be 16-byte aligned", fn);
  if ((((uintptr_t)residuals) & (nbits - 1)) != 0)
    return fail(TMS_ERR_INVALID, "%s: residuals must be %d-byte aligned", fn, nbits);
  if (nq > ((int64_t)1 << 24)) return fail(TMS_ERR_UNSUPPORTED, "%s: too many query tokens", fn);
  memset(&a, 0, sizeof(a));
  a.Q = (const uint8_t*)Q;
  a.centroids = (const uint8_t*)centroids;
  a.codes = codes;
  a.residuals = residuals;
  a.offsets = offsets;
  a.pids = pids;
  a.weights = (const uint16_t*)bucket_weights;
  a.out = out;
  a.B = B;
  a.ndocs = ndocs;
  a.T = total_tokens;
  a.ncent = ncent;
  a.pad_len = pad_len;
  a.nq = (int32_t)nq;
  a.nbq = (int32_t)((nq + 31) / 32);
  a.d = (int32_t)d;
  a.rb = (int32_t)(d * nbits / 8);
  return TMS_OK;
}

}  // namespace tms

extern "C" {

int tms_residual_decompress(const int32_t* codes, const uint8_t* residuals, int64_t T, const void* centroids,
                            int64_t ncent, int64_t d, const void* bucket_weights, int nbits, void* out, void* stream) {
  using namespace tms;
  const char* fn = "tms_residual_decompress";
  if (T < 0 || d < 0 || ncent < 0) return fail(TMS_ERR_INVALID, "%s: negative size", fn);
  int rc = check_format(fn, d, nbits, ncent, centroids, bucket_weights);
  if (rc) return rc;
  if (T == 0) return TMS_OK;
  if (!codes || !residuals || !out) return fail(TMS_ERR_INVALID, "%s: NULL pointer", fn);
  if (((uintptr_t)out & 15) != 0) return fail(TMS_ERR_INVALID, "%s: out must be 16-byte aligned", fn);
  if ((((uintptr_t)residuals) & (nbits - 1)) != 0)
    return fail(TMS_ERR_INVALID, "%s: residuals must be %d-byte aligned", fn, nbits);
  ResArgs a;
  memset(&a, 0, sizeof(a));
  a.centroids = (const uint8_t*)centroids;
  a.codes = codes;
  a.residuals = residuals;
  a.weights = (const uint16_t*)bucket_weights;
  a.out = (float*)out;
  a.T = T;
  a.ncent = ncent;
  a.d = (int32_t)d;
  a.rb = (int32_t)(d * nbits / 8);
  const int64_t grid = (T + 15) / 16;
  hipStream_t st = (hipStream_t)stream;
  if (nbits == 1) hipLaunchKernelGGL(residual_decompress_kernel<1>, dim3((unsigned)grid), dim3(256), 0, st, a);
  else if (nbits == 2) hipLaunchKernelGGL(residual_decompress_kernel<2>, dim3((unsigned)grid), dim3(256), 0, st, a);
  else hipLaunchKernelGGL(residual_decompress_kernel<4>, dim3((unsigned)grid), dim3(256), 0, st, a);
  return check_launch("residual_decompress_kernel");
}

int tms_maxsim_residual(const void* Q, int64_t nq, int64_t d, const void* centroids, int64_t ncent,
                        const void* bucket_weights, int nbits, const int32_t* codes, const uint8_t* residuals,
                        int64_t total_tokens, const int64_t* offsets, int64_t ndocs, const int64_t* pids, int64_t B,
                        int64_t pad_len, float* out, void* stream) {
  using namespace tms;
  hipStream_t st = (hipStream_t)stream;
  ResArgs a;
  int rc = prep_maxsim("tms_maxsim_residual", Q, 1, nq, d, centroids, ncent, bucket_weights, nbits, codes, residuals,
                       total_tokens, offsets, ndocs, pids, B, pad_len, out, st, a);
  if (rc) return rc < 0 ? TMS_OK : rc;
  // about TMS_RES_TOKENS_PER_WAVE tokens per wave (whole documents), at least two rounds
  // of the chip's resident waves
  const int64_t hint = ndocs > 0 ? total_tokens / ndocs : 1;
  int64_t dpw = hint > 0 ? TMS_RES_TOKENS_PER_WAVE / hint : 1;
  if (dpw > 1 && B / dpw < (int64_t)256 * 16 * 2) dpw = B / ((int64_t)256 * 16 * 2);
  if (dpw < 1) dpw = 1;
  if (dpw > 64) dpw = 64;  // one lane per document holds its bounds
  a.docs_per_wave = (int32_t)dpw;
  // Small calls (PLAID's final stage scores about 64 .. 1,024 candidates per query):
  // documents split over up to four waves while the call still fits the waves the chip
  // holds at once (three per SIMD at this kernel's registers), at most one wave per
  // tile of an average document.
  a.wpd = 1;
  const int64_t tiles = (hint + 15) / 16;
  if (rerank_fits(B, hint))  // the dense entry points' small-batch limit (tms_set_rerank_limit)
    while (a.wpd < 4 && B * a.wpd * 2 <= TMS_RES_SPLIT_WAVES && 2 * a.wpd <= tiles) a.wpd *= 2;
  if (a.wpd > 1) a.docs_per_wave = 1;
  const int64_t grid = a.wpd > 1 ? (B * a.wpd + 3) / 4 : ((B + dpw - 1) / dpw + 3) / 4;
  for (int blk = 0; blk < a.nbq; blk++) {
    a.blk0 = blk;
    switch (d / 32) {
      case 1: rc = launch_fused_ks<1>(a, nbits, grid, st); break;
      case 2: rc = launch_fused_ks<2>(a, nbits, grid, st); break;
      case 3: rc = launch_fused_ks<3>(a, nbits, grid, st); break;
      default: rc = launch_fused_ks<4>(a, nbits, grid, st); break;
    }
    if (rc) return rc;
  }
  return TMS_OK;
}

int tms_maxsim_residual_batched(const void* Qs, int64_t nQ, int64_t nq, int64_t d, const void* centroids,
                                int64_t ncent, const void* bucket_weights, int nbits, const int32_t* codes,
                                const uint8_t* residuals, int64_t total_tokens, const int64_t* offsets, int64_t ndocs,
                                const int64_t* pids, int64_t B, int64_t pad_len, float* out, void* stream) {
  using namespace tms;
  const char* fn = "tms_maxsim_residual_batched";
  hipStream_t st = (hipStream_t)stream;
  ResArgs a;
  int rc = prep_maxsim(fn, Qs, nQ, nq, d, centroids, ncent, bucket_weights, nbits, codes, residuals, total_tokens,
                       offsets, ndocs, pids, B, pad_len, out, st, a);
  if (rc) return rc < 0 ? TMS_OK : rc;
  const int64_t nblocks = nQ * (int64_t)a.nbq;
  if (a.nbq > kResMaxBlocksPerWave || nblocks < 2) {  // one query at a time
    for (int64_t qi = 0; qi < nQ; qi++) {
      rc = tms_maxsim_residual((const uint8_t*)Qs + qi * nq * d * 2, nq, d, centroids, ncent, bucket_weights, nbits,
                               codes, residuals, total_tokens, offsets, ndocs, pids, B, pad_len, out + qi * B, stream);
      if (rc) return rc;
    }
    return TMS_OK;
  }
  if (nblocks > ((int64_t)1 << 30)) return fail(TMS_ERR_UNSUPPORTED, "%s: too many queries", fn);
  // Blocks per wave: the smallest of 1, 2, 4 whose launch covers every block in one pass
  // (a wave computes all of its slots, used or not), else 4. A wave holds whole queries.
  int nb = kResMaxBlocksPerWave;
  for (int c = 1; c < kResMaxBlocksPerWave; c *= 2)
    if (c >= a.nbq && nblocks <= (int64_t)kResBatchedWaves * ((c / a.nbq) * a.nbq)) {
      nb = c;
      break;
    }
  a.nblk = (nb / a.nbq) * a.nbq;
  // about TMS_RES_BATCHED_TOKENS tokens per workgroup (whole documents, at most 64), at
  // least four rounds of one workgroup per CU
  const int64_t hint = ndocs > 0 ? total_tokens / ndocs : 1;
  int64_t dpw = hint > 0 ? TMS_RES_BATCHED_TOKENS / hint : 1;
  if (dpw > 1 && B / dpw < (int64_t)256 * 4) dpw = B / ((int64_t)256 * 4);
  if (dpw < 1) dpw = 1;
  if (dpw > 64) dpw = 64;
  a.docs_per_wave = (int32_t)dpw;
  const int64_t grid = (B + dpw - 1) / dpw;
  if (grid > 0x7fffffff) return fail(TMS_ERR_UNSUPPORTED, "%s: too many documents", fn);
  const int64_t per_launch = (int64_t)kResBatchedWaves * a.nblk;
  for (int64_t b0 = 0; b0 < nblocks; b0 += per_launch) {
    a.blk0 = (int32_t)b0;
    a.blk_end = (int32_t)(nblocks - b0 < per_launch ? nblocks : b0 + per_launch);
    switch (d / 32) {
      case 1: rc = launch_batched_ks<1>(a, nbits, nb, grid, st); break;
      case 2: rc = launch_batched_ks<2>(a, nbits, nb, grid, st); break;
      case 3: rc = launch_batched_ks<3>(a, nbits, nb, grid, st); break;
      default: rc = launch_batched_ks<4>(a, nbits, nb, grid, st); break;
    }
    if (rc) return rc;
  }
  return TMS_OK;
}

}  // extern "C"
