// Dense MaxSim, d <= 128, query fragments in VGPRs, over fixed-length documents or
// documents at offsets: the streaming kernel with a control-flow shape the compiler's
// memory-counter tracking follows exactly.
//
// The general kernel (tms_dense.hip) walks documents with a cursor whose branches make
// the compiler drain every outstanding load before each tile. Here:
//  * a wave's tiles are a flat sequence; each document is padded to a multiple of
//    R = PFD + 1 tiles with clamped duplicates of its last token (a duplicate cannot
//    change a max), so every document starts at ring slot 0; with offsets, lane j holds
//    document j's first row and length and the walk reads them with readlane;
//  * the inner loop body is straight-line and unrolled R times: it issues the loads of
//    tile g + PFD (index clamped to the last tile, so the count never varies) and scores
//    tile g from the ring; the per-document reduction sits between inner loops;
//  * scores are staged in registers (lane i holds document i of the wave's run) and
//    stored once, coalesced, after the loop.
// Every wave streams its own documents with the same (one or two) query blocks. Batched
// queries use batched_tile_kernel below, whose workgroups share tiles through LDS (for
// fixed-length documents at implicit offsets b * nd).
//
// Semantics as tms_dense.hip: fp32 accumulation, query rows past nq contribute 0, an
// empty document scores -inf.
#include <string.h>

#include "tms_common.h"

namespace tms {

struct StreamArgs {
  const uint8_t* Q;          // (nQ * nq, d)
  const uint8_t* D;          // fixed length: (B, nd, d); variable length: (T, d)
  const int64_t* offsets;    // variable length: (B + 1)
  float* out;                // (nQ, B)
  int64_t B, nd, T, pad_len;  // pad_len > 0 (variable length): score as if zero-padded to it
  int32_t nq, nbq;           // tokens per query, 32-token blocks per query
  int32_t blk0;              // first global query block of this launch
  int32_t blk_end;           // one past the last block of this launch
  int32_t nblk;              // blocks per wave
  int32_t d;                 // 32 * KS
  int32_t docs_per_wave;     // documents per wave; <= 64
};

// VARLEN: documents at offsets (T >= 1 rows). Lane j of a wave holds its document j's first
// row and length, which the walk reads with readlane, so the tile sequence stays
// straight-line as for fixed lengths. An empty document, or one with invalid offsets,
// takes R tiles of row 0 whose maxima are dropped: its score is -inf (0 when padded),
// or NaN for invalid offsets.
template <int DT, int KS, int NB, int PFD, bool VARLEN>
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

  // VARLEN: lane j holds document b_begin + j's first row (0 if it has no rows) and its
  // length (-1: invalid offsets).
  int64_t dbase = 0;
  int32_t dlen = 0;
  if constexpr (VARLEN) {
    dlen = -1;
    if (lane < ndocs) {
      const int64_t b = b_begin + lane;
      const int64_t s0 = a.offsets[b], e0 = a.offsets[b + 1];
      if (s0 >= 0 && e0 >= s0 && e0 <= a.T && e0 - s0 <= 0x7fffffff) {
        dlen = (int32_t)(e0 - s0);
        dbase = dlen > 0 ? s0 : 0;
      }
    }
  }
  auto doc_len = [&](int64_t dd) -> int64_t {
    if constexpr (VARLEN) return (int32_t)__builtin_amdgcn_readlane((uint32_t)dlen, (int)dd);
    else return a.nd;
  };
  auto doc_base = [&](int64_t dd) -> int64_t {
    if constexpr (VARLEN) {
      const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)dbase, (int)dd);
      const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)((uint64_t)dbase >> 32), (int)dd);
      return (int64_t)(((uint64_t)hi << 32) | lo);
    } else {
      return (b_begin + dd) * a.nd;
    }
  };
  // tiles of a document of `len` rows, padded to a multiple of R (at least R)
  auto doc_tiles = [&](int64_t len) -> int64_t {
    const int64_t t = len > 0 ? (len + 15) / 16 : 1;
    return (t + R - 1) / R * R;
  };

  float pend[NB];
#pragma unroll
  for (int j = 0; j < NB; j++) pend[j] = NEG_INF;

  if (VARLEN || a.nd > 0) {
    const int64_t tpd = doc_tiles(a.nd);  // fixed length: tiles per document
    int64_t total;                        // tiles of the wave's documents
    if constexpr (VARLEN) {  // 64-bit: documents may overlap, each up to 2^31 rows
      int64_t n = lane < ndocs ? doc_tiles(dlen) : 0;
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) n += __shfl_xor(n, o);
      const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)n);
      const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)n >> 32));
      total = (int64_t)(((uint64_t)hi << 32) | lo);
    } else {
      total = ndocs * tpd;
    }
    const int64_t row_bytes = (int64_t)a.d * 2;
    // LINES (rows of 128 or 256 bytes): each load covers whole 128-byte lines of eight rows
    // (line_frags); lane 16 g + 8 s + t reads bytes 64 s + 16 g of a line of row t or 8 + t.
    // Otherwise lane (r, g) reads chunk 4 s + g of row r, a quarter line per load.
    constexpr bool LINES = KS % 2 == 0;
    const int t8 = lane & 7;
    const uint8_t* base = a.D + (LINES ? (int64_t)(64 * ((lane >> 3) & 1) + 16 * g) : (int64_t)(8 * g) * 2);

    // Address of a token row of tile (document dd of the wave, tile t): row i of the
    // tile, clamped to the document's last row (row 0 for a document without rows).
    int64_t c_base = doc_base(0), c_len = doc_len(0);  // the prefetch cursor's document
    auto tile_ptr = [&](int64_t t, int i) -> const uint8_t* {
      int64_t tok = t * 16 + i;
      const int64_t last = c_len > 0 ? c_len - 1 : 0;
      if (tok > last) tok = last;
      return base + (c_base + tok) * row_bytes;
    };
    // Prefetch cursor: tile index pf (tile pt of document pd), saturating at the last tile
    // (the prefetches past the end re-read it, so each iteration issues KS loads).
    int64_t pd = 0, pt = 0, pf = 0, c_tiles = VARLEN ? doc_tiles(c_len) : tpd;
    auto pf_next = [&]() {
      const bool more = pf < total - 1;
      pf += more ? 1 : 0;
      pt += more ? 1 : 0;
      const bool wrap = pt == c_tiles;
      pt = wrap ? 0 : pt;
      pd += wrap ? 1 : 0;
      if constexpr (VARLEN) {  // pd < ndocs: the cursor stops at the last tile
        c_base = doc_base(pd);
        c_len = doc_len(pd);
        c_tiles = doc_tiles(c_len);
      } else {
        c_base = (b_begin + pd) * a.nd;
      }
    };

    u32x4 ring[R][KS];
    auto load = [&](u32x4 (&buf)[KS]) {
      if constexpr (LINES) {  // buf[2i], buf[2i+1]: line i of rows t and 8 + t
        const uint8_t* p0 = tile_ptr(pt, t8);
        const uint8_t* p1 = tile_ptr(pt, 8 + t8);
#pragma unroll
        for (int i = 0; i < KS / 2; i++) {
          buf[2 * i] = ld_stream<u32x4, true>(p0 + 128 * i);
          buf[2 * i + 1] = ld_stream<u32x4, true>(p1 + 128 * i);
        }
      } else {
        const uint8_t* p = tile_ptr(pt, r);
#pragma unroll
        for (int s = 0; s < KS; s++) buf[s] = ld_stream<u32x4, false>(p + 64 * s);
      }
    };
#pragma unroll
    for (int k = 0; k < PFD; k++) {
      load(ring[k]);
      pf_next();
    }

    float rmax[NB][2];
    auto score = [&](const u32x4 (&raw)[KS]) {
      u32x4 buf[KS];  // A-operand fragments: chunk 4 s + g of row r
      if constexpr (LINES) {
#pragma unroll
        for (int i = 0; i < KS / 2; i++) line_frags(raw[2 * i], raw[2 * i + 1], buf[2 * i], buf[2 * i + 1]);
      } else {
#pragma unroll
        for (int s = 0; s < KS; s++) buf[s] = raw[s];
      }
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
      const int64_t len = doc_len(dd);
      const int64_t nt = VARLEN ? doc_tiles(len) : tpd;
      for (int64_t t = 0; t < nt; t += R) {
#pragma unroll
        for (int k = 0; k < R; k++) {
          load(ring[(k + PFD) % R]);
          pf_next();
          score(ring[k]);
        }
      }
      // document done: max over the 64 rows of each column, sum over query tokens
      const bool padded = VARLEN && len < a.pad_len;  // zero padding adds dot products of 0
      float blk[NB];
#pragma unroll
      for (int j = 0; j < NB; j++) {
        float s = 0.f;
#pragma unroll
        for (int h = 0; h < 2; h++) {
          float m = rmax[j][h];
          m = fmaxf(m, __shfl_xor(m, 16));
          m = fmaxf(m, __shfl_xor(m, 32));
          if (padded) m = fmaxf(m, 0.f);
          int64_t row;
          s += q_valid(j, h, row) ? m : 0.f;
        }
        s += __shfl_xor(s, 8);
        s += __shfl_xor(s, 4);
        s += __shfl_xor(s, 2);
        s += __shfl_xor(s, 1);
        if (VARLEN && len <= 0) s = a.pad_len > 0 ? 0.f : NEG_INF;  // no rows (the tiles read row 0)
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
        if (VARLEN && dlen < 0) store_nan_score(o);  // invalid offsets
        else *o = (qi * a.nbq < my_blk0) ? *o + s : s;
        s = 0.f;
      }
    }
  }
}

template <int K>
struct RingSlotS {
  static constexpr int value = K;
};

#ifndef TMS_STREAM_PFD
#define TMS_STREAM_PFD 2  // tiles in flight ahead of the one being scored (single-query path)
#endif
#ifndef TMS_STREAM_MIN_WAVES
#define TMS_STREAM_MIN_WAVES (256 * 16 * 2)  // fewer documents per wave below this many waves
#endif
#ifndef TMS_STREAM_TOKENS_PER_WAVE
#define TMS_STREAM_TOKENS_PER_WAVE 768  // document tokens one wave streams (rounded to whole documents)
#endif

template <int DT, int KS, int NB>
static int stream_launch(const StreamArgs& a, int64_t grid, hipStream_t st) {
  if (a.offsets)
    hipLaunchKernelGGL((stream_maxsim_kernel<DT, KS, NB, TMS_STREAM_PFD, true>), dim3((unsigned)grid), dim3(256), 0,
                       st, a);
  else
    hipLaunchKernelGGL((stream_maxsim_kernel<DT, KS, NB, TMS_STREAM_PFD, false>), dim3((unsigned)grid), dim3(256), 0,
                       st, a);
  return check_launch("stream_maxsim_kernel");
}

#ifndef TMS_BATCHED_WAVES
#define TMS_BATCHED_WAVES 8  // waves per workgroup (one workgroup per CU) in the batched kernel
#endif
constexpr int kMaxBlocksPerWave = 4;  // query blocks held in VGPRs per wave there: 1, 2 or 4

template <int DT, int NB>
static int stream_ks(const StreamArgs& a, int64_t grid, hipStream_t st) {
  switch (a.d / 32) {
    case 1: return stream_launch<DT, 1, NB>(a, grid, st);
    case 2: return stream_launch<DT, 2, NB>(a, grid, st);
    case 3: return stream_launch<DT, 3, NB>(a, grid, st);
    default: return stream_launch<DT, 4, NB>(a, grid, st);
  }
}

// ---------------------------------------------------------------------------------
// Batched queries: many query blocks share each document tile through LDS. One workgroup
// of eight waves per CU (two per SIMD) walks a run of at most 64 documents (document b is
// rows [offsets[b], offsets[b+1]) of D, or [b nd, (b+1) nd) for fixed-length documents)
// in 16-token tiles, every wave the same tiles; the last tile of a document repeats its
// last token, which cannot change a max. Wave w holds a.nblk query blocks (whole
// queries) in VGPRs, so one pass over D serves up to 8 * a.nblk blocks. Wave w < KS
// loads k-step w of each tile (lane (r, g): chunk 4 w + g of token r, the MFMA A-operand
// layout) NS tiles ahead; step i writes tile i+1 to the LDS ring, passes one LDS-only
// barrier (the loads in flight are not waited for), reads tile i+1's fragments and
// scores tile i. The MFMA cluster runs at raised wave priority, so a wave that has its
// operands keeps the matrix pipe fed ahead of the other wave's bookkeeping; the running
// max takes two v_max3 per fragment and each document's reduction uses the row swaps and
// DPP. pad_len > 0 gives the zero-padding semantics of tms_maxsim_varlen_padded; invalid
// offsets score NaN.
struct BatchedArgs {
  const uint8_t* Q;         // (nQ * nq, d)
  const uint8_t* D;         // (T, d) tokens, or (T, M) PQ codes
  const int64_t* offsets;   // (B + 1), or null: document b is rows [b * nd, (b + 1) * nd)
  const uint8_t* codebook;  // PQ: (M, K, dsub) elements of the input dtype
  float* out;               // (nQ, B)
  int64_t B, T, pad_len, nd;
  int32_t nq, nbq, blk0, blk_end, nblk, d, docs_per_wg, M, K;
};

// Tile sources. A loading wave fetches, per tile, the raw data of its lane's 8-dimension
// chunk c of token `row`; the source turns it into the MFMA A-operand fragment.
// Each tile chunk goes to the LDS ring as kParts 16-byte MFMA fragments: the fragment
// itself, or (fp32 rows) its bf16 hi and lo terms.
struct DenseTiles {  // fp16 / bf16 rows, stored to the ring as loaded
  static constexpr bool kDirect = true;
  static constexpr int kParts = 1;
  static constexpr bool kQ32 = false;  // queries of the rows' type
  typedef u32x4 Raw;
  __device__ static Raw load(const BatchedArgs& a, int64_t row, int c) {
    return *(const u32x4*)(a.D + row * a.d * 2 + 16 * c);
  }
  __device__ static u32x4 decode(const u32x4*, int, Raw raw, int) { return raw; }
  __device__ static void parts(const Raw& raw, u32x4 (&out)[1]) { out[0] = raw; }
};
// fp16 / bf16 rows scored against fp32 queries: each query element is split into hi + lo
// terms of the rows' type (fp16 after the token's power-of-two scale, split_f16) and a
// product takes two MFMAs, d*q_lo + d*q_hi, as in the per-query kernels: the query is
// never rounded to 16 bits.
struct DenseTilesQ32 : DenseTiles {
  static constexpr bool kQ32 = true;
};
// fp32 rows (and fp32 queries): every element split into bf16 hi + lo terms as it goes
// to the ring, a product formed from three bf16 MFMAs (lo*q_hi + hi*q_lo + hi*q_hi, the
// per-query fp32 kernel's order), as in tms_dense_kernel.h.
struct F32Tiles {
  static constexpr bool kDirect = true;
  static constexpr int kParts = 2;
  static constexpr bool kQ32 = true;
  typedef u32x8 Raw;
  __device__ static Raw load(const BatchedArgs& a, int64_t row, int c) {
    const u32x4* p = (const u32x4*)(a.D + row * a.d * 4 + 32 * c);
    const u32x4 x0 = p[0], x1 = p[1];
    return Raw{x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
  }
  __device__ static void parts(const Raw& raw, u32x4 (&out)[2]) { split_bf16(raw, out[0], out[1]); }
};
// uint8 PQ codes (M per token), decoded through the codebook held in LDS: chunk c covers
// subspaces 8c / DSUB .. (8c + 7) / DSUB. Codes >= K are clamped into the table.
template <int DSUB>
struct PqTiles {
  static constexpr bool kDirect = false;
  static constexpr int kParts = 1;
  static constexpr bool kQ32 = false;
  typedef uint32_t Raw;
  __device__ static Raw load(const BatchedArgs& a, int64_t row, int c) {
    const uint8_t* p = a.D + row * a.M;
    if constexpr (DSUB == 8) return p[c];
    else if constexpr (DSUB == 4) return *(const uint16_t*)(p + 2 * c);
    else if constexpr (DSUB == 2) return *(const uint32_t*)(p + 4 * c);
    else return p[c / (DSUB / 8)];
  }
  __device__ static u32x4 decode(const u32x4* cb, int K, Raw raw, int c) {
    auto code = [&](int i) -> uint32_t {
      const uint32_t x = (raw >> (8 * i)) & 0xffu;
      return x < (uint32_t)K ? x : (uint32_t)K - 1u;
    };
    if constexpr (DSUB >= 8) {
      constexpr int P = DSUB / 8;  // 16-byte pieces per codeword
      return cb[((int64_t)(c / P) * K + code(0)) * P + c % P];
    } else if constexpr (DSUB == 4) {
      const uint2* cb8 = (const uint2*)cb;
      u32x4 v;
#pragma unroll
      for (int i = 0; i < 2; i++) {
        const uint2 x = cb8[(int64_t)(2 * c + i) * K + code(i)];
        v[2 * i] = x.x;
        v[2 * i + 1] = x.y;
      }
      return v;
    } else {
      const uint32_t* cb4 = (const uint32_t*)cb;
      u32x4 v;
#pragma unroll
      for (int i = 0; i < 4; i++) v[i] = cb4[(int64_t)(4 * c + i) * K + code(i)];
      return v;
    }
  }
};

template <int DT, int KS, int NB, class SRC>
__global__ void __launch_bounds__(64 * TMS_BATCHED_WAVES, 2) batched_tile_kernel(BatchedArgs a) {
  constexpr int NS = 4;  // LDS ring slots and load lead, in tiles
  constexpr int NP = SRC::kParts;
  constexpr bool SPLIT = NP == 2;        // fp32 rows and queries: DT is the MFMA type, bf16
  constexpr bool QLO = SRC::kQ32;        // fp32 queries: every query fragment has a lo term
  constexpr bool QSCALE = QLO && !SPLIT && DT == TMS_DTYPE_F16;  // fp16 terms of a scaled token
  static_assert(!SPLIT || DT == TMS_DTYPE_BF16, "split fp32 terms are bf16");
  __shared__ u32x4 ring[NS][NP][4][64];
  extern __shared__ u32x4 cb[];  // PQ codebook
  const int lane = threadIdx.x & 63;
  const int r = lane & 15, g = lane >> 4;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const float NEG_INF = -__builtin_inff();
  if constexpr (!SRC::kDirect) {  // codebook -> LDS (d * K elements, a multiple of 16 bytes)
    const int n16 = a.d * a.K * 2 / 16;
    for (int i = threadIdx.x; i < n16; i += 64 * TMS_BATCHED_WAVES) cb[i] = ((const u32x4*)a.codebook)[i];
    __syncthreads();
  }

  const int64_t b_begin = wave_uniform((int64_t)blockIdx.x * a.docs_per_wg);
  const int64_t b_end = (b_begin + a.docs_per_wg < a.B) ? b_begin + a.docs_per_wg : a.B;
  const int64_t ndocs = b_end - b_begin;  // >= 1: the host launches no empty workgroup

  const int my_blk0 = a.blk0 + wid * a.nblk;
  int my_nblk = a.blk_end - my_blk0;  // <= 0 for a wave with no query
  if (my_nblk > a.nblk) my_nblk = a.nblk;
  u32x4 qf[NB][KS][2];
  u32x4 qfl[QLO ? NB : 1][QLO ? KS : 1][2];  // fp32 queries: the lo terms
  float qinv[QSCALE ? NB : 1][2];           // QSCALE: 1 / the token's scale (a power of two)
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
      if constexpr (QLO) {
        u32x8 raw[KS];
        float am = 0.f;
#pragma unroll
        for (int s = 0; s < KS; s++) {
          const u32x4* p = (const u32x4*)(a.Q + (row * a.d + 8 * (4 * s + g)) * 4);
          const u32x4 x0 = p[0], x1 = p[1];
          raw[s] = qv[j][h] ? u32x8{x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]}
                            : u32x8{0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
          if constexpr (QSCALE) am = fmaxf(am, absmax8(raw[s]));
        }
        float sc = 1.f;
        if constexpr (QSCALE) {  // the token's chunks sit in lanes r, r+16, r+32, r+48
          am = fmaxf(am, __shfl_xor(am, 16));
          am = fmaxf(am, __shfl_xor(am, 32));
          sc = pow2_scale(am, qinv[j][h]);
        }
#pragma unroll
        for (int s = 0; s < KS; s++) {
          if constexpr (QSCALE) split_f16(raw[s], sc, qf[j][s][h], qfl[j][s][h]);
          else split_bf16(raw[s], qf[j][s][h], qfl[j][s][h]);
        }
      } else {
#pragma unroll
        for (int s = 0; s < KS; s++) {
          const u32x4 v = *(const u32x4*)(a.Q + (row * a.d + 8 * (4 * s + g)) * 2);
          qf[j][s][h] = qv[j][h] ? v : u32x4{0u, 0u, 0u, 0u};
        }
      }
    }

  // lane j holds document b_begin + j's first row and length (-1: invalid offsets)
  int64_t dbase = 0;
  int32_t dlen = -1;
  if (lane < ndocs) {
    const int64_t b = b_begin + lane;
    const int64_t s0 = a.offsets ? a.offsets[b] : b * a.nd, e0 = a.offsets ? a.offsets[b + 1] : (b + 1) * a.nd;
    if (s0 >= 0 && e0 >= s0 && e0 <= a.T && e0 - s0 <= 0x7fffffff) {
      dbase = s0;
      dlen = (int32_t)(e0 - s0);
    }
  }
  float pend[NB];  // lane j: scores of document b_begin + j
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
  // First document at or after b with a token; with `record`, the empty or invalid ones
  // passed on the way get their scores. Past the end the cursor keeps its last tile.
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
      if (record) {  // invalid offsets (len < 0): the final store writes NaN for the lane
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

  Cur wc, wl;  // scoring (tile i), loads (tile i + NS)
  wc.b = b_end;
  wc.base = 0;
  wc.len = 1;
  wc.t0 = 0;
  seek(wc, b_begin, true);

  // Instantiated for loading and non-loading waves, so each copy's loads are straight-line
  // code whose outstanding count the compiler tracks exactly.
  auto pipeline = [&](auto ld_tag) {
    constexpr bool LD = decltype(ld_tag)::value == 1;
    wl = wc;
    const int chunk = 4 * (LD ? wid : 0) + g;
    typedef typename SRC::Raw Raw;
    auto load = [&]() -> Raw {
      Raw v{};
      if constexpr (LD) {
        int32_t t = wl.t0 + r;
        if (t > wl.len - 1) t = wl.len - 1;
        v = SRC::load(a, wl.base + t, chunk);
      }
      advance(wl, false);
      return v;
    };
    auto sync = [&]() {  // LDS-only fence: the loads in flight are not waited for
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    };
    // Direct sources store tile i+1 from its load slot at step i; decoding sources decode
    // tile i+2 at step i into `ahead` (the LDS gathers overlap the step) and store it a
    // step later.
    Raw stg[NS];
    u32x4 ahead = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int t = 0; t < NS; t++) stg[t] = load();
    auto put = [&](int slot, const Raw& raw) {  // a direct source's tile to a ring slot
      u32x4 pv[NP];
      if constexpr (SRC::kDirect) SRC::parts(raw, pv);
#pragma unroll
      for (int p = 0; p < NP; p++) ring[slot][p][wid][lane] = pv[p];
    };
    if constexpr (LD) {
      if constexpr (SRC::kDirect) {
        put(0, stg[0]);
      } else {
        ring[0][0][wid][lane] = SRC::decode(cb, a.K, stg[0], chunk);
        ahead = SRC::decode(cb, a.K, stg[1], chunk);
      }
    }
    sync();
    u32x4 frag[2][NP][KS];
#pragma unroll
    for (int p = 0; p < NP; p++)
#pragma unroll
      for (int s = 0; s < KS; s++) frag[0][p][s] = ring[0][p][s][lane];
    float rmax[NB][2];
#pragma unroll
    for (int j = 0; j < NB; j++) rmax[j][0] = rmax[j][1] = NEG_INF;

    DocEnd<NB, QSCALE> doc_end;
    doc_end.init(qv, qinv, lane);

    auto step = [&](auto slot) -> bool {
      constexpr int i = decltype(slot)::value;  // step index mod NS
      constexpr int s1 = (i + 1) % NS;
      constexpr int f = i & 1;
      stg[i] = load();  // tile i + NS (stg[i] was tile i, in the ring since the last step)
      if constexpr (LD) {
        if constexpr (SRC::kDirect) {
          put(s1, stg[s1]);  // tile i+1
        } else {
          ring[s1][0][wid][lane] = ahead;                            // tile i+1
          ahead = SRC::decode(cb, a.K, stg[(i + 2) % NS], chunk);  // tile i+2
        }
      }
      sync();
#pragma unroll
      for (int p = 0; p < NP; p++)
#pragma unroll
        for (int s = 0; s < KS; s++) frag[f ^ 1][p][s] = ring[s1][p][s][lane];
      const u32x4(&t)[KS] = frag[f][0];
      const u32x4(&tl)[KS] = frag[f][NP - 1];  // SPLIT: the lo terms
      f32x4 acc[NB][2];
#pragma unroll
      for (int j = 0; j < NB; j++) acc[j][0] = acc[j][1] = f32x4{0.f, 0.f, 0.f, 0.f};
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int s = 0; s < KS; s++)
#pragma unroll
        for (int j = 0; j < NB; j++)
#pragma unroll
          for (int h = 0; h < 2; h++) {
            if constexpr (SPLIT) acc[j][h] = mfma16x16x32<DT>(tl[s], qf[j][s][h], acc[j][h]);
            if constexpr (QLO) acc[j][h] = mfma16x16x32<DT>(t[s], qfl[j][s][h], acc[j][h]);
            acc[j][h] = mfma16x16x32<DT>(t[s], qf[j][s][h], acc[j][h]);
          }
      __builtin_amdgcn_s_setprio(0);
#pragma unroll
      for (int j = 0; j < NB; j++)
#pragma unroll
        for (int h = 0; h < 2; h++)
          rmax[j][h] = fmaxf(fmaxf(fmaxf(fmaxf(rmax[j][h], acc[j][h][0]), acc[j][h][1]), acc[j][h][2]), acc[j][h][3]);
      if (wc.t0 + 16 >= wc.len) {  // document wc.b ends with this tile
        const bool padded = wc.len < a.pad_len;
        doc_end.finish(rmax, padded, lane, (int)(wc.b - b_begin), pend);
      }
      advance(wc, true);
      return wc.b >= b_end;
    };
    while (true) {
      if (step(RingSlotS<0>{})) break;
      if (step(RingSlotS<1>{})) break;
      if (step(RingSlotS<2>{})) break;
      if (step(RingSlotS<3>{})) break;
    }
  };
  if (wc.b < b_end) {
    if (wid < KS) pipeline(RingSlotS<1>{});
    else pipeline(RingSlotS<0>{});
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
        if (dlen < 0) store_nan_score(o);  // invalid offsets
        else *o = s;
        s = 0.f;
      }
    }
  }
}

template <int DT, int NB, class SRC>
static int batched_ks(const BatchedArgs& a, int64_t grid, size_t lds, hipStream_t st) {
  const dim3 blk(64 * TMS_BATCHED_WAVES);
  switch (a.d / 32) {
    case 1: hipLaunchKernelGGL((batched_tile_kernel<DT, 1, NB, SRC>), dim3((unsigned)grid), blk, lds, st, a); break;
    case 2: hipLaunchKernelGGL((batched_tile_kernel<DT, 2, NB, SRC>), dim3((unsigned)grid), blk, lds, st, a); break;
    case 3: hipLaunchKernelGGL((batched_tile_kernel<DT, 3, NB, SRC>), dim3((unsigned)grid), blk, lds, st, a); break;
    default: hipLaunchKernelGGL((batched_tile_kernel<DT, 4, NB, SRC>), dim3((unsigned)grid), blk, lds, st, a); break;
  }
  return check_launch("batched_tile_kernel");
}
// Query blocks a wave holds in VGPRs: 4 for 16-bit queries, 2 for fp32 ones (their hi
// and lo terms take twice the registers).
template <class SRC>
constexpr int batched_max_blocks() {
  return SRC::kQ32 ? 2 : kMaxBlocksPerWave;
}
template <int DT, class SRC>
static int batched_nb(int nb, const BatchedArgs& a, int64_t grid, size_t lds, hipStream_t st) {
  switch (nb) {
    case 1: return batched_ks<DT, 1, SRC>(a, grid, lds, st);
    case 2: return batched_ks<DT, 2, SRC>(a, grid, lds, st);
    default:
      if constexpr (batched_max_blocks<SRC>() > 2) return batched_ks<DT, kMaxBlocksPerWave, SRC>(a, grid, lds, st);
      else return fail(TMS_ERR_UNSUPPORTED, "batched MaxSim: %d query blocks per wave", nb);
  }
}
template <class SRC>
static int batched_dt(int dtype, int nb, const BatchedArgs& a, int64_t grid, size_t lds, hipStream_t st) {
  if constexpr (SRC::kParts == 2) return batched_nb<TMS_DTYPE_BF16, SRC>(nb, a, grid, lds, st);  // fp32
  else
    return dtype == TMS_DTYPE_F16 ? batched_nb<TMS_DTYPE_F16, SRC>(nb, a, grid, lds, st)
                                  : batched_nb<TMS_DTYPE_BF16, SRC>(nb, a, grid, lds, st);
}

// Blocks per wave and launches over the query blocks, shared by the entry points below:
// the smallest of 1, 2, 4 (at most max_nb) blocks per wave whose launch covers every block
// in one pass (a wave computes all of its slots, used or not), else max_nb; a wave holds
// whole queries.
template <class LAUNCH>
static int batched_launches(BatchedArgs& a, int64_t nQ, LAUNCH launch, int max_nb = kMaxBlocksPerWave) {
  const int64_t nblocks = nQ * (int64_t)a.nbq;
  int nb = max_nb;
  for (int c = 1; c < max_nb; c *= 2)
    if (c >= a.nbq && nblocks <= (int64_t)TMS_BATCHED_WAVES * ((c / a.nbq) * a.nbq)) {
      nb = c;
      break;
    }
  a.nblk = (nb / a.nbq) * a.nbq;
  const int64_t per_launch = (int64_t)TMS_BATCHED_WAVES * a.nblk;
  for (int64_t b0 = 0; b0 < nblocks; b0 += per_launch) {
    a.blk0 = (int32_t)b0;
    a.blk_end = (int32_t)(nblocks - b0 < per_launch ? nblocks : b0 + per_launch);
    const int rc = launch(nb);
    if (rc) return rc;
  }
  return TMS_OK;
}

#ifndef TMS_VARLEN_BATCHED_TOKENS
#define TMS_VARLEN_BATCHED_TOKENS 4096  // document tokens one workgroup walks (whole documents, at most 64)
#endif

// Batched-query entry (tms_dense.hip for variable-length documents and fp32 ones,
// run_stream for fixed 16-bit ones): d in {32, 64, 96, 128}, 16-byte aligned Q and D,
// queries of at most 4 blocks (2 for fp32 queries, q32: fp32 queries against 16-bit rows).
int run_varlen_batched(const void* Q, int64_t nQ, int64_t nq, int64_t d, const void* D, int64_t T,
                       const int64_t* offsets, int64_t nd, int64_t B, int64_t pad_len, int dtype, float* out,
                       hipStream_t st, bool q32) {
  BatchedArgs a;
  memset(&a, 0, sizeof(a));
  a.Q = (const uint8_t*)Q;
  a.D = (const uint8_t*)D;
  a.offsets = offsets;
  a.out = out;
  a.B = B;
  a.T = T;
  a.pad_len = pad_len;
  a.nd = nd;
  a.nq = (int32_t)nq;
  a.nbq = (int32_t)((nq + 31) / 32);
  a.d = (int32_t)d;
  const int64_t hint = B > 0 ? T / B : 1;
  int64_t dpw = hint > 0 ? TMS_VARLEN_BATCHED_TOKENS / hint : 64;
  if (dpw > 1 && B / dpw < (int64_t)256 * 4) dpw = B / ((int64_t)256 * 4);
  if (dpw < 1) dpw = 1;
  if (dpw > 64) dpw = 64;
  a.docs_per_wg = (int32_t)dpw;
  const int64_t grid = (B + dpw - 1) / dpw;
  if (grid > 0x7fffffff) return fail(TMS_ERR_UNSUPPORTED, "batched MaxSim: too many documents");
  if (dtype == TMS_DTYPE_F32)
    return batched_launches(a, nQ, [&](int nb) { return batched_dt<F32Tiles>(dtype, nb, a, grid, 0, st); },
                            batched_max_blocks<F32Tiles>());
  if (q32)
    return batched_launches(a, nQ, [&](int nb) { return batched_dt<DenseTilesQ32>(dtype, nb, a, grid, 0, st); },
                            batched_max_blocks<DenseTilesQ32>());
  return batched_launches(a, nQ, [&](int nb) { return batched_dt<DenseTiles>(dtype, nb, a, grid, 0, st); });
}

// PQ batched entry (tms_pq.hip): fixed-length documents of uint8 codes, the codebook
// (d * K elements, at most 64 KiB) copied to LDS by each workgroup, which walks 64
// documents. Shapes as the single-query MFMA PQ kernel's.
int run_pq_batched(const void* Q, int64_t nQ, int64_t nq, const void* codebook, int64_t M, int64_t K, int64_t dsub,
                   int dtype, const uint8_t* codes, int64_t B, int64_t nd, float* out, hipStream_t st) {
  BatchedArgs a;
  memset(&a, 0, sizeof(a));
  a.Q = (const uint8_t*)Q;
  a.D = codes;
  a.codebook = (const uint8_t*)codebook;
  a.out = out;
  a.B = B;
  a.T = B * nd;
  a.nd = nd;
  a.nq = (int32_t)nq;
  a.nbq = (int32_t)((nq + 31) / 32);
  a.d = (int32_t)(M * dsub);
  a.M = (int32_t)M;
  a.K = (int32_t)K;
  a.docs_per_wg = 64;  // the most a workgroup's lanes hold; amortises the codebook copy
  const int64_t grid = (B + 63) / 64;
  if (grid > 0x7fffffff) return fail(TMS_ERR_UNSUPPORTED, "batched PQ: too many documents");
  const size_t lds = (size_t)a.d * K * 2;
  return batched_launches(a, nQ, [&](int nb) {
    switch (dsub) {
      case 2: return batched_dt<PqTiles<2>>(dtype, nb, a, grid, lds, st);
      case 4: return batched_dt<PqTiles<4>>(dtype, nb, a, grid, lds, st);
      case 8: return batched_dt<PqTiles<8>>(dtype, nb, a, grid, lds, st);
      case 16: return batched_dt<PqTiles<16>>(dtype, nb, a, grid, lds, st);
      default: return batched_dt<PqTiles<32>>(dtype, nb, a, grid, lds, st);
    }
  });
}

// Entry used by tms_dense.hip for d in {32, 64, 96, 128}, 16-byte aligned Q and D:
// fixed-length documents (offsets null), or documents at offsets into T >= 1 rows
// (pad_len > 0: scored as if zero-padded to pad_len tokens). nQ queries of nq tokens;
// out is (nQ, B).
int run_stream(const void* Q, int64_t nQ, int64_t nq, int64_t d, const void* D, int64_t B, int64_t nd,
               const int64_t* offsets, int64_t T, int64_t pad_len, int dtype, float* out, hipStream_t st) {
  StreamArgs a;
  memset(&a, 0, sizeof(a));
  a.Q = (const uint8_t*)Q;
  a.D = (const uint8_t*)D;
  a.offsets = offsets;
  a.out = out;
  a.B = B;
  a.nd = offsets ? 0 : nd;
  a.T = T;
  a.pad_len = pad_len;
  a.nq = (int32_t)nq;
  a.nbq = (int32_t)((nq + 31) / 32);
  a.d = (int32_t)d;
  const int64_t nblocks = nQ * (int64_t)a.nbq;
  if (!offsets && a.nbq <= kMaxBlocksPerWave && nblocks >= 4)  // batched: documents at implicit offsets b * nd
    return run_varlen_batched(Q, nQ, nq, d, D, B * nd, nullptr, nd, B, 0, dtype, out, st, false);
  const int64_t hint = offsets ? (B > 0 ? T / B : 1) : nd;  // tokens per document
  int64_t dpw = hint > 0 ? TMS_STREAM_TOKENS_PER_WAVE / hint : 1;
  const int64_t min_waves = TMS_STREAM_MIN_WAVES;
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
