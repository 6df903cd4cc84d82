// Dense / masked / variable-length MaxSim on gfx950 MFMA: the kernel template and its
// launch helpers, shared by tms_dense.hip (query and documents of one type) and
// tms_dense_q32.hip (fp32 queries against fp16 / bf16 documents).
//
// score[qi][b] = sum_{i < nq} max_{j < len(b)} <Q[qi, i], D_b[j]>, fp32 accumulation.
//
// Reference semantics (src/flash_maxsim_v2.py:73-190, src/flash_maxsim_kernel.py:248-273,
// src/e2e_retrieval_quality.py:105-110): doc rows outside the document are -inf
// before the max, query rows past nq contribute 0, an empty document scores -inf.
//
// Design (one wave = one independent stream of whole documents):
//  * Query tokens are grouped in blocks of 32 (two 16-column halves). A launch covers
//    NQB consecutive blocks; their fragments stay in VGPRs (d <= 128), in LDS (any
//    other d whose fragments fit it), or are read from memory with each tile (wider
//    d), and the block -> (query, token) map lets one launch score several queries
//    against one pass over D.
//  * Each document token is read from HBM exactly once, straight into MFMA A-operand
//    registers: lane (r = l%16, g = l/16) loads the 16-byte chunk 4*s + g of token
//    r at k-step s. Four lanes cover 64 contiguous bytes of a token per instruction.
//    Full, aligned tiles (16-bit d % 64 == 0, fp32 d % 32 == 0) instead read whole
//    128-byte lines of eight rows per instruction with non-temporal loads, which stream
//    faster on this part (about 7.0 against 6.3 TB/s), and rebuild the fragments with
//    a DPP row rotate (line_frags).
//  * A tile is 16*NSUB tokens x 128 dims; the next tile's loads are issued before the
//    current tile's MFMAs (register double buffer). Tokens past the end of a
//    document are clamped to its last token: a duplicate cannot change a max, so
//    no -inf masking is needed and nothing outside the document is fetched.
//  * The per-(query token, row) running max lives in the MFMA accumulator layout; the
//    cross-lane max and the sum over query tokens happen once per document.
//  * fp32 embeddings: a lane's 8 elements are 32 bytes (two 16-byte loads), split into
//    bf16 hi and lo terms before the MFMAs, and each product is formed from three bf16
//    MFMAs (split_bf16 in tms_common.h); tiles are one 16-token block with Q in VGPRs.
//    Under whole-line loads a lane holds elements 4g..4g+3 and 16+4g..16+4g+3 of a
//    32-dimension step, and the query fragments take the same elements.
//  * fp32 queries against 16-bit documents: the query alone is split, into two terms of
//    the document type, and a product takes two MFMAs.
#pragma once
#include <string.h>

#include "tms_common.h"

namespace tms {

enum { MODE_FIXED = 0, MODE_VARLEN = 1, MODE_MASKED = 2 };

struct DenseArgs {
  const uint8_t* Q;        // (nQ * nq, d) elements of the input dtype
  const uint8_t* D;        // fixed / masked: (B, nd, d); varlen: (total_tokens, d)
  const int64_t* offsets;  // varlen: (B + 1)
  const uint8_t* mask;     // masked: (B, nd)
  float* out;              // (nQ, B)
  int64_t B, nd, total_tokens;
  int32_t nq;              // tokens per query
  int32_t nbq;             // 32-token blocks per query = ceil(nq / 32)
  int32_t blk0;            // first global query block of this launch
  int32_t nblk;            // blocks in this launch (<= NQB template)
  int32_t d, nchunk, nstep, nkg;
  int32_t docs_per_wave;
  int64_t pad_len;         // varlen: score as if zero-padded to this many tokens (0 = off)
  int32_t mask4;           // masked: nd % 4 == 0 and a 4-byte aligned mask (word loads)
};

// Elements 8c .. 8c+7 of row `row` (16 bytes; 32 for fp32), zero outside [0, d).
template <int DT, bool ALIGNED>
__device__ __forceinline__ typename Raw8<DT>::T load_chunk(const uint8_t* base, int64_t row, int c, int d, int nchunk) {
  typename Raw8<DT>::T v = {};
  if constexpr (DT == TMS_DTYPE_F32) {
    const uint32_t* p = (const uint32_t*)base + row * d + 8 * (int64_t)c;
    if constexpr (ALIGNED) {  // d % 8 == 0 and a 16-byte aligned base: two 16-byte loads
      if (c < nchunk) {
        const u32x4 a0 = *(const u32x4*)p, a1 = *(const u32x4*)(p + 4);
        v = u32x8{a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; j++) v[j] = (8 * c + j < d) ? p[j] : 0u;
    }
  } else if constexpr (ALIGNED) {
    if (c < nchunk) v = *(const u32x4*)(base + (row * d + 8 * (int64_t)c) * 2);
  } else {
    const uint16_t* p = (const uint16_t*)base + row * d;
    uint16_t e[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
      int k = 8 * c + j;
      e[j] = (k < d) ? p[k] : (uint16_t)0;
    }
    v[0] = e[0] | ((uint32_t)e[1] << 16);
    v[1] = e[2] | ((uint32_t)e[3] << 16);
    v[2] = e[4] | ((uint32_t)e[5] << 16);
    v[3] = e[6] | ((uint32_t)e[7] << 16);
  }
  return v;
}

// fp32 rows read as whole lines (LINES32 below): a k-step is one 128-byte line per row,
// and line_frags leaves lane (r, g) with elements 4g .. 4g+3 and 16+4g .. 16+4g+3 of the
// step's 32. The query fragments take the same elements, so each MFMA sums the same
// products in another order over k. `step` < d / 32; d % 32 == 0, 16-byte aligned base.
__device__ __forceinline__ u32x8 load_chunk_f32_lines(const uint8_t* base, int64_t row, int step, int g, int d) {
  const uint32_t* p = (const uint32_t*)base + row * d + 32 * (int64_t)step + 4 * g;
  const u32x4 a0 = *(const u32x4*)p, a1 = *(const u32x4*)(p + 16);
  return u32x8{a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
}

struct Cursor {
  int64_t b;     // document index
  int64_t base;  // first token row of the document
  int64_t len;   // tokens in the document
  int64_t t0;    // first token of the current tile
  int32_t kg;    // current 128-dim k-group
};

// DT: document element type; QDT: query element type (DT, or fp32 against fp16 / bf16
// documents).
// KS_REG > 0: Q fragments in VGPRs, d == 32 * KS_REG (single k-group).
// KS_REG == 0: Q fragments in LDS, k-groups of 4 steps (128 dims), any d.
// KS_REG < 0: Q fragments read from memory (L2) with each tile's loads, for widths whose
// fragments do not fit the LDS (one query block per launch).
template <int DT, int QDT, int MODE, int NQB, int KS_REG, bool FULL, bool ALIGNED, int NSUB, int PFD, int NT>
__global__ void __launch_bounds__(NT, 1) dense_maxsim_kernel(DenseArgs a) {
  constexpr bool QREG = KS_REG > 0;
  constexpr bool QGLB = KS_REG < 0;
  constexpr int KS = QREG ? KS_REG : 4;
  constexpr int TT = 16 * NSUB;
  // fp32 documents (and queries): every fragment is split into bf16 hi + lo terms and a
  // product takes three bf16 MFMAs (hi*hi + hi*lo + lo*hi).
  constexpr bool F32 = DT == TMS_DTYPE_F32;
  // fp32 queries against fp16 / bf16 documents: each query element is split into hi + lo
  // terms of the document's type (fp16: after the token's power-of-two scale, split_f16)
  // and a product takes two MFMAs, d * q_lo + d * q_hi, so the query is not rounded to
  // 16 bits (the reference computes fp32 x fp16 products with TF32 tl.dot).
  constexpr bool QSPLIT = !F32 && QDT == TMS_DTYPE_F32;
  constexpr bool QSCALE = QSPLIT && DT == TMS_DTYPE_F16;
  constexpr bool QLO = F32 || QSPLIT;  // every query fragment has a lo term
  static_assert(QDT == DT || QSPLIT, "query and document types: equal, or fp32 queries");
  constexpr int MDT = F32 ? TMS_DTYPE_BF16 : DT;
  using Raw = typename Raw8<DT>::T;
  using QRaw = typename Raw8<QDT>::T;
  extern __shared__ u32x4 qlds[];
  __shared__ float qamax[QSCALE && !QREG ? 2 * 32 : 1];  // largest |q| of each query token of the launch

  const int lane = threadIdx.x & 63;
  const int r = lane & 15, g = lane >> 4;
  const int wid = threadIdx.x >> 6;
  // LINES (16-bit rows, every 64-dimension pair of k-steps whole, d % 64 == 0) and LINES32
  // (fp32 rows, every 32-dimension k-step whole; not with the query read from memory,
  // whose extra loads spill there): each document load covers whole 128-byte lines of
  // eight rows, non-temporal; line_frags turns two such loads into MFMA fragments when
  // the tile is scored. Lane 16 g + 8 s + t reads bytes 64 s + 16 g of a line of row t
  // or 8 + t.
  constexpr bool LINES = FULL && ALIGNED && !F32 && KS % 2 == 0;
  constexpr bool LINES32 = FULL && ALIGNED && F32 && !QGLB;
  // query elements of fragment (row, step S, lane group gg): chunk 4 S + gg, or under
  // LINES32 the elements its line_frags gives the documents' fragment
  auto q_chunk = [&](int64_t row, int S, int gg) -> QRaw {
    if constexpr (LINES32) return load_chunk_f32_lines(a.Q, row, S, gg, a.d);
    else return load_chunk<QDT, ALIGNED>(a.Q, row, 4 * S + gg, a.d, a.nchunk);
  };

  // Query blocks of this launch: [my_blk0, my_blk0 + my_nblk).
  const int my_blk0 = a.blk0, my_nblk = a.nblk;

  // ---- query fragments -------------------------------------------------------
  // Fragment (block j, step S, half h) for this lane: query row of block j, token
  // 16h + r, elements of chunk 4S + g.
  auto q_row = [&](int j, int h, int rr, bool& valid) -> int64_t {
    int jb = my_blk0 + j;
    int qi = jb / a.nbq;
    int tok = (jb - qi * a.nbq) * 32 + 16 * h + rr;
    valid = (j < my_nblk) && (tok < a.nq);
    return (int64_t)qi * a.nq + tok;
  };

  // fp16 / bf16: the fragment itself; split queries: the hi term here and the lo term in
  // qfl (LDS path: the lo terms follow the nfrag hi fragments).
  u32x4 qf[QREG ? NQB : 1][QREG ? KS : 1][2];
  u32x4 qfl[QREG && QLO ? NQB : 1][QREG && QLO ? KS : 1][2];
  // QSCALE: the power-of-two scale of this lane's column token (16h + r of block j), and
  // its inverse, applied to the column's max before the sum over query tokens
  float qscl[NQB][2], qinv[NQB][2];
  auto to_frag = [&](const QRaw& raw, float scale, u32x4& hi, u32x4& lo) {
    if constexpr (F32) split_bf16(raw, hi, lo);
    else if constexpr (QSCALE) split_f16(raw, scale, hi, lo);
    else if constexpr (QSPLIT) split_bf16(raw, hi, lo);
    else hi = raw;
  };
  const int nfrag = NQB * a.nstep * 2 * 64;
  if constexpr (QREG) {
#pragma unroll
    for (int j = 0; j < NQB; j++)
#pragma unroll
      for (int h = 0; h < 2; h++) {
        bool valid;
        const int64_t row = q_row(j, h, r, valid);
        QRaw raw[KS];
        float am = 0.f;
#pragma unroll
        for (int s = 0; s < KS; s++) {
          raw[s] = valid ? q_chunk(row, s, g) : QRaw{};
          if constexpr (QSCALE) am = fmaxf(am, absmax8(raw[s]));
        }
        float sc = 1.f;
        if constexpr (QSCALE) {  // the token's chunks are spread over lanes r, r+16, r+32, r+48
          am = fmaxf(am, __shfl_xor(am, 16));
          am = fmaxf(am, __shfl_xor(am, 32));
          sc = pow2_scale(am, qinv[j][h]);
        }
#pragma unroll
        for (int s = 0; s < KS; s++) to_frag(raw[s], sc, qf[j][s][h], qfl[QLO ? j : 0][QLO ? s : 0][h]);
      }
  } else {
    if constexpr (QSCALE) {  // one wave per query token: its largest |q|
      for (int t = wid; t < NQB * 32; t += NT / 64) {
        bool valid;
        const int64_t row = q_row(t >> 5, (t >> 4) & 1, t & 15, valid);
        float am = 0.f;
        if (valid)
          for (int k = lane; k < a.d; k += 64) am = fmaxf(am, fabsf(((const float*)a.Q)[row * a.d + k]));
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) am = fmaxf(am, __shfl_xor(am, o));
        if (lane == 0) qamax[t] = am;
      }
      __syncthreads();
#pragma unroll
      for (int j = 0; j < NQB; j++)
#pragma unroll
        for (int h = 0; h < 2; h++) qscl[j][h] = pow2_scale(qamax[32 * j + 16 * h + r], qinv[j][h]);
    }
    if constexpr (!QGLB) {
      for (int f = threadIdx.x; f < nfrag; f += blockDim.x) {
        int fl = f & 63, rest = f >> 6;
        int h = rest & 1;
        rest >>= 1;
        int S = rest % a.nstep, j = rest / a.nstep;
        bool valid;
        int64_t row = q_row(j, h, fl & 15, valid);
        const QRaw raw = valid ? q_chunk(row, S, fl >> 4) : QRaw{};
        float sc = 1.f;
        if constexpr (QSCALE) {
          float unused;
          sc = pow2_scale(qamax[32 * j + 16 * h + (fl & 15)], unused);
        }
        u32x4 hi, lo;
        to_frag(raw, sc, hi, lo);
        qlds[f] = hi;
        if constexpr (QLO) qlds[nfrag + f] = lo;
      }
      __syncthreads();
    }
  }

  const int64_t wave = (int64_t)blockIdx.x * (blockDim.x >> 6) + wid;
  const int64_t b_begin = wave * a.docs_per_wave;
  if (b_begin >= a.B || my_nblk <= 0) return;
  const int64_t b_end = (b_begin + a.docs_per_wave < a.B) ? b_begin + a.docs_per_wave : a.B;

  const float NEG_INF = -__builtin_inff();

  // ---- per-query output ------------------------------------------------------
  // Block sums are added per query; a query whose first block precedes this wave's
  // blocks accumulates onto the previous launch's partial score. Lane 0 writes each
  // document's score when the document finishes.
  auto write_doc = [&](int64_t b, const float (&blk)[NQB]) {
    if (lane == 0) {
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < NQB; j++) {
        if (j >= my_nblk) break;
        int jb = my_blk0 + j;
        int qi = jb / a.nbq;
        s += blk[j];
        bool last_of_query = (j == my_nblk - 1) || ((jb + 1) / a.nbq != qi);
        if (last_of_query) {
          float* o = a.out + (int64_t)qi * a.B + b;
          bool cont = (qi * a.nbq) < my_blk0;  // query began in an earlier launch
          *o = cont ? (*o + s) : s;
          s = 0.f;
        }
      }
    }
  };

  auto write_empty = [&](int64_t b, float v) {
    float blk[NQB];
#pragma unroll
    for (int j = 0; j < NQB; j++) blk[j] = v;  // every block in range holds a real token
    write_doc(b, blk);
  };
  // A document with invalid offsets scores NaN for every query of the launch, written
  // as an integer (every launch over it writes the same bits, with no float arithmetic).
  auto write_bad = [&](int64_t b) {
    if (lane == 0) {
#pragma unroll
      for (int j = 0; j < NQB; j++) {
        if (j >= my_nblk) break;
        const int jb = my_blk0 + j;
        const int qi = jb / a.nbq;
        if (j == my_nblk - 1 || (jb + 1) / a.nbq != qi) store_nan_score(a.out + (int64_t)qi * a.B + b);
      }
    }
  };

  // ---- document cursor -------------------------------------------------------
  auto doc_info = [&](int64_t b, int64_t& base, bool& bad) -> int64_t {
    bad = false;
    if constexpr (MODE == MODE_VARLEN) {
      int64_t s = a.offsets[b], e = a.offsets[b + 1];
      if (s < 0 || e < s || e > a.total_tokens) {
        bad = true;
        base = 0;
        return 0;
      }
      base = s;
      return e - s;
    } else {
      base = b * a.nd;
      return a.nd;
    }
  };
  // Move to the first document at or after b with at least one token; documents
  // skipped on the way are written (-inf, or NaN for invalid offsets).
  auto seek = [&](Cursor& c, int64_t b) {
    for (; b < b_end; b++) {
      bool bad;
      int64_t base;
      int64_t len = doc_info(b, base, bad);
      if (len > 0) {
        c.b = b;
        c.base = base;
        c.len = len;
        c.t0 = 0;
        c.kg = 0;
        return;
      }
      // an empty document zero-padded to pad_len > 0 tokens has every max equal to 0
      if (bad) write_bad(b);
      else write_empty(b, a.pad_len > 0 ? 0.f : NEG_INF);
    }
    c.b = b_end;
  };
  auto advance = [&](Cursor& c) {
    if (c.kg + 1 < a.nkg) {
      c.kg++;
      return;
    }
    c.kg = 0;
    c.t0 += TT;
    if (c.t0 >= c.len) seek(c, c.b + 1);
  };

  // ---- tile buffers ------------------------------------------------------------
  struct Buf {
    Raw f[NSUB][KS];
    uint32_t m[NSUB];  // masked mode: validity bits of this lane's 4 output rows
    QRaw q[QGLB ? NQB : 1][QGLB ? KS : 1][2];  // memory-resident Q: the k-group's query chunks
  };
  const int t8 = lane & 7;
  const int64_t line_off = 64 * ((lane >> 3) & 1) + 16 * g;
  auto load_tile = [&](Buf& buf, const Cursor& c) {
    if constexpr (QGLB) {  // issued with the tile's loads, so waiting for them never drains the prefetch
#pragma unroll
      for (int j = 0; j < NQB; j++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
          bool valid;
          const int64_t row = q_row(j, h, r, valid);
#pragma unroll
          for (int s = 0; s < KS; s++) {
            const int S = c.kg * KS + s;
            buf.q[j][s][h] = (valid && S < a.nstep) ? q_chunk(row, S, g) : QRaw{};
          }
        }
    }
#pragma unroll
    for (int sub = 0; sub < NSUB; sub++) {
      if constexpr (LINES) {  // f[sub][2i], f[sub][2i+1]: line i of the k-group, rows t and 8 + t
        int64_t t0 = c.t0 + 16 * sub + t8, t1 = t0 + 8;
        if (t0 > c.len - 1) t0 = c.len - 1;
        if (t1 > c.len - 1) t1 = c.len - 1;
        const uint8_t* p0 = a.D + (c.base + t0) * a.d * 2 + (int64_t)c.kg * 256 + line_off;
        const uint8_t* p1 = a.D + (c.base + t1) * a.d * 2 + (int64_t)c.kg * 256 + line_off;
#pragma unroll
        for (int i = 0; i < KS / 2; i++) {
          if (!QREG && c.kg * KS + 2 * i >= a.nstep) {  // nstep is even: both k-steps past the end
            buf.f[sub][2 * i] = buf.f[sub][2 * i + 1] = Raw{};
          } else {
            buf.f[sub][2 * i] = ld_stream<u32x4, true>(p0 + 128 * i);
            buf.f[sub][2 * i + 1] = ld_stream<u32x4, true>(p1 + 128 * i);
          }
        }
      } else if constexpr (LINES32) {  // f[sub][s]: line S of rows t (elements 0-3) and 8 + t (4-7)
        int64_t t0 = c.t0 + 16 * sub + t8, t1 = t0 + 8;
        if (t0 > c.len - 1) t0 = c.len - 1;
        if (t1 > c.len - 1) t1 = c.len - 1;
        const uint8_t* p0 = a.D + (c.base + t0) * a.d * 4 + line_off;
        const uint8_t* p1 = a.D + (c.base + t1) * a.d * 4 + line_off;
#pragma unroll
        for (int s = 0; s < KS; s++) {
          const int S = c.kg * KS + s;
          if (!QREG && S >= a.nstep) {
            buf.f[sub][s] = Raw{};
          } else {
            const u32x4 x0 = ld_stream<u32x4, true>(p0 + 128 * (int64_t)S);
            const u32x4 x1 = ld_stream<u32x4, true>(p1 + 128 * (int64_t)S);
            buf.f[sub][s] = Raw{x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
          }
        }
      } else {
        int64_t tok = c.t0 + 16 * sub + r;
        if (tok > c.len - 1) tok = c.len - 1;
        const int64_t row = c.base + tok;
#pragma unroll
        for (int s = 0; s < KS; s++) {
          const int S = c.kg * KS + s;
          if (!QREG && S >= a.nstep) {
            buf.f[sub][s] = Raw{};
          } else if constexpr (FULL && ALIGNED && !F32) {
            buf.f[sub][s] = *(const u32x4*)(a.D + (row * a.d + 8 * (int64_t)(4 * S + g)) * 2);
          } else {
            buf.f[sub][s] = load_chunk<DT, ALIGNED>(a.D, row, 4 * S + g, a.d, a.nchunk);
          }
        }
      }
      if constexpr (MODE == MODE_MASKED) {
        uint32_t bits = 0;
        if (c.kg == a.nkg - 1) {
          const int64_t t0 = c.t0 + 16 * sub + 4 * g;
          if (a.mask4 && c.t0 + 16 * sub + 16 <= c.len) {  // a whole 16-token block: one word per lane
            const uint32_t w = *(const uint32_t*)(a.mask + c.b * a.nd + t0);
#pragma unroll
            for (int i = 0; i < 4; i++) bits |= (((w >> (8 * i)) & 0xffu) != 0u ? 1u : 0u) << i;
          } else {
#pragma unroll
            for (int i = 0; i < 4; i++) {
              int64_t t = t0 + i;
              if (t > c.len - 1) t = c.len - 1;
              bits |= (a.mask[c.b * a.nd + t] != 0 ? 1u : 0u) << i;
            }
          }
        }
        buf.m[sub] = bits;
      }
    }
  };

  // Accumulators that persist across k-groups (LDS-query path only).
  f32x4 acc[QREG ? 1 : NSUB][QREG ? 1 : NQB][2];
  // Running max of this lane's column (query token 16h + r of block j) over every row
  // it has seen; the four rows of each MFMA result fold in with a tree of maxes.
  float rmax[NQB][2];
#pragma unroll
  for (int j = 0; j < NQB; j++) rmax[j][0] = rmax[j][1] = NEG_INF;
  auto fold = [&](float& m, f32x4 v, uint32_t valid_bits) {
    if constexpr (MODE == MODE_MASKED) {
#pragma unroll
      for (int i = 0; i < 4; i++) v[i] = ((valid_bits >> i) & 1u) ? v[i] : NEG_INF;
    }
    m = fmaxf(m, fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3])));
  };
  if constexpr (!QREG) {
#pragma unroll
    for (int sub = 0; sub < NSUB; sub++)
#pragma unroll
      for (int j = 0; j < NQB; j++) acc[sub][j][0] = acc[sub][j][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  auto finish_doc = [&](int64_t b, int64_t len) {
    // zero padding up to pad_len adds dot products equal to 0 to a shorter document
    const bool padded = (MODE == MODE_VARLEN) && len < a.pad_len;
    float blk[NQB];
#pragma unroll
    for (int j = 0; j < NQB; j++) {
      float s = 0.f;
#pragma unroll
      for (int h = 0; h < 2; h++) {
        float m = rmax[j][h];
        m = fmaxf(m, __shfl_xor(m, 16));
        m = fmaxf(m, __shfl_xor(m, 32));
        if constexpr (QSCALE) m *= qinv[j][h];  // exact: a power of two (-inf stays -inf)
        if (padded) m = fmaxf(m, 0.f);
        bool valid;
        (void)q_row(j, h, r, valid);
        s += valid ? m : 0.f;
      }
      s += __shfl_xor(s, 8);
      s += __shfl_xor(s, 4);
      s += __shfl_xor(s, 2);
      s += __shfl_xor(s, 1);
      blk[j] = s;
      rmax[j][0] = rmax[j][1] = NEG_INF;
    }
    write_doc(b, blk);
  };

  auto compute_tile = [&](const Buf& buf, const Cursor& c) {
    Raw lf[LINES ? NSUB : 1][LINES ? KS : 1];  // LINES: the fragments of the tile's loads
    if constexpr (LINES) {
#pragma unroll
      for (int sub = 0; sub < NSUB; sub++)
#pragma unroll
        for (int i = 0; i < KS / 2; i++)
          line_frags(buf.f[sub][2 * i], buf.f[sub][2 * i + 1], lf[sub][2 * i], lf[sub][2 * i + 1]);
    }
    auto F = [&](int sub, int s) -> const Raw& {  // chunk 4 s + g of row r of subtile sub
      if constexpr (LINES) return lf[sub][s];
      else return buf.f[sub][s];
    };
    // fp32: the 8 elements of row r this lane scores at step s (LINES32: rebuilt from the
    // two row halves' whole-line loads)
    auto F32frag = [&](int sub, int s) -> Raw {
      if constexpr (LINES32) {
        const Raw& x = buf.f[sub][s];
        u32x4 k0, k1;
        line_frags(u32x4{x[0], x[1], x[2], x[3]}, u32x4{x[4], x[5], x[6], x[7]}, k0, k1);
        return Raw{k0[0], k0[1], k0[2], k0[3], k1[0], k1[1], k1[2], k1[3]};
      } else {
        return buf.f[sub][s];
      }
    };
    if constexpr (QREG) {
      // One k-group: each query block is finished before the next, so only one
      // block's accumulators are live (what lets a wave hold several blocks).
#pragma unroll
      for (int j = 0; j < NQB; j++) {
        if (j >= my_nblk) break;
        f32x4 acc1[NSUB][2];
#pragma unroll
        for (int sub = 0; sub < NSUB; sub++) acc1[sub][0] = acc1[sub][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KS; s++) {
          if constexpr (F32) {
#pragma unroll
            for (int sub = 0; sub < NSUB; sub++) {
              u32x4 dh, dl;
              split_bf16(F32frag(sub, s), dh, dl);
#pragma unroll
              for (int h = 0; h < 2; h++) {
                acc1[sub][h] = mfma16x16x32<MDT>(dl, qf[j][s][h], acc1[sub][h]);
                acc1[sub][h] = mfma16x16x32<MDT>(dh, qfl[j][s][h], acc1[sub][h]);
                acc1[sub][h] = mfma16x16x32<MDT>(dh, qf[j][s][h], acc1[sub][h]);
              }
            }
          } else if constexpr (QSPLIT) {
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
              for (int sub = 0; sub < NSUB; sub++) {
                acc1[sub][h] = mfma16x16x32<MDT>(F(sub, s), qfl[j][s][h], acc1[sub][h]);
                acc1[sub][h] = mfma16x16x32<MDT>(F(sub, s), qf[j][s][h], acc1[sub][h]);
              }
          } else {
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
              for (int sub = 0; sub < NSUB; sub++)
                acc1[sub][h] = mfma16x16x32<MDT>(F(sub, s), qf[j][s][h], acc1[sub][h]);
          }
        }
#pragma unroll
        for (int sub = 0; sub < NSUB; sub++)
#pragma unroll
          for (int h = 0; h < 2; h++) fold(rmax[j][h], acc1[sub][h], MODE == MODE_MASKED ? buf.m[sub] : 0u);
      }
      if (c.t0 + TT >= c.len) finish_doc(c.b, c.len);
      return;
    }
#pragma unroll
    for (int s = 0; s < KS; s++) {
      const int S = c.kg * KS + s;
      if (!QREG && S >= a.nstep) break;
      u32x4 dh[NSUB], dl[F32 ? NSUB : 1];
#pragma unroll
      for (int sub = 0; sub < NSUB; sub++) {
        if constexpr (F32) split_bf16(F32frag(sub, s), dh[sub], dl[sub]);
        else dh[sub] = F(sub, s);
      }
#pragma unroll
      for (int j = 0; j < NQB; j++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
          u32x4 qv, qlv;
          if constexpr (QGLB) {
            to_frag(buf.q[j][s][h], QSCALE ? qscl[j][h] : 1.f, qv, qlv);
          } else {
            const int qi = ((j * a.nstep + S) * 2 + h) * 64 + lane;
            qv = qlds[qi];
            if constexpr (QLO) qlv = qlds[nfrag + qi];
          }
          if constexpr (F32) {
#pragma unroll
            for (int sub = 0; sub < NSUB; sub++) {
              acc[sub][j][h] = mfma16x16x32<MDT>(dl[sub], qv, acc[sub][j][h]);
              acc[sub][j][h] = mfma16x16x32<MDT>(dh[sub], qlv, acc[sub][j][h]);
              acc[sub][j][h] = mfma16x16x32<MDT>(dh[sub], qv, acc[sub][j][h]);
            }
          } else if constexpr (QSPLIT) {
#pragma unroll
            for (int sub = 0; sub < NSUB; sub++) {
              acc[sub][j][h] = mfma16x16x32<MDT>(dh[sub], qlv, acc[sub][j][h]);
              acc[sub][j][h] = mfma16x16x32<MDT>(dh[sub], qv, acc[sub][j][h]);
            }
          } else {
#pragma unroll
            for (int sub = 0; sub < NSUB; sub++) acc[sub][j][h] = mfma16x16x32<MDT>(dh[sub], qv, acc[sub][j][h]);
          }
        }
    }
    if (c.kg == a.nkg - 1) {
#pragma unroll
      for (int sub = 0; sub < NSUB; sub++)
#pragma unroll
        for (int j = 0; j < NQB; j++)
#pragma unroll
          for (int h = 0; h < 2; h++) {
            fold(rmax[j][h], acc[sub][j][h], MODE == MODE_MASKED ? buf.m[sub] : 0u);
            acc[sub][j][h] = f32x4{0.f, 0.f, 0.f, 0.f};
          }
      if (c.t0 + TT >= c.len) finish_doc(c.b, c.len);
    }
  };

  // ---- pipelined main loop -----------------------------------------------------
  // A ring of PFD + 1 tile buffers: the loads of the next PFD tiles are in flight
  // while a tile is scored. The ring is unrolled so every buffer index is static.
  Cursor next;
  seek(next, b_begin);
  if (next.b >= b_end) return;
  Buf ring[PFD + 1];
  Cursor at[PFD + 1];
#pragma unroll
  for (int k = 0; k < PFD; k++) {
    at[k] = next;
    if (next.b < b_end) {
      load_tile(ring[k], next);
      advance(next);
    }
  }
  while (true) {
#pragma unroll
    for (int k = 0; k <= PFD; k++) {
      constexpr int kPf = PFD;
      const int slot_in = (k + kPf) % (kPf + 1);
      at[slot_in] = next;
      if (next.b < b_end) {
        load_tile(ring[slot_in], next);
        advance(next);
      }
      if (at[k].b >= b_end) return;
      compute_tile(ring[k], at[k]);
    }
  }
}

#ifndef TMS_DENSE_NSUB
#define TMS_DENSE_NSUB 2  // 16-token MFMA row blocks per tile (tile = 16 * NSUB tokens)
#endif
#ifndef TMS_DENSE_TOKENS_PER_WAVE
#define TMS_DENSE_TOKENS_PER_WAVE 192  // document tokens one wave streams (rounded to whole documents)
#endif
constexpr int kNSub = TMS_DENSE_NSUB;
#ifndef TMS_DENSE_F32_NSUB
#define TMS_DENSE_F32_NSUB 1  // 16-token row blocks per tile for fp32 documents, Q in VGPRs
#endif
#ifndef TMS_DENSE_F32_LDS_NSUB
#define TMS_DENSE_F32_LDS_NSUB 2  // the same with Q in LDS
#endif
constexpr int kMaxQldsBytes = 64 * 1024;
constexpr int kMaxDim = 1 << 16;  // widest embedding the dense entry points take
constexpr size_t kStaticLds = 256;  // the kernel's static LDS (per-token query scales) beside the fragments
#ifndef TMS_DENSE_PFD
#define TMS_DENSE_PFD 1  // tiles in flight ahead of the one being scored
#endif

// LDS bytes of the query fragments of one launch (split queries: hi and lo terms).
static inline size_t qlds_bytes(int dtype, int qdtype, int nqb, int nstep) {
  const bool split = dtype == TMS_DTYPE_F32 || qdtype == TMS_DTYPE_F32;
  return (size_t)nqb * nstep * 2 * 64 * 16 * (split ? 2 : 1);
}

// The device's LDS bytes per workgroup (160 KiB on gfx950).
static inline int lds_limit(int& cap) {
  int dev = 0;
  cap = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cap, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
    return fail(TMS_ERR_HIP, "dense_maxsim_kernel: cannot query the LDS limit");
  return TMS_OK;
}

template <int DT, int QDT, int MODE, int NQB, int KS_REG, bool FULL, bool ALIGNED, int NT>
static int launch_nt(const DenseArgs& a, int64_t waves, size_t lds, hipStream_t st) {
  // fp32 tiles hold twice the bytes per token: with Q in VGPRs, one 16-token row block
  // per tile keeps the bytes in flight per wave where the 16-bit path has them; with Q
  // in LDS (d > 128: its lo terms take up to 128 KiB, one or two workgroups per CU) two
  // blocks per tile keep more bytes in flight per wave (measured: +20 % at d = 768,
  // +12 % at d = 1000, within 4 % either way at d = 200 .. 512)
  // (split queries against 16-bit documents keep the 16-bit tile: the same bytes per token)
  constexpr int NS = DT == TMS_DTYPE_F32 ? (KS_REG > 0 ? TMS_DENSE_F32_NSUB : TMS_DENSE_F32_LDS_NSUB) : kNSub;
  const int64_t grid = (waves + NT / 64 - 1) / (NT / 64);
  if (lds > 64 * 1024) {
    int cap = 0;
    const int rc = lds_limit(cap);
    if (rc != TMS_OK) return rc;
    if (lds > (size_t)cap)
      return fail(TMS_ERR_UNSUPPORTED, "dense_maxsim_kernel: query fragments need %zu bytes of LDS, the device has %d",
                  lds, cap);
  }
  hipLaunchKernelGGL((dense_maxsim_kernel<DT, QDT, MODE, NQB, KS_REG, FULL, ALIGNED, NS, TMS_DENSE_PFD, NT>),
                     dim3((unsigned)grid), dim3(NT), lds, st, a);
  return check_launch("dense_maxsim_kernel");
}

// Q in LDS above 80 KiB (fp32 or split queries at d >= 768, 16-bit at d > 1280: room for
// one workgroup per CU): 8-wave workgroups, so the CU still holds two waves per SIMD
// (fp32, d = 768: 5.2 -> 5.8 TB/s, d = 1000: 4.5 -> 5.1 TB/s). Below that, 4-wave
// workgroups (8-wave ones measured 5 % slower at d = 200 and 512).
template <int DT, int QDT, int MODE, int NQB, int KS_REG, bool FULL, bool ALIGNED>
static int launch_one(const DenseArgs& a, int64_t waves, size_t lds, hipStream_t st) {
  if constexpr (KS_REG == 0) {
    if (lds > 80 * 1024) return launch_nt<DT, QDT, MODE, NQB, KS_REG, FULL, ALIGNED, 512>(a, waves, lds, st);
  }
  return launch_nt<DT, QDT, MODE, NQB, KS_REG, FULL, ALIGNED, 256>(a, waves, lds, st);
}

template <int DT, int QDT, int MODE, int NQB>
static int launch_nqb(const DenseArgs& a, bool aligned, int64_t waves, hipStream_t st) {
  // every pair of k-steps whole (the tiles' whole-line loads): d % 64 == 0; d % 64 == 32
  // takes the bounds-checked loads
  const bool full = aligned && (a.d % 64 == 0);
  if (aligned && a.d > 0 && a.d <= 128 && a.d % 32 == 0) {
    switch (a.d / 32) {
      case 1: return launch_one<DT, QDT, MODE, NQB, 1, true, true>(a, waves, 0, st);
      case 2: return launch_one<DT, QDT, MODE, NQB, 2, true, true>(a, waves, 0, st);
      case 3: return launch_one<DT, QDT, MODE, NQB, 3, true, true>(a, waves, 0, st);
      default: return launch_one<DT, QDT, MODE, NQB, 4, true, true>(a, waves, 0, st);
    }
  }
  size_t lds = qlds_bytes(DT, QDT, NQB, a.nstep);
  if (lds == 0) lds = 16;
  if (lds > 64 * 1024) {
    int cap = 0;
    const int rc = lds_limit(cap);
    if (rc != TMS_OK) return rc;
    if (lds + kStaticLds > (size_t)cap) {
      // wider than the LDS holds (16-bit d >= 2560, fp32 or split d >= 1280): the query
      // fragments are read from memory with each tile (one block per launch)
      if constexpr (NQB == 1) {
        if (full) return launch_one<DT, QDT, MODE, 1, -1, true, true>(a, waves, 0, st);
        if (aligned) return launch_one<DT, QDT, MODE, 1, -1, false, true>(a, waves, 0, st);
        return launch_one<DT, QDT, MODE, 1, -1, false, false>(a, waves, 0, st);
      }
      return fail(TMS_ERR_UNSUPPORTED, "dense_maxsim_kernel: %d query blocks at d=%d exceed the LDS", NQB, a.d);
    }
  }
  if (full) return launch_one<DT, QDT, MODE, NQB, 0, true, true>(a, waves, lds, st);
  if (aligned) return launch_one<DT, QDT, MODE, NQB, 0, false, true>(a, waves, lds, st);
  return launch_one<DT, QDT, MODE, NQB, 0, false, false>(a, waves, lds, st);
}

// nQ queries (a.nbq blocks each) over the documents of `a`, NQB <= 2 blocks per launch.
template <int DT, int QDT>
static int run_dense(DenseArgs a, int64_t nQ, int mode, bool aligned, hipStream_t st) {
  const int64_t nblocks_total = nQ * (int64_t)a.nbq;
  const int64_t waves = (a.B + a.docs_per_wave - 1) / a.docs_per_wave;
  // Blocks per launch: two when Q fits in VGPRs or its LDS copy stays small.
  int maxq = 2;
  if (!(aligned && a.d > 0 && a.d <= 128 && a.d % 32 == 0) && qlds_bytes(DT, QDT, 2, a.nstep) > (size_t)kMaxQldsBytes)
    maxq = 1;
  for (int64_t blk0 = 0; blk0 < nblocks_total; blk0 += maxq) {
    a.blk0 = (int32_t)blk0;
    a.nblk = (int32_t)((nblocks_total - blk0 < maxq) ? nblocks_total - blk0 : maxq);
    int rc;
    if (a.nblk == 2) {
      if (mode == MODE_FIXED) rc = launch_nqb<DT, QDT, MODE_FIXED, 2>(a, aligned, waves, st);
      else if (mode == MODE_VARLEN) rc = launch_nqb<DT, QDT, MODE_VARLEN, 2>(a, aligned, waves, st);
      else rc = launch_nqb<DT, QDT, MODE_MASKED, 2>(a, aligned, waves, st);
    } else {
      if (mode == MODE_FIXED) rc = launch_nqb<DT, QDT, MODE_FIXED, 1>(a, aligned, waves, st);
      else if (mode == MODE_VARLEN) rc = launch_nqb<DT, QDT, MODE_VARLEN, 1>(a, aligned, waves, st);
      else rc = launch_nqb<DT, QDT, MODE_MASKED, 1>(a, aligned, waves, st);
    }
    if (rc != TMS_OK) return rc;
  }
  return TMS_OK;
}

}  // namespace tms
