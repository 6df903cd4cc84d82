// Dense / masked / variable-length MaxSim on gfx950 MFMA.
//
// score[qi][b] = sum_{i < nq} max_{j < len(b)} <Q[qi, i], D_b[j]>, fp32 accumulation.
//
// Reference semantics (src/flash_maxsim_v2.py:73-190, src/flash_maxsim_kernel.py:248-273,
// src/e2e_retrieval_quality.py:105-110): doc rows outside the document are -inf
// before the max, query rows past nq contribute 0, an empty document scores -inf.
//
// Design (one wave = one independent stream of whole documents):
//  * Query tokens are grouped in blocks of 32 (two 16-column halves). A launch covers
//    NQB consecutive blocks; their fragments stay in VGPRs (d <= 128) or in LDS
//    (any other d), and the block -> (query, token) map lets one launch score several
//    queries against one pass over D.
//  * Each document token is read from HBM exactly once, straight into MFMA A-operand
//    registers: lane (r = l%16, g = l/16) loads the 16-byte chunk 4*s + g of token
//    r at k-step s. Four lanes cover 64 contiguous bytes of a token per instruction,
//    which streams at the same rate as a fully coalesced copy on this part.
//  * A tile is 16*NSUB tokens x 128 dims; the next tile's loads are issued before the
//    current tile's MFMAs (register double buffer). Tokens past the end of a
//    document are clamped to its last token: a duplicate cannot change a max, so
//    no -inf masking is needed and nothing outside the document is fetched.
//  * The per-(query token, row) running max lives in the MFMA accumulator layout; the
//    cross-lane max and the sum over query tokens happen once per document.
//  * fp32 embeddings: a lane's 8-element chunk is 32 bytes (two 16-byte loads), split
//    into bf16 hi and lo terms before the MFMAs, and each product is formed from three
//    bf16 MFMAs (split_bf16 in tms_common.h); tiles are one 16-token block.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "tms_common.h"

namespace tms {

// Fixed-length documents with d in {32, 64, 96, 128} (tms_stream.hip).
int run_stream(const void* Q, int64_t nQ, int64_t nq, int64_t d, const void* D, int64_t B, int64_t nd, int dtype,
               float* out, hipStream_t st);
// Variable-length documents, d in {32, 64, 96, 128}, several query blocks (tms_stream.hip).
int run_varlen_batched(const void* Q, int64_t nQ, int64_t nq, int64_t d, const void* D, int64_t T,
                       const int64_t* offsets, int64_t nd, int64_t B, int64_t pad_len, int dtype, float* out,
                       hipStream_t st);

static thread_local char g_err[512];

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TMS_ERR_HIP, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
  return TMS_OK;
}

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

struct Cursor {
  int64_t b;     // document index
  int64_t base;  // first token row of the document
  int64_t len;   // tokens in the document
  int64_t t0;    // first token of the current tile
  int32_t kg;    // current 128-dim k-group
};

// KS_REG > 0: Q fragments in VGPRs, d == 32 * KS_REG (single k-group).
// KS_REG == 0: Q fragments in LDS, k-groups of 4 steps (128 dims), any d.
template <int DT, int MODE, int NQB, int KS_REG, bool FULL, bool ALIGNED, int NSUB, int PFD, int NT>
__global__ void __launch_bounds__(NT, 1) dense_maxsim_kernel(DenseArgs a) {
  constexpr bool QREG = KS_REG > 0;
  constexpr int KS = QREG ? KS_REG : 4;
  constexpr int TT = 16 * NSUB;
  // fp32 inputs: every fragment is split into bf16 hi + lo terms and a product takes
  // three bf16 MFMAs (hi*hi + hi*lo + lo*hi); F32 == false is the one-MFMA path.
  constexpr bool F32 = DT == TMS_DTYPE_F32;
  constexpr int MDT = F32 ? TMS_DTYPE_BF16 : DT;
  using Raw = typename Raw8<DT>::T;
  extern __shared__ u32x4 qlds[];

  const int lane = threadIdx.x & 63;
  const int r = lane & 15, g = lane >> 4;
  const int wid = threadIdx.x >> 6;

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

  // fp16 / bf16: the fragment itself; fp32: its bf16 hi term here and lo term in qfl
  // (LDS path: the lo terms follow the nfrag hi fragments).
  u32x4 qf[QREG ? NQB : 1][QREG ? KS : 1][2];
  u32x4 qfl[QREG && F32 ? NQB : 1][QREG && F32 ? KS : 1][2];
  auto to_frag = [&](const Raw& raw, u32x4& hi, u32x4& lo) {
    if constexpr (F32) split_bf16(raw, hi, lo);
    else hi = raw;
  };
  const int nfrag = NQB * a.nstep * 2 * 64;
  if constexpr (QREG) {
#pragma unroll
    for (int j = 0; j < NQB; j++)
#pragma unroll
      for (int s = 0; s < KS; s++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
          bool valid;
          int64_t row = q_row(j, h, r, valid);
          const Raw raw = valid ? load_chunk<DT, true>(a.Q, row, 4 * s + g, a.d, a.nchunk) : Raw{};
          to_frag(raw, qf[j][s][h], qfl[F32 ? j : 0][F32 ? s : 0][h]);
        }
  } else {
    for (int f = threadIdx.x; f < nfrag; f += blockDim.x) {
      int fl = f & 63, rest = f >> 6;
      int h = rest & 1;
      rest >>= 1;
      int S = rest % a.nstep, j = rest / a.nstep;
      bool valid;
      int64_t row = q_row(j, h, fl & 15, valid);
      const Raw raw = valid ? load_chunk<DT, ALIGNED>(a.Q, row, 4 * S + (fl >> 4), a.d, a.nchunk) : Raw{};
      u32x4 hi, lo;
      to_frag(raw, hi, lo);
      qlds[f] = hi;
      if constexpr (F32) qlds[nfrag + f] = lo;
    }
    __syncthreads();
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
  };
  auto load_tile = [&](Buf& buf, const Cursor& c) {
#pragma unroll
    for (int sub = 0; sub < NSUB; sub++) {
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
      if constexpr (MODE == MODE_MASKED) {
        uint32_t bits = 0;
        if (c.kg == a.nkg - 1) {
#pragma unroll
          for (int i = 0; i < 4; i++) {
            int64_t t = c.t0 + 16 * sub + 4 * g + i;
            if (t > c.len - 1) t = c.len - 1;
            bits |= (a.mask[c.b * a.nd + t] != 0 ? 1u : 0u) << i;
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
              split_bf16(buf.f[sub][s], dh, dl);
#pragma unroll
              for (int h = 0; h < 2; h++) {
                acc1[sub][h] = mfma16x16x32<MDT>(dl, qf[j][s][h], acc1[sub][h]);
                acc1[sub][h] = mfma16x16x32<MDT>(dh, qfl[j][s][h], acc1[sub][h]);
                acc1[sub][h] = mfma16x16x32<MDT>(dh, qf[j][s][h], acc1[sub][h]);
              }
            }
          } else {
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
              for (int sub = 0; sub < NSUB; sub++)
                acc1[sub][h] = mfma16x16x32<MDT>(buf.f[sub][s], qf[j][s][h], acc1[sub][h]);
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
        if constexpr (F32) split_bf16(buf.f[sub][s], dh[sub], dl[sub]);
        else dh[sub] = buf.f[sub][s];
      }
#pragma unroll
      for (int j = 0; j < NQB; j++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
          const int qi = ((j * a.nstep + S) * 2 + h) * 64 + lane;
          const u32x4 qv = qlds[qi];
          if constexpr (F32) {
            const u32x4 qlv = qlds[nfrag + qi];
#pragma unroll
            for (int sub = 0; sub < NSUB; sub++) {
              acc[sub][j][h] = mfma16x16x32<MDT>(dl[sub], qv, acc[sub][j][h]);
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

// Writes v into out[0..n).
__global__ void fill_kernel(float* out, int64_t n, float v) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = v;
}

static int fill(float* out, int64_t n, float v, hipStream_t st) {
  if (n <= 0) return TMS_OK;
  int64_t grid = (n + 255) / 256;
  hipLaunchKernelGGL(fill_kernel, dim3((unsigned)grid), dim3(256), 0, st, out, n, v);
  return check_launch("fill");
}

// ------------------------------------------------------------------------------
// host dispatch
// ------------------------------------------------------------------------------
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
#ifndef TMS_DENSE_PFD
#define TMS_DENSE_PFD 1  // tiles in flight ahead of the one being scored
#endif

// LDS bytes of the query fragments of one launch (fp32: hi and lo terms).
static size_t qlds_bytes(int dtype, int nqb, int nstep) {
  return (size_t)nqb * nstep * 2 * 64 * 16 * (dtype == TMS_DTYPE_F32 ? 2 : 1);
}

template <int DT, int MODE, int NQB, int KS_REG, bool FULL, bool ALIGNED, int NT>
static int launch_nt(const DenseArgs& a, int64_t waves, size_t lds, hipStream_t st) {
  // fp32 tiles hold twice the bytes per token: with Q in VGPRs, one 16-token row block
  // per tile keeps the bytes in flight per wave where the 16-bit path has them; with Q
  // in LDS (d > 128: its lo terms take up to 128 KiB, one or two workgroups per CU) two
  // blocks per tile keep more bytes in flight per wave (measured: +20 % at d = 768,
  // +12 % at d = 1000, within 4 % either way at d = 200 .. 512)
  constexpr int NS = DT == TMS_DTYPE_F32 ? (KS_REG > 0 ? TMS_DENSE_F32_NSUB : TMS_DENSE_F32_LDS_NSUB) : kNSub;
  const int64_t grid = (waves + NT / 64 - 1) / (NT / 64);
  if (lds > 64 * 1024) {
    int dev = 0, cap = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cap, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
      return fail(TMS_ERR_HIP, "dense_maxsim_kernel: cannot query the LDS limit");
    if (lds > (size_t)cap)
      return fail(TMS_ERR_UNSUPPORTED, "dense_maxsim_kernel: query fragments need %zu bytes of LDS, the device has %d",
                  lds, cap);
  }
  hipLaunchKernelGGL((dense_maxsim_kernel<DT, MODE, NQB, KS_REG, FULL, ALIGNED, NS, TMS_DENSE_PFD, NT>),
                     dim3((unsigned)grid), dim3(NT), lds, st, a);
  return check_launch("dense_maxsim_kernel");
}

// fp32 with Q in LDS above 80 KiB (d >= 768: the query's hi and lo terms leave room for
// one workgroup per CU): 8-wave workgroups, so the CU still holds two waves per SIMD
// (d = 768: 5.2 -> 5.8 TB/s, d = 1000: 4.5 -> 5.1 TB/s). Below that, 4-wave
// workgroups (8-wave ones measured 5 % slower at d = 200 and 512).
template <int DT, int MODE, int NQB, int KS_REG, bool FULL, bool ALIGNED>
static int launch_one(const DenseArgs& a, int64_t waves, size_t lds, hipStream_t st) {
  if constexpr (DT == TMS_DTYPE_F32 && KS_REG == 0) {
    if (lds > 80 * 1024) return launch_nt<DT, MODE, NQB, KS_REG, FULL, ALIGNED, 512>(a, waves, lds, st);
  }
  return launch_nt<DT, MODE, NQB, KS_REG, FULL, ALIGNED, 256>(a, waves, lds, st);
}

template <int DT, int MODE, int NQB>
static int launch_nqb(const DenseArgs& a, bool aligned, int64_t waves, hipStream_t st) {
  const bool full = aligned && (a.d % 32 == 0);
  if (aligned && a.d > 0 && a.d <= 128 && a.d % 32 == 0) {
    switch (a.d / 32) {
      case 1: return launch_one<DT, MODE, NQB, 1, true, true>(a, waves, 0, st);
      case 2: return launch_one<DT, MODE, NQB, 2, true, true>(a, waves, 0, st);
      case 3: return launch_one<DT, MODE, NQB, 3, true, true>(a, waves, 0, st);
      default: return launch_one<DT, MODE, NQB, 4, true, true>(a, waves, 0, st);
    }
  }
  size_t lds = qlds_bytes(DT, NQB, a.nstep);
  if (lds == 0) lds = 16;
  if (full) return launch_one<DT, MODE, NQB, 0, true, true>(a, waves, lds, st);
  if (aligned) return launch_one<DT, MODE, NQB, 0, false, true>(a, waves, lds, st);
  return launch_one<DT, MODE, NQB, 0, false, false>(a, waves, lds, st);
}

// Documents per wave: short waves (about TMS_DENSE_TOKENS_PER_WAVE tokens, i.e. one
// document at typical ColBERT lengths) keep every CU's load pipeline full until the
// end of the launch and let the dispatcher balance ragged documents; the grid still
// spans at least two rounds of the chip's resident waves, and a wave never carries
// fewer tokens than it spends loading its query fragments.
static int pick_docs_per_wave(int64_t B, int64_t tokens_per_doc_hint) {
  int64_t dpw = tokens_per_doc_hint > 0 ? TMS_DENSE_TOKENS_PER_WAVE / tokens_per_doc_hint : 1;
  const int64_t min_waves = (int64_t)256 * 16 * 2;
  if (dpw > 1 && B / dpw < min_waves) dpw = B / min_waves;
  if (dpw < 1) dpw = 1;
  if (dpw > 64) dpw = 64;
  return (int)dpw;
}

template <int DT>
static int run_dense(DenseArgs a, int64_t nQ, int mode, bool aligned, hipStream_t st) {
  const int64_t nblocks_total = nQ * (int64_t)a.nbq;
  const int64_t waves = (a.B + a.docs_per_wave - 1) / a.docs_per_wave;
  // Blocks per launch: two when Q fits in VGPRs or its LDS copy stays small.
  int maxq = 2;
  if (!(aligned && a.d > 0 && a.d <= 128 && a.d % 32 == 0) && qlds_bytes(DT, 2, a.nstep) > (size_t)kMaxQldsBytes)
    maxq = 1;
  for (int64_t blk0 = 0; blk0 < nblocks_total; blk0 += maxq) {
    a.blk0 = (int32_t)blk0;
    a.nblk = (int32_t)((nblocks_total - blk0 < maxq) ? nblocks_total - blk0 : maxq);
    int rc;
    if (a.nblk == 2) {
      if (mode == MODE_FIXED) rc = launch_nqb<DT, MODE_FIXED, 2>(a, aligned, waves, st);
      else if (mode == MODE_VARLEN) rc = launch_nqb<DT, MODE_VARLEN, 2>(a, aligned, waves, st);
      else rc = launch_nqb<DT, MODE_MASKED, 2>(a, aligned, waves, st);
    } else {
      if (mode == MODE_FIXED) rc = launch_nqb<DT, MODE_FIXED, 1>(a, aligned, waves, st);
      else if (mode == MODE_VARLEN) rc = launch_nqb<DT, MODE_VARLEN, 1>(a, aligned, waves, st);
      else rc = launch_nqb<DT, MODE_MASKED, 1>(a, aligned, waves, st);
    }
    if (rc != TMS_OK) return rc;
  }
  return TMS_OK;
}

static int dense_entry(const char* fn, const void* Q, int64_t nQ, int64_t nq, int64_t d, const void* D, int64_t B,
                       int64_t nd, int64_t total_tokens, const int64_t* offsets, const uint8_t* mask, int mode,
                       int dtype, float* out, void* stream, int64_t pad_len = 0) {
  if (dtype != TMS_DTYPE_F16 && dtype != TMS_DTYPE_BF16 && dtype != TMS_DTYPE_F32)
    return fail(TMS_ERR_UNSUPPORTED, "%s: unsupported dtype %d", fn, dtype);
  if (pad_len < 0) return fail(TMS_ERR_INVALID, "%s: negative pad_len %lld", fn, (long long)pad_len);
  if (nQ < 0 || nq < 0 || d < 0 || B < 0 || nd < 0 || total_tokens < 0)
    return fail(TMS_ERR_INVALID, "%s: negative size (nQ=%lld nq=%lld d=%lld B=%lld nd=%lld T=%lld)", fn, (long long)nQ,
                (long long)nq, (long long)d, (long long)B, (long long)nd, (long long)total_tokens);
  if (B == 0 || nQ == 0) return TMS_OK;
  if (!out) return fail(TMS_ERR_INVALID, "%s: out is NULL", fn);
  hipStream_t st = (hipStream_t)stream;
  if (nq == 0) return fill(out, nQ * B, 0.f, st);
  if (!Q) return fail(TMS_ERR_INVALID, "%s: Q is NULL", fn);
  if (mode == MODE_VARLEN && !offsets) return fail(TMS_ERR_INVALID, "%s: offsets is NULL", fn);
  if (mode == MODE_MASKED && nd > 0 && !mask) return fail(TMS_ERR_INVALID, "%s: mask is NULL", fn);
  const int64_t rows = (mode == MODE_VARLEN) ? total_tokens : B * nd;
  if (rows > 0 && d > 0 && !D) return fail(TMS_ERR_INVALID, "%s: D is NULL", fn);
  if (d > 1024) return fail(TMS_ERR_UNSUPPORTED, "%s: d=%lld > 1024 is not supported", fn, (long long)d);
  if (nq > (int64_t)1 << 24 || nQ > (int64_t)1 << 20 || nQ * ((nq + 31) / 32) > ((int64_t)1 << 30))
    return fail(TMS_ERR_UNSUPPORTED, "%s: too many query tokens", fn);

  DenseArgs a;
  memset(&a, 0, sizeof(a));
  a.Q = (const uint8_t*)Q;
  a.D = (const uint8_t*)D;
  a.offsets = offsets;
  a.mask = mask;
  a.out = out;
  a.B = B;
  a.nd = nd;
  a.total_tokens = total_tokens;
  a.nq = (int32_t)nq;
  a.nbq = (int32_t)((nq + 31) / 32);
  a.d = (int32_t)d;
  a.nchunk = (int32_t)((d + 7) / 8);
  a.nstep = (int32_t)((d + 31) / 32);
  a.nkg = (int32_t)((a.nstep + 3) / 4);
  if (a.nkg < 1) a.nkg = 1;
  int64_t hint = (mode == MODE_VARLEN) ? (B > 0 ? total_tokens / B : 0) : nd;
  a.docs_per_wave = pick_docs_per_wave(B, hint);
  a.pad_len = pad_len;
  const bool aligned = (d % 8 == 0) && (((uintptr_t)Q & 15) == 0) && (((uintptr_t)D & 15) == 0);
  const bool qreg = aligned && d > 0 && d <= 128 && d % 32 == 0;
  if (dtype == TMS_DTYPE_F32) return run_dense<TMS_DTYPE_F32>(a, nQ, mode, aligned, st);
  if (mode == MODE_FIXED && qreg) return run_stream(Q, nQ, nq, d, D, B, nd, dtype, out, st);
  if (mode == MODE_VARLEN && qreg && a.nbq <= 4 && nQ * a.nbq >= 4)  // one pass for up to 32 blocks
    return run_varlen_batched(Q, nQ, nq, d, D, total_tokens, offsets, 0, B, pad_len, dtype, out, st);
  if (dtype == TMS_DTYPE_F16) return run_dense<TMS_DTYPE_F16>(a, nQ, mode, aligned, st);
  return run_dense<TMS_DTYPE_BF16>(a, nQ, mode, aligned, st);
}

}  // namespace tms

extern "C" {

int tms_version(void) { return 100; }

const char* tms_last_error(void) { return tms::g_err; }

int tms_maxsim_dense(const void* Q, int64_t nq, int64_t d, const void* D, int64_t B, int64_t nd, int dtype, float* out,
                     void* stream) {
  return tms::dense_entry("tms_maxsim_dense", Q, 1, nq, d, D, B, nd, 0, nullptr, nullptr, tms::MODE_FIXED, dtype, out,
                          stream);
}

int tms_maxsim_masked(const void* Q, int64_t nq, int64_t d, const void* D, const uint8_t* mask, int64_t B, int64_t nd,
                      int dtype, float* out, void* stream) {
  return tms::dense_entry("tms_maxsim_masked", Q, 1, nq, d, D, B, nd, 0, nullptr, mask, tms::MODE_MASKED, dtype, out,
                          stream);
}

int tms_maxsim_varlen(const void* Q, int64_t nq, int64_t d, const void* D_flat, int64_t total_tokens,
                      const int64_t* offsets, int64_t B, int dtype, float* out, void* stream) {
  return tms::dense_entry("tms_maxsim_varlen", Q, 1, nq, d, D_flat, B, 0, total_tokens, offsets, nullptr,
                          tms::MODE_VARLEN, dtype, out, stream);
}

int tms_maxsim_varlen_padded(const void* Q, int64_t nq, int64_t d, const void* D_flat, int64_t total_tokens,
                             const int64_t* offsets, int64_t B, int64_t pad_len, int dtype, float* out, void* stream) {
  return tms::dense_entry("tms_maxsim_varlen_padded", Q, 1, nq, d, D_flat, B, 0, total_tokens, offsets, nullptr,
                          tms::MODE_VARLEN, dtype, out, stream, pad_len);
}

int tms_maxsim_varlen_batched(const void* Qs, int64_t nQ, int64_t nq, int64_t d, const void* D_flat,
                              int64_t total_tokens, const int64_t* offsets, int64_t B, int64_t pad_len, int dtype,
                              float* out, void* stream) {
  return tms::dense_entry("tms_maxsim_varlen_batched", Qs, nQ, nq, d, D_flat, B, 0, total_tokens, offsets, nullptr,
                          tms::MODE_VARLEN, dtype, out, stream, pad_len);
}

int tms_maxsim_dense_batched(const void* Qs, int64_t nQ, int64_t nq, int64_t d, const void* D, int64_t B, int64_t nd,
                             int dtype, float* out, void* stream) {
  return tms::dense_entry("tms_maxsim_dense_batched", Qs, nQ, nq, d, D, B, nd, 0, nullptr, nullptr, tms::MODE_FIXED,
                          dtype, out, stream);
}

}  // extern "C"
