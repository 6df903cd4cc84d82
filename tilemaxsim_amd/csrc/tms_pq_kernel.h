// Product-quantised (PQ / ADC) MaxSim on MFMA: the codebook-gather kernel template and
// its launch helpers, shared by tms_pq.hip (uint8 codes, a query of the codebook's type),
// tms_pq_wide.hip (int16 / int32 codes) and tms_pq_q32.hip (fp32 queries against a
// 16-bit codebook), which build in parallel.
//
// Reference: src/flash_pqsim_kernel.py. Documents are (B, nd, M) codes into a codebook
// (M, K, dsub); token t decodes to concat_m codebook[m, codes[t, m]], and
//   score[b] = sum_q max_t <Q[q], decoded token t>,
// which is what the reference's table gather computes (:127-173, :283-313).
//
// The codebook (d * K elements, 64 KiB at M = 16, K = 256, dsub = 8, fp16) lives in LDS;
// each lane rebuilds its MFMA A-operand fragment (8 dims of one token) with one 16-byte
// LDS gather per (token, 8 dims), and the q . token dots run on MFMA with fp32
// accumulation, exactly like the dense kernel: 256 bytes of LDS per token instead of the
// fp32 table's 2 KiB, and the decoded vectors never touch HBM.
#pragma once
#include <string.h>

#include "tms_common.h"

#ifndef TMS_PQ_UT
#define TMS_PQ_UT 4  // 16-token subtiles per pipelined unit of the MFMA PQ kernel
#endif
#ifndef TMS_PQ_PIPE
#define TMS_PQ_PIPE 2  // 1: gathers one subtile ahead; 2: two ahead, split accumulators
#endif
#ifndef TMS_PQ_WAVE_ROUNDS
#define TMS_PQ_WAVE_ROUNDS 4  // grid covers the chip's resident waves about this many times
#endif

namespace tms {

struct PqArgs {
  const uint8_t* Q;         // (nq, d) elements of the query dtype
  const uint8_t* codebook;  // (M, K, DSUB)
  const uint8_t* codes;     // (B, nd, M) codes of CWB bytes each
  float* out;               // (B)
  int64_t B, nd;
  int32_t nq, nbq, blk0, nblk, K;
  int32_t docs_per_wave;
};

// Code i of a lane's code words: CWB-byte codes, little-endian, packed in 32-bit words.
template <int CWB>
__device__ __forceinline__ uint32_t code_at(const uint32_t* w, int i) {
  if constexpr (CWB == 1) return (w[i / 4] >> (8 * (i % 4))) & 0xffu;
  else if constexpr (CWB == 2) return (w[i / 2] >> (16 * (i % 2))) & 0xffffu;
  else return w[i];
}

// Lane (r = l%16, g = l/16) owns chunks c = g*KS + s (s < KS) of every token, i.e.
// dims [8*g*KS, 8*(g+1)*KS): a contiguous run of CB = 8*KS/DSUB subspaces whose
// codes are CB contiguous codes of the token's code row.
constexpr int kPqThreads = 512;  // 8 waves: two workgroups per CU next to a 64 KiB codebook

// DT: codebook type; QDT: query type (DT, or fp32: each query element split into hi + lo
// terms of DT, two MFMAs per product, as in the dense kernel); CWB: bytes per code (1, 2
// or 4); CLAMP: codes >= K (invalid input) are clamped into the table -- off only for
// uint8 codes with K == 256, where every byte is a valid code and K is a constant.
template <int DT, int QDT, int CWB, bool CLAMP, int DSUB, int KS, int NQB, int UT>
__global__ void __launch_bounds__(kPqThreads) pq_mfma_score_kernel(PqArgs a) {
  constexpr int D = 32 * KS;
  constexpr int M = D / DSUB;
  constexpr int CB = M / 4;                  // codes per lane per token
  constexpr int LB = CB * CWB;               // ... their bytes
  constexpr int CW = (LB + 3) / 4;           // ... in 32-bit words
  // widest load dividing a lane's run (and so a token row, 4 runs, 16-byte aligned codes)
  constexpr int LU = LB % 16 == 0 ? 16 : LB % 8 == 0 ? 8 : LB % 4 == 0 ? 4 : LB % 2 == 0 ? 2 : 1;
  constexpr bool QSPLIT = QDT == TMS_DTYPE_F32;
  constexpr bool QSCALE = QSPLIT && DT == TMS_DTYPE_F16;
  static_assert(!QSPLIT || DT != TMS_DTYPE_F32, "fp32 codebooks take the table path");
  static_assert(CLAMP || CWB == 1, "only uint8 codes can skip the clamp (with K == 256)");
  using QRaw = typename Raw8<QDT>::T;
  extern __shared__ u32x4 cb_lds[];          // codebook, M*K*DSUB elements
  const int lane = threadIdx.x & 63;
  const int r = lane & 15, g = lane >> 4;
  const int K = CLAMP ? a.K : 256;

  {  // codebook -> LDS (16-byte units; M*K*DSUB*2 is a multiple of 16 since D % 32 == 0)
    const int64_t n16 = (int64_t)M * K * DSUB * 2 / 16;
    const u32x4* src = (const u32x4*)a.codebook;
    for (int64_t i = threadIdx.x; i < n16; i += blockDim.x) cb_lds[i] = src[i];
  }

  // Query fragments: block j, half h, step s -> row token 16h + r, chunk g*KS + s.
  auto q_row = [&](int j, int h, int rr, bool& valid) -> int64_t {
    int jb = a.blk0 + j;
    int tok = jb * 32 + 16 * h + rr;
    valid = (j < a.nblk) && (tok < a.nq);
    return tok;
  };
  u32x4 qf[NQB][KS][2];
  u32x4 qfl[QSPLIT ? NQB : 1][QSPLIT ? KS : 1][2];  // split queries: the lo terms
  float qinv[NQB][2];                               // QSCALE: 1 / the column token's scale
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
        if constexpr (QSPLIT) {
          const u32x4* p = (const u32x4*)(a.Q + (row * D + 8 * (g * KS + s)) * 4);
          const u32x4 x0 = valid ? p[0] : u32x4{0u, 0u, 0u, 0u}, x1 = valid ? p[1] : u32x4{0u, 0u, 0u, 0u};
          raw[s] = QRaw{x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
          if constexpr (QSCALE) am = fmaxf(am, absmax8(raw[s]));
        } else {
          raw[s] = valid ? *(const u32x4*)(a.Q + (row * D + 8 * (g * KS + s)) * 2) : u32x4{0u, 0u, 0u, 0u};
        }
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
        else if constexpr (QSPLIT) split_bf16(raw[s], qf[j][s][h], qfl[j][s][h]);
        else qf[j][s][h] = raw[s];
      }
    }
  __syncthreads();

  const int64_t wave = (int64_t)blockIdx.x * (kPqThreads / 64) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t b_begin = wave_uniform(wave * a.docs_per_wave);
  if (b_begin >= a.B) return;
  const int64_t b_end = (b_begin + a.docs_per_wave < a.B) ? b_begin + a.docs_per_wave : a.B;
  const float NEG_INF = -__builtin_inff();
  const int64_t nd = a.nd;

  f32x4 rmax[NQB][2];
#pragma unroll
  for (int j = 0; j < NQB; j++) rmax[j][0] = rmax[j][1] = f32x4{NEG_INF, NEG_INF, NEG_INF, NEG_INF};

  auto write_doc = [&](int64_t b, float s_total) {
    if (lane == 0) {
      float* o = a.out + b;
      *o = (a.blk0 > 0) ? (*o + s_total) : s_total;
    }
  };
  // Max over the document's tokens (the 4 accumulator rows of a lane, then the four
  // 16-lane row groups) and sum over the query tokens (the 16 columns of a row). The
  // cross-lane steps use row swaps and DPP, which leave the LDS to the gathers.
  auto finish_doc = [&](int64_t b) {
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < NQB; j++)
#pragma unroll
      for (int h = 0; h < 2; h++) {
        float m = fmaxf(fmaxf(rmax[j][h][0], rmax[j][h][1]), fmaxf(rmax[j][h][2], rmax[j][h][3]));
        m = cross_row_max(m);
        if constexpr (QSCALE) m *= qinv[j][h];  // exact: a power of two
        bool valid;
        (void)q_row(j, h, r, valid);
        s += valid ? m : 0.f;
        rmax[j][h] = f32x4{NEG_INF, NEG_INF, NEG_INF, NEG_INF};
      }
    write_doc(b, row_sum16(s));
  };

  // Code words of this lane for UT subtiles of 16 tokens starting at token t0 of doc b.
  struct Codes {
    uint32_t w[UT][CW];
  };
  // b and t0 are wave-uniform, so the unit's base address is scalar; each lane adds a
  // 32-bit offset. Tokens past the document's end are clamped to its last token.
  auto load_codes = [&](Codes& c, int64_t b, int64_t t0) {
    const uint8_t* base = a.codes + (b * nd + t0) * (M * CWB);
    const int64_t left = nd - 1 - t0;
    const int last = left < 16 * UT ? (int)left : 16 * UT - 1;
#pragma unroll
    for (int u = 0; u < UT; u++) {
      const int tr = min(16 * u + r, last);
      const uint8_t* p = base + (uint32_t)((tr * M + g * CB) * CWB);
      if constexpr (LU == 16) {
#pragma unroll
        for (int i = 0; i < LB / 16; i++) {
          const u32x4 v = ld_stream<u32x4, true>(p + 16 * i);
          c.w[u][4 * i] = v[0];
          c.w[u][4 * i + 1] = v[1];
          c.w[u][4 * i + 2] = v[2];
          c.w[u][4 * i + 3] = v[3];
        }
      } else if constexpr (LU == 8) {
#pragma unroll
        for (int i = 0; i < LB / 8; i++) {
          const u32x2 v = ld_stream<u32x2, true>(p + 8 * i);
          c.w[u][2 * i] = v[0];
          c.w[u][2 * i + 1] = v[1];
        }
      } else if constexpr (LU == 4) {
#pragma unroll
        for (int i = 0; i < LB / 4; i++) c.w[u][i] = ld_stream<uint32_t, true>(p + 4 * i);
      } else {
#pragma unroll
        for (int i = 0; i < CW; i++) c.w[u][i] = 0;
        if constexpr (LU == 2) {
#pragma unroll
          for (int i = 0; i < LB / 2; i++) c.w[u][i / 2] |= (uint32_t)ld_stream<uint16_t, true>(p + 2 * i) << (16 * (i % 2));
        } else {
#pragma unroll
          for (int i = 0; i < LB; i++) c.w[u][i / 4] |= (uint32_t)ld_stream<uint8_t, true>(p + i) << (8 * (i % 4));
        }
      }
    }
  };
  auto code_of = [&](const Codes& c, int u, int i) -> uint32_t {
    const uint32_t x = code_at<CWB>(c.w[u], i);
    if constexpr (CLAMP) return min(x, (uint32_t)(K - 1));
    else return x;
  };

  // Decoded A fragment for chunk g*KS + s of the token held in subtile u.
  auto gather = [&](const Codes& c, int u, int s) -> u32x4 {
    const int cidx = g * KS + s;
    if constexpr (DSUB >= 8) {
      constexpr int P = DSUB / 8;  // 16-byte pieces per sub-vector
      const int m = cidx / P;
      const uint32_t code = code_of(c, u, s / P);
      return cb_lds[((uint32_t)m * (uint32_t)K + code) * P + (cidx % P)];
    } else {
      constexpr int P = 8 / DSUB;  // sub-vectors per chunk
      u32x4 v;
      if constexpr (DSUB == 4) {
        const uint2* cb8 = (const uint2*)cb_lds;
#pragma unroll
        for (int p = 0; p < 2; p++) {
          const int m = cidx * P + p;
          uint2 x = cb8[(uint32_t)m * (uint32_t)K + code_of(c, u, s * P + p)];
          v[2 * p] = x.x;
          v[2 * p + 1] = x.y;
        }
      } else {  // DSUB == 2
        const uint32_t* cb4 = (const uint32_t*)cb_lds;
#pragma unroll
        for (int p = 0; p < 4; p++) {
          const int m = cidx * P + p;
          v[p] = cb4[(uint32_t)m * (uint32_t)K + code_of(c, u, s * P + p)];
        }
      }
      return v;
    }
  };

  // q . token for one query block half: fp32 queries add the lo term's MFMA first.
  auto mma = [&](const u32x4 (&fr)[KS], int j, int h, f32x4 acc) -> f32x4 {
#pragma unroll
    for (int s = 0; s < KS; s++) {
      if constexpr (QSPLIT) acc = mfma16x16x32<DT>(fr[s], qfl[j][s][h], acc);
      acc = mfma16x16x32<DT>(fr[s], qf[j][s][h], acc);
    }
    return acc;
  };

  // Subtiles past the end of a document hold clamped duplicates of its last token,
  // which cannot change a max, so every unit runs all UT subtiles without a branch.
  // The LDS gathers of subtile u+1 are issued before the MFMAs of subtile u.
  auto gather_sub = [&](u32x4 (&fr)[KS], const Codes& c, int u) {
#pragma unroll
    for (int s = 0; s < KS; s++) fr[s] = gather(c, u, s);
  };
  auto mfma_sub = [&](const u32x4 (&fr)[KS]) {
#pragma unroll
    for (int j = 0; j < NQB; j++)
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const f32x4 acc = mma(fr, j, h, f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
        for (int i = 0; i < 4; i++) rmax[j][h][i] = fmaxf(rmax[j][h][i], acc[i]);
      }
  };
#if TMS_PQ_PIPE == 1
  auto compute = [&](const Codes& c, int64_t) {
    u32x4 fa[KS], fb[KS];
    gather_sub(fa, c, 0);
#pragma unroll
    for (int u = 0; u < UT; u += 2) {
      if (u + 1 < UT) gather_sub(fb, c, u + 1);
      mfma_sub(fa);
      if (u + 2 < UT) gather_sub(fa, c, u + 2);
      if (u + 1 < UT) mfma_sub(fb);
    }
  };
#else
  // Gathers run two subtiles ahead (three fragment buffers) and the running max of
  // subtile u-1 is taken after the MFMAs of subtile u are issued (two accumulator
  // sets), so LDS latency and MFMA latency overlap with independent work.
  auto compute = [&](const Codes& c, int64_t) {
    u32x4 fr[3][KS];
    f32x4 acc[2][NQB][2];
    gather_sub(fr[0], c, 0);
    if (UT > 1) gather_sub(fr[1], c, 1);
    auto take_max = [&](int p) {
#pragma unroll
      for (int j = 0; j < NQB; j++)
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
          for (int i = 0; i < 4; i++) rmax[j][h][i] = fmaxf(rmax[j][h][i], acc[p][j][h][i]);
    };
#pragma unroll
    for (int u = 0; u < UT; u++) {
#pragma unroll
      for (int j = 0; j < NQB; j++)
#pragma unroll
        for (int h = 0; h < 2; h++) acc[u & 1][j][h] = mma(fr[u % 3], j, h, f32x4{0.f, 0.f, 0.f, 0.f});
      if (u + 2 < UT) gather_sub(fr[(u + 2) % 3], c, u + 2);
      if (u > 0) take_max((u - 1) & 1);
    }
    take_max((UT - 1) & 1);
  };
#endif

  if (nd == 0) {
    for (int64_t b = b_begin; b < b_end; b++) write_doc(b, NEG_INF);
    return;
  }
  constexpr int TT = 16 * UT;
  // Pipeline over (doc, t0) units of TT tokens: codes of the next unit are in flight
  // while the current unit is decoded and scored.
  int64_t cb = b_begin, ct = 0;
  Codes c0, c1;
  load_codes(c0, cb, ct);
  auto step = [&](int64_t& b, int64_t& t) {
    t += TT;
    if (t >= nd) {
      t = 0;
      b++;
    }
  };
  while (true) {
    int64_t nb = cb, nt = ct;
    step(nb, nt);
    if (nb < b_end) load_codes(c1, nb, nt);
    compute(c0, ct);
    if (ct + TT >= nd) finish_doc(cb);
    if (nb >= b_end) break;
    cb = nb;
    ct = nt;
    step(nb, nt);
    if (nb < b_end) load_codes(c0, nb, nt);
    compute(c1, ct);
    if (ct + TT >= nd) finish_doc(cb);
    if (nb >= b_end) break;
    cb = nb;
    ct = nt;
  }
}

// ------------------------------------------------------------------------------
// launch helpers
// ------------------------------------------------------------------------------
constexpr int kPqUT = TMS_PQ_UT;

template <int DT, int QDT, int CWB, bool CLAMP, int DSUB, int KS, int NQB>
static int launch_mfma_one(const PqArgs& a, int64_t grid, size_t lds, hipStream_t st) {
  hipLaunchKernelGGL((pq_mfma_score_kernel<DT, QDT, CWB, CLAMP, DSUB, KS, NQB, kPqUT>), dim3((unsigned)grid),
                     dim3(kPqThreads), lds, st, a);
  return check_launch("pq_mfma_score_kernel");
}

// Query blocks per launch: two, or one for split queries and wide codes, whose lo terms
// and code words would otherwise spill at two blocks.
template <int QDT, int CWB>
constexpr int pq_max_blocks() {
  return (QDT == TMS_DTYPE_F32 || CWB > 1) ? 1 : 2;
}

template <int DT, int QDT, int CWB, bool CLAMP, int DSUB, int KS>
static int launch_mfma_nqb(const PqArgs& a, int64_t grid, size_t lds, hipStream_t st) {
  if constexpr (pq_max_blocks<QDT, CWB>() == 2) {
    if (a.nblk == 2) return launch_mfma_one<DT, QDT, CWB, CLAMP, DSUB, KS, 2>(a, grid, lds, st);
  }
  return launch_mfma_one<DT, QDT, CWB, CLAMP, DSUB, KS, 1>(a, grid, lds, st);
}

// Only the (dsub, d = 32 * ks) pairs with M = d / dsub a multiple of 4 are instantiated.
template <int DT, int QDT, int CWB, bool CLAMP, int DSUB>
static int launch_mfma_ks(const PqArgs& a, int ks, int64_t grid, size_t lds, hipStream_t st) {
  if constexpr (DSUB <= 8) {
    switch (ks) {
      case 1: return launch_mfma_nqb<DT, QDT, CWB, CLAMP, DSUB, 1>(a, grid, lds, st);
      case 2: return launch_mfma_nqb<DT, QDT, CWB, CLAMP, DSUB, 2>(a, grid, lds, st);
      case 3: return launch_mfma_nqb<DT, QDT, CWB, CLAMP, DSUB, 3>(a, grid, lds, st);
      default: return launch_mfma_nqb<DT, QDT, CWB, CLAMP, DSUB, 4>(a, grid, lds, st);
    }
  } else if constexpr (DSUB == 16) {
    if (ks == 2) return launch_mfma_nqb<DT, QDT, CWB, CLAMP, DSUB, 2>(a, grid, lds, st);
    return launch_mfma_nqb<DT, QDT, CWB, CLAMP, DSUB, 4>(a, grid, lds, st);
  } else {
    return launch_mfma_nqb<DT, QDT, CWB, CLAMP, DSUB, 4>(a, grid, lds, st);
  }
}

template <int DT, int QDT, int CWB, bool CLAMP>
static int launch_mfma_dsub(const PqArgs& a, int dsub, int ks, int64_t grid, size_t lds, hipStream_t st) {
  switch (dsub) {
    case 2: return launch_mfma_ks<DT, QDT, CWB, CLAMP, 2>(a, ks, grid, lds, st);
    case 4: return launch_mfma_ks<DT, QDT, CWB, CLAMP, 4>(a, ks, grid, lds, st);
    case 8: return launch_mfma_ks<DT, QDT, CWB, CLAMP, 8>(a, ks, grid, lds, st);
    case 16: return launch_mfma_ks<DT, QDT, CWB, CLAMP, 16>(a, ks, grid, lds, st);
    default: return launch_mfma_ks<DT, QDT, CWB, CLAMP, 32>(a, ks, grid, lds, st);
  }
}

// One query (a.nbq blocks of 32 tokens, up to two per launch) over every document. The host has
// checked the shape (mfma_shape_ok in tms_pq.hip). A codebook above 64 KiB of LDS leaves
// room for one 8-wave workgroup per CU instead of two.
template <int DT, int QDT, int CWB>
static int run_pq_mfma(PqArgs a, int64_t M, int64_t dsub, hipStream_t st) {
  const int64_t d = M * dsub;
  const int ks = (int)(d / 32);
  const size_t lds = (size_t)d * a.K * 2;
  const int64_t wg_per_cu = lds > 64 * 1024 ? 1 : 2;
  // each wave gets a long run of documents (about TMS_PQ_WAVE_ROUNDS rounds of the chip)
  // so the per-workgroup codebook load is amortised and the last round stays short
  const int64_t waves_per_wg = kPqThreads / 64;
  const int64_t target_waves = (int64_t)256 * wg_per_cu * waves_per_wg * TMS_PQ_WAVE_ROUNDS;
  int64_t dpw = (a.B + target_waves - 1) / target_waves;
  if (dpw < 1) dpw = 1;
  a.docs_per_wave = (int32_t)dpw;
  const int64_t waves = (a.B + dpw - 1) / dpw;
  const int64_t grid = (waves + waves_per_wg - 1) / waves_per_wg;
  const bool clamp = !(CWB == 1 && a.K == 256);
  constexpr int kMaxB = pq_max_blocks<QDT, CWB>();
  for (int64_t blk0 = 0; blk0 < a.nbq; blk0 += kMaxB) {
    a.blk0 = (int32_t)blk0;
    a.nblk = (int32_t)((a.nbq - blk0 < kMaxB) ? a.nbq - blk0 : kMaxB);
    int rc;
    if constexpr (CWB == 1) {
      rc = clamp ? launch_mfma_dsub<DT, QDT, CWB, true>(a, (int)dsub, ks, grid, lds, st)
                 : launch_mfma_dsub<DT, QDT, CWB, false>(a, (int)dsub, ks, grid, lds, st);
    } else {
      rc = launch_mfma_dsub<DT, QDT, CWB, true>(a, (int)dsub, ks, grid, lds, st);
    }
    if (rc) return rc;
  }
  return TMS_OK;
}

// Entry points of the other translation units (same arguments as run_pq_mfma; dtype is
// the codebook's 16-bit type).
int run_pq_mfma_wide(const PqArgs& a, int dtype, int code_bytes, int64_t M, int64_t dsub, hipStream_t st);
int run_pq_mfma_q32(const PqArgs& a, int dtype, int64_t M, int64_t dsub, hipStream_t st);

}  // namespace tms
