// Product-quantised (PQ / ADC) MaxSim on gfx950.
//
// Reference: src/flash_pqsim_kernel.py. Documents are (B, nd, M) uint8 codes into a
// codebook (M, K, dsub); token t decodes to concat_m codebook[m, codes[t, m]].
//   score[b] = sum_q max_t sum_m lut[q, m, codes[b, t, m]],
//   lut[q, m, k] = sum_j Q[q, m*dsub + j] * codebook[m, k, j]          (:31-67, :127-173)
// which equals MaxSim of Q against the decoded vectors (:283-313).
//
// Three kernels:
//  * pq_build_lut_kernel  -- the fp32 distance table (TileMaxSimPQ.build_distance_table).
//  * pq_lut_score_kernel  -- the reference algorithm: gathers from the fp32 table held
//    in LDS (a slice of QG query tokens at a time), fp32 adds in ascending m.
//    Any M, K <= 256, dsub. LDS-gather bound: 4 bytes of LDS per (token, q, m).
//  * pq_mfma_score_kernel -- the fast path: the codebook (64 KiB at M=16, K=256,
//    dsub=8, fp16) lives in LDS; each lane rebuilds its MFMA A-operand fragment
//    (8 dims of one token) with one 16-byte LDS gather per (token, 8 dims), and the
//    q . token dots run on MFMA with fp32 accumulation, exactly like the dense
//    kernel. 256 bytes of LDS per token instead of the table's 2 KiB, and the
//    decoded vectors never touch HBM.
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

template <int DT>
__device__ __forceinline__ float elem_to_f32(uint16_t bits) {
  if constexpr (DT == TMS_DTYPE_F16) {
    return (float)__builtin_bit_cast(_Float16, bits);
  } else {
    return __builtin_bit_cast(float, (uint32_t)bits << 16);
  }
}

// ------------------------------------------------------------------------------
// distance table
// ------------------------------------------------------------------------------
// Element i of an fp16 / bf16 / fp32 array, as fp32 (exact).
template <int DT>
__device__ __forceinline__ float load_elem(const void* __restrict__ p, int64_t i) {
  if constexpr (DT == TMS_DTYPE_F32) return ((const float*)p)[i];
  else return elem_to_f32<DT>(((const uint16_t*)p)[i]);
}

// T[q, m, k] = sum_j Q[q, m*dsub + j] * C[m, k, j] in fp32, accumulated with fused
// multiply-adds in j order (the reference's _build_distance_table_kernel,
// src/flash_pqsim_kernel.py:31-67, rounds each product and sums them with tl.sum; for
// fp16 / bf16 inputs the products are exact either way).
template <int DT>
__global__ void __launch_bounds__(256) pq_build_lut_kernel(const void* __restrict__ Q, const void* __restrict__ C,
                                                           float* __restrict__ lut, int64_t total, int M, int K,
                                                           int dsub) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int k = (int)(i % K);
  const int m = (int)((i / K) % M);
  const int64_t q = i / ((int64_t)K * M);
  const int64_t qb = (q * M + m) * dsub;
  const int64_t cb = ((int64_t)m * K + k) * dsub;
  float s = 0.f;
  for (int j = 0; j < dsub; j++) s = __builtin_fmaf(load_elem<DT>(Q, qb + j), load_elem<DT>(C, cb + j), s);
  lut[i] = s;
}

// ------------------------------------------------------------------------------
// table-gather scoring (reference algorithm)
// ------------------------------------------------------------------------------
struct LutArgs {
  const float* lut;      // (nq, M, K)
  const uint8_t* codes;  // (B, nd, M)
  float* out;            // (B)
  int64_t B, nd;
  int32_t nq, M, K;
  int32_t docs_per_wave;  // <= 64
};

// One lane per document token; a workgroup of 16 waves shares one slice of the table in
// LDS: QG query tokens, [m][k][QG] fp32 (zero past nq), at most 64 KiB, so two
// workgroups (32 waves) share a CU and hide each other's gather latency. Each lane loads
// its token's M code bytes with one or a few wide loads, gathers its M rows of QG values
// and adds them in ascending m, as the reference sums them (:154-167), then keeps a
// running max per query token. A document's maxima are taken across the wave with DPP and
// row swaps, and its partial score (the slice's query tokens) accumulates in lane
// b - b_begin. Slices loop inside the kernel, so the codes are read once per slice.
// CW: 4 = M is 16 and each token's codes are one 16-byte load; 1 = M % 4 == 0, 4-byte
// loads; 0 = byte loads (any M).
#ifndef TMS_LUT_SLICE_FLOATS
#define TMS_LUT_SLICE_FLOATS 16384  // table slice in LDS: 64 KiB, two workgroups per CU
#endif
constexpr int kLutThreads = 1024;
constexpr int kLutSliceFloats = TMS_LUT_SLICE_FLOATS;

__device__ __forceinline__ float row_max16(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_f32<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_f32<0x141>(v));  // row_half_mirror
  v = fmaxf(v, dpp_f32<0x140>(v));  // row_mirror
  return v;
}

template <int QG, int CW>
__global__ void __launch_bounds__(kLutThreads) pq_lut_score_kernel(LutArgs a) {
  __shared__ float lds[kLutSliceFloats];
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * (kLutThreads / 64) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t b_begin = wave_uniform(wave * a.docs_per_wave);
  const int64_t b_end = (b_begin + a.docs_per_wave < a.B) ? b_begin + a.docs_per_wave : a.B;
  const int M = a.M, K = a.K, MK = a.M * a.K;
  const int64_t nd = a.nd;
  const float NEG_INF = -__builtin_inff();

  // Accumulate the rows of the code bytes in `word` (subspaces m0 .. m0+n-1) into s.
  auto gather4 = [&](float (&s)[QG], uint32_t word, int m0, int n) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      if (i < n) {
        const uint32_t code = min((word >> (8 * i)) & 0xffu, (uint32_t)(K - 1));
        const float* row = lds + ((uint32_t)(m0 + i) * (uint32_t)K + code) * QG;
#pragma unroll
        for (int j = 0; j < QG; j++) s[j] += row[j];
      }
    }
  };

  float partial = 0.f;  // lane j: running score of document b_begin + j
  for (int q0 = 0; q0 < a.nq; q0 += QG) {
    __syncthreads();
    for (int i = threadIdx.x; i < MK * QG; i += kLutThreads) {  // reads run along mk
      const int qq = i / MK, mk = i - qq * MK;
      const int q = q0 + qq;
      lds[mk * QG + qq] = (q < a.nq) ? a.lut[(int64_t)q * MK + mk] : 0.f;
    }
    __syncthreads();
    for (int64_t b = b_begin; b < b_end; b++) {
      float mx[QG];
#pragma unroll
      for (int j = 0; j < QG; j++) mx[j] = NEG_INF;
      for (int64_t t0 = 0; t0 < nd; t0 += 64) {
        const int64_t t = (t0 + lane < nd) ? t0 + lane : nd - 1;  // duplicate of the last token: max unchanged
        const uint8_t* cp = a.codes + (b * nd + t) * M;
        float s[QG];
#pragma unroll
        for (int j = 0; j < QG; j++) s[j] = 0.f;
        if constexpr (CW == 4) {
          const uint4 v = *(const uint4*)cp;
          gather4(s, v.x, 0, 4);
          gather4(s, v.y, 4, 4);
          gather4(s, v.z, 8, 4);
          gather4(s, v.w, 12, 4);
        } else if constexpr (CW == 1) {
          for (int m0 = 0; m0 < M; m0 += 4) gather4(s, *(const uint32_t*)(cp + m0), m0, 4);
        } else {
          for (int m = 0; m < M; m++) gather4(s, cp[m], m, 1);
        }
#pragma unroll
        for (int j = 0; j < QG; j++) mx[j] = fmaxf(mx[j], s[j]);
      }
      float tot = 0.f;
#pragma unroll
      for (int j = 0; j < QG; j++) {
        const float v = cross_row_max(row_max16(mx[j]));
        tot += (q0 + j < a.nq) ? v : 0.f;
      }
      if (nd == 0) tot = NEG_INF;
      if (lane == (int)(b - b_begin)) partial += tot;
    }
  }
  if (b_begin < a.B && lane < b_end - b_begin) a.out[b_begin + lane] = partial;
}

// ------------------------------------------------------------------------------
// codebook-gather + MFMA scoring (fast path)
// ------------------------------------------------------------------------------
struct PqArgs {
  const uint8_t* Q;         // (nq, d) elements of the input dtype
  const uint8_t* codebook;  // (M, K, DSUB)
  const uint8_t* codes;     // (B, nd, M)
  float* out;               // (B)
  int64_t B, nd;
  int32_t nq, nbq, blk0, nblk, K;
  int32_t docs_per_wave;
};

// Lane (r = l%16, g = l/16) owns chunks c = g*KS + s (s < KS) of every token, i.e.
// dims [8*g*KS, 8*(g+1)*KS): a contiguous run of CB = 8*KS/DSUB subspaces whose
// codes are CB contiguous bytes of the token's code row.
constexpr int kPqThreads = 512;  // 8 waves: two workgroups per CU next to a 64 KiB codebook

template <int DT, int DSUB, int KS, int NQB, int UT>
__global__ void __launch_bounds__(kPqThreads) pq_mfma_score_kernel(PqArgs a) {
  constexpr int D = 32 * KS;
  constexpr int M = D / DSUB;
  constexpr int CB = M / 4;                  // code bytes per lane per token
  constexpr int CW = (CB + 3) / 4;           // ... in 32-bit words
  extern __shared__ u32x4 cb_lds[];          // codebook, M*K*DSUB elements
  const int lane = threadIdx.x & 63;
  const int r = lane & 15, g = lane >> 4;
  const int K = a.K;

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
#pragma unroll
  for (int j = 0; j < NQB; j++)
#pragma unroll
    for (int h = 0; h < 2; h++) {
      bool valid;
      int64_t row = q_row(j, h, r, valid);
#pragma unroll
      for (int s = 0; s < KS; s++)
        qf[j][s][h] = valid ? *(const u32x4*)(a.Q + (row * D + 8 * (g * KS + s)) * 2) : u32x4{0u, 0u, 0u, 0u};
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
  // 32-bit offset (the host guarantees nd * M < 2^31). Tokens past the document's end
  // are clamped to its last token.
  auto load_codes = [&](Codes& c, int64_t b, int64_t t0) {
    const uint8_t* base = a.codes + (b * nd + t0) * M;
    const int64_t left = nd - 1 - t0;
    const int last = left < 16 * UT ? (int)left : 16 * UT - 1;
#pragma unroll
    for (int u = 0; u < UT; u++) {
      const int tr = min(16 * u + r, last);
      const uint8_t* p = base + (uint32_t)(tr * M + g * CB);
      if constexpr (CB == 4) {
        c.w[u][0] = *(const uint32_t*)p;
      } else if constexpr (CB == 8) {
        uint2 v = *(const uint2*)p;
        c.w[u][0] = v.x;
        c.w[u][1] = v.y;
      } else if constexpr (CB == 16) {
        uint4 v = *(const uint4*)p;
        c.w[u][0] = v.x;
        c.w[u][1] = v.y;
        c.w[u][2] = v.z;
        c.w[u][3] = v.w;
      } else if constexpr (CB == 2) {
        c.w[u][0] = *(const uint16_t*)p;
      } else {
#pragma unroll
        for (int i = 0; i < CW; i++) c.w[u][i] = 0;
#pragma unroll
        for (int i = 0; i < CB; i++) c.w[u][i / 4] |= (uint32_t)p[i] << (8 * (i % 4));
      }
    }
  };
  // codes >= K (invalid input) are clamped so the gather stays inside the table
  auto code_byte = [&](const Codes& c, int u, int i) -> uint32_t {
    return min((c.w[u][i / 4] >> (8 * (i % 4))) & 0xffu, (uint32_t)(K - 1));
  };

  // Decoded A fragment for chunk g*KS + s of the token held in subtile u.
  auto gather = [&](const Codes& c, int u, int s) -> u32x4 {
    const int cidx = g * KS + s;
    if constexpr (DSUB >= 8) {
      constexpr int P = DSUB / 8;  // 16-byte pieces per sub-vector
      const int m = cidx / P;
      const uint32_t code = code_byte(c, u, s / P);
      return cb_lds[((int64_t)m * K + code) * P + (cidx % P)];
    } else {
      constexpr int P = 8 / DSUB;  // sub-vectors per chunk
      u32x4 v;
      if constexpr (DSUB == 4) {
        const uint2* cb8 = (const uint2*)cb_lds;
#pragma unroll
        for (int p = 0; p < 2; p++) {
          const int m = cidx * P + p;
          uint2 x = cb8[(int64_t)m * K + code_byte(c, u, s * P + p)];
          v[2 * p] = x.x;
          v[2 * p + 1] = x.y;
        }
      } else {  // DSUB == 2
        const uint32_t* cb4 = (const uint32_t*)cb_lds;
#pragma unroll
        for (int p = 0; p < 4; p++) {
          const int m = cidx * P + p;
          v[p] = cb4[(int64_t)m * K + code_byte(c, u, s * P + p)];
        }
      }
      return v;
    }
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
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KS; s++) acc = mfma16x16x32<DT>(fr[s], qf[j][s][h], acc);
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
        for (int h = 0; h < 2; h++) {
          f32x4 a4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int s = 0; s < KS; s++) a4 = mfma16x16x32<DT>(fr[u % 3][s], qf[j][s][h], a4);
          acc[u & 1][j][h] = a4;
        }
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
// host side
// ------------------------------------------------------------------------------
template <int DT>
static int build_lut(const void* Q, int64_t nq, const void* C, int64_t M, int64_t K, int64_t dsub, float* lut,
                     hipStream_t st) {
  const int64_t total = nq * M * K;
  if (total == 0) return TMS_OK;
  const int64_t grid = (total + 255) / 256;
  hipLaunchKernelGGL(pq_build_lut_kernel<DT>, dim3((unsigned)grid), dim3(256), 0, st, Q, C, lut, total, (int)M,
                     (int)K, (int)dsub);
  return check_launch("pq_build_lut_kernel");
}

static int fill_scores(float* out, int64_t n, float v, hipStream_t st);
// Batched queries over PQ codes (tms_stream.hip): the shared-tile kernel with the codebook
// gather as its tile source.
int run_pq_batched(const void* Q, int64_t nQ, int64_t nq, const void* codebook, int64_t M, int64_t K, int64_t dsub,
                   int dtype, const uint8_t* codes, int64_t B, int64_t nd, float* out, hipStream_t st);

template <int QG, int CW>
static int launch_lut_score(const LutArgs& a, hipStream_t st) {
  const int64_t waves = (a.B + a.docs_per_wave - 1) / a.docs_per_wave;
  const int64_t grid = (waves + kLutThreads / 64 - 1) / (kLutThreads / 64);
  hipLaunchKernelGGL((pq_lut_score_kernel<QG, CW>), dim3((unsigned)grid), dim3(kLutThreads), 0, st, a);
  return check_launch("pq_lut_score_kernel");
}
template <int QG>
static int launch_lut_cw(const LutArgs& a, const uint8_t* codes, hipStream_t st) {
  if (a.M == 16 && ((uintptr_t)codes & 15) == 0) return launch_lut_score<QG, 4>(a, st);
  if (a.M % 4 == 0 && ((uintptr_t)codes & 3) == 0) return launch_lut_score<QG, 1>(a, st);
  return launch_lut_score<QG, 0>(a, st);
}

constexpr int kPqUT = TMS_PQ_UT;

template <int DT, int DSUB, int KS, int NQB>
static int launch_mfma_one(const PqArgs& a, int64_t grid, size_t lds, hipStream_t st) {
  hipLaunchKernelGGL((pq_mfma_score_kernel<DT, DSUB, KS, NQB, kPqUT>), dim3((unsigned)grid), dim3(kPqThreads), lds, st,
                     a);
  return check_launch("pq_mfma_score_kernel");
}

template <int DT, int DSUB, int KS>
static int launch_mfma_nqb(const PqArgs& a, int64_t grid, size_t lds, hipStream_t st) {
  if (a.nblk == 2) return launch_mfma_one<DT, DSUB, KS, 2>(a, grid, lds, st);
  return launch_mfma_one<DT, DSUB, KS, 1>(a, grid, lds, st);
}

template <int DT, int DSUB>
static int launch_mfma_ks(const PqArgs& a, int ks, int64_t grid, size_t lds, hipStream_t st) {
  switch (ks) {
    case 1: return launch_mfma_nqb<DT, DSUB, 1>(a, grid, lds, st);
    case 2: return launch_mfma_nqb<DT, DSUB, 2>(a, grid, lds, st);
    case 3: return launch_mfma_nqb<DT, DSUB, 3>(a, grid, lds, st);
    default: return launch_mfma_nqb<DT, DSUB, 4>(a, grid, lds, st);
  }
}

template <int DT>
static int launch_mfma_dsub(const PqArgs& a, int dsub, int ks, int64_t grid, size_t lds, hipStream_t st) {
  switch (dsub) {
    case 2: return launch_mfma_ks<DT, 2>(a, ks, grid, lds, st);
    case 4: return launch_mfma_ks<DT, 4>(a, ks, grid, lds, st);
    case 8: return launch_mfma_ks<DT, 8>(a, ks, grid, lds, st);
    case 16: return launch_mfma_ks<DT, 16>(a, ks, grid, lds, st);
    default: return launch_mfma_ks<DT, 32>(a, ks, grid, lds, st);
  }
}

// The fast kernel needs: d = M*dsub in {32, 64, 96, 128}, dsub in {2, 4, 8, 16, 32}
// with M a multiple of 4, K <= 256, a codebook that fits 64 KiB of LDS, 16-byte
// aligned Q / codebook / code rows, and fewer than 2^31 code bytes per document.
static bool mfma_supported(const void* Q, const void* C, const uint8_t* codes, int64_t M, int64_t K, int64_t dsub,
                           int64_t nd) {
  const int64_t d = M * dsub;
  if (nd * M >= ((int64_t)1 << 31)) return false;  // a document's code bytes are addressed with 32-bit offsets
  if (!(dsub == 2 || dsub == 4 || dsub == 8 || dsub == 16 || dsub == 32)) return false;
  if (d % 32 != 0 || d > 128 || d == 0 || M % 4 != 0) return false;
  if (K > 256 || K < 1 || d * K * 2 > 64 * 1024) return false;
  if (((uintptr_t)Q & 15) || ((uintptr_t)C & 15) || ((uintptr_t)codes & 15)) return false;
  return true;
}

static int score_lut(const float* lut, int64_t nq, int64_t M, int64_t K, const uint8_t* codes, int64_t B, int64_t nd,
                     float* out, hipStream_t st) {
  LutArgs a;
  memset(&a, 0, sizeof(a));
  a.lut = lut;
  a.codes = codes;
  a.out = out;
  a.B = B;
  a.nd = nd;
  a.nq = (int32_t)nq;
  a.M = (int32_t)M;
  a.K = (int32_t)K;
  // at most 64 documents per wave (one lane each); fewer when B is small, so that the
  // grid still covers every CU
  const int64_t per_wave = (B + 256 * 16 - 1) / (256 * 16);
  a.docs_per_wave = (int32_t)(per_wave < 1 ? 1 : (per_wave > 64 ? 64 : per_wave));
  const int64_t mk = M * K;  // <= 16384, checked by the caller
  if (mk * 8 <= kLutSliceFloats) return launch_lut_cw<8>(a, codes, st);
  if (mk * 4 <= kLutSliceFloats) return launch_lut_cw<4>(a, codes, st);
  if (mk * 2 <= kLutSliceFloats) return launch_lut_cw<2>(a, codes, st);
  return launch_lut_cw<1>(a, codes, st);
}

}  // namespace tms

using namespace tms;

static int pq_common_checks(const char* fn, int64_t nq, int64_t M, int64_t K, int64_t dsub, int64_t B, int64_t nd) {
  if (nq < 0 || M < 0 || K < 0 || dsub < 0 || B < 0 || nd < 0)
    return fail(TMS_ERR_INVALID, "%s: negative size", fn);
  if (K > 256) return fail(TMS_ERR_UNSUPPORTED, "%s: K=%lld > 256 does not fit uint8 codes", fn, (long long)K);
  return TMS_OK;
}

extern "C" {

int tms_pq_build_lut(const void* Q, int64_t nq, const void* codebook, int64_t M, int64_t K, int64_t dsub, int dtype,
                     float* lut, void* stream) {
  const char* fn = "tms_pq_build_lut";
  if (dtype != TMS_DTYPE_F16 && dtype != TMS_DTYPE_BF16 && dtype != TMS_DTYPE_F32)
    return fail(TMS_ERR_UNSUPPORTED, "%s: unsupported dtype %d", fn, dtype);
  if (nq < 0 || M < 0 || K < 0 || dsub < 0) return fail(TMS_ERR_INVALID, "%s: negative size", fn);
  if (nq * M * K == 0) return TMS_OK;
  if (!Q || !codebook || !lut) return fail(TMS_ERR_INVALID, "%s: NULL pointer", fn);
  if (nq * M * K > ((int64_t)1 << 40)) return fail(TMS_ERR_UNSUPPORTED, "%s: table too large", fn);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == TMS_DTYPE_F16) return build_lut<TMS_DTYPE_F16>(Q, nq, codebook, M, K, dsub, lut, st);
  if (dtype == TMS_DTYPE_F32) return build_lut<TMS_DTYPE_F32>(Q, nq, codebook, M, K, dsub, lut, st);
  return build_lut<TMS_DTYPE_BF16>(Q, nq, codebook, M, K, dsub, lut, st);
}

int tms_pq_score_lut(const float* lut, int64_t nq, int64_t M, int64_t K, const uint8_t* codes, int64_t B, int64_t nd,
                     float* out, void* stream) {
  const char* fn = "tms_pq_score_lut";
  int rc = pq_common_checks(fn, nq, M, K, 1, B, nd);
  if (rc) return rc;
  if (B == 0) return TMS_OK;
  if (!out) return fail(TMS_ERR_INVALID, "%s: out is NULL", fn);
  if (nd > 0 && M > 0 && !codes) return fail(TMS_ERR_INVALID, "%s: codes is NULL", fn);
  if (nq > 0 && M > 0 && K > 0 && !lut) return fail(TMS_ERR_INVALID, "%s: lut is NULL", fn);
  if (M * K > 16384) return fail(TMS_ERR_UNSUPPORTED, "%s: M*K=%lld > 16384 does not fit LDS", fn, (long long)(M * K));
  if (M == 0 || K == 0) return fail(TMS_ERR_UNSUPPORTED, "%s: M and K must be positive", fn);
  hipStream_t st = (hipStream_t)stream;
  return score_lut(lut, nq, M, K, codes, B, nd, out, st);
}

int tms_pq_score(const void* Q, int64_t nq, const void* codebook, int64_t M, int64_t K, int64_t dsub, int dtype,
                 const uint8_t* codes, int64_t B, int64_t nd, float* out, void* stream) {
  const char* fn = "tms_pq_score";
  if (dtype != TMS_DTYPE_F16 && dtype != TMS_DTYPE_BF16) return fail(TMS_ERR_UNSUPPORTED, "%s: unsupported dtype %d", fn, dtype);
  int rc = pq_common_checks(fn, nq, M, K, dsub, B, nd);
  if (rc) return rc;
  if (B == 0) return TMS_OK;
  if (!out) return fail(TMS_ERR_INVALID, "%s: out is NULL", fn);
  if (nd > 0 && M > 0 && !codes) return fail(TMS_ERR_INVALID, "%s: codes is NULL", fn);
  if (nq > 0 && (!Q || !codebook)) return fail(TMS_ERR_INVALID, "%s: Q or codebook is NULL", fn);
  if (M == 0 || K == 0 || dsub == 0) return fail(TMS_ERR_UNSUPPORTED, "%s: M, K and dsub must be positive", fn);
  hipStream_t st = (hipStream_t)stream;
  // no query tokens: 0; no document tokens: -inf (the running max never moves)
  if (nq == 0 || nd == 0) return fill_scores(out, B, nq == 0 ? 0.f : -__builtin_inff(), st);
  if (mfma_supported(Q, codebook, codes, M, K, dsub, nd)) {
    PqArgs a;
    memset(&a, 0, sizeof(a));
    a.Q = (const uint8_t*)Q;
    a.codebook = (const uint8_t*)codebook;
    a.codes = codes;
    a.out = out;
    a.B = B;
    a.nd = nd;
    a.nq = (int32_t)nq;
    a.nbq = (int32_t)((nq + 31) / 32);
    a.K = (int32_t)K;
    const int64_t d = M * dsub;
    const int ks = (int)(d / 32);
    // Two 8-wave workgroups per CU fit next to a 64 KiB codebook; each wave gets a long
    // run of documents (about four rounds of the chip) so the per-workgroup codebook
    // load is amortised and the last round stays short.
    const int64_t waves_per_wg = kPqThreads / 64;
    const int64_t target_waves = (int64_t)256 * 2 * waves_per_wg * TMS_PQ_WAVE_ROUNDS;
    int64_t dpw = (B + target_waves - 1) / target_waves;
    if (dpw < 1) dpw = 1;
    a.docs_per_wave = (int32_t)dpw;
    const int64_t waves = (B + dpw - 1) / dpw;
    const int64_t grid = (waves + waves_per_wg - 1) / waves_per_wg;
    const size_t lds = (size_t)d * K * 2;
    for (int64_t blk0 = 0; blk0 < a.nbq; blk0 += 2) {
      a.blk0 = (int32_t)blk0;
      a.nblk = (int32_t)((a.nbq - blk0 < 2) ? a.nbq - blk0 : 2);
      if (dtype == TMS_DTYPE_F16) rc = launch_mfma_dsub<TMS_DTYPE_F16>(a, (int)dsub, ks, grid, lds, st);
      else rc = launch_mfma_dsub<TMS_DTYPE_BF16>(a, (int)dsub, ks, grid, lds, st);
      if (rc) return rc;
    }
    return TMS_OK;
  }
  // Other shapes go through tms_pq_build_lut + tms_pq_score_lut: the table needs
  // storage this allocation-free entry point cannot own, so the host wrapper
  // allocates it and picks that path.
  return fail(TMS_ERR_UNSUPPORTED,
              "%s: shape M=%lld K=%lld dsub=%lld (or alignment) not supported by the MFMA kernel; "
              "use tms_pq_build_lut + tms_pq_score_lut",
              fn, (long long)M, (long long)K, (long long)dsub);
}

int tms_pq_score_batched(const void* Qs, int64_t nQ, int64_t nq, const void* codebook, int64_t M, int64_t K,
                         int64_t dsub, int dtype, const uint8_t* codes, int64_t B, int64_t nd, float* out,
                         void* stream) {
  const char* fn = "tms_pq_score_batched";
  if (dtype != TMS_DTYPE_F16 && dtype != TMS_DTYPE_BF16) return fail(TMS_ERR_UNSUPPORTED, "%s: unsupported dtype %d", fn, dtype);
  if (nQ < 0) return fail(TMS_ERR_INVALID, "%s: negative size", fn);
  int rc = pq_common_checks(fn, nq, M, K, dsub, B, nd);
  if (rc) return rc;
  if (B == 0 || nQ == 0) return TMS_OK;
  if (!out) return fail(TMS_ERR_INVALID, "%s: out is NULL", fn);
  if (nd > 0 && M > 0 && !codes) return fail(TMS_ERR_INVALID, "%s: codes is NULL", fn);
  if (nq > 0 && (!Qs || !codebook)) return fail(TMS_ERR_INVALID, "%s: Q or codebook is NULL", fn);
  if (M == 0 || K == 0 || dsub == 0) return fail(TMS_ERR_UNSUPPORTED, "%s: M, K and dsub must be positive", fn);
  if (nq > ((int64_t)1 << 24) || nQ > ((int64_t)1 << 20)) return fail(TMS_ERR_UNSUPPORTED, "%s: too many queries", fn);
  hipStream_t st = (hipStream_t)stream;
  if (nq == 0 || nd == 0) return fill_scores(out, nQ * B, nq == 0 ? 0.f : -__builtin_inff(), st);
  if (!mfma_supported(Qs, codebook, codes, M, K, dsub, nd))
    return fail(TMS_ERR_UNSUPPORTED,
                "%s: shape M=%lld K=%lld dsub=%lld (or alignment) not supported by the MFMA kernels; score per "
                "query with tms_pq_build_lut + tms_pq_score_lut",
                fn, (long long)M, (long long)K, (long long)dsub);
  const int64_t nbq = (nq + 31) / 32;
  if (nbq > 4 || nQ * nbq < 2) {  // one query at a time
    const int64_t qbytes = nq * M * dsub * 2;
    for (int64_t q = 0; q < nQ; q++) {
      rc = tms_pq_score((const uint8_t*)Qs + q * qbytes, nq, codebook, M, K, dsub, dtype, codes, B, nd, out + q * B,
                        stream);
      if (rc) return rc;
    }
    return TMS_OK;
  }
  return run_pq_batched(Qs, nQ, nq, codebook, M, K, dsub, dtype, codes, B, nd, out, st);
}

}  // extern "C"

namespace tms {
__global__ void pq_fill_kernel(float* out, int64_t n, float v) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = v;
}
static int fill_scores(float* out, int64_t n, float v, hipStream_t st) {
  if (n <= 0) return TMS_OK;
  hipLaunchKernelGGL(pq_fill_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, out, n, v);
  return check_launch("pq_fill_kernel");
}
}  // namespace tms
