// Product-quantised (PQ / ADC) MaxSim on gfx950: the distance table, the table-gather
// kernels (the reference algorithm) and the host entry points of every PQ path.
//
// Reference: src/flash_pqsim_kernel.py. Documents are (B, nd, M) codes into a codebook
// (M, K, dsub); token t decodes to concat_m codebook[m, codes[t, m]].
//   score[b] = sum_q max_t sum_m lut[q, m, codes[b, t, m]],
//   lut[q, m, k] = sum_j Q[q, m*dsub + j] * codebook[m, k, j]          (:31-67, :127-173)
// which equals MaxSim of Q against the decoded vectors (:283-313).
//
// Kernels:
//  * pq_build_lut_kernel  -- the fp32 distance table (TileMaxSimPQ.build_distance_table),
//    from an fp16 / bf16 / fp32 query of its own type (never rounded to the codebook's).
//  * pq_lut_score_kernel  -- the reference algorithm: gathers from the fp32 table held
//    in LDS (a slice of QG query tokens x every subspace at a time), fp32 adds in
//    ascending m. Tables of M * K <= 16384 entries per query token; any code width.
//  * pq_lut_mtile_kernel  -- the same for larger tables: the slice is also tiled over m,
//    with per-token partial sums in VGPRs across the slices.
//  * pq_lut_score_kernel<GLB> -- gathers straight from the table in memory (K > 16384, or
//    documents too long for the m-tiled kernel's token run).
//  * pq_mfma_score_kernel (tms_pq_kernel.h) -- the fast path: codebook gathers into MFMA
//    fragments.
#include <string.h>

#include "tms_pq_kernel.h"

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
// src/flash_pqsim_kernel.py:31-67, loads both operands .to(tl.float32), rounds each
// product and sums them with tl.sum: within dsub * 2^-24 relative of each other). QDT is
// the query's type, CDT the codebook's: an fp32 query against a 16-bit codebook is used
// unrounded, as the reference uses it.
template <int QDT, int CDT>
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
  for (int j = 0; j < dsub; j++) s = __builtin_fmaf(load_elem<QDT>(Q, qb + j), load_elem<CDT>(C, cb + j), s);
  lut[i] = s;
}

// ------------------------------------------------------------------------------
// table-gather scoring (reference algorithm)
// ------------------------------------------------------------------------------
struct LutArgs {
  const float* lut;      // (nq, M, K)
  const uint8_t* codes;  // (B, nd, M) codes of CWB bytes
  float* out;            // (B)
  int64_t B, nd;
  int32_t nq, M, K;
  int32_t docs_per_wave;  // q-sliced kernel: documents per wave (<= 64); m-tiled: per workgroup
  int32_t ms;             // m-tiled kernel: subspaces per slice
};

#ifndef TMS_LUT_SLICE_FLOATS
#define TMS_LUT_SLICE_FLOATS 16384  // table slice in LDS: 64 KiB, two workgroups per CU
#endif
constexpr int kLutThreads = 1024;
constexpr int kLutSliceFloats = TMS_LUT_SLICE_FLOATS;
constexpr int kMtileTPL = 4;  // tokens per thread of the m-tiled kernel: runs of up to 4096 tokens

__device__ __forceinline__ float row_max16(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_f32<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_f32<0x141>(v));  // row_half_mirror
  v = fmaxf(v, dpp_f32<0x140>(v));  // row_mirror
  return v;
}

// Code (m) of the code row at p (CWB bytes per code), clamped into [0, K).
template <int CWB>
__device__ __forceinline__ uint32_t load_code(const uint8_t* p, int m, int K) {
  uint32_t c;
  if constexpr (CWB == 1) c = p[m];
  else if constexpr (CWB == 2) c = ((const uint16_t*)p)[m];
  else c = ((const uint32_t*)p)[m];
  return min(c, (uint32_t)(K - 1));
}

// One lane per document token; a workgroup of 16 waves shares one slice of the table in
// LDS: QG query tokens, [m][k][QG] fp32 (zero past nq), at most 64 KiB, so two
// workgroups (32 waves) share a CU and hide each other's gather latency. Each lane loads
// its token's M codes with one or a few wide loads, gathers its M rows of QG values
// and adds them in ascending m, as the reference sums them (:154-167), then keeps a
// running max per query token. A document's maxima are taken across the wave with DPP and
// row swaps, and its partial score (the slice's query tokens) accumulates in lane
// b - b_begin. Slices loop inside the kernel, so the codes are read once per slice.
// CW: 4 = each token's code row is one 16-byte load (M * CWB == 16); 1 = 4-byte loads
// ((M * CWB) % 4 == 0); 0 = one load per code. CWB: bytes per code (1, 2, 4).
// GLB: no slice; QG == 1 and every row is read from the table in memory (tables with
// K > 16384, or with documents too long for the m-tiled kernel).
template <int QG, int CW, int CWB, bool GLB>
__global__ void __launch_bounds__(kLutThreads) pq_lut_score_kernel(LutArgs a) {
  static_assert(!GLB || QG == 1, "the in-memory table is gathered one query token at a time");
  __shared__ float lds[GLB ? 1 : kLutSliceFloats];
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * (kLutThreads / 64) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t b_begin = wave_uniform(wave * a.docs_per_wave);
  const int64_t b_end = (b_begin + a.docs_per_wave < a.B) ? b_begin + a.docs_per_wave : a.B;
  const int M = a.M, K = a.K, MK = a.M * a.K;
  const int64_t nd = a.nd;
  const float NEG_INF = -__builtin_inff();
  constexpr int CPW = 4 / CWB;  // codes per 32-bit word

  int q0 = 0;
  auto add_code = [&](float (&s)[QG], uint32_t code, int m) {
    code = min(code, (uint32_t)(K - 1));  // codes >= K (invalid input) stay inside the table
    if constexpr (GLB) {
      s[0] += a.lut[((int64_t)q0 * M + m) * K + code];
    } else {
      const float* row = lds + ((uint32_t)m * (uint32_t)K + code) * QG;
#pragma unroll
      for (int j = 0; j < QG; j++) s[j] += row[j];
    }
  };
  // Accumulate the rows of the codes in `word` (subspaces m0 .. m0+n-1) into s.
  auto gather_word = [&](float (&s)[QG], uint32_t word, int m0, int n) {
#pragma unroll
    for (int i = 0; i < CPW; i++)
      if (i < n) add_code(s, code_at<CWB>(&word, i), m0 + i);
  };

  float partial = 0.f;  // lane j: running score of document b_begin + j
  for (; q0 < a.nq; q0 += QG) {
    if constexpr (!GLB) {
      __syncthreads();
      for (int i = threadIdx.x; i < MK * QG; i += kLutThreads) {  // reads run along mk
        const int qq = i / MK, mk = i - qq * MK;
        const int q = q0 + qq;
        lds[mk * QG + qq] = (q < a.nq) ? a.lut[(int64_t)q * MK + mk] : 0.f;
      }
      __syncthreads();
    }
    for (int64_t b = b_begin; b < b_end; b++) {
      float mx[QG];
#pragma unroll
      for (int j = 0; j < QG; j++) mx[j] = NEG_INF;
      for (int64_t t0 = 0; t0 < nd; t0 += 64) {
        const int64_t t = (t0 + lane < nd) ? t0 + lane : nd - 1;  // duplicate of the last token: max unchanged
        const uint8_t* cp = a.codes + (b * nd + t) * M * CWB;
        float s[QG];
#pragma unroll
        for (int j = 0; j < QG; j++) s[j] = 0.f;
        if constexpr (CW == 4) {
          const uint4 v = *(const uint4*)cp;
          gather_word(s, v.x, 0, CPW);
          gather_word(s, v.y, CPW, CPW);
          gather_word(s, v.z, 2 * CPW, CPW);
          gather_word(s, v.w, 3 * CPW, CPW);
        } else if constexpr (CW == 1) {
          for (int m0 = 0; m0 < M; m0 += CPW) gather_word(s, *(const uint32_t*)(cp + m0 * CWB), m0, CPW);
        } else {
          for (int m = 0; m < M; m++) add_code(s, load_code<CWB>(cp, m, K), m);
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

// Tables whose subspaces do not all fit one slice (M * K > 16384 entries per query
// token): the slice is tiled over m as well. A workgroup takes a run of whole documents,
// at most kLutThreads * TPL tokens (thread t holds tokens t, t + 1024, ... of the run).
// For each group of QG query tokens it streams the table through LDS in slices of a.ms
// subspaces x K x QG and adds each slice's rows to per-token partial sums held in VGPRs,
// in ascending m as the reference sums them (:154-167). After the last slice the token
// sums go to LDS, and wave w takes the max over the tokens of documents w, w + 16, ...
// of the run and adds it to their scores. Codes are clamped into [0, K).
template <int QG, int TPL, int CWB>
__global__ void __launch_bounds__(kLutThreads) pq_lut_mtile_kernel(LutArgs a) {
  static_assert(QG * TPL * kLutThreads <= kLutSliceFloats, "the token sums fit the slice buffer");
  constexpr int kWaves = kLutThreads / 64;
  constexpr int kDocsPerWave = 4;  // a run holds at most kWaves * 4 = 64 documents
  __shared__ float lds[kLutSliceFloats];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int M = a.M, K = a.K;
  const int64_t nd = a.nd;
  const int64_t b0 = (int64_t)blockIdx.x * a.docs_per_wave;
  const int64_t b1 = (b0 + a.docs_per_wave < a.B) ? b0 + a.docs_per_wave : a.B;
  const int ndocs = (int)(b1 - b0);
  const int ntok = ndocs * (int)nd;  // <= kLutThreads * TPL (host)
  const uint8_t* cbase = a.codes + b0 * nd * M * CWB;
  const float NEG_INF = -__builtin_inff();

  float part[kDocsPerWave];  // wave w: scores of documents w + 16 i of the run
#pragma unroll
  for (int i = 0; i < kDocsPerWave; i++) part[i] = 0.f;
  for (int q0 = 0; q0 < a.nq; q0 += QG) {
    float acc[TPL][QG];
#pragma unroll
    for (int tp = 0; tp < TPL; tp++)
#pragma unroll
      for (int j = 0; j < QG; j++) acc[tp][j] = 0.f;
    for (int m0 = 0; m0 < M; m0 += a.ms) {
      const int ms = (a.ms < M - m0) ? a.ms : M - m0;
      const int n = ms * K;  // slice rows: [mm][k], mm < ms
      __syncthreads();
      for (int i = tid; i < n * QG; i += kLutThreads) {  // reads run along (mm, k)
        const int qq = i / n, mk = i - qq * n;
        lds[mk * QG + qq] = (q0 + qq < a.nq) ? a.lut[((int64_t)(q0 + qq) * M + m0) * K + mk] : 0.f;
      }
      __syncthreads();
#pragma unroll
      for (int tp = 0; tp < TPL; tp++) {
        const int t = tid + tp * kLutThreads;
        if (t < ntok) {
          const uint8_t* cp = cbase + (int64_t)t * M * CWB;
          for (int mm = 0; mm < ms; mm++) {
            const uint32_t c = load_code<CWB>(cp, m0 + mm, K);
            const float* row = lds + ((uint32_t)mm * (uint32_t)K + c) * QG;
#pragma unroll
            for (int j = 0; j < QG; j++) acc[tp][j] += row[j];
          }
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int tp = 0; tp < TPL; tp++) {
      const int t = tid + tp * kLutThreads;
      if (t < ntok)
#pragma unroll
        for (int j = 0; j < QG; j++) lds[t * QG + j] = acc[tp][j];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kDocsPerWave; i++) {
      const int doc = wid + kWaves * i;
      if (doc < ndocs) {
        float tot = 0.f;
#pragma unroll
        for (int j = 0; j < QG; j++) {
          float m = NEG_INF;
          for (int t = lane; t < (int)nd; t += 64) m = fmaxf(m, lds[(doc * (int)nd + t) * QG + j]);
          m = cross_row_max(row_max16(m));
          tot += (q0 + j < a.nq) ? m : 0.f;
        }
        part[i] += tot;
      }
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < kDocsPerWave; i++) {
      const int doc = wid + kWaves * i;
      if (doc < ndocs) a.out[b0 + doc] = part[i];
    }
  }
}

// ------------------------------------------------------------------------------
// host side
// ------------------------------------------------------------------------------
template <int QDT, int CDT>
static int build_lut(const void* Q, int64_t nq, const void* C, int64_t M, int64_t K, int64_t dsub, float* lut,
                     hipStream_t st) {
  const int64_t total = nq * M * K;
  if (total == 0) return TMS_OK;
  const int64_t grid = (total + 255) / 256;
  hipLaunchKernelGGL((pq_build_lut_kernel<QDT, CDT>), dim3((unsigned)grid), dim3(256), 0, st, Q, C, lut, total,
                     (int)M, (int)K, (int)dsub);
  return check_launch("pq_build_lut_kernel");
}

static int fill_scores(float* out, int64_t n, float v, hipStream_t st);
// Batched queries over PQ codes (tms_stream.hip): the shared-tile kernel with the codebook
// gather as its tile source.
int run_pq_batched(const void* Q, int64_t nQ, int64_t nq, const void* codebook, int64_t M, int64_t K, int64_t dsub,
                   int dtype, const uint8_t* codes, int64_t B, int64_t nd, float* out, hipStream_t st);

template <int QG, int CW, int CWB, bool GLB>
static int launch_lut_score(const LutArgs& a, hipStream_t st) {
  const int64_t waves = (a.B + a.docs_per_wave - 1) / a.docs_per_wave;
  const int64_t grid = (waves + kLutThreads / 64 - 1) / (kLutThreads / 64);
  hipLaunchKernelGGL((pq_lut_score_kernel<QG, CW, CWB, GLB>), dim3((unsigned)grid), dim3(kLutThreads), 0, st, a);
  return check_launch("pq_lut_score_kernel");
}
template <int QG, int CWB>
static int launch_lut_cw(const LutArgs& a, const uint8_t* codes, hipStream_t st) {
  if (a.M * CWB == 16 && ((uintptr_t)codes & 15) == 0) return launch_lut_score<QG, 4, CWB, false>(a, st);
  if ((a.M * CWB) % 4 == 0 && ((uintptr_t)codes & 3) == 0) return launch_lut_score<QG, 1, CWB, false>(a, st);
  return launch_lut_score<QG, 0, CWB, false>(a, st);
}
template <int CWB>
static int launch_lut_qg(const LutArgs& a, const uint8_t* codes, hipStream_t st) {
  const int64_t mk = (int64_t)a.M * a.K;  // <= kLutSliceFloats
  if (mk * 8 <= kLutSliceFloats) return launch_lut_cw<8, CWB>(a, codes, st);
  if (mk * 4 <= kLutSliceFloats) return launch_lut_cw<4, CWB>(a, codes, st);
  if (mk * 2 <= kLutSliceFloats) return launch_lut_cw<2, CWB>(a, codes, st);
  return launch_lut_cw<1, CWB>(a, codes, st);
}
template <int QG, int CWB>
static int launch_mtile(const LutArgs& a, hipStream_t st) {
  const int64_t grid = (a.B + a.docs_per_wave - 1) / a.docs_per_wave;
  hipLaunchKernelGGL((pq_lut_mtile_kernel<QG, kMtileTPL, CWB>), dim3((unsigned)grid), dim3(kLutThreads), 0, st, a);
  return check_launch("pq_lut_mtile_kernel");
}
template <int CWB>
static int launch_mtile_qg(const LutArgs& a, hipStream_t st) {
  if ((int64_t)a.K * 4 * a.ms <= kLutSliceFloats) return launch_mtile<4, CWB>(a, st);
  if ((int64_t)a.K * 2 * a.ms <= kLutSliceFloats) return launch_mtile<2, CWB>(a, st);
  return launch_mtile<1, CWB>(a, st);
}

template <int CWB>
static int score_lut_cwb(LutArgs a, hipStream_t st) {
  const int64_t mk = (int64_t)a.M * a.K;
  if (mk <= kLutSliceFloats) {
    // at most 64 documents per wave (one lane each); fewer when B is small, so that the
    // grid still covers every CU
    const int64_t per_wave = (a.B + 256 * 16 - 1) / (256 * 16);
    a.docs_per_wave = (int32_t)(per_wave < 1 ? 1 : (per_wave > 64 ? 64 : per_wave));
    return launch_lut_qg<CWB>(a, a.codes, st);
  }
  if (a.K <= kLutSliceFloats && a.nd <= (int64_t)kLutThreads * kMtileTPL) {
    // m-tiled: QG query tokens (4 when a 4-query slice holds a whole subspace) x ms
    // subspaces per slice, runs of whole documents up to kLutThreads * TPL tokens
    const int qg = (int64_t)a.K * 4 <= kLutSliceFloats ? 4 : ((int64_t)a.K * 2 <= kLutSliceFloats ? 2 : 1);
    a.ms = (int32_t)(kLutSliceFloats / ((int64_t)a.K * qg));
    int64_t dpw = ((int64_t)kLutThreads * kMtileTPL) / (a.nd > 0 ? a.nd : 1);
    if (dpw > 64) dpw = 64;
    a.docs_per_wave = (int32_t)dpw;
    return launch_mtile_qg<CWB>(a, st);
  }
  const int64_t per_wave = (a.B + 256 * 16 - 1) / (256 * 16);
  a.docs_per_wave = (int32_t)(per_wave < 1 ? 1 : (per_wave > 64 ? 64 : per_wave));
  return launch_lut_score<1, 0, CWB, true>(a, st);
}

static int score_lut(const float* lut, int64_t nq, int64_t M, int64_t K, const uint8_t* codes, int code_bytes,
                     int64_t B, int64_t nd, float* out, hipStream_t st) {
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
  if (code_bytes == 1) return score_lut_cwb<1>(a, st);
  if (code_bytes == 2) return score_lut_cwb<2>(a, st);
  return score_lut_cwb<4>(a, st);
}

// Bytes per code from the TMS_CODES_* flags of a PQ dtype argument (1 without them).
static int code_bytes_of(int flags) {
  if (flags & TMS_CODES_I32) return 4;
  if (flags & TMS_CODES_I16) return 2;
  return 1;
}

// The MFMA kernels need: d = M*dsub in {32, 64, 96, 128}, dsub in {2, 4, 8, 16, 32}
// with M a multiple of 4, a codebook of d * K 16-bit elements that fits the device's
// LDS, 16-byte aligned Q / codebook / code rows, fewer than 2^31 code bytes per
// document, and (for fp32 queries) uint8 codes.
static int mfma_shape(const char* fn, const void* Q, const void* C, const void* codes, int64_t M, int64_t K,
                      int64_t dsub, int64_t nd, int code_bytes, bool q32) {
  const int64_t d = M * dsub;
  if (nd * M * code_bytes >= ((int64_t)1 << 31))
    return fail(TMS_ERR_UNSUPPORTED, "%s: documents of 2^31 code bytes or more", fn);
  if (!(dsub == 2 || dsub == 4 || dsub == 8 || dsub == 16 || dsub == 32) || d % 32 != 0 || d > 128 || d == 0 ||
      M % 4 != 0)
    return fail(TMS_ERR_UNSUPPORTED,
                "%s: shape M=%lld dsub=%lld not supported by the MFMA kernel; use tms_pq_build_lut + "
                "tms_pq_score_lut_ex",
                fn, (long long)M, (long long)dsub);
  if (((uintptr_t)Q & 15) || ((uintptr_t)C & 15) || ((uintptr_t)codes & 15))
    return fail(TMS_ERR_UNSUPPORTED, "%s: the MFMA kernel needs 16-byte aligned Q, codebook and codes", fn);
  if (q32 && code_bytes != 1)
    return fail(TMS_ERR_UNSUPPORTED, "%s: fp32 queries on the MFMA kernel take uint8 codes", fn);
  const int64_t lds = d * K * 2;
  if (lds > 64 * 1024) {
    int dev = 0, cap = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cap, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
      return fail(TMS_ERR_HIP, "%s: cannot query the LDS limit", fn);
    if (lds > cap)
      return fail(TMS_ERR_UNSUPPORTED, "%s: a codebook of %lld bytes does not fit the %d bytes of LDS", fn,
                  (long long)lds, cap);
  }
  return TMS_OK;
}

}  // namespace tms

using namespace tms;

static int pq_common_checks(const char* fn, int64_t nq, int64_t M, int64_t K, int64_t dsub, int64_t B, int64_t nd) {
  if (nq < 0 || M < 0 || K < 0 || dsub < 0 || B < 0 || nd < 0)
    return fail(TMS_ERR_INVALID, "%s: negative size", fn);
  if (M * K >= ((int64_t)1 << 31) || nq >= ((int64_t)1 << 31))
    return fail(TMS_ERR_UNSUPPORTED, "%s: M*K=%lld or nq=%lld beyond 2^31", fn, (long long)(M * K), (long long)nq);
  return TMS_OK;
}

extern "C" {

int tms_pq_build_lut(const void* Q, int64_t nq, const void* codebook, int64_t M, int64_t K, int64_t dsub, int dtype,
                     float* lut, void* stream) {
  const char* fn = "tms_pq_build_lut";
  const bool q32 = (dtype & TMS_QUERY_F32) != 0;
  dtype &= ~TMS_QUERY_F32;
  if (dtype != TMS_DTYPE_F16 && dtype != TMS_DTYPE_BF16 && dtype != TMS_DTYPE_F32)
    return fail(TMS_ERR_UNSUPPORTED, "%s: unsupported dtype %d", fn, dtype);
  if (nq < 0 || M < 0 || K < 0 || dsub < 0) return fail(TMS_ERR_INVALID, "%s: negative size", fn);
  if (nq * M * K == 0) return TMS_OK;
  if (!Q || !codebook || !lut) return fail(TMS_ERR_INVALID, "%s: NULL pointer", fn);
  if (nq * M * K > ((int64_t)1 << 40) || M * K >= ((int64_t)1 << 31))
    return fail(TMS_ERR_UNSUPPORTED, "%s: table too large", fn);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == TMS_DTYPE_F32) return build_lut<TMS_DTYPE_F32, TMS_DTYPE_F32>(Q, nq, codebook, M, K, dsub, lut, st);
  if (dtype == TMS_DTYPE_F16) {
    if (q32) return build_lut<TMS_DTYPE_F32, TMS_DTYPE_F16>(Q, nq, codebook, M, K, dsub, lut, st);
    return build_lut<TMS_DTYPE_F16, TMS_DTYPE_F16>(Q, nq, codebook, M, K, dsub, lut, st);
  }
  if (q32) return build_lut<TMS_DTYPE_F32, TMS_DTYPE_BF16>(Q, nq, codebook, M, K, dsub, lut, st);
  return build_lut<TMS_DTYPE_BF16, TMS_DTYPE_BF16>(Q, nq, codebook, M, K, dsub, lut, st);
}

int tms_pq_score_lut_ex(const float* lut, int64_t nq, int64_t M, int64_t K, const void* codes, int code_bytes,
                        int64_t B, int64_t nd, float* out, void* stream) {
  const char* fn = "tms_pq_score_lut_ex";
  int rc = pq_common_checks(fn, nq, M, K, 1, B, nd);
  if (rc) return rc;
  if (code_bytes != 1 && code_bytes != 2 && code_bytes != 4)
    return fail(TMS_ERR_INVALID, "%s: code_bytes must be 1, 2 or 4, got %d", fn, code_bytes);
  if (B == 0) return TMS_OK;
  if (!out) return fail(TMS_ERR_INVALID, "%s: out is NULL", fn);
  if (nd > 0 && M > 0 && !codes) return fail(TMS_ERR_INVALID, "%s: codes is NULL", fn);
  if (nq > 0 && M > 0 && K > 0 && !lut) return fail(TMS_ERR_INVALID, "%s: lut is NULL", fn);
  if (M == 0 || K == 0) return fail(TMS_ERR_UNSUPPORTED, "%s: M and K must be positive", fn);
  hipStream_t st = (hipStream_t)stream;
  // no query tokens: 0; no document tokens: -inf (the running max never moves)
  if (nq == 0 || nd == 0) return fill_scores(out, B, nq == 0 ? 0.f : -__builtin_inff(), st);
  return score_lut(lut, nq, M, K, (const uint8_t*)codes, code_bytes, B, nd, out, st);
}

int tms_pq_score_lut(const float* lut, int64_t nq, int64_t M, int64_t K, const uint8_t* codes, int64_t B, int64_t nd,
                     float* out, void* stream) {
  return tms_pq_score_lut_ex(lut, nq, M, K, codes, 1, B, nd, out, stream);
}

int tms_pq_score(const void* Q, int64_t nq, const void* codebook, int64_t M, int64_t K, int64_t dsub, int dtype,
                 const uint8_t* codes, int64_t B, int64_t nd, float* out, void* stream) {
  const char* fn = "tms_pq_score";
  const int flags = dtype & (TMS_QUERY_F32 | TMS_CODES_I16 | TMS_CODES_I32);
  dtype &= ~(TMS_QUERY_F32 | TMS_CODES_I16 | TMS_CODES_I32);
  const bool q32 = (flags & TMS_QUERY_F32) != 0;
  const int cwb = code_bytes_of(flags);
  if (dtype != TMS_DTYPE_F16 && dtype != TMS_DTYPE_BF16)
    return fail(TMS_ERR_UNSUPPORTED, "%s: unsupported dtype %d (fp32 codebooks take the table path)", fn, dtype);
  int rc = pq_common_checks(fn, nq, M, K, dsub, B, nd);
  if (rc) return rc;
  if (B == 0) return TMS_OK;
  if (!out) return fail(TMS_ERR_INVALID, "%s: out is NULL", fn);
  if (nd > 0 && M > 0 && !codes) return fail(TMS_ERR_INVALID, "%s: codes is NULL", fn);
  if (nq > 0 && (!Q || !codebook)) return fail(TMS_ERR_INVALID, "%s: Q or codebook is NULL", fn);
  if (M == 0 || K == 0 || dsub == 0) return fail(TMS_ERR_UNSUPPORTED, "%s: M, K and dsub must be positive", fn);
  // Other shapes go through tms_pq_build_lut + tms_pq_score_lut_ex: the table needs
  // storage this allocation-free entry point cannot own, so the host wrapper allocates it
  // and picks that path.
  rc = mfma_shape(fn, Q, codebook, codes, M, K, dsub, nd, cwb, q32);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  // no query tokens: 0; no document tokens: -inf (the running max never moves)
  if (nq == 0 || nd == 0) return fill_scores(out, B, nq == 0 ? 0.f : -__builtin_inff(), st);
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
  if (q32) return run_pq_mfma_q32(a, dtype, M, dsub, st);
  if (cwb != 1) return run_pq_mfma_wide(a, dtype, cwb, M, dsub, st);
  if (dtype == TMS_DTYPE_F16) return run_pq_mfma<TMS_DTYPE_F16, TMS_DTYPE_F16, 1>(a, M, dsub, st);
  return run_pq_mfma<TMS_DTYPE_BF16, TMS_DTYPE_BF16, 1>(a, M, dsub, st);
}

int tms_pq_score_batched(const void* Qs, int64_t nQ, int64_t nq, const void* codebook, int64_t M, int64_t K,
                         int64_t dsub, int dtype, const uint8_t* codes, int64_t B, int64_t nd, float* out,
                         void* stream) {
  const char* fn = "tms_pq_score_batched";
  const int flags = dtype & (TMS_QUERY_F32 | TMS_CODES_I16 | TMS_CODES_I32);
  const int base = dtype & ~(TMS_QUERY_F32 | TMS_CODES_I16 | TMS_CODES_I32);
  if (base != TMS_DTYPE_F16 && base != TMS_DTYPE_BF16)
    return fail(TMS_ERR_UNSUPPORTED, "%s: unsupported dtype %d", fn, base);
  if (nQ < 0) return fail(TMS_ERR_INVALID, "%s: negative size", fn);
  int rc = pq_common_checks(fn, nq, M, K, dsub, B, nd);
  if (rc) return rc;
  if (B == 0 || nQ == 0) return TMS_OK;
  if (!out) return fail(TMS_ERR_INVALID, "%s: out is NULL", fn);
  if (nd > 0 && M > 0 && !codes) return fail(TMS_ERR_INVALID, "%s: codes is NULL", fn);
  if (nq > 0 && (!Qs || !codebook)) return fail(TMS_ERR_INVALID, "%s: Q or codebook is NULL", fn);
  if (M == 0 || K == 0 || dsub == 0) return fail(TMS_ERR_UNSUPPORTED, "%s: M, K and dsub must be positive", fn);
  if (nq > ((int64_t)1 << 24) || nQ > ((int64_t)1 << 20)) return fail(TMS_ERR_UNSUPPORTED, "%s: too many queries", fn);
  rc = mfma_shape(fn, Qs, codebook, codes, M, K, dsub, nd, code_bytes_of(flags), (flags & TMS_QUERY_F32) != 0);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  if (nq == 0 || nd == 0) return fill_scores(out, nQ * B, nq == 0 ? 0.f : -__builtin_inff(), st);
  const int64_t nbq = (nq + 31) / 32;
  // The shared-tile kernel takes uint8 codes, a query of the codebook's type and a
  // codebook of at most 64 KiB beside its tile ring; other inputs, and queries of more
  // than 4 blocks, are scored one query at a time.
  const bool shared = flags == 0 && M * dsub * K * 2 <= 64 * 1024 && nbq <= 4 && nQ * nbq >= 2;
  if (!shared) {
    const int64_t qbytes = nq * M * dsub * ((flags & TMS_QUERY_F32) ? 4 : 2);
    for (int64_t q = 0; q < nQ; q++) {
      rc = tms_pq_score((const uint8_t*)Qs + q * qbytes, nq, codebook, M, K, dsub, dtype, codes, B, nd, out + q * B,
                        stream);
      if (rc) return rc;
    }
    return TMS_OK;
  }
  return run_pq_batched(Qs, nQ, nq, codebook, M, K, dsub, base, codes, B, nd, out, st);
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
