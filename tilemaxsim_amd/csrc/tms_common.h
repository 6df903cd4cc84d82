// Shared device/host helpers for the tilemaxsim HIP kernels (gfx950 / CDNA4).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tilemaxsim.h"

namespace tms {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

#ifndef TMS_STREAM_NT
#define TMS_STREAM_NT 1
#endif
// A load of streamed document data (tokens, codes: read once per pass). WHOLE: the
// wave's load covers whole 128-byte lines, and is then non-temporal, so the caches treat
// the lines as a stream. A read-only pass over 46 GB measured 6.74-7.08 TB/s with such
// loads against 6.01-6.34 TB/s with plain ones (the cache-coherence bits sc0 / sc1 change
// neither); non-temporal loads that cover half of each line (the other half read by a
// later load) measured 5.53 TB/s, so those stay plain.
template <class T, bool WHOLE>
__device__ __forceinline__ T ld_stream(const void* p) {
#if TMS_STREAM_NT
  if constexpr (WHOLE) return __builtin_nontemporal_load((const T*)p);
#endif
  return *(const T*)p;
}

// Whole-line tile loads. A 16-row tile of 256- (or 128-) byte rows is read as loads of
// eight rows x one 128-byte line: lane 16 g + 8 s + t reads row t (first load) or 8 + t
// (second load), bytes 64 s + 16 g of the line. The line's two MFMA A-operand fragments
// (lane 16 g + r: row r, 16-byte chunk 4 k + g of the line, k = 0, 1) follow with one
// rotate by eight lanes within each row: rows 0-7 of chunk g sit in place in the first
// load, rows 8-15 eight lanes down in the second, and chunk 4 + g the other way round.
// Each word is one DPP move (row_ror:8) whose bank mask writes only the lanes that take
// the rotated value (lanes 8-15 of a row for k0, 0-7 for k1); the others keep the
// unrotated word. The move runs with the whole wave active (no select that could become
// a branch, under which the rotate would read inactive lanes).
__device__ __forceinline__ void line_frags(const u32x4& first8, const u32x4& last8, u32x4& k0, u32x4& k1) {
#pragma unroll
  for (int i = 0; i < 4; i++) {
    k0[i] = (uint32_t)__builtin_amdgcn_update_dpp((int)first8[i], (int)last8[i], 0x128, 0xf, 0xc, false);
    k1[i] = (uint32_t)__builtin_amdgcn_update_dpp((int)last8[i], (int)first8[i], 0x128, 0xf, 0x3, false);
  }
}

// Eight consecutive elements of an embedding row as loaded from memory: 16 bytes for
// fp16 / bf16, 32 bytes for fp32.
template <int DT>
struct Raw8 {
  using T = u32x4;
};
template <>
struct Raw8<TMS_DTYPE_F32> {
  using T = u32x8;
};

// fp32 -> two bf16 terms: hi = bf16(x), lo = bf16(x - hi), both rounded to nearest even.
// x - hi is exact in fp32, so |x - hi - lo| <= 2^-16 |x|; a product x*y is then
// hi_x*hi_y + hi_x*lo_y + lo_x*hi_y up to about 3 * 2^-16 |x*y| (the lo*lo term and the
// two roundings). Returns eight bf16 values packed like an MFMA operand fragment.
__device__ __forceinline__ void split_bf16(u32x8 x, u32x4& hi, u32x4& lo) {
#pragma unroll
  for (int i = 0; i < 4; i++) {
    // elements copied out first: __builtin_bit_cast of a vector-element expression
    // reads element 0 with this compiler
    const uint32_t x0 = x[2 * i], x1 = x[2 * i + 1];
    const f32x2 v = {__builtin_bit_cast(float, x0), __builtin_bit_cast(float, x1)};
    const bf16x2 h = __builtin_convertvector(v, bf16x2);
    const uint32_t hb = __builtin_bit_cast(uint32_t, h);
    const f32x2 hv = {__builtin_bit_cast(float, hb << 16), __builtin_bit_cast(float, hb & 0xffff0000u)};
    const bf16x2 l = __builtin_convertvector(v - hv, bf16x2);
    hi[i] = hb;
    lo[i] = __builtin_bit_cast(uint32_t, l);
  }
}

// fp32 query elements -> two fp16 terms of x * scale: hi = fp16(xs), lo = fp16(xs - hi),
// both rounded to nearest even (xs - hi is exact in fp32). `scale` is the token's power
// of two from pow2_scale, which puts its largest |x| in [2^14, 2^15): hi never overflows,
// and |xs - hi - lo| <= 2^-22 |xs| + 2^-25 (the last term is fp16's subnormal spacing,
// 2^-39 of the token's largest element). Scaling by a power of two is exact, and a
// positive per-token factor commutes with the max over document tokens, so the running
// max is taken on scaled dot products and multiplied by 1 / scale before the sum.
__device__ __forceinline__ void split_f16(u32x8 x, float scale, u32x4& hi, u32x4& lo) {
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t x0 = x[2 * i], x1 = x[2 * i + 1];
    const float a = __builtin_bit_cast(float, x0) * scale, b = __builtin_bit_cast(float, x1) * scale;
    const _Float16 ha = (_Float16)a, hb = (_Float16)b;
    const _Float16 la = (_Float16)(a - (float)ha), lb = (_Float16)(b - (float)hb);
    hi[i] = (uint32_t)__builtin_bit_cast(uint16_t, ha) | ((uint32_t)__builtin_bit_cast(uint16_t, hb) << 16);
    lo[i] = (uint32_t)__builtin_bit_cast(uint16_t, la) | ((uint32_t)__builtin_bit_cast(uint16_t, lb) << 16);
  }
}

// The power of two 2^s that maps amax = f * 2^e (f in [0.5, 1)) into [2^14, 2^15):
// s = 15 - e, clamped to [-126, 126] so that 2^s and 2^-s (returned in inv) are normal.
__device__ __forceinline__ float pow2_scale(float amax, float& inv) {
  const int be = (int)((__builtin_bit_cast(uint32_t, amax) >> 23) & 0xffu);  // 0 for 0 and subnormals
  int s = 15 - (be - 126);
  s = s < -126 ? -126 : (s > 126 ? 126 : s);
  inv = __builtin_bit_cast(float, (uint32_t)(127 - s) << 23);
  return __builtin_bit_cast(float, (uint32_t)(127 + s) << 23);
}

// Largest |x| over eight fp32 elements.
__device__ __forceinline__ float absmax8(u32x8 x) {
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const uint32_t xi = x[i];
    m = fmaxf(m, __builtin_bit_cast(float, xi & 0x7fffffffu));
  }
  return m;
}

// One v_mfma_f32_16x16x32_{f16,bf16}: C(16x16 f32) += A(16x32) * B(32x16).
// Lane l holds A[row l%16][k 8*(l/16) .. +8], B[k 8*(l/16) .. +8][col l%16] and
// C[row 4*(l/16)+i][col l%16] for i = 0..3 (layout checked on the hardware).
template <int DT>
__device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (DT == TMS_DTYPE_F16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
}

// Stores the quiet-NaN score of an invalid document as an integer. Device code is built
// with -fno-honor-nans, under which a NaN that passes through any float operation
// (an add, a select, a max) is undefined, so the marker never enters float arithmetic:
// kernels carry "invalid" as an integer flag and this is the document's final write.
__device__ __forceinline__ void store_nan_score(float* p) { *(uint32_t*)p = 0x7fc00000u; }

// A value the whole wave shares, moved to scalar registers (so control flow that depends
// on it is uniform to the compiler).
__device__ __forceinline__ int64_t wave_uniform(int64_t x) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)x >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// Cross-lane reductions over the four 16-lane rows of a wave (lanes l, l^16, l^32, l^48)
// with gfx950's row swaps, and over the 16 lanes of a row with DPP; every lane taking
// part receives the result.
__device__ __forceinline__ float cross_row_max(float m) {
  const auto p = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, m), __builtin_bit_cast(unsigned, m), false, false);
  m = fmaxf(__builtin_bit_cast(float, (unsigned)p[0]), __builtin_bit_cast(float, (unsigned)p[1]));
  const auto q = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, m), __builtin_bit_cast(unsigned, m), false, false);
  return fmaxf(__builtin_bit_cast(float, (unsigned)q[0]), __builtin_bit_cast(float, (unsigned)q[1]));
}
// Sum over the four rows, added as (row 0 + row 2) + (row 1 + row 3) in every lane.
__device__ __forceinline__ float cross_row_sum(float m) {
  const auto p = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, m), __builtin_bit_cast(unsigned, m), false, false);
  m = __builtin_bit_cast(float, (unsigned)p[0]) + __builtin_bit_cast(float, (unsigned)p[1]);
  const auto q = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, m), __builtin_bit_cast(unsigned, m), false, false);
  return __builtin_bit_cast(float, (unsigned)q[0]) + __builtin_bit_cast(float, (unsigned)q[1]);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, true));
}
__device__ __forceinline__ float row_sum16(float s) {
  s += dpp_f32<0xB1>(s);   // quad_perm [1,0,3,2]
  s += dpp_f32<0x4E>(s);   // quad_perm [2,3,0,1]
  s += dpp_f32<0x141>(s);  // row_half_mirror: the other quad of each half-row
  s += dpp_f32<0x140>(s);  // row_mirror: the other half of the row
  return s;
}

// Document end of the shared-tile kernels: NB query blocks of two 16-token halves, each
// half's running max rmax[j][h] in the MFMA accumulator layout (lane (c, g): the max over
// its rows of query token c). The row swaps move two accumulators at a time: register P
// holds blocks 2P and 2P + 1 (block 0 alone when NB == 1), and its 16-lane row k ends with
// the document's max of accumulator (2P + (k & 1), k >> 1) (of (0, k >> 1) when NB == 1),
// so the query masks and scales of each lane's row are picked once, by init(). Each block
// sums (0 + half 0) + half 1 per query token and then its 16 tokens by row_sum16: the bits
// of reducing every accumulator on its own.
template <int NB, bool QSCALE>
struct DocEnd {
  static constexpr int NPK = NB == 1 ? 1 : NB / 2;
  bool qv_pk[NPK];
  float qinv_pk[QSCALE ? NPK : 1];

  __device__ __forceinline__ void init(const bool (&qv)[NB][2], const float (&qinv)[QSCALE ? NB : 1][2], int lane) {
    const int krow = lane >> 4;
#pragma unroll
    for (int P = 0; P < NPK; P++) {
      qv_pk[P] = false;
      if constexpr (QSCALE) qinv_pk[P] = 1.f;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const int j = NB == 1 ? 0 : 2 * P + (k & 1), h = k >> 1;
        if (krow == k) {
          qv_pk[P] = qv[j][h];
          if constexpr (QSCALE) qinv_pk[P] = qinv[j][h];
        }
      }
    }
  }
  // rows 0-1: max over x's two 32-lane halves; rows 2-3: over y's
  __device__ static __forceinline__ float swap_max32(float x, float y) {
    const auto p = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, x), __builtin_bit_cast(unsigned, y),
                                                    false, false);
    return fmaxf(__builtin_bit_cast(float, (unsigned)p[0]), __builtin_bit_cast(float, (unsigned)p[1]));
  }
  // rows: max(x0, x1), max(y0, y1), max(x2, x3), max(y2, y3)
  __device__ static __forceinline__ float swap_max16(float x, float y) {
    const auto q = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, x), __builtin_bit_cast(unsigned, y),
                                                    false, false);
    return fmaxf(__builtin_bit_cast(float, (unsigned)q[0]), __builtin_bit_cast(float, (unsigned)q[1]));
  }
  // Lane doc_lane of pend[j] gets block j's score; every running max restarts at -inf.
  __device__ __forceinline__ void finish(float (&rmax)[NB][2], bool padded, int lane, int doc_lane,
                                         float (&pend)[NB]) const {
#pragma unroll
    for (int P = 0; P < NPK; P++) {
      float x;
      if constexpr (NB == 1) {
        const float p0 = swap_max32(rmax[0][0], rmax[0][1]);
        x = swap_max16(p0, p0);
      } else {
        const float p0 = swap_max32(rmax[2 * P][0], rmax[2 * P][1]);
        const float p1 = swap_max32(rmax[2 * P + 1][0], rmax[2 * P + 1][1]);
        x = swap_max16(p0, p1);
      }
      if constexpr (QSCALE) x *= qinv_pk[P];  // exact: a power of two
      if (padded) x = fmaxf(x, 0.f);
      x = 0.f + (qv_pk[P] ? x : 0.f);
      const auto q = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, x), __builtin_bit_cast(unsigned, x),
                                                      false, false);
      const float sm = row_sum16(__builtin_bit_cast(float, (unsigned)q[0]) + __builtin_bit_cast(float, (unsigned)q[1]));
#pragma unroll
      for (int b = 0; b < (NB == 1 ? 1 : 2); b++) {
        const int j = NB == 1 ? 0 : 2 * P + b;
        const float v = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sm), 16 * b));
        pend[j] = lane == doc_lane ? v : pend[j];
      }
    }
    const float NEG_INF = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < NB; j++) rmax[j][0] = rmax[j][1] = NEG_INF;
  }
};

// Per-thread last-error text behind tms_last_error().
void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);
int check_launch(const char* what);

}  // namespace tms
