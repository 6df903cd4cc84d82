// Small-batch MaxSim (candidate reranking): one or two query blocks against up to a few
// thousand documents, d in {32, 64, 96, 128}, fp16 / bf16, fixed-length, masked or
// variable-length documents.
//
// At these sizes the streaming kernels give each wave one whole document, so a call of
// 256 documents occupies 64 of the chip's 256 CUs and each wave walks its document's
// tiles one after another. Here a document is split over wpd = 1, 2 or 4 waves of one
// workgroup: wave part p scores the document's 16-token tiles p, p + wpd, p + 2 wpd, ...
// (up to three tiles in flight, none loaded twice), the per-column maxima of the parts
// meet in LDS, and part 0 sums them over query tokens and writes the score. A workgroup
// of four waves holds 4 / wpd documents and loads the query fragments once, into LDS.
//
// Semantics as the streaming kernels (src/flash_maxsim_v2.py:73-190,
// src/flash_maxsim_kernel.py:248-273, src/e2e_retrieval_quality.py:105-110): fp32
// accumulation; masked-out tokens are -inf before the max; query rows past nq contribute
// 0; an empty document scores -inf, or 0 when zero-padded to pad_len > 0 tokens;
// variable-length documents with invalid offsets score NaN (stored as integer bits).
#include <string.h>

#include <atomic>

#include "tms_topk_kernel.h"

namespace tms {

enum { RR_FIXED = 0, RR_VARLEN = 1, RR_MASKED = 2 };

struct RerankArgs {
  const uint8_t* Q;        // (nQ * nq, d)
  const uint8_t* D;        // fixed / masked: (B, nd, d); varlen: (T, d)
  const int64_t* offsets;  // varlen: (B + 1)
  const uint8_t* mask;     // masked: (B, nd), non-zero = real token
  float* out;              // (nQ, B)
  int64_t B, nd, T, pad_len;
  int32_t nq, nbq;         // tokens per query, 32-token blocks per query
  int32_t blk0, nblk;      // query blocks [blk0, blk0 + nblk) of this launch, nblk <= NB
  int32_t d;               // 32 * KS
  int32_t wpd;             // waves per document: 1, 2 or 4
  int32_t mask4;           // masked: nd % 4 == 0 and a 4-byte aligned mask (word loads)
};

// NT threads per workgroup (NT / 64 waves; NT / 64 / wpd documents).
template <int DT, int KS, int NB, int MODE, int NT = 256>
__device__ __forceinline__ void rerank_body(const RerankArgs& a) {
  constexpr int R = 3;  // ring of tiles: two in flight while one is scored
  const int lane = threadIdx.x & 63;
  const int r = lane & 15, g = lane >> 4;
  const int wid = threadIdx.x >> 6;
  const float NEG_INF = -__builtin_inff();
  constexpr int NFRAG = NB * KS * 2 * 64;
  constexpr int NW = NT / 64;
  __shared__ u32x4 qlds[NFRAG];         // query fragments, in the order the waves read them
  __shared__ float red[NW][NB][2][16];  // per-column maxima of each wave

  const int wpd = a.wpd;
  const int part = wid % wpd;
  const int64_t b = (int64_t)blockIdx.x * (NW / wpd) + wid / wpd;
  const bool live = b < a.B;

  // query fragments: block j, half h, step s -> token 16h + rr of the block, chunk 4s + g
  auto q_valid = [&](int j, int h, int rr, int64_t& row) -> bool {
    const int jb = a.blk0 + j;
    const int qi = jb / a.nbq;
    const int tok = (jb - qi * a.nbq) * 32 + 16 * h + rr;
    row = (int64_t)qi * a.nq + tok;
    return j < a.nblk && tok < a.nq;
  };
  // this thread's share of the query fragments (fragment f = ((j KS + s) 2 + h) 64 + lane),
  // loaded now and stored to LDS after the first tiles are in flight
  constexpr int QPT = (NFRAG + NT - 1) / NT;
  u32x4 qtmp[QPT];
#pragma unroll
  for (int i = 0; i < QPT; i++) {
    const int f = threadIdx.x + NT * i;
    const int fl = f & 63, h = (f >> 6) & 1, s = (f >> 7) % KS, j = (f >> 7) / KS;
    int64_t row;
    const bool v = f < NFRAG && q_valid(j, h, fl & 15, row);
    qtmp[i] = v ? *(const u32x4*)(a.Q + (row * a.d + 8 * (4 * s + (fl >> 4))) * 2) : u32x4{0u, 0u, 0u, 0u};
  }

  // the document's rows [base, base + len); invalid offsets mark it bad
  int64_t base = 0, len = 0;
  bool bad = false;
  if (live) {
    if constexpr (MODE == RR_VARLEN) {
      const int64_t s = a.offsets[b], e = a.offsets[b + 1];
      bad = s < 0 || e < s || e > a.T;
      base = bad ? 0 : s;
      len = bad ? 0 : e - s;
    } else {
      base = b * a.nd;
      len = a.nd;
    }
  }
  base = wave_uniform(base);
  len = wave_uniform(len);
  const int64_t ntile = (len + 15) / 16;
  const int64_t mine = ntile > part ? (ntile - part + wpd - 1) / wpd : 0;  // tiles of this part

  const int64_t row_bytes = (int64_t)a.d * 2;
  const uint8_t* dbase = a.D + base * row_bytes + (int64_t)(8 * g) * 2;
  // Tile i < mine of this part; rows past the document repeat its last token (a duplicate
  // cannot change a max).
  auto load = [&](u32x4 (&buf)[KS], uint32_t& bits, int64_t i) {
    const int64_t t = part + (int64_t)wpd * i;
    int64_t tok = t * 16 + r;
    if (tok > len - 1) tok = len - 1;
    const uint8_t* p = dbase + tok * row_bytes;
#pragma unroll
    for (int s = 0; s < KS; s++) buf[s] = *(const u32x4*)(p + 64 * s);
    if constexpr (MODE == RR_MASKED) {
      // validity of this lane's four output rows t*16 + 4g + k; a row past the document
      // repeats its last token, so it takes that token's mask byte
      const int64_t t0 = t * 16 + 4 * g;
      const uint8_t* mrow = a.mask + b * a.nd;
      uint32_t v = 0;
      if (a.mask4 && t * 16 + 16 <= len) {  // a whole tile (uniform): one word per lane
        const uint32_t w = *(const uint32_t*)(mrow + t0);
#pragma unroll
        for (int k = 0; k < 4; k++) v |= (((w >> (8 * k)) & 0xffu) != 0u ? 1u : 0u) << k;
      } else {
#pragma unroll
        for (int k = 0; k < 4; k++) v |= (mrow[t0 + k < len ? t0 + k : len - 1] != 0 ? 1u : 0u) << k;
      }
      bits = v;
    }
  };

  // up to R tiles in flight, then scored: a part holds a few tiles, so one batch is usually
  // all of them; the first batch is issued before the query fragments are waited for
  u32x4 ring[R][KS];
  uint32_t mb[R] = {0u, 0u, 0u};
#pragma unroll
  for (int k = 0; k < R; k++)
    if (k < mine) load(ring[k], mb[k], k);

#pragma unroll
  for (int i = 0; i < QPT; i++)
    if (threadIdx.x + NT * i < NFRAG) qlds[threadIdx.x + NT * i] = qtmp[i];
  __syncthreads();
  u32x4 qf[NB][KS][2];
#pragma unroll
  for (int j = 0; j < NB; j++)
#pragma unroll
    for (int s = 0; s < KS; s++)
#pragma unroll
      for (int h = 0; h < 2; h++) qf[j][s][h] = qlds[((j * KS + s) * 2 + h) * 64 + lane];

  float rmax[NB][2];
#pragma unroll
  for (int j = 0; j < NB; j++) rmax[j][0] = rmax[j][1] = NEG_INF;
  auto score = [&](const u32x4 (&buf)[KS], uint32_t bits) {
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
      for (int h = 0; h < 2; h++) {
        f32x4 v = acc[j][h];
        if constexpr (MODE == RR_MASKED) {
#pragma unroll
          for (int k = 0; k < 4; k++) v[k] = ((bits >> k) & 1u) ? v[k] : NEG_INF;
        }
        rmax[j][h] = fmaxf(rmax[j][h], fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3])));
      }
  };
  for (int64_t i0 = 0; i0 < mine; i0 += R) {
    const int64_t n = mine - i0;
    if (i0 > 0) {
#pragma unroll
      for (int k = 0; k < R; k++)
        if (k < n) load(ring[k], mb[k], i0 + k);
    }
#pragma unroll
    for (int k = 0; k < R; k++)
      if (k < n) score(ring[k], mb[k]);
  }

  // per-column maxima over the wave's rows, then over the document's parts
#pragma unroll
  for (int j = 0; j < NB; j++)
#pragma unroll
    for (int h = 0; h < 2; h++) rmax[j][h] = cross_row_max(rmax[j][h]);
  if (wpd > 1) {
    if (g == 0) {
#pragma unroll
      for (int j = 0; j < NB; j++)
#pragma unroll
        for (int h = 0; h < 2; h++) red[wid][j][h][r] = rmax[j][h];
    }
    __syncthreads();
    if (part == 0) {
      for (int p = 1; p < wpd; p++)
#pragma unroll
        for (int j = 0; j < NB; j++)
#pragma unroll
          for (int h = 0; h < 2; h++) rmax[j][h] = fmaxf(rmax[j][h], red[wid + p][j][h][r]);
    }
  }
  if (part != 0 || !live) return;

  if (bad) {  // every query of the launch scores NaN for this document
    if (lane == 0) {
#pragma unroll
      for (int j = 0; j < NB; j++) {
        if (j >= a.nblk) break;
        const int jb = a.blk0 + j;
        const int qi = jb / a.nbq;
        if (j == a.nblk - 1 || (jb + 1) / a.nbq != qi) store_nan_score(a.out + (int64_t)qi * a.B + b);
      }
    }
    return;
  }
  // zero padding up to pad_len adds dot products equal to 0 to a shorter document
  const bool padded_doc = MODE == RR_VARLEN && len < a.pad_len;
  float blk[NB];
#pragma unroll
  for (int j = 0; j < NB; j++) {
    float s = 0.f;
#pragma unroll
    for (int h = 0; h < 2; h++) {
      float m = rmax[j][h];
      if (padded_doc) m = fmaxf(m, 0.f);
      int64_t row;
      s += q_valid(j, h, r, row) ? m : 0.f;
    }
    // the streaming kernels' butterfly order, so a document scores the same bits on every path
    s += __shfl_xor(s, 8);
    s += __shfl_xor(s, 4);
    s += __shfl_xor(s, 2);
    s += __shfl_xor(s, 1);
    blk[j] = s;
  }
  if (lane == 0) {  // blocks of one query summed in order; a query begun in an earlier launch accumulates
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < NB; j++) {
      if (j >= a.nblk) break;
      const int jb = a.blk0 + j;
      const int qi = jb / a.nbq;
      s += blk[j];
      if (j == a.nblk - 1 || (jb + 1) / a.nbq != qi) {
        float* o = a.out + (int64_t)qi * a.B + b;
        *o = (qi * a.nbq < a.blk0) ? *o + s : s;
        s = 0.f;
      }
    }
  }
}

template <int DT, int KS, int NB, int MODE>
__global__ void __launch_bounds__(256) rerank_maxsim_kernel(RerankArgs a) {
  rerank_body<DT, KS, NB, MODE>(a);
}

// Scores plus their top-k in one launch (one query, B <= kShortRow documents): after a
// workgroup's scores are stored, thread 0 makes them visible device-wide (release fence)
// and takes a ticket; the workgroup that takes the last one fences (acquire), selects the
// top k of the B scores with the 1,024-key chunk of the top-k kernel, and resets the
// counter for the next call. Nothing waits on another workgroup.
//
// Tickets on one address serialise, so a grid of kTicketTwoLevel workgroups or more takes
// them in two levels: workgroup g on group counter g % kTicketGroups, the last of each
// group (after an acquire + release, which passes its group's scores on) on the top
// counter. Each counter has its own 64-byte line (TMS_MAXSIM_TOPK_COUNTER_WORDS words in
// all). Every counter the launch used is zero again when it ends.
struct TopkTail {
  uint32_t* counter;  // TMS_MAXSIM_TOPK_COUNTER_WORDS words, zero before the launch and after it
  float* values;      // (k)
  int64_t* indices;   // (k)
  int32_t k;
};
constexpr uint32_t kTicketGroups = 8, kTicketLine = 16, kTicketTwoLevel = 64;
static_assert(kTicketLine * (1 + kTicketGroups) == TMS_MAXSIM_TOPK_COUNTER_WORDS, "the counter block of the header");
// NT threads a workgroup: four waves while the call has at most 1,024 waves (a 256 x
// 180-token call then spreads over 256 CUs), eight or 16 above that, so that a launch has
// at most 256 workgroups -- or 512 at d = 128 with two query blocks, where workgroups
// stop at eight waves -- since each one takes a ticket and writes its XCD's L2 back, and
// those costs grow with the workgroup count.
template <int DT, int KS, int NB, int NT>
__global__ void __launch_bounds__(NT) rerank_topk_kernel(RerankArgs a, TopkTail t) {
  rerank_body<DT, KS, NB, RR_FIXED, NT>(a);
  __shared__ uint32_t last;
  // The barrier orders every wave's score stores before thread 0's agent-scope release
  // (cumulative: on this part it writes the XCD's L2 back, once per workgroup, not per
  // wave); a ticket is a relaxed RMW in that release sequence; the last workgroup's thread
  // 0 acquires before the second barrier hands the scores to its other waves.
  __syncthreads();
  if (threadIdx.x == 0) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    const uint32_t G = gridDim.x;
    uint32_t l;
    if (G < kTicketTwoLevel) {
      l = __hip_atomic_fetch_add(t.counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == G - 1 ? 1u : 0u;
    } else {
      const uint32_t grp = blockIdx.x % kTicketGroups;
      const uint32_t members = (G - grp + kTicketGroups - 1) / kTicketGroups;  // workgroups with this group
      uint32_t* gc = t.counter + kTicketLine * (1 + grp);
      l = 0u;
      if (__hip_atomic_fetch_add(gc, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == members - 1) {
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "agent");  // the group's scores, passed on
        __hip_atomic_store(gc, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        l = __hip_atomic_fetch_add(t.counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == kTicketGroups - 1
                ? 1u
                : 0u;
      }
    }
    if (l) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    last = l;
  }
  __syncthreads();
  if (!last) return;
  topk_chunk<true, true, NT, kShortRow>(a.out, a.B, nullptr, a.B, a.B, nullptr, 0, t.values, t.indices, t.k, 0, 0);
  if (threadIdx.x == 0) __hip_atomic_store(t.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int DT, int KS, int NB>
static int rerank_launch(const RerankArgs& a, int mode, int64_t grid, hipStream_t st) {
  if (mode == RR_VARLEN)
    hipLaunchKernelGGL((rerank_maxsim_kernel<DT, KS, NB, RR_VARLEN>), dim3((unsigned)grid), dim3(256), 0, st, a);
  else if (mode == RR_MASKED)
    hipLaunchKernelGGL((rerank_maxsim_kernel<DT, KS, NB, RR_MASKED>), dim3((unsigned)grid), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((rerank_maxsim_kernel<DT, KS, NB, RR_FIXED>), dim3((unsigned)grid), dim3(256), 0, st, a);
  return check_launch("rerank_maxsim_kernel");
}

template <int DT, int NB>
static int rerank_ks(const RerankArgs& a, int mode, int64_t grid, hipStream_t st) {
  switch (a.d / 32) {
    case 1: return rerank_launch<DT, 1, NB>(a, mode, grid, st);
    case 2: return rerank_launch<DT, 2, NB>(a, mode, grid, st);
    case 3: return rerank_launch<DT, 3, NB>(a, mode, grid, st);
    default: return rerank_launch<DT, 4, NB>(a, mode, grid, st);
  }
}

#ifndef TMS_RERANK_TARGET_WAVES
#define TMS_RERANK_TARGET_WAVES 2048  // waves a call aims for before splitting documents further
#endif
#ifndef TMS_RERANK_MAX_TILES
#define TMS_RERANK_MAX_TILES 16384  // default: document tiles (16 tokens) up to which a call takes this kernel
#endif
static std::atomic<int64_t> g_rerank_tiles{TMS_RERANK_MAX_TILES};

// Whether a call of B documents averaging `tokens_per_doc` tokens takes the small-batch
// kernel: few enough tiles that the streaming kernels' one-document-per-wave layout
// leaves the chip partly idle.
bool rerank_fits(int64_t B, int64_t tokens_per_doc) {
  const int64_t tiles = (tokens_per_doc + 15) / 16;
  return B > 0 && B * (tiles > 0 ? tiles : 1) <= g_rerank_tiles.load(std::memory_order_relaxed);
}

// Entry used by tms_dense.hip: nQ queries of nq tokens (at most 3 blocks in all, two per
// launch), d in {32, 64, 96, 128}, 16-byte aligned Q and D, fp16 / bf16. mode: 0 fixed,
// 1 variable-length (offsets, pad_len), 2 masked (mask). out is (nQ, B).
int run_rerank(const void* Q, int64_t nQ, int64_t nq, int64_t d, const void* D, int64_t B, int64_t nd, int64_t T,
               const int64_t* offsets, const uint8_t* mask, int64_t pad_len, int mode, int dtype, float* out,
               hipStream_t st) {
  RerankArgs a;
  memset(&a, 0, sizeof(a));
  a.Q = (const uint8_t*)Q;
  a.D = (const uint8_t*)D;
  a.offsets = offsets;
  a.mask = mask;
  a.out = out;
  a.B = B;
  a.nd = nd;
  a.T = T;
  a.pad_len = pad_len;
  a.nq = (int32_t)nq;
  a.nbq = (int32_t)((nq + 31) / 32);
  a.d = (int32_t)d;
  a.mask4 = (nd % 4 == 0 && ((uintptr_t)mask & 3) == 0) ? 1 : 0;
  // waves per document: enough for about two waves per SIMD (2,048), at most one per
  // tile of an average document
  const int64_t mean = mode == RR_VARLEN ? (B > 0 ? T / B : 0) : nd;
  const int64_t tiles = (mean + 15) / 16;
  a.wpd = 1;
  while (a.wpd < 4 && B * a.wpd < TMS_RERANK_TARGET_WAVES && 2 * a.wpd <= tiles) a.wpd *= 2;
  const int64_t grid = (B * a.wpd + 3) / 4;
  if (grid > 0x7fffffff) return fail(TMS_ERR_UNSUPPORTED, "small-batch MaxSim: too many documents");
  const int64_t nblocks = nQ * (int64_t)a.nbq;
  for (int64_t b0 = 0; b0 < nblocks; b0 += 2) {  // two query blocks per launch
    a.blk0 = (int32_t)b0;
    a.nblk = (int32_t)(nblocks - b0 < 2 ? nblocks - b0 : 2);
    int rc;
    if (a.nblk == 2)
      rc = dtype == TMS_DTYPE_F16 ? rerank_ks<TMS_DTYPE_F16, 2>(a, mode, grid, st)
                                  : rerank_ks<TMS_DTYPE_BF16, 2>(a, mode, grid, st);
    else
      rc = dtype == TMS_DTYPE_F16 ? rerank_ks<TMS_DTYPE_F16, 1>(a, mode, grid, st)
                                  : rerank_ks<TMS_DTYPE_BF16, 1>(a, mode, grid, st);
    if (rc) return rc;
  }
  return TMS_OK;
}

}  // namespace tms

namespace tms {

template <int DTV, int KS, int NB>
static void rerank_topk_launch(int nt, int64_t grid, hipStream_t st, const RerankArgs& a, const TopkTail& t) {
  constexpr int kMaxNT = (KS == 4 && NB == 2) ? 512 : 1024;  // never instantiated past the cap
  if (nt == 256)
    hipLaunchKernelGGL((rerank_topk_kernel<DTV, KS, NB, 256>), dim3((unsigned)grid), dim3(256), 0, st, a, t);
  else if (nt == 512)
    hipLaunchKernelGGL((rerank_topk_kernel<DTV, KS, NB, 512>), dim3((unsigned)grid), dim3(512), 0, st, a, t);
  else
    hipLaunchKernelGGL((rerank_topk_kernel<DTV, KS, NB, kMaxNT>), dim3((unsigned)grid), dim3(kMaxNT), 0, st, a, t);
}

template <int DTV>
static void rerank_topk_dispatch(int ks, bool two, int nt, int64_t grid, hipStream_t st, const RerankArgs& a,
                                 const TopkTail& t) {
  switch (ks) {
    case 1: two ? rerank_topk_launch<DTV, 1, 2>(nt, grid, st, a, t) : rerank_topk_launch<DTV, 1, 1>(nt, grid, st, a, t); break;
    case 2: two ? rerank_topk_launch<DTV, 2, 2>(nt, grid, st, a, t) : rerank_topk_launch<DTV, 2, 1>(nt, grid, st, a, t); break;
    case 3: two ? rerank_topk_launch<DTV, 3, 2>(nt, grid, st, a, t) : rerank_topk_launch<DTV, 3, 1>(nt, grid, st, a, t); break;
    default: two ? rerank_topk_launch<DTV, 4, 2>(nt, grid, st, a, t) : rerank_topk_launch<DTV, 4, 1>(nt, grid, st, a, t);
  }
}

}  // namespace tms

extern "C" int64_t tms_set_rerank_limit(int64_t tiles) {
  if (tiles < 0) return tms::g_rerank_tiles.load(std::memory_order_relaxed);
  return tms::g_rerank_tiles.exchange(tiles, std::memory_order_relaxed);
}

extern "C" int tms_maxsim_topk(const void* Q, int64_t nq, int64_t d, const void* D, int64_t B, int64_t nd, int dtype,
                               int64_t k, float* scores, float* out_values, int64_t* out_indices, uint32_t* counter,
                               void* stream) {
  using namespace tms;
  const char* fn = "tms_maxsim_topk";
  if (nq < 0 || d < 0 || B < 0 || nd < 0 || k < 0) return fail(TMS_ERR_INVALID, "%s: negative size", fn);
  if (k > B) return fail(TMS_ERR_INVALID, "%s: k=%lld exceeds the %lld documents", fn, (long long)k, (long long)B);
  if (dtype != TMS_DTYPE_F16 && dtype != TMS_DTYPE_BF16)
    return fail(TMS_ERR_UNSUPPORTED, "%s: fp16 / bf16 only (dtype %d); score, then tms_topk", fn, dtype);
  if (nq < 1 || nq > 64 || d < 32 || d > 128 || d % 32 != 0 || B < 1 || B > kShortRow || k < 1)
    return fail(TMS_ERR_UNSUPPORTED,
                "%s: one launch takes 1..64 query tokens, d in {32, 64, 96, 128} and 1..%d documents with k >= 1 "
                "(nq=%lld d=%lld B=%lld k=%lld); score, then tms_topk",
                fn, kShortRow, (long long)nq, (long long)d, (long long)B, (long long)k);
  if (!Q || !scores || !out_values || !out_indices || !counter || (nd > 0 && !D))
    return fail(TMS_ERR_INVALID, "%s: NULL pointer", fn);
  if (((uintptr_t)Q & 15) || ((uintptr_t)D & 15))
    return fail(TMS_ERR_UNSUPPORTED, "%s: Q and D must be 16-byte aligned; score, then tms_topk", fn);
  RerankArgs a;
  memset(&a, 0, sizeof(a));
  a.Q = (const uint8_t*)Q;
  a.D = (const uint8_t*)D;
  a.out = scores;
  a.B = B;
  a.nd = nd;
  a.nq = (int32_t)nq;
  a.nbq = (int32_t)((nq + 31) / 32);
  a.blk0 = 0;
  a.nblk = a.nbq;
  a.d = (int32_t)d;
  const int64_t tiles = (nd + 15) / 16;
  a.wpd = 1;
  while (a.wpd < 4 && B * a.wpd < TMS_RERANK_TARGET_WAVES && 2 * a.wpd <= tiles) a.wpd *= 2;
  const int64_t waves = B * a.wpd;
  int nt = waves <= 1024 ? 256 : (waves <= 2048 ? 512 : 1024);
  const int ks = (int)(d / 32);
  const bool two = a.nblk == 2;
  if (ks == 4 && two && nt > 512) nt = 512;  // 16 waves of that form spill registers
  const int64_t grid = (waves + nt / 64 - 1) / (nt / 64);
  TopkTail t{counter, out_values, out_indices, (int32_t)k};
  hipStream_t st = (hipStream_t)stream;
  if (dtype == TMS_DTYPE_F16)
    rerank_topk_dispatch<TMS_DTYPE_F16>(ks, two, nt, grid, st, a, t);
  else
    rerank_topk_dispatch<TMS_DTYPE_BF16>(ks, two, nt, grid, st, a, t);
  return check_launch("rerank_topk_kernel");
}
