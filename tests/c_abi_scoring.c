/* A plain C consumer of the C ABI that scores on the GPU: includes tilemaxsim.h, links
 * libtilemaxsim.so and the HIP runtime, owns every device buffer (the library allocates
 * nothing), and checks each call against a float64 restatement computed here.
 *
 *   tms_maxsim_dense   32 query tokens x 300 documents x 40 tokens, d = 128, fp16
 *   tms_maxsim_varlen  the same tokens as ragged documents (an empty one scores -inf)
 *   tms_topk           top-10 of the dense scores (values descending, ties to the lower index)
 *   tms_maxsim_topk    the same scores and top-10 in one launch (a zeroed ticket block)
 *   tms_pq_score       M = 16, K = 256, dsub = 8 codes against an fp16 codebook
 *
 * Inputs are multiples of 2^-10 in [-1, 1], exact in fp16. Scores must lie within the
 * fp32-accumulation bar (d + Nq) * 2^-23 * MaxSim(|Q|, |D|) of the float64 values.
 * Each step prints its name before it runs. Exit status 0 = every check held; otherwise
 * the number of the failed check. */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "tilemaxsim.h"

#define NQ 32
#define DIM 128
#define B 300
#define ND 40
#define TOPK 10
#define PQ_M 16
#define PQ_K 256
#define PQ_DSUB 8

static uint32_t rng_state = 12345u;
static int rnd(int n) { /* xorshift32, uniform enough for test data */
  rng_state ^= rng_state << 13;
  rng_state ^= rng_state >> 17;
  rng_state ^= rng_state << 5;
  return (int)(rng_state % (uint32_t)n);
}

/* fp16 bits of k / 1024 for |k| <= 1024 (exact: at most 11 significant bits) */
static uint16_t half_of(int k) {
  if (k == 0) return 0;
  uint16_t sign = k < 0 ? 0x8000u : 0;
  int a = k < 0 ? -k : k, e = 0;
  while ((a >> e) > 1) e++;          /* a = 2^e * (1 + f), 0 <= e <= 10 */
  int exp = e - 10 + 15;             /* value a * 2^-10 = 2^(e - 10) * (1 + f) */
  int frac = (a << (10 - e)) & 0x3ff;
  return (uint16_t)(sign | (exp << 10) | frac);
}

static double value_of(uint16_t h) {
  int e = (h >> 10) & 0x1f, f = h & 0x3ff;
  double v = e ? ldexp(1.0 + f / 1024.0, e - 15) : ldexp(f / 1024.0, -14);
  return (h & 0x8000u) ? -v : v;
}

static void fill(uint16_t* x, size_t n) {
  for (size_t i = 0; i < n; i++) x[i] = half_of(rnd(2049) - 1024);
}

/* sum_i max_j <q_i, t_j> over tokens t_0 .. t_{nt-1} (rows of `dim` doubles), and the same
 * on absolute values into *abs_out; -inf for no tokens */
static double maxsim(const double* q, const double* t, int nt, int dim, double* abs_out) {
  double s = 0.0, sa = 0.0;
  if (nt == 0) {
    *abs_out = 0.0;
    return -INFINITY;
  }
  for (int i = 0; i < NQ; i++) {
    double m = -INFINITY, ma = -INFINITY;
    for (int j = 0; j < nt; j++) {
      double dot = 0.0, da = 0.0;
      for (int k = 0; k < dim; k++) {
        dot += q[i * dim + k] * t[j * dim + k];
        da += fabs(q[i * dim + k] * t[j * dim + k]);
      }
      if (dot > m) m = dot;
      if (da > ma) ma = da;
    }
    s += m;
    sa += ma;
  }
  *abs_out = sa;
  return s;
}

static int within(const float* got, const double* ref, const double* absref, int n, int dim) {
  for (int b = 0; b < n; b++) {
    if (isinf(ref[b])) {
      if (!(isinf(got[b]) && got[b] < 0)) return 0;
      continue;
    }
    if (fabs((double)got[b] - ref[b]) > (dim + NQ) * ldexp(1.0, -23) * absref[b]) return 0;
  }
  return 1;
}

#define HIP_OK(x)                                                   \
  do {                                                              \
    if ((x) != hipSuccess) {                                        \
      fprintf(stderr, "HIP error at %s:%d\n", __FILE__, __LINE__); \
      return 100;                                                   \
    }                                                               \
  } while (0)

int main(void) {
  static uint16_t hq[NQ * DIM], hd[B * ND * DIM], hcb[PQ_M * PQ_K * PQ_DSUB];
  static uint8_t hcodes[B * ND * PQ_M];
  static double q[NQ * DIM], d[B * ND * DIM], tok[ND * DIM], ref[B], absref[B];
  static float scores[B], vals[TOPK], fvals[TOPK], fscores[B];
  static int64_t idx[TOPK], fidx[TOPK], offsets[B + 1];
  fill(hq, NQ * DIM);
  fill(hd, (size_t)B * ND * DIM);
  fill(hcb, PQ_M * PQ_K * PQ_DSUB);
  for (int i = 0; i < B * ND * PQ_M; i++) hcodes[i] = (uint8_t)rnd(PQ_K);
  for (int i = 0; i < NQ * DIM; i++) q[i] = value_of(hq[i]);
  for (int i = 0; i < B * ND * DIM; i++) d[i] = value_of(hd[i]);

  void *dq, *dd, *dout, *dvals, *didx, *dcnt, *dcb, *dcodes, *doffs, *dfs, *dfv, *dfi;
  HIP_OK(hipMalloc(&dq, sizeof hq));
  HIP_OK(hipMalloc(&dd, sizeof hd));
  HIP_OK(hipMalloc(&dout, sizeof scores));
  HIP_OK(hipMalloc(&dvals, sizeof vals));
  HIP_OK(hipMalloc(&didx, sizeof idx));
  HIP_OK(hipMalloc(&dcnt, TMS_MAXSIM_TOPK_COUNTER_WORDS * sizeof(uint32_t)));
  HIP_OK(hipMalloc(&dcb, sizeof hcb));
  HIP_OK(hipMalloc(&dcodes, sizeof hcodes));
  HIP_OK(hipMalloc(&doffs, sizeof offsets));
  HIP_OK(hipMalloc(&dfs, sizeof fscores));
  HIP_OK(hipMalloc(&dfv, sizeof fvals));
  HIP_OK(hipMalloc(&dfi, sizeof fidx));
  HIP_OK(hipMemcpy(dq, hq, sizeof hq, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dd, hd, sizeof hd, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dcb, hcb, sizeof hcb, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dcodes, hcodes, sizeof hcodes, hipMemcpyHostToDevice));
  HIP_OK(hipMemset(dcnt, 0, TMS_MAXSIM_TOPK_COUNTER_WORDS * sizeof(uint32_t)));

  printf("tms_maxsim_dense\n");
  fflush(stdout);
  if (tms_maxsim_dense(dq, NQ, DIM, dd, B, ND, TMS_DTYPE_F16, (float*)dout, NULL) != TMS_OK) return 1;
  HIP_OK(hipMemcpy(scores, dout, sizeof scores, hipMemcpyDeviceToHost));
  for (int b = 0; b < B; b++) ref[b] = maxsim(q, d + (size_t)b * ND * DIM, ND, DIM, &absref[b]);
  if (!within(scores, ref, absref, B, DIM)) return 2;

  printf("tms_topk\n");
  fflush(stdout);
  int64_t ws = tms_topk_workspace_size(1, B, TOPK);
  if (ws != 0) return 3; /* one 300-score row fits one chunk */
  if (tms_topk((const float*)dout, 1, B, TOPK, NULL, 0, (float*)dvals, (int64_t*)didx, NULL) != TMS_OK) return 4;
  HIP_OK(hipMemcpy(vals, dvals, sizeof vals, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(idx, didx, sizeof idx, hipMemcpyDeviceToHost));
  for (int r = 0; r < TOPK; r++) { /* rank r: the r-th largest score, ties to the lower index */
    int best = -1;
    for (int b = 0; b < B; b++) {
      int taken = 0;
      for (int s = 0; s < r; s++) taken |= (idx[s] == b);
      if (!taken && (best < 0 || scores[b] > scores[best])) best = b;
    }
    if (idx[r] != best || vals[r] != scores[best]) return 5;
  }

  printf("tms_maxsim_topk\n");
  fflush(stdout);
  if (tms_maxsim_topk(dq, NQ, DIM, dd, B, ND, TMS_DTYPE_F16, TOPK, (float*)dfs, (float*)dfv, (int64_t*)dfi,
                      (uint32_t*)dcnt, NULL) != TMS_OK)
    return 6;
  HIP_OK(hipMemcpy(fscores, dfs, sizeof fscores, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(fvals, dfv, sizeof fvals, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(fidx, dfi, sizeof fidx, hipMemcpyDeviceToHost));
  if (memcmp(fscores, scores, sizeof scores) != 0) return 7; /* the same bits as the two calls */
  if (memcmp(fvals, vals, sizeof vals) != 0 || memcmp(fidx, idx, sizeof idx) != 0) return 8;

  printf("tms_maxsim_varlen\n");
  fflush(stdout);
  offsets[0] = 0;
  for (int b = 0; b < B; b++) offsets[b + 1] = offsets[b] + (b == 7 ? 0 : 1 + rnd(ND));
  HIP_OK(hipMemcpy(doffs, offsets, sizeof offsets, hipMemcpyHostToDevice));
  if (tms_maxsim_varlen(dq, NQ, DIM, dd, (int64_t)B * ND, (const int64_t*)doffs, B, TMS_DTYPE_F16, (float*)dout,
                        NULL) != TMS_OK)
    return 9;
  HIP_OK(hipMemcpy(scores, dout, sizeof scores, hipMemcpyDeviceToHost));
  for (int b = 0; b < B; b++)
    ref[b] = maxsim(q, d + offsets[b] * DIM, (int)(offsets[b + 1] - offsets[b]), DIM, &absref[b]);
  if (!within(scores, ref, absref, B, DIM) || !(isinf(scores[7]) && scores[7] < 0)) return 10;

  printf("tms_pq_score\n");
  fflush(stdout);
  if (tms_pq_score(dq, NQ, dcb, PQ_M, PQ_K, PQ_DSUB, TMS_DTYPE_F16, (const uint8_t*)dcodes, B, ND, (float*)dout,
                   NULL) != TMS_OK)
    return 11;
  HIP_OK(hipMemcpy(scores, dout, sizeof scores, hipMemcpyDeviceToHost));
  for (int b = 0; b < B; b++) {
    for (int t = 0; t < ND; t++)
      for (int m = 0; m < PQ_M; m++)
        for (int j = 0; j < PQ_DSUB; j++)
          tok[t * DIM + m * PQ_DSUB + j] =
              value_of(hcb[(m * PQ_K + hcodes[((size_t)b * ND + t) * PQ_M + m]) * PQ_DSUB + j]);
    ref[b] = maxsim(q, tok, ND, DIM, &absref[b]);
  }
  if (!within(scores, ref, absref, B, DIM)) return 12;

  HIP_OK(hipDeviceSynchronize());
  printf("ok\n");
  return 0;
}
