/*
 * C restatement of the MaxSim / PQ-ADC oracle -- TEST INFRASTRUCTURE ONLY.
 *
 * Plain loops in double precision over float inputs (the fp16/bf16 values widened to
 * float by the caller). It is an implementation independent of the numpy oracle
 * (oracle/maxsim_oracle.py: BLAS matmul + reductions) so the two can check each other
 * at sizes where pure-Python brute force is too slow. Only tests/ load it.
 *
 * Reference semantics followed:
 *   src/flash_maxsim_kernel.py:280-288   score[b] = sum_i max_j <Q[i], D[b,j]>
 *   src/flash_maxsim_v2.py:102,120,127   empty document -> -inf, padded queries -> 0
 *   src/e2e_retrieval_quality.py:105-110 masked tokens are -inf before the max
 *   src/flash_maxsim_kernel.py:248-273   variable-length documents by offsets
 *   src/flash_pqsim_kernel.py:31-67      T[q,m,k] = sum_j Q[q,m*dsub+j] C[m,k,j]
 *   src/flash_pqsim_kernel.py:283-313    decompress then score
 */
#include <math.h>
#include <stdint.h>

static double dot(const float* a, const float* b, int64_t d) {
  double s = 0.0;
  for (int64_t k = 0; k < d; k++) s += (double)a[k] * (double)b[k];
  return s;
}

/* rows: pointer to the first token of the document; valid: optional per-token mask */
static double score_doc(const float* Q, int64_t nq, int64_t d, const float* rows, int64_t len,
                        const uint8_t* valid) {
  if (nq == 0) return 0.0;
  double total = 0.0;
  for (int64_t i = 0; i < nq; i++) {
    double best = -INFINITY;
    for (int64_t j = 0; j < len; j++) {
      if (valid && !valid[j]) continue;
      double v = dot(Q + i * d, rows + j * d, d);
      if (v > best) best = v;
    }
    total += best;
  }
  return total;
}

void orc_maxsim_dense(const float* Q, int64_t nq, int64_t d, const float* D, int64_t B, int64_t nd, double* out) {
  for (int64_t b = 0; b < B; b++) out[b] = score_doc(Q, nq, d, D + b * nd * d, nd, 0);
}

void orc_maxsim_masked(const float* Q, int64_t nq, int64_t d, const float* D, const uint8_t* mask, int64_t B,
                       int64_t nd, double* out) {
  for (int64_t b = 0; b < B; b++) out[b] = score_doc(Q, nq, d, D + b * nd * d, nd, mask + b * nd);
}

void orc_maxsim_varlen(const float* Q, int64_t nq, int64_t d, const float* Dflat, const int64_t* offsets, int64_t B,
                       double* out) {
  for (int64_t b = 0; b < B; b++)
    out[b] = score_doc(Q, nq, d, Dflat + offsets[b] * d, offsets[b + 1] - offsets[b], 0);
}

void orc_pq_build_lut(const float* Q, int64_t nq, const float* C, int64_t M, int64_t K, int64_t dsub, double* lut) {
  for (int64_t q = 0; q < nq; q++)
    for (int64_t m = 0; m < M; m++)
      for (int64_t k = 0; k < K; k++)
        lut[(q * M + m) * K + k] = dot(Q + q * M * dsub + m * dsub, C + (m * K + k) * dsub, dsub);
}

/* decompress each token into a double vector, then the dense score */
void orc_pq_score(const float* Q, int64_t nq, const float* C, int64_t M, int64_t K, int64_t dsub,
                  const uint8_t* codes, int64_t B, int64_t nd, double* out) {
  const int64_t d = M * dsub;
  for (int64_t b = 0; b < B; b++) {
    if (nq == 0) {
      out[b] = 0.0;
      continue;
    }
    double total = 0.0;
    for (int64_t i = 0; i < nq; i++) {
      double best = -INFINITY;
      for (int64_t t = 0; t < nd; t++) {
        const uint8_t* c = codes + (b * nd + t) * M;
        double s = 0.0;
        for (int64_t m = 0; m < M; m++) {
          const float* cv = C + (m * K + c[m]) * dsub;
          for (int64_t j = 0; j < dsub; j++) s += (double)Q[i * d + m * dsub + j] * (double)cv[j];
        }
        if (s > best) best = s;
      }
      total += best;
    }
    out[b] = total;
  }
}
