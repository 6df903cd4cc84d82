// The MFMA PQ kernel for fp32 queries against an fp16 / bf16 codebook: each query element
// is split into hi + lo terms of the codebook type (fp16 after a per-token power-of-two
// scale) and a product takes two MFMAs, so the query is not rounded to 16 bits (the
// reference builds its table from the fp32 query, src/flash_pqsim_kernel.py:54-67).
// uint8 codes. Its own translation unit, so these instantiations build in parallel.
#include "tms_pq_kernel.h"

namespace tms {

int run_pq_mfma_q32(const PqArgs& a, int dtype, int64_t M, int64_t dsub, hipStream_t st) {
  if (dtype == TMS_DTYPE_F16) return run_pq_mfma<TMS_DTYPE_F16, TMS_DTYPE_F32, 1>(a, M, dsub, st);
  return run_pq_mfma<TMS_DTYPE_BF16, TMS_DTYPE_F32, 1>(a, M, dsub, st);
}

}  // namespace tms
