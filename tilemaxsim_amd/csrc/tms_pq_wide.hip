// The MFMA PQ kernel for int16 / int32 codes, read at their own width (the reference
// scores int32 codes, src/flash_pqsim_kernel.py:219,233; a codebook of K > 256 centroids
// needs them). Its own translation unit, so these instantiations build in parallel.
#include "tms_pq_kernel.h"

namespace tms {

int run_pq_mfma_wide(const PqArgs& a, int dtype, int code_bytes, int64_t M, int64_t dsub, hipStream_t st) {
  if (dtype == TMS_DTYPE_F16) {
    if (code_bytes == 2) return run_pq_mfma<TMS_DTYPE_F16, TMS_DTYPE_F16, 2>(a, M, dsub, st);
    return run_pq_mfma<TMS_DTYPE_F16, TMS_DTYPE_F16, 4>(a, M, dsub, st);
  }
  if (code_bytes == 2) return run_pq_mfma<TMS_DTYPE_BF16, TMS_DTYPE_BF16, 2>(a, M, dsub, st);
  return run_pq_mfma<TMS_DTYPE_BF16, TMS_DTYPE_BF16, 4>(a, M, dsub, st);
}

}  // namespace tms
