// fp32 queries against fp16 / bf16 documents through the dense kernel: each query element
// is split into hi + lo terms of the document type (fp16 after a per-token power-of-two
// scale) and every product takes two MFMAs, so the query is not rounded to 16 bits. Its
// own translation unit, so these instantiations build in parallel with tms_dense.hip.
#include "tms_dense_kernel.h"

namespace tms {

int run_dense_q32(DenseArgs a, int64_t nQ, int dtype, int mode, bool aligned, hipStream_t st) {
  if (dtype == TMS_DTYPE_F16) return run_dense<TMS_DTYPE_F16, TMS_DTYPE_F32>(a, nQ, mode, aligned, st);
  return run_dense<TMS_DTYPE_BF16, TMS_DTYPE_F32>(a, nQ, mode, aligned, st);
}

}  // namespace tms
