// Host-side pieces of the row-wise top-k shared by tms_topk.hip (tms_topk) and
// tms_topk_noalloc.hip (tms_topk_noalloc). Every level kernel is instantiated and launched
// in tms_topk.hip only, so the no-alloc translation unit holds no kernels: its code
// object carries just the fixed scratch array.
#pragma once
#include <stdint.h>

#include <hip/hip_runtime.h>

namespace tms {

// Device workspace (bytes) of one call: the intermediate keys of every level.
int64_t topk_workspace_bytes(int64_t nrows, int64_t n, int k);

// Argument checks shared by the entry points (TMS_OK, or the status set through fail()).
int topk_checks(const char* fn, const float* scores, int64_t nrows, int64_t n, int64_t k, const float* out_values,
                const int64_t* out_indices);

// Launch every level on `st`; `workspace` holds topk_workspace_bytes(nrows, n, k) bytes.
int topk_run(const float* scores, int64_t nrows, int64_t n, int64_t k, void* workspace, float* out_values,
             int64_t* out_indices, hipStream_t st);

}  // namespace tms
