/* A plain C consumer of the C ABI: includes tilemaxsim.h, links libtilemaxsim.so and
 * calls entry points whose arguments are invalid, so every call returns its error status
 * before any HIP call (this runs on a machine without a GPU). Exit status 0 = all checks
 * held; otherwise the number of the failed check. */
#include <stdio.h>
#include <string.h>

#include "tilemaxsim.h"

int main(void) {
  if (tms_version() <= 0) return 1;
  float out[4];
  /* NULL documents */
  if (tms_maxsim_dense((const void*)out, 32, 128, NULL, 4, 8, TMS_DTYPE_F16, out, NULL) != TMS_ERR_INVALID) return 2;
  if (strlen(tms_last_error()) == 0) return 3;
  /* an unknown dtype */
  if (tms_maxsim_dense((const void*)out, 32, 128, (const void*)out, 4, 8, 7, out, NULL) != TMS_ERR_UNSUPPORTED) return 4;
  /* k larger than the row */
  if (tms_topk(out, 1, 4, 5, NULL, 0, out, NULL, NULL) != TMS_ERR_INVALID) return 5;
  if (tms_topk_workspace_size(1, 4096, 100) != 0) return 6;
  /* PQ codes of 3 bytes (1, 2 and 4 are taken) */
  if (tms_pq_score_lut_ex((const float*)out, 32, 16, 300, (const void*)out, 3, 1, 1, out, NULL) != TMS_ERR_INVALID)
    return 7;
  /* residual format: nbits 3 */
  if (tms_residual_decompress(NULL, NULL, 1, (const void*)out, 1, 128, (const void*)out, 3, out, NULL) !=
      TMS_ERR_UNSUPPORTED)
    return 8;
  /* one-launch score + top-k: more than 1,024 documents, and no ticket counter */
  if (tms_maxsim_topk((const void*)out, 32, 128, (const void*)out, 2000, 8, TMS_DTYPE_F16, 10, out, out, NULL, NULL,
                      NULL) != TMS_ERR_UNSUPPORTED)
    return 9;
  if (tms_maxsim_topk((const void*)out, 32, 128, (const void*)out, 16, 8, TMS_DTYPE_F16, 10, out, out,
                      (int64_t*)out, NULL, NULL) != TMS_ERR_INVALID)
    return 10;
  printf("ok %s\n", tms_last_error());
  return 0;
}
