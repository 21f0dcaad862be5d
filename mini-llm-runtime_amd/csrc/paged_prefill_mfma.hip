// bf16 chunk prefill on gfx950 matrix cores (not yet enabled: every call takes
// the generic kernel in paged_prefill.hip).
#include "paged_prefill.h"

namespace mlr {

bool prefill_mfma_eligible(int dtype, int64_t head_dim, int64_t block_size) {
  (void)dtype;
  (void)head_dim;
  (void)block_size;
  return false;
}

int launch_prefill_mfma(const PrefillParams &p, int64_t max_query_len,
                        hipStream_t stream) {
  (void)p;
  (void)max_query_len;
  (void)stream;
  return set_error(MLR_ERR_UNSUPPORTED, "mlr_paged_prefill: MFMA path disabled");
}

}  // namespace mlr
