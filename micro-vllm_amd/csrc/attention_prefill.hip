// MFMA prefill / chunked-prefill kernel (requests with more than one query).
#include "attention.h"

namespace mvllm {

bool prefill_supported(const AttnArgs&, int32_t) { return false; }

int launch_prefill(const AttnArgs&, int32_t, hipStream_t, hipEvent_t, hipEvent_t) {
  return fail(MVLLM_ERR_UNSUPPORTED, "prefill kernel not available");
}

}  // namespace mvllm
