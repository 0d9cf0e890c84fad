// Chunked prefill (bf16 MFMA) -- placeholder until the MFMA kernel lands.
#include "gqa_internal.h"

namespace lara {

bool prefill_supported(int, int) { return false; }

hipError_t launch_prefill(int, int, const PrefillArgs&, hipStream_t) { return hipErrorInvalidValue; }

}  // namespace lara
