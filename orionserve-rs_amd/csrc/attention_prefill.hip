// Chunked-prefill causal attention over the paged cache (placeholder until
// the MFMA kernel lands).
#include "common.hpp"
#include "kernels.hpp"

namespace orion {

hipError_t launch_paged_prefill(hipStream_t, const KvGeom&, const void*, int64_t, const float*,
                                int64_t, int64_t, const int32_t*, const int32_t*, const uint32_t*,
                                const int64_t*, const uint32_t*, int64_t, int64_t, float*) {
  return hipErrorNotSupported;
}

}  // namespace orion
