// bf16 MFMA products over packed signs (placeholder: not yet routed).
#include "common.hpp"

namespace qste {

int mfma_linear_forward(const void*, int, const uint8_t*, const float*, const float*, void*, int64_t,
                        int64_t, int64_t, hipStream_t) {
  return 1;
}
int mfma_linear_dgrad(const void*, int, const uint8_t*, const float*, void*, int64_t, int64_t, int64_t,
                      hipStream_t) {
  return 1;
}
int mfma_evidence(const void*, int, const uint8_t*, const float*, float*, int64_t, int64_t, int64_t,
                  const float*, const float*, const uint8_t*, float*, hipStream_t) {
  return 1;
}
int64_t mfma_evidence_tiles(int64_t) { return 0; }
int gemv_linear_forward(const void*, int, const uint8_t*, const float*, const float*, void*, int64_t,
                        int64_t, int64_t, hipStream_t) {
  return 1;
}

}  // namespace qste
