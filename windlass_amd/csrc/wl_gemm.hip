// wl_gemm.hip - prefill GEMM (T > 8): placeholder until the MFMA kernel lands; T > 8 runs the
// decode GEMV in passes of 8 tokens.
#include "wl_gemm.h"

namespace wl {

bool gemm_supports(int) { return false; }

hipError_t gemm_launch(int, const uint8_t *, int64_t, int, int, const float *, int, float *, hipStream_t) {
  return hipErrorInvalidValue;
}

}  // namespace wl
