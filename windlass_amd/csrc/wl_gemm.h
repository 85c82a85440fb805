// wl_gemm.h - host-side interface of the prefill GEMM (MFMA) launches.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wl {

bool gemm_supports(int type);
// y[t][r] = dot(W[r], x[t]) for T rows of x; W is rows x cols raw blocks of `type`.
hipError_t gemm_launch(int type, const uint8_t *w, int64_t row_bytes, int rows, int cols, const float *x, int T,
                       float *y, hipStream_t st);

}  // namespace wl
