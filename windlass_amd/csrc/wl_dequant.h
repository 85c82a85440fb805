// wl_dequant.h - host-side interface of the bit-exact dequantization kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wl {

bool dequant_supports(int type);
// dst[r][c] = value (row0 + r, c) of the tensor, r < nrows, c < cols.
hipError_t dequant_launch(int type, const uint8_t *w, int64_t row_bytes, int64_t row0, int64_t nrows,
                          int64_t cols, float *dst, hipStream_t st);

}  // namespace wl
