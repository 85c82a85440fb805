// wl_dequant.h - host-side interface of the bit-exact dequantization kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wl {

bool dequant_supports(int type);
// dst[r][c] = value (row0 + r, c) of the tensor, r < nrows, c < cols.
hipError_t dequant_launch(int type, const uint8_t *w, int64_t row_bytes, int64_t row0, int64_t nrows,
                          int64_t cols, float *dst, hipStream_t st);
// dst[r][c] = value (ids[r], c) for the device row ids ids[0..nrows); an id outside
// [0, tensor_rows) gives a row of zeros.
hipError_t dequant_rows_launch(int type, const uint8_t *w, int64_t row_bytes, const int32_t *ids, int64_t nrows,
                               int64_t tensor_rows, int64_t cols, float *dst, hipStream_t st);

}  // namespace wl
