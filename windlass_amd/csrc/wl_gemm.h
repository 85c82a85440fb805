// wl_gemm.h - host-side interface of the prefill GEMM (bf16 MFMA, fp32 accumulation).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wl {

bool gemm_supports(int type);

// Bytes of scratch gemm_launch needs for T rows of x of `cols` values (x as bf16).
inline int64_t gemm_scratch_bytes(int T, int cols) { return (int64_t)T * cols * 2; }

// y[t * ldy + r] = sum_k W[r][k] * x[t][k] for T rows of x (x is [T][cols] fp32), W rows x cols
// raw blocks of `type`. The operands enter the matrix cores as bf16 (weights decoded exactly in
// fp32, then rounded to nearest even; x rounded the same way into `scratch`); products and sums
// are fp32.
hipError_t gemm_launch(int type, const uint8_t *w, int64_t row_bytes, int rows, int cols, const float *x, int T,
                       float *y, int ldy, void *scratch, hipStream_t st);

}  // namespace wl
