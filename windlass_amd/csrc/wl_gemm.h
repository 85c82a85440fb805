// wl_gemm.h - host-side interface of the prefill GEMM (bf16 MFMA, fp32 accumulation).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wl {

bool gemm_supports(int type);

// K-chunks of a launch (1 when the output tiles alone fill the device).
int gemm_chunks(int type, int rows, int cols, int T, int num_cu);
// Bytes of scratch gemm_launch needs: x as bf16, then the chunk partials when K is split.
int64_t gemm_scratch_bytes(int type, int rows, int cols, int T, int num_cu);

// y[t * ldy + r] = sum_k W[r][k] * x[t][k] for T rows of x (x is [T][cols] fp32), W rows x cols
// raw blocks of `type`. The operands enter the matrix cores as bf16 (weights decoded exactly in
// fp32, then rounded to nearest even; x rounded the same way into `scratch`); products and sums
// are fp32. A split K adds the chunk partials in chunk order, so results are deterministic.
hipError_t gemm_launch(int type, const uint8_t *w, int64_t row_bytes, int rows, int cols, const float *x, int T,
                       float *y, int ldy, void *scratch, int num_cu, hipStream_t st);

// The 512-token tiles for Q4_K / Q6_K prompts of 384 tokens and more (wl_gemm_tall.hip):
// gemm_launch and gemm_scratch_bytes hand such calls to these.
bool gemm_tall_applies(int type, int T);
int64_t gemm_tall_scratch_bytes(int rows, int cols, int T, int num_cu);
hipError_t gemm_tall_launch(int type, const uint8_t *w, int64_t row_bytes, int rows, int cols, const float *x, int T,
                            float *y, int ldy, void *scratch, int num_cu, hipStream_t st);

}  // namespace wl
