// wl_fmma.h - host-side interface of the float decode GEMV on the matrix cores.
#pragma once
#include "wl_gemv.h"

namespace wl {

// Formats the matrix-core float GEMV takes (Q4_K, Q6_K).
bool fmma_supports(int type);
// Whether one fmma_run takes this matrix set: every matrix in such a format, rows a whole
// number of super-blocks, the SwiGLU pair of one format.
bool fmma_applies(const GemvMat *mats, int nmat, int nm, int cols);
// Scratch floats of a launch (its per-unit partials).
int64_t fmma_scratch_floats(const GemvMat *mats, int nmat, int nm, int cols, int T);
// y = W x for nmat matrices sharing x [T][ldx] (1 <= T <= 8) on v_mfma_f32_16x16x32_f16, plus
// one launch adding the 2048-column units in order (SiLU for the pair, the residual add). A
// token's result does not depend on T.
hipError_t fmma_run(const GemvMat *mats, int nmat, int nm, const float *x, int ldx, int cols, int T,
                    float *scratch, int num_cu, hipStream_t st);

}  // namespace wl
