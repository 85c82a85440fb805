// wl_layer.h - host interface of the decoder layer's other operations (wl_layer.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wl {

hipError_t rms_norm_launch(const float *x, int64_t rows, int64_t dim, const float *w, float eps, float *y,
                           hipStream_t st);
// cs: T * n floats of scratch for the cos/sin table
hipError_t rope_launch(float *x, int64_t ldx, int T, int heads, int hd, int n, int neox, const int *pos, int pos0,
                       double base, double freq_scale, const float *freqs, float *cs, hipStream_t st);
hipError_t kv_store_launch(const float *k, const float *v, int64_t n, uint16_t *K, uint16_t *V, hipStream_t st);
// scores: T * heads * (pos0 + T) floats of scratch
hipError_t attention_launch(const float *q, int64_t ldq, int T, const uint16_t *K, const uint16_t *V, int kv_dim,
                            int heads, int kv_heads, int hd, int pos0, float scale, float *scores, float *out,
                            int64_t ldo, hipStream_t st);
hipError_t residual_launch(float *x, const float *o, int64_t n, float rs, hipStream_t st);
hipError_t argmax_launch(const float *logits, int rows, int64_t n, int *out, hipStream_t st);
hipError_t bias_launch(float *y, const float *b, int64_t rows, int64_t dim, hipStream_t st);
hipError_t silu_mul_launch(float *g, const float *u, int64_t n, hipStream_t st);

}  // namespace wl
