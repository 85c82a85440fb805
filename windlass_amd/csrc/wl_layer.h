// wl_layer.h - host interface of the decoder layer's other operations (wl_layer.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wl {

// The rows of a batch step (ForwardBatch): row t is at position pos[t] of cache slot slot[t],
// slots of cap positions each. All null: the rows of one sequence at pos0, pos0 + 1, ...
struct RowMap {
  const int *pos = nullptr;
  const int *slot = nullptr;
  int64_t cap = 0;
};

hipError_t rms_norm_launch(const float *x, int64_t rows, int64_t dim, const float *w, float eps, float *y,
                           hipStream_t st);
// RoPE on T rows of `heads` heads (row t at pos[t], or pos0 + t when pos is null).
hipError_t rope_launch(float *x, int64_t ldx, int T, int heads, int hd, int n, int neox, const int *pos, int pos0,
                       double base, double freq_scale, const float *freqs, hipStream_t st);
// A layer's RoPE on q [T][H*hd] and k [T][KH*hd] and the fp16 stores of k and v into cache rows
// pos0.. of Kc / Vc [positions][KH*hd], in one launch.
hipError_t rope_kv_launch(float *q, float *k, const float *v, int T, int H, int KH, int hd, int n, int neox,
                          int pos0, double base, double freq_scale, const float *freqs, uint16_t *Kc, uint16_t *Vc,
                          const RowMap &rm, hipStream_t st);
hipError_t kv_store_launch(const float *k, const float *v, int64_t n, uint16_t *K, uint16_t *V, hipStream_t st);
// Floats of scratch attention_launch needs for these operands; max_n: the most positions a row
// attends to (pos0 + T for one sequence).
int64_t attention_scratch_floats(int T, int heads, int hd, int kv_dim, int max_n, const uint16_t *K,
                                 const uint16_t *V);
hipError_t attention_launch(const float *q, int64_t ldq, int T, const uint16_t *K, const uint16_t *V, int kv_dim,
                            int heads, int kv_heads, int hd, int pos0, float scale, float *scratch, float *out,
                            int64_t ldo, const RowMap &rm, int max_n, hipStream_t st);
// RoPE angles by position (RopeTable): tab [positions][kRopePairs] of (cos, sin, the frequency
// factor used, 0), the pairs of n rotated dims at positions lo .. lo + count - 1 written by one
// launch. Readers check the factor against the model's and take the angle again on a mismatch.
constexpr int kRopePairs = 64;
hipError_t rope_table_launch(float4 *tab, int lo, int count, int n, double base, double freq_scale,
                             const float *freqs, hipStream_t st);
// Whether rope_attention_launch runs as one launch (and then reads the table) for these rows.
bool rope_attention_fused(int T, const RowMap &rm, int hd, int kv_heads, int n, const uint16_t *Kc,
                          const uint16_t *Vc);
// rope_kv_launch then attention_launch (q [T][H*hd] rotated, k rotated and both caches written,
// out [T][H*hd]) for rows whose earlier positions are all cached: one token of a sequence, or
// batch rows (rm) on distinct slots. Where rope_attention_fused holds this is one launch (the
// RoPE, with the rows' positions' angles from tab, and the cache stores inside it; q and k are
// then left as they were), with the same output and cache bits; otherwise the two launches.
hipError_t rope_attention_launch(float *q, float *k, const float *v, int T, int H, int KH, int hd, int n, int neox,
                                 int pos0, double base, double freq_scale, const float *freqs, const float4 *tab,
                                 uint16_t *Kc, uint16_t *Vc, const RowMap &rm, float scale, float *scratch,
                                 float *out, int max_n, hipStream_t st);
hipError_t residual_launch(float *x, const float *o, int64_t n, float rs, hipStream_t st);
// x[i] *= s
hipError_t scale_launch(float *x, int64_t n, float s, hipStream_t st);
// o [rows][dim] += f_t * sh, f_t = sigmoid(gl[t]) (gl null: 1): MoeFfn's shared expert.
hipError_t shared_expert_launch(float *o, const float *sh, const float *gl, int64_t rows, int64_t dim,
                                hipStream_t st);
// Workgroups per row of the first argmax launch; scratch holds 2 * rows * argmax_parts(n) words.
int argmax_parts(int64_t n);
hipError_t argmax_launch(const float *logits, int rows, int64_t n, int *out, float *scratch, hipStream_t st);
hipError_t bias_launch(float *y, const float *b, int64_t rows, int64_t dim, hipStream_t st);
hipError_t silu_mul_launch(float *g, const float *u, int64_t n, hipStream_t st);

}  // namespace wl
