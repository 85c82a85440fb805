/*
 * windlass_hip.h - C ABI of the MI355X (gfx950) quantized-matmul library.
 *
 * The library takes raw GGUF weight blocks unchanged into one GPU's HBM and runs the
 * matrix-vector / matrix-matrix products of Windlass's decoder layer on hand-written
 * HIP kernels. Every entry point replaces one operator of the reference's CPU path; the
 * comment above each names the reference interface (file:line) it stands in for.
 *
 * Conventions
 *  - Return 0 (WL_OK) on success, a negative WL_E_* code otherwise; wl_last_error()
 *    gives the message (thread-local).
 *  - Activations are fp32 row-major: x is [T][cols], y is [T][rows], exactly the layout of
 *    Transformer.MatMul (src/Transformer.cs:483-486).
 *  - A context may be used by one thread at a time (the reference's engine holds
 *    lock(_run) around every model call, src/Engine.cs:138). Distinct contexts are
 *    independent.
 *  - Host-pointer entry points are synchronous. *_dev entry points take device pointers,
 *    are enqueued on wl_stream(ctx) and return before the GPU finishes.
 */
#ifndef WINDLASS_HIP_H
#define WINDLASS_HIP_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Error codes and the reference exception each maps to. */
#define WL_OK 0
#define WL_E_UNSUPPORTED (-1) /* NotSupportedException (src/Quants.cs:51,186) */
#define WL_E_SHAPE (-2)       /* ArgumentException "MatMul shape mismatch" (src/Transformer.cs:486) */
#define WL_E_DEVICE (-3)      /* HIP runtime failure; the server's BackendException 500 (src/Server.cs:756-761) */
#define WL_E_ARG (-4)         /* ArgumentOutOfRangeException / null argument (src/LayerStream.cs:28) */
#define WL_E_NOMEM (-5)       /* device allocation failed */

/* ggml type ids (enum GgmlType, src/Gguf.cs:19-25). */
#define WL_TYPE_F32 0
#define WL_TYPE_F16 1
#define WL_TYPE_Q4_0 2
#define WL_TYPE_Q4_1 3
#define WL_TYPE_Q5_0 6
#define WL_TYPE_Q5_1 7
#define WL_TYPE_Q8_0 8
#define WL_TYPE_Q2_K 10
#define WL_TYPE_Q3_K 11
#define WL_TYPE_Q4_K 12
#define WL_TYPE_Q5_K 13
#define WL_TYPE_Q6_K 14
#define WL_TYPE_IQ2_XXS 16
#define WL_TYPE_IQ4_NL 20
#define WL_TYPE_IQ3_S 21
#define WL_TYPE_IQ2_S 22
#define WL_TYPE_IQ4_XS 23
#define WL_TYPE_BF16 30
/* Ids the file format lays out (wl_type_layout) that no GPU path decodes: wl_upload refuses them. */
#define WL_TYPE_Q8_1 9
#define WL_TYPE_Q8_K 15
#define WL_TYPE_IQ2_XS 17
#define WL_TYPE_IQ3_XXS 18
#define WL_TYPE_IQ1_S 19
#define WL_TYPE_I8 24
#define WL_TYPE_I16 25
#define WL_TYPE_I32 26
#define WL_TYPE_I64 27
#define WL_TYPE_F64 28
#define WL_TYPE_IQ1_M 29

typedef struct wl_ctx wl_ctx;       /* one per model: a HIP stream plus scratch buffers */
typedef struct wl_weight wl_weight; /* raw GGUF blocks of one tensor in HBM (WeightView, src/LayerStream.cs:15-35) */

/* Library version (major*10000 + minor*100 + patch). */
int wl_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char *wl_last_error(void);

/* Quants.CanDecode (src/Quants.cs:11-21): 1 when wl_dequant_f32 handles the type. */
int wl_can_decode(int ggml_type);

/* Quants.CanDot (src/Quants.cs:56-65) widened to every type the GPU multiplies: 1 when
 * wl_matmul handles the type (the I-quants included, which the CPU path decodes first). */
int wl_can_matmul(int ggml_type);

/* FastMath.CanIntDot (src/FastMath.cs:27-30): 1 for Q8_0, Q4_0, Q4_K, Q5_K and Q6_K. */
int wl_can_int_dot(int ggml_type);

/* Fault injection for tests of the error paths (the reference has no counterpart; its
 * allocations fail with OutOfMemoryException): with n > 0, the n-th device allocation from now
 * on (a weight upload, a stage, a context's scratch growth) fails once with WL_E_NOMEM, without
 * allocating; the context stays usable. n = 0 disarms. Process-wide. */
int wl_debug_fail_alloc(int n);

/* Block geometry, GgmlTypes.TryGetLayout (src/Gguf.cs:30-66). Returns 1 when known. */
int wl_type_layout(int ggml_type, int *block_elems, int *block_bytes);

/* New context on HIP device `device` (the model's Transformer/LayerStream pair owns one;
 * src/Engine.cs:55-91). */
int wl_create(int device, wl_ctx **out);
void wl_destroy(wl_ctx *ctx);

/* The hipStream_t the context launches on, as void*. */
void *wl_stream(wl_ctx *ctx);

/* Waits for every launch queued on the context. Also the point where asynchronous failures of
 * those launches are reported: WL_E_DEVICE when a one-launch MoE (wl_moe_ffn_dev, the MoE layers
 * of wl_layer_dev / wl_layer_batch_dev) gave up one of its bounded waits since the last
 * synchronizing call on this context (its output is wrong). Each failure is reported once. */
int wl_sync(wl_ctx *ctx);

/* Copies raw GGUF blocks unchanged to HBM: LayerStream.Bind's view of one tensor
 * (src/LayerStream.cs:182-203). `rows` is per expert; `experts` stacked expert tensors
 * follow each other (src/Gguf.cs:97-101), 1 for an ordinary matrix. row_bytes must equal
 * cols/block*blockBytes. The host buffer stays the caller's. */
int wl_upload(wl_ctx *ctx, int ggml_type, const void *blocks, int64_t rows, int64_t cols,
              int64_t row_bytes, int32_t experts, wl_weight **out);

/* Releases a weight's device memory (a stage view: only the handle). */
int wl_weight_free(wl_ctx *ctx, wl_weight *w);

/* ---- Stages: LayerStream's slots in HBM (src/LayerStream.cs:36-264) ----
 * A stage is one slot of device memory holding a layer's tensors at 64-byte aligned offsets,
 * as LayerStream.Bind lays them out (:182-203). Resident mode (--cache-gb covering the model,
 * :110-124) uploads every stage once; streaming mode keeps two slots and uploads stage N+1 on
 * the context's copy stream while stage N computes (StartPrefetch / Acquire / WaitSlot,
 * :127-181). Ordering is explicit, as the slot tasks make it there:
 *   wl_stage_upload_async  queue host -> slot copies (host memory from wl_host_alloc copies at
 *                          link speed and must stay unchanged until the copies are done);
 *                          they wait for the slot's last wl_stage_release;
 *   wl_stage_ready         the compute stream waits for the slot's queued copies (Acquire);
 *   wl_stage_release       the compute queued so far is the slot's last reader (WaitSlot);
 *   wl_stage_sync          the host waits for the slot's copies. */
typedef struct wl_stage wl_stage;

/* Pinned host memory (LayerStream's slot buffers, Marshal.AllocHGlobal at :104-108). */
int wl_host_alloc(int64_t bytes, void **out);
int wl_host_free(void *p);

/* A slot of `bytes` (Stage.Bytes with its padding, :88-94). */
int wl_stage_create(wl_ctx *ctx, int64_t bytes, wl_stage **out);
int wl_stage_free(wl_ctx *ctx, wl_stage *stage);

/* LayerStream.Read into the slot (:206-235): `bytes` of host memory to `offset`, asynchronous. */
int wl_stage_upload_async(wl_ctx *ctx, wl_stage *stage, const void *host, int64_t offset, int64_t bytes);
int wl_stage_ready(wl_ctx *ctx, wl_stage *stage);
int wl_stage_release(wl_ctx *ctx, wl_stage *stage);
int wl_stage_sync(wl_ctx *ctx, wl_stage *stage);

/* Bind's WeightView of one tensor in the slot (:188-200): no copy, the arguments of wl_upload
 * at a 64-byte aligned offset. The view reads whatever the slot holds when a call runs. */
int wl_stage_weight(wl_ctx *ctx, wl_stage *stage, int64_t offset, int ggml_type, int64_t rows, int64_t cols,
                    int64_t row_bytes, int32_t experts, wl_weight **out);

/* Transformer.MatMul (src/Transformer.cs:483-537), with ForwardBatch's MatMulEach
 * (:544-561) built in: y[t][r] = dot(W[r], x[t]) for T rows of x; `expert` >= 0 selects
 * WeightView.Slice(expert) (src/LayerStream.cs:26-34), -1 the whole tensor.
 * T <= 8 runs the fp32 decode GEMV, whose result for a token does not depend on T (bit for
 * bit); T > 8 runs the MFMA GEMM (bf16 operands, fp32 accumulation). Synchronous. */
int wl_matmul(wl_ctx *ctx, const wl_weight *w, int32_t expert, const float *x, int32_t T, float *y);

/* Quants.DecodeRow (src/Quants.cs:32-52; src/IQuants.cs:27-42) for rows row0..row0+nrows-1
 * of the whole tensor (experts stacked), bit-exact: dst is [nrows][cols] fp32. */
int wl_dequant_f32(wl_ctx *ctx, const wl_weight *w, int64_t row0, int64_t nrows, float *dst);

/* SwiGlu (src/Transformer.cs:241-251): out = down(silu(gate x) * (up x)); x [T][embd],
 * out [T][down rows]. `expert` as in wl_matmul, applied to all three. Synchronous. */
int wl_swiglu(wl_ctx *ctx, const wl_weight *gate, const wl_weight *up, const wl_weight *down,
              int32_t expert, const float *x, int32_t T, float *out);

/* Route (src/Transformer.cs:313-340) for T tokens: softmax over n logits per token, the k
 * largest (ties to the lower id), renormalised when asked. sel/wts are [T][k]. */
int wl_route(wl_ctx *ctx, const float *logits, int32_t T, int32_t n, int32_t k, int32_t renorm,
             int32_t *sel, float *wts);

/* MoeFfn (src/Transformer.cs:259-294) given the router logits [T][n_expert]: route, run each
 * chosen expert's SwiGLU on its tokens, weighted sum. gate/up/down are stacked expert tensors
 * ([n_expert][ff][embd], [n_expert][ff][embd], [n_expert][embd][ff]). expert_runs (may be
 * NULL) receives the number of distinct experts computed (Transformer.ExpertRuns, :27).
 * Synchronous: WL_E_DEVICE when a one-launch MoE on this context gave up one of its bounded
 * waits since the last synchronizing call (as wl_sync reports it). */
int wl_moe_ffn(wl_ctx *ctx, const float *logits, int32_t k, int32_t renorm,
               const wl_weight *gate_exps, const wl_weight *up_exps, const wl_weight *down_exps,
               const float *x, int32_t T, float *out, int32_t *expert_runs);

/* Transformer.IntDot (src/Transformer.cs:23), set from --int-dot (src/Program.cs:50,215;
 * EngineOptions.IntDot, src/Engine.cs:22,70). Off by default. When on, wl_matmul(_dev), the
 * fused q/k/v entry and the SwiGLU entries multiply wl_can_int_dot weights whose rows are whole
 * activation blocks (FastMath.Fits, src/FastMath.cs:34) with the integer branch of MatMul
 * (src/Transformer.cs:504-524): the T rows of x are quantized once (FastMath.Quantize), then
 * y[t][r] = FastMath.IntDot(W[r], activations of t) (src/FastMath.cs:105-214), bit-identical to
 * the reference for every T. The MoE entries give the experts' gate/up and down products the
 * same branch (MoeFfn -> SwiGlu -> MatMul, src/Transformer.cs:288,241-251): x quantized once per
 * pass, the SwiGLU outputs of every (token, expert) pair quantized for down. */
int wl_set_int_dot(wl_ctx *ctx, int on);

/* The float arithmetic of ForwardBatch (src/Transformer.cs:127-170; MatMulEach, :544-561) on the
 * matrix cores, for an engine started with --batch N (EngineOptions.Batch, src/Engine.cs:21,65;
 * src/Program.cs:213). Off by default. When on, every float decode GEMV of Q4_K and Q6_K weights
 * (wl_matmul(_dev), the fused q/k/v and SwiGLU entries, the layer entries; 1-8 tokens per pass)
 * runs on fp16 MFMA with each token's x split exactly into two fp16 parts: results within the
 * float bar of the reference's DotRow, and a token's bits are the same whatever the number of
 * tokens in the call, so a batched sequence gets the bits it gets alone in the same mode. The
 * bits differ from the default (VALU) arithmetic's in the last places; switch it per context
 * before decoding, not between steps of one sequence. Other formats, the integer branch and
 * the MoE experts are unchanged. */
int wl_set_float_mma(wl_ctx *ctx, int on);

/* FastMath.Quantize (src/FastMath.cs:35-91) of x [T][cols], bit-identical: k = 0 gives Q8_0
 * activations (q int8 [T][cols], d [T][cols/32] rounded through fp16; bsums unused, may be
 * NULL), k = 1 Q8_K (d [T][cols/256], bsums int16 [T][cols/16], the sums of every 16 quants).
 * cols must be whole blocks. Synchronous. */
int wl_quantize(wl_ctx *ctx, const float *x, int32_t T, int32_t cols, int32_t k, int8_t *q, float *d,
                int16_t *bsums);

/* ---- device-pointer variants (activations resident in HBM), asynchronous ---------- */

/* wl_quantize on device buffers. */
int wl_quantize_dev(wl_ctx *ctx, const float *d_x, int32_t T, int32_t cols, int32_t k, int8_t *d_q,
                    float *d_d, int16_t *d_bsums);

/* wl_matmul on device buffers d_x [T][cols], d_y [T][rows]. */
int wl_matmul_dev(wl_ctx *ctx, const wl_weight *w, int32_t expert, const float *d_x, int32_t T,
                  float *d_y);

/* MatMul followed by Layer's residual add (src/Transformer.cs:224,231): d_y [T][rows] +=
 * (W x) * rs, the product rounded to float first and the add as two roundings, so the bits
 * equal wl_matmul_dev then wl_residual_dev. Up to 8 tokens the add is the GEMV's own store (no
 * extra launch). */
int wl_matmul_add_dev(wl_ctx *ctx, const wl_weight *w, int32_t expert, const float *d_x, int32_t T,
                      float *d_y, float rs);

/* Several matrices that read the same x in ONE launch (Layer's q, k and v,
 * src/Transformer.cs:186-188): d_ys[i] is [T][rows_i]. n <= 4; types may differ. */
int wl_matmul_multi_dev(wl_ctx *ctx, int32_t n, const wl_weight *const *ws, const float *d_x,
                        int32_t T, float *const *d_ys);

/* The SwiGLU gate/up half in one launch: d_h [T][ff] = silu(gate x) * (up x)
 * (src/Transformer.cs:245-247). gate and up must share a type. */
int wl_gate_up_dev(wl_ctx *ctx, const wl_weight *gate, const wl_weight *up, int32_t expert,
                   const float *d_x, int32_t T, float *d_h);

/* wl_dequant_f32 into a device buffer. */
int wl_dequant_dev(wl_ctx *ctx, const wl_weight *w, int64_t row0, int64_t nrows, float *d_dst);

/* How the MoE entries run (no counterpart in the reference, whose MoeFfn is one host loop):
 * on = 1 (the default) routes, plans, runs gate/up and down and combines in one launch where
 * the shapes allow it (Q4_K/Q6_K experts, hidden and FFN up to 2048, up to 64 token-expert
 * pairs per pass, up to 256 experts, float products); on = 0 always runs the launch chain
 * (route+plan, gate/up, down, combine). Both give the same bits. */
int wl_set_moe_one_launch(wl_ctx *ctx, int on);

/* Fault injection for the one-launch MoE's error path (no counterpart in the reference): the
 * polls each of its bounded waits makes before it gives up (sets the context's sticky status,
 * reported by the next wl_sync or wl_moe_ffn) and goes on. 0 gives up at once, so the status is
 * set on every such launch while every kernel still exits normally; polls < 0 restores the
 * default. */
int wl_debug_moe_patience(wl_ctx *ctx, int32_t polls);

/* wl_moe_ffn on device buffers (logits, x, out in HBM). Asynchronous: a one-launch failure is
 * reported by the next wl_sync. */
int wl_moe_ffn_dev(wl_ctx *ctx, const float *d_logits, int32_t k, int32_t renorm,
                   const wl_weight *gate_exps, const wl_weight *up_exps,
                   const wl_weight *down_exps, const float *d_x, int32_t T, float *d_out);

/* ---- The rest of a decoder layer on device-resident activations ----
 * Transformer.Layer's other operations (src/Transformer.cs:177-232), stream-ordered on the
 * context like the *_dev products, so a whole decode step runs with its activations in HBM.
 * Pointers are device memory. */

/* RmsNormRows (src/Transformer.cs:446-457): y[r] = x[r] / sqrt(mean(x[r]^2) + eps) * w, the sum
 * of squares in double; in place allowed. */
int wl_rms_norm_dev(wl_ctx *ctx, const float *d_x, int64_t rows, int64_t dim, const float *d_w, float eps,
                    float *d_y);

/* RopeTable + Rope (src/Transformer.cs:396-431) on T rows of `heads` heads, in place: the
 * first rope_dims values of each head rotate by the angles (pos * freq_scale) * base^(-2i/n),
 * each divided by d_freqs[i] when d_freqs (rope_freqs.weight, n/2 device floats) is given;
 * pairs (2i, 2i+1), or (i, i + n/2) when neox. Row t's position is d_pos[t], or pos0 + t when
 * d_pos is null. */
int wl_rope_dev(wl_ctx *ctx, float *d_x, int32_t T, int32_t heads, int32_t head_dim, int32_t rope_dims,
                int32_t neox, int32_t pos0, const int32_t *d_pos, double base, double freq_scale,
                const float *d_freqs);

/* ToHalf (src/Transformer.cs:342-348): rows pos0..pos0+T-1 of the fp16 K and V caches. */
int wl_kv_store_dev(wl_ctx *ctx, const float *d_k, const float *d_v, int32_t T, int32_t kv_dim, uint16_t *d_K,
                    uint16_t *d_V, int32_t pos0);

/* Attention (src/Transformer.cs:351-393): row t attends to positions 0..pos0+t of the fp16
 * caches; softmax with exp and the denominator in double; grouped KV heads. */
int wl_attention_dev(wl_ctx *ctx, const float *d_q, int32_t T, int32_t heads, int32_t kv_heads, int32_t head_dim,
                     const uint16_t *d_K, const uint16_t *d_V, int32_t pos0, float scale, float *d_out);

/* The residual add of Layer (src/Transformer.cs:224,231): x += o * rs. */
int wl_residual_dev(wl_ctx *ctx, float *d_x, const float *d_o, int64_t n, float rs);

/* Greedy sampling (src/Engine.cs:356-360): the first index of each row's largest logit. */
int wl_argmax_dev(wl_ctx *ctx, const float *d_logits, int32_t rows, int64_t n, int32_t *d_out);

/* LayerStream.EmbedRow (src/LayerStream.cs:238-257): the decoded embedding rows of T tokens
 * (token ids on the host) into d_x [T][cols]. */
int wl_embed_dev(wl_ctx *ctx, const wl_weight *embd, const int32_t *tokens, int32_t T, float *d_x);

/* wl_embed_dev with the token ids in device memory (d_tokens [T], e.g. wl_argmax_dev's output),
 * so a decode loop feeds each sampled token to the next step without a host round trip. The ids
 * cannot be checked on the host: an id outside the vocabulary gives a row of zeros. */
int wl_embed_dev_ids(wl_ctx *ctx, const wl_weight *embd, const int32_t *d_tokens, int32_t T, float *d_x);

/* One decoder layer: the weights and vectors Transformer.Layer reads from its stage
 * (src/Transformer.cs:177-232) and the model constants it uses (ModelConfig). Vectors are
 * device fp32 arrays; the optional ones are null when the architecture has none (biases: qwen2;
 * q/k norms per head: qwen3; RoPE frequency factors: rope_freqs.weight of Llama 3.1 and later,
 * shared by every layer, src/Transformer.cs:37). Zero scales mean the defaults (1/sqrt(head_dim),
 * 1). */
typedef struct wl_layer_desc {
  const wl_weight *attn_q, *attn_k, *attn_v, *attn_output, *ffn_gate, *ffn_up, *ffn_down;
  const float *d_attn_norm, *d_ffn_norm;
  const float *d_q_bias, *d_k_bias, *d_v_bias;
  const float *d_q_norm, *d_k_norm, *d_rope_freqs;
  int32_t embd, heads, kv_heads, head_dim, rope_dims, neox;
  double rope_base, rope_freq_scale;
  float eps, attention_scale, residual_scale;
  /* MoeFfn (src/Transformer.cs:229,259-311) when ffn_gate_inp (the router, [n_expert][embd]) is
   * set: ffn_gate / ffn_up / ffn_down are then the stacked experts, expert_used of them chosen
   * per token (weights renormalised when expert_weights_norm). The shared expert
   * (ffn_*_shexp, qwen2moe) is optional, and so is its gate ffn_gate_inp_shexp ([1][embd]):
   * without it the shared expert's weight is 1. NULL ffn_gate_inp: the dense SwiGLU FFN. */
  const wl_weight *ffn_gate_inp, *ffn_gate_shexp, *ffn_up_shexp, *ffn_down_shexp, *ffn_gate_inp_shexp;
  int32_t expert_used, expert_weights_norm;
  /* OLMo 2's post-norms (ModelConfig.PostNorms, src/Transformer.cs:182,224-230): when both are
   * set there are no pre-norms (d_attn_norm / d_ffn_norm are not read: q/k/v and the FFN read x
   * itself), and each branch's output is RMS-normed with these before its residual add. */
  const float *d_post_attention_norm, *d_post_ffw_norm;
  /* ModelConfig.QkNormFull (OLMo 2, :192-196): d_q_norm / d_k_norm cover the whole q and k rows
   * (heads * head_dim, kv_heads * head_dim values) instead of one head. */
  int32_t qk_norm_full;
} wl_layer_desc;

/* x[i] *= s for n floats of device memory, in place, stream-ordered: Granite's embedding scale
 * on the embedding rows (src/Transformer.cs:94,150) and its logit scale, as the reciprocal
 * 1f / LogitScale, on the logits (:123). */
int wl_scale_dev(wl_ctx *ctx, float *d_x, int64_t n, float s);

/* Transformer.Layer (src/Transformer.cs:177-232) for T tokens at positions pos0.. of one
 * sequence: x [T][embd] (device) is updated in place and the tokens' keys and values go to
 * rows pos0.. of the fp16 caches d_K / d_V [positions][kv_heads * head_dim]. Every activation
 * stays in HBM (the context's scratch); stream-ordered, no host wait. Up to 8 tokens the
 * products are the decode GEMVs (o and down add into x in their own store); more tokens take
 * the GEMMs. The caches must hold pos0 + T positions: the library cannot check their size.
 * Like the reference's RopeTable (src/Transformer.cs:396-414) the context keeps the RoPE angles
 * of the positions it has seen, for the last setting (rope dims, base, frequency scale,
 * rope_freqs pointer); each entry records the frequency factors it was made with, and an entry
 * whose factors no longer match the tensor's values is computed again. */
int wl_layer_dev(wl_ctx *ctx, const wl_layer_desc *layer, float *d_x, int32_t T, int32_t pos0, uint16_t *d_K,
                 uint16_t *d_V);

/* Transformer.ForwardBatch's layer (src/Transformer.cs:127-170): N rows, row i the next token
 * of its own sequence, at position pos[i] of cache slot slot[i] (host arrays, checked: slots
 * distinct and below `slots`, positions below slot_positions). d_K / d_V are this layer's pools
 * [slots][slot_positions][kv_heads * head_dim]. Every product runs the GEMV in passes of at most
 * 8 rows (EachToken), so row i's bits equal wl_layer_dev of that token alone on its sequence. */
int wl_layer_batch_dev(wl_ctx *ctx, const wl_layer_desc *layer, float *d_x, int32_t N, const int32_t *pos,
                       const int32_t *slot, int32_t slots, int32_t slot_positions, uint16_t *d_K, uint16_t *d_V);

/* ---- Allocation-free product (no counterpart in the reference) ----
 * For callers that cannot allocate device memory: code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc. The same operation and results as wl_matmul_dev (bit
 * for bit: the same kernels), but every kernel's scratch is a static per-GPU array of 32 MiB that
 * the library resolves in wl_create, so the call allocates nothing. A call that would need more
 * scratch than that (large GEMMs: T > 8 with T * cols * 2 bytes of bf16 activations near 32 MiB)
 * returns WL_E_SHAPE before anything is launched. Calls on one GPU share the array: calls that
 * overlap (other streams, other contexts, other host threads) race. */
int wl_matmul_dev_noalloc(wl_ctx *ctx, const wl_weight *w, int32_t expert, const float *d_x, int32_t T,
                          float *d_y);

/* ---- Replayed step (no counterpart in the reference; it serves the per-token loop of
 * src/Engine.cs:198-203, one Model.Forward per generated token) ----
 * wl_capture_begin starts recording the context's stream; every _dev call until wl_capture_end
 * is recorded, not run, and wl_capture_end returns the recording as one graph. wl_graph_launch
 * replays it on the context's stream: the same kernels with the same arguments (the same device
 * buffers, the same weights), enqueued by one host call. A call that would grow the context's
 * scratch during a capture fails with WL_E_ARG (run the same calls once before capturing), and
 * the MoE entries take their launch chain while capturing (the same bits as one launch).
 * Host-buffer entries synchronise and must not be called while capturing. */
typedef struct wl_graph wl_graph;
int wl_capture_begin(wl_ctx *ctx);
int wl_capture_end(wl_ctx *ctx, wl_graph **out);
int wl_graph_launch(wl_ctx *ctx, const wl_graph *g);
int wl_graph_free(wl_graph *g);

/* ---- Calibration (no counterpart in the reference) ----
 * A plain streaming read of `bytes` (a multiple of 16) of device memory at d_src by `workgroups`
 * workgroups of 256 threads (0: eight per CU), each over one contiguous chunk with nontemporal
 * 16-byte loads, stream-ordered on the context. It only loads; the
 * rate it reaches is the HBM read ceiling the decode GEMVs' roofline fractions are set against.
 * d_out (one uint32, device) is written only in a case real data does not produce. */
int wl_read_peak_dev(wl_ctx *ctx, const void *d_src, int64_t bytes, int32_t workgroups, uint32_t *d_out);

#ifdef __cplusplus
}
#endif
#endif
