/*
 * wl_oracle.h - CPU restatement of Windlass's quantized-matmul arithmetic.
 *
 * TEST INFRASTRUCTURE. This is the oracle: only the tests, the smoke check and the
 * benchmark's CPU-baseline leg load it, and only as the checker or as the timed CPU
 * baseline. The product library (windlass_amd/libwindlass_hip.so) never links it.
 *
 * Every function restates one reference function; the citation is on the declaration.
 * Compiled with -O2 -fno-tree-vectorize -ffp-contract=off and no fast-math, so each
 * float operation rounds separately, in the order the reference C# writes it
 * (RyuJIT x64 scalar SSE semantics).
 */
#ifndef WL_ORACLE_H
#define WL_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (src/Gguf.cs:19-25). Only the ones this path decodes are named. */
enum {
    WLO_F32 = 0, WLO_F16 = 1, WLO_Q4_0 = 2, WLO_Q4_1 = 3, WLO_Q5_0 = 6, WLO_Q5_1 = 7,
    WLO_Q8_0 = 8, WLO_Q2_K = 10, WLO_Q3_K = 11, WLO_Q4_K = 12, WLO_Q5_K = 13, WLO_Q6_K = 14,
    WLO_IQ2_XXS = 16, WLO_IQ4_NL = 20, WLO_IQ3_S = 21, WLO_IQ2_S = 22, WLO_IQ4_XS = 23, WLO_BF16 = 30
};

/* fp16 -> fp32, exact incl. subnormals, Inf and NaN payloads (src/Half.cs:59-90). */
float wlo_half_to_float(uint16_t h);
/* fp32 -> fp16, round to nearest even, overflow to Inf (src/Half.cs:29-57). */
uint16_t wlo_half_from_float(float f);
/* Table[FromFloat(f)] (src/Half.cs:24-27). */
float wlo_half_round(float f);
void wlo_half_to_float_n(const uint16_t *h, int64_t n, float *out);
void wlo_half_from_float_n(const float *f, int64_t n, uint16_t *out);

/* xorshift64* Rng of tests/TinyModels.cs:89-97. The state is one uint64.
 * Parity unpinned: the reference's tests hold no vector of this stream, and Normal() uses
 * libm log/cos/sqrt where the reference uses .NET Math. It only generates seeded test data;
 * every check reads the same generated data on both of its sides. */
void wlo_rng_init(uint64_t *state, uint64_t seed);
uint64_t wlo_rng_next(uint64_t *state);
void wlo_rng_bytes(uint64_t *state, int64_t n, uint8_t *out);      /* Rng.Byte() n times */
void wlo_rng_uniforms(uint64_t *state, int64_t n, double *out);    /* Rng.Uniform() */
void wlo_rng_normals(uint64_t *state, int64_t n, float *out);      /* Rng.Normal() (libm) */

/* Block geometry (src/Gguf.cs:30-66). Returns 1 when known. */
int wlo_layout(int type, int *block_elems, int *block_bytes);
/* Quants.CanDecode / CanDot restricted to this path's types (src/Quants.cs:11-21,56-65). */
int wlo_can_decode(int type);
int wlo_can_dot(int type);

/* Quants.DecodeRow / IQuants.DecodeRow (src/Quants.cs:32-52; src/IQuants.cs:27-42).
 * Returns 0, or -1 for an unsupported type. */
int wlo_decode_row(int type, const uint8_t *src, int64_t n, float *dst);
/* Quants.DotRow (src/Quants.cs:67-187). Returns 0, or -1 when the type has no fused dot. */
int wlo_dot_row(int type, const uint8_t *b, const float *x, int n, float *out);
/* FastMath.Block (src/FastMath.cs:216-264). */
void wlo_block(const float *w, int ws, int nr, const float *x, int xs, int nt, int cols,
               float *y, int ystride);
/* Transformer.MatMul (src/Transformer.cs:479-537) and MatMulEach (:539-561).
 * each_token selects the ForwardBatch behaviour (src/Transformer.cs:488).
 * threads <= 0 means every core. Returns 0, -1 unsupported type. */
int wlo_matmul(int type, const uint8_t *data, int rows, int cols, int64_t row_bytes,
               const float *x, int T, float *y, int each_token, int threads);
/* mode for wlo_swiglu / wlo_moe_ffn: bit 0 EachToken (src/Transformer.cs:488), bit 1 IntDot
 * (src/Transformer.cs:23): each product of a FastMath.CanIntDot type whose rows are whole
 * activation blocks takes MatMul's integer branch (wlo_int_matmul). */
#define WLO_EACH_TOKEN 1
#define WLO_INT_DOT 2
/* SwiGlu (src/Transformer.cs:241-251): out = down(silu(gate x) * (up x)); each_token is the
 * mode above. */
int wlo_swiglu(int gtype, const uint8_t *gate, int64_t g_row_bytes,
               int utype, const uint8_t *up, int64_t u_row_bytes,
               int dtype, const uint8_t *down, int64_t d_row_bytes,
               int ff, int embd, const float *x, int T, float *out, int each_token, int threads);
/* Route (src/Transformer.cs:313-340) for one token. */
void wlo_route(const float *logits, int n, int k, int renorm, int *sel, float *wts, int *count);
/* MoeFfn (src/Transformer.cs:253-294) given the router logits [T][n_expert].
 * Stacked expert tensors: gate/up [n_expert][ff][embd], down [n_expert][embd][ff]
 * (WeightView.Slice, src/LayerStream.cs:26-34). */
int wlo_moe_ffn(const float *logits, int n_expert, int k, int renorm,
                int gtype, const uint8_t *gate, int utype, const uint8_t *up,
                int dtype, const uint8_t *down, int ff, int embd,
                const float *x, int T, float *out, int each_token, int threads,
                int *expert_runs);

/* TinyModels.Matrix (tests/TinyModels.cs:342-381): random block bytes whose scale fields
 * are then set so the decoded RMS is about rms. out holds rows*cols/block*bytes bytes.
 * Parity unpinned (the scale fields depend on Rng.Normal, above); test data only. */
int wlo_matrix(uint64_t *rng_state, int type, int rows, int cols, float rms, uint8_t *out);

/* FastMath.Quantize (src/FastMath.cs:35-91) for one activation row.
 * k = 0: Q8_0 layout (blocks of 32, fp16-rounded d); k = 1: Q8_K (256, float d, bsums). */
void wlo_quantize_row(const float *x, int cols, int k, int8_t *q, float *d, int16_t *bsums);
/* FastMath.IntDot (src/FastMath.cs:105-214) for Q8_0 / Q4_K / Q6_K weights. */
int wlo_int_dot(int type, const uint8_t *b, const int8_t *q, const float *d,
                const int16_t *bsums, int n, float *out);
/* FastMath.CanIntDot / NeedsK / Fits (src/FastMath.cs:27-34). */
int wlo_can_int_dot(int type);
int wlo_int_fits(int type, int cols);
/* Transformer.MatMul's integer branch (src/Transformer.cs:504-524): each of the T rows of x
 * quantized (FastMath.Quantize, Q8_K for the K-quants), then y[t][r] = FastMath.IntDot. Returns
 * 0, -1 when the type has no integer dot or the rows are not whole activation blocks. */
int wlo_int_matmul(int type, const uint8_t *data, int rows, int cols, int64_t row_bytes,
                   const float *x, int T, float *y, int threads);

/* Table data of src/IqTables.cs:9-57 (kmask, ksigns, kvalues, iq2xxs grid). */
const uint64_t *wlo_iq2xxs_grid(void);
const uint64_t *wlo_iq2s_grid(void);
const uint32_t *wlo_iq3s_grid(void);
const uint8_t *wlo_ksigns_iq2xs(void);
const int8_t *wlo_kvalues_iq4nl(void);

#ifdef __cplusplus
}
#endif
#endif
