// wl_intdot.h - host interface of the integer-dot path: 8-bit activations (FastMath.Quantize)
// and integer dot products against the raw weight blocks (FastMath.IntDot).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wl {

// FastMath.CanIntDot (src/FastMath.cs:27-30) for this build's formats: Q8_0, Q4_K, Q6_K.
bool intdot_supports(int type);
// FastMath.NeedsK (src/FastMath.cs:32): the weights take Q8_K activations (256-wide, bsums).
bool intdot_needs_k(int type);
// FastMath.Fits (src/FastMath.cs:34): whole activation blocks per row.
bool intdot_fits(int type, int cols);

// The activations of T rows (FastMath.QActs, src/FastMath.cs:17-23) in one buffer:
// q int8 [T][cols], then d float [T][cols / block], then (Q8_K only) bsums int16 [T][cols / 16].
struct QActsDev {
  int8_t *q;
  float *d;
  int16_t *bsums;
  // Q8_K of at most 8 tokens, also in the matrix-core kernel's operand order (16 token slots,
  // slots past T zero): per 256-block b, qf[b][run s][slot t][32 quants] and df[b][t]; so one
  // wave load of a run's B operand reads 512 contiguous bytes. Null otherwise.
  int8_t *qf;
  float *df;
};
int64_t qacts_bytes(int T, int cols, int k);
QActsDev qacts_at(void *buf, int T, int cols, int k);

// FastMath.Quantize (src/FastMath.cs:35-91) of x [T][cols]: k = 0 Q8_0 (blocks of 32, d rounded
// through fp16), k = 1 Q8_K (blocks of 256, float d, sums of every 16 quants). Bit-identical.
hipError_t quantize_launch(const float *x, int T, int cols, int k, QActsDev a, hipStream_t st);

// Tokens one launch can take for a row of `cols` (the larger of the matrix-core kernel's and of
// as many as the VALU kernel's staged terms fit the workgroup's LDS); nm = 2 for the SwiGLU pair.
// 0 when not even one fits.
int intdot_max_tokens(int type, int cols, int nm);

// y[t * ldy + r] = FastMath.IntDot(W[r], the activations of token t) (src/FastMath.cs:105-214)
// for T <= intdot_max_tokens tokens whose activations start at a (token 0). Bit-identical to
// the reference: each block's integer sums are exact, its float term is formed with the
// reference's operations, and a row's terms are added in block order.
hipError_t intdot_launch(int type, const uint8_t *w, int64_t row_bytes, int rows, int cols, QActsDev a, int T,
                         float *y, int ldy, int num_cu, hipStream_t st);

// The int8 matrix-core kernel (wl_intmma.hip) for 2..8 tokens of Q4_K or Q6_K: the same
// results as intdot_launch, bit for bit (exact integer sums, the reference's float terms added
// in block order). w2 non-null: the SwiGLU pair (nm = 2), y = silu(gate) * up.
bool intmma_supports(int type, int cols, int T, int nm);
int intmma_max_tokens(int type, int cols, int nm);  // 0 when the kernel does not take the rows
hipError_t intmma_launch(int type, const uint8_t *w, const uint8_t *w2, int64_t row_bytes, int rows, int cols,
                         QActsDev qa, int T, float *y, int ldy, hipStream_t st);
// Up to three matrices of `cols` columns that read the same activations, in one launch (each
// result as intmma_launch gives it).
struct MmaMat {
  const uint8_t *w;
  int64_t row_bytes;
  int rows, type;
  float *y;
  int ldy;
};
bool intmma_multi_supports(const int *types, int n, int cols, int T);
hipError_t intmma_multi_launch(const MmaMat *mats, int n, int cols, QActsDev qa, int T, hipStream_t st);

struct MoePlan;
// The integer products of routed experts (MoeFfn's SwiGlu under IntDot, src/Transformer.cs:
// 288,241-251,504-524), one launch for every slot of the plan: slot s multiplies expert
// slot_expert[s] of the stacked tensors (estride bytes apart) with its tokens' activations
// (rows slot_pair of qa when x_by_pair, else slot_tok) into rows slot_pair of y. T: the most
// tokens a slot may hold (<= 8); slots: the most slots the plan may use. Each (row, token) is
// FastMath.IntDot's bits, as for intdot_launch. w2 non-null: y = silu(gate) * up.
hipError_t intdot_moe_launch(int type, const uint8_t *w, const uint8_t *w2, int64_t row_bytes, int64_t estride,
                             int rows, int cols, QActsDev qa, const MoePlan *plan, int x_by_pair, int T, int slots,
                             float *y, int ldy, int num_cu, hipStream_t st);

// SwiGlu's gate/up half on the integer kernels, one launch: y = silu(IntDot(gate)) * IntDot(up)
// per (row, token) (src/Transformer.cs:245-247), both products on the same activations a.
hipError_t intdot_swiglu_launch(int type, const uint8_t *wg, const uint8_t *wu, int64_t row_bytes, int rows,
                                int cols, QActsDev a, int T, float *y, int ldy, int num_cu, hipStream_t st);

}  // namespace wl
