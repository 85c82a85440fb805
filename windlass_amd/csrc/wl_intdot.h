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
};
int64_t qacts_bytes(int T, int cols, int k);
QActsDev qacts_at(void *buf, int T, int cols, int k);

// FastMath.Quantize (src/FastMath.cs:35-91) of x [T][cols]: k = 0 Q8_0 (blocks of 32, d rounded
// through fp16), k = 1 Q8_K (blocks of 256, float d, sums of every 16 quants). Bit-identical.
hipError_t quantize_launch(const float *x, int T, int cols, int k, QActsDev a, hipStream_t st);

// Floats of scratch one intdot_launch needs for its per-block terms (T <= 8 tokens).
int64_t intdot_terms_floats(int type, int rows, int cols, int T);

// y[t * ldy + r] = FastMath.IntDot(W[r], the activations of token t) (src/FastMath.cs:105-214)
// for T <= 8 tokens whose activations start at a (token 0). Bit-identical to the reference: each
// block's integer sums are exact, its float term is formed with the reference's operations,
// and a row's terms are added in block order by a second launch.
hipError_t intdot_launch(int type, const uint8_t *w, int64_t row_bytes, int rows, int cols, QActsDev a, int T,
                         float *terms, float *y, int ldy, int num_cu, hipStream_t st);

// h[i] = silu(g[i]) * u[i] (SwiGlu's elementwise step, src/Transformer.cs:247), in place on g.
hipError_t silu_mul_launch(float *g, const float *u, int64_t n, hipStream_t st);

}  // namespace wl
