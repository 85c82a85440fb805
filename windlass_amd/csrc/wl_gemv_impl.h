// wl_gemv_impl.h - the wave-level decode GEMV body shared by the dense and the MoE launches.
#pragma once
#include "wl_codecs.h"

namespace wl {

// SiLU(g) * u as src/Transformer.cs:247 writes it: g / (1 + exp(-g)) * u, the exponential in
// double (Math.Exp) cast to float. Compiled without contraction by every includer.
__device__ __forceinline__ float silu_mul(float g, float u) {
  return g / (1.0f + (float)exp((double)(-g))) * u;
}

// Rows row0..row0+R-1 of w (and of w2 when NM == 2) times T <= TM activation rows.
//   x row of token t:  x + (xrow ? xrow[t] : t) * ldx
//   y of (token t, row r): y[(yrow ? yrow[t] : t) * ldy + r]
// NM == 2 stores silu(w x) * (w2 x) instead (the SwiGLU gate/up pair).
template <class C, int TM, int R, int NM>
__device__ __forceinline__ void gemv_rows(const uint8_t *__restrict__ w, const uint8_t *__restrict__ w2,
                                          int64_t row_bytes, int rows, int row0,
                                          const float *__restrict__ x, const int *xrow, int64_t ldx,
                                          int cols, int T, float *__restrict__ y, const int *yrow,
                                          int64_t ldy, const Lds &lds) {
  const int lane = threadIdx.x & 63;
  const int sub = lane % C::LPB;
  const int bslot = lane / C::LPB;
  constexpr int BPW = 64 / C::LPB;
  const int nb = cols / C::BLOCK;
  const uint8_t *wm[2] = {w, w2};

  const float *xr[TM];
#pragma unroll
  for (int t = 0; t < TM; t++) xr[t] = x + (int64_t)(xrow ? xrow[t < T ? t : 0] : t) * ldx;

  // Rows past the end re-read the last row (valid memory); their results are dropped.
  int64_t roff[R];
#pragma unroll
  for (int r = 0; r < R; r++) roff[r] = (int64_t)min(row0 + r, rows - 1) * row_bytes;

  float acc[NM][R][TM];
#pragma unroll
  for (int m = 0; m < NM; m++)
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
      for (int t = 0; t < TM; t++) acc[m][r][t] = 0.f;

  for (int b = bslot; b < nb; b += BPW) {
    typename C::W wr[NM][R];
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
      for (int r = 0; r < R; r++) C::decode(wm[m] + roff[r] + (int64_t)b * C::BYTES, sub, lds, wr[m][r]);
#pragma unroll
    for (int t = 0; t < TM; t++) {
      if (t < T) {
        typename C::Xs xs;
        C::load_x(xr[t] + (int64_t)b * C::BLOCK, sub, xs);
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
          for (int r = 0; r < R; r++) acc[m][r][t] += C::dot(wr[m][r], xs);
      }
    }
  }

#pragma unroll
  for (int r = 0; r < R; r++) {
#pragma unroll
    for (int t = 0; t < TM; t++) {
      if (t < T) {
        float v = wave_sum(acc[0][r][t]);
        if (NM == 2) v = silu_mul(v, wave_sum(acc[NM - 1][r][t]));
        if (lane == 0 && row0 + r < rows) y[(int64_t)(yrow ? yrow[t] : t) * ldy + row0 + r] = v;
      }
    }
  }
}

}  // namespace wl
