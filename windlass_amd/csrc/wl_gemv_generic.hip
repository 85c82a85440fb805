// wl_gemv_generic.hip - the decode GEMV of formats without a lane codec (IQ3_S, IQ2_S): the
// exact block decoders of wl_blocks.h, one wave per row. Lane i decodes the row's 16-value runs
// i, i + 64, ... and adds run by run into one fp32 sum per token (a run's 16 products in order),
// then a fixed shuffle tree adds the 64 lane sums. A token's sum does not depend on how many
// tokens share the launch, so up to 8 tokens per launch keep MatMulEach's per-token bits.
#include "wl_blocks.h"
#include "wl_gemv.h"
#include "wl_gemv_impl.h"

#pragma clang fp contract(off)

namespace wl {

struct GenericMat {
  const uint8_t *w, *w2;  // w2: the SwiGLU pair's up matrix (nm = 2)
  int64_t row_bytes;
  float *y;
  int ldy, rows, add;
  float rs;
};

template <class B, int NM>
__global__ __launch_bounds__(256) void gemv_generic_kernel(GenericMat m, const float *__restrict__ x, int ldx, int cols,
                                                           int T) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= m.rows) return;  // whole waves: no barrier below
  float acc[NM][8];
#pragma unroll
  for (int a = 0; a < NM; a++)
#pragma unroll
    for (int t = 0; t < 8; t++) acc[a][t] = 0.f;
  const int runs = cols / 16;
  for (int r = lane; r < runs; r += 64) {
    const int k = 16 * r;
#pragma unroll
    for (int a = 0; a < NM; a++) {
      const uint8_t *blk = (a ? m.w2 : m.w) + (int64_t)row * m.row_bytes + (int64_t)(k / B::BLOCK) * B::BYTES;
      typename B::Raw raw;
      B::load(blk, k % B::BLOCK, raw);
      float v[16];
      B::dec(raw, k % B::BLOCK, v);
#pragma unroll
      for (int t = 0; t < 8; t++) {
        if (t < T) {
          const float *xt = x + (int64_t)t * ldx + k;
          float s = 0.f;
#pragma unroll
          for (int j = 0; j < 16; j++) s += v[j] * xt[j];
          acc[a][t] += s;
        }
      }
    }
  }
#pragma unroll
  for (int a = 0; a < NM; a++)
#pragma unroll
    for (int t = 0; t < 8; t++)
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) acc[a][t] += __shfl_xor(acc[a][t], o, 64);
  if (lane == 0) {
    for (int t = 0; t < T; t++) {
      float s = acc[0][t];
      if constexpr (NM == 2) s = silu_mul(s, acc[1][t]);
      float *y = m.y + (int64_t)t * m.ldy + row;
      *y = m.add ? add_scaled(*y, s, m.rs) : s;
    }
  }
}

template <class B>
static hipError_t launch_generic(const GenericMat &m, int nm, const float *x, int ldx, int cols, int T, hipStream_t st) {
  const dim3 grid((unsigned)((m.rows + 3) / 4));
  if (nm == 2)
    hipLaunchKernelGGL((gemv_generic_kernel<B, 2>), grid, dim3(256), 0, st, m, x, ldx, cols, T);
  else
    hipLaunchKernelGGL((gemv_generic_kernel<B, 1>), grid, dim3(256), 0, st, m, x, ldx, cols, T);
  return hipGetLastError();
}

bool gemv_generic_supports(int type) { return type == 21 || type == 22; }

hipError_t gemv_generic_run(const GemvMat *mats, int nmat, int nm, const float *x, int ldx, int cols, int T,
                            hipStream_t st) {
  if (T < 1 || T > 8 || cols % 256) return hipErrorInvalidValue;
  for (int i = 0; i < nmat; i++) {
    const GemvMat &g = mats[i];
    const GenericMat m{g.w, g.w2, g.row_bytes, g.y, g.ldy, g.rows, g.add, g.rs};
    hipError_t e = hipErrorInvalidValue;
    if (g.type == 21) e = launch_generic<BIQ3S>(m, nm, x, ldx, cols, T, st);
    if (g.type == 22) e = launch_generic<BIQ2S>(m, nm, x, ldx, cols, T, st);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace wl
