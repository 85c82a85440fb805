// wl_gemv.h - host-side interface of the decode GEMV launches.
#pragma once
#include "wl_codecs.h"

namespace wl {

constexpr int GEMV_MAX_SEGS = 4;

// One matrix of a launch: rows [0, rows) of w (and of w2 when two matrices share the rows),
// results to y[t * ldy + r].
struct GemvSeg {
  const uint8_t *w;
  const uint8_t *w2;
  int64_t row_bytes;
  float *y;
  int rows;
  int ldy;
  int wg_begin;  // first workgroup of this segment (set by the launcher)
  int nwg;       // workgroups of this segment (set by the launcher)
  int type;
};

struct GemvParams {
  GemvSeg seg[GEMV_MAX_SEGS];
  int nseg;
  const float *x;  // [T][ldx]
  int ldx;
  int cols;
  int T;
};

bool gemv_supports(int type);
bool gemv_mixed_supports(int type);
// nm = 1: y = W x. nm = 2: y = silu(W x) * (W2 x) (the SwiGLU gate/up pair). num_cu sizes
// the grid (a few waves per SIMD across the device).
hipError_t gemv_launch(int type, int nm, GemvParams &p, int num_cu, hipStream_t st);
hipError_t gemv_launch_mixed(GemvParams &p, int num_cu, hipStream_t st);
// Waves per workgroup for a row of `cols` values.
int gemv_waves(int cols);

}  // namespace wl
