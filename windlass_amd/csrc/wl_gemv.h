// wl_gemv.h - host-side interface of the decode GEMV launches.
#pragma once
#include "wl_codecs.h"

namespace wl {

constexpr int GEMV_MAX_MATS = 4;   // matrices that share x in one launch (q, k, v)
constexpr int GEMV_MAX_SEGS = 16;  // (matrix, K-chunk) segments of one launch

// One matrix of a launch: y[t * ldy + r] = W[r] . x[t] (nm = 2: silu(W x) * (W2 x)); with add,
// y[t * ldy + r] += (W[r] . x[t]) * rs instead (the residual add, rounded as two operations).
struct GemvMat {
  const uint8_t *w;
  const uint8_t *w2;
  int64_t row_bytes;
  int rows;
  int type;
  float *y;
  int ldy;
  int add = 0;
  float rs = 1.f;
};

// One segment: a K-chunk [col0, col0 + cols) of one matrix, written to out (the result, or a
// partial the combine kernel adds when the row is split).
struct GemvSeg {
  const uint8_t *w;
  const uint8_t *w2;
  int64_t row_bytes;
  float *out;
  int64_t ldo;
  int rows;
  int col0;
  int type;
  int wg_begin;
  int nwg;
  int add;  // out += result * rs (unsplit segments only)
  float rs;
};

struct GemvParams {
  GemvSeg seg[GEMV_MAX_SEGS];
  int nseg;
  int ileave;  // the segments' workgroups interleaved in runs of 8 (set by the launch's grid plan)
  int cols;  // columns of every segment
  const float *x;
  int ldx;
  int T;
};

bool gemv_supports(int type);
bool gemv_mixed_supports(int type);

// K-chunks a row of `cols` values is split into when nmat matrices share a launch (1: no split).
int gemv_chunks(int nmat, int cols);
// Scratch floats a launch needs for partials (0 without a split).
int64_t gemv_scratch_floats(const GemvMat *mats, int nmat, int nm, int cols, int T);

// y = W x for nmat matrices sharing x [T][ldx] (T <= 8), in one launch (plus one combine
// launch when rows are split along K). Types may differ only among Q4_K / Q6_K / Q8_0.
// scratch holds gemv_scratch_floats(...) floats. num_cu sizes the grid.
hipError_t gemv_run(const GemvMat *mats, int nmat, int nm, const float *x, int ldx, int cols, int T,
                    float *scratch, int num_cu, hipStream_t st);

}  // namespace wl
