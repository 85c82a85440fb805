// wl_gemv.hip - decode GEMV for raw GGUF blocks (batch 1..8), bandwidth-bound, no MFMA.
//
// Replaces the CPU path's Transformer.MatMul T==1 branch (src/Transformer.cs:494-502, one
// Quants.DotRow per row) and MatMulEach (:544-561, one DotRow per (row, token)), plus the
// decode-then-Block path the I-quants take (:526-536). The kernel body is cs_gemv
// (wl_gemv_impl.h): column-stationary lanes, each weight byte read once per launch.
//
// Rows wider than four wave-columns (8192 values) are cut along K into equal chunks of 2-4
// wave-columns; every chunk is a segment of the same launch whose lanes keep their x slices in
// registers, the chunks' partial sums go to scratch, and a combine launch adds them in chunk
// order: y = ((chunk 0 + chunk 1) + chunk 2) + ... The cut depends only on the row length and
// the number of matrices, so a token's bits do not depend on how many tokens share the launch.
#include "wl_gemv_launch.h"

extern "C" int wl_type_layout(int ggml_type, int *block_elems, int *block_bytes);

namespace wl {

// Rows per group of the mixed kernel's codecs.
static int mixed_rows_per_group(int type, int tm) {
  if (tm > 1) return 4;
  return type == 12 ? Q4K::R1 : type == 14 ? Q6K::R1 : Q80::R1;
}

// Segments of different formats in one launch (q/k Q4_K with v Q6_K): the codec is chosen
// per workgroup; every segment's workgroups stay on that segment.
template <int TM, int SP>
__global__ __launch_bounds__(64 * kMaxWaves) void gemv_mixed_kernel(GemvParams p, int split) {
  const GemvSeg &s = p.seg[find_seg(p)];
  switch (s.type) {
    case 12: run_seg<Q4K, TM, rows_per_group<Q4K, TM, 1>(), 1, SP>(p, s, split); break;
    case 14: run_seg<Q6K, TM, rows_per_group<Q6K, TM, 1>(), 1, SP>(p, s, split); break;
    case 8: run_seg<Q80, TM, rows_per_group<Q80, TM, 1>(), 1, SP>(p, s, split); break;
    default: break;
  }
}

// y = the chunk partials added in chunk order (SwiGLU pair: silu(gate sum) * (up sum)).
struct CombineParams {
  const float *part[GEMV_MAX_MATS];  // per matrix: [S][NM][T][rows]
  float *y[GEMV_MAX_MATS];
  int ldy[GEMV_MAX_MATS];
  int rows[GEMV_MAX_MATS];
  int add[GEMV_MAX_MATS];  // y += result * rs
  float rs[GEMV_MAX_MATS];
  int S, NM, T;
};

__global__ __launch_bounds__(256) void combine_kernel(CombineParams cp) {
  const int m = blockIdx.y;
  const int rows = cp.rows[m];
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)cp.T * rows) return;
  const int t = (int)(i / rows), r = (int)(i % rows);
  const int64_t plane = (int64_t)cp.T * rows;
  const float *p = cp.part[m] + (int64_t)t * rows + r;
  // every chunk's partial is loaded before the in-order sum, so the loads overlap
  float pg[GEMV_MAX_SEGS], pu[GEMV_MAX_SEGS];
#pragma unroll
  for (int c = 0; c < GEMV_MAX_SEGS; c++) {
    pg[c] = c < cp.S ? p[(int64_t)c * cp.NM * plane] : 0.f;
    pu[c] = c < cp.S && cp.NM == 2 ? p[(int64_t)c * 2 * plane + plane] : 0.f;
  }
  float g = pg[0], u = pu[0];
#pragma unroll
  for (int c = 1; c < GEMV_MAX_SEGS; c++) {
    if (c < cp.S) {
      g += pg[c];
      u += pu[c];
    }
  }
  if (cp.NM == 2) g = silu_mul(g, u);
  float *y = cp.y[m] + (int64_t)t * cp.ldy[m] + r;
  *y = cp.add[m] ? add_scaled(*y, g, cp.rs[m]) : g;
}

int gemv_chunks(int nmat, int cols) {
  if (cols % kColsPerWave) return 1;
  const int u = cols / kColsPerWave;
  if (u <= 4) return 1;
  for (int w = 4; w >= 2; w--)
    if (u % w == 0) return nmat * (u / w) <= GEMV_MAX_SEGS ? u / w : 1;
  return 1;  // prime widths run unsplit (one or more passes)
}

// The wave-columns a one-token launch splits a row into (S chunks of W waves, one pass each), or
// 0 when a row needs more than one pass (then tokens run the per-group path below).
static int batch_columns(int nmat, int cols, int *S_out, int *W_out) {
  const int S = gemv_chunks(nmat, cols);
  int passes, nwv;
  cs_shape(cols / S, &passes, &nwv);
  if (passes != 1) return 0;
  *S_out = S;
  *W_out = nwv;
  return S * nwv;
}

// Matrices of different formats that the mixed kernels do not hold run one launch each.
static bool per_matrix(const GemvMat *mats, int nmat) {
  bool same = true, mixable = true;
  for (int i = 0; i < nmat; i++) {
    same = same && mats[i].type == mats[0].type;
    mixable = mixable && gemv_mixed_supports(mats[i].type);
  }
  return !same && !mixable;
}

int64_t gemv_scratch_floats(const GemvMat *mats, int nmat, int nm, int cols, int T) {
  if (nmat > 1 && per_matrix(mats, nmat)) {
    int64_t most = 0;
    for (int i = 0; i < nmat; i++) {
      const int64_t f = gemv_scratch_floats(&mats[i], 1, nm, cols, T);
      most = f > most ? f : most;
    }
    return most;
  }
  const int S = gemv_chunks(nmat, cols);
  int64_t n = 0;
  if (S > 1)
    for (int i = 0; i < nmat; i++) n += (int64_t)S * nm * T * mats[i].rows;
  int bs, bw;
  const int u = T > 1 ? batch_columns(nmat, cols, &bs, &bw) : 0;
  int64_t nb = 0;
  for (int i = 0; i < nmat; i++) nb += (int64_t)u * nm * T * mats[i].rows;
  return n > nb ? n : nb;
}

template <int TM>
static hipError_t launch_mixed_tm(GemvParams &p, int split, int num_cu, hipStream_t st) {
  int passes, nwv;
  cs_shape(p.cols, &passes, &nwv);
  const int nwg = plan_grid(p, [](int type) { return mixed_rows_per_group(type, TM); }, nwv, num_cu);
  if (nwg == 0) return hipSuccess;
  const size_t smem = sizeof(float) * 2 * GS * nwv * 8 * TM;  // the largest R*TM of the three codecs
  if (TM == 1 && passes == 1)
    hipLaunchKernelGGL((gemv_mixed_kernel<TM, TM == 1 ? 1 : 0>), dim3(nwg), dim3(64 * nwv), smem, st, p, split);
  else if (TM == 1 && passes == 2)
    hipLaunchKernelGGL((gemv_mixed_kernel<TM, TM == 1 ? 2 : 0>), dim3(nwg), dim3(64 * nwv), smem, st, p, split);
  else
    hipLaunchKernelGGL((gemv_mixed_kernel<TM, 0>), dim3(nwg), dim3(64 * nwv), smem, st, p, split);
  return hipGetLastError();
}

#ifndef WL_BATCH_MIXED_OCC
#define WL_BATCH_MIXED_OCC 4
#endif

// Matrices of different formats in one launch (q/k Q4_K with v Q6_K): the codec is chosen per
// workgroup, every workgroup stays on one matrix.
template <int TM>
__global__ __launch_bounds__(64 * kBatchWaves) __attribute__((amdgpu_waves_per_eu(WL_BATCH_MIXED_OCC)))
void gemv_batch_mixed_kernel(BatchArgs a) {
  const int mi = batch_mat(a);
  const BatchMat &M = a.m[mi];
  const int wgx = (int)blockIdx.x - M.wg_begin, nwg = batch_nwg(a, mi);
  switch (M.type) {
    case 12: batch_body<Q4K, TM, kBatchR1, 1>(a, M, wgx, nwg); break;
    case 14: batch_body<Q6K, TM, kBatchR1, 1>(a, M, wgx, nwg); break;
    case 8: batch_body<Q80, TM, kBatchR1, 1>(a, M, wgx, nwg); break;
    default: break;
  }
}

template <int TM>
static hipError_t launch_batch_mixed_tm(BatchArgs a, int num_cu, hipStream_t st) {
  constexpr size_t s1 = batch_lds_bytes<Q4K, TM>(), s2 = batch_lds_bytes<Q6K, TM>(), s3 = batch_lds_bytes<Q80, TM>();
  constexpr size_t smem = s1 > s2 ? (s1 > s3 ? s1 : s3) : (s2 > s3 ? s2 : s3);
  static bool raised = false;
  hipError_t e = raise_lds(&gemv_batch_mixed_kernel<TM>, smem, raised);
  if (e != hipSuccess) return e;
  const int gx = plan_batch(a, kBatchR1, num_cu);
  hipLaunchKernelGGL((gemv_batch_mixed_kernel<TM>), dim3(gx, a.u), dim3(64 * kBatchWaves), smem, st, a);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  return launch_batch_combine<1>(a, st);
}

// The codecs of this unit and the lookup over every unit.
const GemvOps *gemv_ops_base(int type) {
  static constexpr GemvOps q4k = gemv_ops_of<Q4K>(), q6k = gemv_ops_of<Q6K>(), q80 = gemv_ops_of<Q80>(),
                           iq4xs = gemv_ops_of2<IQ4XS, IQ4XSR>(), iq2xxs = gemv_ops_of<IQ2XXS>();
  switch (type) {
    case 12: return &q4k;
    case 14: return &q6k;
    case 8: return &q80;
    case 23: return &iq4xs;
    case 16: return &iq2xxs;
  }
  return nullptr;
}

static const GemvOps *gemv_ops(int type) {
  if (const GemvOps *o = gemv_ops_base(type)) return o;
  if (const GemvOps *o = gemv_ops_k(type)) return o;
  if (const GemvOps *o = gemv_ops_32(type)) return o;
  return gemv_ops_f(type);
}

#ifndef WL_GEMV_BATCH
#define WL_GEMV_BATCH 1
#endif

// The batched path for every matrix of a launch of T >= 2 tokens, when the one-token launch runs
// its rows in single passes. Returns hipErrorNotSupported when it does not apply.
static hipError_t gemv_batch_run(const GemvMat *mats, int nmat, int nm, const float *x, int ldx, int cols, int T,
                                 float *scratch, int num_cu, hipStream_t st) {
  if (!WL_GEMV_BATCH || T < 2 || !scratch) return hipErrorNotSupported;
  BatchArgs a{};
  a.u = batch_columns(nmat, cols, &a.S, &a.W);
  if (a.u == 0) return hipErrorNotSupported;
  a.nmat = nmat;
  a.cols = cols;
  a.x = x;
  a.ldx = ldx;
  a.T = T;
  bool same = true;
  float *part = scratch;
  for (int i = 0; i < nmat; i++) {
    const GemvMat &m = mats[i];
    a.m[i] = BatchMat{m.w, m.w2, m.row_bytes, part, m.y, m.ldy, m.rows, m.type, 0, m.add, m.rs};
    part += (int64_t)a.u * nm * T * m.rows;
    same = same && m.type == mats[0].type;
  }
  if (same) {
    const GemvOps *o = gemv_ops(mats[0].type);
    return o ? o->batch[nm - 1](a, num_cu, st) : hipErrorInvalidValue;
  }
  for (int i = 0; i < nmat; i++)
    if (!gemv_mixed_supports(mats[i].type)) return hipErrorNotSupported;
  if (T <= 2) return launch_batch_mixed_tm<2>(a, num_cu, st);
  if (T <= 4) return launch_batch_mixed_tm<4>(a, num_cu, st);
  return launch_batch_mixed_tm<8>(a, num_cu, st);
}

hipError_t gemv_run(const GemvMat *mats, int nmat, int nm, const float *x, int ldx, int cols, int T,
                    float *scratch, int num_cu, hipStream_t st) {
  if (nmat < 1 || nmat > GEMV_MAX_MATS || T < 1 || T > 8 || (nm != 1 && nm != 2)) return hipErrorInvalidValue;
  bool same = true;
  for (int i = 1; i < nmat; i++) same = same && mats[i].type == mats[0].type;
  if (!same && nm != 1) return hipErrorInvalidValue;
  if (per_matrix(mats, nmat)) {
    // formats the mixed kernels do not hold: one launch per matrix (each needs less scratch
    // than the whole set)
    for (int i = 0; i < nmat; i++) {
      const hipError_t e = gemv_run(&mats[i], 1, nm, x, ldx, cols, T, scratch, num_cu, st);
      if (e != hipSuccess) return e;
    }
    return hipSuccess;
  }
  {
    const hipError_t e = gemv_batch_run(mats, nmat, nm, x, ldx, cols, T, scratch, num_cu, st);
    if (e != hipErrorNotSupported) return e;
  }
  const int S = gemv_chunks(nmat, cols);
  if (S > 1 && !scratch) return hipErrorInvalidValue;
  GemvParams p{};
  p.cols = cols / S;
  p.x = x;
  p.ldx = ldx;
  p.T = T;
  CombineParams cp{};
  cp.S = S;
  cp.NM = nm;
  cp.T = T;
  float *part = scratch;
  int maxrows = 0;
  for (int i = 0; i < nmat; i++) {
    const GemvMat &m = mats[i];
    int be = 0, bb = 0;
    if (!wl_type_layout(m.type, &be, &bb)) return hipErrorInvalidValue;
    const int64_t chunk_bytes = (int64_t)(p.cols / be) * bb;
    for (int c = 0; c < S; c++) {
      GemvSeg &s = p.seg[p.nseg++];
      s.w = m.w + c * chunk_bytes;
      s.w2 = m.w2 ? m.w2 + c * chunk_bytes : nullptr;
      s.row_bytes = m.row_bytes;
      s.rows = m.rows;
      s.col0 = c * p.cols;
      s.type = m.type;
      s.add = m.add;
      s.rs = m.rs;
      if (S == 1) {
        s.out = m.y;
        s.ldo = m.ldy;
      } else {
        s.out = part + (int64_t)c * nm * T * m.rows;
        s.ldo = m.rows;
      }
    }
    if (S > 1) {
      cp.part[i] = part;
      cp.y[i] = m.y;
      cp.ldy[i] = m.ldy;
      cp.rows[i] = m.rows;
      cp.add[i] = m.add;
      cp.rs[i] = m.rs;
      part += (int64_t)S * nm * T * m.rows;
    }
    maxrows = m.rows > maxrows ? m.rows : maxrows;
  }
  const int split = S > 1;
  hipError_t e;
  if (same) {
    const GemvOps *o = gemv_ops(mats[0].type);
    e = o ? o->launch[nm - 1](p, split, num_cu, st) : hipErrorInvalidValue;
  } else if (T <= 1) {
    e = launch_mixed_tm<1>(p, split, num_cu, st);
  } else if (T <= 2) {
    e = launch_mixed_tm<2>(p, split, num_cu, st);
  } else if (T <= 4) {
    e = launch_mixed_tm<4>(p, split, num_cu, st);
  } else {
    e = launch_mixed_tm<8>(p, split, num_cu, st);
  }
  if (e != hipSuccess || !split || maxrows == 0) return e;
  const int64_t n = (int64_t)T * maxrows;
  hipLaunchKernelGGL(combine_kernel, dim3((unsigned)((n + 255) / 256), nmat), dim3(256), 0, st, cp);
  return hipGetLastError();
}

bool gemv_supports(int type) { return gemv_ops(type) != nullptr; }

bool gemv_mixed_supports(int type) { return type == 12 || type == 14 || type == 8; }

}  // namespace wl
