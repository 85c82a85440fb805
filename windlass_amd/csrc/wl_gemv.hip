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
#include "wl_gemv.h"
#include "wl_gemv_impl.h"

#pragma clang fp contract(off)

namespace wl {

extern "C" __shared__ uint8_t wl_dyn_lds[];

__device__ __forceinline__ int find_seg(const GemvParams &p) {
  int si = 0;
#pragma unroll
  for (int i = 1; i < GEMV_MAX_SEGS; i++)
    if (i < p.nseg && (int)blockIdx.x >= p.seg[i].wg_begin) si = i;
  return si;
}

// split: the segment writes partials; for the SwiGLU pair the up partial follows the gate
// partial at out + T * ldo.
template <class C, int TM, int R, int NM, int SP>
__device__ __forceinline__ void run_seg(const GemvParams &p, const GemvSeg &s, int split) {
  const CsRows W{s.w, s.w2, s.row_bytes, s.rows};
  float *y2 = (NM == 2 && split) ? s.out + (int64_t)p.T * s.ldo : nullptr;
  const CsIO io{p.x + s.col0, nullptr, p.ldx, s.out, nullptr, s.ldo, p.T, y2};
  cs_gemv<C, TM, R, NM, SP>(W, io, p.cols, (int)blockIdx.x - s.wg_begin, s.nwg, wl_dyn_lds);
}

template <class C, int TM, int R, int NM, int SP>
__global__ __launch_bounds__(64 * kMaxWaves) void gemv_kernel(GemvParams p, int split) {
  run_seg<C, TM, R, NM, SP>(p, p.seg[find_seg(p)], split);
}

// Rows per group: V = NM*R*TM partials per lane go through the exchange butterfly.
template <class C, int TM, int NM>
constexpr int rows_per_group() {
  return TM == 1 ? (NM == 1 ? C::R1 : C::R1 / 2) : (NM == 1 ? 4 : 2);
}

static int rows_per_group_rt(int type, int tm, int nm) {
  if (tm > 1) return nm == 1 ? 4 : 2;
  const int r1 = type == 12 ? Q4K::R1 : type == 14 ? Q6K::R1 : type == 8 ? Q80::R1 : type == 23 ? IQ4XS::R1
                                                                                                    : IQ2XXS::R1;
  return nm == 1 ? r1 : r1 / 2;
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
  cp.y[m][(int64_t)t * cp.ldy[m] + r] = g;
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

int64_t gemv_scratch_floats(const GemvMat *mats, int nmat, int nm, int cols, int T) {
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

// Grid: about kWavesPerCu waves per CU, split over the segments in proportion to their groups.
static int plan_grid(GemvParams &p, int tm, int nm, int nwv, int num_cu) {
  int total = 0, groups[GEMV_MAX_SEGS];
  for (int i = 0; i < p.nseg; i++) {
    const int R = rows_per_group_rt(p.seg[i].type, tm, nm);
    groups[i] = (p.seg[i].rows + R - 1) / R;
    total += groups[i];
  }
  if (total == 0) return 0;
  const int target = (num_cu * kWavesPerCu + nwv - 1) / nwv;
  int nwg = 0;
  for (int i = 0; i < p.nseg; i++) {
    int n = (int)(((int64_t)target * groups[i] + total - 1) / total);
    if (n < 1) n = 1;
    if (n > groups[i]) n = groups[i];
    p.seg[i].wg_begin = nwg;
    p.seg[i].nwg = n;
    nwg += n;
  }
  return nwg;
}

template <class C, int TM, int NM>
static hipError_t launch_one(GemvParams &p, int split, int num_cu, hipStream_t st) {
  constexpr int R = rows_per_group<C, TM, NM>();
  int passes, nwv;
  cs_shape(p.cols, &passes, &nwv);
  const int nwg = plan_grid(p, TM, NM, nwv, num_cu);
  if (nwg == 0) return hipSuccess;
  const size_t smem = cs_lds_bytes<C, TM, R, NM>(nwv);
  if (TM == 1 && passes == 1)
    hipLaunchKernelGGL((gemv_kernel<C, TM, R, NM, TM == 1 ? 1 : 0>), dim3(nwg), dim3(64 * nwv), smem, st, p, split);
  else if (TM == 1 && passes == 2 && C::SP2)
    hipLaunchKernelGGL((gemv_kernel<C, TM, R, NM, TM == 1 ? 2 : 0>), dim3(nwg), dim3(64 * nwv), smem, st, p, split);
  else
    hipLaunchKernelGGL((gemv_kernel<C, TM, R, NM, 0>), dim3(nwg), dim3(64 * nwv), smem, st, p, split);
  return hipGetLastError();
}

template <class C, int NM>
static hipError_t launch_tm(GemvParams &p, int split, int num_cu, hipStream_t st) {
  if (p.T <= 1) return launch_one<C, 1, NM>(p, split, num_cu, st);
  if (p.T <= 2) return launch_one<C, 2, NM>(p, split, num_cu, st);
  if (p.T <= 4) return launch_one<C, 4, NM>(p, split, num_cu, st);
  return launch_one<C, 8, NM>(p, split, num_cu, st);
}

template <int NM>
static hipError_t launch_type(int type, GemvParams &p, int split, int num_cu, hipStream_t st) {
  switch (type) {
    case 12: return launch_tm<Q4K, NM>(p, split, num_cu, st);
    case 14: return launch_tm<Q6K, NM>(p, split, num_cu, st);
    case 8: return launch_tm<Q80, NM>(p, split, num_cu, st);
    case 23: return launch_tm<IQ4XS, NM>(p, split, num_cu, st);
    case 16: return launch_tm<IQ2XXS, NM>(p, split, num_cu, st);
  }
  return hipErrorInvalidValue;
}

template <int TM>
static hipError_t launch_mixed_tm(GemvParams &p, int split, int num_cu, hipStream_t st) {
  int passes, nwv;
  cs_shape(p.cols, &passes, &nwv);
  const int nwg = plan_grid(p, TM, 1, nwv, num_cu);
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

static int block_bytes(int type) {
  return type == 12 ? 144 : type == 14 ? 210 : type == 8 ? 34 : type == 23 ? 136 : 66;
}

// ------------------------------------------------------------------ batched tokens (T >= 2)
// The one-token launch's decomposition, kept bit for bit, with the tokens' x slices staged in
// LDS once per workgroup: a workgroup owns ONE wave-column c (blocks c*BPW .. +BPW: the slices a
// wave of the one-token launch owns) for a stripe of row groups of one matrix; its waves walk
// row groups independently (no barrier after staging). Per (matrix, token, row) a lane forms the
// codec's dot on its slice, the 64 lanes fold it with the same exchange butterfly, and the
// wave-column's result goes to part[m][t][row][c]. batch_combine_kernel then adds the
// wave-columns as the one-token launch does: in wave order within each K-chunk, then in chunk
// order, SiLU last for the SwiGLU pair. So every token's bits equal its one-token result.
// All matrices of a call (q, k, v) share one launch and one combine launch.
struct BatchMat {
  const uint8_t *w, *w2;
  int64_t row_bytes;
  float *part;  // [NM][T][rows][u]
  float *y;
  int ldy, rows, type;
  int wg_begin;  // first blockIdx.x of this matrix
};

struct BatchArgs {
  BatchMat m[GEMV_MAX_MATS];
  int nmat, cols;
  const float *x;
  int ldx, T;
  int u;     // wave-columns
  int S, W;  // the one-token launch's K-chunks and waves per chunk (u = S * W)
};

template <class C>
constexpr int xs_u4() {
  return (int)((sizeof(typename C::Xs) + 15) / 16);
}

template <class C, int TM>
__host__ __device__ constexpr size_t batch_lds_bytes() {
  return (C::NEED_LDS ? sizeof(Lds) : 0) + (size_t)TM * xs_u4<C>() * 64 * 16;
}

#ifndef WL_BATCH_WAVES
#define WL_BATCH_WAVES 8  // waves per workgroup of the batched kernel
#endif
constexpr int kBatchWaves = WL_BATCH_WAVES;

__device__ __forceinline__ int batch_mat(const BatchArgs &a) {
  int mi = 0;
#pragma unroll
  for (int i = 1; i < GEMV_MAX_MATS; i++)
    if (i < a.nmat && (int)blockIdx.x >= a.m[i].wg_begin) mi = i;
  return mi;
}

// wgx: this workgroup's index among the matrix's nwg workgroups of column blockIdx.y.
template <class C, int TM, int R, int NM>
__device__ __forceinline__ void batch_body(const BatchArgs &a, const BatchMat &M, int wgx, int nwg) {
  constexpr int V = NM * R * TM, LOW = 6 - ilog2(V), BPW = 64 / C::LPB, NX = xs_u4<C>();
  static_assert((1 << ilog2(V)) == V && V <= 64, "partials per lane must be a power of two <= 64");
  const Lds &lds = *reinterpret_cast<const Lds *>(wl_dyn_lds);
  uint4 *xl = reinterpret_cast<uint4 *>(wl_dyn_lds + (C::NEED_LDS ? sizeof(Lds) : 0));  // [TM][NX][64]
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int c = blockIdx.y, nb = a.cols / C::BLOCK;
  const int sub = lane % C::LPB, b = c * BPW + lane / C::LPB;
  const bool live = b < nb;
  const typename C::Lane L = C::lane(sub);
  if constexpr (C::NEED_LDS) C::init_lds(*reinterpret_cast<Lds *>(wl_dyn_lds));
  // stage: wave w prepares tokens w, w + kBatchWaves, ... as the one-token launch prepares its slice
  for (int t = wv; t < TM; t += kBatchWaves) {
    if (t < a.T && live) {
      typename C::Xs xs;
      C::load_x(a.x + (int64_t)t * a.ldx + (int64_t)b * C::BLOCK, L, xs);
      uint4 v[NX] = {};
      __builtin_memcpy(v, &xs, sizeof(xs));
#pragma unroll
      for (int i = 0; i < NX; i++) xl[(t * NX + i) * 64 + lane] = v[i];
    }
  }
  __syncthreads();
  const uint8_t *wm[2] = {M.w, M.w2};
  const int ngroups = (M.rows + R - 1) / R;
  for (int g = wgx * kBatchWaves + wv; g < ngroups; g += nwg * kBatchWaves) {
    float acc[NM][R][TM];
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
      for (int r = 0; r < R; r++)
#pragma unroll
        for (int t = 0; t < TM; t++) acc[m][r][t] = 0.f;
    if (live) {
      typename C::Raw raw[NM][R];
#pragma unroll
      for (int m = 0; m < NM; m++)
#pragma unroll
        for (int r = 0; r < R; r++) {
          // rows past the end re-read the last row (valid memory); their results are dropped
          const int row = min(g * R + r, M.rows - 1);
          C::load(wm[m] + (int64_t)row * M.row_bytes + (int64_t)b * C::BYTES, L, raw[m][r]);
        }
      typename C::W w[NM][R];
#pragma unroll
      for (int m = 0; m < NM; m++)
#pragma unroll
        for (int r = 0; r < R; r++) C::unpack(raw[m][r], L, lds, w[m][r]);
#pragma unroll
      for (int t = 0; t < TM; t++) {
        if (t < a.T) {
          uint4 v[NX];
#pragma unroll
          for (int i = 0; i < NX; i++) v[i] = xl[(t * NX + i) * 64 + lane];
          typename C::Xs xs;
          __builtin_memcpy(&xs, v, sizeof(xs));
#pragma unroll
          for (int m = 0; m < NM; m++)
#pragma unroll
            for (int r = 0; r < R; r++) acc[m][r][t] += C::dot(w[m][r], xs);
        }
      }
    }
    // value index v = (m*TM + t)*R + r, as the one-token launch folds it
    float vals[V];
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
      for (int t = 0; t < TM; t++)
#pragma unroll
        for (int r = 0; r < R; r++) vals[(m * TM + t) * R + r] = acc[m][r][t];
    const float q = exch_reduce<V, 5>(vals, lane);
    if ((lane & ((1 << LOW) - 1)) == 0) {
      const int v = lane >> LOW, r = v % R, t = (v / R) % TM, m = v / (R * TM);
      const int row = g * R + r;
      if (t < a.T && row < M.rows) M.part[(((int64_t)m * a.T + t) * M.rows + row) * a.u + c] = q;
    }
  }
}

__device__ __forceinline__ int batch_nwg(const BatchArgs &a, int mi) {
  return (mi + 1 < a.nmat ? a.m[mi + 1].wg_begin : (int)gridDim.x) - a.m[mi].wg_begin;
}

// Waves per SIMD the register budget is cut for: four (two resident workgroups of eight waves
// per CU, at most 128 VGPRs), except where that would spill (the Q6_K SwiGLU pair).
template <class C, int NM>
constexpr int batch_occupancy() {
  return NM == 2 && C::BYTES == 210 ? 2 : 4;
}

template <class C, int TM, int R, int NM>
__global__ __launch_bounds__(64 * kBatchWaves) __attribute__((amdgpu_waves_per_eu(batch_occupancy<C, NM>())))
void gemv_batch_kernel(BatchArgs a) {
  const int mi = batch_mat(a);
  batch_body<C, TM, R, NM>(a, a.m[mi], (int)blockIdx.x - a.m[mi].wg_begin, batch_nwg(a, mi));
}

#ifndef WL_BATCH_R1
#define WL_BATCH_R1 2  // rows per group of a single matrix
#endif
#ifndef WL_BATCH_R2
#define WL_BATCH_R2 1  // rows per group of the SwiGLU pair
#endif
#ifndef WL_BATCH_WPC
#define WL_BATCH_WPC 64  // waves per CU the grid aims at (about four rounds of resident workgroups)
#endif
constexpr int kBatchR1 = WL_BATCH_R1, kBatchR2 = WL_BATCH_R2;

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

// y[t][r] from the wave-column partials: waves in order within each of S chunks of W, then the
// chunks in order (the one-token launch's wave-0 sum and chunk combine); SiLU for the pair.
__device__ __forceinline__ float batch_sum(const float *p, int S, int W) {
  float y = 0.f;
  for (int c = 0; c < S; c++) {
    float s = p[c * W];
    for (int k = 1; k < W; k++) s += p[c * W + k];
    y = c == 0 ? s : y + s;
  }
  return y;
}

// blockIdx.y: the matrix.
template <int NM>
__global__ __launch_bounds__(256) void batch_combine_kernel(BatchArgs a) {
  const BatchMat &M = a.m[blockIdx.y];
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)a.T * M.rows) return;
  const int t = (int)(i / M.rows), r = (int)(i % M.rows);
  float s = batch_sum(M.part + i * a.u, a.S, a.W);
  if constexpr (NM == 2) s = silu_mul(s, batch_sum(M.part + ((int64_t)a.T * M.rows + i) * a.u, a.S, a.W));
  M.y[(int64_t)t * M.ldy + r] = s;
}

// Workgroups per matrix along x: about WL_BATCH_WPC waves per CU over all columns, split over
// the matrices in proportion to their row groups. Returns the grid's x size.
static int plan_batch(BatchArgs &a, int R, int num_cu) {
  int total = 0;
  for (int i = 0; i < a.nmat; i++) total += (a.m[i].rows + R - 1) / R;
  const int target = (num_cu * WL_BATCH_WPC / kBatchWaves + a.u - 1) / a.u;
  int gx = 0;
  for (int i = 0; i < a.nmat; i++) {
    const int groups = (a.m[i].rows + R - 1) / R;
    int n = (int)(((int64_t)target * groups + total - 1) / total);
    const int most = (groups + kBatchWaves - 1) / kBatchWaves;
    if (n > most) n = most;
    if (n < 1) n = 1;
    a.m[i].wg_begin = gx;
    gx += n;
  }
  return gx;
}

template <class K>
static hipError_t raise_lds(K *kernel, size_t smem, bool &raised) {
  if (smem > 65536 && !raised) {
    if (hipFuncSetAttribute(reinterpret_cast<const void *>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)smem) != hipSuccess)
      return hipErrorInvalidConfiguration;
    raised = true;
  }
  return hipSuccess;
}

template <int NM>
static hipError_t launch_batch_combine(const BatchArgs &a, hipStream_t st) {
  int most = 0;
  for (int i = 0; i < a.nmat; i++) most = a.m[i].rows > most ? a.m[i].rows : most;
  const int64_t n = (int64_t)a.T * most;
  hipLaunchKernelGGL(batch_combine_kernel<NM>, dim3((unsigned)((n + 255) / 256), a.nmat), dim3(256), 0, st, a);
  return hipGetLastError();
}

template <class C, int TM, int NM>
static hipError_t launch_batch_tm(BatchArgs a, int num_cu, hipStream_t st) {
  constexpr int R = NM == 1 ? kBatchR1 : kBatchR2;
  const size_t smem = batch_lds_bytes<C, TM>();
  static bool raised = false;
  hipError_t e = raise_lds(&gemv_batch_kernel<C, TM, R, NM>, smem, raised);
  if (e != hipSuccess) return e;
  const int gx = plan_batch(a, R, num_cu);
  hipLaunchKernelGGL((gemv_batch_kernel<C, TM, R, NM>), dim3(gx, a.u), dim3(64 * kBatchWaves), smem, st, a);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  return launch_batch_combine<NM>(a, st);
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

template <class C, int NM>
static hipError_t launch_batch(const BatchArgs &a, int num_cu, hipStream_t st) {
  if (a.T <= 2) return launch_batch_tm<C, 2, NM>(a, num_cu, st);
  if (a.T <= 4) return launch_batch_tm<C, 4, NM>(a, num_cu, st);
  return launch_batch_tm<C, 8, NM>(a, num_cu, st);
}

template <int NM>
static hipError_t launch_batch_type(int type, const BatchArgs &a, int num_cu, hipStream_t st) {
  switch (type) {
    case 12: return launch_batch<Q4K, NM>(a, num_cu, st);
    case 14: return launch_batch<Q6K, NM>(a, num_cu, st);
    case 8: return launch_batch<Q80, NM>(a, num_cu, st);
    case 23: return launch_batch<IQ4XS, NM>(a, num_cu, st);
    case 16: return launch_batch<IQ2XXS, NM>(a, num_cu, st);
  }
  return hipErrorInvalidValue;
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
    a.m[i] = BatchMat{m.w, m.w2, m.row_bytes, part, m.y, m.ldy, m.rows, m.type, 0};
    part += (int64_t)a.u * nm * T * m.rows;
    same = same && m.type == mats[0].type;
  }
  if (same) return nm == 2 ? launch_batch_type<2>(mats[0].type, a, num_cu, st)
                           : launch_batch_type<1>(mats[0].type, a, num_cu, st);
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
    const int be = m.type == 8 ? 32 : 256;
    const int64_t chunk_bytes = (int64_t)(p.cols / be) * block_bytes(m.type);
    for (int c = 0; c < S; c++) {
      GemvSeg &s = p.seg[p.nseg++];
      s.w = m.w + c * chunk_bytes;
      s.w2 = m.w2 ? m.w2 + c * chunk_bytes : nullptr;
      s.row_bytes = m.row_bytes;
      s.rows = m.rows;
      s.col0 = c * p.cols;
      s.type = m.type;
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
      part += (int64_t)S * nm * T * m.rows;
    }
    maxrows = m.rows > maxrows ? m.rows : maxrows;
  }
  const int split = S > 1;
  hipError_t e;
  if (same) {
    e = nm == 1 ? launch_type<1>(mats[0].type, p, split, num_cu, st)
                : launch_type<2>(mats[0].type, p, split, num_cu, st);
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

bool gemv_supports(int type) { return type == 12 || type == 14 || type == 8 || type == 23 || type == 16; }

bool gemv_mixed_supports(int type) { return type == 12 || type == 14 || type == 8; }

}  // namespace wl
