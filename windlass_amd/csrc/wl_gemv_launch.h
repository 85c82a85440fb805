// wl_gemv_launch.h - the decode GEMV launch templates. Every codec's kernels are instantiated
// in the one translation unit that owns the codec (wl_gemv.hip for Q4_K, Q6_K, Q8_0, IQ4_XS and
// IQ2_XXS; wl_gemv_k.hip, wl_gemv_32.hip and wl_gemv_f.hip for the other formats), which hands
// its launchers to gemv_run through GemvOps.
#pragma once
#include "wl_gemv.h"
#include "wl_gemv_impl.h"

#pragma clang fp contract(off)

namespace wl {

extern "C" __shared__ uint8_t wl_dyn_lds[];

// The launch's workgroup w belongs to segment find_seg(p): segments in consecutive ranges, or
// (ILV, a launch whose grid plan set ileave) in runs of 8 taken in turn, so that workgroup j of
// every segment is dispatched at about the same time and on the same XCD (j % 8).
template <bool ILV = false>
__device__ __forceinline__ int find_seg(const GemvParams &p) {
  if constexpr (ILV) return ((int)blockIdx.x >> 3) % p.nseg;
  int si = 0;
#pragma unroll
  for (int i = 1; i < GEMV_MAX_SEGS; i++)
    if (i < p.nseg && (int)blockIdx.x >= p.seg[i].wg_begin) si = i;
  return si;
}

// split: the segment writes partials; for the SwiGLU pair the up partial follows the gate
// partial at out + T * ldo.
template <class C, int TM, int R, int NM, int SP, bool PIPE = false, bool ILV = false>
__device__ __forceinline__ void run_seg(const GemvParams &p, const GemvSeg &s, int split) {
  const CsRows W{s.w, s.w2, s.row_bytes, s.rows};
  float *y2 = (NM == 2 && split) ? s.out + (int64_t)p.T * s.ldo : nullptr;
  const CsIO io{p.x + s.col0, nullptr, p.ldx, s.out, nullptr, s.ldo, p.T, y2, split ? 0 : s.add, s.rs};
  const int local = ILV ? ((int)blockIdx.x / (8 * p.nseg)) * 8 + ((int)blockIdx.x & 7) : (int)blockIdx.x - s.wg_begin;
  cs_gemv<C, TM, R, NM, SP, false, PIPE>(W, io, p.cols, local, s.nwg, wl_dyn_lds);
}

template <class C, int TM, int R, int NM, int SP, bool PIPE = false, bool ILV = false>
__global__ __launch_bounds__(64 * kMaxWaves) void gemv_kernel(GemvParams p, int split) {
  run_seg<C, TM, R, NM, SP, PIPE, ILV>(p, p.seg[find_seg<ILV>(p)], split);
}

// Rows per group: V = NM*R*TM partials per lane go through the exchange butterfly.
template <class C, int TM, int NM>
constexpr int rows_per_group() {
  return TM == 1 ? (NM == 1 ? C::R1 : C::R1 / 2) : (NM == 1 ? 4 : 2);
}

// Grid: about kWavesPerCu waves per CU, split over the segments in proportion to their groups
// (rows_of(type): rows per group of a segment's codec).
template <class RowsOf>
static int plan_grid(GemvParams &p, RowsOf rows_of, int nwv, int num_cu) {
  int total = 0, groups[GEMV_MAX_SEGS];
  for (int i = 0; i < p.nseg; i++) {
    const int R = rows_of(p.seg[i].type);
    groups[i] = (p.seg[i].rows + R - 1) / R;
    total += groups[i];
  }
  if (total == 0) return 0;
  const int target = (num_cu * kWavesPerCu + nwv - 1) / nwv;
  int nwg = 0;
  for (int i = 0; i < p.nseg; i++) {
    int n = (int)(((int64_t)target * groups[i] + total - 1) / total);
    // a multiple of the 8 XCDs (the dispatcher deals workgroup w to XCD w % 8)
    n = (n + 7) & ~7;
    if (n < 1) n = 1;
    if (n > groups[i]) n = groups[i];
    p.seg[i].wg_begin = nwg;
    p.seg[i].nwg = n;
    nwg += n;
  }
  // Segments of equal grids (the K-chunks of a split row) interleaved in runs of 8: row group g
  // of every chunk is then computed at about the same time on one XCD, whose L2 serves the
  // 128-byte line two neighbouring chunks share once.
  p.ileave = p.nseg > 1 && p.seg[0].nwg % 8 == 0;
  for (int i = 1; i < p.nseg; i++) p.ileave = p.ileave && p.seg[i].nwg == p.seg[0].nwg;
  return nwg;
}

// Codecs whose one-token launches of one matrix set take smaller row groups when the matrices
// are too small to give each SIMD four waves (the 4096-wide matrices of an 8B layer: o is 512
// row groups of 8, one wave per SIMD; in 2-row groups 8.4 -> 6.5 us, q/k/v in 4-row groups
// 9.0 -> 8.0 us). A row's sum does not depend on the grouping, so the bits are the same. Q8_0
// 4096x4096 measured slower in 2-row groups.
template <class C>
inline constexpr bool kSmallGroups = false;
template <>
inline constexpr bool kSmallGroups<Q4K> = true;
template <>
inline constexpr bool kSmallGroups<Q6K> = true;

template <class C, int TM, int R, int NM>
static hipError_t launch_r(GemvParams &p, int split, int num_cu, hipStream_t st);

// Q6_K single matrices of one token (the 70B down projection's chunks) in 2-row groups with the
// next group's weights loaded during the current one's work: 47.5 -> 45.9 us for the 70B down
// (the same loop for Q4_K, the q/k/v launch or larger groups was slower).
template <class C>
inline constexpr bool kPipelined = false;
template <>
inline constexpr bool kPipelined<Q6K> = true;

// Codecs whose one-token split rows run with the K-chunks interleaved (plan_grid): those whose
// 4096-column chunks do not end on 128-byte lines, where it measured faster (8192 x 28672, one
// token: IQ2_XXS 32.3 -> 30.2 us, IQ2_S 49.6 -> 46.8, IQ3_S 50.1 -> 49.4; Q6_K through the
// pipelined path; Q2_K 38.3 -> 42.6 and Q3_K within noise, so not those). The translation unit
// that owns a codec sets it.
template <class C>
inline constexpr bool kInterleaved = false;
template <>
inline constexpr bool kInterleaved<IQ2XXS> = true;

template <class C, int TM, int NM>
static hipError_t launch_one(GemvParams &p, int split, int num_cu, hipStream_t st) {
  constexpr int R = rows_per_group<C, TM, NM>();
  if constexpr (kPipelined<C> && TM == 1 && NM == 1) {
    int passes, nwv;
    cs_shape(p.cols, &passes, &nwv);
    if (passes == 1) {
      const int nwg = plan_grid(p, [](int) { return 2; }, nwv, num_cu);
      if (nwg == 0) return hipSuccess;
      const size_t smem = cs_lds_bytes<C, 1, 2, 1>(nwv);
      // the K-chunks of a split row (equal segments) interleaved: see plan_grid
      if (p.ileave)
        hipLaunchKernelGGL((gemv_kernel<C, 1, 2, 1, 1, true, true>), dim3(nwg), dim3(64 * nwv), smem, st, p, split);
      else
        hipLaunchKernelGGL((gemv_kernel<C, 1, 2, 1, 1, true>), dim3(nwg), dim3(64 * nwv), smem, st, p, split);
      return hipGetLastError();
    }
  }
  if constexpr (TM == 1 && NM == 1 && kSmallGroups<C> && R >= 4) {
    int passes, nwv;
    cs_shape(p.cols, &passes, &nwv);
    int64_t waves = 0;
    for (int i = 0; i < p.nseg; i++) waves += (int64_t)((p.seg[i].rows + R - 1) / R) * nwv;
    const int64_t want = (int64_t)num_cu * 16;  // four waves per SIMD
    if (waves * 4 <= want) return launch_r<C, TM, R / 4, NM>(p, split, num_cu, st);
    if (waves * 2 <= want) return launch_r<C, TM, R / 2, NM>(p, split, num_cu, st);
  }
  return launch_r<C, TM, R, NM>(p, split, num_cu, st);
}

template <class C, int TM, int R, int NM>
static hipError_t launch_r(GemvParams &p, int split, int num_cu, hipStream_t st) {
  int passes, nwv;
  cs_shape(p.cols, &passes, &nwv);
  const int nwg = plan_grid(p, [](int) { return R; }, nwv, num_cu);
  if (nwg == 0) return hipSuccess;
  const size_t smem = cs_lds_bytes<C, TM, R, NM>(nwv);
  if constexpr (kInterleaved<C> && TM == 1 && NM == 1) {
    if (passes == 1 && p.ileave) {  // the K-chunks of a split row interleaved: see plan_grid
      hipLaunchKernelGGL((gemv_kernel<C, 1, R, 1, 1, false, true>), dim3(nwg), dim3(64 * nwv), smem, st, p, split);
      return hipGetLastError();
    }
  }
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
  int add;       // y += result * rs
  float rs;
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
  return dyn_table_bytes<C>() + (size_t)TM * xs_u4<C>() * 64 * 16;
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
  const Lds &lds = tables_of<C>(wl_dyn_lds);
  uint4 *xl = reinterpret_cast<uint4 *>(wl_dyn_lds + dyn_table_bytes<C>());  // [TM][NX][64]
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int c = blockIdx.y, nb = a.cols / C::BLOCK;
  const int sub = lane % C::LPB, b = c * BPW + lane / C::LPB;
  const bool live = b < nb;
  const typename C::Lane L = C::lane(sub);
  if constexpr (C::NEED_LDS) C::init_lds(tables_of<C>(wl_dyn_lds));
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
static __global__ __launch_bounds__(256) void batch_combine_kernel(BatchArgs a) {
  const BatchMat &M = a.m[blockIdx.y];
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)a.T * M.rows) return;
  const int t = (int)(i / M.rows), r = (int)(i % M.rows);
  float s = batch_sum(M.part + i * a.u, a.S, a.W);
  if constexpr (NM == 2) s = silu_mul(s, batch_sum(M.part + ((int64_t)a.T * M.rows + i) * a.u, a.S, a.W));
  float *y = M.y + (int64_t)t * M.ldy + r;
  *y = M.add ? add_scaled(*y, s, M.rs) : s;
}

// Workgroups per matrix along x: about WL_BATCH_WPC waves per CU over all columns, split over
// the matrices in proportion to their row groups. Returns the grid's x size.
static inline int plan_batch(BatchArgs &a, int R, int num_cu) {
  int total = 0;
  for (int i = 0; i < a.nmat; i++) total += (a.m[i].rows + R - 1) / R;
  const int target = (num_cu * WL_BATCH_WPC / kBatchWaves + a.u - 1) / a.u;
  int gx = 0;
  for (int i = 0; i < a.nmat; i++) {
    const int groups = (a.m[i].rows + R - 1) / R;
    int n = (int)(((int64_t)target * groups + total - 1) / total);
    // a multiple of the 8 XCDs: workgroup (x, c) is dispatched as x + c * gx and dealt to XCD
    // (x + c * gx) % 8, so the wave-columns c of a row set x then share one L2, where the
    // 128-byte line two neighbouring columns share is fetched once
    n = (n + 7) & ~7;
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

template <class C, int NM>
static hipError_t launch_batch(const BatchArgs &a, int num_cu, hipStream_t st) {
  if (a.T <= 2) return launch_batch_tm<C, 2, NM>(a, num_cu, st);
  if (a.T <= 4) return launch_batch_tm<C, 4, NM>(a, num_cu, st);
  return launch_batch_tm<C, 8, NM>(a, num_cu, st);
}

// The launchers of one codec: one token (any T through the per-group path) and the batched
// path, for a single matrix set (index 0) and the SwiGLU pair (index 1).
struct GemvOps {
  hipError_t (*launch[2])(GemvParams &, int, int, hipStream_t);
  hipError_t (*batch[2])(const BatchArgs &, int, hipStream_t);
};

template <class C>
constexpr GemvOps gemv_ops_of() {
  return GemvOps{{&launch_tm<C, 1>, &launch_tm<C, 2>}, {&launch_batch<C, 1>, &launch_batch<C, 2>}};
}
// A codec whose batched launches take another codec of the same values (CB builds the same
// weight words and shares C's dot, so every token's bits are the same).
template <class C, class CB>
constexpr GemvOps gemv_ops_of2() {
  return GemvOps{{&launch_tm<C, 1>, &launch_tm<C, 2>}, {&launch_batch<CB, 1>, &launch_batch<CB, 2>}};
}

// Each codec-owning unit: the ops of a format it holds, or nullptr.
const GemvOps *gemv_ops_base(int type);  // wl_gemv.hip
const GemvOps *gemv_ops_k(int type);     // wl_gemv_k.hip
const GemvOps *gemv_ops_32(int type);    // wl_gemv_32.hip
const GemvOps *gemv_ops_f(int type);     // wl_gemv_f.hip

}  // namespace wl
