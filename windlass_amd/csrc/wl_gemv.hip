// wl_gemv.hip - decode GEMV for raw GGUF blocks (batch 1..8), bandwidth-bound, no MFMA.
//
// Replaces the CPU path's Transformer.MatMul T==1 branch (src/Transformer.cs:494-502, one
// Quants.DotRow per row) and MatMulEach (:544-561, one DotRow per (row, token)), plus the
// decode-then-Block path the I-quants take (:526-536). The kernel body is cs_gemv
// (wl_gemv_impl.h): column-stationary lanes, each weight byte read once per launch.
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

template <class C, int TM, int R, int NM, int SP>
__device__ __forceinline__ void run_seg(const GemvParams &p, const GemvSeg &s) {
  const CsRows W{s.w, s.w2, s.row_bytes, s.rows};
  const CsIO io{p.x, nullptr, p.ldx, s.y, nullptr, s.ldy, p.T};
  cs_gemv<C, TM, R, NM, SP>(W, io, p.cols, (int)blockIdx.x - s.wg_begin, s.nwg, wl_dyn_lds);
}

template <class C, int TM, int R, int NM, int SP>
__global__ __launch_bounds__(512) void gemv_kernel(GemvParams p) {
  run_seg<C, TM, R, NM, SP>(p, p.seg[find_seg(p)]);
}

// Segments of different formats in one launch (q/k Q4_K with v Q6_K): the codec is chosen
// per workgroup; every segment's workgroups stay on that segment.
// Rows per group: V = NM*R*TM partials per lane go through the exchange butterfly.
template <class C, int TM, int NM>
constexpr int rows_per_group() {
  return TM == 1 ? (NM == 1 ? C::R1 : C::R1 / 2) : (NM == 1 ? 4 : 2);
}

template <int TM, int SP>
__global__ __launch_bounds__(512) void gemv_mixed_kernel(GemvParams p) {
  const GemvSeg &s = p.seg[find_seg(p)];
  switch (s.type) {
    case 12: run_seg<Q4K, TM, rows_per_group<Q4K, TM, 1>(), 1, SP>(p, s); break;
    case 14: run_seg<Q6K, TM, rows_per_group<Q6K, TM, 1>(), 1, SP>(p, s); break;
    case 8: run_seg<Q80, TM, rows_per_group<Q80, TM, 1>(), 1, SP>(p, s); break;
    default: break;
  }
}

int gemv_waves(int cols) {
  int passes, waves;
  cs_shape(cols, &passes, &waves);
  return waves;
}

static int gemv_passes(int cols) {
  int passes, waves;
  cs_shape(cols, &passes, &waves);
  return passes;
}

// Split the grid over the segments in proportion to their row groups: about 16 waves per CU.
// rows_of(i) gives segment i's rows per group.
template <class RowsPerGroup>
static int plan_grid(GemvParams &p, RowsPerGroup rows_of, int nwv, int num_cu) {
  int total_groups = 0;
  for (int i = 0; i < p.nseg; i++) total_groups += (p.seg[i].rows + rows_of(i) - 1) / rows_of(i);
  if (total_groups == 0) return 0;
  const int target = (num_cu * 16 + nwv - 1) / nwv;
  int nwg = 0;
  for (int i = 0; i < p.nseg; i++) {
    const int R = rows_of(i);
    const int groups = (p.seg[i].rows + R - 1) / R;
    int n = (int)(((int64_t)target * groups + total_groups - 1) / total_groups);
    if (n < 1) n = 1;
    if (n > groups) n = groups;
    p.seg[i].wg_begin = nwg;
    p.seg[i].nwg = n;
    nwg += n;
  }
  return nwg;
}

template <class C, int TM, int NM>
static hipError_t launch_one(GemvParams &p, int num_cu, hipStream_t st) {
  constexpr int R = rows_per_group<C, TM, NM>();
  const int nwv = gemv_waves(p.cols), passes = gemv_passes(p.cols);
  const int nwg = plan_grid(p, [](int) { return R; }, nwv, num_cu);
  if (nwg == 0) return hipSuccess;
  const size_t smem = cs_lds_bytes<C, TM, R, NM>(nwv);
  if (TM == 1 && passes == 1)
    hipLaunchKernelGGL((gemv_kernel<C, TM, R, NM, TM == 1 ? 1 : 0>), dim3(nwg), dim3(64 * nwv), smem, st, p);
  else if (TM == 1 && passes == 2)
    hipLaunchKernelGGL((gemv_kernel<C, TM, R, NM, TM == 1 ? 2 : 0>), dim3(nwg), dim3(64 * nwv), smem, st, p);
  else
    hipLaunchKernelGGL((gemv_kernel<C, TM, R, NM, 0>), dim3(nwg), dim3(64 * nwv), smem, st, p);
  return hipGetLastError();
}

template <class C, int NM>
static hipError_t launch_tm(GemvParams &p, int num_cu, hipStream_t st) {
  if (p.T <= 1) return launch_one<C, 1, NM>(p, num_cu, st);
  if (p.T <= 2) return launch_one<C, 2, NM>(p, num_cu, st);
  if (p.T <= 4) return launch_one<C, 4, NM>(p, num_cu, st);
  return launch_one<C, 8, NM>(p, num_cu, st);
}

hipError_t gemv_launch(int type, int nm, GemvParams &p, int num_cu, hipStream_t st) {
  if (nm == 1) {
    switch (type) {
      case 12: return launch_tm<Q4K, 1>(p, num_cu, st);
      case 14: return launch_tm<Q6K, 1>(p, num_cu, st);
      case 8: return launch_tm<Q80, 1>(p, num_cu, st);
      case 23: return launch_tm<IQ4XS, 1>(p, num_cu, st);
      case 16: return launch_tm<IQ2XXS, 1>(p, num_cu, st);
    }
  } else {
    switch (type) {
      case 12: return launch_tm<Q4K, 2>(p, num_cu, st);
      case 14: return launch_tm<Q6K, 2>(p, num_cu, st);
      case 8: return launch_tm<Q80, 2>(p, num_cu, st);
      case 23: return launch_tm<IQ4XS, 2>(p, num_cu, st);
      case 16: return launch_tm<IQ2XXS, 2>(p, num_cu, st);
    }
  }
  return hipErrorInvalidValue;
}

static int mixed_rows(int type, int tm) {
  if (tm > 1) return 4;
  return type == 12 ? Q4K::R1 : type == 14 ? Q6K::R1 : Q80::R1;
}

template <int TM>
static hipError_t launch_mixed_tm(GemvParams &p, int num_cu, hipStream_t st) {
  const int nwv = gemv_waves(p.cols), passes = gemv_passes(p.cols);
  const int nwg = plan_grid(p, [&](int i) { return mixed_rows(p.seg[i].type, TM); }, nwv, num_cu);
  if (nwg == 0) return hipSuccess;
  const size_t smem = sizeof(float) * 2 * nwv * 8 * TM;  // the largest R*TM of the three codecs
  if (TM == 1 && passes == 1)
    hipLaunchKernelGGL((gemv_mixed_kernel<TM, TM == 1 ? 1 : 0>), dim3(nwg), dim3(64 * nwv), smem, st, p);
  else if (TM == 1 && passes == 2)
    hipLaunchKernelGGL((gemv_mixed_kernel<TM, TM == 1 ? 2 : 0>), dim3(nwg), dim3(64 * nwv), smem, st, p);
  else
    hipLaunchKernelGGL((gemv_mixed_kernel<TM, 0>), dim3(nwg), dim3(64 * nwv), smem, st, p);
  return hipGetLastError();
}

hipError_t gemv_launch_mixed(GemvParams &p, int num_cu, hipStream_t st) {
  if (p.T <= 1) return launch_mixed_tm<1>(p, num_cu, st);
  if (p.T <= 2) return launch_mixed_tm<2>(p, num_cu, st);
  if (p.T <= 4) return launch_mixed_tm<4>(p, num_cu, st);
  return launch_mixed_tm<8>(p, num_cu, st);
}

bool gemv_supports(int type) { return type == 12 || type == 14 || type == 8 || type == 23 || type == 16; }

bool gemv_mixed_supports(int type) { return type == 12 || type == 14 || type == 8; }

}  // namespace wl
