// wl_gemv.hip - decode GEMV for raw GGUF blocks (batch 1..8), bandwidth-bound, no MFMA.
//
// Replaces the CPU path's Transformer.MatMul T==1 branch (src/Transformer.cs:494-502, one
// Quants.DotRow per row) and MatMulEach (:544-561, one DotRow per (row, token)), plus the
// decode-then-Block path the I-quants take (:526-536).
//
// Work decomposition: a workgroup is 4 waves; each wave owns R consecutive rows (of one or
// two matrices that read the same x). In each step a lane reads one fixed slice of one block
// of each of its rows (see wl_codecs.h), unpacks it in registers, and for every token loads
// the matching x slice and accumulates a partial dot; the partials of the 64 lanes are summed
// with one fixed butterfly at the end. Weight bytes are read exactly once per launch.
#include "wl_gemv.h"
#include "wl_gemv_impl.h"

#pragma clang fp contract(off)

namespace wl {

extern "C" __shared__ uint8_t wl_dyn_lds[];

template <class C, int TM, int R, int NM>
__global__ __launch_bounds__(256) void gemv_kernel(GemvParams p) {
  Lds &lds = *reinterpret_cast<Lds *>(wl_dyn_lds);
  if constexpr (C::NEED_LDS) {
    C::init_lds(lds);
    __syncthreads();
  }
  const int wg = blockIdx.x;
  int si = 0;
#pragma unroll
  for (int i = 1; i < GEMV_MAX_SEGS; i++)
    if (i < p.nseg && wg >= p.seg[i].wg_begin) si = i;
  const GemvSeg &s = p.seg[si];
  const int row0 = ((wg - s.wg_begin) * 4 + (int)(threadIdx.x >> 6)) * R;
  if (row0 >= s.rows) return;
  gemv_rows<C, TM, R, NM>(s.w, s.w2, s.row_bytes, s.rows, row0, p.x, nullptr, p.ldx, p.cols, p.T, s.y,
                          nullptr, s.ldy, lds);
}

// Segments of different formats in one launch (q/k Q4_K with v Q6_K): the codec is chosen
// per workgroup.
template <int TM, int R>
__global__ __launch_bounds__(256) void gemv_mixed_kernel(GemvParams p) {
  Lds &lds = *reinterpret_cast<Lds *>(wl_dyn_lds);
  const int wg = blockIdx.x;
  int si = 0;
#pragma unroll
  for (int i = 1; i < GEMV_MAX_SEGS; i++)
    if (i < p.nseg && wg >= p.seg[i].wg_begin) si = i;
  const GemvSeg &s = p.seg[si];
  const int row0 = ((wg - s.wg_begin) * 4 + (int)(threadIdx.x >> 6)) * R;
  if (row0 >= s.rows) return;
  switch (s.type) {
    case 12: gemv_rows<Q4K, TM, R, 1>(s.w, nullptr, s.row_bytes, s.rows, row0, p.x, nullptr, p.ldx, p.cols, p.T,
                                     s.y, nullptr, s.ldy, lds); break;
    case 14: gemv_rows<Q6K, TM, R, 1>(s.w, nullptr, s.row_bytes, s.rows, row0, p.x, nullptr, p.ldx, p.cols, p.T,
                                     s.y, nullptr, s.ldy, lds); break;
    case 8: gemv_rows<Q80, TM, R, 1>(s.w, nullptr, s.row_bytes, s.rows, row0, p.x, nullptr, p.ldx, p.cols, p.T,
                                     s.y, nullptr, s.ldy, lds); break;
    default: break;
  }
}

template <class C>
constexpr int rows_per_wave(int nm) {
  return nm == 2 ? 2 : 4;
}

template <class C, int TM, int NM>
static hipError_t launch_one(const GemvParams &p, int nwg, hipStream_t st) {
  constexpr int R = rows_per_wave<C>(NM);
  const size_t smem = C::NEED_LDS ? sizeof(Lds) : 0;
  hipLaunchKernelGGL((gemv_kernel<C, TM, R, NM>), dim3(nwg), dim3(256), smem, st, p);
  return hipGetLastError();
}

template <class C, int NM>
static hipError_t launch_tm(const GemvParams &p, int nwg, hipStream_t st) {
  if (p.T <= 1) return launch_one<C, 1, NM>(p, nwg, st);
  if (p.T <= 2) return launch_one<C, 2, NM>(p, nwg, st);
  if (p.T <= 4) return launch_one<C, 4, NM>(p, nwg, st);
  return launch_one<C, 8, NM>(p, nwg, st);
}

int gemv_rows_per_wg(int type, int nm) {
  (void)type;
  return 4 * (nm == 2 ? 2 : 4);
}

hipError_t gemv_launch(int type, int nm, GemvParams &p, hipStream_t st) {
  int nwg = 0;
  const int rpw = gemv_rows_per_wg(type, nm);
  for (int i = 0; i < p.nseg; i++) {
    p.seg[i].wg_begin = nwg;
    nwg += (p.seg[i].rows + rpw - 1) / rpw;
  }
  if (nwg == 0) return hipSuccess;
  if (nm == 1) {
    switch (type) {
      case 12: return launch_tm<Q4K, 1>(p, nwg, st);
      case 14: return launch_tm<Q6K, 1>(p, nwg, st);
      case 8: return launch_tm<Q80, 1>(p, nwg, st);
      case 23: return launch_tm<IQ4XS, 1>(p, nwg, st);
      case 16: return launch_tm<IQ2XXS, 1>(p, nwg, st);
    }
  } else {
    switch (type) {
      case 12: return launch_tm<Q4K, 2>(p, nwg, st);
      case 14: return launch_tm<Q6K, 2>(p, nwg, st);
      case 8: return launch_tm<Q80, 2>(p, nwg, st);
      case 23: return launch_tm<IQ4XS, 2>(p, nwg, st);
      case 16: return launch_tm<IQ2XXS, 2>(p, nwg, st);
    }
  }
  return hipErrorInvalidValue;
}

hipError_t gemv_launch_mixed(GemvParams &p, hipStream_t st) {
  constexpr int R = 4;
  int nwg = 0;
  for (int i = 0; i < p.nseg; i++) {
    p.seg[i].wg_begin = nwg;
    nwg += (p.seg[i].rows + 4 * R - 1) / (4 * R);
  }
  if (nwg == 0) return hipSuccess;
  if (p.T <= 1) hipLaunchKernelGGL((gemv_mixed_kernel<1, R>), dim3(nwg), dim3(256), 0, st, p);
  else if (p.T <= 2) hipLaunchKernelGGL((gemv_mixed_kernel<2, R>), dim3(nwg), dim3(256), 0, st, p);
  else if (p.T <= 4) hipLaunchKernelGGL((gemv_mixed_kernel<4, R>), dim3(nwg), dim3(256), 0, st, p);
  else hipLaunchKernelGGL((gemv_mixed_kernel<8, R>), dim3(nwg), dim3(256), 0, st, p);
  return hipGetLastError();
}

bool gemv_supports(int type) { return type == 12 || type == 14 || type == 8 || type == 23 || type == 16; }

bool gemv_mixed_supports(int type) { return type == 12 || type == 14 || type == 8; }

}  // namespace wl
