// wl_moe_launch.h - the grouped expert GEMV launch templates. Every codec's MoE kernels are
// instantiated in the unit that owns the codec and reach moe_launch through MoeOps.
#pragma once
#include "wl_gemv.h"
#include "wl_gemv_impl.h"
#include "wl_moe.h"

#pragma clang fp contract(off)

namespace wl {

extern "C" __shared__ uint8_t wl_moe_dyn_lds[];

// blockIdx.y = slot (one chosen expert); the slot's workgroups stride over the expert's rows.
template <class C, int TM, int R, int NM, int SP>
__global__ __launch_bounds__(64 * kMaxWaves) void moe_gemv_kernel(MoeGemvArgs a) {
  const MoePlan *plan = a.plan;
  const int s = blockIdx.y;
  if (s >= plan->nslots) return;  // uniform over the workgroup
  const int e = plan->slot_expert[s];
  const int64_t eoff = (int64_t)e * a.rows * a.row_bytes;
  const CsRows W{a.w + eoff, NM == 2 ? a.w2 + eoff : nullptr, a.row_bytes, a.rows};
  const CsIO io{a.x, a.x_by_pair ? plan->slot_pair[s] : plan->slot_tok[s], a.ldx, a.y, plan->slot_pair[s],
                a.ldy, plan->slot_ntok[s]};
  cs_gemv<C, TM, R, NM, SP>(W, io, a.cols, (int)blockIdx.x, (int)gridDim.x, wl_moe_dyn_lds);
}

template <class C, int TM, int NM>
static hipError_t launch_moe_gemv(const MoeGemvArgs &a, int max_slots, int num_cu, hipStream_t st) {
  constexpr int R = TM == 1 ? (NM == 1 ? C::R1 : C::R1 / 2) : (NM == 1 ? 4 : 2);
  int passes, nwv;
  cs_shape(a.cols, &passes, &nwv);
  const int groups = (a.rows + R - 1) / R;
  // about 16 waves per CU over all slots
  int gx = (num_cu * kWavesPerCu / nwv + max_slots - 1) / max_slots;
  if (gx < 1) gx = 1;
  if (gx > groups) gx = groups;
  const size_t smem = cs_lds_bytes<C, TM, R, NM>(nwv);
  if (TM == 1 && passes == 1)
    hipLaunchKernelGGL((moe_gemv_kernel<C, TM, R, NM, TM == 1 ? 1 : 0>), dim3(gx, max_slots), dim3(64 * nwv), smem, st, a);
  else
    hipLaunchKernelGGL((moe_gemv_kernel<C, TM, R, NM, 0>), dim3(gx, max_slots), dim3(64 * nwv), smem, st, a);
  return hipGetLastError();
}

template <class C, int NM>
static hipError_t launch_moe_tm(const MoeGemvArgs &a, int T, int max_slots, int num_cu, hipStream_t st) {
  if (T <= 1) return launch_moe_gemv<C, 1, NM>(a, max_slots, num_cu, st);
  if (T <= 2) return launch_moe_gemv<C, 2, NM>(a, max_slots, num_cu, st);
  if (T <= 4) return launch_moe_gemv<C, 4, NM>(a, max_slots, num_cu, st);
  return launch_moe_gemv<C, 8, NM>(a, max_slots, num_cu, st);
}

// The expert GEMV launchers of one codec: one matrix set (index 0) and the SwiGLU pair (1).
struct MoeOps {
  hipError_t (*launch[2])(const MoeGemvArgs &, int, int, int, hipStream_t);
};

template <class C>
constexpr MoeOps moe_ops_of() {
  return MoeOps{{&launch_moe_tm<C, 1>, &launch_moe_tm<C, 2>}};
}

// Each codec-owning unit: the ops of a format it holds, or nullptr.
const MoeOps *moe_ops_base(int type);  // wl_moe.hip
const MoeOps *moe_ops_k(int type);     // wl_gemv_k.hip
const MoeOps *moe_ops_32(int type);    // wl_gemv_32.hip
const MoeOps *moe_ops_f(int type);     // wl_gemv_f.hip

}  // namespace wl
