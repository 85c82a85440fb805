// wl_moe.hip - routed mixture-of-experts FFN on the GPU.
//
// Restates MoeFfn + Route (src/Transformer.cs:253-340) without a host round trip:
//   1. route_kernel    one thread per token runs the reference's sequential routing: softmax
//                      with a double denominator, k largest with ties to the lower id,
//                      renormalisation clamped at 6.103515625e-5 (:315-340);
//   2. plan_kernel     one thread orders the (expert, token) pairs: experts ascending, tokens
//                      ascending within an expert (the gather order of :271-286);
//   3. moe_gate_up     grouped decode GEMV over the chosen experts' gate/up slices
//                      (WeightView.Slice, src/LayerStream.cs:26-34), SiLU epilogue;
//   4. moe_down        grouped decode GEMV of each pair's hidden row with its expert's down;
//   5. combine_kernel  out[t] = sum over t's experts, ascending, of w * y (:289-293).
// Only the chosen experts are read (tests/MoeTests.cs:164-181).
#include "wl_moe.h"
#include "wl_gemv.h"
#include "wl_gemv_impl.h"

#pragma clang fp contract(off)

namespace wl {

#define WL_MIN_EXPERT_WEIGHT_SUM 6.103515625e-5f  // src/Transformer.cs:253

__global__ void route_kernel(const float *__restrict__ logits, int T, int n, int k, int renorm,
                             int *__restrict__ sel, float *__restrict__ wts, float *__restrict__ prob) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= T) return;
  const float *l = logits + (int64_t)t * n;
  float *p = prob + (int64_t)t * n;
  float mx = -INFINITY;
  for (int i = 0; i < n; i++)
    if (l[i] > mx) mx = l[i];
  double sum = 0;
  for (int i = 0; i < n; i++) {
    p[i] = (float)exp((double)(l[i] - mx));
    sum += p[i];
  }
  const float inv = (float)(1.0 / sum);
  for (int i = 0; i < n; i++) p[i] *= inv;
  float chosen = 0;
  for (int j = 0; j < k; j++) {
    int best = -1;
    // Taken entries hold -1, which no probability (>= 0, or NaN) equals; like the reference's
    // taken[] test, the first untaken entry is a candidate even when it is NaN.
    for (int i = 0; i < n; i++)
      if (p[i] != -1.f && (best < 0 || p[i] > p[best])) best = i;
    sel[t * k + j] = best;
    wts[t * k + j] = p[best];
    chosen += p[best];
    p[best] = -1.f;
  }
  if (renorm) {
    const float div = chosen > WL_MIN_EXPERT_WEIGHT_SUM ? chosen : WL_MIN_EXPERT_WEIGHT_SUM;
    for (int j = 0; j < k; j++) wts[t * k + j] /= div;
  }
}

__global__ void plan_kernel(const int *__restrict__ sel, const float *__restrict__ wts, int T, int k, int ne,
                            MoePlan *__restrict__ plan) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  int ns = 0, np = 0;
  for (int e = 0; e < ne; e++) {
    int n = 0;
    for (int t = 0; t < T; t++)
      for (int j = 0; j < k; j++)
        if (sel[t * k + j] == e) {
          plan->slot_tok[ns][n] = t;
          plan->slot_pair[ns][n] = np;
          plan->tok_pair[t][j] = np;
          plan->tok_w[t][j] = wts[t * k + j];
          n++;
          np++;
        }
    if (n) {
      plan->slot_expert[ns] = e;
      plan->slot_ntok[ns] = n;
      ns++;
    }
  }
  plan->nslots = ns;
  // each token's pairs in ascending expert order: sort its k entries by the chosen expert id
  for (int t = 0; t < T; t++) {
    int ord[MOE_MAX_K];
    for (int j = 0; j < k; j++) ord[j] = j;
    for (int a = 1; a < k; a++)
      for (int b = a; b > 0 && sel[t * k + ord[b]] < sel[t * k + ord[b - 1]]; b--) {
        int tmp = ord[b]; ord[b] = ord[b - 1]; ord[b - 1] = tmp;
      }
    for (int j = 0; j < k; j++) {
      plan->comb_pair[t][j] = plan->tok_pair[t][ord[j]];
      plan->comb_w[t][j] = plan->tok_w[t][ord[j]];
    }
  }
}

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

__global__ void combine_kernel(const MoePlan *__restrict__ plan, const float *__restrict__ yd, int T, int k,
                               int embd, float *__restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)T * embd) return;
  const int t = (int)(i / embd), d = (int)(i % embd);
  float o = 0.f;
  for (int j = 0; j < k; j++) o += plan->comb_w[t][j] * yd[(int64_t)plan->comb_pair[t][j] * embd + d];
  out[i] = o;
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

template <int NM>
static hipError_t launch_moe_type(int type, const MoeGemvArgs &a, int T, int max_slots, int num_cu, hipStream_t st) {
  switch (type) {
    case 12: return launch_moe_tm<Q4K, NM>(a, T, max_slots, num_cu, st);
    case 14: return launch_moe_tm<Q6K, NM>(a, T, max_slots, num_cu, st);
    case 8: return launch_moe_tm<Q80, NM>(a, T, max_slots, num_cu, st);
    case 23: return launch_moe_tm<IQ4XS, NM>(a, T, max_slots, num_cu, st);
    case 16: return launch_moe_tm<IQ2XXS, NM>(a, T, max_slots, num_cu, st);
  }
  return hipErrorInvalidValue;
}

hipError_t route_launch(const float *logits, int T, int n, int k, int renorm, int *sel, float *wts, float *prob,
                        hipStream_t st) {
  hipLaunchKernelGGL(route_kernel, dim3((T + 63) / 64), dim3(64), 0, st, logits, T, n, k, renorm, sel, wts, prob);
  return hipGetLastError();
}

hipError_t moe_launch(const MoeLaunch &m, int num_cu, hipStream_t st) {
  hipError_t err = route_launch(m.logits, m.T, m.ne, m.k, m.renorm, m.sel, m.wts, m.prob, st);
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(plan_kernel, dim3(1), dim3(64), 0, st, m.sel, m.wts, m.T, m.k, m.ne, m.plan);
  if ((err = hipGetLastError()) != hipSuccess) return err;
  const int max_slots = m.T * m.k < m.ne ? m.T * m.k : m.ne;
  MoeGemvArgs gu{};
  gu.plan = m.plan;
  gu.w = m.gate; gu.w2 = m.up; gu.row_bytes = m.gu_row_bytes; gu.rows = m.ff; gu.cols = m.embd;
  gu.x = m.x; gu.ldx = m.embd; gu.x_by_pair = 0; gu.y = m.h; gu.ldy = m.ff;
  if ((err = launch_moe_type<2>(m.gu_type, gu, m.T, max_slots, num_cu, st)) != hipSuccess) return err;
  MoeGemvArgs dn{};
  dn.plan = m.plan;
  dn.w = m.down; dn.w2 = nullptr; dn.row_bytes = m.d_row_bytes; dn.rows = m.embd; dn.cols = m.ff;
  dn.x = m.h; dn.ldx = m.ff; dn.x_by_pair = 1; dn.y = m.yd; dn.ldy = m.embd;
  if ((err = launch_moe_type<1>(m.d_type, dn, m.T, max_slots, num_cu, st)) != hipSuccess) return err;
  const int64_t total = (int64_t)m.T * m.embd;
  hipLaunchKernelGGL(combine_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, m.plan, m.yd, m.T,
                     m.k, m.embd, m.out);
  return hipGetLastError();
}

bool moe_supports(int type) { return type == 12 || type == 14 || type == 8 || type == 23 || type == 16; }

}  // namespace wl
