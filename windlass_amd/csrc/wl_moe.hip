// wl_moe.hip - routed mixture-of-experts FFN on the GPU.
//
// Restates MoeFfn + Route (src/Transformer.cs:253-340) without a host round trip:
//   1. route + plan    one workgroup: wave t runs the reference's routing of token t (softmax
//                      with a double denominator, k largest with ties to the lower id,
//                      renormalisation clamped at 6.103515625e-5, :315-340), then one thread per
//                      (token, choice) pair numbers the pairs: experts ascending, tokens
//                      ascending within an expert (the gather order of :271-286);
//   3. moe_gate_up     grouped decode GEMV over the chosen experts' gate/up slices
//                      (WeightView.Slice, src/LayerStream.cs:26-34), SiLU epilogue;
//   4. moe_down        grouped decode GEMV of each pair's hidden row with its expert's down;
//   5. combine_kernel  out[t] = sum over t's experts, ascending, of w * y (:289-293).
// Only the chosen experts are read (tests/MoeTests.cs:164-181).
#include "wl_moe_launch.h"

#pragma clang fp contract(off)

namespace wl {

#define WL_MIN_EXPERT_WEIGHT_SUM 6.103515625e-5f  // src/Transformer.cs:253

// Serial routing, one thread per token (expert counts above kRouteWaveMax).
__global__ void route_serial_kernel(const float *__restrict__ logits, int T, int n, int k, int renorm,
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

// Routing of one token per wave (n <= 64 * PER experts, k <= 64): lane l holds probabilities l, l + 64,
// ...; the same values as route_serial_kernel. The maximum ignores NaN like the reference's `>`
// scan; the softmax denominator is summed in double in index order. The k picks are the entries
// of rank < k, an entry's rank being how many entries are larger, or equal at a lower id: what
// the reference's k rounds of sequential scans pick, in the same order. A NaN probability (then
// every probability is NaN, through the denominator) takes the scan's choice for NaN: the first
// untaken entry each round. The wave's probabilities, sort keys and picks pass through LDS (pl:
// room for n 64-bit keys; rk_i, rk_w: k entries each).
constexpr int kRouteWaveMax = 64 * 32;

template <int PER>
__device__ __forceinline__ void route_wave(const float *__restrict__ l, int n, int k, int renorm,
                                           int *__restrict__ sel, float *__restrict__ wts, float *__restrict__ pl,
                                           int *__restrict__ rk_i, float *__restrict__ rk_w) {
  const int lane = threadIdx.x & 63;
  float v[PER];
  float mx = -INFINITY;
#pragma unroll
  for (int m = 0; m < PER; m++) {
    const int i = lane + 64 * m;
    v[m] = i < n ? l[i] : -INFINITY;
    if (v[m] > mx) mx = v[m];
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float u = __shfl_xor(mx, o, 64);
    if (u > mx) mx = u;
  }
#pragma unroll
  for (int m = 0; m < PER; m++) {
    const int i = lane + 64 * m;
    if (i < n) {
      v[m] = (float)exp((double)(v[m] - mx));
      pl[i] = v[m];
    }
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  // the denominator in double, entries in index order, read back sixteen at a time so the reads
  // overlap the dependent adds
  const float4 *p4 = reinterpret_cast<const float4 *>(pl);
  double sum = 0;
  int i = 0;
  for (; i + 16 <= n; i += 16) {
    float4 q[4];
#pragma unroll
    for (int u = 0; u < 4; u++) q[u] = p4[i / 4 + u];
#pragma unroll
    for (int u = 0; u < 4; u++) {
      sum += (double)q[u].x;
      sum += (double)q[u].y;
      sum += (double)q[u].z;
      sum += (double)q[u].w;
    }
  }
  for (; i < n; i++) sum += (double)pl[i];
  const float inv = (float)(1.0 / sum);
  int nan = 0;
#pragma unroll
  for (int m = 0; m < PER; m++) {
    v[m] *= inv;
    nan |= (int)(lane + 64 * m < n) & (int)(v[m] != v[m]);
  }
  if (__any(nan)) {
    if (lane < k) {
      sel[lane] = lane;
      wts[lane] = __builtin_nanf("");
    }
    return;
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  // The probabilities are finite and not negative here, so their bit patterns order like the
  // values; key = (bits << 32) | ~id orders by probability, then by lower id, and an entry's
  // rank is how many keys exceed its own. The keys replace the probabilities in LDS (pl holds
  // 2n floats' room).
  uint64_t *keys = reinterpret_cast<uint64_t *>(pl);
  uint64_t key[PER];
  int rank[PER], me[PER];
#pragma unroll
  for (int m = 0; m < PER; m++) {
    me[m] = lane + 64 * m;
    rank[m] = 0;
    key[m] = ((uint64_t)__float_as_uint(v[m]) << 32) | (uint32_t)~me[m];
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
  for (int m = 0; m < PER; m++)
    if (me[m] < n) keys[me[m]] = key[m];
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  const ulonglong2 *k2 = reinterpret_cast<const ulonglong2 *>(keys);
  int j = 0;
  for (; j + 8 <= n; j += 8) {
    ulonglong2 q[4];
#pragma unroll
    for (int u = 0; u < 4; u++) q[u] = k2[j / 2 + u];
#pragma unroll
    for (int u = 0; u < 4; u++)
#pragma unroll
      for (int m = 0; m < PER; m++) rank[m] += (int)(q[u].x > key[m]) + (int)(q[u].y > key[m]);
  }
  for (; j < n; j++) {
    const uint64_t q = keys[j];
#pragma unroll
    for (int m = 0; m < PER; m++) rank[m] += (int)(q > key[m]);
  }
#pragma unroll
  for (int m = 0; m < PER; m++)
    if (me[m] < n && rank[m] < k) {
      rk_i[rank[m]] = me[m];
      rk_w[rank[m]] = v[m];
    }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  float chosen = 0;
  for (int c = 0; c < k; c++) chosen += rk_w[c];  // in pick order, as the reference adds them
  if (lane < k) {
    float w = rk_w[lane];
    if (renorm) {
      const float div = chosen > WL_MIN_EXPERT_WEIGHT_SUM ? chosen : WL_MIN_EXPERT_WEIGHT_SUM;
      w /= div;
    }
    sel[lane] = rk_i[lane];
    wts[lane] = w;
  }
}

template <int PER>
__global__ __launch_bounds__(64) void route_wave_kernel(const float *__restrict__ logits, int n, int k, int renorm,
                                                        int *__restrict__ sel, float *__restrict__ wts) {
  __shared__ __attribute__((aligned(16))) float lds[128 * PER + 128];
  const int t = blockIdx.x;
  route_wave<PER>(logits + (int64_t)t * n, n, k, renorm, sel + t * k, wts + t * k, lds, (int *)(lds + 128 * PER),
                  lds + 128 * PER + 64);
}

// The routing plan from T tokens' k choices, one thread per (token, choice) pair. Pairs are
// numbered experts ascending, tokens ascending within an expert (the gather order of
// src/Transformer.cs:271-286); each token's pairs are listed again in ascending expert order for
// the combine (:289-293).
constexpr int kPlanMaskExperts = 8192;  // experts the plan's bitmask covers; more use pair scans

__device__ __forceinline__ void plan_pairs(const int *__restrict__ sel, const float *__restrict__ wts, int T, int k,
                                           int n, MoePlan *__restrict__ plan) {
  __shared__ __attribute__((aligned(16))) int se[MOE_MAX_PAIRS];
  __shared__ int first_of[MOE_MAX_PAIRS];              // pair a is the lowest-index pair of its expert
  __shared__ uint32_t emask[kPlanMaskExperts / 32];  // experts chosen by any pair
  const int P = T * k, i = threadIdx.x, nw = (n + 31) / 32;
  const bool masked = n <= kPlanMaskExperts;
  if (masked)
    for (int w = i; w < nw; w += blockDim.x) emask[w] = 0;
  if (i < P) se[i] = sel[i];
  __syncthreads();
  if (i < P) {
    if (masked) {
      atomicOr(&emask[se[i] >> 5], 1u << (se[i] & 31));
    } else {
      int f = 1;
      for (int b = 0; b < i; b++) f &= (int)(se[b] != se[i]);
      first_of[i] = f;
    }
  }
  __syncthreads();
  if (i >= P) return;
  const int e = se[i], t = i / k, j = i - t * k;
  // distinct experts below e (the slot) and in all
  int slot = 0, nslots = 0;
  if (masked) {
    for (int w = 0; w < nw; w++) {
      const uint32_t m = emask[w];
      const int c = __popc(m);
      nslots += c;
      slot += w < (e >> 5) ? c : (w == (e >> 5) ? __popc(m & ((1u << (e & 31)) - 1u)) : 0);
    }
  } else {
    for (int a = 0; a < P; a++) {
      nslots += first_of[a];
      slot += first_of[a] & (int)(se[a] < e);
    }
  }
  // pairs before this one in the numbering (experts ascending, tokens ascending), and this
  // expert's tokens before t and in all
  int rank = 0, before = 0, same = 0;
  for (int ta = 0; ta < T; ta++) {
    const int tb = (int)(ta < t);
    for (int c = 0; c < k; c++) {
      const int ea = se[ta * k + c], lt = (int)(ea < e), eq = (int)(ea == e);
      rank += lt | (eq & tb);
      same += eq;
      before += eq & tb;
    }
  }
  int pos = 0;  // this token's pairs of lower experts
  for (int c = 0; c < k; c++) pos += (int)(se[t * k + c] < e);
  plan->slot_tok[slot][before] = t;
  plan->slot_pair[slot][before] = rank;
  plan->tok_pair[t][j] = rank;
  plan->tok_w[t][j] = wts[i];
  plan->comb_pair[t][pos] = rank;
  plan->comb_w[t][pos] = wts[i];
  if (before == 0) {
    plan->slot_expert[slot] = e;
    plan->slot_ntok[slot] = same;
  }
  if (i == 0) plan->nslots = nslots;
}

// Routing and plan in one workgroup of T waves (64 * T threads, at least one per pair): wave t routes token t (unless `route` is 0 and
// sel/wts already hold the choices), then the pairs are numbered (after the barrier every choice
// is visible to the workgroup).
template <int PER>
__global__ __launch_bounds__(64 * MOE_MAX_T) void route_plan_kernel(const float *__restrict__ logits, int T, int n,
                                                                    int k, int renorm, int route, int *__restrict__ sel,
                                                                    float *__restrict__ wts, MoePlan *__restrict__ plan) {
  extern __shared__ __attribute__((aligned(16))) float route_lds[];  // per wave: 128 * PER + 128 floats
  const int t = threadIdx.x >> 6;
  float *mine = route_lds + t * (128 * PER + 128);
  if (route && t < T)
    route_wave<PER>(logits + (int64_t)t * n, n, k, renorm, sel + t * k, wts + t * k, mine, (int *)(mine + 128 * PER),
                    mine + 128 * PER + 64);
  __syncthreads();
  plan_pairs(sel, wts, T, k, n, plan);
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

// The codecs of this unit and the lookup over every unit.
const MoeOps *moe_ops_base(int type) {
  static constexpr MoeOps q4k = moe_ops_of<Q4K>(), q6k = moe_ops_of<Q6K>(), q80 = moe_ops_of<Q80>(),
                          iq4xs = moe_ops_of<IQ4XS>(), iq2xxs = moe_ops_of<IQ2XXS>();
  switch (type) {
    case 12: return &q4k;
    case 14: return &q6k;
    case 8: return &q80;
    case 23: return &iq4xs;
    case 16: return &iq2xxs;
  }
  return nullptr;
}

static const MoeOps *moe_ops(int type) {
  if (const MoeOps *o = moe_ops_base(type)) return o;
  if (const MoeOps *o = moe_ops_k(type)) return o;
  if (const MoeOps *o = moe_ops_32(type)) return o;
  return moe_ops_f(type);
}

template <int NM>
static hipError_t launch_moe_type(int type, const MoeGemvArgs &a, int T, int max_slots, int num_cu, hipStream_t st) {
  const MoeOps *o = moe_ops(type);
  return o ? o->launch[NM - 1](a, T, max_slots, num_cu, st) : hipErrorInvalidValue;
}

static int route_per(int n) { return n <= 64 ? 1 : n <= 128 ? 2 : n <= 256 ? 4 : n <= 512 ? 8 : n <= 1024 ? 16 : 32; }

hipError_t route_launch(const float *logits, int T, int n, int k, int renorm, int *sel, float *wts, float *prob,
                        hipStream_t st) {
  if (n > kRouteWaveMax || k > 64) {  // the wave kernel keeps choice j in lane j
    hipLaunchKernelGGL(route_serial_kernel, dim3((T + 63) / 64), dim3(64), 0, st, logits, T, n, k, renorm, sel, wts,
                       prob);
    return hipGetLastError();
  }
  switch (route_per(n)) {
    case 1: hipLaunchKernelGGL(route_wave_kernel<1>, dim3(T), dim3(64), 0, st, logits, n, k, renorm, sel, wts); break;
    case 2: hipLaunchKernelGGL(route_wave_kernel<2>, dim3(T), dim3(64), 0, st, logits, n, k, renorm, sel, wts); break;
    case 4: hipLaunchKernelGGL(route_wave_kernel<4>, dim3(T), dim3(64), 0, st, logits, n, k, renorm, sel, wts); break;
    case 8: hipLaunchKernelGGL(route_wave_kernel<8>, dim3(T), dim3(64), 0, st, logits, n, k, renorm, sel, wts); break;
    case 16: hipLaunchKernelGGL(route_wave_kernel<16>, dim3(T), dim3(64), 0, st, logits, n, k, renorm, sel, wts); break;
    default: hipLaunchKernelGGL(route_wave_kernel<32>, dim3(T), dim3(64), 0, st, logits, n, k, renorm, sel, wts); break;
  }
  return hipGetLastError();
}

// Dynamic LDS above 64 KB needs the kernel's limit raised once.
template <class K>
static hipError_t raise_route_lds(K *kernel, size_t smem, bool &raised) {
  if (smem > 65536 && !raised) {
    if (hipFuncSetAttribute(reinterpret_cast<const void *>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)smem) != hipSuccess)
      return hipErrorInvalidConfiguration;
    raised = true;
  }
  return hipSuccess;
}

static hipError_t route_plan_launch(const MoeLaunch &m, hipStream_t st) {
  if (m.ne > kRouteWaveMax) {
    hipError_t e = route_launch(m.logits, m.T, m.ne, m.k, m.renorm, m.sel, m.wts, m.prob, st);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(route_plan_kernel<1>, dim3(1), dim3(64 * m.T), 0, st, m.logits, m.T, m.ne, m.k, m.renorm,
                       0, m.sel, m.wts, m.plan);
    return hipGetLastError();
  }
#define WL_RP(P)                                                                                                  \
  {                                                                                                                   \
    static bool raised = false;                                                                                       \
    const size_t smem = (size_t)(128 * P + 128) * 4 * m.T;                                                             \
    if (hipError_t e = raise_route_lds(&route_plan_kernel<P>, smem, raised)) return e;                                \
    hipLaunchKernelGGL(route_plan_kernel<P>, dim3(1), dim3(64 * m.T), smem, st, m.logits, m.T, m.ne, m.k, m.renorm,   \
                       1, m.sel, m.wts, m.plan);                                                                      \
  }
  switch (route_per(m.ne)) {
    case 1: WL_RP(1); break;
    case 2: WL_RP(2); break;
    case 4: WL_RP(4); break;
    case 8: WL_RP(8); break;
    case 16: WL_RP(16); break;
    default: WL_RP(32); break;
  }
#undef WL_RP
  return hipGetLastError();
}

hipError_t moe_launch(const MoeLaunch &m, int num_cu, hipStream_t st) {
  hipError_t err = route_plan_launch(m, st);
  if (err != hipSuccess) return err;
  const int max_slots = m.T * m.k < m.ne ? m.T * m.k : m.ne;
  if (m.gu_int) {
    // MatMul's integer branch for gate and up: the tokens' activations quantized once
    if ((err = quantize_launch(m.x, m.T, m.embd, intdot_needs_k(m.gu_type) ? 1 : 0, m.qx, st)) != hipSuccess) return err;
    if ((err = intdot_moe_launch(m.gu_type, m.gate, m.up, m.gu_row_bytes, (int64_t)m.ff * m.gu_row_bytes, m.ff,
                                 m.embd, m.qx, m.plan, 0, m.T, max_slots, m.h, m.ff, num_cu, st)) != hipSuccess)
      return err;
  } else {
    MoeGemvArgs gu{};
    gu.plan = m.plan;
    gu.w = m.gate; gu.w2 = m.up; gu.row_bytes = m.gu_row_bytes; gu.rows = m.ff; gu.cols = m.embd;
    gu.x = m.x; gu.ldx = m.embd; gu.x_by_pair = 0; gu.y = m.h; gu.ldy = m.ff;
    if ((err = launch_moe_type<2>(m.gu_type, gu, m.T, max_slots, num_cu, st)) != hipSuccess) return err;
  }
  if (m.d_int) {
    // every pair's row of h quantized (each token's k choices are distinct experts, so all
    // T * k rows were written)
    if ((err = quantize_launch(m.h, m.T * m.k, m.ff, intdot_needs_k(m.d_type) ? 1 : 0, m.qh, st)) != hipSuccess)
      return err;
    if ((err = intdot_moe_launch(m.d_type, m.down, nullptr, m.d_row_bytes, (int64_t)m.embd * m.d_row_bytes, m.embd,
                                 m.ff, m.qh, m.plan, 1, m.T, max_slots, m.yd, m.embd, num_cu, st)) != hipSuccess)
      return err;
  } else {
    MoeGemvArgs dn{};
    dn.plan = m.plan;
    dn.w = m.down; dn.w2 = nullptr; dn.row_bytes = m.d_row_bytes; dn.rows = m.embd; dn.cols = m.ff;
    dn.x = m.h; dn.ldx = m.ff; dn.x_by_pair = 1; dn.y = m.yd; dn.ldy = m.embd;
    if ((err = launch_moe_type<1>(m.d_type, dn, m.T, max_slots, num_cu, st)) != hipSuccess) return err;
  }
  const int64_t total = (int64_t)m.T * m.embd;
  hipLaunchKernelGGL(combine_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, m.plan, m.yd, m.T,
                     m.k, m.embd, m.out);
  return hipGetLastError();
}

bool moe_supports(int type) { return moe_ops(type) != nullptr; }

}  // namespace wl
