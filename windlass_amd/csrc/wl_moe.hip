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
#include <climits>

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

template <int PER, bool WT = false>
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
      put<WT>(&sel[lane], lane);
      put<WT>(&wts[lane], __builtin_nanf(""));
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
    put<WT>(&sel[lane], rk_i[lane]);
    put<WT>(&wts[lane], w);
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

template <bool WT = false>
__device__ __forceinline__ void plan_pairs(const int *__restrict__ sel, const float *__restrict__ wts, int T, int k,
                                           int n, MoePlan *__restrict__ plan) {
  // se: the choices, then INT_MAX up to a multiple of 4 (no expert is above or equal to it);
  // emask: experts chosen by any pair, cleared to a multiple of 4 words. Both are read 16 bytes
  // at a time so the reads of a scan are in flight together.
  __shared__ __attribute__((aligned(16))) int se[MOE_MAX_PAIRS + 4];
  __shared__ int first_of[MOE_MAX_PAIRS];              // pair a is the lowest-index pair of its expert
  __shared__ __attribute__((aligned(16))) uint32_t emask[kPlanMaskExperts / 32];
  const int P = T * k, P4 = (P + 3) & ~3, i = threadIdx.x, nw = (n + 31) / 32, nw4 = (nw + 3) & ~3;
  const bool masked = n <= kPlanMaskExperts;
  if (masked)
    for (int w = i; w < nw4; w += blockDim.x) emask[w] = 0;
  if (i < P) se[i] = sel[i];
  else if (i < P4) se[i] = INT_MAX;
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
    const uint4 *m4 = reinterpret_cast<const uint4 *>(emask);
    for (int w0 = 0; w0 < nw4; w0 += 4) {
      const uint4 q = m4[w0 >> 2];
      const uint32_t mv[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int w = w0 + u;
        const int c = __popc(mv[u]);
        nslots += c;
        slot += w < (e >> 5) ? c : (w == (e >> 5) ? __popc(mv[u] & ((1u << (e & 31)) - 1u)) : 0);
      }
    }
  } else {
    for (int a = 0; a < P; a++) {
      nslots += first_of[a];
      slot += first_of[a] & (int)(se[a] < e);
    }
  }
  // pairs before this one in the numbering (experts ascending, tokens ascending), this expert's
  // tokens before t and in all, and this token's pairs of lower experts; pair a is (token ta,
  // choice c)
  int rank = 0, before = 0, same = 0, pos = 0, ta = 0, c = 0;
  const int4 *s4 = reinterpret_cast<const int4 *>(se);
  for (int a0 = 0; a0 < P4; a0 += 4) {
    const int4 q = s4[a0 >> 2];
    const int ev[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int ea = ev[u], tb = (int)(ta < t), lt = (int)(ea < e), eq = (int)(ea == e);
      rank += lt | (eq & tb);
      same += eq;
      before += eq & tb;
      pos += lt & (int)(ta == t);
      if (++c == k) {
        c = 0;
        ta++;
      }
    }
  }
  put<WT>(&plan->slot_tok[slot][before], t);
  put<WT>(&plan->slot_pair[slot][before], rank);
  put<WT>(&plan->tok_pair[t][j], rank);
  put<WT>(&plan->tok_w[t][j], wts[i]);
  put<WT>(&plan->comb_pair[t][pos], rank);
  put<WT>(&plan->comb_w[t][pos], wts[i]);
  if (before == 0) {
    put<WT>(&plan->slot_expert[slot], e);
    put<WT>(&plan->slot_ntok[slot], same);
  }
  if (i == 0) put<WT>(&plan->nslots, nslots);
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

// ------------------------------------------------------------------ one launch for the layer
// Route, plan, gate/up, down and the combine in one launch of G workgroups of eight waves, G no
// more than the device holds at once, so every workgroup is eventually resident while the
// others wait (a bounded wait in any case):
//   phase 1  every workgroup routes the T tokens itself (route_group: route_wave's results
//            with 512 / T threads per token) and numbers the pairs into its LDS; workgroup 0
//            also stores the plan for the host;
//   phase 2  the waves take the gate/up row groups i = gw, gw + 8G, ... of the chosen slots
//            (gw the wave's index in the grid; slot i / groups, group i % groups) and write h;
//            then a grid barrier (16 arrival counters, a count of the complete ones, a flag
//            on 64 replicas);
//   phase 3  workgroup w takes the down row groups w, w + G, ...; its waves take the slots of a
//            group in turn, the slots' rows meet in LDS, and the workgroup adds the tokens'
//            pairs for each row in ascending expert order, as combine_kernel does.
// Each row group is computed by cs_group_wave, whose results are cs_gemv's for a one-wave
// workgroup, as the launch chain runs these shapes: the same bits. h crosses workgroups: it is
// stored at agent scope (written through to the point of coherence), and its readers acquire
// once per CU after the barrier (the polling wave's acquire; the others follow it through the
// workgroup barrier). Every wait is bounded (a.spin polls); one that runs out sets `err`.
struct MoeFusedArgs {
  const float *logits;
  int T, ne, k, renorm;
  MoePlan *plan;
  const uint8_t *gate, *up, *down;
  int64_t gu_row_bytes, d_row_bytes, gu_stride, d_stride;  // bytes per row, per expert
  int ff, embd;
  const float *x;
  float *h, *yd, *out;
  MoeSync *sync;
  int parity, max_slots, spin;
};

constexpr int kMoeWaves = 8;

// Polls *p until it reaches v, then acquires (one cache invalidation, not one per poll). False
// when the patience (spin polls) runs out (err set).
__device__ __forceinline__ bool moe_wait_ge(unsigned *p, unsigned v, MoeSync *sy, int spin) {
  for (int i = 0; i < spin; i++) {
    if (__hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= v) {
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      return true;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  if ((threadIdx.x & 63) == 0) atomicOr(&sy->err[0], 1u);
  return false;
}

// One atomic add by the wave's lane 0; the old value goes to every lane of the wave. The
// caller has made the workgroup's stores visible at agent scope first (every wave waits for its
// agent-scope stores to complete before the workgroup barrier that precedes the arrival).
__device__ __forceinline__ unsigned moe_arrive(unsigned *p) {
  unsigned old = 0;
  if ((threadIdx.x & 63) == 0) old = atomicAdd(p, 1u);
  return __builtin_amdgcn_readfirstlane(old);
}

// Routing of the T tokens by the whole workgroup: G = 512 / T' threads per token (T' = T
// rounded up to a power of two), the same results as route_wave.
//   - The softmax denominator: when every nonzero probability is at least 2^-20, each partial
//     sum of up to 256 of them is a multiple of 2^-43 below 2^9, exact in double, so the sum
//     does not depend on the order and a tree adds it; otherwise one thread adds in index
//     order, as the reference does.
//   - The ranks: an entry's rank (keys above its own) is counted over S slices of the keys by
//     S threads and added in LDS (integers: exact).
constexpr int kRouteMaxN = 256;
struct RouteLds {
  float p[kMoeWaves][kRouteMaxN];     // probabilities by group (a group's rows: G / 64 waves)
  __attribute__((aligned(16))) uint64_t key[kMoeWaves][kRouteMaxN];
  int rank[kMoeWaves][kRouteMaxN];
  double dsum[kMoeWaves * 64 / 64];   // per wave
  float fmax[kMoeWaves];
  int rk_i[kMoeWaves][MOE_MAX_K];
  float rk_w[kMoeWaves][MOE_MAX_K];
  int inexact, nan[kMoeWaves];
};

// wave_max_f / wave_sum_d (wl_device.h): DPP wave reductions. The maximum is exact in any order
// (no NaN reaches it); the denominator's tree only runs when its sum is exact (below).

__device__ void route_group(const float *__restrict__ logits, int T, int n, int k, int renorm, int *__restrict__ sel,
                            float *__restrict__ wts, RouteLds &L) {
  const int tid = threadIdx.x, Tp = T <= 1 ? 1 : T <= 2 ? 2 : T <= 4 ? 4 : 8;
  const int gs = 64 * kMoeWaves / Tp, grp = tid / gs, li = tid % gs, wv = tid >> 6;
  const int wpg = gs / 64, w0 = grp * wpg;  // the group's waves
  const bool act = grp < T;
  const float *l = logits + (int64_t)(act ? grp : 0) * n;
  constexpr int PM = kRouteMaxN / 64;
  float v[PM];
  float mx = -INFINITY;
#pragma unroll
  for (int m = 0; m < PM; m++) {
    const int e = li + gs * m;
    v[m] = act && e < n ? l[e] : -INFINITY;
    if (v[m] > mx) mx = v[m];  // NaN never wins, as in the reference's scan
  }
  mx = wave_max_f(mx);
  if ((tid & 63) == 0) L.fmax[wv] = mx;
  if (tid == 0) L.inexact = 0;
  __syncthreads();
  mx = L.fmax[w0];
  for (int j = 1; j < wpg; j++) {
    const float u = L.fmax[w0 + j];
    if (u > mx) mx = u;
  }
  double part = 0;
  int inexact = 0;
#pragma unroll
  for (int m = 0; m < PM; m++) {
    const int e = li + gs * m;
    if (act && e < n) {
      v[m] = (float)exp((double)(v[m] - mx));
      L.p[grp][e] = v[m];
      part += (double)v[m];
      inexact |= (int)(v[m] != 0.f && !(v[m] >= 0x1p-20f));  // tiny, or NaN
    }
  }
  if (inexact) L.inexact = 1;
  part = wave_sum_d(part);
  if ((tid & 63) == 0) L.dsum[wv] = part;
  __syncthreads();
  double sum = 0;
  if (!L.inexact) {  // uniform over the workgroup
    for (int j = 0; j < wpg; j++) sum += L.dsum[w0 + j];
  } else {  // index order, one thread per group, the result through LDS
    __syncthreads();  // every wave has read its partial sums' slot before it is reused
    if (li == 0 && act) {
      for (int e = 0; e < n; e++) sum += (double)L.p[grp][e];
      L.dsum[w0] = sum;
    }
    __syncthreads();
    sum = L.dsum[w0];
  }
  const float inv = (float)(1.0 / sum);
  int nan = 0;
#pragma unroll
  for (int m = 0; m < PM; m++) {
    const int e = li + gs * m;
    if (act && e < n) {
      v[m] *= inv;
      nan |= (int)(v[m] != v[m]);
      // finite and not negative unless NaN: the bits order like the values; ties to the lower id
      L.key[grp][e] = ((uint64_t)__float_as_uint(v[m]) << 32) | (uint32_t)~e;
      L.rank[grp][e] = 0;
    }
  }
  nan = __any(nan);
  if ((tid & 63) == 0) L.nan[wv] = nan;
  __syncthreads();
  nan = 0;
  for (int j = 0; j < wpg; j++) nan |= L.nan[w0 + j];
  // ranks: the n keys of the group in S slices; unit u = (entry e, slice u / n)
  int np = 1;
  while (np < n) np <<= 1;
  const int S = gs > np ? gs / np : 1, span = (n + S - 1) / S;
  if (!nan && act) {
    for (int u = li; u < n * S; u += gs) {
      const int e = u % n, sl = u / n, j0 = sl * span, j1 = min(n, j0 + span);
      const uint64_t me = L.key[grp][e];
      int c = 0, j = j0;
      for (; j + 8 <= j1 && !(j & 1); j += 8) {  // eight keys per round, the LDS reads in flight together
        const ulonglong2 *k2 = reinterpret_cast<const ulonglong2 *>(&L.key[grp][j]);
        ulonglong2 q[4];
#pragma unroll
        for (int u = 0; u < 4; u++) q[u] = k2[u];
#pragma unroll
        for (int u = 0; u < 4; u++) c += (int)(q[u].x > me) + (int)(q[u].y > me);
      }
      for (; j < j1; j++) c += (int)(L.key[grp][j] > me);
      if (S == 1) L.rank[grp][e] = c;
      else atomicAdd(&L.rank[grp][e], c);
    }
  }
  __syncthreads();
  if (!nan && act) {
#pragma unroll
    for (int m = 0; m < PM; m++) {
      const int e = li + gs * m;
      if (e < n) {
        const int r = L.rank[grp][e];
        if (r < k) {
          L.rk_i[grp][r] = e;
          L.rk_w[grp][r] = v[m];
        }
      }
    }
  }
  __syncthreads();
  if (act && li < k) {
    if (nan) {  // every probability is NaN (through the denominator): the scan's first k entries
      sel[grp * k + li] = li;
      wts[grp * k + li] = __builtin_nanf("");
    } else {
      float chosen = 0;
      for (int c = 0; c < k; c++) chosen += L.rk_w[grp][c];  // in pick order, as the reference adds them
      float w = L.rk_w[grp][li];
      if (renorm) {
        const float div = chosen > WL_MIN_EXPERT_WEIGHT_SUM ? chosen : WL_MIN_EXPERT_WEIGHT_SUM;
        w /= div;
      }
      sel[grp * k + li] = L.rk_i[grp][li];
      wts[grp * k + li] = w;
    }
  }
  __syncthreads();
}

template <class CG, class CD, int TM>
__global__ __launch_bounds__(64 * kMoeWaves) void moe_fused_kernel(MoeFusedArgs a) {
  __shared__ RouteLds s_route;
  __shared__ int s_sel[MOE_MAX_PAIRS];
  __shared__ float s_wts[MOE_MAX_PAIRS];
  __shared__ MoePlan s_plan;
  __shared__ float s_part[kMoeWaves][64];
  __shared__ float s_yd[MOE_MAX_PAIRS * 8];  // a down row group's rows (up to 8) of every pair
  constexpr int RG = TM == 1 ? CG::R1 / 2 : 2, RD = TM == 1 ? CD::R1 : 4;
  MoeSync *sy = a.sync;
  MoeSyncSet &S = sy->set[a.parity];
  const int w = blockIdx.x, G = gridDim.x, tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6), gw = w * kMoeWaves + wv, NW = G * kMoeWaves;

  {  // the other set, for the next launch (the previous launch, which used it, has ended)
    unsigned *o = reinterpret_cast<unsigned *>(&sy->set[a.parity ^ 1]);
    const int n = (int)(sizeof(MoeSyncSet) / sizeof(unsigned));
    for (int i = w * 64 * kMoeWaves + tid; i < n; i += G * 64 * kMoeWaves) o[i] = 0;
  }

  // phase 1: the routing and the plan, in this workgroup's LDS
  route_group(a.logits, a.T, a.ne, a.k, a.renorm, s_sel, s_wts, s_route);
  plan_pairs(s_sel, s_wts, a.T, a.k, a.ne, &s_plan);
  __syncthreads();
  const MoePlan &pl = s_plan;
  if (w == 0) {  // the plan for the host (expert runs)
    const int *src = reinterpret_cast<const int *>(&s_plan);
    int *dst = reinterpret_cast<int *>(a.plan);
    for (int i = tid; i < (int)(sizeof(MoePlan) / 4); i += 64 * kMoeWaves) dst[i] = src[i];
  }
  const int nslots = min(pl.nslots, a.max_slots);

  // phase 2: gate/up
  const int ggu = (a.ff + RG - 1) / RG;
  for (int i = gw; i < nslots * ggu; i += NW) {
    const int s = i / ggu, g = i % ggu;
    const int64_t eoff = (int64_t)pl.slot_expert[s] * a.gu_stride;
    const CsRows W{a.gate + eoff, a.up + eoff, a.gu_row_bytes, a.ff};
    const CsIO io{a.x, pl.slot_tok[s], a.embd, a.h, pl.slot_pair[s], a.ff, pl.slot_ntok[s]};
    cs_group_wave<CG, TM, RG, 2, true>(W, io, a.embd, g, s_part[wv]);
  }
  // every wave's h stores (agent-scope stores, written through to the point of coherence) have
  // completed before the workgroup barrier, so wave 0's arrival below follows all of them: the
  // wave waits for its outstanding memory operations (gfx9's vmcnt counts stores), which is the
  // whole of an agent-scope release for such stores (no cache write-back: nothing the other
  // workgroups read was stored through the cache)
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0), expcnt and lgkmcnt not waited for
  // this wave's first down row group (group w, slot wv): one dword of each of its weights'
  // 128-byte lines, read across the barrier so the lines are in the caches when phase 3 reads them
  const int gd = (a.embd + RD - 1) / RD;
  uint32_t touch = 0;
  {
    const int lpr = (int)((a.d_row_bytes + 127) / 128);  // lines per row
    if (w < gd && wv < nslots && lane < RD * lpr) {
      const int r = min(w * RD + lane / lpr, a.embd - 1);
      const int64_t off = min((int64_t)(lane % lpr) * 128, a.d_row_bytes - 4);
      const uint8_t *row = a.down + (int64_t)pl.slot_expert[wv] * a.d_stride + (int64_t)r * a.d_row_bytes;
      touch = *reinterpret_cast<const uint32_t *>(row + (off & ~(int64_t)3));
    }
  }
  __syncthreads();
  if (wv == 0) {  // grid barrier
    const int nsub = G < MOE_SYNC_SUB ? G : MOE_SYNC_SUB, sub = w % nsub;
    const unsigned per = (unsigned)((G - sub + nsub - 1) / nsub);
    if (moe_arrive(&S.arrive[sub * MOE_SYNC_LINE]) == per - 1 && moe_arrive(&S.top[0]) == (unsigned)nsub - 1)
      __hip_atomic_store(&S.h_ready[lane * MOE_SYNC_LINE], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    moe_wait_ge(&S.h_ready[(w % MOE_SYNC_REP) * MOE_SYNC_LINE], 1u, sy, a.spin);  // acquires for the CU
  }
  __syncthreads();

  // phase 3: row groups g = w, w + G, ... of the down rows; wave v takes the slots v, v + 8, ...,
  // the slots' rows of the group meet in LDS, and the workgroup adds the tokens' pairs for each
  // row in ascending expert order, as combine_kernel does
  for (int g = w; g < gd; g += G) {
    for (int s = wv; s < nslots; s += kMoeWaves) {
      if (g == w && s == wv) asm volatile("" ::"v"(touch));  // the prefetch has landed (long ago)
      const int64_t eoff = (int64_t)pl.slot_expert[s] * a.d_stride;
      const CsRows W{a.down + eoff, nullptr, a.d_row_bytes, a.embd};
      const CsIO io{a.h, pl.slot_pair[s], a.ff, s_yd, pl.slot_pair[s], RD, pl.slot_ntok[s]};
      cs_group_wave<CD, TM, RD, 1, false>(W, io, a.ff, g, s_part[wv], g * RD);
    }
    __syncthreads();
    for (int q = tid; q < RD * a.T; q += 64 * kMoeWaves) {
      const int t = q / RD, r = q % RD;
      if (g * RD + r < a.embd) {
        float o = 0.f;
        for (int j = 0; j < a.k; j++) o += pl.comb_w[t][j] * s_yd[pl.comb_pair[t][j] * RD + r];
        a.out[(int64_t)t * a.embd + g * RD + r] = o;
      }
    }
    __syncthreads();  // s_yd is the next group's
  }
}

__global__ void moe_sync_init_kernel(unsigned *p, int n) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) p[i] = 0;
}

hipError_t moe_sync_init(MoeSync *s, hipStream_t st) {
  hipLaunchKernelGGL(moe_sync_init_kernel, dim3(1), dim3(256), 0, st, reinterpret_cast<unsigned *>(s),
                     (int)(sizeof(MoeSync) / sizeof(unsigned)));
  return hipGetLastError();
}

// The grid: one workgroup per CU (the barrier needs every workgroup resident in the end; the
// kernel is checked once to fit at least one per CU).
template <class CG, class CD, int TM>
static hipError_t moe_fused_go(const MoeFusedArgs &a, int num_cu, hipStream_t st) {
  static int fits = -1;  // per instantiation
  if (fits < 0) {
    int n = 0;
    fits = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, moe_fused_kernel<CG, CD, TM>, 64 * kMoeWaves, 0) ==
               hipSuccess && n >= 1;
  }
  if (!fits) return hipErrorInvalidConfiguration;
  const int g = num_cu;
  hipLaunchKernelGGL((moe_fused_kernel<CG, CD, TM>), dim3((unsigned)g), dim3(64 * kMoeWaves), 0, st, a);
  return hipGetLastError();
}

template <class CG, class CD>
static hipError_t moe_fused_tm(const MoeFusedArgs &a, int num_cu, hipStream_t st) {
  if (a.T <= 1) return moe_fused_go<CG, CD, 1>(a, num_cu, st);
  if (a.T <= 2) return moe_fused_go<CG, CD, 2>(a, num_cu, st);
  if (a.T <= 4) return moe_fused_go<CG, CD, 4>(a, num_cu, st);
  return moe_fused_go<CG, CD, 8>(a, num_cu, st);
}

// Formats and shapes of the one-launch path: gate/up and down in one wave-column each (embd and
// ff up to 2048, whole 256-blocks), Q4_K/Q6_K experts, up to 64 (token, choice) pairs and 256
// experts, float products (IntDot keeps the chain).
bool moe_uses_one_launch(const MoeLaunch &m) {
  int pg, wg, pd, wd;
  cs_shape(m.embd, &pg, &wg);
  cs_shape(m.ff, &pd, &wd);
  const bool types = (m.gu_type == 12 || m.gu_type == 14) && (m.d_type == 12 || m.d_type == 14) &&
                     !(m.gu_type == 14 && m.d_type == 12);
  return m.sync && !m.gu_int && !m.d_int && types && pg == 1 && wg == 1 && pd == 1 && wd == 1 &&
         m.T * m.k <= 64 && m.T <= kMoeWaves && m.ne <= kRouteMaxN;
}

static hipError_t moe_fused_launch(const MoeLaunch &m, int num_cu, hipStream_t st) {
  MoeFusedArgs a{};
  a.logits = m.logits; a.T = m.T; a.ne = m.ne; a.k = m.k; a.renorm = m.renorm;
  a.plan = m.plan;
  a.gate = m.gate; a.up = m.up; a.down = m.down;
  a.gu_row_bytes = m.gu_row_bytes; a.d_row_bytes = m.d_row_bytes;
  a.gu_stride = (int64_t)m.ff * m.gu_row_bytes; a.d_stride = (int64_t)m.embd * m.d_row_bytes;
  a.ff = m.ff; a.embd = m.embd;
  a.x = m.x; a.h = m.h; a.yd = m.yd; a.out = m.out;
  a.sync = m.sync; a.parity = m.parity & 1; a.spin = m.spin < 0 ? 0 : m.spin;
  a.max_slots = m.T * m.k < m.ne ? m.T * m.k : m.ne;
  if (m.gu_type == 12 && m.d_type == 12) return moe_fused_tm<Q4K, Q4K>(a, num_cu, st);
  if (m.gu_type == 12) return moe_fused_tm<Q4K, Q6K>(a, num_cu, st);
  return moe_fused_tm<Q6K, Q6K>(a, num_cu, st);
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
  if (moe_uses_one_launch(m)) return moe_fused_launch(m, num_cu, st);
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
