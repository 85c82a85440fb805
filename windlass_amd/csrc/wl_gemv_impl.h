// wl_gemv_impl.h - the column-stationary decode GEMV body shared by every GEMV launch.
//
// Work decomposition. A row of nb blocks is covered by P passes of NWV waves (P = ceil(nb /
// (8*BPW)), NWV = ceil(nb / (P*BPW)) <= 8, BPW = blocks per wave); in pass p, wave w, lane l
// owns block column b = (p*NWV + w)*BPW + l/LPB, slice l%LPB, of EVERY row. For one token and
// at most two passes (cols <= 32768) the lane's x slices are read once for the whole launch
// and stay in registers. The workgroup walks row groups of R rows with a stride of gridDim; for
// each group every lane reads its slice of the R rows (one coalesced read per row and wave),
// forms its partial dot per (row, token), the wave folds its 64 partials with one fixed
// exchange butterfly, and wave 0 adds the waves' results in wave order.
//
// Summation order of y[t][r] (fixed, independent of T, R and the launch's other rows):
//   lane partial  = sum over passes of the codec's dot on that lane's slice
//   wave partial  = pairwise tree over lanes (i, i^32), then (i, i^16), ..., (i, i^1)
//   y             = ((wave 0 + wave 1) + wave 2) + ...
// so a token's result is bit-identical whatever the token count or row grouping.
#pragma once
#include "wl_codecs.h"

namespace wl {

#ifndef WL_GEMV_MAX_WAVES
#define WL_GEMV_MAX_WAVES 8
#endif
#ifndef WL_GEMV_WAVES_PER_CU
#define WL_GEMV_WAVES_PER_CU 32
#endif
constexpr int kColsPerWave = 2048;                // every codec: 64/LPB blocks of BLOCK values per wave
constexpr int kMaxWaves = WL_GEMV_MAX_WAVES;      // waves per workgroup (the kernels' launch bound)
constexpr int kWavesPerCu = WL_GEMV_WAVES_PER_CU;  // grid target: resident waves per CU

// Passes and waves for a row of `cols` values (the same for every token count).
__host__ __device__ inline void cs_shape(int cols, int *passes, int *waves) {
  const int units = (cols + kColsPerWave - 1) / kColsPerWave;  // wave-columns needed
  const int p = (units + kMaxWaves - 1) / kMaxWaves;
  *passes = p < 1 ? 1 : p;
  *waves = (units + *passes - 1) / *passes;
  if (*waves < 1) *waves = 1;
}

// SiLU(g) * u as src/Transformer.cs:247 writes it: g / (1 + exp(-g)) * u, the exponential in
// double (Math.Exp) cast to float. Compiled without contraction by every includer.
__device__ __forceinline__ float silu_mul(float g, float u) {
  return g / (1.0f + (float)exp((double)(-g))) * u;
}

// The residual add x += o * rs (src/Transformer.cs:224,231) on a product's result: a product
// and a sum, never fused into one rounding.
__device__ __forceinline__ float add_scaled(float x, float v, float rs) {
#pragma clang fp contract(off)
  return x + v * rs;
}

// The partner exchanges of the folding tree. Bits 5 and 4 pair lane l with l^32 and l^16
// through the permlane swaps, which deliver both partners' values in one instruction; bits 3..0
// use DPP: l^8 (row_ror:8), l^7 within each eight lanes (row_half_mirror), l^2 and l^1
// (quad_perm). Every partner flips the level's bit, so bit BIT of a lane still says which half
// of the values it keeps.
template <int BIT>
__device__ __forceinline__ float dpp_partner(float x) {
  constexpr int ctrl = BIT == 3 ? 0x128 : BIT == 2 ? 0x141 : BIT == 1 ? 0x4E : 0xB1;
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), ctrl, 0xF, 0xF, false));
}

// Lanes with bit BIT clear return a + (partner's a), the others b + (partner's b).
template <int BIT>
__device__ __forceinline__ float exch_pair(float a, float b, int lane) {
  if constexpr (BIT == 5) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  } else if constexpr (BIT == 4) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  } else {
    const bool hi = (lane >> BIT) & 1;
    const float send = hi ? a : b, keep = hi ? b : a;
    return keep + dpp_partner<BIT>(send);
  }
}

// Folds V = 2^k values per lane over the 64 lanes. Lane l returns the full sum of value
// index (l >> (6-k)): the first k levels exchange halves of the value set between partner
// lanes (bits 5, 4, ...), the rest fold the one remaining value. Every value is added over the
// same pairwise tree (one pair per level), whatever V is.
template <int V, int BIT>
__device__ __forceinline__ float exch_reduce(const float *v, int lane) {
  if constexpr (V == 1) {
    float q = v[0];
    if constexpr (BIT >= 0) {
      q = exch_pair<BIT>(q, q, lane);
      return exch_reduce<1, BIT - 1>(&q, lane);
    }
    return q;
  } else {
    float u[V / 2];
#pragma unroll
    for (int k = 0; k < V / 2; k++) u[k] = exch_pair<BIT>(v[k], v[k + V / 2], lane);
    return exch_reduce<V / 2, BIT - 1>(u, lane);
  }
}

constexpr int ilog2(int v) { return v <= 1 ? 0 : 1 + ilog2(v / 2); }

// One matrix set of a launch: rows of w (and of w2 for the SwiGLU pair, NM == 2).
struct CsRows {
  const uint8_t *w, *w2;
  int64_t row_bytes;
  int rows;
};

// Activations: token t reads x + (xrow ? xrow[t] : t) * ldx; results go to
// y[(yrow ? yrow[t] : t) * ldy + r]. For the SwiGLU pair, y2 non-null keeps the two sums
// apart (gate to y, up to y2, same indexing) for a later combine instead of applying SiLU.
struct CsIO {
  const float *x;
  const int *xrow;
  int64_t ldx;
  float *y;
  const int *yrow;
  int64_t ldy;
  int T;
  float *y2;
  int add;  // y += result * rs
  float rs;
};

// Row groups whose wave results are buffered in LDS between two barriers.
#ifndef WL_GEMV_GROUPS_PER_SYNC
#define WL_GEMV_GROUPS_PER_SYNC 4
#endif
constexpr int GS = WL_GEMV_GROUPS_PER_SYNC;

// Dynamic LDS of a launch: the codec tables (NEED_LDS 1), then the double-buffered wave partials.
template <class C>
constexpr size_t dyn_table_bytes() {
  return C::NEED_LDS == 1 ? sizeof(Lds) : 0;
}
template <class C, int TM, int R, int NM>
inline size_t cs_lds_bytes(int nwv) {
  return dyn_table_bytes<C>() + sizeof(float) * 2 * GS * nwv * NM * R * TM;
}

// The codec's tables: static LDS (NEED_LDS 2) or the start of the dynamic LDS.
template <class C>
__device__ __forceinline__ Lds &tables_of(uint8_t *lds_raw) {
  if constexpr (C::NEED_LDS == 2) return codec_lds();
  else return *reinterpret_cast<Lds *>(lds_raw);
}

// The weights of row group g for block column b: R rows of each of the NM matrices. Rows past
// the end re-read the last row (valid memory); their results are dropped.
template <class C, int R, int NM>
__device__ __forceinline__ void cs_load(const CsRows &W, int g, int b, const typename C::Lane &L,
                                        typename C::Raw (&raw)[NM][R]) {
  // the row's base is uniform and the lane's offset a 32-bit value, so the loads can take a
  // scalar base address with a vector offset (no 64-bit address arithmetic per row)
  const uint32_t off = (uint32_t)b * (uint32_t)C::BYTES;
#pragma unroll
  for (int m = 0; m < NM; m++)
#pragma unroll
    for (int r = 0; r < R; r++) {
      const int row = min(g * R + r, W.rows - 1);
      const uint8_t *rowp = (m ? W.w2 : W.w) + (int64_t)row * W.row_bytes;
      C::load(rowp + off, L, raw[m][r]);
    }
}

// Where the wave results of the buffered groups go, and which group the buffer starts at.
struct CsSlots {
  int buf, slot, gfirst;
};

// Folds row group g's lane partials over the wave into LDS slot `slot` of buffer `buf`. Every
// GS groups (and after the last) one barrier, then wave 0 finishes the buffered groups while
// the other waves go on into the other buffer. g and the slot state are uniform over the
// workgroup, so every wave takes the same branches.
// A store another workgroup reads in the same launch (WT): written through to the device's
// point of coherence (an agent-scope store), so the reader needs no cache write-back from the
// writer. Otherwise a plain store.
template <bool WT, class V>
__device__ __forceinline__ void put(V *p, V v) {
  if constexpr (WT) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else *p = v;
}

template <int TM, int R, int NM, bool WT = false>
__device__ __forceinline__ void cs_finish(const float (&acc)[NM][R][TM], int g, int gstride, int ngroups,
                                          CsSlots &st, float *part, const CsRows &W, const CsIO &io) {
  constexpr int V = NM * R * TM;
  constexpr int LOW = 6 - ilog2(V);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nwv = blockDim.x >> 6;
  // value index v = (m*TM + t)*R + r
  float vals[V];
#pragma unroll
  for (int m = 0; m < NM; m++)
#pragma unroll
    for (int t = 0; t < TM; t++)
#pragma unroll
      for (int r = 0; r < R; r++) vals[(m * TM + t) * R + r] = acc[m][r][t];
  const float q = exch_reduce<V, 5>(vals, lane);
  if ((lane & ((1 << LOW) - 1)) == 0) part[((st.buf * GS + st.slot) * nwv + wv) * V + (lane >> LOW)] = q;
  if (st.slot + 1 < GS && g + gstride < ngroups) {
    st.slot++;
    return;
  }
  __syncthreads();
  if (wv == 0) {
    for (int i = lane; i < (st.slot + 1) * R * TM; i += 64) {
      const int sl = i / (R * TM), rt = i % (R * TM);
      const int r = rt % R, t = rt / R;
      const int row = (st.gfirst + sl * gstride) * R + r;
      if (t < io.T && row < W.rows) {
        const float *pb = part + (st.buf * GS + sl) * nwv * V;
        float s = pb[t * R + r];
        for (int w = 1; w < nwv; w++) s += pb[w * V + t * R + r];
        const int64_t o = (int64_t)(io.yrow ? io.yrow[t] : t) * io.ldy + row;
        if constexpr (NM == 2) {
          float s1 = pb[(TM + t) * R + r];
          for (int w = 1; w < nwv; w++) s1 += pb[w * V + (TM + t) * R + r];
          if (io.y2) {
            io.y2[o] = s1;
          } else {
            s = silu_mul(s, s1);
          }
        }
        put<WT>(&io.y[o], io.add ? add_scaled(io.y[o], s, io.rs) : s);
      }
    }
  }
  st.buf ^= 1;
  st.slot = 0;
  st.gfirst = g + gstride;
}

// SP: passes whose x slices stay in registers (0: x read per row group; 1 or 2 only for TM 1).
// PIPE (one token, one pass): the next row group's weights are loaded while the current one is
// computed; the same sums in the same order.
template <class C, int TM, int R, int NM, int SP, bool WT = false, bool PIPE = false>
__device__ __forceinline__ void cs_gemv(const CsRows &W, const CsIO &io, int cols, int g0, int gstride,
                                        uint8_t *lds_raw) {
  constexpr int V = NM * R * TM;
  static_assert((1 << ilog2(V)) == V && V <= 64, "partials per lane must be a power of two <= 64");
  static_assert(SP == 0 || TM == 1, "stationary x slices are for one token");
  constexpr int BPW = 64 / C::LPB;
  const Lds &lds = tables_of<C>(lds_raw);
  float *part = reinterpret_cast<float *>(lds_raw + dyn_table_bytes<C>());
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nwv = blockDim.x >> 6;
  const int sub = lane % C::LPB, bslot = lane / C::LPB;
  const typename C::Lane L = C::lane(sub);
  const int nb = cols / C::BLOCK;
  const int npass = (nb + nwv * BPW - 1) / (nwv * BPW);
  const int ngroups = (W.rows + R - 1) / R;

  const float *xr[TM];
#pragma unroll
  for (int t = 0; t < TM; t++) xr[t] = io.x + (int64_t)(io.xrow ? io.xrow[t < io.T ? t : 0] : t) * io.ldx;

  CsSlots st{0, 0, g0};

  // x slices of the stationary passes, read once
  typename C::Xs xs0[SP > 0 ? SP : 1];
#pragma unroll
  for (int p = 0; p < SP; p++) {
    const int b = (p * nwv + wv) * BPW + bslot;
    if (b < nb) C::load_x(xr[0] + (int64_t)b * C::BLOCK, L, xs0[p]);
  }

  if constexpr (C::NEED_LDS) {
    C::init_lds(tables_of<C>(lds_raw));
    __syncthreads();
  }

  if constexpr (PIPE) {
    static_assert(TM == 1 && SP == 1, "the pipelined loop is for one token in one pass");
    // Every load is issued (past the last group it re-reads the last one; a lane past the
    // row's blocks reads block 0 and adds nothing), so the load counter's waits stay exact: a
    // conditional load makes the compiler wait for every load in flight.
    const int b = wv * BPW + bslot;
    const bool bok = b < nb;
    const int bl = bok ? b : 0;
    typename C::Raw ra[NM][R], rb[NM][R];
    auto group = [&](int g, const typename C::Raw(&raw)[NM][R]) {
      float acc[NM][R][TM];
#pragma unroll
      for (int m = 0; m < NM; m++)
#pragma unroll
        for (int r = 0; r < R; r++) acc[m][r][0] = 0.f;
      if (bok) {
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
          for (int r = 0; r < R; r++) {
            typename C::W w;
            C::unpack(raw[m][r], L, lds, w);
            acc[m][r][0] += C::dot(w, xs0[0]);
          }
      }
      cs_finish<TM, R, NM, WT>(acc, g, gstride, ngroups, st, part, W, io);
    };
    if (g0 < ngroups) {
      cs_load<C, R, NM>(W, g0, bl, L, ra);
      for (int g = g0; g < ngroups; g += 2 * gstride) {
        cs_load<C, R, NM>(W, min(g + gstride, ngroups - 1), bl, L, rb);
        group(g, ra);
        if (g + gstride >= ngroups) break;  // uniform over the workgroup
        cs_load<C, R, NM>(W, min(g + 2 * gstride, ngroups - 1), bl, L, ra);
        group(g + gstride, rb);
      }
    }
    return;
  }

  for (int g = g0; g < ngroups; g += gstride) {
    float acc[NM][R][TM];
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
      for (int r = 0; r < R; r++)
#pragma unroll
        for (int t = 0; t < TM; t++) acc[m][r][t] = 0.f;

    for (int p = 0; p < npass; p++) {
      const int b = (p * nwv + wv) * BPW + bslot;
      if (b < nb) {
        typename C::Raw raw[NM][R];
        cs_load<C, R, NM>(W, g, b, L, raw);
        if constexpr (TM == 1) {
          typename C::Xs xs;
          if constexpr (SP == 1) xs = xs0[0];
          else if constexpr (SP == 2) xs = p == 0 ? xs0[0] : xs0[1];
          else C::load_x(xr[0] + (int64_t)b * C::BLOCK, L, xs);
#pragma unroll
          for (int m = 0; m < NM; m++)
#pragma unroll
            for (int r = 0; r < R; r++) {
              typename C::W w;
              C::unpack(raw[m][r], L, lds, w);
              acc[m][r][0] += C::dot(w, xs);
            }
        } else {
          typename C::W w[NM][R];
#pragma unroll
          for (int m = 0; m < NM; m++)
#pragma unroll
            for (int r = 0; r < R; r++) C::unpack(raw[m][r], L, lds, w[m][r]);
#pragma unroll
          for (int t = 0; t < TM; t++) {
            if (t < io.T) {
              typename C::Xs xs;
              C::load_x(xr[t] + (int64_t)b * C::BLOCK, L, xs);
#pragma unroll
              for (int m = 0; m < NM; m++)
#pragma unroll
                for (int r = 0; r < R; r++) acc[m][r][t] += C::dot(w[m][r], xs);
            }
          }
        }
      }
    }
    cs_finish<TM, R, NM, WT>(acc, g, gstride, ngroups, st, part, W, io);
  }
}

// Row group g of W (R rows of each of the NM matrices, all cols up to one wave-column: 64 / LPB
// blocks) by one wave, with nothing shared with the other waves of its workgroup: the lanes'
// partials as cs_gemv forms them (the same unpack and dot), folded by the same tree and added
// across nothing (one wave), so each result has cs_gemv's bits for a one-wave workgroup.
// cs_group_load issues the group's weight loads (they may be in flight across other work);
// cs_group_finish takes them from there. `part` is the wave's own LDS scratch of NM * R * TM
// floats. WT: agent-scope stores (read by another workgroup in the same launch). Results go to
// io.y[yrow * ldy + row - row0] (row0: where io.y's rows start, e.g. an LDS tile of the group).
template <class C, int R, int NM>
__device__ __forceinline__ void cs_group_load(const CsRows &W, int cols, int g, typename C::Raw (&raw)[NM][R]) {
  const int lane = threadIdx.x & 63;
  const int b = lane / C::LPB;
  if (b < cols / C::BLOCK) cs_load<C, R, NM>(W, g, b, C::lane(lane % C::LPB), raw);
}

template <class C, int TM, int R, int NM, bool WT>
__device__ __forceinline__ void cs_group_finish(const CsRows &W, const CsIO &io, int cols, int g, float *part,
                                                const typename C::Raw (&raw)[NM][R], int row0 = 0) {
  constexpr int V = NM * R * TM;
  constexpr int LOW = 6 - ilog2(V);
  static_assert(!C::NEED_LDS, "codecs with LDS tables run through cs_gemv");
  const Lds &lds = *reinterpret_cast<const Lds *>(part);  // unused by these codecs
  const int lane = threadIdx.x & 63;
  const int sub = lane % C::LPB, b = lane / C::LPB;
  const typename C::Lane L = C::lane(sub);
  float acc[NM][R][TM];
#pragma unroll
  for (int m = 0; m < NM; m++)
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
      for (int t = 0; t < TM; t++) acc[m][r][t] = 0.f;
  if (b < cols / C::BLOCK) {
    typename C::W wv[NM][R];
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
      for (int r = 0; r < R; r++) C::unpack(raw[m][r], L, lds, wv[m][r]);
#pragma unroll
    for (int t = 0; t < TM; t++) {
      if (t < io.T) {
        const float *xr = io.x + (int64_t)(io.xrow ? io.xrow[t] : t) * io.ldx;
        typename C::Xs xs;
        C::load_x(xr + (int64_t)b * C::BLOCK, L, xs);
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
          for (int r = 0; r < R; r++) acc[m][r][t] += C::dot(wv[m][r], xs);
      }
    }
  }
  float vals[V];
#pragma unroll
  for (int m = 0; m < NM; m++)
#pragma unroll
    for (int t = 0; t < TM; t++)
#pragma unroll
      for (int r = 0; r < R; r++) vals[(m * TM + t) * R + r] = acc[m][r][t];
  const float q = exch_reduce<V, 5>(vals, lane);
  if ((lane & ((1 << LOW) - 1)) == 0) part[lane >> LOW] = q;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  for (int i = lane; i < R * TM; i += 64) {
    const int r = i % R, t = i / R;
    const int row = g * R + r;
    if (t < io.T && row < W.rows) {
      float v = part[t * R + r];
      if constexpr (NM == 2) v = silu_mul(v, part[(TM + t) * R + r]);
      put<WT>(&io.y[(int64_t)(io.yrow ? io.yrow[t] : t) * io.ldy + row - row0], v);
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();  // part is reused by the wave's next group
}

template <class C, int TM, int R, int NM, bool WT>
__device__ __forceinline__ void cs_group_wave(const CsRows &W, const CsIO &io, int cols, int g, float *part,
                                              int row0 = 0) {
  typename C::Raw raw[NM][R];
  cs_group_load<C, R, NM>(W, cols, g, raw);
  cs_group_finish<C, TM, R, NM, WT>(W, io, cols, g, part, raw, row0);
}

}  // namespace wl
