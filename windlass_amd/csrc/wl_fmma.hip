// wl_fmma.hip - the float decode GEMV on the matrix cores: Q4_K and Q6_K rows times 1-8 tokens
// of fp32 activations on v_mfma_f32_16x16x32_f16 (Transformer.MatMul / MatMulEach,
// src/Transformer.cs:483-561, float branch), with a token's result independent of how many
// tokens share the launch.
//
// Arithmetic. A token's x is cut into units of 2048 values. Each unit is scaled by a power of
// two f that puts its largest finite |x| in [2^14, 2^15), and split into two fp16 parts,
// hi = fp16(x f) and lo = fp16(x f - hi), which keep 22 significant bits of every value. A weight
// enters the matrix core as an fp16 integer that it represents exactly: Q4_K's n * sc (at most
// 15 * 63), Q6_K's (q - 32) * sl and (q - 32) * sh for the signed scale sc = 16 sh + sl (at most
// 480 and 256 in magnitude). fp16 products are exact in the fp32 accumulator. Per super-block the
// MFMAs accumulate, for 16 rows and 16 columns, the scaled sums over its 256 values; column 2t
// holds token t's hi part, 2t + 1 its lo part. Columns are independent dot products, so a
// token's sums do not depend on the other columns (absent tokens are zero columns). Q4_K's
// minimum term, dmin * sum_j m_j * (sum of x over sub-block j), is a 16x16x4 fp32 MFMA of the
// rows' mins and the sub-block sums of each part. The partial of (row, token, unit) is
// (hi sum + lo sum) / f, and a second launch adds the units in order (SiLU for the gate/up pair,
// the residual add), so every token's bits are the same for T = 1..8.
//
// Layout. A workgroup (eight waves) owns one unit of one matrix: its waves first write the
// tokens' fp16 parts into LDS in the MFMA operand order (64 KB, plus Q4_K's sub-block sums),
// then each wave takes 16-row tiles on its own: lane (q = l / 16, rr = l % 16) reads row rr's
// quarter q of each super-block and feeds the MFMA's B operand; the A operand (16 columns of x
// parts) comes from LDS, one 16-byte read per MFMA, conflict-free.
#include "wl_fmma.h"
#include "wl_gemv_launch.h"

#pragma clang fp contract(off)

namespace wl {

typedef _Float16 fh2 __attribute__((ext_vector_type(2)));
typedef _Float16 fh4 __attribute__((ext_vector_type(4)));
typedef _Float16 fh8 __attribute__((ext_vector_type(8)));
typedef float ff4 __attribute__((ext_vector_type(4)));

constexpr int FM_UNIT = 2048;                        // columns per unit: 8 super-blocks
constexpr int FM_NS = 16;                            // MFMA columns (two per token)
constexpr int FM_XBYTES = 8 * 8 * 4 * FM_NS * 16;    // x parts: [sb][m][q][slot] of 8 halves
constexpr int FM_SBYTES = 8 * 2 * 4 * FM_NS * 4;     // Q4_K sub-block sums: [sb][half][q][slot]
constexpr int FM_WAVES = 8;

__device__ __forceinline__ fh2 as_fh2(uint32_t u) { return __builtin_bit_cast(fh2, u); }
__device__ __forceinline__ uint32_t as_u32(fh2 v) { return __builtin_bit_cast(uint32_t, v); }

// The unit's scale: f = 2^(15 - e) for the largest finite |x| = m 2^e (m in [0.5, 1)), and 1/f;
// both powers of two, clamped to the normal range. An all-zero (or non-finite) unit takes f = 1.
__device__ __forceinline__ void unit_scale(float mx, float &f, float &inv) {
  if (!(mx > 0.f)) {
    f = 1.f;
    inv = 1.f;
    return;
  }
  int e;
  frexpf(mx, &e);
  int s = 15 - e;
  s = s > 126 ? 126 : s;
  f = ldexpf(1.f, s);
  inv = ldexpf(1.f, -s);
}

// One token's parts of one unit, by one wave: lane (sb = l / 8, e = l % 8) reads 32 values,
// the wave takes the largest finite |x|, and the lane writes its values' hi and lo halves to
// their operand slots through C::put. n: valid values of the unit (a multiple of 256).
template <class C>
__device__ __forceinline__ float prep_token(const float *xu, int n, int t, uint8_t *lds) {
  const int lane = threadIdx.x & 63, sb = lane >> 3, e = lane & 7;
  const int off = C::prep_offset(sb, e);
  float v[32];
  if (256 * sb < n) {
    const float4 *src = reinterpret_cast<const float4 *>(xu + off);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float4 a = src[i];
      v[4 * i] = a.x;
      v[4 * i + 1] = a.y;
      v[4 * i + 2] = a.z;
      v[4 * i + 3] = a.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 32; i++) v[i] = 0.f;
  }
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < 32; i++) {
    const float a = fabsf(v[i]);
    m = a < INFINITY ? fmaxf(m, a) : m;  // NaN and infinities take no part
  }
#pragma unroll
  for (int o = 32; o; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  float f, inv;
  unit_scale(m, f, inv);
  _Float16 hi[32], lo[32];
#pragma unroll
  for (int i = 0; i < 32; i++) {
    const float X = v[i] * f;
    hi[i] = (_Float16)X;
    lo[i] = (_Float16)(__builtin_isinf(X) ? 0.f : X - (float)hi[i]);  // an infinity is all hi
  }
  C::put(hi, lo, sb, e, t, lds);
  return inv;
}

// Zero columns of an absent token (slots 2t, 2t + 1) in every operand chunk and sum.
__device__ __forceinline__ void prep_zero(int t, uint8_t *lds) {
  const int lane = threadIdx.x & 63;
  for (int i = lane; i < 8 * 8 * 4; i += 64) {
    *reinterpret_cast<uint4 *>(lds + (int64_t)(i * FM_NS + 2 * t) * 16) = make_uint4(0, 0, 0, 0);
    *reinterpret_cast<uint4 *>(lds + (int64_t)(i * FM_NS + 2 * t + 1) * 16) = make_uint4(0, 0, 0, 0);
  }
  float *S = reinterpret_cast<float *>(lds + FM_XBYTES);
  for (int i = lane; i < 8 * 2 * 4; i += 64) {
    S[i * FM_NS + 2 * t] = 0.f;
    S[i * FM_NS + 2 * t + 1] = 0.f;
  }
}

// ------------------------------------------------------------------------------------ Q4_K
// Quarter q of a super-block is sub-block pair q: qs bytes 32q..32q+31, whose low nibbles are
// values 64q + i and high nibbles 64q + 32 + i (src/Quants.cs:333-351). MFMA m takes the lane's
// qs dword m (bytes 4m..4m+3 of the pair) as the values 64q + {4m, 4m+2, 4m+1, 4m+3} and
// 64q + 32 + {4m, 4m+2, 4m+1, 4m+3}: each fp16 pair is (dword & mask) | 0x6400 (1024 + n or
// 1024 + 16n) times the sub-block scale minus 1024 sc, one packed FMA, exact.
struct FQ4K {
  static constexpr int BYTES = 144;
  struct Raw { uint4 h, q0, q1; };

  __device__ static int prep_offset(int sb, int e) { return 256 * sb + 32 * e; }
  // lane (sb, e): sub-block e of super-block sb, i.e. pair e / 2, half e % 2
  __device__ static void put(const _Float16 (&hi)[32], const _Float16 (&lo)[32], int sb, int e, int t,
                             uint8_t *lds) {
    const int q = e >> 1, h = e & 1;
    float shi = 0.f, slo = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) {
      shi += (float)hi[i];
      slo += (float)lo[i];
    }
#pragma unroll
    for (int m = 0; m < 8; m++) {
      const fh4 a = {hi[4 * m], hi[4 * m + 2], hi[4 * m + 1], hi[4 * m + 3]};
      const fh4 b = {lo[4 * m], lo[4 * m + 2], lo[4 * m + 1], lo[4 * m + 3]};
      uint8_t *c = lds + (int64_t)(((sb * 8 + m) * 4 + q) * FM_NS + 2 * t) * 16 + 8 * h;
      *reinterpret_cast<fh4 *>(c) = a;
      *reinterpret_cast<fh4 *>(c + 16) = b;
    }
    float *S = reinterpret_cast<float *>(lds + FM_XBYTES);
    S[((sb * 2 + h) * 4 + q) * FM_NS + 2 * t] = shi;
    S[((sb * 2 + h) * 4 + q) * FM_NS + 2 * t + 1] = slo;
  }

  __device__ static void load(const uint8_t *blk, int q, Raw &r) {
    r.h = ldw16(blk);
    r.q0 = ldw16(blk + 16 + 32 * q);
    r.q1 = ldw16(blk + 32 + 32 * q);
  }

  // acc (columns 4q..4q+3 of row rr) += d * sum(n * sc * x) - dmin * sum_j m_j * S_j
  __device__ static void step(const Raw &r, int q, int rr, const uint8_t *lds, int sb, ff4 &acc) {
    const uint4 h = r.h;
    const int k = 16 * (q & 1);
    // get_scale_min_k4 (src/Quants.cs:321-330) for sub-blocks 2q, 2q + 1
    const uint32_t S = q < 2 ? (h.y & 0x3F3F3F3Fu) : ((h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u));
    const uint32_t M = q < 2 ? (h.z & 0x3F3F3F3Fu) : (((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u));
    const float sclo = (float)((S >> k) & 0xFF), schi = (float)((S >> (k + 8)) & 0xFF);
    const float mlo = (float)((M >> k) & 0xFF), mhi = (float)((M >> (k + 8)) & 0xFF);
    const _Float16 a = (_Float16)sclo, b = (_Float16)(schi * 0.0625f);
    const fh2 sl = {a, a}, nl = {(_Float16)(-1024.f * sclo), (_Float16)(-1024.f * sclo)};
    const fh2 sh = {b, b}, nh = {(_Float16)(-64.f * schi), (_Float16)(-64.f * schi)};
    const uint32_t qd[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
    const uint8_t *xs = lds + (int64_t)sb * 8 * 4 * FM_NS * 16;
    ff4 C = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < 8; m++) {
      const uint32_t D = qd[m], D8 = D >> 8;
      const fh2 p0 = __builtin_elementwise_fma(as_fh2((D & 0x000F000Fu) | 0x64006400u), sl, nl);
      const fh2 p1 = __builtin_elementwise_fma(as_fh2((D8 & 0x000F000Fu) | 0x64006400u), sl, nl);
      const fh2 p2 = __builtin_elementwise_fma(as_fh2((D & 0x00F000F0u) | 0x64006400u), sh, nh);
      const fh2 p3 = __builtin_elementwise_fma(as_fh2((D8 & 0x00F000F0u) | 0x64006400u), sh, nh);
      const fh8 bv = {p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
      const fh8 av = *reinterpret_cast<const fh8 *>(xs + (int64_t)((m * 4 + q) * FM_NS + rr) * 16);
      C = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, C, 0, 0, 0);
    }
    const float *Ss = reinterpret_cast<const float *>(lds + FM_XBYTES) + (int64_t)sb * 2 * 4 * FM_NS;
    ff4 Mn = {0.f, 0.f, 0.f, 0.f};
    Mn = __builtin_amdgcn_mfma_f32_16x16x4f32(Ss[(0 * 4 + q) * FM_NS + rr], mlo, Mn, 0, 0, 0);
    Mn = __builtin_amdgcn_mfma_f32_16x16x4f32(Ss[(1 * 4 + q) * FM_NS + rr], mhi, Mn, 0, 0, 0);
    const float d = half_lo(h.x), dmin = half_hi(h.x);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      acc[i] = __builtin_fmaf(d, C[i], acc[i]);
      acc[i] = __builtin_fmaf(-dmin, Mn[i], acc[i]);
    }
  }
};

// ------------------------------------------------------------------------------------ Q6_K
// Quarter q = 2hh + ih of a super-block: half hh (128 values), i in [16 ih, 16 ih + 16) of its
// four 32-value groups g, whose 6-bit values are ql[64hh + i] (g 0, 2: low, high nibble) or
// ql[64hh + 32 + i] (g 1, 3) with bits 2g..2g+1 of qh[32hh + i], scale sc[8hh + ih + 2g]
// (src/Quants.cs:373-395). MFMA m = 2g + p takes values 128hh + 32g + 16ih + 8p + 0..7 in order;
// each byte pair becomes (1024 + q) halves by one byte permute, then two packed FMAs give
// (q - 32) sl and (q - 32) sh for the two accumulators.
struct FQ6K {
  static constexpr int BYTES = 210;
  struct Raw { Win<16> l1, l2, qh; Win<8> sc; uint32_t dw; };  // sc: the half's 8 scales

  __device__ static int prep_offset(int sb, int e) { return 256 * sb + 128 * (e >> 2) + 32 * (e & 3); }
  // lane (sb, e): group g = e % 4 of half hh = e / 4, 32 values -> quarters 2hh + ih, MFMAs 2g + p
  __device__ static void put(const _Float16 (&hi)[32], const _Float16 (&lo)[32], int sb, int e, int t,
                             uint8_t *lds) {
    const int hh = e >> 2, g = e & 3;
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const int ih = c >> 1, p = c & 1, o = 8 * c;
      const fh8 a = {hi[o], hi[o + 1], hi[o + 2], hi[o + 3], hi[o + 4], hi[o + 5], hi[o + 6], hi[o + 7]};
      const fh8 b = {lo[o], lo[o + 1], lo[o + 2], lo[o + 3], lo[o + 4], lo[o + 5], lo[o + 6], lo[o + 7]};
      uint8_t *ch = lds + (int64_t)(((sb * 8 + 2 * g + p) * 4 + 2 * hh + ih) * FM_NS + 2 * t) * 16;
      *reinterpret_cast<fh8 *>(ch) = a;
      *reinterpret_cast<fh8 *>(ch + 16) = b;
    }
  }

  __device__ static void load(const uint8_t *blk, int q, Raw &r) {
    const int hh = q >> 1, ih = q & 1;
    r.l1.load(blk + 64 * hh + 16 * ih);
    r.l2.load(blk + 64 * hh + 32 + 16 * ih);
    r.qh.load(blk + 128 + 32 * hh + 16 * ih);
    r.sc.load(blk + 192 + 8 * hh);
    r.dw = ldw4(align4_down(blk) + 52);  // d: low half (block at 0 mod 4) or high half (2 mod 4)
  }

  __device__ static void step(const Raw &r, int q, int rr, const uint8_t *lds, int sb, ff4 &acc) {
    const int ih = q & 1;
    const uint32_t K64 = 0x64646464u;
    const uint8_t *xs = lds + (int64_t)sb * 8 * 4 * FM_NS * 16;
    ff4 Cl = {0.f, 0.f, 0.f, 0.f}, Ch = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const uint32_t sw = r.sc.dw(g >> 1);
      const int sc = (int)(int8_t)(sw >> (8 * (ih + 2 * (g & 1))));
      const int sl = sc & 15, shv = sc >> 4;
      const _Float16 a = (_Float16)(float)sl, na = (_Float16)(float)(-1056 * sl);
      const _Float16 b = (_Float16)(float)shv, nb = (_Float16)(float)(-1056 * shv);
      const fh2 SL = {a, a}, NL = {na, na}, SH = {b, b}, NH = {nb, nb};
#pragma unroll
      for (int p = 0; p < 2; p++) {
        uint32_t v[2];
#pragma unroll
        for (int i = 0; i < 2; i++) {
          const uint32_t L = (g & 1) ? r.l2.dw(2 * p + i) : r.l1.dw(2 * p + i), H = r.qh.dw(2 * p + i);
          // the four 6-bit values of bytes 4i..4i+3 (src/Quants.cs:384-387)
          if (g == 0) v[i] = (L & 0x0F0F0F0Fu) | ((H << 4) & 0x30303030u);
          else if (g == 1) v[i] = (L & 0x0F0F0F0Fu) | ((H << 2) & 0x30303030u);
          else if (g == 2) v[i] = ((L >> 4) & 0x0F0F0F0Fu) | (H & 0x30303030u);
          else v[i] = ((L >> 4) & 0x0F0F0F0Fu) | ((H >> 2) & 0x30303030u);
        }
        // (1024 + q) halves of bytes (0, 1) and (2, 3)
        const uint32_t P[4] = {__builtin_amdgcn_perm(K64, v[0], 0x04010400u), __builtin_amdgcn_perm(K64, v[0], 0x04030402u),
                               __builtin_amdgcn_perm(K64, v[1], 0x04010400u), __builtin_amdgcn_perm(K64, v[1], 0x04030402u)};
        fh2 wl[4], wh[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
          wl[j] = __builtin_elementwise_fma(as_fh2(P[j]), SL, NL);
          wh[j] = __builtin_elementwise_fma(as_fh2(P[j]), SH, NH);
        }
        const fh8 bl = {wl[0][0], wl[0][1], wl[1][0], wl[1][1], wl[2][0], wl[2][1], wl[3][0], wl[3][1]};
        const fh8 bh = {wh[0][0], wh[0][1], wh[1][0], wh[1][1], wh[2][0], wh[2][1], wh[3][0], wh[3][1]};
        const fh8 av = *reinterpret_cast<const fh8 *>(xs + (int64_t)(((2 * g + p) * 4 + q) * FM_NS + rr) * 16);
        Cl = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bl, Cl, 0, 0, 0);
        Ch = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bh, Ch, 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);  // one group's operands live at a time
    }
    const float d = half_lo(r.l1.sh ? (r.dw >> 16) : r.dw);
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i] = __builtin_fmaf(d, __builtin_fmaf(16.f, Ch[i], Cl[i]), acc[i]);
  }
};

// ------------------------------------------------------------------------------------ kernel
// Loads in flight per wave: PF work items (one matrix's super-block) ahead of the one computed,
// as many as the register budget (128 VGPRs, four waves per SIMD) holds without spilling.
#ifndef WL_FMMA_PF_Q4K
#define WL_FMMA_PF_Q4K 1
#endif
#ifndef WL_FMMA_PF_Q6K
#define WL_FMMA_PF_Q6K 1
#endif
template <class C, int NM>
constexpr int fmma_ahead() {
  return NM == 2 ? 1 : C::BYTES == 144 ? WL_FMMA_PF_Q4K : WL_FMMA_PF_Q6K;
}

template <class C>
__device__ __forceinline__ void fmma_prep(const BatchArgs &a, uint8_t *lds, float *inv) {
  const int wv = threadIdx.x >> 6, u = blockIdx.y;
  const int n = a.cols - u * FM_UNIT < FM_UNIT ? a.cols - u * FM_UNIT : FM_UNIT;
  if (wv < a.T) {
    const float iv = prep_token<C>(a.x + (int64_t)wv * a.ldx + (int64_t)u * FM_UNIT, n, wv, lds);
    if ((threadIdx.x & 63) == 0) inv[wv] = iv;
  } else {
    prep_zero(wv, lds);
  }
}

// One workgroup's work: the tokens' x parts of its unit into LDS, then the tiles of one matrix
// (pair): wave wv takes tiles wgx * 8 + wv, + nwg * 8, .... The unit's items (super-block b,
// matrix m, in that order) are computed with the loads of the next PF items in flight; the
// first tile's first loads are issued before the x parts are prepared.
template <class C, int NM>
__device__ __forceinline__ void fmma_body(const BatchArgs &a, const BatchMat &M, int wgx, int nwg, uint8_t *lds,
                                          float *inv) {
  constexpr int PF = fmma_ahead<C, NM>();
  // a ring of PF + 1 load buffers; a loop body of K items keeps every buffer's role and every
  // item's matrix fixed at compile time. Past the last item the last one is re-read (valid
  // memory, unused), so every load is issued and the load counters' waits stay exact.
  constexpr int K = (PF + 1) % NM == 0 ? PF + 1 : (PF + 1) * NM;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int q = lane >> 4, rr = lane & 15, u = blockIdx.y;
  const int rem = (a.cols - u * FM_UNIT) / 256;
  const int nsb = rem < 8 ? rem : 8, NI = nsb * NM;
  const int ntiles = (M.rows + 15) / 16, first = wgx * FM_WAVES + wv;
  const uint8_t *wr[NM];
  auto rows_of = [&](int tile) {
    const int row = min(tile * 16 + rr, M.rows - 1);
    wr[0] = M.w + (int64_t)row * M.row_bytes + (int64_t)u * 8 * C::BYTES;
    if constexpr (NM == 2) wr[1] = M.w2 + (int64_t)row * M.row_bytes + (int64_t)u * 8 * C::BYTES;
  };
  typename C::Raw rg[PF + 1];
  auto preload = [&]() {
#pragma unroll
    for (int i = 0; i < PF; i++) {
      const int j = i < NI ? i : NI - 1;
      C::load(wr[i % NM] + (int64_t)(j / NM) * C::BYTES, q, rg[i]);
    }
  };
  if (first < ntiles) {
    rows_of(first);
    preload();
  }
  fmma_prep<C>(a, lds, inv);
  __syncthreads();
  for (int tile = first; tile < ntiles; tile += nwg * FM_WAVES) {
    if (tile != first) {
      rows_of(tile);
      preload();
    }
    ff4 acc[NM];
#pragma unroll
    for (int m = 0; m < NM; m++) acc[m] = ff4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
    for (int base = 0; base < NI; base += K) {
#pragma unroll
      for (int k = 0; k < K; k++) {
        const int i = base + k;
        if (i < NI) {  // uniform
          const int j = i + PF < NI ? i + PF : NI - 1;
          C::load(wr[(k + PF) % NM] + (int64_t)(j / NM) * C::BYTES, q, rg[(k + PF) % (PF + 1)]);
          C::step(rg[k % (PF + 1)], q, rr, lds, i / NM, acc[k % NM]);
        }
      }
    }
    const int r = tile * 16 + rr;
    if (r < M.rows) {
      const int t0 = 2 * q, t1 = 2 * q + 1;
#pragma unroll
      for (int m = 0; m < NM; m++) {
        float *pm = M.part + (int64_t)m * a.T * M.rows * a.u;
        if (t0 < a.T) pm[((int64_t)t0 * M.rows + r) * a.u + u] = (acc[m][0] + acc[m][1]) * inv[t0];
        if (t1 < a.T) pm[((int64_t)t1 * M.rows + r) * a.u + u] = (acc[m][2] + acc[m][3]) * inv[t1];
      }
    }
  }
}

// KINDS: the formats present (1: Q4_K, 2: Q6_K, 3: both, the fused q/k/v of a Q4_K_M layer);
// a kernel holds only the codecs it needs, so each stays within its register budget.
template <int NM, int KINDS>
__global__ __launch_bounds__(64 * FM_WAVES) __attribute__((amdgpu_waves_per_eu(4))) void fmma_kernel(BatchArgs a) {
  __shared__ float inv[FM_WAVES];
  uint8_t *lds = wl_dyn_lds;
  const int mi = batch_mat(a);
  const BatchMat &M = a.m[mi];
  const int wgx = (int)blockIdx.x - M.wg_begin, nwg = batch_nwg(a, mi);
  const bool q4 = KINDS == 1 || (KINDS == 3 && M.type == 12);  // uniform over the workgroup
  if constexpr (KINDS & 1)
    if (q4) fmma_body<FQ4K, NM>(a, M, wgx, nwg, lds, inv);
  if constexpr ((KINDS & 2) != 0)
    if (!q4) fmma_body<FQ6K, NM>(a, M, wgx, nwg, lds, inv);
}

template <int NM, int KINDS>
static hipError_t fmma_launch(const BatchArgs &a, int gx, size_t smem, hipStream_t st) {
  static bool raised = false;
  hipError_t e = raise_lds(&fmma_kernel<NM, KINDS>, smem, raised);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((fmma_kernel<NM, KINDS>), dim3(gx, a.u), dim3(64 * FM_WAVES), smem, st, a);
  return hipGetLastError();
}

// ------------------------------------------------------------------------------------ host
bool fmma_supports(int type) { return type == 12 || type == 14; }

bool fmma_applies(const GemvMat *mats, int nmat, int nm, int cols) {
  if (nmat < 1 || nmat > GEMV_MAX_MATS || cols <= 0 || cols % 256) return false;
  for (int i = 0; i < nmat; i++) {
    if (!fmma_supports(mats[i].type) || mats[i].rows <= 0) return false;
    if (nm == 2 && (!mats[i].w2 || mats[i].type != mats[0].type)) return false;
  }
  return true;
}

static int fmma_units(int cols) { return (cols + FM_UNIT - 1) / FM_UNIT; }

int64_t fmma_scratch_floats(const GemvMat *mats, int nmat, int nm, int cols, int T) {
  int64_t n = 0;
  for (int i = 0; i < nmat; i++) n += (int64_t)fmma_units(cols) * nm * T * mats[i].rows;
  return n;
}

hipError_t fmma_run(const GemvMat *mats, int nmat, int nm, const float *x, int ldx, int cols, int T,
                    float *scratch, int num_cu, hipStream_t st) {
  if (!fmma_applies(mats, nmat, nm, cols) || T < 1 || T > 8 || !scratch || num_cu < 1) return hipErrorInvalidValue;
  BatchArgs a{};
  a.u = fmma_units(cols);
  a.S = 1;
  a.W = a.u;
  a.nmat = nmat;
  a.cols = cols;
  a.x = x;
  a.ldx = ldx;
  a.T = T;
  // one round of two resident workgroups per CU: tiles per wave so that the grid covers every
  // (matrix, unit) tile once, then workgroups per matrix in proportion to its tiles
  int64_t tiles = 0;
  for (int i = 0; i < nmat; i++) tiles += (mats[i].rows + 15) / 16;
  const int64_t waves = (int64_t)num_cu * 2 * FM_WAVES;
  int64_t tpw = (tiles * a.u + waves - 1) / waves;
  if (tpw < 1) tpw = 1;
  float *part = scratch;
  int gx = 0;
  for (int i = 0; i < nmat; i++) {
    const GemvMat &m = mats[i];
    a.m[i] = BatchMat{m.w, m.w2, m.row_bytes, part, m.y, m.ldy, m.rows, m.type, gx, m.add, m.rs};
    part += (int64_t)a.u * nm * T * m.rows;
    const int64_t t = (m.rows + 15) / 16;
    gx += (int)((t + FM_WAVES * tpw - 1) / (FM_WAVES * tpw));
  }
  const size_t smem = FM_XBYTES + FM_SBYTES;
  int kinds = 0;
  for (int i = 0; i < nmat; i++) kinds |= mats[i].type == 12 ? 1 : 2;
  hipError_t e;
  if (nm == 2) e = kinds == 1 ? fmma_launch<2, 1>(a, gx, smem, st) : fmma_launch<2, 2>(a, gx, smem, st);
  else if (kinds == 1) e = fmma_launch<1, 1>(a, gx, smem, st);
  else if (kinds == 2) e = fmma_launch<1, 2>(a, gx, smem, st);
  else e = fmma_launch<1, 3>(a, gx, smem, st);
  if (e != hipSuccess) return e;
  return nm == 1 ? launch_batch_combine<1>(a, st) : launch_batch_combine<2>(a, st);
}

}  // namespace wl
