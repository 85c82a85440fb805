// wl_intmma.hip - the integer-dot path for 2..8 tokens on the int8 matrix cores.
//
// Transformer.MatMul's integer branch (src/Transformer.cs:504-524) for several tokens at once,
// as ForwardBatch runs it (one FastMath.IntDot per (row, token), src/FastMath.cs:105-214). The
// integer sums of FastMath.IntDot are exact, so they may come from any order of products: here
// v_mfma_i32_16x16x32_i8 forms them for 16 rows x 16 tokens x one 32-value run at a time, with
// the weight quants as the A operand and the tokens' 8-bit activations as B. Each row's
// scale terms and the float term of every block are the reference's, and the terms of a row's
// blocks are added in block order, as the reference's `sum +=` does: every (row, token) result is
// bit-identical to FastMath.IntDot, whatever the token count, and to the one-token integer kernel
// (wl_intdot.hip).
//
// Operand layout of v_mfma_i32_16x16x32_i8: lane l holds A[row l%16][k 8*(l/16) .. +7] and
// B[k 8*(l/16) .. +7][token l%16]; the result holds D[row 4*(l/16) + i][token l%16], i < 4. So a
// lane loads the weight bytes of row l%16 (the "A row") and the activations of token l%16, and
// its results are rows 4*(l/16) .. +3 of that token (its "D rows"). Each block's per-row scales
// reach the D rows through a small LDS slab per wave: every A lane decodes two sub-blocks'
// (scale, min) of its row, and every D lane reads the rows it owns.
#include "wl_device.h"
#include "wl_gemv_impl.h"
#include "wl_intdot.h"

#pragma clang fp contract(off)

namespace wl {

typedef int32_t i32x4_t __attribute__((ext_vector_type(4)));

constexpr int kMmaWaves = 4;     // waves per workgroup: one 16-row tile, its blocks in four parts
constexpr int kMmaTokens = 8;    // tokens per launch (of the MFMA's 16 columns)
constexpr int kSlab = 20;        // dwords per row in the scale slab

__device__ __forceinline__ i32x4_t mma(uint2 a, uint2 b, i32x4_t c) {
  return __builtin_amdgcn_mfma_i32_16x16x32_i8((long)__builtin_bit_cast(uint64_t, a),
                                               (long)__builtin_bit_cast(uint64_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ uint2 ld8(const void *p) { return *reinterpret_cast<const uint2 *>(p); }

// ------------------------------------------------------------------------------------ Q4_K
// A lane (q4 = l/16, row l%16) of block b: qs bytes 32j + 8 q4 .. +8 (j < 4) of its row are the
// A operands of sub-blocks 2j (low nibbles) and 2j + 1 (high nibbles). Its slab entries are the
// (scale, min) of sub-blocks 2 q4 and 2 q4 + 1 (get_scale_min_k4, src/Quants.cs:321-330) and
// the row's (d, dmin).
struct MQ4K {
  static constexpr int BYTES = 144, SUBS = 8, TERMS = 1;
  struct Raw { uint4 h; uint2 q[4]; };
  __device__ static void load(const uint8_t *blk, int q4, Raw &r) {
    r.h = *reinterpret_cast<const uint4 *>(blk);
#pragma unroll
    for (int j = 0; j < 4; j++) r.q[j] = ld8(blk + 16 + 32 * j + 8 * q4);
  }
  // the same bytes from a staged copy of the block in LDS (16-byte aligned)
  __device__ static void load_lds(const uint8_t *blk, int q4, Raw &r) {
    r.h = *reinterpret_cast<const uint4 *>(blk);
#pragma unroll
    for (int j = 0; j < 4; j++) r.q[j] = *reinterpret_cast<const uint2 *>(blk + 16 + 32 * j + 8 * q4);
  }
  __device__ static uint2 operand(const Raw &r, int s) {
    const uint2 v = r.q[s >> 1];
    const int sh = 4 * (s & 1);
    return make_uint2((v.x >> sh) & 0x0F0F0F0Fu, (v.y >> sh) & 0x0F0F0F0Fu);
  }
  // slab row: dwords 0..7 scales, 8..15 mins, 16 the (d, dmin) halves
  __device__ static void stage(const Raw &r, int q4, uint32_t *row) {
    uint32_t sc[2], mn[2];
#pragma unroll
    for (int e = 0; e < 2; e++) {
      const int s = 2 * q4 + e, k = 8 * (s & 3);
      const uint32_t Y = (r.h.y >> k) & 0xFF, Z = (r.h.z >> k) & 0xFF, W = (r.h.w >> k) & 0xFF;
      sc[e] = s < 4 ? (Y & 63) : ((W & 0xF) | ((Y >> 6) << 4));
      mn[e] = s < 4 ? (Z & 63) : ((W >> 4) | ((Z >> 6) << 4));
    }
    *reinterpret_cast<uint2 *>(row + 2 * q4) = make_uint2(sc[0], sc[1]);
    *reinterpret_cast<uint2 *>(row + 8 + 2 * q4) = make_uint2(mn[0], mn[1]);
    if (q4 == 0) row[16] = r.h.x;
  }
};

// ------------------------------------------------------------------------------------ Q6_K
// A lane (q4, row) of block b, half hh, 32-value run s' (values 128 hh + 32 s' + 8 q4 .. +8):
// quants ((ql >> 4 (s' >> 1)) & 15) | (((qh >> 2 s') & 3) << 4) from ql bytes
// 64 hh + 32 (s' & 1) + 8 q4 and qh bytes 128 + 32 hh + 8 q4 (src/Quants.cs:381-392). A run holds
// two scale groups of 16 values (lanes q4 < 2 and q4 >= 2), so each run is two products whose B
// operand keeps one group's activations. Slab: the 16 int8 scales as ints, and d.
struct MQ6K {
  static constexpr int BYTES = 210, SUBS = 16, TERMS = 2;
  struct Raw { uint32_t l[2][2][3], h[2][3], s, d, sh; };  // aligned dword windows (2-byte-aligned blocks)
  __device__ static void load(const uint8_t *blk, int q4, Raw &r) {
    gu32 *a = align4_down(blk);
    r.sh = misalign4(blk) * 8;
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
#pragma unroll
      for (int p = 0; p < 2; p++) {
        const int o = (64 * hh + 32 * p + 8 * q4) / 4;
        r.l[hh][p][0] = a[o];
        r.l[hh][p][1] = a[o + 1];
        r.l[hh][p][2] = a[o + 2];
      }
      const int o = (128 + 32 * hh + 8 * q4) / 4;
      r.h[hh][0] = a[o];
      r.h[hh][1] = a[o + 1];
      r.h[hh][2] = a[o + 2];
    }
    r.s = a[(192 + 4 * q4) / 4];
    r.d = a[208 / 4];
    // one extra dword for the scale window when the block is at 2 mod 4
    r.s = __builtin_amdgcn_alignbit(a[(192 + 4 * q4) / 4 + 1], r.s, r.sh);
  }
  __device__ static uint2 win(const uint32_t (&w)[3], uint32_t sh) {
    return make_uint2(__builtin_amdgcn_alignbit(w[1], w[0], sh), __builtin_amdgcn_alignbit(w[2], w[1], sh));
  }
  // quants of run sp (0..3) of half hh
  __device__ static uint2 operand(const Raw &r, int hh, int sp) {
    const uint2 ql = win(r.l[hh][sp & 1], r.sh), qh = win(r.h[hh], r.sh);
    const int s1 = 4 * (sp >> 1), s2 = 2 * sp;
    return make_uint2(((ql.x >> s1) & 0x0F0F0F0Fu) | (((qh.x >> s2) & 0x03030303u) << 4),
                      ((ql.y >> s1) & 0x0F0F0F0Fu) | (((qh.y >> s2) & 0x03030303u) << 4));
  }
  // slab row: dwords 0..15 the scales (sign-extended), 16 the d half
  __device__ static void stage(const Raw &r, int q4, uint32_t *row) {
    const uint32_t s = r.s;
    *reinterpret_cast<uint4 *>(row + 4 * q4) =
        make_uint4((uint32_t)(int)(int8_t)(s & 0xFF), (uint32_t)(int)(int8_t)((s >> 8) & 0xFF),
                   (uint32_t)(int)(int8_t)((s >> 16) & 0xFF), (uint32_t)(int)(int8_t)(s >> 24));
    if (q4 == 0) row[16] = r.sh ? (r.d >> 16) : (r.d & 0xFFFF);
  }
};

struct MmaArgs {
  const uint8_t *w, *w2;  // w2: the up matrix of the SwiGLU pair (NM = 2)
  int64_t row_bytes;
  int rows, cols;
  const int8_t *q;  // token t's quants at q + t * cols
  const float *d;   // token t's block scales at d + t * (cols / 256)
  const int16_t *bs;
  int T;
  float *y;
  int ldy;
  // the same activations in operand order (QActsDev::qf/bf/df), or null
  const int8_t *qf;
  const int16_t *bf;
  const float *df;
};

// A workgroup owns one 16-row tile (of each matrix); wave w walks the w-th quarter of the row's
// blocks in order. Wave 0 adds its blocks' terms as it goes; waves 1..3 leave theirs in LDS
// (the D lanes of the first 8 tokens), and after one barrier wave 0 adds them on in block
// order: the reference's single `sum +=` chain over the whole row.
// Staged weights (Q4_K): a wave reads its tile's 16 rows x kStageBlocks blocks with coalesced
// nontemporal 16-byte loads (every byte once; a wave load covers about two rows' contiguous
// bytes instead of 16 rows' separate lines), one chunk ahead in registers, into its own LDS
// area, and the lanes take their operand bytes from there.
constexpr int kStageBlocks = 2;
constexpr int kStageRow = kStageBlocks * 144 + 16;                          // LDS bytes per row (padded)
constexpr int kStageChunks = 16 * kStageBlocks * 144 / 16;                  // 16-byte chunks of a stage
constexpr int kStageLoads = (kStageChunks + 63) / 64;                       // loads per lane

// FRAG: the activations come from the operand-order copy (one 512-byte wave load per run of 32
// values, 16 tokens' bsums and scales in one 512- and one 64-byte range) instead of the tokens'
// rows (16 tokens' separate lines per wave load). STG: staged weights (Q4_K).
template <class M, int NM, bool FRAG, bool STG = false>
__global__ __launch_bounds__(64 * kMmaWaves) void intmma_kernel(MmaArgs a) {
  __shared__ __attribute__((aligned(16))) uint32_t slab[kMmaWaves][NM][16 * kSlab];
  __shared__ __attribute__((aligned(16))) uint8_t stage[STG ? kMmaWaves : 1][STG ? NM : 1][STG ? 16 * kStageRow : 16];
  extern __shared__ __attribute__((aligned(16))) float4 mma_terms[];  // [3][bw][NM][TERMS][32]
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, q4 = lane >> 4, c16 = lane & 15;
  const int tile = blockIdx.x;  // uniform: the barrier below is reached by every wave
  const int nb = a.cols / 256, bw = (nb + kMmaWaves - 1) / kMmaWaves;
  const int b_lo = min(nb, wv * bw), b_hi = min(nb, b_lo + bw);
  const int dl = q4 * 8 + c16;  // D lane index among the first 8 tokens' lanes
  const int arow = min(tile * 16 + c16, a.rows - 1);  // rows past the end re-read the last row
  const int tok = min(c16, a.T - 1);                    // tokens past T re-read the last token
  const uint8_t *wr[2] = {a.w + (int64_t)arow * a.row_bytes, NM == 2 ? a.w2 + (int64_t)arow * a.row_bytes : nullptr};
  const int8_t *xq = a.q + (int64_t)tok * a.cols + 8 * q4;
  const float *xd = a.d + (int64_t)tok * nb;
  const int16_t *xb = a.bs + (int64_t)tok * (a.cols / 16);

  float sum[NM][4];
#pragma unroll
  for (int m = 0; m < NM; m++)
#pragma unroll
    for (int i = 0; i < 4; i++) sum[m][i] = 0.f;

  // a block's operands: the weight bytes of the tile's rows, the token's quants, bsums and scale
  struct Ops {
    typename M::Raw raw[NM];
    uint2 xs[8];
    uint4 b0, b1;
    float dt;
  };
  auto fetch = [&](int b, Ops &o) {
#pragma unroll
    for (int m = 0; m < NM; m++) M::load(wr[m] + (int64_t)b * M::BYTES, q4, o.raw[m]);
    if constexpr (FRAG) {
#pragma unroll
      for (int s = 0; s < 8; s++) o.xs[s] = ld8(a.qf + (((int64_t)b * 8 + s) * 16 + c16) * 32 + 8 * q4);
      const int16_t *bb = a.bf + ((int64_t)b * 16 + c16) * 16;
      o.b0 = *reinterpret_cast<const uint4 *>(bb);
      o.b1 = *reinterpret_cast<const uint4 *>(bb + 8);
      o.dt = a.df[(int64_t)b * 16 + c16];
    } else {
#pragma unroll
      for (int s = 0; s < 8; s++) o.xs[s] = ld8(xq + (int64_t)b * 256 + 32 * s);
      o.b0 = *reinterpret_cast<const uint4 *>(xb + (int64_t)b * 16);
      o.b1 = *reinterpret_cast<const uint4 *>(xb + (int64_t)b * 16 + 8);
      o.dt = xd[b];
    }
  };
  // blocks b and b + 1 in flight: block b's operands were fetched two blocks earlier
  auto body = [&](const Ops &op, float (&tm)[NM][M::TERMS][4]) {
    const typename M::Raw(&cur)[NM] = op.raw;
    const uint2(&xs)[8] = op.xs;
    const uint4 b0 = op.b0, b1 = op.b1;
    const float dt = op.dt;
    // the slab of this block (the wave's own region; a wave barrier orders it)
#pragma unroll
    for (int m = 0; m < NM; m++) M::stage(cur[m], q4, &slab[wv][m][c16 * kSlab]);
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    // bsums of the token: 16 int16 of the block
    const uint32_t bv[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
    int bsum[16];
#pragma unroll
    for (int g = 0; g < 8; g++) {
      bsum[2 * g] = (int)(int16_t)(bv[g] & 0xFFFF);
      bsum[2 * g + 1] = (int)(int16_t)(bv[g] >> 16);
    }
#pragma unroll
    for (int m = 0; m < NM; m++) {
      if constexpr (M::TERMS == 1) {
        // Q4_K: sumi = sum_s sc_s a_s, summ = sum_s m_s (bsums of the sub-block), one term
        i32x4_t acc[8];
#pragma unroll
        for (int s = 0; s < 8; s++) acc[s] = mma(M::operand(cur[m], s), xs[s], i32x4_t{0, 0, 0, 0});
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const uint32_t *row = &slab[wv][m][(4 * q4 + i) * kSlab];
          const uint4 s0 = *reinterpret_cast<const uint4 *>(row), s1 = *reinterpret_cast<const uint4 *>(row + 4);
          const uint4 m0 = *reinterpret_cast<const uint4 *>(row + 8), m1 = *reinterpret_cast<const uint4 *>(row + 12);
          const uint32_t dd = row[16];
          const int sc[8] = {(int)s0.x, (int)s0.y, (int)s0.z, (int)s0.w, (int)s1.x, (int)s1.y, (int)s1.z, (int)s1.w};
          const int mn[8] = {(int)m0.x, (int)m0.y, (int)m0.z, (int)m0.w, (int)m1.x, (int)m1.y, (int)m1.z, (int)m1.w};
          int sumi = 0, summ = 0;
#pragma unroll
          for (int s = 0; s < 8; s++) {
            // 24-bit products (sc, m < 64; |a| < 2^16; |bsum pair| < 2^12): exact, full rate
            sumi += __mul24(sc[s], acc[s][i]);
            summ += __mul24(mn[s], bsum[2 * s] + bsum[2 * s + 1]);
          }
          const float d = half_lo(dd), dmin = half_hi(dd);
          tm[m][0][i] = dt * (d * (float)sumi - dmin * (float)summ);  // src/FastMath.cs:155
        }
      } else {
        // Q6_K: per half, eight groups of 16: acc_g = sum q x - 32 sum x; part = sum_g sc_g acc_g
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
          i32x4_t acc[8];
#pragma unroll
          for (int sp = 0; sp < 4; sp++) {
            const uint2 wop = M::operand(cur[m], hh, sp), x = xs[4 * hh + sp];
            const uint2 zero = make_uint2(0u, 0u);
            acc[2 * sp] = mma(wop, q4 < 2 ? x : zero, i32x4_t{0, 0, 0, 0});
            acc[2 * sp + 1] = mma(wop, q4 < 2 ? zero : x, i32x4_t{0, 0, 0, 0});
          }
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const uint32_t *row = &slab[wv][m][(4 * q4 + i) * kSlab];
            const uint4 sv = *reinterpret_cast<const uint4 *>(row + 8 * hh),
                        sw = *reinterpret_cast<const uint4 *>(row + 8 * hh + 4);
            const int sc[8] = {(int)sv.x, (int)sv.y, (int)sv.z, (int)sv.w, (int)sw.x, (int)sw.y, (int)sw.z, (int)sw.w};
            int part = 0;
#pragma unroll
            for (int g = 0; g < 8; g++)  // |sc| <= 128, |acc - 32 bsum| < 2^18: 24-bit products, exact
              part += __mul24(sc[g], acc[g][i] - 32 * bsum[8 * hh + g]);
            const float d = half_lo(row[16]);
            tm[m][hh][i] = dt * d * (float)part;  // src/FastMath.cs:209
          }
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  };
  // wave 0 adds a block's terms to the running sums; the others keep them for wave 0
  auto take = [&](int b, const float (&tm)[NM][M::TERMS][4]) {
    if (wv == 0) {
#pragma unroll
      for (int m = 0; m < NM; m++)
#pragma unroll
        for (int h = 0; h < M::TERMS; h++)
#pragma unroll
          for (int i = 0; i < 4; i++) sum[m][i] += tm[m][h][i];
    } else if (c16 < 8) {
      float4 *p = mma_terms + (((int64_t)(wv - 1) * bw + (b - b_lo)) * NM * M::TERMS) * 32 + dl;
#pragma unroll
      for (int m = 0; m < NM; m++)
#pragma unroll
        for (int h = 0; h < M::TERMS; h++)
          p[(m * M::TERMS + h) * 32] = make_float4(tm[m][h][0], tm[m][h][1], tm[m][h][2], tm[m][h][3]);
    }
  };
  if constexpr (STG) {
    // stage loads: chunk f = 64 i + lane of the 16 x kStageBlocks block region is row f / per,
    // 16-byte piece f % per of it (per = kStageBlocks * 9)
    constexpr int per = kStageBlocks * 9;
    int soff[kStageLoads], lofs[kStageLoads];
    bool sok[kStageLoads];
#pragma unroll
    for (int i = 0; i < kStageLoads; i++) {
      const int f = 64 * i + lane, r = f / per, c = f % per;
      sok[i] = f < kStageChunks;
      const int row = min(tile * 16 + r, a.rows - 1);
      soff[i] = 0;
      lofs[i] = r * kStageRow + 16 * c;
      // row offsets fit 32 bits only per tile; the tile's first row is added once below
      soff[i] = (row - min(tile * 16, a.rows - 1)) * (int)a.row_bytes + 16 * c;
    }
    const int64_t tbase = (int64_t)min(tile * 16, a.rows - 1) * a.row_bytes;
    u32x4_t sreg[NM][kStageLoads];
    auto issue = [&](int c0) {  // blocks c0 .. c0 + kStageBlocks - 1 (clamped to the row)
      const int cb = min(c0, nb - kStageBlocks);
#pragma unroll
      for (int m = 0; m < NM; m++) {
        const uint8_t *base = (m ? a.w2 : a.w) + tbase + (int64_t)cb * 144;
#pragma unroll
        for (int i = 0; i < kStageLoads; i++)
          if (sok[i]) sreg[m][i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(base + soff[i]));
      }
      return cb;
    };
    auto commit = [&]() {
      asm volatile("" ::: "memory");
#pragma unroll
      for (int m = 0; m < NM; m++)
#pragma unroll
        for (int i = 0; i < kStageLoads; i++)
          if (sok[i]) *reinterpret_cast<u32x4_t *>(&stage[wv][m][lofs[i]]) = sreg[m][i];
      asm volatile("" ::: "memory");
    };
    struct Xo {
      uint2 xs[8];
      uint4 b0, b1;
      float dt;
    };
    auto fetch_x = [&](int b, Xo &o) {
#pragma unroll
      for (int s = 0; s < 8; s++) o.xs[s] = ld8(a.qf + (((int64_t)b * 8 + s) * 16 + c16) * 32 + 8 * q4);
      const int16_t *bb = a.bf + ((int64_t)b * 16 + c16) * 16;
      o.b0 = *reinterpret_cast<const uint4 *>(bb);
      o.b1 = *reinterpret_cast<const uint4 *>(bb + 8);
      o.dt = a.df[(int64_t)b * 16 + c16];
    };
    auto block = [&](int b, int cb, const Xo &xo) {
      Ops op;
#pragma unroll
      for (int m = 0; m < NM; m++) M::load_lds(&stage[wv][m][c16 * kStageRow + (b - cb) * 144], q4, op.raw[m]);
#pragma unroll
      for (int s = 0; s < 8; s++) op.xs[s] = xo.xs[s];
      op.b0 = xo.b0;
      op.b1 = xo.b1;
      op.dt = xo.dt;
      float tm[NM][M::TERMS][4];
      body(op, tm);
      take(b, tm);
    };
    if (tile * 16 < a.rows && b_lo < b_hi) {
      Xo xr[2];
      int cb = issue(b_lo);
      fetch_x(b_lo, xr[0]);
      if (b_lo + 1 < b_hi) fetch_x(b_lo + 1, xr[1]);
      for (int c = b_lo; c < b_hi; c += kStageBlocks) {
        commit();
        const int cur = cb;
        if (c + kStageBlocks < b_hi) cb = issue(c + kStageBlocks);
        {
          const Xo xo = xr[0];
          if (c + 2 < b_hi) fetch_x(c + 2, xr[0]);
          block(c, cur, xo);
        }
        if (c + 1 < b_hi) {
          const Xo xo = xr[1];
          if (c + 3 < b_hi) fetch_x(c + 3, xr[1]);
          block(c + 1, cur, xo);
        }
      }
    }
  } else if (tile * 16 < a.rows && b_lo < b_hi) {
    Ops ring[2];
    fetch(b_lo, ring[0]);
    if (b_lo + 1 < b_hi) fetch(b_lo + 1, ring[1]);
    for (int b = b_lo; b < b_hi; b += 2) {
      {
        const Ops op = ring[0];
        if (b + 2 < b_hi) fetch(b + 2, ring[0]);
        float tm[NM][M::TERMS][4];
        body(op, tm);
        take(b, tm);
      }
      if (b + 1 < b_hi) {
        const Ops op = ring[1];
        if (b + 3 < b_hi) fetch(b + 3, ring[1]);
        float tm[NM][M::TERMS][4];
        body(op, tm);
        take(b + 1, tm);
      }
    }
  }
  __syncthreads();
  if (wv != 0 || tile * 16 >= a.rows) return;
  // the other quarters' terms, in block order
  if (c16 < 8)
    for (int b = min(nb, bw); b < nb; b++) {
      const float4 *p = mma_terms + (int64_t)(b - bw) * NM * M::TERMS * 32 + dl;
#pragma unroll
      for (int m = 0; m < NM; m++)
#pragma unroll
        for (int h = 0; h < M::TERMS; h++) {
          const float4 v = p[(m * M::TERMS + h) * 32];
          sum[m][0] += v.x;
          sum[m][1] += v.y;
          sum[m][2] += v.z;
          sum[m][3] += v.w;
        }
    }
  if (c16 < a.T) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int row = tile * 16 + 4 * q4 + i;
      if (row < a.rows) {
        float v = sum[0][i];
        if constexpr (NM == 2) v = silu_mul(v, sum[1][i]);
        a.y[(int64_t)c16 * a.ldy + row] = v;
      }
    }
  }
}

// The staged terms of waves 1..3 are the launch's dynamic LDS; rows longer than this allows
// (more than about 200 K of Q6_K values) take the VALU kernel.
constexpr size_t kMmaMaxLds = 96 * 1024;

static size_t mma_lds(int type, int cols, int nm) {
  const int bw = (cols / 256 + kMmaWaves - 1) / kMmaWaves;
  return (size_t)(kMmaWaves - 1) * bw * nm * (type == 14 ? 2 : 1) * 32 * sizeof(float4);
}

bool intmma_supports(int type, int cols, int T, int nm) {
  return (type == 12 || type == 14) && cols > 0 && cols % 256 == 0 && T >= 2 && T <= kMmaTokens &&
         mma_lds(type, cols, nm) <= kMmaMaxLds;
}

int intmma_max_tokens(int type, int cols, int nm) { return intmma_supports(type, cols, 2, nm) ? kMmaTokens : 0; }

template <class M, int NM, bool FRAG, bool STG = false>
static hipError_t go_frag(const MmaArgs &a, int grid, size_t smem, hipStream_t st) {
  static bool raised = false;
  if (smem > 65536 && !raised) {
    if (hipFuncSetAttribute(reinterpret_cast<const void *>(&intmma_kernel<M, NM, FRAG, STG>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMmaMaxLds) != hipSuccess)
      return hipErrorInvalidConfiguration;
    raised = true;
  }
  hipLaunchKernelGGL((intmma_kernel<M, NM, FRAG, STG>), dim3(grid), dim3(64 * kMmaWaves), smem, st, a);
  return hipGetLastError();
}

// Q4_K rows of at least one stage take the staged weights (with the operand-order activations).
template <class M, int NM>
static hipError_t go(const MmaArgs &a, int grid, size_t smem, hipStream_t st) {
  if constexpr (M::BYTES == 144)
    if (a.qf && a.cols / 256 >= kStageBlocks) return go_frag<M, NM, true, true>(a, grid, smem, st);
  return a.qf ? go_frag<M, NM, true>(a, grid, smem, st) : go_frag<M, NM, false>(a, grid, smem, st);
}

hipError_t intmma_launch(int type, const uint8_t *w, const uint8_t *w2, int64_t row_bytes, int rows, int cols,
                         QActsDev qa, int T, float *y, int ldy, hipStream_t st) {
  if (rows <= 0) return hipSuccess;
  if (!intmma_supports(type, cols, T, w2 ? 2 : 1) || !qa.q || !qa.d || !qa.bsums) return hipErrorInvalidValue;
  const MmaArgs a{w, w2, row_bytes, rows, cols, qa.q, qa.d, qa.bsums, T, y, ldy, qa.qf, qa.bf, qa.df};
  const int grid = (rows + 15) / 16;
  const size_t smem = mma_lds(type, cols, w2 ? 2 : 1);
  hipError_t e = hipSuccess;
  if (type == 12) {
    if (w2) e = go<MQ4K, 2>(a, grid, smem, st);
    else e = go<MQ4K, 1>(a, grid, smem, st);
  } else {
    if (w2) e = go<MQ6K, 2>(a, grid, smem, st);
    else e = go<MQ6K, 1>(a, grid, smem, st);
  }
  return e;
}

}  // namespace wl
