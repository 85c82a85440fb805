// wl_intmma.hip - the integer-dot path for 2..8 tokens on the int8 matrix cores.
//
// Transformer.MatMul's integer branch (src/Transformer.cs:504-524) for several tokens at once,
// as ForwardBatch runs it (one FastMath.IntDot per (row, token), src/FastMath.cs:105-214). The
// integer sums of FastMath.IntDot are exact, so they may come from any order of products: here
// v_mfma_i32_16x16x32_i8 forms them for 16 rows x 16 columns x one 32-value run at a time, with
// the weight quants as the A operand and the tokens' 8-bit activations as B. Each row's scale
// terms and the float term of every block are the reference's, and the terms of a row's blocks
// are added in block order, as the reference's `sum +=` does: every (row, token) result is
// bit-identical to FastMath.IntDot, whatever the token count, and to the one-token integer kernel
// (wl_intdot.hip).
//
// Operand layout of v_mfma_i32_16x16x32_i8: lane l holds A[row l%16][k 8*(l/16) .. +7] and
// B[k 8*(l/16) .. +7][column l%16]; the result holds D[row 4*(l/16) + i][column l%16], i < 4. So
// a lane loads the weight bytes of row l%16 (its "A row") and one column's activations, and its
// results are rows 4*(l/16) .. +3 of that column (its "D rows"). Each block's per-row scales reach
// the D rows through a small LDS slab per wave: the A lanes decode their row's scales into it,
// and the D lanes read the rows they own.
//
// Sums the matrix cores take over from the VALU (all exact in int32):
//   Q4_K  summ = sum_s m_s * (bsums of sub-block s) = sum_k m_s(k) * x_k: one more product per run
//         with every A byte the run's min, accumulated over the block's eight runs;
//   Q6_K  acc_g = sum (q - 32) x = sum q x + sum (-32) x: a second product per run with every A
//         byte -32, accumulated onto the first.
// Q6_K's scale groups are 16 values, two per run: columns 0..7 carry tokens 0..7 with the run's
// first group (the other group's B bytes read a zero slot) and columns 8..15 the same tokens with
// the second group, so one product serves both groups and a lane adds its partner column's
// scaled sums (integers, any order) to complete a half's `part`.
#include "wl_device.h"
#include "wl_gemv_impl.h"
#include "wl_intdot.h"

#pragma clang fp contract(off)

namespace wl {

typedef int32_t i32x4_t __attribute__((ext_vector_type(4)));

constexpr int kMmaTokens = 8;  // tokens per launch (of the MFMA's 16 columns)
constexpr int kSlab = 20;      // dwords per row in the scale slab

__device__ __forceinline__ i32x4_t mma(uint2 a, uint2 b, i32x4_t c) {
  return __builtin_amdgcn_mfma_i32_16x16x32_i8((long)__builtin_bit_cast(uint64_t, a),
                                               (long)__builtin_bit_cast(uint64_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ uint2 ld8(const void *p) { return *reinterpret_cast<const uint2 *>(p); }

// ------------------------------------------------------------------------------------ Q4_K
// A lane (q4 = l/16, row l%16) of block b: qs bytes 32j + 8 q4 .. +8 (j < 4) of its row are the
// A operands of sub-blocks 2j (low nibbles) and 2j + 1 (high nibbles); the header gives the
// sub-blocks' 6-bit scales and mins (get_scale_min_k4, src/Quants.cs:321-330).
struct MQ4K {
  static constexpr int BYTES = 144, TERMS = 1;
  static constexpr int SCH = 9, SROW = 176;  // staging: 16-byte pieces per row, LDS bytes per row
  struct Raw { uint4 h; uint2 q[4]; };
  // the lane's bytes from a staged copy of the block in LDS (16-byte aligned)
  __device__ static void load_lds(const uint8_t *blk, const uint8_t *, int q4, Raw &r) {
    r.h = *reinterpret_cast<const uint4 *>(blk);
#pragma unroll
    for (int j = 0; j < 4; j++) r.q[j] = *reinterpret_cast<const uint2 *>(blk + 16 + 32 * j + 8 * q4);
  }
  // the B slot of lane (q4, c16): its column's token (slots 8..15 are zero, their results unused)
  __device__ static int slot(int, int c16) { return c16; }
  __device__ static uint2 operand(const Raw &r, int s) {
    const uint2 v = r.q[s >> 1];
    const int sh = 4 * (s & 1);
    return make_uint2((v.x >> sh) & 0x0F0F0F0Fu, (v.y >> sh) & 0x0F0F0F0Fu);
  }
  // the eight mins as bytes: sub-blocks 0..3 are the low 6 bits of header bytes 8..11, 4..7 the
  // high nibbles of bytes 12..15 with the top two bits of bytes 8..11
  __device__ static void mins(const Raw &r, uint32_t &m03, uint32_t &m47) {
    m03 = r.h.z & 0x3F3F3F3Fu;
    m47 = ((r.h.w >> 4) & 0x0F0F0F0Fu) | ((r.h.z >> 2) & 0x30303030u);
  }
  // slab row: dwords 0..7 the scales of sub-blocks 0..7, 8 the (d, dmin) halves; lane q4 writes
  // sub-blocks 2 q4 and 2 q4 + 1 (scales 0..3: the low 6 bits of header bytes 4..7; 4..7: the
  // low nibbles of bytes 12..15 with the top two bits of bytes 4..7)
  __device__ static void stage(const Raw &r, int q4, uint32_t *row) {
    const uint32_t sb = q4 < 2 ? (r.h.y & 0x3F3F3F3Fu) : ((r.h.w & 0x0F0F0F0Fu) | ((r.h.y >> 2) & 0x30303030u));
    const int k = 16 * (q4 & 1);
    *reinterpret_cast<uint2 *>(row + 2 * q4) = make_uint2((sb >> k) & 0xFF, (sb >> (k + 8)) & 0xFF);
    if (q4 == 0) row[8] = r.h.x;
  }
};

// ------------------------------------------------------------------------------------ Q6_K
// A lane (q4, row) of block b, half hh, 32-value run s' (values 128 hh + 32 s' + 8 q4 .. +8):
// quants ((ql >> 4 (s' >> 1)) & 15) | (((qh >> 2 s') & 3) << 4) from ql bytes
// 64 hh + 32 (s' & 1) + 8 q4 and qh bytes 128 + 32 hh + 8 q4 (src/Quants.cs:381-392).
struct MQ6K {
  static constexpr int BYTES = 210, TERMS = 2;
  // staging: 224 bytes from the dword at or below the block's start (the block and its offset
  // of 0 or 2 bytes); LDS rows of 240 bytes put the 16 rows' reads in distinct banks
  static constexpr int SCH = 14, SROW = 240;
  struct Raw { uint32_t l[2][2][3], h[2][3], s, d, sh; };  // aligned dword windows (2-byte-aligned blocks)
  // the lane's dword windows from a staged copy in LDS whose first dword is the one at or below
  // the global block gblk's start; sh = the block's offset in bits (0 or 16)
  __device__ static void load_lds(const uint8_t *row, const uint8_t *gblk, int q4, Raw &r) {
    const uint32_t *a = reinterpret_cast<const uint32_t *>(row);
    r.sh = misalign4(gblk) * 8;
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
    r.d = a[208 / 4];
    r.s = __builtin_amdgcn_alignbit(a[(192 + 4 * q4) / 4 + 1], a[(192 + 4 * q4) / 4], r.sh);
  }
  // A run's values 0..15 (lanes q4 < 2) are one scale group and 16..31 (q4 >= 2) the next:
  // column c16 < 8 is token c16 with the first group, c16 >= 8 token c16 - 8 with the second;
  // a lane whose values belong to the other group reads a zero slot (8..15: at most 8 tokens)
  __device__ static int slot(int q4, int c16) { return ((q4 >= 2) == (c16 >= 8)) ? (c16 & 7) : (c16 | 8); }
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
  // slab row: group g = 2 sp + s of half hh (scale byte 8 hh + g, sign-extended) at dword
  // 8 hh + 4 s + sp, so the four scales a D lane of group s needs per half are one 16-byte read;
  // 16 the d half. Lane q4 holds scale bytes 4 q4 .. +3: half q4 >> 1, g = 4 (q4 & 1) + e.
  __device__ static void stage(const Raw &r, int q4, uint32_t *row) {
    const uint32_t s = r.s;
    const int o = 8 * (q4 >> 1) + 2 * (q4 & 1);
    const uint32_t e0 = (uint32_t)(int)(int8_t)(s & 0xFF), e1 = (uint32_t)(int)(int8_t)((s >> 8) & 0xFF),
                   e2 = (uint32_t)(int)(int8_t)((s >> 16) & 0xFF), e3 = (uint32_t)(int)(int8_t)(s >> 24);
    *reinterpret_cast<uint2 *>(row + o) = make_uint2(e0, e2);      // s = 0: sp, sp + 1
    *reinterpret_cast<uint2 *>(row + o + 4) = make_uint2(e1, e3);  // s = 1
    if (q4 == 0) row[16] = r.sh ? (r.d >> 16) : (r.d & 0xFFFF);
  }
};

struct MmaArgs {
  const uint8_t *w, *w2;  // w2: the up matrix of the SwiGLU pair (NM = 2)
  int64_t row_bytes;
  int rows, cols;
  // the activations in operand order (QActsDev::qf/df): per 256-block b, qf[b][run][slot][32]
  // and df[b][slot], slots past T zero; or null, and the tokens' rows q [T][cols], d [T][cols/256]
  const int8_t *qf;
  const float *df;
  const int8_t *q;
  const float *d;
  int T;
  float *y;
  int ldy;
};

// A workgroup owns one 16-row tile (of each matrix). Its W waves take the row's blocks in rounds:
// in round r wave w takes block r W + w, its loads issued one round ahead. Each block's terms
// (for the 8 token columns: 16 rows x 8 tokens x TERMS floats per matrix) go to an LDS ring of
// two groups of RPS rounds; after a group's barrier every wave adds the group's terms, in block
// order, for its share of the (row, token) pairs: the reference's single `sum +=` chain over
// the whole row.
// Staged weights: a wave reads its block's 16 rows (per matrix) with coalesced nontemporal
// 16-byte loads, one round ahead, into its own LDS area, and the lanes take their operand bytes
// from there. A wave load covers about four to seven rows' contiguous bytes, where an operand
// load touches sixteen rows' lines: for Q6_K's 2-byte-aligned windows the L1 cache's accesses
// (TCP_TOTAL_CACHE_ACCESSES) were 694 per block and wave, close to one per cycle.

// FRAG: the operand-order copy (one 512-byte wave load per run); otherwise the tokens' rows.
// The kernel's LDS: the scale slabs, the terms ring of two groups of RPS rounds (MH floats per
// (row, token) and block: matrices x terms per block), and the staged weights.
template <int W, int NM, int MH, int RPS, int SROW>
struct MmaLds {
  uint32_t slab[W][NM][16 * kSlab];
  float4 terms[2 * RPS][W][MH][32];
  uint8_t stg[W][NM][16 * SROW];
};

// Tile `tile` of a (every wave of the workgroup calls it: it holds workgroup barriers).
template <class M, int NM, int W, bool FRAG, int RPS, class L>
__device__ __forceinline__ void mma_tile(const MmaArgs &a, const int tile, L &lds) {
  auto &slab = lds.slab;
  auto &terms = lds.terms;
  auto &stg = lds.stg;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, q4 = lane >> 4, c16 = lane & 15;
  const int nb = a.cols / 256, nr = (nb + W - 1) / W;
  const int arow = min(tile * 16 + c16, a.rows - 1);  // rows past the end re-read the last row
  const uint8_t *wr[2] = {a.w + (int64_t)arow * a.row_bytes, NM == 2 ? a.w2 + (int64_t)arow * a.row_bytes : nullptr};
  // FRAG: slot M::slot's quants at xq + (8 b + run) * 512, its scale at xd + 16 b; rows: token
  // tok's at xq + 256 b + 32 run and xd + b, and a lane of the other Q6_K group takes zeros
  const int slot = M::slot(q4, c16), tok = min(c16 & 7, a.T - 1);
  const bool xzero = !FRAG && slot >= 8 && M::TERMS == 2;
  const int8_t *xq = FRAG ? a.qf + slot * 32 + 8 * q4 : a.q + (int64_t)tok * a.cols + 8 * q4;
  const float *xd = FRAG ? a.df + (c16 & 7) : a.d + (int64_t)tok * (a.cols / 256);
  const int dl = q4 * 8 + c16;                                 // D lane among the token columns (c16 < 8)

  // staging: piece f = 64 i + lane of a block's 16 rows is row f / 9, bytes 16 (f % 9) ..
  // piece f = 64 i + lane is row f / SCH, bytes 16 (f % SCH) .. of the row's staged range
  constexpr int SCH = M::SCH, SCHUNKS = 16 * M::SCH, SLOADS = (SCHUNKS + 63) / 64;
  int soff[SLOADS], lofs[SLOADS];
  bool sok[SLOADS];
#pragma unroll
  for (int i = 0; i < SLOADS; i++) {
    const int f = 64 * i + lane, r = f / SCH, c = f % SCH;
    sok[i] = f < SCHUNKS;
    soff[i] = (min(tile * 16 + r, a.rows - 1) - tile * 16) * (int)a.row_bytes + 16 * c;  // tile*16 < rows
    lofs[i] = r * M::SROW + 16 * c;
  }
  const int64_t tbase = (int64_t)tile * 16 * a.row_bytes;

  struct Xo {
    uint2 xs[8];
    float dt;
  };
  auto fetch_x = [&](int b, Xo &o) {
    if constexpr (FRAG) {
#pragma unroll
      for (int s = 0; s < 8; s++) o.xs[s] = ld8(xq + ((int64_t)b * 8 + s) * 512);
      o.dt = xd[(int64_t)b * 16];
    } else {
#pragma unroll
      for (int s = 0; s < 8; s++) o.xs[s] = xzero ? make_uint2(0u, 0u) : ld8(xq + (int64_t)b * 256 + 32 * s);
      o.dt = xd[b];
    }
  };
  struct Ops {
    u32x4_t sg[NM][SLOADS];
    Xo x;
  };
  auto fetch = [&](int b, Ops &o) {
#pragma unroll
    for (int m = 0; m < NM; m++) {
      const uint8_t *base = (m ? a.w2 : a.w) + tbase + (int64_t)b * M::BYTES;
#pragma unroll
      for (int i = 0; i < SLOADS; i++)
        if (sok[i]) {
          // Q6_K blocks start 2-byte aligned: pieces from the dword at or below the row's block
          // start (16 c keeps the low bits), dword-aligned loads
          const uint8_t *p = base + soff[i];
          if constexpr (M::BYTES % 4 != 0) p -= misalign4(p);
          o.sg[m][i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4a4_t *>(p));
        }
    }
    fetch_x(b, o.x);
  };

  // one block's terms into ring slot buf
  auto body = [&](const Ops &op, const Xo &xo, int buf, int b) {
    // the staged pieces to this wave's LDS area (its previous block's reads are done: one
    // wave's LDS accesses complete in order), then each lane's operand bytes from there
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
      for (int i = 0; i < SLOADS; i++)
        if (sok[i]) *reinterpret_cast<u32x4_t *>(&stg[wv][m][lofs[i]]) = op.sg[m][i];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    typename M::Raw raw[NM];
#pragma unroll
    for (int m = 0; m < NM; m++) M::load_lds(&stg[wv][m][c16 * M::SROW], wr[m] + (int64_t)b * M::BYTES, q4, raw[m]);
#pragma unroll
    for (int m = 0; m < NM; m++) M::stage(raw[m], q4, &slab[wv][m][c16 * kSlab]);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const i32x4_t zero = {0, 0, 0, 0};
#pragma unroll
    for (int m = 0; m < NM; m++) {
      if constexpr (M::TERMS == 1) {
        // Q4_K: sumi = sum_s sc_s a_s (VALU), summ by the matrix cores
        i32x4_t acc[8], accm = zero;
        uint32_t m03, m47;
        M::mins(raw[m], m03, m47);
#pragma unroll
        for (int s = 0; s < 8; s++) {
          acc[s] = mma(M::operand(raw[m], s), xo.xs[s], zero);
          const uint32_t mb = __builtin_amdgcn_perm(s < 4 ? m03 : m47, s < 4 ? m03 : m47, 0x01010101u * (s & 3));
          accm = mma(make_uint2(mb, mb), xo.xs[s], accm);
        }
        float tm[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const uint32_t *row = &slab[wv][m][(4 * q4 + i) * kSlab];
          const uint4 s0 = *reinterpret_cast<const uint4 *>(row), s1 = *reinterpret_cast<const uint4 *>(row + 4);
          const uint32_t dd = row[8];
          const int sc[8] = {(int)s0.x, (int)s0.y, (int)s0.z, (int)s0.w, (int)s1.x, (int)s1.y, (int)s1.z, (int)s1.w};
          int sumi = 0;
#pragma unroll
          for (int s = 0; s < 8; s++) sumi += __mul24(sc[s], acc[s][i]);  // sc < 64, |a| < 2^16: exact
          const float d = half_lo(dd), dmin = half_hi(dd);
          tm[i] = xo.dt * (d * (float)sumi - dmin * (float)accm[i]);  // src/FastMath.cs:155
        }
        if (c16 < 8) terms[buf][wv][m][dl] = make_float4(tm[0], tm[1], tm[2], tm[3]);
      } else {
        // Q6_K: per half, the group sums of (q - 32) x; part = sum_g sc_g acc_g
        const uint2 m32 = make_uint2(0xE0E0E0E0u, 0xE0E0E0E0u);  // int8 -32
        i32x4_t acc[2][4];
#pragma unroll
        for (int hh = 0; hh < 2; hh++)
#pragma unroll
          for (int sp = 0; sp < 4; sp++) {
            const uint2 x = xo.xs[4 * hh + sp];
            acc[hh][sp] = mma(m32, x, mma(M::operand(raw[m], hh, sp), x, zero));
          }
        const int gs = c16 >> 3;  // this column's group within each run
        float tm[2][4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const uint32_t *row = &slab[wv][m][(4 * q4 + i) * kSlab];
          const float f = xo.dt * half_lo(row[16]);
#pragma unroll
          for (int hh = 0; hh < 2; hh++) {
            const uint4 sv = *reinterpret_cast<const uint4 *>(row + 8 * hh + 4 * gs);
            // |sc| <= 128, |acc| < 2^17: 24-bit products, exact
            int p = __mul24((int)sv.x, acc[hh][0][i]) + __mul24((int)sv.y, acc[hh][1][i]) +
                    __mul24((int)sv.z, acc[hh][2][i]) + __mul24((int)sv.w, acc[hh][3][i]);
            p += __builtin_amdgcn_update_dpp(0, p, 0x128, 0xF, 0xF, false);  // column c16 ^ 8: the other groups
            tm[hh][i] = f * (float)p;                                          // src/FastMath.cs:209
          }
        }
        if (c16 < 8) {
          terms[buf][wv][2 * m][dl] = make_float4(tm[0][0], tm[0][1], tm[0][2], tm[0][3]);
          terms[buf][wv][2 * m + 1][dl] = make_float4(tm[1][0], tm[1][1], tm[1][2], tm[1][3]);
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();  // the slab is the next block's
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };

  // the chain: lane l of wave w owns pair p = l W + w < 128 (D lane p / 4, row offset p % 4)
  const int p = lane * W + wv;
  const bool owner = p < 128;
  float sum[NM];
#pragma unroll
  for (int m = 0; m < NM; m++) sum[m] = 0.f;
  auto drain = [&](int r) {
    if (owner) {
      for (int w = 0; w < W && r * W + w < nb; w++)
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
          for (int h = 0; h < M::TERMS; h++)
            sum[m] += reinterpret_cast<const float *>(&terms[r % (2 * RPS)][w][m * M::TERMS + h][0])[p];
    }
  };

  // round r: its block's operands were fetched a round earlier; those of round r + 1 go to the
  // set that round r - 1 used. Every fetch is issued (past the row's end it re-reads the last
  // block), so the load counter's waits are the same on every path: a conditional fetch makes
  // the compiler wait for all loads in flight, the prefetched ones too. (Two rounds in flight
  // measured the same.)
  auto round = [&](int r, const Ops &cur, Ops &nxt) {
    const int b = r * W + wv;
    fetch(min(b + W, nb - 1), nxt);
    if (b < nb) body(cur, cur.x, r % (2 * RPS), b);
    if (r % RPS == RPS - 1 || r + 1 == nr) {  // uniform
      __syncthreads();
      for (int q = r - r % RPS; q <= r; q++) drain(q);
    }
  };
  Ops o0, o1;
  fetch(min(wv, nb - 1), o0);
  for (int r = 0; r < nr; r += 2) {
    round(r, o0, o1);
    if (r + 1 < nr) round(r + 1, o1, o0);
  }
  if (owner) {
    const int d = p >> 2, t = d & 7;
    const int row = tile * 16 + 4 * (d >> 3) + (p & 3);
    if (t < a.T && row < a.rows) {
      float v = sum[0];
      if constexpr (NM == 2) v = silu_mul(v, sum[1]);
      a.y[(int64_t)t * a.ldy + row] = v;
    }
  }
}

// Rounds per barrier: the most of 8, 4, 2, 1 whose ring leaves the workgroup's LDS within
// 80 KB (two workgroups per CU). For a 70B layer, one barrier per 1, 2, 4 and 8 rounds measured
// 242, 238, 228 and 250 us (the SwiGLU pair at 8: one workgroup per CU).
constexpr int rounds_per_barrier(int fixed_bytes, int bytes_per_round) {
  return fixed_bytes + 8 * bytes_per_round <= 80 * 1024   ? 8
         : fixed_bytes + 4 * bytes_per_round <= 80 * 1024 ? 4
         : fixed_bytes + 2 * bytes_per_round <= 80 * 1024 ? 2
                                                          : 1;
}

template <class M, int NM, int W, bool FRAG>
__global__ __launch_bounds__(64 * W) void intmma_kernel(MmaArgs a) {
  constexpr int MH = NM * M::TERMS;
  constexpr int RPS = rounds_per_barrier(sizeof(MmaLds<W, NM, MH, 1, M::SROW>) - 2 * W * MH * 512,
                                         2 * W * MH * 512);
  __shared__ MmaLds<W, NM, MH, RPS, M::SROW> lds;
  mma_tile<M, NM, W, FRAG, RPS>(a, blockIdx.x, lds);
}

// Several matrices that read the same activations (q, k and v) in one launch: the workgroups
// of matrix i are tiles tile_end[i - 1] .. tile_end[i] - 1; each takes its format's body.
// Launched apart, k and v (1024 rows: 64 tiles each) leave most of the device idle.
struct MmaMulti {
  MmaArgs seg[3];
  int type[3], tile_end[3];
};

template <int W, bool FRAG>
__global__ __launch_bounds__(64 * W) void intmma_multi_kernel(MmaMulti mm) {
  constexpr int RPS = 4;  // one workgroup's LDS fits three per CU
  __shared__ MmaLds<W, 1, 2, RPS, MQ6K::SROW> lds;
  const int bid = blockIdx.x;  // uniform: the segment and its branch are the workgroup's
  const int i = bid < mm.tile_end[0] ? 0 : bid < mm.tile_end[1] ? 1 : 2;
  const MmaArgs a = i == 0 ? mm.seg[0] : i == 1 ? mm.seg[1] : mm.seg[2];
  const int type = i == 0 ? mm.type[0] : i == 1 ? mm.type[1] : mm.type[2];
  const int tile = bid - (i == 0 ? 0 : i == 1 ? mm.tile_end[0] : mm.tile_end[1]);
  if (type == 12)
    mma_tile<MQ4K, 1, W, FRAG, RPS>(a, tile, lds);
  else
    mma_tile<MQ6K, 1, W, FRAG, RPS>(a, tile, lds);
}

bool intmma_supports(int type, int cols, int T, int) {
  return (type == 12 || type == 14) && cols > 0 && cols % 256 == 0 && T >= 2 && T <= kMmaTokens;
}

int intmma_max_tokens(int type, int cols, int nm) { return intmma_supports(type, cols, 2, nm) ? kMmaTokens : 0; }

// Four waves per workgroup: a 70B layer's 8192-row down matrix is 512 tiles, two per CU; six or
// eight waves (more blocks per round) measured slower, and they split a Q4_K row of 32 blocks
// unevenly.
constexpr int kMmaWaves = 4;

template <class M, int NM>
static hipError_t go(const MmaArgs &a, int grid, hipStream_t st) {
  constexpr int W = kMmaWaves;
  if (a.qf)
    hipLaunchKernelGGL((intmma_kernel<M, NM, W, true>), dim3(grid), dim3(64 * W), 0, st, a);
  else
    hipLaunchKernelGGL((intmma_kernel<M, NM, W, false>), dim3(grid), dim3(64 * W), 0, st, a);
  return hipGetLastError();
}

hipError_t intmma_launch(int type, const uint8_t *w, const uint8_t *w2, int64_t row_bytes, int rows, int cols,
                         QActsDev qa, int T, float *y, int ldy, hipStream_t st) {
  if (rows <= 0) return hipSuccess;
  if (!intmma_supports(type, cols, T, w2 ? 2 : 1) || !qa.q || !qa.d || (qa.qf && !qa.df)) return hipErrorInvalidValue;
  const MmaArgs a{w, w2, row_bytes, rows, cols, qa.qf, qa.df, qa.q, qa.d, T, y, ldy};
  const int grid = (rows + 15) / 16;
  if (type == 12) return w2 ? go<MQ4K, 2>(a, grid, st) : go<MQ4K, 1>(a, grid, st);
  return w2 ? go<MQ6K, 2>(a, grid, st) : go<MQ6K, 1>(a, grid, st);
}

bool intmma_multi_supports(const int *types, int n, int cols, int T) {
  if (n < 1 || n > 3) return false;
  for (int i = 0; i < n; i++)
    if (!intmma_supports(types[i], cols, T, 1)) return false;
  return true;
}

hipError_t intmma_multi_launch(const MmaMat *mats, int n, int cols, QActsDev qa, int T, hipStream_t st) {
  int types[3];
  for (int i = 0; i < n && i < 3; i++) types[i] = mats[i].type;
  if (!intmma_multi_supports(types, n, cols, T) || !qa.q || !qa.d || (qa.qf && !qa.df)) return hipErrorInvalidValue;
  MmaMulti mm{};
  int tiles = 0;
  for (int i = 0; i < 3; i++) {
    const MmaMat &m = mats[i < n ? i : n - 1];
    const int rows = i < n ? m.rows : 0;  // past n: empty segments
    mm.seg[i] = MmaArgs{m.w, nullptr, m.row_bytes, rows > 0 ? rows : 1, cols, qa.qf, qa.df, qa.q, qa.d, T, m.y, m.ldy};
    mm.type[i] = m.type;
    tiles += (rows + 15) / 16;
    mm.tile_end[i] = tiles;
  }
  if (tiles == 0) return hipSuccess;
  constexpr int W = kMmaWaves;
  if (qa.qf)
    hipLaunchKernelGGL((intmma_multi_kernel<W, true>), dim3(tiles), dim3(64 * W), 0, st, mm);
  else
    hipLaunchKernelGGL((intmma_multi_kernel<W, false>), dim3(tiles), dim3(64 * W), 0, st, mm);
  return hipGetLastError();
}

}  // namespace wl
