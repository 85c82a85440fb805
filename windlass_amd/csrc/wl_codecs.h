// wl_codecs.h - per-format lane codecs for the decode GEMV.
//
// Every lane of a wave owns one fixed slice of one block column (LPB lanes per block, 64/LPB
// consecutive blocks per wave, i.e. 2048 columns per wave for every format). A codec knows,
// for its block format:
//   Lane   - the lane's constant offsets and masks (from its slice index `sub`),
//   Xs     - the lane's x slice for one token, pre-scaled so the unpacked quants can enter the
//            multiply-add as fp16 subnormals (load_x also forms the sums the format needs),
//   Raw    - one row's block slice as loaded (load: memory reads only),
//   W      - that slice unpacked into registers (unpack; reused for every token),
//   dot    - the lane's partial sum of W * x for one token, in the reference's units.
//   R1     - rows per group at one token (bounded by the registers a row's Raw takes).
//   SP2    - whether rows of two passes keep both x slices in registers (1) or re-read them.
// The partial of a lane is a fixed sequence of fp32 operations on that lane's slice, the same
// for every token count, so a token's result never depends on how many tokens run with it.
//
// Integer quants enter v_fma_mix_f32 as the fp16 subnormal n * 2^-24 (n in the low bits of a
// half, no exponent bits): an exact integer-to-float conversion fused into the multiply-add.
// The 2^24 is folded into x once (an exact power-of-two scaling), so the products are the
// reference's n * x.
//
// Block layouts (ggml-common.h, restated in src/Quants.cs and src/IQuants.cs):
//   Q8_0    34 B / 32:  d f16 | q int8[32]                                (src/Quants.cs:251-259)
//   Q4_K   144 B / 256: d f16 | dmin f16 | scales[12] | qs[128]           (src/Quants.cs:332-350)
//   Q6_K   210 B / 256: ql[128] | qh[64] | scales int8[16] | d f16        (src/Quants.cs:372-396)
//   IQ4_XS 136 B / 256: d f16 | scales_h u16 | scales_l[4] | qs[128]      (src/IQuants.cs:60-80)
//   IQ2_XXS 66 B / 256: d f16 | 8 x (4 grid bytes, u32 signs+scale)       (src/IQuants.cs:147-170)
#pragma once
#include "wl_device.h"
#include "wl_tables.h"

namespace wl {

constexpr float kTwo24 = 16777216.f;
constexpr float kTwo20 = 1048576.f;

// LDS tables some codecs use; filled once per workgroup by init_lds. A launch runs one codec, so
// the formats' tables share the space. NEED_LDS 1: the tables lead the launch's dynamic LDS;
// NEED_LDS 2: they are a static LDS object (codec_lds), whose addresses are constants the
// compiler folds, so a lookup of table[byte k of a word] is one shift with a byte-select operand
// (SDWA) feeding the LDS read: IQ4_XS 617 -> 489 VALU instructions per 8-row group.
struct Lds {
  union {
    struct {
      uint2 grid8[256];   // IQ2_XXS grid entries: 8 value bytes (8, 25 or 43)
      uint2 signs8[128];  // IQ2_XXS sign patterns: 8 bytes, 0x80 where the value is negated
    };
    uint32_t iq4[256];    // IQ4_XS qs byte -> (kvalue[low nibble] + 128, kvalue[high nibble] + 128) as fp16 pair
    struct {
      uint2 grid2s[1024];  // IQ2_S grid entries: 8 value bytes
      uint2 sgn2s[256];    // a sign byte -> 8 bytes, 0x80 where the value is negated
    };
    struct {
      uint32_t grid3s[512];  // IQ3_S grid entries: 4 value bytes (odd, 1..15)
      uint2 sgn3s[256];      // as sgn2s
    };
  };
};

// The kernel's static table object (NEED_LDS 2); referenced only by such codecs' launches.
__device__ __forceinline__ Lds &codec_lds() {
  __shared__ Lds t;
  return t;
}

// ---------------------------------------------------------------------------- Q4_K
// Lane slice: 16 bytes of qs, i.e. 16 low nibbles of sub-block 2j (x[64j+16h .. +16]) and
// 16 high nibbles of sub-block 2j+1 (x[64j+32+16h .. +16]), with j = sub/2, h = sub%2.
#ifndef WL_Q4K_R1
#define WL_Q4K_R1 8
#endif
struct Q4K {
  static constexpr int BLOCK = 256, BYTES = 144, LPB = 8, NEED_LDS = 0, R1 = WL_Q4K_R1, SP2 = 1;
  struct Lane {
    int j, h, sh;
    bool jlo;
    uint32_t m1, m2;
    // the header permute: t1 = bytes (b, b+1) of scales 0-3 and of scales 4-7, t3 = bytes
    // (b, b+1) of scales 8-11 twice, b = 2j (j < 2) or 2j - 4
    uint32_t selA, selW, mA, mB, mC, mD;
  };
  struct Xs { float lo[16], hi[16], slo, shi; };
  struct Raw { uint4 hdr, q; };
  struct W { uint32_t m[16]; float fs1, fs2, fm1, fm2, d, dmin; };

  __device__ static Lane lane(int sub) {
    Lane L;
    L.j = sub >> 1;
    L.h = sub & 1;
    L.sh = 16 * (L.j & 1);
    L.jlo = L.j < 2;
    L.m1 = L.jlo ? 0x3F3F3F3Fu : 0x0F0F0F0Fu;
    L.m2 = L.jlo ? 0u : 0x30303030u;
    const uint32_t b = L.jlo ? 2 * L.j : 2 * L.j - 4;
    L.selA = b | (b + 1) << 8 | (b + 4) << 16 | (b + 5) << 24;
    L.selW = b | (b + 1) << 8 | b << 16 | (b + 1) << 24;
    L.mA = L.jlo ? 0x3F3F3F3Fu : 0u;
    L.mB = L.jlo ? 0u : 0x30303030u;
    L.mC = L.jlo ? 0u : 0x00000F0Fu;
    L.mD = L.jlo ? 0u : 0x0F0F0000u;
    return L;
  }

  __device__ static void load_x(const float *xb, const Lane &L, Xs &x) {
    ld_x16(xb + 64 * L.j + 16 * L.h, x.lo);
    ld_x16(xb + 64 * L.j + 32 + 16 * L.h, x.hi);
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i++) { a += x.lo[i]; b += x.hi[i]; }
    x.slo = a;
    x.shi = b;
    // low nibbles enter as n*2^-24, high nibbles (kept in bits 4-7) as n*2^-20
#pragma unroll
    for (int i = 0; i < 16; i++) { x.lo[i] *= kTwo24; x.hi[i] *= kTwo20; }
  }

  __device__ static void load(const uint8_t *blk, const Lane &L, Raw &r) {
    r.hdr = ldw16(blk);
    r.q = ldw16(blk + 16 + 16 * (2 * L.j + L.h));
  }

  __device__ static void unpack(const Raw &r, const Lane &L, const Lds &, W &w) {
    const uint4 h = r.hdr;
    // The 6-bit scales and mins of sub-blocks 2j and 2j+1 (get_scale_min_k4,
    // src/Quants.cs:321-330) as the four bytes of one word: sub-blocks 0-3 are the low 6 bits
    // of bytes 0-7; 4-7 take their low 4 bits from bytes 8-11 and the top two from the top of
    // bytes 0-7. Two byte permutes with lane-constant selectors gather the lane's bytes, and
    // lane-constant masks keep what each case takes; each byte then converts on its own.
    const uint32_t t1 = __builtin_amdgcn_perm(h.z, h.y, L.selA);
    const uint32_t t3 = __builtin_amdgcn_perm(h.w, h.w, L.selW);
    const uint32_t W4 = (t1 & L.mA) | ((t1 >> 2) & L.mB) | (t3 & L.mC) | ((t3 >> 4) & L.mD);
    w.fs1 = (float)(W4 & 0xFF);
    w.fs2 = (float)((W4 >> 8) & 0xFF);
    w.fm1 = (float)((W4 >> 16) & 0xFF);
    w.fm2 = (float)(W4 >> 24);
    w.d = half_lo(h.x);
    w.dmin = half_hi(h.x);
    const uint32_t qq[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t v = qq[i], v8 = v >> 8;
      w.m[4 * i + 0] = v & 0x000F000Fu;   // low nibbles of bytes 0, 2
      w.m[4 * i + 1] = v8 & 0x000F000Fu;  // low nibbles of bytes 1, 3
      w.m[4 * i + 2] = v & 0x00F000F0u;   // high nibbles of bytes 0, 2
      w.m[4 * i + 3] = v8 & 0x00F000F0u;  // high nibbles of bytes 1, 3
    }
  }

  __device__ static float dot(const W &w, const Xs &x) {
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      a = fma_lo(w.m[4 * i + 0], x.lo[4 * i + 0], a);
      a = fma_hi(w.m[4 * i + 0], x.lo[4 * i + 2], a);
      a = fma_lo(w.m[4 * i + 1], x.lo[4 * i + 1], a);
      a = fma_hi(w.m[4 * i + 1], x.lo[4 * i + 3], a);
      b = fma_lo(w.m[4 * i + 2], x.hi[4 * i + 0], b);
      b = fma_hi(w.m[4 * i + 2], x.hi[4 * i + 2], b);
      b = fma_lo(w.m[4 * i + 3], x.hi[4 * i + 1], b);
      b = fma_hi(w.m[4 * i + 3], x.hi[4 * i + 3], b);
    }
    // d*(s1*a1 + s2*a2) - dmin*(m1*x1 + m2*x2)   (src/Quants.cs:129)
    const float sc = __builtin_fmaf(w.fs2, b, w.fs1 * a);
    const float mn = __builtin_fmaf(w.fm2, x.shi, w.fm1 * x.slo);
    return __builtin_fmaf(w.d, sc, -(w.dmin * mn));
  }
};

// ---------------------------------------------------------------------------- Q6_K
// Lane slice: half hh = sub/4 of the block (128 values) and l = 8g..8g+7 with g = sub%4:
// the four values l, l+32, l+64, l+96 of each l (scales sc[l/16 + 0,2,4,6]).
#ifndef WL_Q6K_R1
#define WL_Q6K_R1 4
#endif
#ifndef WL_Q6K_SP2
#define WL_Q6K_SP2 1
#endif
struct Q6K {
  static constexpr int BLOCK = 256, BYTES = 210, LPB = 8, NEED_LDS = 0, R1 = WL_Q6K_R1, SP2 = WL_Q6K_SP2;
  struct Lane { int hh, g, s; uint32_t ssel; };
  struct Xs { float v[4][8]; float s[4]; };
  // the aligned dwords around each 2-byte-aligned field, and the byte shift (0 or 16)
  struct Raw { uint32_t l1[3], l2[3], h[3], sc[3], dw; uint32_t sh; };
  struct W { uint32_t p[4][4]; float dq[4]; };

  __device__ static Lane lane(int sub) {
    Lane L;
    L.hh = sub >> 2;
    L.g = sub & 3;
    L.s = L.g >> 1;
    L.ssel = (uint32_t)L.s | (uint32_t)(L.s + 2) << 8 | (uint32_t)(L.s + 4) << 16 | (uint32_t)(L.s + 6) << 24;
    return L;
  }

  __device__ static void load_x(const float *xb, const Lane &L, Xs &x) {
    const float *base = xb + 128 * L.hh + 8 * L.g;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      ld_x8(base + 32 * k, x.v[k]);
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < 8; i++) s += x.v[k][i];
      x.s[k] = s;
#pragma unroll
      for (int i = 0; i < 8; i++) x.v[k][i] *= kTwo24;
    }
  }

  __device__ static void load(const uint8_t *blk, const Lane &L, Raw &r) {
    // every field offset below is a multiple of 8, so all share the block's alignment
    gu32 *a = align4_down(blk);
    r.sh = misalign4(blk) * 8;
    const int o1 = (64 * L.hh + 8 * L.g) / 4, o2 = (64 * L.hh + 32 + 8 * L.g) / 4,
              oh = (128 + 32 * L.hh + 8 * L.g) / 4, os = (192 + 8 * L.hh) / 4;
    ldw12(a + o1, r.l1);
    ldw12(a + o2, r.l2);
    ldw12(a + oh, r.h);
    ldw12(a + os, r.sc);
    r.dw = ldw4(a + 208 / 4);  // d: low half (aligned block) or high half (block at 2 mod 4)
  }

  __device__ static uint2 field(const uint32_t (&f)[3], uint32_t sh) {
    return make_uint2(__builtin_amdgcn_alignbit(f[1], f[0], sh), __builtin_amdgcn_alignbit(f[2], f[1], sh));
  }

  __device__ static void unpack(const Raw &r, const Lane &L, const Lds &, W &w) {
    const uint2 ql1 = field(r.l1, r.sh), ql2 = field(r.l2, r.sh), qh = field(r.h, r.sh), sc = field(r.sc, r.sh);
    const float d = half_lo(r.sh ? (r.dw >> 16) : r.dw);
    // signed scale bytes s, s+2 (first dword) and s+4, s+6 (second dword), gathered into one
    // word by a byte permute with a lane-constant selector
    const uint32_t sg = __builtin_amdgcn_perm(sc.y, sc.x, L.ssel);
    const float scs[4] = {(float)(int8_t)sg, (float)(int8_t)(sg >> 8), (float)(int8_t)(sg >> 16),
                          (float)(int8_t)(sg >> 24)};
#pragma unroll
    for (int k = 0; k < 4; k++) w.dq[k] = d * scs[k];
    const uint32_t L1[2] = {ql1.x, ql1.y}, L2[2] = {ql2.x, ql2.y}, QH[2] = {qh.x, qh.y};
#pragma unroll
    for (int i = 0; i < 2; i++) {
      // Four 6-bit values per dword (one per byte), for the four quarter-runs
      // (src/Quants.cs:384-387).
      const uint32_t a = (L1[i] & 0x0F0F0F0Fu) | ((QH[i] << 4) & 0x30303030u);
      const uint32_t b = (L2[i] & 0x0F0F0F0Fu) | ((QH[i] << 2) & 0x30303030u);
      const uint32_t c = ((L1[i] >> 4) & 0x0F0F0F0Fu) | (QH[i] & 0x30303030u);
      const uint32_t e = ((L2[i] >> 4) & 0x0F0F0F0Fu) | ((QH[i] >> 2) & 0x30303030u);
      const uint32_t q4[4] = {a, b, c, e};
#pragma unroll
      for (int k = 0; k < 4; k++) {
        w.p[k][2 * i + 0] = q4[k] & 0x00FF00FFu;                          // bytes 0, 2 as subnormal halves
        w.p[k][2 * i + 1] = __builtin_amdgcn_perm(q4[k], q4[k], 0x0C030C01u);  // bytes 1, 3 (zero-filled)
      }
    }
  }

  __device__ static float dot(const W &w, const Xs &x) {
    float r = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      float a = 0.f;
#pragma unroll
      for (int i = 0; i < 2; i++) {
        a = fma_lo(w.p[k][2 * i + 0], x.v[k][4 * i + 0], a);
        a = fma_hi(w.p[k][2 * i + 0], x.v[k][4 * i + 2], a);
        a = fma_lo(w.p[k][2 * i + 1], x.v[k][4 * i + 1], a);
        a = fma_hi(w.p[k][2 * i + 1], x.v[k][4 * i + 3], a);
      }
      // (d*sc) * sum((q-32)*x) = (d*sc) * (sum(q*x) - 32*sum(x))   (src/Quants.cs:173-180)
      r = __builtin_fmaf(w.dq[k], __builtin_fmaf(-32.f, x.s[k], a), r);
    }
    return r;
  }
};

// ---------------------------------------------------------------------------- Q8_0
// Lane slice: one whole 32-value block (blocks start 2-byte aligned).
struct Q80 {
  static constexpr int BLOCK = 32, BYTES = 34, LPB = 1, NEED_LDS = 0, R1 = 4, SP2 = 1;
  struct Lane {};
  struct Xs { float v[32]; float s; };
  // the 10 aligned dwords covering the block and the byte shift (0 or 16)
  struct Raw { uint32_t win[10]; uint32_t sh; };
  struct W { uint32_t p[16]; float d; };

  __device__ static Lane lane(int) { return Lane{}; }

  __device__ static void load_x(const float *xb, const Lane &, Xs &x) {
    ld_x16(xb, x.v);
    ld_x16(xb + 16, x.v + 16);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) s += x.v[i];
    x.s = s;
#pragma unroll
    for (int i = 0; i < 32; i++) x.v[i] *= kTwo24;
  }

  __device__ static void load(const uint8_t *blk, const Lane &, Raw &r) {
    gu32 *a = align4_down(blk);
    r.sh = misalign4(blk) * 8;
#pragma unroll
    for (int i = 0; i < 10; i++) r.win[i] = ldw4(a + i);
  }

  __device__ static void unpack(const Raw &r, const Lane &, const Lds &, W &w) {
    // d: bytes 0-1 of the block; q: bytes 2..33, i.e. the window shifted by sh + 16 bits
    w.d = half_lo(__builtin_amdgcn_alignbit(r.win[1], r.win[0], r.sh));
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const uint32_t lo = __builtin_amdgcn_alignbit(r.win[i + 1], r.win[i], r.sh);
      const uint32_t hi = __builtin_amdgcn_alignbit(r.win[i + 2], r.win[i + 1], r.sh);
      // int8 q + 128 as an unsigned byte, then bytes 0,2 / 1,3 as subnormal halves
      const uint32_t v = __builtin_amdgcn_alignbit(hi, lo, 16) ^ 0x80808080u;
      w.p[2 * i] = v & 0x00FF00FFu;
      w.p[2 * i + 1] = __builtin_amdgcn_perm(v, v, 0x0C030C01u);  // bytes 1, 3 (zero-filled)
    }
  }

  // Two accumulators (even and odd values, as the reference's DotRow keeps two partial sums,
  // src/Quants.cs:86-97): independent multiply-add chains issue without the wait a chain of
  // dependent v_fma_mix_f32 needs on gfx950.
  __device__ static float dot(const W &w, const Xs &x) {
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      a = fma_lo(w.p[2 * i], x.v[4 * i + 0], a);
      b = fma_lo(w.p[2 * i + 1], x.v[4 * i + 1], b);
      a = fma_hi(w.p[2 * i], x.v[4 * i + 2], a);
      b = fma_hi(w.p[2 * i + 1], x.v[4 * i + 3], b);
    }
    // d * sum(q*x) = d * (sum((q+128)*x) - 128*sum(x))   (src/Quants.cs:93-94)
    return w.d * __builtin_fmaf(-128.f, x.s, a + b);
  }
};

// -------------------------------------------------------------------------- IQ4_XS
// Lane slice: sub-block ib = sub (32 values, 16 bytes of qs). Word k of a lane's W holds the
// values of qs byte k, kvalue[low nibble] + 128 and kvalue[high nibble] + 128 (values k and
// 16 + k), as two fp16 subnormals. TABLE: the word is read from an LDS table indexed by the
// byte (the one-token launches); otherwise it is looked up in registers (byte permutes over the
// 16 kvalues; the batched launches, whose LDS carries the tokens' x). Both build the same words
// and share the dot, so a token's bits do not depend on which launch computed it.
template <bool TABLE>
struct IQ4XSc {
  static constexpr int BLOCK = 256, BYTES = 136, LPB = 8, NEED_LDS = TABLE ? 2 : 0, R1 = 8, SP2 = 1;
  struct Lane { int ib; };
  struct Xs { float v[32]; float s; };
  struct Raw { uint2 hdr, q01, q23; };
  struct W { uint32_t p[16]; float dl; };

  __device__ static Lane lane(int sub) { return Lane{sub}; }

  __device__ static void load_x(const float *xb, const Lane &L, Xs &x) {
    ld_x16(xb + 32 * L.ib, x.v);
    ld_x16(xb + 32 * L.ib + 16, x.v + 16);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) s += x.v[i];
    x.s = s;
#pragma unroll
    for (int i = 0; i < 32; i++) x.v[i] *= kTwo24;
  }

  // blocks are 8-byte aligned (136 = 8*17): 8-byte loads for the header and the 16 qs bytes
  __device__ static void load(const uint8_t *blk, const Lane &L, Raw &r) {
    r.hdr = ldw8(blk);  // d | scales_h | scales_l[4]
    r.q01 = ldw8(blk + 8 + 16 * L.ib);
    r.q23 = ldw8(blk + 16 + 16 * L.ib);
  }

  // kvalues_iq4nl + 128 (all in 1..241) as bytes: table index n -> byte n.
  static constexpr uint32_t kT0 = (uint32_t)(uint8_t)(-127 + 128) | (uint32_t)(uint8_t)(-104 + 128) << 8 |
                                  (uint32_t)(uint8_t)(-83 + 128) << 16 | (uint32_t)(uint8_t)(-65 + 128) << 24;
  static constexpr uint32_t kT1 = (uint32_t)(uint8_t)(-49 + 128) | (uint32_t)(uint8_t)(-35 + 128) << 8 |
                                  (uint32_t)(uint8_t)(-22 + 128) << 16 | (uint32_t)(uint8_t)(-10 + 128) << 24;
  static constexpr uint32_t kT2 = (uint32_t)(uint8_t)(1 + 128) | (uint32_t)(uint8_t)(13 + 128) << 8 |
                                  (uint32_t)(uint8_t)(25 + 128) << 16 | (uint32_t)(uint8_t)(38 + 128) << 24;
  static constexpr uint32_t kT3 = (uint32_t)(uint8_t)(53 + 128) | (uint32_t)(uint8_t)(69 + 128) << 8 |
                                  (uint32_t)(uint8_t)(89 + 128) << 16 | (uint32_t)(uint8_t)(113 + 128) << 24;

  // Four 4-bit indices (one per byte) -> four table bytes: two byte-permutes over the
  // 8-entry halves, then a per-byte select on index bit 3.
  __device__ static uint32_t lookup(uint32_t idx) {
    const uint32_t i3 = idx & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(kT1, kT0, i3);
    const uint32_t hi = __builtin_amdgcn_perm(kT3, kT2, i3);
    // selector 12 -> 0x00, 13 -> 0xFF: a byte mask from bit 3 of each index
    const uint32_t m = __builtin_amdgcn_perm(0u, 0u, ((idx >> 3) & 0x01010101u) | 0x0C0C0C0Cu);
    return (hi & m) | (lo & ~m);
  }

  __device__ static void unpack(const Raw &r, const Lane &L, const Lds &lds, W &w) {
    const uint2 hdr = r.hdr;
    const int ib = L.ib;
    const float d = half_lo(hdr.x);
    const uint32_t scales_h = hdr.x >> 16;
    const int ls = (int)((hdr.y >> (8 * (ib >> 1) + 4 * (ib & 1))) & 0xF) | (int)(((scales_h >> (2 * ib)) & 3) << 4);
    w.dl = d * (float)(ls - 32);  // src/IQuants.cs:71-72
    const uint32_t qq[4] = {r.q01.x, r.q01.y, r.q23.x, r.q23.y};
    if constexpr (TABLE) {
#pragma unroll
      for (int k = 0; k < 16; k++) w.p[k] = lds.iq4[(qq[k >> 2] >> (8 * (k & 3))) & 0xFF];
    } else {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        // the low nibbles' and the high nibbles' values of qs bytes 4i .. 4i+3, then byte b of
        // each into word 4i + b: [low value, 0, high value, 0]
        const uint32_t lo = lookup(qq[i] & 0x0F0F0F0Fu);
        const uint32_t hi = lookup((qq[i] >> 4) & 0x0F0F0F0Fu);
#pragma unroll
        for (int b = 0; b < 4; b++)
          w.p[4 * i + b] = __builtin_amdgcn_perm(hi, lo, (uint32_t)b | 0x0C00u | (uint32_t)(4 + b) << 16 | 0x0C000000u);
      }
    }
  }

  // Two accumulators (the low and the high nibbles' values): independent chains issue without
  // the wait a chain of dependent v_fma_mix_f32 needs on gfx950.
  __device__ static float dot(const W &w, const Xs &x) {
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int k = 0; k < 16; k++) {
      a = fma_lo(w.p[k], x.v[k], a);
      b = fma_hi(w.p[k], x.v[16 + k], b);
    }
    // dl * sum(kv*x) = dl * (sum((kv+128)*x) - 128*sum(x))
    return w.dl * __builtin_fmaf(-128.f, x.s, a + b);
  }

  // byte b -> fp16 pair (kvalues[b & 15] + 128, kvalues[b >> 4] + 128) as subnormals
  __device__ static void init_lds(Lds &lds) {
    for (int i = threadIdx.x; i < 256; i += blockDim.x)
      lds.iq4[i] = (uint32_t)(kKvaluesIq4nl[i & 15] + 128) | (uint32_t)(kKvaluesIq4nl[i >> 4] + 128) << 16;
  }
};
using IQ4XS = IQ4XSc<true>;    // one-token launches, the MoE experts
using IQ4XSR = IQ4XSc<false>;  // the batched launches

// ------------------------------------------------------------------------- IQ2_XXS
// Lane slice: sub-block ib32 = sub: four groups of 8 values, each a grid entry (8 bytes of
// 8/25/43) with eight signs from a 7-bit index plus a parity bit.
struct IQ2XXS {
  static constexpr int BLOCK = 256, BYTES = 66, LPB = 8, NEED_LDS = 2, R1 = 8, SP2 = 1;
  struct Lane { int ib; };
  struct Xs { float v[32]; };
  struct Raw { uint32_t dw, a[3]; uint32_t dsh, sh; };
  struct W { uint32_t p[16]; float db; };

  __device__ static Lane lane(int sub) { return Lane{sub}; }

  __device__ static void load_x(const float *xb, const Lane &L, Xs &x) {
    ld_x16(xb + 32 * L.ib, x.v);
    ld_x16(xb + 32 * L.ib + 16, x.v + 16);
#pragma unroll
    for (int i = 0; i < 32; i++) x.v[i] *= kTwo24;
  }

  __device__ static void load(const uint8_t *blk, const Lane &L, Raw &r) {
    const uint8_t *pa = blk + 2 + 8 * L.ib;
    r.dw = ldw4(align4_down(blk));
    r.dsh = misalign4(blk) & 2;
    gu32 *a = align4_down(pa);
    r.sh = misalign4(pa) * 8;
    r.a[0] = ldw4(a);
    r.a[1] = ldw4(a + 1);
    r.a[2] = ldw4(a + 2);
  }

  __device__ static void unpack(const Raw &r, const Lane &, const Lds &lds, W &w) {
    const float d = half_lo(r.dsh ? (r.dw >> 16) : r.dw);
    const uint2 aux = make_uint2(__builtin_amdgcn_alignbit(r.a[1], r.a[0], r.sh),
                                 __builtin_amdgcn_alignbit(r.a[2], r.a[1], r.sh));
    // db = d * (0.5 + scale4) * 0.25   (src/IQuants.cs:159)
    w.db = d * (0.5f + (float)(aux.y >> 28)) * 0.25f;
#pragma unroll
    for (int l = 0; l < 4; l++) {
      const uint32_t gi = (aux.x >> (8 * l)) & 0xFF;
      const uint32_t si = (aux.y >> (7 * l)) & 127;
      const uint2 g = lds.grid8[gi], sg = lds.signs8[si];
      // fp16 pairs (value bytes a, b as subnormals, sign bytes as their high bytes):
      // bytes [g_a, s_a, g_b, s_b] for the pairs (0,2) (1,3) of each half
      w.p[4 * l + 0] = __builtin_amdgcn_perm(sg.x, g.x, 0x06020400u);
      w.p[4 * l + 1] = __builtin_amdgcn_perm(sg.x, g.x, 0x07030501u);
      w.p[4 * l + 2] = __builtin_amdgcn_perm(sg.y, g.y, 0x06020400u);
      w.p[4 * l + 3] = __builtin_amdgcn_perm(sg.y, g.y, 0x07030501u);
    }
  }

  // Two accumulators (groups 0, 2 and groups 1, 3): independent chains issue without the wait a
  // chain of dependent v_fma_mix_f32 needs on gfx950.
  __device__ static float dot(const W &w, const Xs &x) {
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int l = 0; l < 4; l += 2) {
      const float *xa = x.v + 8 * l, *xb = x.v + 8 * (l + 1);
      const uint32_t *pa = w.p + 4 * l, *pb = w.p + 4 * (l + 1);
      // pairs (0,2) (1,3) (4,6) (5,7) of each group, as init_lds lays them out
      a = fma_lo(pa[0], xa[0], a);
      b = fma_lo(pb[0], xb[0], b);
      a = fma_hi(pa[0], xa[2], a);
      b = fma_hi(pb[0], xb[2], b);
      a = fma_lo(pa[1], xa[1], a);
      b = fma_lo(pb[1], xb[1], b);
      a = fma_hi(pa[1], xa[3], a);
      b = fma_hi(pb[1], xb[3], b);
      a = fma_lo(pa[2], xa[4], a);
      b = fma_lo(pb[2], xb[4], b);
      a = fma_hi(pa[2], xa[6], a);
      b = fma_hi(pb[2], xb[6], b);
      a = fma_lo(pa[3], xa[5], a);
      b = fma_lo(pb[3], xb[5], b);
      a = fma_hi(pa[3], xa[7], a);
      b = fma_hi(pb[3], xb[7], b);
    }
    return w.db * (a + b);
  }

  // The grid entries as their 8 value bytes and the 128 sign patterns (ksigns_iq2xs: index plus
  // an even-parity bit) as 8 bytes of 0x80 / 0x00; unpack merges them into fp16 pairs.
  __device__ static void init_lds(Lds &lds) {
    for (int i = threadIdx.x; i < 256; i += blockDim.x) {
      uint32_t b[8];
      for (int j = 0; j < 8; j++) b[j] = iq2_code_byte((kIq2xxsCodes[i] >> (2 * j)) & 3);
      lds.grid8[i] = make_uint2(b[0] | b[1] << 8 | b[2] << 16 | b[3] << 24, b[4] | b[5] << 8 | b[6] << 16 | b[7] << 24);
    }
    for (int i = threadIdx.x; i < 128; i += blockDim.x) {
      const uint32_t sg = (uint32_t)i | ((uint32_t)(__builtin_popcount(i) & 1) << 7);
      uint32_t m[8];
      for (int j = 0; j < 8; j++) m[j] = ((sg >> j) & 1) ? 0x80u : 0u;
      lds.signs8[i] = make_uint2(m[0] | m[1] << 8 | m[2] << 16 | m[3] << 24, m[4] | m[5] << 8 | m[6] << 16 | m[7] << 24);
    }
  }
};

}  // namespace wl
