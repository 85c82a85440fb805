// wl_codecs.h - per-format lane codecs for the decode GEMV.
//
// A wave64 walks a group of weight rows; in each step every lane owns one fixed slice of one
// GGUF block (LPB lanes per block, 64/LPB consecutive blocks per step) and the matching slice
// of x. A codec knows, for its block format:
//   Xs     - the x slice of a lane for one token (values plus the sums the format needs),
//   W      - one row's block slice unpacked into registers (done once, reused for every token),
//   load_x - read the x slice,  decode - read and unpack the weight slice,
//   dot    - the lane's partial sum of W * x for one token.
// The partial of a lane is a fixed sequence of fp32 operations on that lane's slice, the same
// for every token count, so a token's result never depends on how many tokens run with it.
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

// LDS tables some codecs use; filled once per workgroup by init_lds.
struct Lds {
  uint32_t grid16[256][4];   // IQ2_XXS grid entries as four fp16-subnormal byte pairs
  uint32_t signs16[128][4];  // IQ2_XXS sign patterns as fp16 sign-bit masks, same pairing
};

// ---------------------------------------------------------------------------- Q4_K
// Lane slice: 16 bytes of qs, i.e. 16 low nibbles of sub-block 2j (x[64j+16h .. +16]) and
// 16 high nibbles of sub-block 2j+1 (x[64j+32+16h .. +16]), with j = sub/2, h = sub%2.
struct Q4K {
  static constexpr int BLOCK = 256, BYTES = 144, LPB = 8, NEED_LDS = 0;
  struct Xs { float lo[16], hi[16], slo, shi; };
  struct W { uint32_t m[16]; float ds1, ds2, dm1, dm2; };

  __device__ static void load_x(const float *xb, int sub, Xs &x) {
    const int j = sub >> 1, h = sub & 1;
    ld_x16(xb + 64 * j + 16 * h, x.lo);
    ld_x16(xb + 64 * j + 32 + 16 * h, x.hi);
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i++) { a += x.lo[i]; b += x.hi[i]; }
    x.slo = a; x.shi = b;
  }

  __device__ static void decode(const uint8_t *blk, int sub, const Lds &, W &w) {
    const uint4 hdr = ld16(blk);
    const uint4 q = ld16(blk + 16 + 16 * sub);
    const int j = sub >> 1;
    // The 6-bit scales and mins of all eight sub-blocks as bytes (get_scale_min_k4,
    // src/Quants.cs:321-330): sub-blocks 0-3 from bytes 0-7, 4-7 from bytes 8-11 plus the
    // top two bits of bytes 0-7.
    uint32_t S, M;
    if (j < 2) {
      S = hdr.y & 0x3F3F3F3Fu;
      M = hdr.z & 0x3F3F3F3Fu;
    } else {
      S = (hdr.w & 0x0F0F0F0Fu) | ((hdr.y >> 2) & 0x30303030u);
      M = ((hdr.w >> 4) & 0x0F0F0F0Fu) | ((hdr.z >> 2) & 0x30303030u);
    }
    const int sh = (j & 1) * 16;
    const float s1 = (float)((S >> sh) & 0xFF), s2 = (float)((S >> (sh + 8)) & 0xFF);
    const float m1 = (float)((M >> sh) & 0xFF), m2 = (float)((M >> (sh + 8)) & 0xFF);
    const float d = half_lo(hdr.x), dmin = half_hi(hdr.x);
    // Low nibbles enter as n*2^-24, high nibbles (kept in bits 4-7) as n*2^-20.
    w.ds1 = d * (s1 * 16777216.f);
    w.ds2 = d * (s2 * 1048576.f);
    w.dm1 = dmin * m1;
    w.dm2 = dmin * m2;
    const uint32_t qq[4] = {q.x, q.y, q.z, q.w};
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
    float mins = __builtin_fmaf(w.dm2, x.shi, w.dm1 * x.slo);
    float r = __builtin_fmaf(w.ds2, b, w.ds1 * a);
    return r - mins;
  }
};

// ---------------------------------------------------------------------------- Q6_K
// Lane slice: half hh = sub/4 of the block (128 values) and l = 8g..8g+7 with g = sub%4:
// the four values l, l+32, l+64, l+96 of each l (scales sc[l/16 + 0,2,4,6]).
struct Q6K {
  static constexpr int BLOCK = 256, BYTES = 210, LPB = 8, NEED_LDS = 0;
  struct Xs { float v[4][8]; float s[4]; };
  struct W { uint32_t p[4][4]; float dq[4], dz[4]; };

  __device__ static void load_x(const float *xb, int sub, Xs &x) {
    const int hh = sub >> 2, g = sub & 3;
    const float *base = xb + 128 * hh + 8 * g;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      ld_x8(base + 32 * k, x.v[k]);
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < 8; i++) s += x.v[k][i];
      x.s[k] = s;
    }
  }

  __device__ static void decode(const uint8_t *blk, int sub, const Lds &, W &w) {
    const int hh = sub >> 2, g = sub & 3;
    const uint2 ql1 = ld8_a2(blk + 64 * hh + 8 * g);
    const uint2 ql2 = ld8_a2(blk + 64 * hh + 32 + 8 * g);
    const uint2 qh = ld8_a2(blk + 128 + 32 * hh + 8 * g);
    const uint2 sc = ld8_a2(blk + 192 + 8 * hh);
    const float d = half_lo(ld_half_a2(blk + 208));
    const int s = g >> 1;
    // signed scale bytes s, s+2 (first dword) and s+4, s+6 (second dword)
    const float sc0 = (float)(int8_t)(sc.x >> (8 * s)), sc1 = (float)(int8_t)(sc.x >> (8 * s + 16));
    const float sc2 = (float)(int8_t)(sc.y >> (8 * s)), sc3 = (float)(int8_t)(sc.y >> (8 * s + 16));
    const float scs[4] = {sc0, sc1, sc2, sc3};
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const float dk = d * scs[k];
      w.dq[k] = dk * 16777216.f;  // the 6-bit values enter as q*2^-24
      w.dz[k] = dk * 32.f;        // the -32 offset, applied to the sum of x
    }
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
        w.p[k][2 * i + 0] = q4[k] & 0x00FF00FFu;         // bytes 0, 2 as subnormal halves
        w.p[k][2 * i + 1] = (q4[k] >> 8) & 0x00FF00FFu;  // bytes 1, 3
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
      // (d*sc) * sum((q-32)*x) = dq*a - dz*sum(x)   (src/Quants.cs:173-180)
      r = __builtin_fmaf(w.dq[k], a, r);
      r = __builtin_fmaf(-w.dz[k], x.s[k], r);
    }
    return r;
  }
};

// ---------------------------------------------------------------------------- Q8_0
// Lane slice: one whole 32-value block (blocks start 2-byte aligned).
struct Q80 {
  static constexpr int BLOCK = 32, BYTES = 34, LPB = 1, NEED_LDS = 0;
  struct Xs { float v[32]; float s; };
  struct W { uint32_t p[16]; float dq, dz; };

  __device__ static void load_x(const float *xb, int, Xs &x) {
    ld_x16(xb, x.v);
    ld_x16(xb + 16, x.v + 16);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) s += x.v[i];
    x.s = s;
  }

  __device__ static void decode(const uint8_t *blk, int, const Lds &, W &w) {
    const float d = half_lo(ld_half_a2(blk));
    const uint8_t *q = blk + 2;
    const uint32_t *a = reinterpret_cast<const uint32_t *>(reinterpret_cast<uintptr_t>(q) & ~uintptr_t(3));
    const uint32_t sh = (uint32_t)(reinterpret_cast<uintptr_t>(q) & 3) * 8;
    uint32_t win[9];
#pragma unroll
    for (int i = 0; i < 9; i++) win[i] = a[i];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      // int8 q + 128 as an unsigned byte, then bytes 0,2 / 1,3 as subnormal halves
      const uint32_t v = __builtin_amdgcn_alignbit(win[i + 1], win[i], sh) ^ 0x80808080u;
      w.p[2 * i] = v & 0x00FF00FFu;
      w.p[2 * i + 1] = (v >> 8) & 0x00FF00FFu;
    }
    w.dq = d * 16777216.f;
    w.dz = d * 128.f;
  }

  __device__ static float dot(const W &w, const Xs &x) {
    float a = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      a = fma_lo(w.p[2 * i], x.v[4 * i + 0], a);
      a = fma_hi(w.p[2 * i], x.v[4 * i + 2], a);
      a = fma_lo(w.p[2 * i + 1], x.v[4 * i + 1], a);
      a = fma_hi(w.p[2 * i + 1], x.v[4 * i + 3], a);
    }
    // d * sum(q*x) = dq*sum((q+128)*x*2^-24) - 128*d*sum(x)   (src/Quants.cs:93-94)
    return __builtin_fmaf(w.dq, a, -(w.dz * x.s));
  }
};

// -------------------------------------------------------------------------- IQ4_XS
// Lane slice: sub-block ib = sub (32 values, 16 bytes of qs).
struct IQ4XS {
  static constexpr int BLOCK = 256, BYTES = 136, LPB = 8, NEED_LDS = 0;
  struct Xs { float v[32]; float s; };
  struct W { uint32_t p[16]; float dq, dz; };

  __device__ static void load_x(const float *xb, int sub, Xs &x) {
    ld_x16(xb + 32 * sub, x.v);
    ld_x16(xb + 32 * sub + 16, x.v + 16);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) s += x.v[i];
    x.s = s;
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

  __device__ static void decode(const uint8_t *blk, int sub, const Lds &, W &w) {
    // blocks are 8-byte aligned (136 = 8*17): two 8-byte loads for the 16 bytes of qs
    const uint2 hdr = *reinterpret_cast<const uint2 *>(blk);  // d | scales_h | scales_l[4]
    const uint2 q01 = *reinterpret_cast<const uint2 *>(blk + 8 + 16 * sub);
    const uint2 q23 = *reinterpret_cast<const uint2 *>(blk + 16 + 16 * sub);
    const float d = half_lo(hdr.x);
    const uint32_t scales_h = hdr.x >> 16;
    const int ls = (int)((hdr.y >> (8 * (sub >> 1) + 4 * (sub & 1))) & 0xF) |
                   (int)(((scales_h >> (2 * sub)) & 3) << 4);
    const float dl = d * (float)(ls - 32);  // src/IQuants.cs:71-72
    w.dq = dl * 16777216.f;
    w.dz = dl * 128.f;
    const uint32_t qq[4] = {q01.x, q01.y, q23.x, q23.y};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      // qs byte 4i+k: low nibble -> value 4i+k, high nibble -> value 16+4i+k
      const uint32_t lo = lookup(qq[i] & 0x0F0F0F0Fu);
      const uint32_t hi = lookup((qq[i] >> 4) & 0x0F0F0F0Fu);
      w.p[2 * i] = lo & 0x00FF00FFu;
      w.p[2 * i + 1] = (lo >> 8) & 0x00FF00FFu;
      w.p[8 + 2 * i] = hi & 0x00FF00FFu;
      w.p[8 + 2 * i + 1] = (hi >> 8) & 0x00FF00FFu;
    }
  }

  __device__ static float dot(const W &w, const Xs &x) {
    float a = 0.f;
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float *xv = x.v + 16 * h + 4 * i;
        a = fma_lo(w.p[8 * h + 2 * i], xv[0], a);
        a = fma_hi(w.p[8 * h + 2 * i], xv[2], a);
        a = fma_lo(w.p[8 * h + 2 * i + 1], xv[1], a);
        a = fma_hi(w.p[8 * h + 2 * i + 1], xv[3], a);
      }
    return __builtin_fmaf(w.dq, a, -(w.dz * x.s));
  }
};

// ------------------------------------------------------------------------- IQ2_XXS
// Lane slice: sub-block ib32 = sub: four groups of 8 values, each a grid entry (8 bytes of
// 8/25/43) with eight signs from a 7-bit index plus a parity bit.
struct IQ2XXS {
  static constexpr int BLOCK = 256, BYTES = 66, LPB = 8, NEED_LDS = 1;
  struct Xs { float v[32]; };
  struct W { uint32_t p[16]; float db; };

  __device__ static void load_x(const float *xb, int sub, Xs &x) {
    ld_x16(xb + 32 * sub, x.v);
    ld_x16(xb + 32 * sub + 16, x.v + 16);
  }

  __device__ static void decode(const uint8_t *blk, int sub, const Lds &lds, W &w) {
    const float d = half_lo(ld_half_a2(blk));
    const uint2 aux = ld8_a2(blk + 2 + 8 * sub);
    // db = d * (0.5 + scale4) * 0.25; grid bytes enter as n*2^-24   (src/IQuants.cs:159)
    const float db = d * (0.5f + (float)(aux.y >> 28)) * 0.25f;
    w.db = db * 16777216.f;
#pragma unroll
    for (int l = 0; l < 4; l++) {
      const uint32_t gi = (aux.x >> (8 * l)) & 0xFF;
      const uint32_t si = (aux.y >> (7 * l)) & 127;
      const uint4 g = *reinterpret_cast<const uint4 *>(lds.grid16[gi]);
      const uint4 s = *reinterpret_cast<const uint4 *>(lds.signs16[si]);
      w.p[4 * l + 0] = g.x | s.x;
      w.p[4 * l + 1] = g.y | s.y;
      w.p[4 * l + 2] = g.z | s.z;
      w.p[4 * l + 3] = g.w | s.w;
    }
  }

  __device__ static float dot(const W &w, const Xs &x) {
    float a = 0.f;
#pragma unroll
    for (int l = 0; l < 4; l++) {
      const float *xv = x.v + 8 * l;
      // pairs (0,2) (1,3) (4,6) (5,7) of the group, as init_lds lays them out
      a = fma_lo(w.p[4 * l + 0], xv[0], a);
      a = fma_hi(w.p[4 * l + 0], xv[2], a);
      a = fma_lo(w.p[4 * l + 1], xv[1], a);
      a = fma_hi(w.p[4 * l + 1], xv[3], a);
      a = fma_lo(w.p[4 * l + 2], xv[4], a);
      a = fma_hi(w.p[4 * l + 2], xv[6], a);
      a = fma_lo(w.p[4 * l + 3], xv[5], a);
      a = fma_hi(w.p[4 * l + 3], xv[7], a);
    }
    return w.db * a;
  }

  // Grid entries as subnormal-half pairs (bytes 0,2 | 1,3 | 4,6 | 5,7) and the 128 sign
  // patterns (ksigns_iq2xs: index plus an even-parity bit) as sign-bit masks on the same pairs.
  __device__ static void init_lds(Lds &lds) {
    for (int i = threadIdx.x; i < 256; i += blockDim.x) {
      uint32_t b[8];
      for (int j = 0; j < 8; j++) b[j] = iq2_code_byte((kIq2xxsCodes[i] >> (2 * j)) & 3);
      lds.grid16[i][0] = b[0] | b[2] << 16;
      lds.grid16[i][1] = b[1] | b[3] << 16;
      lds.grid16[i][2] = b[4] | b[6] << 16;
      lds.grid16[i][3] = b[5] | b[7] << 16;
    }
    for (int i = threadIdx.x; i < 128; i += blockDim.x) {
      const uint32_t s = (uint32_t)i | ((uint32_t)(__builtin_popcount(i) & 1) << 7);
      uint32_t m[8];
      for (int j = 0; j < 8; j++) m[j] = ((s >> j) & 1) ? 0x8000u : 0u;
      lds.signs16[i][0] = m[0] | m[2] << 16;
      lds.signs16[i][1] = m[1] | m[3] << 16;
      lds.signs16[i][2] = m[4] | m[6] << 16;
      lds.signs16[i][3] = m[5] | m[7] << 16;
    }
  }
};

}  // namespace wl
