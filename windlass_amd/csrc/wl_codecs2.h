// wl_codecs2.h - decode GEMV lane codecs of the formats beyond the benchmark's five: Q4_0,
// Q4_1, Q5_0, Q5_1, IQ4_NL (32-value blocks, one lane per block), Q2_K, Q3_K, Q5_K (256-value
// blocks, eight lanes per block) and F32/F16/BF16 rows (runs of 32 values, one lane per run).
// The codec interface and the fp16-subnormal multiply-add are those of wl_codecs.h: quants enter
// v_fma_mix_f32 as n * 2^-24 (n in the low bits of a half) against x pre-scaled by 2^24, or by
// 2^20 for fields that sit four bits up.
//
// Block layouts: see wl_blocks.h (the exact decoders of the same formats).
#pragma once
#include "wl_codecs.h"

namespace wl {

// ------------------------------------------------------------ 32-value nibble formats
// The lane owns one whole block. Its x slice: values 0-15 (the low nibbles) scaled by 2^24,
// values 16-31 (the high nibbles, kept in bits 4-7) by 2^20, and the plain sum.
struct Xs32 { float v[32]; float s; };

__device__ __forceinline__ void load_x32(const float *xb, Xs32 &x) {
  ld_x16(xb, x.v);
  ld_x16(xb + 16, x.v + 16);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 32; i++) s += x.v[i];
  x.s = s;
#pragma unroll
  for (int i = 0; i < 16; i++) {
    x.v[i] *= kTwo24;
    x.v[16 + i] *= kTwo20;
  }
}

// Bit c of the 4-bit value b moved to bit 0 of byte c (the four shifted copies do not overlap,
// so the product has no carries).
__device__ __forceinline__ uint32_t spread4(uint32_t b) { return (b * 0x00204081u) & 0x01010101u; }

// The 16 qs bytes of a block as four dwords, the low nibbles (values 4i+c) and high nibbles
// (values 16+4i+c) of dword i as fp16 pairs: p[4i] = values (4i, 4i+2), p[4i+1] = (4i+1, 4i+3),
// p[4i+2] / p[4i+3] the same for the high nibbles (times 16). With qh (Q5 formats) the fifth
// bit of value e (bit e of qh) joins as bit 4 of the value.
template <bool Q5>
__device__ __forceinline__ void unpack_nibbles(const uint32_t (&q)[4], uint32_t qh, uint32_t (&p)[16]) {
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t v = q[i], v8 = v >> 8;
    uint32_t l02 = v & 0x000F000Fu, l13 = v8 & 0x000F000Fu, h02 = v & 0x00F000F0u, h13 = v8 & 0x00F000F0u;
    if constexpr (Q5) {
      const uint32_t sl = spread4((qh >> (4 * i)) & 0xF), sh = spread4((qh >> (16 + 4 * i)) & 0xF);
      l02 |= (sl << 4) & 0x00100010u;
      l13 |= (sl >> 4) & 0x00100010u;
      h02 |= (sh << 8) & 0x01000100u;
      h13 |= sh & 0x01000100u;
    }
    p[4 * i] = l02;
    p[4 * i + 1] = l13;
    p[4 * i + 2] = h02;
    p[4 * i + 3] = h13;
  }
}

__device__ __forceinline__ float dot_nibbles(const uint32_t (&p)[16], const Xs32 &x) {
  float a = 0.f;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    a = fma_lo(p[4 * i], x.v[4 * i + 0], a);
    a = fma_hi(p[4 * i], x.v[4 * i + 2], a);
    a = fma_lo(p[4 * i + 1], x.v[4 * i + 1], a);
    a = fma_hi(p[4 * i + 1], x.v[4 * i + 3], a);
    a = fma_lo(p[4 * i + 2], x.v[16 + 4 * i + 0], a);
    a = fma_hi(p[4 * i + 2], x.v[16 + 4 * i + 2], a);
    a = fma_lo(p[4 * i + 3], x.v[16 + 4 * i + 1], a);
    a = fma_hi(p[4 * i + 3], x.v[16 + 4 * i + 3], a);
  }
  return a;
}

// One 32-value block as loaded: the aligned dwords around it (blocks start 2-byte aligned) and
// the byte shift.
template <int BYTES_>
struct Raw32 {
  Win<(BYTES_ + 3) / 4 * 4> w;
  // dword i of the block's bytes from byte offset `off` (even)
  __device__ uint32_t at(int off, int i) const {
    return off % 4 == 0 ? w.dw(off / 4 + i) : __builtin_amdgcn_alignbit(w.dw(off / 4 + i + 1), w.dw(off / 4 + i), 16);
  }
};

// Q4_0 (src/Quants.cs:98-109): y = d * (n - 8).  Q4_1: y = n * d + m.
// Q5_0 (src/Quants.cs:216-231): y = d * (n5 - 16).  Q5_1: y = n5 * d + m.
template <int BYTES_, int QS, int QH, bool MIN>
struct Q32 {
  static constexpr int BLOCK = 32, BYTES = BYTES_, LPB = 1, NEED_LDS = 0, R1 = 4, SP2 = 1;
  struct Lane {};
  typedef Xs32 Xs;
  typedef Raw32<BYTES_> Raw;
  struct W { uint32_t p[16]; float d, m; };

  __device__ static Lane lane(int) { return Lane{}; }
  __device__ static void load_x(const float *xb, const Lane &, Xs &x) { load_x32(xb, x); }
  __device__ static void load(const uint8_t *blk, const Lane &, Raw &r) { r.w.load(blk); }

  __device__ static void unpack(const Raw &r, const Lane &, const Lds &, W &w) {
    const uint32_t h0 = r.w.dw(0);
    w.d = half_lo(h0);
    w.m = MIN ? half_hi(h0) : 0.f;
    const uint32_t q[4] = {r.at(QS, 0), r.at(QS, 1), r.at(QS, 2), r.at(QS, 3)};
    unpack_nibbles<(QH > 0)>(q, QH > 0 ? r.at(QH, 0) : 0u, w.p);
  }

  __device__ static float dot(const W &w, const Xs &x) {
    const float a = dot_nibbles(w.p, x);
    if constexpr (MIN) return __builtin_fmaf(w.d, a, w.m * x.s);  // sum((n*d + m) * x)
    constexpr float off = QH > 0 ? -16.f : -8.f;
    return w.d * __builtin_fmaf(off, x.s, a);                      // d * sum((n - off) * x)
  }
};

typedef Q32<18, 2, 0, false> Q40;
typedef Q32<20, 4, 0, true> Q41;
typedef Q32<22, 6, 2, false> Q50;
typedef Q32<24, 8, 4, true> Q51;

// IQ4_NL (src/IQuants.cs:45-58): y = d * kvalues[n], through IQ4_XS's LDS table of
// (kvalue[low] + 128, kvalue[high] + 128) fp16 pairs indexed by a whole qs byte.
// TABLE: the words of the qs bytes from the LDS table (one-token launches); otherwise looked up
// in registers into the same words (the batched launches), as IQ4_XS does.
template <bool TABLE>
struct IQ4NLc {
  static constexpr int BLOCK = 32, BYTES = 18, LPB = 1, NEED_LDS = TABLE ? 2 : 0, R1 = 4, SP2 = 1;
  struct Lane {};
  struct Xs { float v[32]; float s; };
  typedef Raw32<18> Raw;
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
  __device__ static void load(const uint8_t *blk, const Lane &, Raw &r) { r.w.load(blk); }
  __device__ static void unpack(const Raw &r, const Lane &, const Lds &lds, W &w) {
    w.d = half_lo(r.w.dw(0));
    const uint32_t q[4] = {r.at(2, 0), r.at(2, 1), r.at(2, 2), r.at(2, 3)};
    if constexpr (TABLE) {
#pragma unroll
      for (int k = 0; k < 16; k++) w.p[k] = lds.iq4[(q[k >> 2] >> (8 * (k & 3))) & 0xFF];
    } else {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint32_t lo = IQ4XS::lookup(q[i] & 0x0F0F0F0Fu);
        const uint32_t hi = IQ4XS::lookup((q[i] >> 4) & 0x0F0F0F0Fu);
#pragma unroll
        for (int b = 0; b < 4; b++)
          w.p[4 * i + b] = __builtin_amdgcn_perm(hi, lo, (uint32_t)b | 0x0C00u | (uint32_t)(4 + b) << 16 | 0x0C000000u);
      }
    }
  }
  __device__ static float dot(const W &w, const Xs &x) {
    float a = 0.f;
#pragma unroll
    for (int k = 0; k < 16; k++) {
      a = fma_lo(w.p[k], x.v[k], a);
      a = fma_hi(w.p[k], x.v[16 + k], a);
    }
    return w.d * __builtin_fmaf(-128.f, x.s, a);  // d * sum((kv + 128) * x - 128 * x)
  }
  __device__ static void init_lds(Lds &lds) { IQ4XS::init_lds(lds); }
};
using IQ4NL = IQ4NLc<true>;    // one-token launches, the MoE experts
using IQ4NLR = IQ4NLc<false>;  // the batched launches

// ------------------------------------------------------------------ Q2_K and Q3_K
// Lane slice: run r = sub of the block, i.e. 128-value half kk = sub / 4 and 2-bit field
// shift 2j with j = sub % 4: values 32*sub + l for l = 0..31, the fields of the half's 32 qs
// bytes; values l < 16 take scale 8kk + 2j, the rest 8kk + 2j + 1.
struct LaneK2 { int kk, j; };
struct XsK2 { float v[32]; float s0, s1; };

__device__ __forceinline__ void load_x_k2(const float *xb, int sub, XsK2 &x) {
  ld_x16(xb + 32 * sub, x.v);
  ld_x16(xb + 32 * sub + 16, x.v + 16);
  float a = 0.f, b = 0.f;
#pragma unroll
  for (int i = 0; i < 16; i++) {
    a += x.v[i];
    b += x.v[16 + i];
  }
  x.s0 = a;
  x.s1 = b;
#pragma unroll
  for (int i = 0; i < 32; i++) x.v[i] *= kTwo24;
}

// The 2-bit fields (plus the Q3_K high bit at bit 2) of bytes l = 4i..4i+3 as fp16 pairs:
// p[2i] = (l, l+2), p[2i+1] = (l+1, l+3); the two 16-value runs' partial sums.
__device__ __forceinline__ void dot_k2(const uint32_t (&p)[16], const XsK2 &x, float &a0, float &a1) {
  a0 = 0.f;
  a1 = 0.f;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    a0 = fma_lo(p[2 * i], x.v[4 * i + 0], a0);
    a0 = fma_hi(p[2 * i], x.v[4 * i + 2], a0);
    a0 = fma_lo(p[2 * i + 1], x.v[4 * i + 1], a0);
    a0 = fma_hi(p[2 * i + 1], x.v[4 * i + 3], a0);
    a1 = fma_lo(p[8 + 2 * i], x.v[16 + 4 * i + 0], a1);
    a1 = fma_hi(p[8 + 2 * i], x.v[16 + 4 * i + 2], a1);
    a1 = fma_lo(p[8 + 2 * i + 1], x.v[16 + 4 * i + 1], a1);
    a1 = fma_hi(p[8 + 2 * i + 1], x.v[16 + 4 * i + 3], a1);
  }
}

#ifndef WL_Q2K_R1
#define WL_Q2K_R1 4
#endif
#ifndef WL_Q3K_R1
#define WL_Q3K_R1 4
#endif

// Q2_K (src/Quants.cs:261-285): y = d*(s & 15) * q2 - dmin*(s >> 4). Blocks are 4-byte aligned.
struct Q2K {
  static constexpr int BLOCK = 256, BYTES = 84, LPB = 8, NEED_LDS = 0, R1 = WL_Q2K_R1, SP2 = 1;
  typedef LaneK2 Lane;
  typedef XsK2 Xs;
  struct Raw { uint32_t q[8], sc, d; };
  struct W { uint32_t p[16]; float dl0, ml0, dl1, ml1; };

  __device__ static Lane lane(int sub) { return Lane{sub >> 2, sub & 3}; }
  __device__ static void load_x(const float *xb, const Lane &L, Xs &x) { load_x_k2(xb, 4 * L.kk + L.j, x); }
  __device__ static void load(const uint8_t *blk, const Lane &L, Raw &r) {
    gu32 *a = align4_down(blk);  // aligned: 84 = 4 * 21
    if constexpr (WL_WIDE_LOADS) {
#pragma unroll
      for (int i = 0; i < 8; i += 4) {
        const u32x4a4_t v = *reinterpret_cast<gu32x4 *>(a + 4 + 8 * L.kk + i);
        r.q[i] = v.x;
        r.q[i + 1] = v.y;
        r.q[i + 2] = v.z;
        r.q[i + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; i++) r.q[i] = ldw4(a + 4 + 8 * L.kk + i);
    }
    r.sc = ldw4(a + (8 * L.kk + 2 * L.j) / 4);
    r.d = ldw4(a + 20);
  }
  __device__ static void unpack(const Raw &r, const Lane &L, const Lds &, W &w) {
    const uint32_t s = r.sc >> (8 * ((2 * L.j) & 3)), s0 = s & 0xFF, s1 = (s >> 8) & 0xFF;
    const float d = half_lo(r.d), dmin = half_hi(r.d);
    w.dl0 = d * (float)(s0 & 0xF);
    w.ml0 = dmin * (float)(s0 >> 4);
    w.dl1 = d * (float)(s1 & 0xF);
    w.ml1 = dmin * (float)(s1 >> 4);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const uint32_t t = r.q[i] >> (2 * L.j);
      w.p[2 * i] = t & 0x00030003u;
      w.p[2 * i + 1] = (t >> 8) & 0x00030003u;
    }
  }
  __device__ static float dot(const W &w, const Xs &x) {
    float a0, a1;
    dot_k2(w.p, x, a0, a1);
    return __builtin_fmaf(w.dl0, a0, -(w.ml0 * x.s0)) + __builtin_fmaf(w.dl1, a1, -(w.ml1 * x.s1));
  }
};

// Q3_K (src/Quants.cs:287-319): y = d*(sc - 32) * (q2 - (h ? 0 : 4)), h = bit 4kk + j of
// hmask[l]; q2 + 4h enters as a 3-bit field and 4 * sum(x) is taken off.
struct Q3K {
  static constexpr int BLOCK = 256, BYTES = 110, LPB = 8, NEED_LDS = 0, R1 = WL_Q3K_R1, SP2 = 1;
  typedef LaneK2 Lane;
  typedef XsK2 Xs;
  struct Raw { Win<32> q, hm; Win<12> sc; Win<4> d; };
  struct W { uint32_t p[16]; float dl0, dl1; };

  __device__ static Lane lane(int sub) { return Lane{sub >> 2, sub & 3}; }
  __device__ static void load_x(const float *xb, const Lane &L, Xs &x) { load_x_k2(xb, 4 * L.kk + L.j, x); }
  __device__ static void load(const uint8_t *blk, const Lane &L, Raw &r) {
    r.q.load(blk + 32 + 32 * L.kk);
    r.hm.load(blk);
    r.sc.load(blk + 96);
    r.d.load(blk + 108);
  }
  // the 6-bit scale i (lane-constant, not a compile-time index) from the 12 packed bytes s0..s2,
  // selected arithmetically (an array here would be indexed through scratch memory)
  __device__ static int scale(uint32_t s0, uint32_t s1, uint32_t s2, int i) {
    const int i8 = i & 7;
    const uint32_t lowb = ((i8 < 4 ? s0 : s1) >> (8 * (i8 & 3))) & 0xFFu;
    const uint32_t low4 = i < 8 ? lowb & 0xF : lowb >> 4;
    const uint32_t high2 = (s2 >> (8 * (i % 4) + 2 * (i / 4))) & 3;
    return (int)(low4 | (high2 << 4)) - 32;
  }
  __device__ static void unpack(const Raw &r, const Lane &L, const Lds &, W &w) {
    const float dall = half_lo(r.d.dw(0));
    const uint32_t s0 = r.sc.dw(0), s1 = r.sc.dw(1), s2 = r.sc.dw(2);
    const int i0 = 8 * L.kk + 2 * L.j;
    w.dl0 = dall * (float)scale(s0, s1, s2, i0);
    w.dl1 = dall * (float)scale(s0, s1, s2, i0 + 1);
    const int hb = 4 * L.kk + L.j;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const uint32_t t = r.q.dw(i) >> (2 * L.j), g = r.hm.dw(i) >> hb;
      w.p[2 * i] = (t & 0x00030003u) | ((g & 0x00010001u) << 2);
      w.p[2 * i + 1] = ((t >> 8) & 0x00030003u) | (((g >> 8) & 0x00010001u) << 2);
    }
  }
  __device__ static float dot(const W &w, const Xs &x) {
    float a0, a1;
    dot_k2(w.p, x, a0, a1);
    return __builtin_fmaf(w.dl1, __builtin_fmaf(-4.f, x.s1, a1), w.dl0 * __builtin_fmaf(-4.f, x.s0, a0));
  }
};

// ------------------------------------------------------------------------- Q5_K
// Q4_K's lane slice, Xs, W and dot (src/Quants.cs:134-158) with the fifth bit of every value
// from qh[l] (bit 2j for the low nibbles, 2j+1 for the high ones) merged into the fp16 pairs.
struct Q5K : Q4K {
  static constexpr int BYTES = 176;
  struct Raw { uint4 hdr, q, qh; };

  __device__ static void load(const uint8_t *blk, const Lane &L, Raw &r) {
    r.hdr = ldw16(blk);
    r.q = ldw16(blk + 48 + 16 * (2 * L.j + L.h));
    r.qh = ldw16(blk + 16 + 16 * L.h);
  }
  __device__ static void unpack(const Raw &r, const Lane &L, const Lds &lds, W &w) {
    Q4K::Raw r4;
    r4.hdr = r.hdr;
    r4.q = r.q;
    Q4K::unpack(r4, L, lds, w);
    const uint32_t qh[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t hs = qh[i] >> (2 * L.j);  // bit 0 of each byte: low nibble's bit, bit 1: high's
      w.m[4 * i + 0] |= (hs << 4) & 0x00100010u;
      w.m[4 * i + 1] |= (hs >> 4) & 0x00100010u;
      w.m[4 * i + 2] |= (hs << 7) & 0x01000100u;
      w.m[4 * i + 3] |= (hs >> 1) & 0x01000100u;
    }
  }
};

// ------------------------------------------------------------------- float rows
// F32 / F16 / BF16 rows (src/Quants.cs:67-85) in runs of 32 values, one lane per run.
struct F16c {
  static constexpr int BLOCK = 32, BYTES = 64, LPB = 1, NEED_LDS = 0, R1 = 4, SP2 = 1;
  struct Lane {};
  struct Xs { float v[32]; };
  struct Raw { uint4 q[4]; };
  struct W { uint32_t p[16]; };

  __device__ static Lane lane(int) { return Lane{}; }
  __device__ static void load_x(const float *xb, const Lane &, Xs &x) {
    ld_x16(xb, x.v);
    ld_x16(xb + 16, x.v + 16);
  }
  __device__ static void load(const uint8_t *blk, const Lane &, Raw &r) {
#pragma unroll
    for (int i = 0; i < 4; i++) r.q[i] = ldw16(blk + 16 * i);
  }
  __device__ static void unpack(const Raw &r, const Lane &, const Lds &, W &w) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      w.p[4 * i] = r.q[i].x;
      w.p[4 * i + 1] = r.q[i].y;
      w.p[4 * i + 2] = r.q[i].z;
      w.p[4 * i + 3] = r.q[i].w;
    }
  }
  __device__ static float dot(const W &w, const Xs &x) {
    float a = 0.f;
#pragma unroll
    for (int k = 0; k < 16; k++) {
      a = fma_lo(w.p[k], x.v[2 * k], a);  // the weights are fp16 already
      a = fma_hi(w.p[k], x.v[2 * k + 1], a);
    }
    return a;
  }
};

template <bool BF>
struct F32Row {
  static constexpr int BLOCK = 32, BYTES = BF ? 64 : 128, LPB = 1, NEED_LDS = 0, R1 = 2, SP2 = 0;
  struct Lane {};
  struct Xs { float v[32]; };
  struct Raw { uint4 q[BF ? 4 : 8]; };
  struct W { float v[32]; };

  __device__ static Lane lane(int) { return Lane{}; }
  __device__ static void load_x(const float *xb, const Lane &, Xs &x) {
    ld_x16(xb, x.v);
    ld_x16(xb + 16, x.v + 16);
  }
  __device__ static void load(const uint8_t *blk, const Lane &, Raw &r) {
#pragma unroll
    for (int i = 0; i < (BF ? 4 : 8); i++) r.q[i] = ldw16(blk + 16 * i);
  }
  __device__ static void unpack(const Raw &r, const Lane &, const Lds &, W &w) {
#pragma unroll
    for (int i = 0; i < (BF ? 4 : 8); i++) {
      const uint32_t u[4] = {r.q[i].x, r.q[i].y, r.q[i].z, r.q[i].w};
#pragma unroll
      for (int c = 0; c < 4; c++) {
        if constexpr (BF) {
          w.v[8 * i + 2 * c] = __uint_as_float(u[c] << 16);  // Quants.Bf16 (src/Quants.cs:23-27)
          w.v[8 * i + 2 * c + 1] = __uint_as_float(u[c] & 0xFFFF0000u);
        } else {
          w.v[4 * i + c] = __uint_as_float(u[c]);
        }
      }
    }
  }
  __device__ static float dot(const W &w, const Xs &x) {
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int k = 0; k < 16; k++) {
      a = __builtin_fmaf(w.v[2 * k], x.v[2 * k], a);
      b = __builtin_fmaf(w.v[2 * k + 1], x.v[2 * k + 1], b);
    }
    return a + b;
  }
};
typedef F32Row<false> F32c;
typedef F32Row<true> BF16c;

// Float rows whose length is a multiple of 2048, read coalesced: the whole wave-column is one
// "block" (LPB = 64) and lane `sub` owns the 16-byte pieces at 1024k + 16*sub of it (k < 4 for
// 2-byte values, k < 8 for F32), so every load instruction of a wave reads 1 KB contiguous. (The
// 32-value runs above give each lane 64 or 128 contiguous bytes, which a wave reads 16 bytes per
// lane at a 64- or 128-byte stride.) KIND: 0 F32, 1 F16, 2 BF16.
template <int KIND>
struct FWide {
  static constexpr int E = KIND == 0 ? 4 : 2;            // bytes per value
  static constexpr int NQ = KIND == 0 ? 8 : 4;           // 16-byte pieces per lane
  static constexpr int PER = 16 / E;                     // values per piece
  static constexpr int BLOCK = 2048, BYTES = 2048 * E, LPB = 64, NEED_LDS = 0, R1 = KIND == 1 ? 4 : 2, SP2 = 0;
  struct Lane { int sub; };
  struct Xs { float v[32]; };
  struct Raw { uint4 q[NQ]; };
  struct W { uint32_t p[KIND == 1 ? 16 : 32]; };

  __device__ static Lane lane(int sub) { return Lane{sub}; }
  // piece k holds values (1024k + 16 sub) / E .. + PER of the wave-column
  __device__ static void load_x(const float *xb, const Lane &L, Xs &x) {
#pragma unroll
    for (int k = 0; k < NQ; k++) {
      const float4 *q = reinterpret_cast<const float4 *>(xb + (1024 * k + 16 * L.sub) / E);
#pragma unroll
      for (int i = 0; i < PER / 4; i++) {
        const float4 f = q[i];
        x.v[PER * k + 4 * i] = f.x;
        x.v[PER * k + 4 * i + 1] = f.y;
        x.v[PER * k + 4 * i + 2] = f.z;
        x.v[PER * k + 4 * i + 3] = f.w;
      }
    }
  }
  __device__ static void load(const uint8_t *blk, const Lane &L, Raw &r) {
#pragma unroll
    for (int k = 0; k < NQ; k++) r.q[k] = ldw16(blk + 1024 * k + 16 * L.sub);
  }
  __device__ static void unpack(const Raw &r, const Lane &, const Lds &, W &w) {
#pragma unroll
    for (int k = 0; k < NQ; k++) {
      const uint32_t u[4] = {r.q[k].x, r.q[k].y, r.q[k].z, r.q[k].w};
#pragma unroll
      for (int c = 0; c < 4; c++) {
        if constexpr (KIND == 1) {
          w.p[4 * k + c] = u[c];  // two fp16 values, used as they are
        } else if constexpr (KIND == 2) {
          w.p[8 * k + 2 * c] = u[c] << 16;  // Quants.Bf16 (src/Quants.cs:23-27)
          w.p[8 * k + 2 * c + 1] = u[c] & 0xFFFF0000u;
        } else {
          w.p[4 * k + c] = u[c];
        }
      }
    }
  }
  __device__ static float dot(const W &w, const Xs &x) {
    float a = 0.f, b = 0.f;
    if constexpr (KIND == 1) {
#pragma unroll
      for (int k = 0; k < 16; k++) {
        a = fma_lo(w.p[k], x.v[2 * k], a);
        b = fma_hi(w.p[k], x.v[2 * k + 1], b);
      }
    } else {
#pragma unroll
      for (int k = 0; k < 16; k++) {
        a = __builtin_fmaf(__uint_as_float(w.p[2 * k]), x.v[2 * k], a);
        b = __builtin_fmaf(__uint_as_float(w.p[2 * k + 1]), x.v[2 * k + 1], b);
      }
    }
    return a + b;
  }
};
typedef FWide<0> F32w;
typedef FWide<1> F16w;
typedef FWide<2> BF16w;


// A sign byte's 8 bits as 8 bytes, 0x80 where the bit is set (the fp16 sign bit of a value byte
// placed below it): one LDS table of the 256 patterns.
__device__ inline void init_sign_bytes(uint2 *t) {
  for (int i = threadIdx.x; i < 256; i += blockDim.x) {
    uint32_t m[8];
    for (int j = 0; j < 8; j++) m[j] = ((i >> j) & 1) ? 0x80u : 0u;
    t[i] = make_uint2(m[0] | m[1] << 8 | m[2] << 16 | m[3] << 24, m[4] | m[5] << 8 | m[6] << 16 | m[7] << 24);
  }
}

// Eight signed values as four fp16 pairs from value bytes g and sign bytes sg (0x80 / 0x00): the
// pairs (0,2) (1,3) (4,6) (5,7), each value a subnormal with its sign.
__device__ __forceinline__ void signed_pairs(uint2 g, uint2 sg, uint32_t *p) {
  p[0] = __builtin_amdgcn_perm(sg.x, g.x, 0x06020400u);
  p[1] = __builtin_amdgcn_perm(sg.x, g.x, 0x07030501u);
  p[2] = __builtin_amdgcn_perm(sg.y, g.y, 0x06020400u);
  p[3] = __builtin_amdgcn_perm(sg.y, g.y, 0x07030501u);
}

// The dot of one group of 8 (pairs as signed_pairs lays them out) onto chain acc.
__device__ __forceinline__ float group_dot(const uint32_t *p, const float *x, float acc) {
  acc = fma_lo(p[0], x[0], acc);
  acc = fma_hi(p[0], x[2], acc);
  acc = fma_lo(p[1], x[1], acc);
  acc = fma_hi(p[1], x[3], acc);
  acc = fma_lo(p[2], x[4], acc);
  acc = fma_hi(p[2], x[6], acc);
  acc = fma_lo(p[3], x[5], acc);
  return fma_hi(p[3], x[7], acc);
}

// The byte at p (any alignment) from its aligned dword.
__device__ __forceinline__ uint32_t ld_byte(const uint8_t *p) {
  return (ldw4(align4_down(p)) >> (8 * misalign4(p))) & 0xFF;
}

// -------------------------------------------------------------------------- IQ2_S
// block_iq2_s (82 B, src/IQuants.cs:199-222): d f16 | 32 grid bytes | 32 sign bytes | qh[8] |
// scales[8]. Lane slice: sub-block ib = sub (32 values): grid bytes 4ib.. with two index bits
// each from qh[ib] (10-bit index into the 1024-entry grid), sign bytes 4ib.., and the scales
// byte ib (groups 0, 1: low nibble; 2, 3: high), db = d * (0.5 + s) * 0.25.
struct IQ2S {
  static constexpr int BLOCK = 256, BYTES = 82, LPB = 8, NEED_LDS = 1, R1 = 8, SP2 = 1;
  struct Lane { int ib; };
  struct Xs { float v[32]; };
  struct Raw { uint32_t dw, g[2], s[2], qh, sc; uint32_t dsh, sh; };
  struct W { uint32_t p[16]; float db0, db1; };

  __device__ static Lane lane(int sub) { return Lane{sub}; }

  __device__ static void load_x(const float *xb, const Lane &L, Xs &x) {
    ld_x16(xb + 32 * L.ib, x.v);
    ld_x16(xb + 32 * L.ib + 16, x.v + 16);
#pragma unroll
    for (int i = 0; i < 32; i++) x.v[i] *= kTwo24;
  }

  __device__ static void load(const uint8_t *blk, const Lane &L, Raw &r) {
    r.dw = ldw4(align4_down(blk));
    r.dsh = misalign4(blk) & 2;
    const uint8_t *pg = blk + 2 + 4 * L.ib;  // the sign bytes follow 32 bytes later: the same alignment
    gu32 *a = align4_down(pg), *b = align4_down(pg + 32);
    r.sh = misalign4(pg) * 8;
    r.g[0] = ldw4(a);
    r.g[1] = ldw4(a + 1);
    r.s[0] = ldw4(b);
    r.s[1] = ldw4(b + 1);
    r.qh = ld_byte(blk + 66 + L.ib);
    r.sc = ld_byte(blk + 74 + L.ib);
  }

  __device__ static void unpack(const Raw &r, const Lane &, const Lds &lds, W &w) {
    const float d = half_lo(r.dsh ? (r.dw >> 16) : r.dw);
    w.db0 = d * (0.5f + (float)(r.sc & 0xF)) * 0.25f;  // src/IQuants.cs:210-211
    w.db1 = d * (0.5f + (float)(r.sc >> 4)) * 0.25f;
    const uint32_t g4 = __builtin_amdgcn_alignbit(r.g[1], r.g[0], r.sh);
    const uint32_t s4 = __builtin_amdgcn_alignbit(r.s[1], r.s[0], r.sh);
#pragma unroll
    for (int l = 0; l < 4; l++) {
      const uint32_t gi = ((g4 >> (8 * l)) & 0xFF) | (((r.qh >> (2 * l)) & 3) << 8);  // :215
      signed_pairs(lds.grid2s[gi], lds.sgn2s[(s4 >> (8 * l)) & 0xFF], w.p + 4 * l);
    }
  }

  // groups 0, 1 (scale db0) on one chain and 2, 3 (db1) on the other, interleaved
  __device__ static float dot(const W &w, const Xs &x) {
    float a = 0.f, b = 0.f;
    a = group_dot(w.p, x.v, a);
    b = group_dot(w.p + 8, x.v + 16, b);
    a = group_dot(w.p + 4, x.v + 8, a);
    b = group_dot(w.p + 12, x.v + 24, b);
    return __builtin_fmaf(w.db1, b, w.db0 * a);
  }

  __device__ static void init_lds(Lds &lds) {
    for (int i = threadIdx.x; i < 1024; i += blockDim.x) {
      uint32_t b[8];
      for (int j = 0; j < 8; j++) b[j] = iq2s_grid_byte(i, j);
      lds.grid2s[i] = make_uint2(b[0] | b[1] << 8 | b[2] << 16 | b[3] << 24, b[4] | b[5] << 8 | b[6] << 16 | b[7] << 24);
    }
    init_sign_bytes(lds.sgn2s);
  }
};

// -------------------------------------------------------------------------- IQ3_S
// block_iq3_s (110 B, src/IQuants.cs:112-143): d f16 | qs[64] | qh[8] | signs[32] | scales[4].
// Lane slice: sub-block ib = sub: grid indices qs[8ib..] with a ninth bit each from qh[ib]
// (512-entry grid of 4 values), sign bytes 4ib.. (one per 8 values), and the nibble ib & 1 of
// scales[ib / 2], db = d * (1 + 2 s).
struct IQ3S {
  static constexpr int BLOCK = 256, BYTES = 110, LPB = 8, NEED_LDS = 1, R1 = 8, SP2 = 1;
  struct Lane { int ib; };
  struct Xs { float v[32]; };
  struct Raw { uint32_t dw, q[3], s[2], qh, sc; uint32_t dsh, sh; };
  struct W { uint32_t p[16]; float db; };

  __device__ static Lane lane(int sub) { return Lane{sub}; }

  __device__ static void load_x(const float *xb, const Lane &L, Xs &x) {
    ld_x16(xb + 32 * L.ib, x.v);
    ld_x16(xb + 32 * L.ib + 16, x.v + 16);
#pragma unroll
    for (int i = 0; i < 32; i++) x.v[i] *= kTwo24;
  }

  __device__ static void load(const uint8_t *blk, const Lane &L, Raw &r) {
    r.dw = ldw4(align4_down(blk));
    r.dsh = misalign4(blk) & 2;
    const uint8_t *pq = blk + 2 + 8 * L.ib, *ps = blk + 74 + 4 * L.ib;  // both at the block's alignment
    gu32 *a = align4_down(pq), *b = align4_down(ps);
    r.sh = misalign4(pq) * 8;
    r.q[0] = ldw4(a);
    r.q[1] = ldw4(a + 1);
    r.q[2] = ldw4(a + 2);
    r.s[0] = ldw4(b);
    r.s[1] = ldw4(b + 1);
    r.qh = ld_byte(blk + 66 + L.ib);
    r.sc = ld_byte(blk + 106 + L.ib / 2) >> (4 * (L.ib & 1));
  }

  __device__ static void unpack(const Raw &r, const Lane &, const Lds &lds, W &w) {
    const float d = half_lo(r.dsh ? (r.dw >> 16) : r.dw);
    w.db = d * (float)(1 + 2 * (int)(r.sc & 0xF));  // src/IQuants.cs:121-122
    const uint32_t q03 = __builtin_amdgcn_alignbit(r.q[1], r.q[0], r.sh);
    const uint32_t q47 = __builtin_amdgcn_alignbit(r.q[2], r.q[1], r.sh);
    const uint32_t s4 = __builtin_amdgcn_alignbit(r.s[1], r.s[0], r.sh);
    const uint32_t h = r.qh;
#pragma unroll
    for (int l = 0; l < 4; l++) {
      const uint32_t qw = l < 2 ? q03 : q47;
      const uint32_t i1 = ((qw >> (16 * (l & 1))) & 0xFF) | ((h << (8 - 2 * l)) & 256);      // :130
      const uint32_t i2 = ((qw >> (16 * (l & 1) + 8)) & 0xFF) | ((h << (7 - 2 * l)) & 256);  // :131
      signed_pairs(make_uint2(lds.grid3s[i1], lds.grid3s[i2]), lds.sgn3s[(s4 >> (8 * l)) & 0xFF], w.p + 4 * l);
    }
  }

  // groups 0, 2 and 1, 3 on two chains
  __device__ static float dot(const W &w, const Xs &x) {
    float a = 0.f, b = 0.f;
    a = group_dot(w.p, x.v, a);
    b = group_dot(w.p + 4, x.v + 8, b);
    a = group_dot(w.p + 8, x.v + 16, a);
    b = group_dot(w.p + 12, x.v + 24, b);
    return w.db * (a + b);
  }

  __device__ static void init_lds(Lds &lds) {
    for (int i = threadIdx.x; i < 512; i += blockDim.x) {
      uint32_t g = 0;
      for (int j = 0; j < 4; j++) g |= iq3s_grid_byte(i, j) << (8 * j);
      lds.grid3s[i] = g;
    }
    init_sign_bytes(lds.sgn3s);
  }
};

}  // namespace wl
