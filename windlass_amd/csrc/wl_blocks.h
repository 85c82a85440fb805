// wl_blocks.h - exact decoders of the GGUF block formats that have no hand-tuned GEMV codec
// of their own in the dequant and prefill kernels: Q4_0, Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, Q5_K
// and IQ4_NL.
//
// A decoder knows, for its block format (BLOCK values in BYTES bytes):
//   Raw   - the bytes 16 consecutive values of a block need, as aligned dwords,
//   load  - fetches them for the values at offset k (k % 16 == 0) of the block at blk,
//   dec   - produces those 16 values with the reference DecodeRow's fp32 operations in its
//           order (src/Quants.cs:189-370; src/IQuants.cs:45-58): the results are bit-exact.
// Blocks start at any 2-byte aligned address (18-, 22- and 110-byte blocks follow each other),
// so every load goes through an aligned dword window.
//
// Block layouts (ggml-common.h, restated in src/Quants.cs and src/IQuants.cs):
//   Q4_0    18 B / 32:  d f16 | qs[16]                  (low nibbles: values 0-15, high: 16-31)
//   Q4_1    20 B / 32:  d f16 | m f16 | qs[16]
//   Q5_0    22 B / 32:  d f16 | qh u32 | qs[16]         (bit e of qh: fifth bit of value e)
//   Q5_1    24 B / 32:  d f16 | m f16 | qh u32 | qs[16]
//   Q2_K    84 B / 256: scales[16] | qs[64] | d f16 | dmin f16
//   Q3_K   110 B / 256: hmask[32] | qs[64] | scales[12] | d f16
//   Q5_K   176 B / 256: d f16 | dmin f16 | scales[12] | qh[32] | qs[128]
//   IQ4_NL  18 B / 32:  d f16 | qs[16]                  (nibbles index kvalues_iq4nl)
#pragma once
#include "wl_device.h"
#include "wl_tables.h"

namespace wl {

// fp16 at byte offset `off` (even) of a dword window: the hardware conversion is exact for
// every finite half, and half_bits_exact keeps Inf/NaN payloads as the reference's table does.
template <int N>
__device__ __forceinline__ float win_half(const Win<N> &w, int off) {
  return half_bits_exact((w.dw(off / 4) >> (8 * (off % 4))) & 0xFFFFu);
}

// ---------------------------------------------------------------- 32-value formats
// Values k..k+15 of a 32-block: the low nibbles (k = 0) or the high nibbles (k = 16) of the
// block's 16 qs bytes.
__device__ __forceinline__ int nib(const Win<24> &w, int qs, int k, int j) {
  const uint32_t b = w.byte(qs + j);
  return (int)(k ? b >> 4 : b & 0xF);
}

// Every 32-value format's block fits one 24-byte window.
struct BlkSmall {
  struct Raw { Win<24> w; };
  __device__ static void load(const uint8_t *blk, int, Raw &r) { r.w.load(blk); }
};

struct BQ40 : BlkSmall {
  static constexpr int BLOCK = 32, BYTES = 18;
  __device__ static void dec(const Raw &r, int k, float (&y)[16]) {
    const float d = win_half(r.w, 0);
#pragma unroll
    for (int j = 0; j < 16; j++) y[j] = (float)(nib(r.w, 2, k, j) - 8) * d;  // src/Quants.cs:196-197
  }
};

struct BQ41 : BlkSmall {
  static constexpr int BLOCK = 32, BYTES = 20;
  __device__ static void dec(const Raw &r, int k, float (&y)[16]) {
    const float d = win_half(r.w, 0), m = win_half(r.w, 2);
#pragma unroll
    for (int j = 0; j < 16; j++) y[j] = (float)nib(r.w, 4, k, j) * d + m;  // src/Quants.cs:210-211
  }
};

// The 32-bit qh field at byte offset qh (2 or 4) of the block.
__device__ __forceinline__ uint32_t qh32(const Win<24> &w, int qh) {
  return qh % 4 == 0 ? w.dw(qh / 4) : __builtin_amdgcn_alignbit(w.dw(qh / 4 + 1), w.dw(qh / 4), 8 * (qh % 4));
}

// the fifth bit of value k + j is bit k + j of qh
__device__ __forceinline__ int q5(const Win<24> &w, int qh, int qs, int k, int j) {
  return nib(w, qs, k, j) | (int)(((qh32(w, qh) >> (k + j)) & 1u) << 4);
}

struct BQ50 : BlkSmall {
  static constexpr int BLOCK = 32, BYTES = 22;
  __device__ static void dec(const Raw &r, int k, float (&y)[16]) {
    const float d = win_half(r.w, 0);
#pragma unroll
    for (int j = 0; j < 16; j++) y[j] = (float)(q5(r.w, 2, 6, k, j) - 16) * d;  // src/Quants.cs:227-228
  }
};

struct BQ51 : BlkSmall {
  static constexpr int BLOCK = 32, BYTES = 24;
  __device__ static void dec(const Raw &r, int k, float (&y)[16]) {
    const float d = win_half(r.w, 0), m = win_half(r.w, 2);
#pragma unroll
    for (int j = 0; j < 16; j++) y[j] = (float)q5(r.w, 4, 8, k, j) * d + m;  // src/Quants.cs:245-246
  }
};

struct BIQ4NL : BlkSmall {
  static constexpr int BLOCK = 32, BYTES = 18;
  __device__ static void dec(const Raw &r, int k, float (&y)[16]) {
    const float d = win_half(r.w, 0);
#pragma unroll
    for (int j = 0; j < 16; j++) y[j] = d * (float)kKvaluesIq4nl[nib(r.w, 2, k, j)];  // src/IQuants.cs:54-55
  }
};

// ---------------------------------------------------------------- IQ3_S and IQ2_S
// The 16 values at offset k of a block: 32-value sub-block sub = k / 32 and its 8-value groups
// l = 2 * ((k % 32) / 16) and l + 1. Read byte by byte from the block (Raw keeps its address).
struct BIqRaw {
  struct Raw { const uint8_t *b; };
  __device__ static void load(const uint8_t *blk, int, Raw &r) { r.b = blk; }
};

// IQ3_S (src/IQuants.cs:112-143): d, qs[64], qh[8], signs[32], scales[4]. y = db * grid byte *
// sign with db = d * (1 + 2 * the sub-block's scale nibble); grid index = qs byte 2l (values
// 0-3 of the group) or 2l + 1 (values 4-7) with bit 2l or 2l + 1 of qh[sub] as bit 8.
struct BIQ3S : BIqRaw {
  static constexpr int BLOCK = 256, BYTES = 110;
  __device__ static void dec(const Raw &r, int k, float (&y)[16]) {
    const uint8_t *b = r.b;
    const int sub = k / 32, l0 = 2 * ((k % 32) / 16);
    const float d = half_bits_exact((uint32_t)b[0] | ((uint32_t)b[1] << 8));
    const int sc = b[106 + sub / 2];
    const float db = d * (float)(1 + 2 * ((sub & 1) ? sc >> 4 : sc & 0xF));
    const int h = b[66 + sub];
#pragma unroll
    for (int g = 0; g < 2; g++) {
      const int l = l0 + g;
      const int i1 = b[2 + 8 * sub + 2 * l] | ((h << (8 - 2 * l)) & 256);
      const int i2 = b[2 + 8 * sub + 2 * l + 1] | ((h << (7 - 2 * l)) & 256);
      const int sg = b[74 + 4 * sub + l];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        y[8 * g + j] = db * (float)iq3s_grid_byte(i1, j) * ((sg >> j) & 1 ? -1.0f : 1.0f);
        y[8 * g + 4 + j] = db * (float)iq3s_grid_byte(i2, j) * ((sg >> (j + 4)) & 1 ? -1.0f : 1.0f);
      }
    }
  }
};

// IQ2_S (src/IQuants.cs:199-222): d, qs[32] grid bytes, signs[32], qh[8], scales[8]. y = dl *
// grid byte * sign, dl = d * (0.5 + nibble) * 0.25 (low nibble for groups 0-1, high for 2-3);
// grid index = qs byte of the group with bits 2l..2l+1 of qh[sub] as bits 8-9.
struct BIQ2S : BIqRaw {
  static constexpr int BLOCK = 256, BYTES = 82;
  __device__ static void dec(const Raw &r, int k, float (&y)[16]) {
    const uint8_t *b = r.b;
    const int sub = k / 32, l0 = 2 * ((k % 32) / 16);
    const float d = half_bits_exact((uint32_t)b[0] | ((uint32_t)b[1] << 8));
    const int sc = b[74 + sub], h = b[66 + sub];
#pragma unroll
    for (int g = 0; g < 2; g++) {
      const int l = l0 + g;
      const float dl = d * (0.5f + (float)(l < 2 ? sc & 0xF : sc >> 4)) * 0.25f;
      const int gi = b[2 + 4 * sub + l] | ((h << (8 - 2 * l)) & 0x300);
      const int sg = b[34 + 4 * sub + l];
#pragma unroll
      for (int j = 0; j < 8; j++) y[8 * g + j] = dl * (float)iq2s_grid_byte(gi, j) * ((sg >> j) & 1 ? -1.0f : 1.0f);
    }
  }
};

// ---------------------------------------------------------------- K-quants
// The 16 values at offset k of a Q2_K/Q3_K block: 128-value half h = k / 128, 2-bit field
// shift 2j with j = (k % 128) / 32, bytes l0 .. l0 + 15 of the half's 32 qs bytes
// (l0 = k % 32), scale index 8h + 2j + l0 / 16.
struct KRun {
  int h, j, l0, idx;
  __device__ explicit KRun(int k) : h(k / 128), j((k % 128) / 32), l0(k % 32), idx(8 * (k / 128) + 2 * ((k % 128) / 32) + (k % 32) / 16) {}
};

struct BQ2K {
  static constexpr int BLOCK = 256, BYTES = 84;
  struct Raw { Win<16> q; Win<4> s; Win<4> d; };
  __device__ static void load(const uint8_t *blk, int k, Raw &r) {
    const KRun u(k);
    r.q.load(blk + 16 + 32 * u.h + u.l0);
    r.s.load(blk + (u.idx & ~1));
    r.d.load(blk + 80);
  }
  __device__ static void dec(const Raw &r, int k, float (&y)[16]) {
    const KRun u(k);
    const float d = win_half(r.d, 0), dmin = win_half(r.d, 2);
    const uint32_t s = r.s.byte(u.idx & 1);
    const float dl = d * (float)(s & 0xF), ml = dmin * (float)(s >> 4);  // src/Quants.cs:272-273
#pragma unroll
    for (int l = 0; l < 16; l++) y[l] = dl * (float)((r.q.byte(l) >> (2 * u.j)) & 3) - ml;  // :274
  }
};

struct BQ3K {
  static constexpr int BLOCK = 256, BYTES = 110;
  struct Raw { Win<16> q, hm; Win<12> sc; Win<4> d; };
  __device__ static void load(const uint8_t *blk, int k, Raw &r) {
    const KRun u(k);
    r.q.load(blk + 32 + 32 * u.h + u.l0);
    r.hm.load(blk + u.l0);
    r.sc.load(blk + 96);
    r.d.load(blk + 108);
  }
  __device__ static void dec(const Raw &r, int k, float (&y)[16]) {
    const KRun u(k);
    const float dall = win_half(r.d, 0);
    // the 6-bit scale idx from its 12 packed bytes (the kmask shuffle, src/Quants.cs:295-301):
    // low four bits from byte idx (idx < 8) or the high nibble of byte idx - 8, top two bits
    // from bits 2*(idx/4) of byte 8 + idx % 4
    const uint32_t d0 = r.sc.dw(0), d1 = r.sc.dw(1), d2 = r.sc.dw(2);  // idx is not a constant:
    const int i8 = u.idx & 7;                                          // select, do not index
    const uint32_t lowb = ((i8 < 4 ? d0 : d1) >> (8 * (i8 & 3))) & 0xFFu;
    const uint32_t low4 = u.idx < 8 ? lowb & 0xF : lowb >> 4;
    const uint32_t high2 = (d2 >> (8 * (u.idx % 4) + 2 * (u.idx / 4))) & 3;
    const int sc = (int)(int8_t)(uint8_t)(low4 | (high2 << 4));
    const float dl = dall * (float)(sc - 32);  // src/Quants.cs:309
    const int m = 4 * u.h + u.j;               // the hmask bit of this run
#pragma unroll
    for (int l = 0; l < 16; l++) {
      const int q = (int)((r.q.byte(l) >> (2 * u.j)) & 3) - (((r.hm.byte(l) >> m) & 1) ? 0 : 4);
      y[l] = dl * (float)q;  // src/Quants.cs:310
    }
  }
};

// get_scale_min_k4 (src/Quants.cs:322-330) on the 12 scale bytes held in dwords 1..3 of a
// 16-byte header.
__device__ __forceinline__ void scale_min_k4_hdr(const uint4 &h, int j, int &sc, int &m) {
  const uint32_t w[3] = {h.y, h.z, h.w};
  auto B = [&](int i) { return (int)((w[i >> 2] >> (8 * (i & 3))) & 0xFFu); };
  if (j < 4) {
    sc = B(j) & 63;
    m = B(j + 4) & 63;
  } else {
    sc = (B(j + 4) & 0xF) | ((B(j - 4) >> 6) << 4);
    m = (B(j + 4) >> 4) | ((B(j) >> 6) << 4);
  }
}

struct BQ5K {
  static constexpr int BLOCK = 256, BYTES = 176;  // blocks are 16-byte aligned
  struct Raw { uint4 h, qh, ql; };
  __device__ static void load(const uint8_t *blk, int k, Raw &r) {
    const int sub = k / 32, l0 = k % 32;
    r.h = ld16(blk);
    r.qh = ld16(blk + 16 + l0);
    r.ql = ld16(blk + 48 + 32 * (sub / 2) + l0);
  }
  __device__ static void dec(const Raw &r, int k, float (&y)[16]) {
    const int sub = k / 32;
    const float d = half_bits_exact(r.h.x & 0xFFFFu), dmin = half_bits_exact(r.h.x >> 16);
    int s, m;
    scale_min_k4_hdr(r.h, sub, s, m);
    const float d1 = d * (float)s, m1 = dmin * (float)m;  // src/Quants.cs:362-363
    const uint32_t ql[4] = {r.ql.x, r.ql.y, r.ql.z, r.ql.w}, qh[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
#pragma unroll
    for (int l = 0; l < 16; l++) {
      const uint32_t b = (ql[l / 4] >> (8 * (l % 4))) & 0xFFu, hb = (qh[l / 4] >> (8 * (l % 4) + sub)) & 1u;
      const int q = (int)((sub & 1 ? b >> 4 : b & 0xF) + (hb ? 16 : 0));
      y[l] = d1 * (float)q - m1;  // src/Quants.cs:364-365
    }
  }
};

// ---------------------------------------------------------------- float rows
// F32 / F16 / BF16 rows (src/Quants.cs:36-38) in runs of 32 values, so they share the 32-value
// formats' geometry.
struct BF32 {
  static constexpr int BLOCK = 32, BYTES = 128;
  struct Raw { uint4 v[4]; };
  __device__ static void load(const uint8_t *blk, int k, Raw &r) {
#pragma unroll
    for (int i = 0; i < 4; i++) r.v[i] = ld16(blk + 4 * k + 16 * i);
  }
  __device__ static void dec(const Raw &r, int, float (&y)[16]) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      y[4 * i] = __uint_as_float(r.v[i].x);
      y[4 * i + 1] = __uint_as_float(r.v[i].y);
      y[4 * i + 2] = __uint_as_float(r.v[i].z);
      y[4 * i + 3] = __uint_as_float(r.v[i].w);
    }
  }
};

template <bool BF>
struct BHalfRow {
  static constexpr int BLOCK = 32, BYTES = 64;
  struct Raw { uint4 v[2]; };
  __device__ static void load(const uint8_t *blk, int k, Raw &r) {
    r.v[0] = ld16(blk + 2 * k);
    r.v[1] = ld16(blk + 2 * k + 16);
  }
  __device__ static void dec(const Raw &r, int, float (&y)[16]) {
    const uint32_t w[8] = {r.v[0].x, r.v[0].y, r.v[0].z, r.v[0].w, r.v[1].x, r.v[1].y, r.v[1].z, r.v[1].w};
#pragma unroll
    for (int i = 0; i < 8; i++) {
      if constexpr (BF) {
        y[2 * i] = __uint_as_float(w[i] << 16);  // Quants.Bf16 (src/Quants.cs:23-27)
        y[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
      } else {
        y[2 * i] = half_bits_exact(w[i] & 0xFFFFu);
        y[2 * i + 1] = half_bits_exact(w[i] >> 16);
      }
    }
  }
};
typedef BHalfRow<false> BF16h;
typedef BHalfRow<true> BBF16;

}  // namespace wl
