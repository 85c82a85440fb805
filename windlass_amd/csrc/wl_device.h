// wl_device.h - device-side building blocks shared by the kernels: fp16 decoding, aligned
// loads of 2-byte-aligned GGUF fields, and the fp16-denormal multiply-add used by the GEMVs.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wl {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

// Exact fp16 -> fp32 from the bit fields (sign, 5-bit exponent, 10-bit mantissa), including
// subnormals, Inf and NaN payloads, as the reference's table decode does
// (src/Half.cs:59-90). Used where the result must be bit-exact (dequantization).
__device__ __forceinline__ float half_bits_exact(uint32_t h) {
  uint32_t sign = (h >> 15) << 31;
  uint32_t exp = (h >> 10) & 0x1F;
  uint32_t mant = h & 0x3FF;
  uint32_t bits;
  if (exp == 0) {
    if (mant == 0) {
      bits = sign;
    } else {
      // normalise: the leading one of mant moves to bit 10
      uint32_t lz = __builtin_clz(mant) - 21;  // shifts needed, 1..10
      mant = (mant << lz) & 0x3FF;
      bits = sign | ((113u - lz) << 23) | (mant << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7F800000u | (mant << 13);
  } else {
    bits = sign | ((exp + 112u) << 23) | (mant << 13);
  }
  return __uint_as_float(bits);
}

// binary32 -> binary16 as Half.FromFloat gives it (src/Half.cs:29-57): round to nearest even
// through the subnormals, overflow to infinity, a NaN to the quiet NaN 0x7e00 with its sign.
// Integer arithmetic, so the bits do not depend on the hardware conversion's rounding mode or
// its handling of fp16 subnormals.
__device__ __forceinline__ uint16_t to_half(float v) {
  const uint32_t f = __builtin_bit_cast(uint32_t, v);
  const uint32_t sign = (f >> 16) & 0x8000u, fe = (f >> 23) & 0xffu;
  uint32_t m = f & 0x7fffffu;
  if (fe == 0xffu) return (uint16_t)(sign | 0x7c00u | (m ? 0x200u : 0u));
  const int e = (int)fe - 112;  // the binary16 biased exponent
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  uint32_t h, rem, halfway;
  if (e <= 0) {  // subnormal result: the implicit bit joins the shifted significand
    if (e < -10) return (uint16_t)sign;
    m |= 0x800000u;
    const int sh = 14 - e;
    h = m >> sh;
    rem = m & ((1u << sh) - 1u);
    halfway = 1u << (sh - 1);
  } else {
    h = ((uint32_t)e << 10) | (m >> 13);
    rem = m & 0x1fffu;
    halfway = 0x1000u;
  }
  h += (rem > halfway || (rem == halfway && (h & 1u))) ? 1u : 0u;  // a carry may reach the exponent
  return (uint16_t)(sign | h);
}

// Hardware fp16 -> fp32 (exact for every finite value; used inside the GEMVs).
__device__ __forceinline__ float half_lo(uint32_t w) {
  return (float)__builtin_bit_cast(half2_t, w).x;
}
__device__ __forceinline__ float half_hi(uint32_t w) {
  return (float)__builtin_bit_cast(half2_t, w).y;
}

// acc + f16(pair.lo/hi) * x in one v_fma_mix_f32. With a small integer n in the low bits of
// a half (no exponent bits), the half is the subnormal n * 2^-24, so this is an exact
// integer-to-float conversion fused into the multiply-add, scaled by a power of two that
// the caller folds back into the block scale.
__device__ __forceinline__ float fma_lo(uint32_t pair, float x, float acc) {
  return __builtin_fmaf(half_lo(pair), x, acc);
}
__device__ __forceinline__ float fma_hi(uint32_t pair, float x, float acc) {
  return __builtin_fmaf(half_hi(pair), x, acc);
}

__device__ __forceinline__ uint4 ld16(const uint8_t *p) {
  return *reinterpret_cast<const uint4 *>(p);
}

// Weight loads. WL_WEIGHT_NT = 1 adds the nontemporal hint. It is off: neighbouring lanes of
// a wave read overlapping dword windows and shared block headers, and those reads hit in the
// cache only when the lines are kept (measured on the 70B layer: Q6_K down 3.98 -> 2.63 TB/s
// with the hint).
#ifndef WL_WEIGHT_NT
#define WL_WEIGHT_NT 0
#endif
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 ldw16(const uint8_t *p) {
  if constexpr (WL_WEIGHT_NT) {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
  } else {
    return *reinterpret_cast<const uint4 *>(p);
  }
}
__device__ __forceinline__ uint2 ldw8(const uint8_t *p) {
  if constexpr (WL_WEIGHT_NT) {
    const u32x2_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t *>(p));
    return make_uint2(v.x, v.y);
  } else {
    return *reinterpret_cast<const uint2 *>(p);
  }
}
__device__ __forceinline__ uint32_t ld4(const uint8_t *p) {
  return *reinterpret_cast<const uint32_t *>(p);
}

// Byte offset of p within its dword.
__device__ __forceinline__ uint32_t misalign4(const void *p) {
  return (uint32_t)(reinterpret_cast<uintptr_t>(p) & 3);
}

// Weight and activation buffers live in global memory; loads through this pointer type are
// global loads (a generic pointer rebuilt from an integer would otherwise become a flat load).
typedef const __attribute__((address_space(1))) uint32_t gu32;

// The dword-aligned address at or below p, in the global address space.
// (Clearing the low bits is one VALU instruction on the address's low dword; subtracting the
// misalignment was a 64-bit subtraction with borrow. 70B down 46.9 -> 45.7 us, Q8_0 4096x4096
// 7.63 -> 7.38 us.)
__device__ __forceinline__ gu32 *align4_down(const uint8_t *p) {
  return (gu32 *)(reinterpret_cast<uintptr_t>(p) & ~(uintptr_t)3);
}

// One weight dword (nontemporal as ldw16).
__device__ __forceinline__ uint32_t ldw4(gu32 *p) {
  if constexpr (WL_WEIGHT_NT) return __builtin_nontemporal_load(p);
  else return *p;
}

// Three consecutive weight dwords at a dword-aligned address in one load instruction (the
// hardware takes dword-aligned multi-dword global loads). WL_WIDE_LOADS = 0 issues three.
#ifndef WL_WIDE_LOADS
#define WL_WIDE_LOADS 1
#endif
typedef uint32_t u32x3a4_t __attribute__((ext_vector_type(3), aligned(4)));
typedef const __attribute__((address_space(1))) u32x3a4_t gu32x3;
typedef uint32_t u32x4a4_t __attribute__((ext_vector_type(4), aligned(4)));
typedef const __attribute__((address_space(1))) u32x4a4_t gu32x4;
__device__ __forceinline__ void ldw12(gu32 *p, uint32_t (&o)[3]) {
  if constexpr (WL_WIDE_LOADS) {
    const u32x3a4_t v = *reinterpret_cast<gu32x3 *>(p);
    o[0] = v.x;
    o[1] = v.y;
    o[2] = v.z;
  } else {
#pragma unroll
    for (int i = 0; i < 3; i++) o[i] = ldw4(p + i);
  }
}

// N (multiple of 4) bytes starting at a 2-byte aligned address: the dword window holding them
// (N/4 + 1 dwords) and the bit offset of the first byte.
template <int N>
struct Win {
  uint32_t w[N / 4 + 1];
  uint32_t sh;
  __device__ void load(const uint8_t *p) {
    gu32 *a = align4_down(p);
    sh = misalign4(p) * 8;
    constexpr int n = N / 4 + 1;
    if constexpr (WL_WIDE_LOADS) {
      // groups of four dwords in one instruction each, then the rest
#pragma unroll
      for (int i = 0; i + 4 <= n; i += 4) {
        const u32x4a4_t v = *reinterpret_cast<gu32x4 *>(a + i);
        w[i] = v.x;
        w[i + 1] = v.y;
        w[i + 2] = v.z;
        w[i + 3] = v.w;
      }
#pragma unroll
      for (int i = n / 4 * 4; i < n; i++) w[i] = a[i];
    } else {
#pragma unroll
      for (int i = 0; i < n; i++) w[i] = a[i];
    }
  }
  // dword i of the N bytes, and byte i
  __device__ uint32_t dw(int i) const { return __builtin_amdgcn_alignbit(w[i + 1], w[i], sh); }
  __device__ uint32_t byte(int i) const { return (dw(i / 4) >> (8 * (i % 4))) & 0xFFu; }
};

__device__ __forceinline__ void ld_x16(const float *p, float *v) {
  const float4 *q = reinterpret_cast<const float4 *>(p);
#pragma unroll
  for (int i = 0; i < 4; i++) {
    float4 f = q[i];
    v[4 * i] = f.x; v[4 * i + 1] = f.y; v[4 * i + 2] = f.z; v[4 * i + 3] = f.w;
  }
}

__device__ __forceinline__ void ld_x8(const float *p, float *v) {
  const float4 *q = reinterpret_cast<const float4 *>(p);
#pragma unroll
  for (int i = 0; i < 2; i++) {
    float4 f = q[i];
    v[4 * i] = f.x; v[4 * i + 1] = f.y; v[4 * i + 2] = f.z; v[4 * i + 3] = f.w;
  }
}

// Sum over the 64 lanes of a wave, the same tree on every lane and every call.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// Wave-wide reductions through DPP: lanes xor 1 and xor 2 (quad permutes), rotations by 4 and
// 8 within each row of 16 lanes, then lane 0 of each row, combined as (r0 + r1) + (r2 + r3).
// The result is uniform. Every lane of the wave must be active.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ double dpp64(double v) {
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  return __builtin_bit_cast(double, (uint64_t)dpp32<CTRL>((uint32_t)(b >> 32)) << 32 | dpp32<CTRL>((uint32_t)b));
}
__device__ __forceinline__ float lane_f(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
__device__ __forceinline__ double lane_d(double v, int l) {
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, l);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), l);
  return __builtin_bit_cast(double, (uint64_t)hi << 32 | lo);
}
__device__ __forceinline__ float wave_max_f(float v) {
  v = fmaxf(v, __builtin_bit_cast(float, dpp32<0xB1>(__builtin_bit_cast(uint32_t, v))));   // quad_perm 1,0,3,2
  v = fmaxf(v, __builtin_bit_cast(float, dpp32<0x4E>(__builtin_bit_cast(uint32_t, v))));   // quad_perm 2,3,0,1
  v = fmaxf(v, __builtin_bit_cast(float, dpp32<0x124>(__builtin_bit_cast(uint32_t, v))));  // row_ror 4
  v = fmaxf(v, __builtin_bit_cast(float, dpp32<0x128>(__builtin_bit_cast(uint32_t, v))));  // row_ror 8
  return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}
__device__ __forceinline__ double wave_sum_d(double v) {
  v += dpp64<0xB1>(v);
  v += dpp64<0x4E>(v);
  v += dpp64<0x124>(v);
  v += dpp64<0x128>(v);
  return (lane_d(v, 0) + lane_d(v, 16)) + (lane_d(v, 32) + lane_d(v, 48));
}

}  // namespace wl
