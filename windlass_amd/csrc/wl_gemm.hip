// wl_gemm.hip - prefill GEMM over raw GGUF rows on the bf16 matrix cores (T > 8).
//
// Replaces the CPU path's batch branch of Transformer.MatMul (src/Transformer.cs:526-536):
// decode a tile of weight rows, then FastMath.Block (src/FastMath.cs:216-264) multiplies it by
// every token. Here a workgroup owns a BM x BN tile of y (weight rows x tokens) and walks K in
// steps of BK: each thread decodes 32 consecutive weights of one row with the reference's fp32
// arithmetic, rounds them to bf16 into LDS, the token tile (x already rounded to bf16) is staged
// beside it, and four waves (2 x 2) multiply 64 x 64 sub-tiles with v_mfma_f32_16x16x32_bf16.
//
// MFMA operand layout (16x16x32 bf16, checked on the device): lane l holds A[row l%16][k 8*(l/16)
// .. +7] and B[k 8*(l/16) .. +7][col l%16]; the result holds D[row 4*(l/16) + i][col l%16], i < 4.
// With A = weights and B = tokens, a lane's four results are four consecutive rows of one token.
#include "wl_gemm.h"

#include "wl_device.h"
#include "wl_tables.h"

#pragma clang fp contract(off)

namespace wl {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int LDA = BK + 8;  // padded row: 144 bytes, so 8 lanes reading 16 bytes each hit distinct banks

// fp32 -> bf16, round to nearest even (NaN kept quiet).
__device__ __forceinline__ uint32_t bf16_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) { return bf16_bits(lo) | (bf16_bits(hi) << 16); }

// 2 bytes at p (p 2-byte aligned) as uint16.
__device__ __forceinline__ uint32_t rd_u16(const uint8_t *p) {
  return (*align4_down(p) >> (8 * misalign4(p))) & 0xFFFFu;
}

// n (multiple of 4) bytes starting at a 2-byte aligned address, as n/4 dwords.
template <int N>
__device__ __forceinline__ void rd_bytes(const uint8_t *p, uint32_t *out) {
  gu32 *a = align4_down(p);
  const uint32_t sh = misalign4(p) * 8;
  uint32_t w[N / 4 + 1];
#pragma unroll
  for (int i = 0; i <= N / 4; i++) w[i] = a[i];
#pragma unroll
  for (int i = 0; i < N / 4; i++) out[i] = __builtin_amdgcn_alignbit(w[i + 1], w[i], sh);
}

__device__ __forceinline__ uint32_t byte_of(const uint32_t *w, int i) { return (w[i >> 2] >> (8 * (i & 3))) & 0xFFu; }

// Decoders of 32 consecutive values starting at column k (k % 32 == 0) of one row; the same
// fp32 operations in the same order as the reference's DecodeRow, so the values are exact.
struct GQ80 {
  static constexpr int BLOCK = 32, BYTES = 34;
  __device__ static void dq32(const uint8_t *row, int k, float *y) {
    const uint8_t *b = row + (k / 32) * 34;
    const float d = half_bits_exact(rd_u16(b));
    uint32_t q[8];
    rd_bytes<32>(b + 2, q);
#pragma unroll
    for (int j = 0; j < 32; j++) y[j] = (float)(int8_t)byte_of(q, j) * d;  // src/Quants.cs:257
  }
};

struct GQ4K {
  static constexpr int BLOCK = 256, BYTES = 144;
  __device__ static void dq32(const uint8_t *row, int k, float *y) {
    const uint8_t *b = row + (k / 256) * 144;
    const int o = k % 256, j = o / 64, hi = (o % 64) / 32, s = 2 * j + hi;
    const uint4 h = *reinterpret_cast<const uint4 *>(b);  // blocks are 16-byte aligned
    const float d = half_bits_exact(h.x & 0xFFFF), dmin = half_bits_exact(h.x >> 16);
    const uint32_t sc[3] = {h.y, h.z, h.w};
    int scv, mv;  // get_scale_min_k4 (src/Quants.cs:322-330)
    if (s < 4) {
      scv = byte_of(sc, s) & 63;
      mv = byte_of(sc, s + 4) & 63;
    } else {
      scv = (byte_of(sc, s + 4) & 0xF) | ((byte_of(sc, s - 4) >> 6) << 4);
      mv = (byte_of(sc, s + 4) >> 4) | ((byte_of(sc, s) >> 6) << 4);
    }
    const float d1 = d * (float)scv, m1 = dmin * (float)mv;
    const uint4 q0 = *reinterpret_cast<const uint4 *>(b + 16 + 32 * j);
    const uint4 q1 = *reinterpret_cast<const uint4 *>(b + 32 + 32 * j);
    const uint32_t q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
    for (int l = 0; l < 32; l++) {
      const uint32_t v = byte_of(q, l);
      y[l] = d1 * (float)(hi ? v >> 4 : v & 0xF) - m1;  // src/Quants.cs:345-346
    }
  }
};

struct GQ6K {
  static constexpr int BLOCK = 256, BYTES = 210;
  __device__ static void dq32(const uint8_t *row, int k, float *y) {
    const uint8_t *b = row + (k / 256) * 210;
    const int o = k % 256, n = o / 128, qq = (o % 128) / 32;
    const float d = half_bits_exact(rd_u16(b + 208));
    uint32_t ql[8], qh[8], scw[2];
    rd_bytes<32>(b + 64 * n + 32 * (qq & 1), ql);
    rd_bytes<32>(b + 128 + 32 * n, qh);
    rd_bytes<8>(b + 192 + 8 * n, scw);
    const float s0 = (float)(int8_t)byte_of(scw, 2 * qq), s1 = (float)(int8_t)byte_of(scw, 2 * qq + 1);
#pragma unroll
    for (int l = 0; l < 32; l++) {  // src/Quants.cs:381-392
      const uint32_t lo = byte_of(ql, l), hb = byte_of(qh, l);
      const int q = (int)(((qq >> 1) ? lo >> 4 : lo & 0xF) | (((hb >> (2 * qq)) & 3) << 4)) - 32;
      y[l] = d * (l < 16 ? s0 : s1) * (float)q;
    }
  }
};

struct GIQ4XS {
  static constexpr int BLOCK = 256, BYTES = 136;
  __device__ static void dq32(const uint8_t *row, int k, float *y) {
    const uint8_t *b = row + (k / 256) * 136;  // 8-byte aligned
    const int ib = (k % 256) / 32;
    const uint2 hd = *reinterpret_cast<const uint2 *>(b);
    const float d = half_bits_exact(hd.x & 0xFFFF);
    const int scales_h = (int)(hd.x >> 16);
    const int ls = (int)((hd.y >> (8 * (ib / 2) + 4 * (ib % 2))) & 0xF) | (((scales_h >> (2 * ib)) & 3) << 4);
    const float dl = d * (float)(ls - 32);  // src/IQuants.cs:72
    const uint2 qa = *reinterpret_cast<const uint2 *>(b + 8 + 16 * ib);
    const uint2 qb = *reinterpret_cast<const uint2 *>(b + 16 + 16 * ib);
    const uint32_t q[4] = {qa.x, qa.y, qb.x, qb.y};
#pragma unroll
    for (int j = 0; j < 16; j++) {
      const uint32_t v = byte_of(q, j);
      y[j] = dl * (float)kKvaluesIq4nl[v & 0xF];
      y[j + 16] = dl * (float)kKvaluesIq4nl[v >> 4];
    }
  }
};

struct GIQ2XXS {
  static constexpr int BLOCK = 256, BYTES = 66;
  __device__ static void dq32(const uint8_t *row, int k, float *y) {
    const uint8_t *b = row + (k / 256) * 66;
    const int ib = (k % 256) / 32;
    const float d = half_bits_exact(rd_u16(b));
    uint32_t aux[2];
    rd_bytes<8>(b + 2 + 8 * ib, aux);
    const float db = d * (0.5f + (float)(aux[1] >> 28)) * 0.25f;  // src/IQuants.cs:159
#pragma unroll
    for (int l = 0; l < 4; l++) {
      const uint32_t code = kIq2xxsCodes[(aux[0] >> (8 * l)) & 0xFF];
      const uint32_t s7 = (aux[1] >> (7 * l)) & 127;
      const uint32_t signs = s7 | ((uint32_t)(__builtin_popcount(s7) & 1) << 7);
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const float g = (float)iq2_code_byte((code >> (2 * j)) & 3);
        y[8 * l + j] = db * g * (((signs >> j) & 1) ? -1.0f : 1.0f);  // src/IQuants.cs:165
      }
    }
  }
};

// x [T][cols] fp32 -> xb [T][cols] bf16.
__global__ __launch_bounds__(256) void to_bf16_kernel(const float *__restrict__ x, int64_t n4,
                                                      uint2 *__restrict__ xb) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (int64_t)gridDim.x * blockDim.x) {
    const float4 v = reinterpret_cast<const float4 *>(x)[i];
    xb[i] = make_uint2(pack_bf16(v.x, v.y), pack_bf16(v.z, v.w));
  }
}

template <class G>
__global__ __launch_bounds__(256) void gemm_kernel(const uint8_t *__restrict__ w, int64_t row_bytes, int rows,
                                                   int cols, const uint16_t *__restrict__ xb, int T,
                                                   float *__restrict__ y, int ldy) {
  __shared__ __attribute__((aligned(16))) uint16_t As[BM * LDA];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[BN * LDA];
  const int m0 = blockIdx.x * BM, n0 = blockIdx.y * BN;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int wm = wv >> 1, wn = wv & 1;
  // staging: thread -> (row or token) tid/2, 32 values at k0 + 32*(tid&1)
  const int sr = tid >> 1, sh = tid & 1;
  const int wrow = min(m0 + sr, rows - 1);  // rows past the end decode the last row; never stored
  const int xrow = min(n0 + sr, T - 1);
  const uint8_t *wr = w + (int64_t)wrow * row_bytes;
  const uint16_t *xr = xb + (int64_t)xrow * cols;

  f32x4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  for (int k0 = 0; k0 < cols; k0 += BK) {
    const int kk = k0 + 32 * sh;
    float v[32];
    G::dq32(wr, kk, v);
    const uint4 *xs = reinterpret_cast<const uint4 *>(xr + kk);
    const uint4 x0 = xs[0], x1 = xs[1], x2 = xs[2], x3 = xs[3];
    __syncthreads();  // the previous step's reads of As/Bs are done
    uint4 *ad = reinterpret_cast<uint4 *>(As + sr * LDA + 32 * sh);
#pragma unroll
    for (int i = 0; i < 4; i++)
      ad[i] = make_uint4(pack_bf16(v[8 * i], v[8 * i + 1]), pack_bf16(v[8 * i + 2], v[8 * i + 3]),
                         pack_bf16(v[8 * i + 4], v[8 * i + 5]), pack_bf16(v[8 * i + 6], v[8 * i + 7]));
    uint4 *bd = reinterpret_cast<uint4 *>(Bs + sr * LDA + 32 * sh);
    bd[0] = x0;
    bd[1] = x1;
    bd[2] = x2;
    bd[3] = x3;
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < BK; ks += 32) {
      bf16x8_t a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint4 t = *reinterpret_cast<const uint4 *>(As + (64 * wm + 16 * i + (lane & 15)) * LDA + ks + 8 * (lane >> 4));
        a[i] = __builtin_bit_cast(bf16x8_t, t);
      }
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint4 t = *reinterpret_cast<const uint4 *>(Bs + (64 * wn + 16 * j + (lane & 15)) * LDA + ks + 8 * (lane >> 4));
        b[j] = __builtin_bit_cast(bf16x8_t, t);
      }
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
  }

  // lane holds rows r0..r0+3 of token t for each (i, j) sub-tile
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int r0 = m0 + 64 * wm + 16 * i + 4 * (lane >> 4);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int t = n0 + 64 * wn + 16 * j + (lane & 15);
      if (t < T) {
        float *yp = y + (int64_t)t * ldy + r0;
#pragma unroll
        for (int q = 0; q < 4; q++)
          if (r0 + q < rows) yp[q] = acc[i][j][q];
      }
    }
  }
}

template <class G>
static hipError_t launch(const uint8_t *w, int64_t row_bytes, int rows, int cols, const uint16_t *xb, int T,
                         float *y, int ldy, hipStream_t st) {
  const dim3 grid((rows + BM - 1) / BM, (T + BN - 1) / BN);
  hipLaunchKernelGGL((gemm_kernel<G>), grid, dim3(256), 0, st, w, row_bytes, rows, cols, xb, T, y, ldy);
  return hipGetLastError();
}

bool gemm_supports(int type) { return type == 8 || type == 12 || type == 14 || type == 23 || type == 16; }

hipError_t gemm_launch(int type, const uint8_t *w, int64_t row_bytes, int rows, int cols, const float *x, int T,
                       float *y, int ldy, void *scratch, hipStream_t st) {
  if (rows <= 0 || T <= 0) return hipSuccess;
  if (cols <= 0 || cols % 256 || !scratch) return hipErrorInvalidValue;
  const int64_t n4 = (int64_t)T * cols / 4;
  int64_t g = (n4 + 255) / 256;
  if (g > 4096) g = 4096;
  hipLaunchKernelGGL(to_bf16_kernel, dim3((unsigned)g), dim3(256), 0, st, x, n4, reinterpret_cast<uint2 *>(scratch));
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const uint16_t *xb = reinterpret_cast<const uint16_t *>(scratch);
  switch (type) {
    case 8: return launch<GQ80>(w, row_bytes, rows, cols, xb, T, y, ldy, st);
    case 12: return launch<GQ4K>(w, row_bytes, rows, cols, xb, T, y, ldy, st);
    case 14: return launch<GQ6K>(w, row_bytes, rows, cols, xb, T, y, ldy, st);
    case 23: return launch<GIQ4XS>(w, row_bytes, rows, cols, xb, T, y, ldy, st);
    case 16: return launch<GIQ2XXS>(w, row_bytes, rows, cols, xb, T, y, ldy, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace wl
