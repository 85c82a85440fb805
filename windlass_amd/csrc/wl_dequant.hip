// wl_dequant.hip - bit-exact dequantization of raw GGUF blocks to fp32.
//
// GPU counterpart of Quants.DecodeRow / IQuants.DecodeRow (src/Quants.cs:32-52,251-396;
// src/IQuants.cs:27-80,147-170). Every value is produced by the same fp32 operations, in the
// same order, as the reference writes them; contraction into FMA is off for this file, and
// the fp16 scales are decoded from their bit fields (subnormals, Inf and NaN payloads exact).
#include "wl_dequant.h"

#include "wl_blocks.h"
#include "wl_device.h"
#include "wl_tables.h"

#pragma clang fp contract(off)

namespace wl {

__device__ __forceinline__ uint32_t rd16(const uint8_t *p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }

// One work item = one chunk of a block; CHUNKS chunks per block.
struct DqQ80 {
  static constexpr int BLOCK = 32, BYTES = 34, CHUNKS = 1;
  __device__ static void run(const uint8_t *b, int, float *y) {
    const float d = half_bits_exact(rd16(b));
    const int8_t *q = reinterpret_cast<const int8_t *>(b + 2);
    for (int j = 0; j < 32; j++) y[j] = (float)q[j] * d;  // src/Quants.cs:257
  }
};

__device__ __forceinline__ void scale_min_k4(int j, const uint8_t *q, int &sc, int &m) {
  if (j < 4) {
    sc = q[j] & 63;
    m = q[j + 4] & 63;
  } else {
    sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
    m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
  }
}

struct DqQ4K {
  static constexpr int BLOCK = 256, BYTES = 144, CHUNKS = 4;  // one chunk = 64 values
  __device__ static void run(const uint8_t *b, int c, float *y) {
    const float d = half_bits_exact(rd16(b)), dmin = half_bits_exact(rd16(b + 2));
    const uint8_t *sc = b + 4, *q = b + 16 + 32 * c;
    int s, m;
    scale_min_k4(2 * c, sc, s, m);
    const float d1 = d * (float)s, m1 = dmin * (float)m;
    scale_min_k4(2 * c + 1, sc, s, m);
    const float d2 = d * (float)s, m2 = dmin * (float)m;
    y += 64 * c;
    for (int l = 0; l < 32; l++) y[l] = d1 * (float)(q[l] & 0xF) - m1;       // src/Quants.cs:345
    for (int l = 0; l < 32; l++) y[32 + l] = d2 * (float)(q[l] >> 4) - m2;   // src/Quants.cs:346
  }
};

struct DqQ6K {
  static constexpr int BLOCK = 256, BYTES = 210, CHUNKS = 8;  // chunk = (half, 8 values of l)
  __device__ static void run(const uint8_t *b, int c, float *y) {
    const int k = c >> 2, l0 = 8 * (c & 3);
    const float d = half_bits_exact(rd16(b + 208));
    const uint8_t *ql = b + 64 * k, *qh = b + 128 + 32 * k;
    const int8_t *sc = reinterpret_cast<const int8_t *>(b + 192 + 8 * k);
    y += 128 * k;
    for (int l = l0; l < l0 + 8; l++) {                                        // src/Quants.cs:381-392
      const int s = l / 16;
      const int q1 = ((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
      const int q2 = ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
      const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
      const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
      y[l] = d * (float)sc[s] * (float)q1;
      y[l + 32] = d * (float)sc[s + 2] * (float)q2;
      y[l + 64] = d * (float)sc[s + 4] * (float)q3;
      y[l + 96] = d * (float)sc[s + 6] * (float)q4;
    }
  }
};

struct DqIQ4XS {
  static constexpr int BLOCK = 256, BYTES = 136, CHUNKS = 8;  // chunk = sub-block of 32
  __device__ static void run(const uint8_t *b, int ib, float *y) {
    const float d = half_bits_exact(rd16(b));
    const int scales_h = (int)rd16(b + 2);
    const uint8_t *scales_l = b + 4, *q = b + 8 + 16 * ib;
    const int ls = ((scales_l[ib / 2] >> (4 * (ib % 2))) & 0xF) | (((scales_h >> (2 * ib)) & 3) << 4);
    const float dl = d * (float)(ls - 32);                                      // src/IQuants.cs:72
    y += 32 * ib;
    for (int j = 0; j < 16; j++) {
      y[j] = dl * (float)kKvaluesIq4nl[q[j] & 0xF];
      y[j + 16] = dl * (float)kKvaluesIq4nl[q[j] >> 4];
    }
  }
};

struct DqIQ2XXS {
  static constexpr int BLOCK = 256, BYTES = 66, CHUNKS = 8;  // chunk = sub-block of 32
  __device__ static void run(const uint8_t *b, int ib, float *y) {
    const float d = half_bits_exact(rd16(b));
    const uint8_t *qs = b + 2 + 8 * ib;
    const uint32_t aux0 = rd16(qs) | (rd16(qs + 2) << 16), aux1 = rd16(qs + 4) | (rd16(qs + 6) << 16);
    const float db = d * (0.5f + (float)(aux1 >> 28)) * 0.25f;                  // src/IQuants.cs:159
    y += 32 * ib;
    for (int l = 0; l < 4; l++) {
      const uint32_t code = kIq2xxsCodes[(aux0 >> (8 * l)) & 0xFF];
      const uint32_t s7 = (aux1 >> (7 * l)) & 127;
      const uint32_t signs = s7 | ((uint32_t)(__builtin_popcount(s7) & 1) << 7);
      for (int j = 0; j < 8; j++) {
        const float g = (float)iq2_code_byte((code >> (2 * j)) & 3);
        y[8 * l + j] = db * g * (((signs >> j) & 1) ? -1.0f : 1.0f);         // src/IQuants.cs:165
      }
    }
  }
};

// F32 / F16 / BF16 rows (src/Quants.cs:36-38), 32 values per work item.
struct DqF32 {
  static constexpr int BLOCK = 32, BYTES = 128, CHUNKS = 1;
  __device__ static void run(const uint8_t *b, int, float *y) {
    const float *s = reinterpret_cast<const float *>(b);
    for (int j = 0; j < 32; j++) y[j] = s[j];
  }
};
struct DqF16 {
  static constexpr int BLOCK = 32, BYTES = 64, CHUNKS = 1;
  __device__ static void run(const uint8_t *b, int, float *y) {
    for (int j = 0; j < 32; j++) y[j] = half_bits_exact(rd16(b + 2 * j));
  }
};
struct DqBF16 {
  static constexpr int BLOCK = 32, BYTES = 64, CHUNKS = 1;
  __device__ static void run(const uint8_t *b, int, float *y) {
    for (int j = 0; j < 32; j++) y[j] = __uint_as_float(rd16(b + 2 * j) << 16);
  }
};

// The formats of wl_blocks.h: one work item = 16 values of a block.
template <class B>
struct DqBlk {
  static constexpr int BLOCK = B::BLOCK, BYTES = B::BYTES, CHUNKS = B::BLOCK / 16;
  __device__ static void run(const uint8_t *b, int c, float *y) {
    typename B::Raw r;
    B::load(b, 16 * c, r);
    float v[16];
    B::dec(r, 16 * c, v);
#pragma unroll
    for (int j = 0; j < 16; j++) y[16 * c + j] = v[j];
  }
};

// Rows row0.. of the tensor, or (ids non-null) rows ids[0..nrows): an id outside
// [0, tensor_rows) gives a row of zeros, never a read outside the tensor.
template <class D>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t *__restrict__ w, int64_t row_bytes,
                                                      int64_t row0, int64_t nrows, int64_t cols,
                                                      float *__restrict__ dst, const int32_t *__restrict__ ids,
                                                      int64_t tensor_rows) {
  const int64_t nb = cols / D::BLOCK;
  const int64_t per_row = nb * D::CHUNKS;
  const int64_t total = nrows * per_row;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / per_row, rem = i % per_row;
    const int64_t b = rem / D::CHUNKS;
    const int c = (int)(rem % D::CHUNKS);
    const int64_t row = ids ? (int64_t)ids[r] : row0 + r;
    float *y = dst + r * cols + b * D::BLOCK;
    if (ids && (row < 0 || row >= tensor_rows)) {
      for (int j = c * (D::BLOCK / D::CHUNKS); j < (c + 1) * (D::BLOCK / D::CHUNKS); j++) y[j] = 0.f;
      continue;
    }
    D::run(w + row * row_bytes + b * D::BYTES, c, y);
  }
}

template <class D>
static hipError_t launch(const uint8_t *w, int64_t row_bytes, int64_t row0, int64_t nrows, int64_t cols,
                         float *dst, const int32_t *ids, int64_t tensor_rows, hipStream_t st) {
  const int64_t total = nrows * (cols / D::BLOCK) * D::CHUNKS;
  if (total == 0) return hipSuccess;
  int64_t grid = (total + 255) / 256;
  if (grid > 65536) grid = 65536;
  hipLaunchKernelGGL((dequant_kernel<D>), dim3((unsigned)grid), dim3(256), 0, st, w, row_bytes, row0, nrows, cols, dst,
                     ids, tensor_rows);
  return hipGetLastError();
}

bool dequant_supports(int type) {
  switch (type) {
    case 0: case 1: case 30: case 8: case 12: case 14: case 23: case 16:
    case 2: case 3: case 6: case 7: case 10: case 11: case 13: case 20: case 21: case 22: return true;
  }
  return false;
}

static hipError_t dequant_any(int type, const uint8_t *w, int64_t row_bytes, int64_t row0, int64_t nrows,
                              int64_t cols, float *dst, const int32_t *ids, int64_t tensor_rows, hipStream_t st) {
  switch (type) {
    case 0: return launch<DqF32>(w, row_bytes, row0, nrows, cols, dst, ids, tensor_rows, st);
    case 1: return launch<DqF16>(w, row_bytes, row0, nrows, cols, dst, ids, tensor_rows, st);
    case 30: return launch<DqBF16>(w, row_bytes, row0, nrows, cols, dst, ids, tensor_rows, st);
    case 8: return launch<DqQ80>(w, row_bytes, row0, nrows, cols, dst, ids, tensor_rows, st);
    case 12: return launch<DqQ4K>(w, row_bytes, row0, nrows, cols, dst, ids, tensor_rows, st);
    case 14: return launch<DqQ6K>(w, row_bytes, row0, nrows, cols, dst, ids, tensor_rows, st);
    case 23: return launch<DqIQ4XS>(w, row_bytes, row0, nrows, cols, dst, ids, tensor_rows, st);
    case 16: return launch<DqIQ2XXS>(w, row_bytes, row0, nrows, cols, dst, ids, tensor_rows, st);
    case 2: return launch<DqBlk<BQ40>>(w, row_bytes, row0, nrows, cols, dst, ids, tensor_rows, st);
    case 3: return launch<DqBlk<BQ41>>(w, row_bytes, row0, nrows, cols, dst, ids, tensor_rows, st);
    case 6: return launch<DqBlk<BQ50>>(w, row_bytes, row0, nrows, cols, dst, ids, tensor_rows, st);
    case 7: return launch<DqBlk<BQ51>>(w, row_bytes, row0, nrows, cols, dst, ids, tensor_rows, st);
    case 10: return launch<DqBlk<BQ2K>>(w, row_bytes, row0, nrows, cols, dst, ids, tensor_rows, st);
    case 11: return launch<DqBlk<BQ3K>>(w, row_bytes, row0, nrows, cols, dst, ids, tensor_rows, st);
    case 13: return launch<DqBlk<BQ5K>>(w, row_bytes, row0, nrows, cols, dst, ids, tensor_rows, st);
    case 20: return launch<DqBlk<BIQ4NL>>(w, row_bytes, row0, nrows, cols, dst, ids, tensor_rows, st);
    case 21: return launch<DqBlk<BIQ3S>>(w, row_bytes, row0, nrows, cols, dst, ids, tensor_rows, st);
    case 22: return launch<DqBlk<BIQ2S>>(w, row_bytes, row0, nrows, cols, dst, ids, tensor_rows, st);
  }
  return hipErrorInvalidValue;
}

hipError_t dequant_launch(int type, const uint8_t *w, int64_t row_bytes, int64_t row0, int64_t nrows,
                          int64_t cols, float *dst, hipStream_t st) {
  return dequant_any(type, w, row_bytes, row0, nrows, cols, dst, nullptr, 0, st);
}

hipError_t dequant_rows_launch(int type, const uint8_t *w, int64_t row_bytes, const int32_t *ids, int64_t nrows,
                               int64_t tensor_rows, int64_t cols, float *dst, hipStream_t st) {
  return dequant_any(type, w, row_bytes, 0, nrows, cols, dst, ids, tensor_rows, st);
}

}  // namespace wl
