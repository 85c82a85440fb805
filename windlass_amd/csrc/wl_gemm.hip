// wl_gemm.hip - prefill GEMM over raw GGUF rows on the bf16 matrix cores (T > 8).
//
// Replaces the CPU path's batch branch of Transformer.MatMul (src/Transformer.cs:526-536):
// decode a tile of weight rows, then FastMath.Block (src/FastMath.cs:216-264) multiplies it by
// every token. Here a workgroup owns a 128 x 256 tile of y (weight rows x tokens) and walks K in
// steps of 32: each thread decodes 16 consecutive weights of one row with the reference's fp32
// arithmetic and rounds them to bf16 into LDS, stages one token's 32 values (x rounded to bf16
// once, before the launch) beside them, and four waves (2 x 2) multiply 64 x 128 sub-tiles with
// v_mfma_f32_16x16x32_bf16. LDS is double-buffered and the next step's bytes are loaded into
// registers before the barrier, so one barrier per step separates staging from the products.
//
// MFMA operand layout (16x16x32 bf16, checked on the device): lane l holds A[row l%16][k 8*(l/16)
// .. +7] and B[k 8*(l/16) .. +7][col l%16]; the result holds D[row 4*(l/16) + i][col l%16], i < 4.
// With A = weights and B = tokens, a lane's four results are four consecutive rows of one token.
#include "wl_gemm.h"

#include "wl_blocks.h"
#include "wl_device.h"
#include "wl_codecs.h"
#include "wl_tables.h"

#pragma clang fp contract(off)

namespace wl {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int BM = 128, BN = 256, BK = 32;
// padded LDS rows of 40 bf16 (80 bytes): the 16-byte reads of 8 consecutive rows cover all 32
// banks once
constexpr int LDK = BK + 8;
#ifndef WL_GEMM_DEPTH
#define WL_GEMM_DEPTH 2  // K-steps whose bytes are in flight in registers (1 or 2)
#endif
#ifndef WL_GEMM_WPE
#define WL_GEMM_WPE 2  // waves per SIMD the register budget must allow
#endif

__device__ __forceinline__ uint32_t half_at(uint32_t dword, uint32_t byte_off) { return (dword >> (8 * byte_off)) & 0xFFFFu; }

__device__ __forceinline__ uint32_t pk(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  bf16x2_t v;
  v.x = (__bf16)a;  // round to nearest even (v_cvt_pk_bf16_f32)
  v.y = (__bf16)b;
  return __builtin_bit_cast(uint32_t, v);
}

// Per format: Raw = the bytes 16 consecutive values at column k (k % 16 == 0) of one row need,
// load() fetches them, dec() produces the 16 values as bf16 pairs. The fp32 values are the
// reference DecodeRow's, computed by the same operations in the same order.
struct GQ80 {
  struct Raw { uint32_t dw, dsh; Win<16> q; };
  __device__ static void load(const uint8_t *row, int k, Raw &r) {
    const uint8_t *b = row + (k / 32) * 34;
    r.dw = *align4_down(b);
    r.dsh = misalign4(b);
    r.q.load(b + 2 + 16 * ((k / 16) & 1));
  }
  __device__ static void dec(const Raw &r, int, uint32_t *o) {
    const float d = half_bits_exact(half_at(r.dw, r.dsh));
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t v = r.q.dw(i);
      float y[4];
#pragma unroll
      for (int c = 0; c < 4; c++) y[c] = (float)(int8_t)(v >> (8 * c)) * d;  // src/Quants.cs:257
      o[2 * i] = pk(y[0], y[1]);
      o[2 * i + 1] = pk(y[2], y[3]);
    }
  }
};

struct GQ4K {
  struct Raw { uint4 h, q; };
  __device__ static void load(const uint8_t *row, int k, Raw &r) {
    const uint8_t *b = row + (k / 256) * 144;  // 16-byte aligned
    const int o = k % 256;
    r.h = *reinterpret_cast<const uint4 *>(b);
    r.q = *reinterpret_cast<const uint4 *>(b + 16 + 32 * (o / 64) + 16 * ((o / 16) & 1));
  }
  __device__ static void dec(const Raw &r, int k, uint32_t *o) {
    const int ob = k % 256, j = ob / 64, hi = (ob / 32) & 1, s = 2 * j + hi;
    const float d = half_bits_exact(r.h.x & 0xFFFF), dmin = half_bits_exact(r.h.x >> 16);
    const uint32_t sc[3] = {r.h.y, r.h.z, r.h.w};
    auto B = [&](int i) { return (sc[i >> 2] >> (8 * (i & 3))) & 0xFFu; };
    int scv, mv;  // get_scale_min_k4 (src/Quants.cs:322-330)
    if (s < 4) {
      scv = B(s) & 63;
      mv = B(s + 4) & 63;
    } else {
      scv = (B(s + 4) & 0xF) | ((B(s - 4) >> 6) << 4);
      mv = (B(s + 4) >> 4) | ((B(s) >> 6) << 4);
    }
    const float d1 = d * (float)scv, m1 = dmin * (float)mv;
    const uint32_t q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t v = (q[i] >> (4 * hi)) & 0x0F0F0F0Fu;
      float y[4];
#pragma unroll
      for (int c = 0; c < 4; c++) y[c] = d1 * (float)((v >> (8 * c)) & 0xFF) - m1;  // src/Quants.cs:345-346
      o[2 * i] = pk(y[0], y[1]);
      o[2 * i + 1] = pk(y[2], y[3]);
    }
  }
};

struct GQ6K {
  struct Raw { Win<16> ql, qh; uint32_t sw, ssh, dw, dsh; };
  __device__ static void load(const uint8_t *row, int k, Raw &r) {
    const uint8_t *b = row + (k / 256) * 210;
    const int o = k % 256, n = o / 128, qq = (o % 128) / 32, l0 = o % 32;
    r.ql.load(b + 64 * n + 32 * (qq & 1) + l0);
    r.qh.load(b + 128 + 32 * n + l0);
    const uint8_t *ps = b + 192 + 8 * n + 2 * qq + l0 / 16;
    r.sw = *align4_down(ps);
    r.ssh = misalign4(ps);
    r.dw = *align4_down(b + 208);
    r.dsh = misalign4(b + 208);
  }
  __device__ static void dec(const Raw &r, int k, uint32_t *o) {
    const int qq = (k % 128) / 32;
    const float d = half_bits_exact(half_at(r.dw, r.dsh));
    const float ds = d * (float)(int8_t)(r.sw >> (8 * r.ssh));
#pragma unroll
    for (int i = 0; i < 4; i++) {  // src/Quants.cs:381-392
      const uint32_t v = ((r.ql.dw(i) >> (4 * (qq >> 1))) & 0x0F0F0F0Fu) | (((r.qh.dw(i) >> (2 * qq)) & 0x03030303u) << 4);
      float y[4];
#pragma unroll
      for (int c = 0; c < 4; c++) y[c] = ds * (float)((int)((v >> (8 * c)) & 0xFF) - 32);
      o[2 * i] = pk(y[0], y[1]);
      o[2 * i + 1] = pk(y[2], y[3]);
    }
  }
};

struct GIQ4XS {
  struct Raw { uint2 h, q0, q1; };
  __device__ static void load(const uint8_t *row, int k, Raw &r) {
    const uint8_t *b = row + (k / 256) * 136;  // 8-byte aligned
    const int ib = (k % 256) / 32;
    r.h = *reinterpret_cast<const uint2 *>(b);
    r.q0 = *reinterpret_cast<const uint2 *>(b + 8 + 16 * ib);
    r.q1 = *reinterpret_cast<const uint2 *>(b + 16 + 16 * ib);
  }
  // kvalues_iq4nl + 128 as bytes (the same table as the GEMV codec)
  __device__ static uint32_t lookup(uint32_t idx) {
    const uint32_t i3 = idx & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(IQ4XS::kT1, IQ4XS::kT0, i3);
    const uint32_t hi = __builtin_amdgcn_perm(IQ4XS::kT3, IQ4XS::kT2, i3);
    const uint32_t m = __builtin_amdgcn_perm(0u, 0u, ((idx >> 3) & 0x01010101u) | 0x0C0C0C0Cu);
    return (hi & m) | (lo & ~m);
  }
  __device__ static void dec(const Raw &r, int k, uint32_t *o) {
    const int ib = (k % 256) / 32, h = (k / 16) & 1;
    const float d = half_bits_exact(r.h.x & 0xFFFF);
    const int scales_h = (int)(r.h.x >> 16);
    const int ls = (int)((r.h.y >> (8 * (ib / 2) + 4 * (ib % 2))) & 0xF) | (((scales_h >> (2 * ib)) & 3) << 4);
    const float dl = d * (float)(ls - 32);  // src/IQuants.cs:72
    const uint32_t q[4] = {r.q0.x, r.q0.y, r.q1.x, r.q1.y};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t v = lookup((q[i] >> (4 * h)) & 0x0F0F0F0Fu);
      float y[4];
#pragma unroll
      for (int c = 0; c < 4; c++) y[c] = dl * (float)((int)((v >> (8 * c)) & 0xFF) - 128);
      o[2 * i] = pk(y[0], y[1]);
      o[2 * i + 1] = pk(y[2], y[3]);
    }
  }
};

struct GIQ2XXS {
  struct Raw { Win<8> a; uint32_t dw, dsh; };
  __device__ static void load(const uint8_t *row, int k, Raw &r) {
    const uint8_t *b = row + (k / 256) * 66;
    r.a.load(b + 2 + 8 * ((k % 256) / 32));
    r.dw = *align4_down(b);
    r.dsh = misalign4(b);
  }
  __device__ static void dec(const Raw &r, int k, uint32_t *o) {
    const int h = (k / 16) & 1;
    const float d = half_bits_exact(half_at(r.dw, r.dsh));
    const uint32_t aux0 = r.a.dw(0), aux1 = r.a.dw(1);
    const float db = d * (0.5f + (float)(aux1 >> 28)) * 0.25f;  // src/IQuants.cs:159
#pragma unroll
    for (int e = 0; e < 2; e++) {
      const int l = 2 * h + e;
      const uint32_t code = kIq2xxsCodes[(aux0 >> (8 * l)) & 0xFF];
      const uint32_t s7 = (aux1 >> (7 * l)) & 127;
      const uint32_t signs = s7 | ((uint32_t)(__builtin_popcount(s7) & 1) << 7);
      float y[8];
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const float g = (float)iq2_code_byte((code >> (2 * j)) & 3);
        y[j] = db * g * (((signs >> j) & 1) ? -1.0f : 1.0f);  // src/IQuants.cs:165
      }
#pragma unroll
      for (int j = 0; j < 4; j++) o[4 * e + j] = pk(y[2 * j], y[2 * j + 1]);
    }
  }
};

// x [T][cols] fp32 -> xb [T][cols] bf16.
// The formats of wl_blocks.h: their exact fp32 values rounded to bf16.
template <class B>
struct GBlk {
  struct Raw { typename B::Raw r; };
  __device__ static void load(const uint8_t *row, int k, Raw &r) {
    B::load(row + (k / B::BLOCK) * B::BYTES, k % B::BLOCK, r.r);
  }
  __device__ static void dec(const Raw &r, int k, uint32_t *o) {
    float y[16];
    B::dec(r.r, k % B::BLOCK, y);
#pragma unroll
    for (int i = 0; i < 8; i++) o[i] = pk(y[2 * i], y[2 * i + 1]);
  }
};

__global__ __launch_bounds__(256) void to_bf16_kernel(const float *__restrict__ x, int64_t n4,
                                                      uint2 *__restrict__ xb) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (int64_t)gridDim.x * blockDim.x) {
    const float4 v = reinterpret_cast<const float4 *>(x)[i];
    xb[i] = make_uint2(pk(v.x, v.y), pk(v.z, v.w));
  }
}

// Step k0 of the staging: the thread's weight run (row tid/2, 16 values at k0 + 16*(tid&1)) and
// its token run (token tid, 32 values at k0).
template <class G>
struct Stage {
  typename G::Raw raw;
  uint4 xv[4];
  __device__ void load(const uint8_t *wr, const uint16_t *xr, int k0, int sh) {
    G::load(wr, k0 + 16 * sh, raw);
    const uint4 *xs = reinterpret_cast<const uint4 *>(xr + k0);
#pragma unroll
    for (int i = 0; i < 4; i++) xv[i] = xs[i];
  }
  __device__ void store(uint16_t *as, uint16_t *bs, int k0, int sh) const {
    uint32_t o[8];
    G::dec(raw, k0 + 16 * sh, o);
    uint4 *ad = reinterpret_cast<uint4 *>(as);
    ad[0] = make_uint4(o[0], o[1], o[2], o[3]);
    ad[1] = make_uint4(o[4], o[5], o[6], o[7]);
    uint4 *bd = reinterpret_cast<uint4 *>(bs);
#pragma unroll
    for (int i = 0; i < 4; i++) bd[i] = xv[i];
  }
};

// The products of one staged step: 4 x 8 MFMA sub-tiles of 16 x 16 per wave.
__device__ __forceinline__ void mfma_step(const uint16_t *as, const uint16_t *bs, f32x4_t (&acc)[4][8]) {
  bf16x8_t a[4];
#pragma unroll
  for (int i = 0; i < 4; i++) a[i] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4 *>(as + 16 * i * LDK));
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const bf16x8_t b = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4 *>(bs + 16 * j * LDK));
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b, acc[i][j], 0, 0, 0);
  }
}

// blockIdx.z = K-chunk c of kc columns; with more than one chunk, y points at chunk c's partial
// [T][rows] plane (ldy = rows) in scratch.
template <class G>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WL_GEMM_WPE))) void gemm_kernel(const uint8_t *__restrict__ w, int64_t row_bytes, int rows,
                                                   int cols, int kc, const uint16_t *__restrict__ xb, int T,
                                                   float *__restrict__ y, int64_t ldy, int64_t zstride) {
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * LDK];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN * LDK];
  const int m0 = blockIdx.x * BM, n0 = blockIdx.y * BN;
  const int kb = blockIdx.z * kc, ke = min(cols, kb + kc);
  y += blockIdx.z * zstride;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int wm = wv >> 1, wn = wv & 1;
  const int ar = tid >> 1, sh = tid & 1;
  // rows / tokens past the end stage the last one; their results are never stored
  const uint8_t *wr = w + (int64_t)min(m0 + ar, rows - 1) * row_bytes;
  const uint16_t *xr = xb + (int64_t)min(n0 + tid, T - 1) * cols;
  uint16_t *ast[2] = {As[0] + ar * LDK + 16 * sh, As[1] + ar * LDK + 16 * sh};
  uint16_t *bst[2] = {Bs[0] + tid * LDK, Bs[1] + tid * LDK};
  const int ao = (64 * wm + (lane & 15)) * LDK + 8 * (lane >> 4);
  const int bo = (128 * wn + (lane & 15)) * LDK + 8 * (lane >> 4);

  f32x4_t acc[4][8];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 8; j++) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int n = (ke - kb) / BK;
#if WL_GEMM_DEPTH == 2
  // Two steps in flight: step s's bytes were loaded into registers during step s-2. Step s
  // writes LDS buffer s&1, last read in step s-2, before every thread passed step s-1's barrier.
  Stage<G> st0, st1;
  st0.load(wr, xr, kb, sh);
  if (n > 1) st1.load(wr, xr, kb + BK, sh);
  for (int s = 0; s < n; s += 2) {
    const int k0 = kb + s * BK;
    st0.store(ast[0], bst[0], k0, sh);
    if (s + 2 < n) st0.load(wr, xr, k0 + 2 * BK, sh);
    __syncthreads();
    mfma_step(As[0] + ao, Bs[0] + bo, acc);
    if (s + 1 < n) {
      st1.store(ast[1], bst[1], k0 + BK, sh);
      if (s + 3 < n) st1.load(wr, xr, k0 + 3 * BK, sh);
      __syncthreads();
      mfma_step(As[1] + ao, Bs[1] + bo, acc);
    }
  }
#else
  // One step in flight: step s+1's bytes are loaded into registers while step s multiplies.
  // Step s writes LDS buffer s&1, last read in step s-2, before every thread passed step s-1's
  // barrier.
  Stage<G> st;
  st.load(wr, xr, kb, sh);
  for (int s = 0; s < n; s++) {
    const int buf = s & 1, k0 = kb + s * BK;
    st.store(ast[buf], bst[buf], k0, sh);
    if (s + 1 < n) st.load(wr, xr, k0 + BK, sh);
    __syncthreads();
    mfma_step(As[buf] + ao, Bs[buf] + bo, acc);
  }
#endif

  // lane holds rows r0..r0+3 of token t for each (i, j) sub-tile
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int r0 = m0 + 64 * wm + 16 * i + 4 * (lane >> 4);
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int t = n0 + 128 * wn + 16 * j + (lane & 15);
      if (t < T) {
        float *yp = y + (int64_t)t * ldy + r0;
#pragma unroll
        for (int q = 0; q < 4; q++)
          if (r0 + q < rows) yp[q] = acc[i][j][q];
      }
    }
  }
}


// y[t][r] = chunk partials added in chunk order.
__global__ __launch_bounds__(256) void gemm_combine_kernel(const float *__restrict__ part, int S, int T, int rows,
                                                           float *__restrict__ y, int64_t ldy) {
  const int64_t plane = (int64_t)T * rows;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < plane; i += (int64_t)gridDim.x * blockDim.x) {
    float v[8];
#pragma unroll
    for (int c = 0; c < 8; c++) v[c] = c < S ? part[c * plane + i] : 0.f;
    float s = v[0];
#pragma unroll
    for (int c = 1; c < 8; c++)
      if (c < S) s += v[c];
    const int64_t t = i / rows, r = i % rows;
    y[t * ldy + r] = s;
  }
}

constexpr int kMaxChunks = 8;

static int split_chunks(int tiles, int target, int cols) {
  if (tiles >= target) return 1;
  int S = (target + tiles - 1) / tiles;
  if (S > kMaxChunks) S = kMaxChunks;
  const int nblk = cols / 256;
  if (S > nblk) S = nblk;
  const int per = (nblk + S - 1) / S;
  return (nblk + per - 1) / per;
}

// K-chunks: a launch with fewer output tiles than the device holds at once is split along K
// (in whole 256-blocks): about two workgroups per CU of the 128 x 256 tiles.
int gemm_chunks(int type, int rows, int cols, int T, int num_cu) {
  return split_chunks(((rows + BM - 1) / BM) * ((T + BN - 1) / BN), 2 * num_cu, cols);
}

int64_t gemm_scratch_bytes(int type, int rows, int cols, int T, int num_cu) {
  if (gemm_tall_applies(type, T)) return gemm_tall_scratch_bytes(rows, cols, T, num_cu);
  const int S = gemm_chunks(type, rows, cols, T, num_cu);
  return (int64_t)T * cols * 2 + (S > 1 ? (int64_t)S * T * rows * 4 : 0);
}

template <class G>
static hipError_t launch(const uint8_t *w, int64_t row_bytes, int rows, int cols, const uint16_t *xb, int T,
                         float *y, int ldy, float *part, int S, hipStream_t st) {
  const int kc = (cols / 256 + S - 1) / S * 256;
  const dim3 grid((rows + BM - 1) / BM, (T + BN - 1) / BN, S);
  if (S == 1) {
    hipLaunchKernelGGL((gemm_kernel<G>), grid, dim3(256), 0, st, w, row_bytes, rows, cols, kc, xb, T, y, (int64_t)ldy,
                       (int64_t)0);
    return hipGetLastError();
  }
  hipLaunchKernelGGL((gemm_kernel<G>), grid, dim3(256), 0, st, w, row_bytes, rows, cols, kc, xb, T, part, (int64_t)rows,
                     (int64_t)T * rows);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  int64_t g = ((int64_t)T * rows + 255) / 256;
  if (g > 8192) g = 8192;
  hipLaunchKernelGGL(gemm_combine_kernel, dim3((unsigned)g), dim3(256), 0, st, part, S, T, rows, y, (int64_t)ldy);
  return hipGetLastError();
}

bool gemm_supports(int type) {
  switch (type) {
    case 0: case 1: case 2: case 3: case 6: case 7: case 8: case 10: case 11: case 12: case 13: case 14: case 16:
    case 20: case 21: case 22: case 23: case 30: return true;
  }
  return false;
}

hipError_t gemm_launch(int type, const uint8_t *w, int64_t row_bytes, int rows, int cols, const float *x, int T,
                       float *y, int ldy, void *scratch, int num_cu, hipStream_t st) {
  if (rows <= 0 || T <= 0) return hipSuccess;
  if (cols <= 0 || cols % 256 || !scratch) return hipErrorInvalidValue;
  if (gemm_tall_applies(type, T))
    return gemm_tall_launch(type, w, row_bytes, rows, cols, x, T, y, ldy, scratch, num_cu, st);
  const int64_t n4 = (int64_t)T * cols / 4;
  int64_t g = (n4 + 255) / 256;
  if (g > 4096) g = 4096;
  hipLaunchKernelGGL(to_bf16_kernel, dim3((unsigned)g), dim3(256), 0, st, x, n4, reinterpret_cast<uint2 *>(scratch));
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const uint16_t *xb = reinterpret_cast<const uint16_t *>(scratch);
  // partials follow the bf16 copy of x (T * cols * 2 bytes, a multiple of 512)
  float *part = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(scratch) + (int64_t)T * cols * 2);
  const int S = gemm_chunks(type, rows, cols, T, num_cu);
  switch (type) {
    case 8: return launch<GQ80>(w, row_bytes, rows, cols, xb, T, y, ldy, part, S, st);
    case 12: return launch<GQ4K>(w, row_bytes, rows, cols, xb, T, y, ldy, part, S, st);
    case 14: return launch<GQ6K>(w, row_bytes, rows, cols, xb, T, y, ldy, part, S, st);
    case 23: return launch<GIQ4XS>(w, row_bytes, rows, cols, xb, T, y, ldy, part, S, st);
    case 16: return launch<GIQ2XXS>(w, row_bytes, rows, cols, xb, T, y, ldy, part, S, st);
    case 0: return launch<GBlk<BF32>>(w, row_bytes, rows, cols, xb, T, y, ldy, part, S, st);
    case 1: return launch<GBlk<BF16h>>(w, row_bytes, rows, cols, xb, T, y, ldy, part, S, st);
    case 30: return launch<GBlk<BBF16>>(w, row_bytes, rows, cols, xb, T, y, ldy, part, S, st);
    case 2: return launch<GBlk<BQ40>>(w, row_bytes, rows, cols, xb, T, y, ldy, part, S, st);
    case 3: return launch<GBlk<BQ41>>(w, row_bytes, rows, cols, xb, T, y, ldy, part, S, st);
    case 6: return launch<GBlk<BQ50>>(w, row_bytes, rows, cols, xb, T, y, ldy, part, S, st);
    case 7: return launch<GBlk<BQ51>>(w, row_bytes, rows, cols, xb, T, y, ldy, part, S, st);
    case 10: return launch<GBlk<BQ2K>>(w, row_bytes, rows, cols, xb, T, y, ldy, part, S, st);
    case 11: return launch<GBlk<BQ3K>>(w, row_bytes, rows, cols, xb, T, y, ldy, part, S, st);
    case 13: return launch<GBlk<BQ5K>>(w, row_bytes, rows, cols, xb, T, y, ldy, part, S, st);
    case 20: return launch<GBlk<BIQ4NL>>(w, row_bytes, rows, cols, xb, T, y, ldy, part, S, st);
    case 21: return launch<GBlk<BIQ3S>>(w, row_bytes, rows, cols, xb, T, y, ldy, part, S, st);
    case 22: return launch<GBlk<BIQ2S>>(w, row_bytes, rows, cols, xb, T, y, ldy, part, S, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace wl
