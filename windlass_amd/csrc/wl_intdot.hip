// wl_intdot.hip - the integer-dot path of Transformer.MatMul (src/Transformer.cs:504-524).
//
// Quantize: one wave per 256 activations (four per lane). Q8_0 takes the block's |x| maximum
// over 8 lanes; Q8_K finds the value of largest magnitude, the first one on ties as the
// reference's strict scan does, by a wave-wide (|x| descending, index ascending) selection.
// The roundings are the reference's: x * id rounded half away from zero (Q8_0), iscale * x
// rounded half to even and clamped at 127 (Q8_K), d = amax / 127 rounded through fp16, d =
// 1 / iscale (correctly rounded divisions).
//
// Dot products: the float GEMV's lane slices and block loads (wl_codecs.h), with v_dot4_i32_i8
// on the quant bytes and the 8-bit activations. A block's integer sums are exact whatever the
// order, so its lanes add their partials with a butterfly; the block's leader lane forms the
// block's float term with the reference's operations and stages it in LDS. A workgroup covers
// whole rows, so after one barrier a lane per (row, token) adds the row's terms in block order,
// which is the reference's `sum +=` loop: y is bit-identical to FastMath.IntDot.
#include "wl_intdot.h"

#include "wl_codecs2.h"
#include "wl_gemv_impl.h"
#include "wl_moe.h"

#pragma clang fp contract(off)

namespace wl {

// FastMath.CanIntDot / NeedsK (src/FastMath.cs:27-32)
bool intdot_supports(int t) { return t == 8 || t == 2 || t == 12 || t == 13 || t == 14; }
bool intdot_needs_k(int t) { return t == 12 || t == 13 || t == 14; }
bool intdot_fits(int t, int cols) { return cols > 0 && cols % (intdot_needs_k(t) ? 256 : 32) == 0; }

static int64_t up16(int64_t n) { return (n + 15) / 16 * 16; }

// The matrix-core operand copy (QActsDev::qf/df) of Q8_K activations of 2..8 tokens.
static bool qacts_mma(int T, int k) { return k && T >= 2 && T <= 8; }
static int64_t mma_bytes(int cols) { return (int64_t)(cols / 256) * (8 * 16 * 32 + 16 * 4); }

int64_t qacts_bytes(int T, int cols, int k) {
  const int bs = k ? 256 : 32;
  return up16((int64_t)T * cols) + up16((int64_t)T * (cols / bs) * 4) + up16(k ? (int64_t)T * (cols / 16) * 2 : 0) +
         (qacts_mma(T, k) ? mma_bytes(cols) : 0);
}

QActsDev qacts_at(void *buf, int T, int cols, int k) {
  const int bs = k ? 256 : 32;
  uint8_t *p = static_cast<uint8_t *>(buf);
  QActsDev a{};
  a.q = reinterpret_cast<int8_t *>(p);
  p += up16((int64_t)T * cols);
  a.d = reinterpret_cast<float *>(p);
  p += up16((int64_t)T * (cols / bs) * 4);
  a.bsums = k ? reinterpret_cast<int16_t *>(p) : nullptr;
  p += up16(k ? (int64_t)T * (cols / 16) * 2 : 0);
  if (qacts_mma(T, k)) {
    const int64_t nb = cols / 256;
    a.qf = reinterpret_cast<int8_t *>(p);
    a.df = reinterpret_cast<float *>(p + nb * 8 * 16 * 32);
  }
  return a;
}

// ------------------------------------------------------------------------------ quantize

__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
  return (uint32_t)(a & 0xFF) | ((uint32_t)(b & 0xFF) << 8) | ((uint32_t)(c & 0xFF) << 16) | ((uint32_t)(d & 0xFF) << 24);
}

// Wave w of the grid quantizes activations [256 c, 256 c + 256) of token t (w = t * nchunk + c).
// With qf (Q8_K of 2..8 tokens), waves of token slots T..15 write that copy's zero slots.
__global__ __launch_bounds__(256) void quantize_kernel(const float *__restrict__ x, int T, int cols, int k,
                                                       int8_t *__restrict__ q, float *__restrict__ d,
                                                       int16_t *__restrict__ bsums, int8_t *__restrict__ qf,
                                                       float *__restrict__ df) {
  const int lane = threadIdx.x & 63;
  const int nchunk = (cols + 255) / 256;
  const int64_t gw = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (gw >= (int64_t)(qf ? 16 : T) * nchunk) return;  // the whole wave
  const int t = (int)(gw / nchunk), c = (int)(gw % nchunk);
  const int base = 256 * c + 4 * lane;  // cols is a multiple of 32, so a lane's 4 values are all in or all out
  if (t >= T) {  // a zero slot of the operand copy
    reinterpret_cast<uint32_t *>(qf)[((c * 8 + lane / 8) * 16 + t) * 8 + lane % 8] = 0u;
    if (lane == 0) df[c * 16 + t] = 0.f;
    return;
  }
  const bool in = base < cols;
  const float *xr = x + (int64_t)t * cols;
  float v[4] = {0.f, 0.f, 0.f, 0.f};
  if (in) {
    const float4 f = *reinterpret_cast<const float4 *>(xr + base);
    v[0] = f.x;
    v[1] = f.y;
    v[2] = f.z;
    v[3] = f.w;
  }
  uint32_t *qw = reinterpret_cast<uint32_t *>(q + (int64_t)t * cols + base);
  if (k == 0) {
    // quantize_row_q8_0 (src/FastMath.cs:54-61): a block of 32 is 8 lanes
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float ax = fabsf(v[i]);
      if (ax > amax) amax = ax;
    }
#pragma unroll
    for (int m = 1; m < 8; m <<= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 64));
    const float dd = amax / 127.f, id = dd != 0.f ? 1.f / dd : 0.f;
    int qi[4];
#pragma unroll
    for (int i = 0; i < 4; i++) qi[i] = (int)roundf(v[i] * id);  // Math.Round(.., AwayFromZero)
    if (in) {
      *qw = pack4(qi[0], qi[1], qi[2], qi[3]);
      if ((lane & 7) == 0) d[(int64_t)t * (cols / 32) + base / 32] = half_bits_exact(to_half(dd));  // Half.Round
    }
    return;
  }
  // quantize_row_q8_K (src/FastMath.cs:62-86): the first value of largest magnitude
  float am = 0.f, mv = 0.f;
  int mi = 0x7FFFFFFF;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const float ax = fabsf(v[i]);
    if (ax > am) {
      am = ax;
      mv = v[i];
      mi = base + i;
    }
  }
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    const float oa = __shfl_xor(am, m, 64), om = __shfl_xor(mv, m, 64);
    const int oi = __shfl_xor(mi, m, 64);
    if (oa > am || (oa == am && oi < mi)) {
      am = oa;
      mv = om;
      mi = oi;
    }
  }
  int qi[4] = {0, 0, 0, 0};
  float iscale = 0.f;
  if (am != 0.f) {
    iscale = -127.f / mv;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int r = (int)rintf(iscale * v[i]);  // Math.Round (to even)
      qi[i] = r > 127 ? 127 : r;
    }
  }
  int s = qi[0] + qi[1] + qi[2] + qi[3];  // bsums: 16 quants = 4 lanes
  s += __shfl_xor(s, 1, 64);
  s += __shfl_xor(s, 2, 64);
  const uint32_t packed = pack4(qi[0], qi[1], qi[2], qi[3]);
  const float dv = am != 0.f ? 1.f / iscale : 0.f;
  *qw = packed;
  if ((lane & 3) == 0) bsums[(int64_t)t * (cols / 16) + base / 16] = (int16_t)s;
  if (lane == 0) d[(int64_t)t * (cols / 256) + c] = dv;
  if (qf) {  // the same values in the matrix-core operand order
    reinterpret_cast<uint32_t *>(qf)[((c * 8 + lane / 8) * 16 + t) * 8 + lane % 8] = packed;
    if (lane == 0) df[c * 16 + t] = dv;
  }
}

hipError_t quantize_launch(const float *x, int T, int cols, int k, QActsDev a, hipStream_t st) {
  if (T <= 0 || cols <= 0) return hipSuccess;
  if (cols % (k ? 256 : 32)) return hipErrorInvalidValue;
  const bool mma = a.qf && qacts_mma(T, k);
  const int64_t waves = (int64_t)(mma ? 16 : T) * ((cols + 255) / 256);
  hipLaunchKernelGGL(quantize_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, st, x, T, cols, k, a.q, a.d,
                     a.bsums, mma ? a.qf : nullptr, a.df);
  return hipGetLastError();
}

// ----------------------------------------------------------------------------- dot codecs
// Per format, on the float codec's lane slice (Lane, Raw, load): Xq is the lane's share of one
// token's activations; part() gives the lane's integer partials of one row's block (si, and
// sm where the format has a min term); the block's lanes add them; term() is the leader's float.

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// Q4_K (src/FastMath.cs:135-157). Lane (j, h): qs bytes 32j + 16h .. +16; low nibbles are
// values 64j + 16h + i of sub-block 2j, high nibbles 64j + 32 + 16h + i of sub-block 2j+1.
struct IQ4K {
  using C = Q4K;
  static constexpr int TERMS = 1;
  struct Xq {
    uint32_t a[4], b[4];
    int B1, B2;  // bsums of the two sub-blocks (lane h = 0 only; 0 on h = 1 so the pair counts them once)
    float d;
  };
  __device__ static void load_x(const int8_t *q, const float *d, const int16_t *bs, int blk, const C::Lane &L,
                                Xq &x) {
    const int8_t *qb = q + (int64_t)blk * 256 + 64 * L.j + 16 * L.h;
    const uint4 a = *reinterpret_cast<const uint4 *>(qb);
    const uint4 b = *reinterpret_cast<const uint4 *>(qb + 32);
    x.a[0] = a.x, x.a[1] = a.y, x.a[2] = a.z, x.a[3] = a.w;
    x.b[0] = b.x, x.b[1] = b.y, x.b[2] = b.z, x.b[3] = b.w;
    const int16_t *s = bs + (int64_t)blk * 16 + 4 * L.j;
    x.B1 = L.h ? 0 : s[0] + s[1];
    x.B2 = L.h ? 0 : s[2] + s[3];
    x.d = d[blk];
  }
  __device__ static void part(const C::Raw &r, const C::Lane &L, const Xq &x, int &si, int &sm) {
    // the 6-bit scales and mins of sub-blocks 2j, 2j+1 (get_scale_min_k4, src/Quants.cs:321-330),
    // decoded as in the float codec
    const uint4 h = r.hdr;
    const uint32_t P = L.jlo ? h.y : h.w;
    const uint32_t Q = L.jlo ? h.z : (h.w >> 4);
    const uint32_t S = ((P & L.m1) | ((h.y >> 2) & L.m2)) >> L.sh;
    const uint32_t M = ((Q & L.m1) | ((h.z >> 2) & L.m2)) >> L.sh;
    const uint32_t qq[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
    int a1 = 0, a2 = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      a1 = dot4(qq[i] & 0x0F0F0F0Fu, x.a[i], a1);
      a2 = dot4((qq[i] >> 4) & 0x0F0F0F0Fu, x.b[i], a2);
    }
    si = (int)(S & 0xFF) * a1 + (int)((S >> 8) & 0xFF) * a2;
    sm = (int)(M & 0xFF) * x.B1 + (int)((M >> 8) & 0xFF) * x.B2;
  }
  __device__ static void reduce(int &si, int &sm) {
#pragma unroll
    for (int m = 1; m < 8; m <<= 1) {
      si += __shfl_xor(si, m, 64);
      sm += __shfl_xor(sm, m, 64);
    }
  }
  __device__ static bool leader(const C::Lane &L) { return L.j == 0 && L.h == 0; }
  __device__ static int term_index(const C::Lane &) { return 0; }
  __device__ static float term(const C::Raw &r, int si, int sm, const Xq &x) {
    const float dd = half_lo(r.hdr.x), dmin = half_hi(r.hdr.x);
    return x.d * (dd * (float)si - dmin * (float)sm);  // src/FastMath.cs:155
  }
};

// Q5_K (src/FastMath.cs:158-184): Q4_K's lanes and terms with the fifth bit of every quant from
// qh (bit 2j of qh[l] for the low nibbles, 2j+1 for the high ones).
struct IQ5K : IQ4K {
  using C = Q5K;
  __device__ static void part(const C::Raw &r, const C::Lane &L, const Xq &x, int &si, int &sm) {
    const uint4 h = r.hdr;
    const uint32_t P = L.jlo ? h.y : h.w;
    const uint32_t Q = L.jlo ? h.z : (h.w >> 4);
    const uint32_t S = ((P & L.m1) | ((h.y >> 2) & L.m2)) >> L.sh;
    const uint32_t M = ((Q & L.m1) | ((h.z >> 2) & L.m2)) >> L.sh;
    const uint32_t qq[4] = {r.q.x, r.q.y, r.q.z, r.q.w}, qh[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
    int a1 = 0, a2 = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t hs = qh[i] >> (2 * L.j);
      a1 = dot4((qq[i] & 0x0F0F0F0Fu) | ((hs & 0x01010101u) << 4), x.a[i], a1);
      a2 = dot4(((qq[i] >> 4) & 0x0F0F0F0Fu) | (((hs >> 1) & 0x01010101u) << 4), x.b[i], a2);
    }
    si = (int)(S & 0xFF) * a1 + (int)((S >> 8) & 0xFF) * a2;
    sm = (int)(M & 0xFF) * x.B1 + (int)((M >> 8) & 0xFF) * x.B2;
  }
  __device__ static float term(const C::Raw &r, int si, int sm, const Xq &x) {
    const float dd = half_lo(r.hdr.x), dmin = half_hi(r.hdr.x);
    return x.d * (dd * (float)si - dmin * (float)sm);  // src/FastMath.cs:182
  }
};

// Q6_K (src/FastMath.cs:185-211). Lane (hh, g): values 128 hh + 8g + 32k + (0..7), k < 4, of
// scale group 2k + g/2 of half hh; that group's other 8 values are on lane g^1.
struct IQ6K {
  using C = Q6K;
  static constexpr int TERMS = 2;  // one per half, in order
  struct Xq {
    uint32_t v[4][2];
    int bsum[4];  // the group sums (lanes with even g only)
    float d;
  };
  __device__ static void load_x(const int8_t *q, const float *d, const int16_t *bs, int blk, const C::Lane &L,
                                Xq &x) {
    const int8_t *qb = q + (int64_t)blk * 256 + 128 * L.hh + 8 * L.g;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const uint2 u = *reinterpret_cast<const uint2 *>(qb + 32 * k);
      x.v[k][0] = u.x;
      x.v[k][1] = u.y;
      x.bsum[k] = (L.g & 1) ? 0 : bs[(int64_t)blk * 16 + 8 * L.hh + L.s + 2 * k];
    }
    x.d = d[blk];
  }
  __device__ static void part(const C::Raw &r, const C::Lane &L, const Xq &x, int &si, int &sm) {
    const uint2 ql1 = C::field(r.l1, r.sh), ql2 = C::field(r.l2, r.sh), qh = C::field(r.h, r.sh),
                sc = C::field(r.sc, r.sh);
    const int s = L.s;
    const int scs[4] = {(int)(int8_t)(sc.x >> (8 * s)), (int)(int8_t)(sc.x >> (8 * s + 16)),
                        (int)(int8_t)(sc.y >> (8 * s)), (int)(int8_t)(sc.y >> (8 * s + 16))};
    const uint32_t L1[2] = {ql1.x, ql1.y}, L2[2] = {ql2.x, ql2.y}, QH[2] = {qh.x, qh.y};
    int p[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 2; i++) {
      // the 6-bit quants q (0..63) of values l, l+32, l+64, l+96 (src/Quants.cs:384-387)
      const uint32_t a = (L1[i] & 0x0F0F0F0Fu) | ((QH[i] << 4) & 0x30303030u);
      const uint32_t b = (L2[i] & 0x0F0F0F0Fu) | ((QH[i] << 2) & 0x30303030u);
      const uint32_t c = ((L1[i] >> 4) & 0x0F0F0F0Fu) | (QH[i] & 0x30303030u);
      const uint32_t e = ((L2[i] >> 4) & 0x0F0F0F0Fu) | ((QH[i] >> 2) & 0x30303030u);
      p[0] = dot4(a, x.v[0][i], p[0]);
      p[1] = dot4(b, x.v[1][i], p[1]);
      p[2] = dot4(c, x.v[2][i], p[2]);
      p[3] = dot4(e, x.v[3][i], p[3]);
    }
    // sum over the group of (q - 32) * x = sum(q * x) - 32 * (sum of the group's x quants)
    int v = 0, w = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      v += scs[k] * p[k];
      w += scs[k] * x.bsum[k];
    }
    si = v - 32 * w;
    sm = 0;
  }
  __device__ static void reduce(int &si, int &) {
    si += __shfl_xor(si, 1, 64);
    si += __shfl_xor(si, 2, 64);
  }
  __device__ static bool leader(const C::Lane &L) { return L.g == 0; }
  __device__ static int term_index(const C::Lane &L) { return L.hh; }
  __device__ static float term(const C::Raw &r, int si, int, const Xq &x) {
    const float dd = half_lo(r.sh ? (r.dw >> 16) : r.dw);
    return x.d * dd * (float)si;  // src/FastMath.cs:209
  }
};

// Q8_0 (src/FastMath.cs:111-122): one lane per 32-value block.
struct IQ80 {
  using C = Q80;
  static constexpr int TERMS = 1;
  struct Xq {
    uint32_t v[8];
    float d;
  };
  __device__ static void load_x(const int8_t *q, const float *d, const int16_t *, int blk, const C::Lane &, Xq &x) {
    const uint4 *p = reinterpret_cast<const uint4 *>(q + (int64_t)blk * 32);
    const uint4 a = p[0], b = p[1];
    x.v[0] = a.x, x.v[1] = a.y, x.v[2] = a.z, x.v[3] = a.w;
    x.v[4] = b.x, x.v[5] = b.y, x.v[6] = b.z, x.v[7] = b.w;
    x.d = d[blk];
  }
  __device__ static void part(const C::Raw &r, const C::Lane &, const Xq &x, int &si, int &sm) {
    int s = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      // quant bytes 4i..4i+3: the window shifted past the 2-byte scale
      const uint32_t lo = __builtin_amdgcn_alignbit(r.win[i + 1], r.win[i], r.sh);
      const uint32_t hi = __builtin_amdgcn_alignbit(r.win[i + 2], r.win[i + 1], r.sh);
      s = dot4(__builtin_amdgcn_alignbit(hi, lo, 16), x.v[i], s);
    }
    si = s;
    sm = 0;
  }
  __device__ static void reduce(int &, int &) {}
  __device__ static bool leader(const C::Lane &) { return true; }
  __device__ static int term_index(const C::Lane &) { return 0; }
  __device__ static float term(const C::Raw &r, int si, int, const Xq &x) {
    const float h = half_lo(__builtin_amdgcn_alignbit(r.win[1], r.win[0], r.sh));
    return h * x.d * (float)si;  // src/FastMath.cs:120
  }
};

// Q4_0 (src/FastMath.cs:123-134): one lane per 32-value block; the reference's s0 + s1 is
// sum((n - 8) * q) = sum(n * q) - 8 * sum(q), the activations' sum formed once per token.
struct IQ40 {
  using C = Q40;
  static constexpr int TERMS = 1;
  struct Xq {
    uint32_t v[8];
    int sq;
    float d;
  };
  __device__ static void load_x(const int8_t *q, const float *d, const int16_t *, int blk, const C::Lane &, Xq &x) {
    const uint4 *p = reinterpret_cast<const uint4 *>(q + (int64_t)blk * 32);
    const uint4 a = p[0], b = p[1];
    x.v[0] = a.x, x.v[1] = a.y, x.v[2] = a.z, x.v[3] = a.w;
    x.v[4] = b.x, x.v[5] = b.y, x.v[6] = b.z, x.v[7] = b.w;
    int s = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) s = dot4(0x01010101u, x.v[i], s);
    x.sq = s;
    x.d = d[blk];
  }
  __device__ static void part(const C::Raw &r, const C::Lane &, const Xq &x, int &si, int &sm) {
    int s = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      // qs dword i: values 4i..4i+3 (low nibbles) and 16+4i.. (high nibbles)
      const uint32_t v = r.at(2, i);
      s = dot4(v & 0x0F0F0F0Fu, x.v[i], s);
      s = dot4((v >> 4) & 0x0F0F0F0Fu, x.v[4 + i], s);
    }
    si = s - 8 * x.sq;
    sm = 0;
  }
  __device__ static void reduce(int &, int &) {}
  __device__ static bool leader(const C::Lane &) { return true; }
  __device__ static int term_index(const C::Lane &) { return 0; }
  __device__ static float term(const C::Raw &r, int si, int, const Xq &x) {
    return half_lo(r.w.dw(0)) * x.d * (float)si;  // src/FastMath.cs:132
  }
};

struct IntArgs {
  const uint8_t *w, *w2;  // w2: the up matrix of the SwiGLU pair (NM = 2)
  int64_t row_bytes;
  int rows, cols;
  const int8_t *q;  // token 0's quants; token t at q + t * cols
  const float *d;   // token t at d + t * (cols / activation block)
  const int16_t *bs;
  int T;
  float *y;
  int ldy;
  int nterm;  // float terms per row
  // routed experts: workgroup row y of the grid runs slot y of the plan, on expert
  // slot_expert of the stacked tensors (estride bytes apart) and the slot's tokens; activation
  // row of its t-th token slot_pair (x_by_pair) or slot_tok, result row slot_pair
  const MoePlan *plan;
  int64_t estride;
  int x_by_pair;
};

constexpr int kIntRows = 4;        // rows per group (of each matrix: 4 / NM)
constexpr int kIntMaxWaves = 8;    // waves per workgroup
constexpr int kIntLds = 65536;     // bytes of terms a workgroup may stage

// The terms of one row added in order, from 0 (the reference's `float sum = 0; sum += ...`);
// p is 16-byte aligned.
__device__ __forceinline__ float sum_in_order(const float *p, int n) {
  float s = 0.f;
  int j = 0;
  for (; j + 4 <= n; j += 4) {
    const float4 v = *reinterpret_cast<const float4 *>(p + j);
    s += v.x;
    s += v.y;
    s += v.z;
    s += v.w;
  }
  for (; j < n; j++) s += p[j];
  return s;
}

// A workgroup of NWV waves covers whole rows: in pass p wave w owns the blocks
// (p * NWV + w) * BPW .. +BPW, lane l block l/LPB of those, slice l%LPB, of every row. For each
// group of R rows the block terms of every (matrix, row, token) go to LDS; after one barrier
// wave 0 adds each row's terms in block order (and applies SiLU to the SwiGLU pair) while the
// other waves go on into the other LDS buffer. SP: one pass, activations kept in registers.
template <class IC, int TM, int NM, bool SP>
__global__ __launch_bounds__(64 * kIntMaxWaves) void intdot_kernel(IntArgs a) {
  extern __shared__ __attribute__((aligned(16))) float wl_int_lds[];
  using C = typename IC::C;
  constexpr int BPW = 64 / C::LPB, R = kIntRows / NM, TT = IC::TERMS;
  constexpr int ab = C::BLOCK;  // activation blocks match the weight blocks (32 for Q8_0, 256 for the K-quants)
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nwv = blockDim.x >> 6;
  const int nb = a.cols / C::BLOCK;
  const int npass = SP ? 1 : (nb + nwv * BPW - 1) / (nwv * BPW);
  const int sub = lane % C::LPB, bslot = lane / C::LPB;
  const typename C::Lane L = C::lane(sub);
  const int ngroups = (a.rows + R - 1) / R;
  const int ld = (a.nterm + 3) & ~3;        // LDS row stride: 16-byte aligned rows
  const int slab = NM * R * TM * ld;          // floats of one LDS buffer
  const uint8_t *wm[2] = {a.w, a.w2};
  int T = a.T, xr[TM], yr[TM];  // tokens; each one's activation and result rows
#pragma unroll
  for (int t = 0; t < TM; t++) xr[t] = yr[t] = t;
  if (a.plan) {
    const int slot = blockIdx.y;
    if (slot >= a.plan->nslots) return;  // the whole workgroup: blockIdx.y is uniform
    T = min(a.plan->slot_ntok[slot], TM);
    const int64_t eo = (int64_t)a.plan->slot_expert[slot] * a.estride;
    wm[0] += eo;
    if (NM == 2) wm[1] += eo;
#pragma unroll
    for (int t = 0; t < TM; t++)
      if (t < T) {
        yr[t] = a.plan->slot_pair[slot][t];
        xr[t] = a.x_by_pair ? yr[t] : a.plan->slot_tok[slot][t];
      }
  }

  auto load_xs = [&](int b, typename IC::Xq(&xs)[TM]) {
#pragma unroll
    for (int t = 0; t < TM; t++)
      if (t < T)
        IC::load_x(a.q + (int64_t)xr[t] * a.cols, a.d + (int64_t)xr[t] * (a.cols / ab),
                   a.bs ? a.bs + (int64_t)xr[t] * (a.cols / 16) : nullptr, b, L, xs[t]);
  };
  typename IC::Xq xs0[TM];
  if (SP && wv * BPW + bslot < nb) load_xs(wv * BPW + bslot, xs0);

  int buf = 0;
  for (int g = blockIdx.x; g < ngroups; g += gridDim.x, buf ^= 1) {
    float *pb = wl_int_lds + buf * slab;
    for (int p = 0; p < npass; p++) {
      const int b = (p * nwv + wv) * BPW + bslot;
      const bool live = b < nb;
      typename IC::Xq xsp[TM];
      if (!SP && live) load_xs(b, xsp);
      const typename IC::Xq(&xs)[TM] = SP ? xs0 : xsp;
      typename C::Raw raw[NM][R];
      if (live) {
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
          for (int r = 0; r < R; r++) {
            // rows past the end re-read the last row (valid memory); their sums are not stored
            const int row = min(g * R + r, a.rows - 1);
            C::load(wm[m] + (int64_t)row * a.row_bytes + (int64_t)b * C::BYTES, L, raw[m][r]);
          }
      }
#pragma unroll
      for (int m = 0; m < NM; m++)
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
          for (int t = 0; t < TM; t++) {
            if (t < T) {
              int si = 0, sm = 0;
              if (live) IC::part(raw[m][r], L, xs[t], si, sm);
              IC::reduce(si, sm);  // every lane takes part (uniform over the wave)
              if (live && IC::leader(L))
                pb[((m * R + r) * TM + t) * ld + b * TT + IC::term_index(L)] = IC::term(raw[m][r], si, sm, xs[t]);
            }
          }
    }
    __syncthreads();
    if (wv == 0) {
      for (int i = lane; i < R * TM; i += 64) {
        const int r = i % R, t = i / R, row = g * R + r;
        if (t < T && row < a.rows) {
          float s = sum_in_order(pb + (r * TM + t) * ld, a.nterm);
          if constexpr (NM == 2) s = silu_mul(s, sum_in_order(pb + ((R + r) * TM + t) * ld, a.nterm));
          a.y[(int64_t)yr[t] * a.ldy + row] = s;
        }
      }
    }
  }
}

static int nterm_of(int type, int cols) {
  return type == 8 || type == 2 ? cols / 32 : type == 14 ? 2 * (cols / 256) : cols / 256;
}

static size_t lds_of(int nm, int tm, int nterm) {
  return sizeof(float) * 2 * kIntRows * tm * ((nterm + 3) & ~3);  // nm matrices of kIntRows / nm rows
}

// slots: grid rows (the plan's slots that may be used; 1 without a plan)
template <class IC, int TM, int NM>
static hipError_t launch_int(const IntArgs &a, int num_cu, hipStream_t st, int slots = 1) {
  using C = typename IC::C;
  const int bpw = 64 / C::LPB, nb = a.cols / C::BLOCK;
  const int units = (nb + bpw - 1) / bpw;
  const int passes = (units + kIntMaxWaves - 1) / kIntMaxWaves;
  const int nwv = (units + passes - 1) / passes;
  const int ngroups = (a.rows + kIntRows / NM - 1) / (kIntRows / NM);
  int nwg = (num_cu * 32 + nwv * slots - 1) / (nwv * slots);  // about 32 waves per CU over all slots
  if (nwg > ngroups) nwg = ngroups;
  if (nwg < 1) nwg = 1;
  const size_t smem = lds_of(NM, TM, a.nterm);
  if (passes == 1)
    hipLaunchKernelGGL((intdot_kernel<IC, TM, NM, true>), dim3(nwg, slots), dim3(64 * nwv), smem, st, a);
  else
    hipLaunchKernelGGL((intdot_kernel<IC, TM, NM, false>), dim3(nwg, slots), dim3(64 * nwv), smem, st, a);
  return hipGetLastError();
}

template <class IC, int NM>
static hipError_t launch_int_tm(const IntArgs &a, int num_cu, hipStream_t st, int slots) {
  if (a.T <= 1) return launch_int<IC, 1, NM>(a, num_cu, st, slots);
  if (a.T <= 2) return launch_int<IC, 2, NM>(a, num_cu, st, slots);
  if (a.T <= 4) return launch_int<IC, 4, NM>(a, num_cu, st, slots);
  return launch_int<IC, 8, NM>(a, num_cu, st, slots);
}

template <int NM>
static hipError_t launch_type(int type, const IntArgs &a, int num_cu, hipStream_t st, int slots = 1) {
  switch (type) {
    case 12: return launch_int_tm<IQ4K, NM>(a, num_cu, st, slots);
    case 13: return launch_int_tm<IQ5K, NM>(a, num_cu, st, slots);
    case 14: return launch_int_tm<IQ6K, NM>(a, num_cu, st, slots);
    case 2: return launch_int_tm<IQ40, NM>(a, num_cu, st, slots);
    default: return launch_int_tm<IQ80, NM>(a, num_cu, st, slots);
  }
}

int intdot_max_tokens(int type, int cols, int nm) {
  const int mm = intmma_max_tokens(type, cols, nm);  // the matrix-core kernel (wl_intmma.hip)
  const int nterm = nterm_of(type, cols);
  for (int tm = 8; tm >= 1; tm /= 2)
    if (lds_of(nm, tm, nterm) <= (size_t)kIntLds) return tm > mm ? tm : mm;
  return mm;
}

static hipError_t run(int type, const uint8_t *w, const uint8_t *w2, int64_t row_bytes, int rows, int cols,
                      QActsDev qa, int T, float *y, int ldy, int num_cu, hipStream_t st) {
  if (rows <= 0 || T <= 0) return hipSuccess;
  const int nm = w2 ? 2 : 1;
  if (!intdot_supports(type) || !intdot_fits(type, cols) || T > intdot_max_tokens(type, cols, nm))
    return hipErrorInvalidValue;
  if (!qa.q || !qa.d || (intdot_needs_k(type) && !qa.bsums)) return hipErrorInvalidValue;
  // two or more tokens of Q4_K / Q6_K: the int8 matrix cores, the same bits
  if (intmma_supports(type, cols, T, nm)) return intmma_launch(type, w, w2, row_bytes, rows, cols, qa, T, y, ldy, st);
  const IntArgs a{w, w2, row_bytes, rows, cols, qa.q, qa.d, qa.bsums, T, y, ldy, nterm_of(type, cols), nullptr, 0, 0};
  return nm == 2 ? launch_type<2>(type, a, num_cu, st) : launch_type<1>(type, a, num_cu, st);
}

hipError_t intdot_launch(int type, const uint8_t *w, int64_t row_bytes, int rows, int cols, QActsDev qa, int T,
                         float *y, int ldy, int num_cu, hipStream_t st) {
  return run(type, w, nullptr, row_bytes, rows, cols, qa, T, y, ldy, num_cu, st);
}

hipError_t intdot_swiglu_launch(int type, const uint8_t *wg, const uint8_t *wu, int64_t row_bytes, int rows,
                                int cols, QActsDev qa, int T, float *y, int ldy, int num_cu, hipStream_t st) {
  return run(type, wg, wu, row_bytes, rows, cols, qa, T, y, ldy, num_cu, st);
}

hipError_t intdot_moe_launch(int type, const uint8_t *w, const uint8_t *w2, int64_t row_bytes, int64_t estride,
                             int rows, int cols, QActsDev qa, const MoePlan *plan, int x_by_pair, int T, int slots,
                             float *y, int ldy, int num_cu, hipStream_t st) {
  if (rows <= 0 || T <= 0 || slots <= 0) return hipSuccess;
  const int nm = w2 ? 2 : 1;
  if (!plan || !intdot_supports(type) || !intdot_fits(type, cols) || T > MOE_MAX_T) return hipErrorInvalidValue;
  const int nterm = nterm_of(type, cols);
  if (lds_of(nm, 8, nterm) > (size_t)kIntLds) return hipErrorInvalidValue;  // up to 8 tokens a slot
  if (!qa.q || !qa.d || (intdot_needs_k(type) && !qa.bsums)) return hipErrorInvalidValue;
  const IntArgs a{w, w2, row_bytes, rows, cols, qa.q, qa.d, qa.bsums, T, y, ldy, nterm, plan, estride, x_by_pair};
  return nm == 2 ? launch_type<2>(type, a, num_cu, st, slots) : launch_type<1>(type, a, num_cu, st, slots);
}

}  // namespace wl
