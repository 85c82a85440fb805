// wl_layer.hip - the rest of a decoder layer on device-resident activations: RMSNorm, RoPE,
// the fp16 KV cache, attention, the residual add and greedy sampling (Transformer.Layer /
// Attention / RopeTable / Rope / RmsNormRows, src/Transformer.cs:177-232,351-457; Engine's
// argmax, src/Engine.cs:356-360). With these and the matrix products every activation of a
// decode step stays in HBM; the host sees only the sampled token.
//
// Each kernel follows the reference's operation order where it is sequential there: the
// attention score is the reference's four-way partial dot ((s0+s1)+(s2+s3)), each output value
// of a head adds its positions in order, RoPE's angles come from the same running product in
// double. The double sums the reference runs sequentially (RMSNorm's sum of squares, the
// softmax denominator) are tree sums here, so their last bit can differ.
#include "wl_layer.h"

#include "wl_device.h"

#include <math.h>

#pragma clang fp contract(off)

namespace wl {

// Block-wide sum of doubles (blockDim.x a multiple of 64, at most 1024; all threads get the
// result; sh holds 16 doubles).
__device__ double block_sum_d(double v, double *sh) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  if (lane == 0) sh[wv] = v;
  __syncthreads();
  double s = 0.0;
  for (int i = 0; i < (int)(blockDim.x >> 6); i++) s += sh[i];
  __syncthreads();
  return s;
}

__device__ float block_max_f(float v, float *sh) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  if (lane == 0) sh[wv] = v;
  __syncthreads();
  float s = sh[0];
  for (int i = 1; i < (int)(blockDim.x >> 6); i++) s = fmaxf(s, sh[i]);
  __syncthreads();
  return s;
}

// Block-wide sum of doubles for rms_norm_kernel: each wave's DPP sum (wave_sum_d), then the
// waves' sums in order; one barrier (sh is not reused).
__device__ __forceinline__ double block_sum_dpp(double v, double *sh) {
  v = wave_sum_d(v);
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  double s = 0.0;
  for (int i = 0; i < (int)(blockDim.x >> 6); i++) s += sh[i];
  return s;
}

// RmsNormRows (src/Transformer.cs:446-457): one workgroup per row. Each thread squares and adds
// its values in double (float4 loads when the row allows), then a tree over the workgroup.
// Enough threads that a thread holds a few loads at most: the row's latency is one or two
// memory round trips, not a chain of them.
__global__ __launch_bounds__(1024) void rms_norm_kernel(const float *x, int64_t dim, const float *__restrict__ w,
                                                        float eps, float *y) {  // x == y allowed
  __shared__ double sh[16];
  const float *xr = x + (int64_t)blockIdx.x * dim;
  float *yr = y + (int64_t)blockIdx.x * dim;
  const bool vec = (dim & 3) == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)y & 15) == 0 &&
                   ((uintptr_t)w & 15) == 0;
  double s = 0.0;
  if (vec && dim <= (int64_t)blockDim.x * 8) {
    // at most two float4 per thread: x and w both loaded before the reduction, one round trip
    const int64_t i0 = (int64_t)threadIdx.x * 4, i1 = i0 + (int64_t)blockDim.x * 4;
    float4 xa = make_float4(0.f, 0.f, 0.f, 0.f), xb = xa, wa = xa, wb = xa;
    if (i0 < dim) {
      xa = *reinterpret_cast<const float4 *>(xr + i0);
      wa = *reinterpret_cast<const float4 *>(w + i0);
    }
    if (i1 < dim) {
      xb = *reinterpret_cast<const float4 *>(xr + i1);
      wb = *reinterpret_cast<const float4 *>(w + i1);
    }
    s += (double)xa.x * (double)xa.x;
    s += (double)xa.y * (double)xa.y;
    s += (double)xa.z * (double)xa.z;
    s += (double)xa.w * (double)xa.w;
    s += (double)xb.x * (double)xb.x;
    s += (double)xb.y * (double)xb.y;
    s += (double)xb.z * (double)xb.z;
    s += (double)xb.w * (double)xb.w;
    s = block_sum_dpp(s, sh);
    const float mean = (float)(s / (double)dim);
    const float scale = 1.0f / (float)sqrt((double)(mean + eps));
    if (i0 < dim)
      *reinterpret_cast<float4 *>(yr + i0) =
          make_float4(xa.x * scale * wa.x, xa.y * scale * wa.y, xa.z * scale * wa.z, xa.w * scale * wa.w);
    if (i1 < dim)
      *reinterpret_cast<float4 *>(yr + i1) =
          make_float4(xb.x * scale * wb.x, xb.y * scale * wb.y, xb.z * scale * wb.z, xb.w * scale * wb.w);
    return;
  }
  if (vec) {
    for (int64_t i = (int64_t)threadIdx.x * 4; i < dim; i += (int64_t)blockDim.x * 4) {
      const float4 v = *reinterpret_cast<const float4 *>(xr + i);
      s += (double)v.x * (double)v.x;
      s += (double)v.y * (double)v.y;
      s += (double)v.z * (double)v.z;
      s += (double)v.w * (double)v.w;
    }
  } else {
    for (int64_t i = threadIdx.x; i < dim; i += blockDim.x) s += (double)xr[i] * (double)xr[i];
  }
  s = block_sum_dpp(s, sh);  // every read of x precedes the writes below (in place)
  const float mean = (float)(s / (double)dim);
  const float scale = 1.0f / (float)sqrt((double)(mean + eps));
  if (vec) {
    for (int64_t i = (int64_t)threadIdx.x * 4; i < dim; i += (int64_t)blockDim.x * 4) {
      const float4 v = *reinterpret_cast<const float4 *>(xr + i), g = *reinterpret_cast<const float4 *>(w + i);
      *reinterpret_cast<float4 *>(yr + i) =
          make_float4(v.x * scale * g.x, v.y * scale * g.y, v.z * scale * g.z, v.w * scale * g.w);
    }
  } else {
    for (int64_t i = threadIdx.x; i < dim; i += blockDim.x) yr[i] = xr[i] * scale * w[i];
  }
}

// The angle of rotated pair i at a position: RopeTable's running product in double
// (src/Transformer.cs:396-414) taken to step i, divided by the pair's frequency factor when the
// model has them (rope_freqs.weight, `half` of them). The product is the same sequence for every
// pair, so a wave runs it once for all its lanes (the trip count `half` is uniform) and each lane
// keeps the value after its own i steps: every lane gets the bits the sequential table has
// without a divergent loop of up to 63 dependent multiplies per lane.
__device__ __forceinline__ void rope_cs(int p, int i, int half, double theta_scale, double freq_scale,
                                        const float *__restrict__ freqs, float &c, float &s) {
  double theta = (double)p * freq_scale, mine = theta;
  for (int k = 1; k < half; k++) {
    theta *= theta_scale;
    if (k == i) mine = theta;
  }
  const double a = freqs && i < half ? mine / (double)freqs[i] : mine;
  c = (float)cos(a);
  s = (float)sin(a);
}

// Rope (src/Transformer.cs:416-431) on pair i of one head: (2i, 2i+1), or (i, i + n/2) NeoX.
__device__ __forceinline__ void rope_pair(float *o, int i, int n, int neox, float c, float s, float &y0,
                                          float &y1, int &a, int &b) {
  a = neox ? i : 2 * i;
  b = neox ? i + n / 2 : 2 * i + 1;
  const float x0 = o[a], x1 = o[b];
  y0 = x0 * c - x1 * s;
  y1 = x0 * s + x1 * c;
  o[a] = y0;
  o[b] = y1;
}

// RopeTable (src/Transformer.cs:396-414, computed once per position and reused by every layer):
// (cos, sin, the pair's frequency factor used, 0) of the rotated pairs at positions lo, lo + 1,
// ..., one wave per position, lane i pair i. A reader compares the factor with the model's (its
// values may have changed under the same pointer) and takes the angle again on a mismatch.
__global__ __launch_bounds__(64) void rope_table_kernel(float4 *__restrict__ tab, int lo, int half,
                                                        double theta_scale, double freq_scale,
                                                        const float *__restrict__ freqs) {
  const int p = lo + (int)blockIdx.x, i = threadIdx.x;
  float c, s;
  rope_cs(p, i, half, theta_scale, freq_scale, freqs, c, s);
  if (i < half) tab[(int64_t)p * kRopePairs + i] = make_float4(c, s, freqs ? freqs[i] : 1.f, 0.f);
}

// RoPE on q (H heads) and k (KH heads) of row t, and ToHalf of the row's keys and values into
// cache row pos0 + t, or row pos[t] of slot slot[t] (slots of cap positions) for a batch step
// (src/Transformer.cs:204-215,342-348). Work items of a row: one per rotated pair of every q and
// k head, then one per key/value column (the value's store, and the key's for columns past
// rope_dims). k, v and the caches are null for RoPE on one tensor.
__global__ __launch_bounds__(256) void rope_qkv_kernel(float *__restrict__ q, int64_t ldq, int H, float *__restrict__ k,
                                                       const float *__restrict__ v, int KH, int hd, int n, int neox,
                                                       const int *__restrict__ pos, int pos0, double theta_scale,
                                                       double freq_scale, const float *__restrict__ freqs,
                                                       uint16_t *__restrict__ Kc, uint16_t *__restrict__ Vc,
                                                       const int *__restrict__ slot, int64_t cap) {
  const int t = blockIdx.y, half = n / 2, KD = KH * hd;
  const int it = blockIdx.x * blockDim.x + threadIdx.x;
  const int npairs = (H + KH) * half;
  const int p = pos ? pos[t] : pos0 + t;
  const int64_t crow = (slot ? (int64_t)slot[t] * cap + p : (int64_t)(pos0 + t)) * KD;
  float c = 0.f, s = 0.f;  // every lane runs the angle product (uniform trip count)
  if (half > 0) rope_cs(p, it < npairs ? it % half : 0, half, theta_scale, freq_scale, freqs, c, s);
  if (it < npairs) {
    const int head = it / half, i = it % half;
    float y0, y1;
    int a, b;
    if (head < H) {
      rope_pair(q + (int64_t)t * ldq + (int64_t)head * hd, i, n, neox, c, s, y0, y1, a, b);
    } else {
      const int kh = head - H;
      rope_pair(k + (int64_t)t * KD + (int64_t)kh * hd, i, n, neox, c, s, y0, y1, a, b);
      if (Kc) {
        Kc[crow + kh * hd + a] = to_half(y0);
        Kc[crow + kh * hd + b] = to_half(y1);
      }
    }
  } else if (it < npairs + KD && Vc) {
    const int j = it - npairs;
    Vc[crow + j] = to_half(v[(int64_t)t * KD + j]);
    if (j % hd >= n) Kc[crow + j] = to_half(k[(int64_t)t * KD + j]);
  }
}

// ToHalf (src/Transformer.cs:342-348) of one token's keys and values.
__global__ void kv_store_kernel(const float *__restrict__ k, const float *__restrict__ v, int64_t n,
                                uint16_t *__restrict__ K, uint16_t *__restrict__ V) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  K[i] = to_half(k[i]);
  V[i] = to_half(v[i]);
}

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// Attention (src/Transformer.cs:351-393): one workgroup per (row, head). Scores with the
// reference's four partial sums, the maximum, exp in double, the denominator summed in double,
// then every output value adds its positions in order.
__global__ __launch_bounds__(256) void attention_kernel(const float *__restrict__ q, int64_t ldq,
                                                        const uint16_t *__restrict__ K,
                                                        const uint16_t *__restrict__ V, int kv_dim, int heads,
                                                        int kv_heads, int hd, int pos0, float scale,
                                                        float *__restrict__ scores, int64_t max_n,
                                                        float *__restrict__ out, int64_t ldo,
                                                        const int *__restrict__ pos, const int *__restrict__ slot,
                                                        int64_t cap) {
  __shared__ double shd[4];
  __shared__ float shf[4];
  const int t = blockIdx.y, h = blockIdx.x, kvh = h / (heads / kv_heads);
  const int n = pos ? pos[t] + 1 : pos0 + t + 1;
  if (slot) {  // row t reads its own sequence's slot
    K += (int64_t)slot[t] * cap * kv_dim;
    V += (int64_t)slot[t] * cap * kv_dim;
  }
  const float *qp = q + (int64_t)t * ldq + (int64_t)h * hd;
  float *sp = scores + ((int64_t)t * heads + h) * max_n;
  float mx = -INFINITY;
  for (int j = threadIdx.x; j < n; j += blockDim.x) {
    const uint16_t *kp = K + (int64_t)j * kv_dim + (int64_t)kvh * hd;
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
    int i = 0;
    for (; i + 4 <= hd; i += 4) {
      s0 += qp[i] * h2f(kp[i]);
      s1 += qp[i + 1] * h2f(kp[i + 1]);
      s2 += qp[i + 2] * h2f(kp[i + 2]);
      s3 += qp[i + 3] * h2f(kp[i + 3]);
    }
    for (; i < hd; i++) s0 += qp[i] * h2f(kp[i]);
    const float d = ((s0 + s1) + (s2 + s3)) * scale;
    sp[j] = d;
    mx = fmaxf(mx, d);
  }
  mx = block_max_f(mx, shf);
  double sum = 0.0;
  for (int j = threadIdx.x; j < n; j += blockDim.x) {
    const float e = (float)exp((double)(sp[j] - mx));
    sp[j] = e;
    sum += (double)e;
  }
  sum = block_sum_d(sum, shd);  // also orders the writes of sp before the reads below
  const float inv = (float)(1.0 / sum);
  float *op = out + (int64_t)t * ldo + (int64_t)h * hd;
  for (int d = threadIdx.x; d < hd; d += blockDim.x) {
    float o = 0.f;
    for (int j = 0; j < n; j++) {
      const float p = sp[j] * inv;
      o += p * h2f(V[(int64_t)j * kv_dim + (int64_t)kvh * hd + d]);
    }
    op[d] = o;
  }
}

// One rounding of f16(w.lo) * x: v_fma_mix_f32 with a +0 addend equals the product except that
// an exact -0 product comes out +0. The sums it feeds start at +0 and cannot become -0 (in
// round-to-nearest x + y is -0 only when both are -0), so adding +0 or -0 leaves them as they are.
__device__ __forceinline__ float mul_lo(uint32_t w, float x) { return __builtin_fmaf(half_lo(w), x, 0.0f); }
__device__ __forceinline__ float mul_hi(uint32_t w, float x) { return __builtin_fmaf(half_hi(w), x, 0.0f); }

// Attention for head dims of 64 and 128 (src/Transformer.cs:351-393): one workgroup of 256
// threads per (query head, chunk of kAttP positions, row). Thread j loads the key of position
// j0 + j with uint4 loads (every lane loads, rows past the chunk clamped to its last) and forms
// its score with the reference's four partial sums; the chunk's values are staged in LDS
// meanwhile. When a row's positions fit one chunk the workgroup finishes it with the
// reference's arithmetic (maximum, exp in double, the double sum, p = e * inv, each output value
// adding its positions in order). A longer row leaves per-chunk partials (unnormalised sums,
// chunk maximum, double sum) that attention_combine_kernel rescales and adds in chunk order.
//
// With ROPE the row's own key and value are this step's: rows whose earlier positions are all
// cached (one token of a sequence, or batch rows on distinct slots). Each workgroup rotates its
// query head itself (rope_pair with the position's angles from the table rope_table_kernel
// fills: the bits rope_qkv_kernel gives), the chunk holding the row's position rotates the new
// key and rounds key and value to fp16 (to_half) for that position, and the first query head of
// each KV group stores them to the caches. Nothing in the launch reads those cache rows, so the
// separate RoPE + KV store launch goes away.
constexpr int kAttP = 256;
constexpr int kAttGroup = 16;  // query heads per KV head that attention_group_kernel takes
#ifndef WL_ATT_ROWS
#define WL_ATT_ROWS 16
#endif

struct RopeArgs {
  const float *k = nullptr, *v = nullptr;  // the rows' keys (not rotated) and values [T][kv_dim]
  int n = 0, neox = 0;                     // rotated dims per head, NeoX pairing
  double theta_scale = 0.0, freq_scale = 1.0;
  const float *freqs = nullptr;
  const float4 *tab = nullptr;            // angles by position: [position][kRopePairs] (rope_table_kernel)
  uint16_t *Kc = nullptr, *Vc = nullptr;  // the caches the rows' keys and values go to
};

template <int HD, bool ROPE>
__global__ __launch_bounds__(256, 2) void attention_chunk_kernel(const float *__restrict__ q, int64_t ldq,
                                                              const uint16_t *K, const uint16_t *V, int kv_dim,
                                                              int heads, int kv_heads, int pos0, float scale,
                                                              float *__restrict__ part, int max_chunks,
                                                              float *__restrict__ out, int64_t ldo,
                                                              const int *__restrict__ pos,
                                                              const int *__restrict__ slot, int64_t cap, RopeArgs ra) {
  constexpr int U = HD / 8;  // uint4 per key row
  __shared__ uint4 vs4[kAttP * U];
  __shared__ __attribute__((aligned(16))) float qs[HD];
  __shared__ __attribute__((aligned(16))) float ps[kAttP];
  __shared__ float shf[4];
  __shared__ double shd[4];
  __shared__ double esd[kAttP];
  __shared__ __attribute__((aligned(16))) float kn[ROPE ? HD : 4];
  __shared__ __attribute__((aligned(16))) uint16_t kh[ROPE ? HD : 8], vh[ROPE ? HD : 8];
  const int h = blockIdx.x, c = blockIdx.y, t = blockIdx.z, tid = threadIdx.x;
  const int kvh = h / (heads / kv_heads);
  const int p = pos ? pos[t] : pos0 + t, n = p + 1, j0 = c * kAttP;
  if (j0 >= n) return;  // uniform over the workgroup
  int64_t crow = p;     // the row's cache row
  if (slot) {           // row t reads its own sequence's slot
    K += (int64_t)slot[t] * cap * kv_dim;
    V += (int64_t)slot[t] * cap * kv_dim;
    crow += (int64_t)slot[t] * cap;
  }
  const int cnt = n - j0 < kAttP ? n - j0 : kAttP;
  const int cnt16 = (cnt + 15) & ~15;
  const int nch = (n + kAttP - 1) / kAttP;
  const bool fresh = ROPE && c == nch - 1;  // the chunk holds the row's position, cnt - 1
  const int nold = fresh ? cnt - 1 : cnt;   // positions read from the caches
  float qv = 0.f, kv = 0.f, vv = 0.f;
  float2 cs = make_float2(0.f, 0.f);  // cos and sin of pair tid's angle at the row's position
  if (tid < HD) qv = q[(int64_t)t * ldq + (int64_t)h * HD + tid];
  if (ROPE && tid < ra.n / 2) {
    const float4 a = ra.tab[(int64_t)p * kRopePairs + tid];
    cs = make_float2(a.x, a.y);
    // an entry made with other frequency factors than the model's now: the angle again here
    if (ra.freqs && __float_as_uint(a.z) != __float_as_uint(ra.freqs[tid]))
      rope_cs(p, tid, ra.n / 2, ra.theta_scale, ra.freq_scale, ra.freqs, cs.x, cs.y);
  }
  if (fresh) {
    const int64_t r = (int64_t)t * kv_dim + (int64_t)kvh * HD;
    if (tid < HD)
      kv = ra.k[r + tid];
    else if (tid < 2 * HD)
      vv = ra.v[r + tid - HD];
  }
  // Loads skip what no position needs by uniform branches (a wave's keys, a step of 256/U value
  // rows); within them every lane loads, rows past the chunk clamped to its last cached one.
  uint4 kr[U], vr[U];
  if (__builtin_amdgcn_readfirstlane(tid) - (__builtin_amdgcn_readfirstlane(tid) & 63) < nold) {
    const int row = tid < nold ? tid : nold - 1;
    const uint4 *kp = reinterpret_cast<const uint4 *>(K + (int64_t)(j0 + row) * kv_dim + (int64_t)kvh * HD);
#pragma unroll
    for (int u = 0; u < U; u++) kr[u] = kp[u];
  } else {
#pragma unroll
    for (int u = 0; u < U; u++) kr[u] = make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int u = 0; u < U; u++) {  // the chunk's values: element e of [rows][U] uint4
    const int e = u * 256 + tid, r = e / U, col = e % U, rc = r < nold ? r : nold - 1;
    vr[u] = make_uint4(0, 0, 0, 0);
    if (u * (256 / U) < nold)
      vr[u] = reinterpret_cast<const uint4 *>(V + (int64_t)(j0 + rc) * kv_dim + (int64_t)kvh * HD)[col];
  }
  if (tid < HD) qs[tid] = qv;
  if (fresh) {
    if (tid < HD)
      kn[tid] = kv;
    else if (tid < 2 * HD)
      vh[tid - HD] = to_half(vv);
  }
  if (ROPE) {
    __syncthreads();
    if (tid < ra.n / 2) {
      float y0, y1;
      int a, b;
      rope_pair(qs, tid, ra.n, ra.neox, cs.x, cs.y, y0, y1, a, b);
      if (fresh) {
        rope_pair(kn, tid, ra.n, ra.neox, cs.x, cs.y, y0, y1, a, b);
        kh[a] = to_half(y0);
        kh[b] = to_half(y1);
      }
    } else if (fresh && tid >= ra.n && tid < HD) {  // key columns past the rotated ones
      kh[tid] = to_half(kn[tid]);
    }
  }
  __syncthreads();
  if (fresh) {
    if (h % (heads / kv_heads) == 0 && tid < HD) {
      const int64_t o = crow * kv_dim + (int64_t)kvh * HD + tid;
      ra.Kc[o] = kh[tid];
      ra.Vc[o] = vh[tid];
    }
    if (tid == cnt - 1) {
#pragma unroll
      for (int u = 0; u < U; u++) kr[u] = reinterpret_cast<const uint4 *>(kh)[u];
    }
  }
#pragma unroll
  for (int u = 0; u < U; u++) {  // values first (frees their registers); rows cnt..cnt16-1 as zeros, p = 0 there
    const int e = u * 256 + tid, r = e / U;
    if (r < cnt16) {
      uint4 w = r < nold ? vr[u] : make_uint4(0, 0, 0, 0);
      if (fresh && r == cnt - 1) w = reinterpret_cast<const uint4 *>(vh)[e % U];
      vs4[e] = w;
    }
  }
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
  for (int u = 0; u < U; u++) {
    const uint4 w = kr[u];
    const float4 qa = reinterpret_cast<const float4 *>(qs)[2 * u], qb = reinterpret_cast<const float4 *>(qs)[2 * u + 1];
    s0 += mul_lo(w.x, qa.x);
    s1 += mul_hi(w.x, qa.y);
    s2 += mul_lo(w.y, qa.z);
    s3 += mul_hi(w.y, qa.w);
    s0 += mul_lo(w.z, qb.x);
    s1 += mul_hi(w.z, qb.y);
    s2 += mul_lo(w.w, qb.z);
    s3 += mul_hi(w.w, qb.w);
  }
  const float d = tid < cnt ? ((s0 + s1) + (s2 + s3)) * scale : -INFINITY;
  const int wv = tid >> 6;
  {
    const float m = wave_max_f(d);
    if ((tid & 63) == 0) shf[wv] = m;
  }
  __syncthreads();
  const float mx = fmaxf(fmaxf(shf[0], shf[1]), fmaxf(shf[2], shf[3]));
  float e = 0.f;
  double sum = 0.0;
  if (tid < cnt) {
    e = (float)exp((double)(d - mx));
    sum = (double)e;
  }
  // the denominator as wave_attend forms it (lane l adds positions l, l + 64, l + 128, l + 192 in
  // that order, then the wave's DPP sum), so every attention kernel gives a row the same bits
  esd[tid] = sum;
  __syncthreads();
  if (wv == 0) {
    double s4 = 0.0;
#pragma unroll
    for (int i = 0; i < 4; i++) s4 += esd[tid + 64 * i];
    s4 = wave_sum_d(s4);
    if (tid == 0) shd[0] = s4;
  }
  __syncthreads();
  sum = shd[0];
  ps[tid] = nch == 1 ? e * (float)(1.0 / sum) : e;  // zero past cnt
  __syncthreads();  // also orders the writes of vs4 before the reads below
  float *rec = part + (((int64_t)t * heads + h) * max_chunks + c) * (HD + 4);
  if (tid < HD) {
    // each output value adds its positions in order, 16 at a time: the 16 values and p's are
    // read first, then the products and sums
    const uint16_t *vc = reinterpret_cast<const uint16_t *>(vs4) + tid;
    const float4 *p4 = reinterpret_cast<const float4 *>(ps);
    float o = 0.f;
    for (int j = 0; j < cnt16; j += 16) {
      const float4 pa = p4[j / 4], pb = p4[j / 4 + 1], pc = p4[j / 4 + 2], pd = p4[j / 4 + 3];
      uint32_t w[16];
#pragma unroll
      for (int i = 0; i < 16; i++) w[i] = vc[(j + i) * HD];
      const float pp[16] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w,
                            pc.x, pc.y, pc.z, pc.w, pd.x, pd.y, pd.z, pd.w};
#pragma unroll
      for (int i = 0; i < 16; i++) o += mul_lo(w[i], pp[i]);
    }
    if (nch == 1)
      out[(int64_t)t * ldo + (int64_t)h * HD + tid] = o;
    else
      rec[tid] = o;  // record: HD unnormalised sums, the chunk maximum, a pad, the double sum
  }
  if (nch > 1 && tid == 0) {
    rec[HD] = mx;
    *reinterpret_cast<double *>(rec + HD + 2) = sum;
  }
}

// One row of one query head against a chunk staged in LDS (keys in rows of KS uint4, values in
// rows of HD/8 uint4), by one wave, every lane active: the reference's four partial sums per
// score (positions lane + 64 i), the maximum, exp in double, the denominator in double, p = e *
// inv, each output value adding its positions in order (lane l adds columns 2l and 2l + 1). A
// row of one chunk writes orow; a longer row writes its chunk's record (HD unnormalised sums,
// the chunk maximum, a pad, the double sum) for attention_combine_kernel. qw: the row's query
// (HD floats in LDS); pw: the wave's own kAttP floats of LDS.
template <int HD, int KS>
__device__ __forceinline__ void wave_attend(const uint4 *__restrict__ ks4, const uint4 *__restrict__ vs4,
                                            const float *qw, float *pw, int cnt, int nch, float scale, int lane,
                                            float *__restrict__ orow, float *__restrict__ rec) {
  constexpr int U = HD / 8;
  // scores of positions lane + 64 i
  float d[4];
  {
    float s[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++) s[i][0] = s[i][1] = s[i][2] = s[i][3] = 0.f;
    const float4 *q4 = reinterpret_cast<const float4 *>(qw);
#pragma unroll 4
    for (int u = 0; u < U; u++) {
      const float4 qa = q4[2 * u], qb = q4[2 * u + 1];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        if (64 * i >= cnt) break;  // uniform: no position of this slot is in the row
        const int j = lane + 64 * i < cnt ? lane + 64 * i : cnt - 1;
        const uint4 k = ks4[j * KS + u];
        s[i][0] += mul_lo(k.x, qa.x);
        s[i][1] += mul_hi(k.x, qa.y);
        s[i][2] += mul_lo(k.y, qa.z);
        s[i][3] += mul_hi(k.y, qa.w);
        s[i][0] += mul_lo(k.z, qb.x);
        s[i][1] += mul_hi(k.z, qb.y);
        s[i][2] += mul_lo(k.w, qb.z);
        s[i][3] += mul_hi(k.w, qb.w);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
      d[i] = lane + 64 * i < cnt ? ((s[i][0] + s[i][1]) + (s[i][2] + s[i][3])) * scale : -INFINITY;
  }
  const float mx = wave_max_f(fmaxf(fmaxf(d[0], d[1]), fmaxf(d[2], d[3])));
  float e[4];
  double sum = 0.0;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    e[i] = 0.f;
    if (lane + 64 * i < cnt) {
      e[i] = (float)exp((double)(d[i] - mx));
      sum += (double)e[i];
    }
  }
  sum = wave_sum_d(sum);
  const float inv = (float)(1.0 / sum);
#pragma unroll
  for (int i = 0; i < 4; i++) pw[lane + 64 * i] = nch == 1 ? e[i] * inv : e[i];
  // the wave's own LDS writes before its reads (no other wave reads pw)
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  float o0 = 0.f, o1 = 0.f;
  if (2 * lane < HD) {
    const uint32_t *vc = reinterpret_cast<const uint32_t *>(vs4) + lane;  // columns 2 lane, 2 lane + 1
    const float4 *p4 = reinterpret_cast<const float4 *>(pw);
    int j = 0;
    for (; j + 4 <= cnt; j += 4) {
      const float4 pj = p4[j / 4];
      const uint32_t v0 = vc[(j + 0) * (HD / 2)], v1 = vc[(j + 1) * (HD / 2)], v2 = vc[(j + 2) * (HD / 2)],
                     v3 = vc[(j + 3) * (HD / 2)];
      o0 += mul_lo(v0, pj.x);
      o1 += mul_hi(v0, pj.x);
      o0 += mul_lo(v1, pj.y);
      o1 += mul_hi(v1, pj.y);
      o0 += mul_lo(v2, pj.z);
      o1 += mul_hi(v2, pj.z);
      o0 += mul_lo(v3, pj.w);
      o1 += mul_hi(v3, pj.w);
    }
    for (; j < cnt; j++) {
      const uint32_t v = vc[j * (HD / 2)];
      const float pj = pw[j];
      o0 += mul_lo(v, pj);
      o1 += mul_hi(v, pj);
    }
    if (nch == 1)
      *reinterpret_cast<float2 *>(orow + 2 * lane) = make_float2(o0, o1);
    else  // record: HD unnormalised sums, the chunk maximum, a pad, the double sum
      *reinterpret_cast<float2 *>(rec + 2 * lane) = make_float2(o0, o1);
  }
  if (nch > 1 && lane == 0) {
    rec[HD] = mx;
    *reinterpret_cast<double *>(rec + HD + 2) = sum;
  }
}

// Attention for the rows of a prompt (T consecutive positions pos0.. of one sequence, head dims 64
// and 128): one workgroup of RW waves per (query head, chunk of kAttP positions, RW rows), the
// chunk's keys (rows padded to HD + 8 halves, so sixteen lanes reading sixteen rows hit every
// bank once) and values staged in LDS once for the RW rows, wave w computing row w of the tile
// with wave-wide reductions and no workgroup barrier after the staging. (One workgroup per row
// loaded the chunk once per row: a 4,000-token prompt of the 70B model took 40 ms per layer in
// attention, now 16 rows share a load.) A row's
// arithmetic is attention_chunk_kernel's: the reference's four partial sums per score, maximum,
// exp in double, the denominator in double, p = e * inv, each output value adding its positions
// in order (lane l adds columns 2l and 2l + 1), and the chunk partials of rows longer than a chunk.
template <int HD, int RW>
__global__ __launch_bounds__(64 * RW) void attention_rows_kernel(const float *__restrict__ q, int64_t ldq,
                                                             const uint16_t *__restrict__ K,
                                                             const uint16_t *__restrict__ V, int kv_dim, int heads,
                                                             int kv_heads, int T, int pos0, float scale,
                                                             float *__restrict__ part, int max_chunks,
                                                             float *__restrict__ out, int64_t ldo) {
  constexpr int U = HD / 8, KS = U + 1;  // uint4 per key row; per padded LDS key row
  __shared__ uint4 ks4[kAttP * KS];
  __shared__ uint4 vs4[kAttP * U];
  __shared__ __attribute__((aligned(16))) float qs[RW][HD];
  __shared__ __attribute__((aligned(16))) float ps[RW][kAttP];
  const int h = blockIdx.x, c = blockIdx.y, t0 = blockIdx.z * RW, tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6), t = t0 + w;
  const int kvh = h / (heads / kv_heads), j0 = c * kAttP;
  const int tl = T - 1 < t0 + RW - 1 ? T - 1 : t0 + RW - 1;  // the tile's last row
  const int nmax = pos0 + tl + 1;
  if (j0 >= nmax) return;  // uniform over the workgroup
  const int cmax = nmax - j0 < kAttP ? nmax - j0 : kAttP;  // positions any row of the tile reads
  const uint16_t *Kb = K + (int64_t)j0 * kv_dim + (int64_t)kvh * HD;
  const uint16_t *Vb = V + (int64_t)j0 * kv_dim + (int64_t)kvh * HD;
  for (int e = tid; e < cmax * U; e += 64 * RW) {
    const int r = e / U, col = e % U;
    ks4[r * KS + col] = reinterpret_cast<const uint4 *>(Kb + (int64_t)r * kv_dim)[col];
    vs4[e] = reinterpret_cast<const uint4 *>(Vb + (int64_t)r * kv_dim)[col];
  }
  if (t < T) {
    const float *qp = q + (int64_t)t * ldq + (int64_t)h * HD;
    for (int i = lane; i < HD; i += 64) qs[w][i] = qp[i];
  }
  __syncthreads();
  const int n = pos0 + t + 1;
  if (t >= T || j0 >= n) return;  // uniform over the wave; no barrier follows
  const int cnt = n - j0 < kAttP ? n - j0 : kAttP, nch = (n + kAttP - 1) / kAttP;
  wave_attend<HD, KS>(ks4, vs4, qs[w], ps[w], cnt, nch, scale, lane, out + (int64_t)t * ldo + (int64_t)h * HD,
                      part + (((int64_t)t * heads + h) * max_chunks + c) * (HD + 4));
}

// Attention for decode rows (one token of a sequence, or batch rows on their own slots; head
// dims 64 and 128, at most 16 query heads per KV head): one workgroup of G = heads / kv_heads
// waves per (KV head, chunk of kAttP positions, row). The chunk's keys and values are staged in
// LDS once for the G query heads that read them (one workgroup per query head loaded them G
// times), wave g computing query head kvh * G + g with wave_attend.
// With ROPE the row's own key and value are this step's (every earlier position of the row is
// cached): each wave rotates its query head with the position's angles from the table
// (rope_table_kernel; an entry made with other frequency factors is taken again with rope_cs),
// and in the chunk holding the row's position wave 0 rotates the new key, rounds key and value to
// fp16 (to_half) into the staged chunk and stores them to the caches. Nothing in the launch reads
// those cache rows, so the RoPE + KV store launch goes away; q and k stay as they were.
template <int HD, bool ROPE>
__global__ __launch_bounds__(1024) void attention_group_kernel(const float *__restrict__ q, int64_t ldq,
                                                               const uint16_t *K, const uint16_t *V, int kv_dim,
                                                               int heads, int kv_heads, int pos0, float scale,
                                                               float *__restrict__ part, int max_chunks,
                                                               float *__restrict__ out, int64_t ldo,
                                                               const int *__restrict__ pos,
                                                               const int *__restrict__ slot, int64_t cap, RopeArgs ra) {
  constexpr int U = HD / 8, KS = U + 1;  // uint4 per key row; per padded LDS key row
  __shared__ uint4 ks4[kAttP * KS];
  __shared__ uint4 vs4[kAttP * U];
  __shared__ __attribute__((aligned(16))) float qs[kAttGroup][HD];
  __shared__ __attribute__((aligned(16))) float ps[kAttGroup][kAttP];
  __shared__ __attribute__((aligned(16))) float kn[ROPE ? HD : 4];
  const int kvh = blockIdx.x, c = blockIdx.y, t = blockIdx.z, tid = threadIdx.x, lane = tid & 63;
  const int G = heads / kv_heads, g = __builtin_amdgcn_readfirstlane(tid >> 6), h = kvh * G + g;
  const int p = pos ? pos[t] : pos0 + t, n = p + 1, j0 = c * kAttP;
  if (j0 >= n) return;  // uniform over the workgroup
  int64_t crow = p;     // the row's cache row
  if (slot) {           // row t reads its own sequence's slot
    K += (int64_t)slot[t] * cap * kv_dim;
    V += (int64_t)slot[t] * cap * kv_dim;
    crow += (int64_t)slot[t] * cap;
  }
  const int cnt = n - j0 < kAttP ? n - j0 : kAttP, nch = (n + kAttP - 1) / kAttP;
  const bool fresh = ROPE && c == nch - 1;  // the chunk holds the row's position, cnt - 1
  const int nold = fresh ? cnt - 1 : cnt;   // positions read from the caches
  const uint16_t *Kb = K + (int64_t)j0 * kv_dim + (int64_t)kvh * HD;
  const uint16_t *Vb = V + (int64_t)j0 * kv_dim + (int64_t)kvh * HD;
  for (int e = tid; e < nold * U; e += 64 * G) {
    const int r = e / U, col = e % U;
    ks4[r * KS + col] = reinterpret_cast<const uint4 *>(Kb + (int64_t)r * kv_dim)[col];
    vs4[e] = reinterpret_cast<const uint4 *>(Vb + (int64_t)r * kv_dim)[col];
  }
  const float *qp = q + (int64_t)t * ldq + (int64_t)h * HD;
  for (int i = lane; i < HD; i += 64) qs[g][i] = qp[i];
  if (ROPE) {
    const int64_t r = (int64_t)t * kv_dim + (int64_t)kvh * HD;
    float2 cs = make_float2(0.f, 0.f);
    if (lane < ra.n / 2) {
      const float4 a = ra.tab[(int64_t)p * kRopePairs + lane];
      cs = make_float2(a.x, a.y);
      if (ra.freqs && __float_as_uint(a.z) != __float_as_uint(ra.freqs[lane]))
        rope_cs(p, lane, ra.n / 2, ra.theta_scale, ra.freq_scale, ra.freqs, cs.x, cs.y);
    }
    if (fresh && g == 0)
      for (int i = lane; i < HD; i += 64) kn[i] = ra.k[r + i];
    // the wave's own LDS writes (qs[g], kn) come before its reads below: one wave's LDS
    // operations run in order
    uint16_t *kh = reinterpret_cast<uint16_t *>(ks4 + (cnt - 1) * KS);
    uint16_t *vh = reinterpret_cast<uint16_t *>(vs4 + (cnt - 1) * U);
    if (lane < ra.n / 2) {
      float y0, y1;
      int a, b;
      rope_pair(qs[g], lane, ra.n, ra.neox, cs.x, cs.y, y0, y1, a, b);
      if (fresh && g == 0) {
        rope_pair(kn, lane, ra.n, ra.neox, cs.x, cs.y, y0, y1, a, b);
        kh[a] = to_half(y0);
        kh[b] = to_half(y1);
      }
    }
    if (fresh && g == 0) {
      for (int i = ra.n + lane; i < HD; i += 64) kh[i] = to_half(kn[i]);  // key columns past the rotated ones
      for (int i = lane; i < HD; i += 64) vh[i] = to_half(ra.v[r + i]);
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's kh / vh writes done
      const int64_t o = crow * kv_dim + (int64_t)kvh * HD;
      for (int i = lane; i < HD; i += 64) {
        ra.Kc[o + i] = kh[i];
        ra.Vc[o + i] = vh[i];
      }
    }
  }
  __syncthreads();
  wave_attend<HD, KS>(ks4, vs4, qs[g], ps[g], cnt, nch, scale, lane, out + (int64_t)t * ldo + (int64_t)h * HD,
                      part + (((int64_t)t * heads + h) * max_chunks + c) * (HD + 4));
}

// Rows longer than one chunk: m = the largest chunk maximum, each chunk weighted by
// exp(m_c - m) (double), the weighted sums over the weighted denominators, chunks in order. The
// chunk weights are formed once per row (a thread per chunk, the denominator by one thread in
// chunk order) and shared through LDS: nch * (8 + 4) bytes of dynamic LDS.
template <int HD>
__global__ __launch_bounds__(HD) void attention_combine_kernel(const float *__restrict__ part, int max_chunks,
                                                               int heads, int pos0, float *__restrict__ out,
                                                               int64_t ldo, const int *__restrict__ pos) {
  extern __shared__ __attribute__((aligned(16))) uint8_t cmb[];
  __shared__ float shm[HD / 64];
  __shared__ double shL;
  const int h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
  const int n = pos ? pos[t] + 1 : pos0 + t + 1, nch = (n + kAttP - 1) / kAttP;
  if (nch == 1) return;  // uniform over the workgroup
  double *ex = reinterpret_cast<double *>(cmb);
  float *wg = reinterpret_cast<float *>(cmb + (size_t)max_chunks * sizeof(double));
  const float *rec = part + ((int64_t)t * heads + h) * max_chunks * (HD + 4);
  float m = -INFINITY;
  for (int c = tid; c < nch; c += HD) m = fmaxf(m, rec[c * (HD + 4) + HD]);
  m = wave_max_f(m);
  if ((tid & 63) == 0) shm[tid >> 6] = m;
  __syncthreads();
  m = shm[0];
  for (int i = 1; i < HD / 64; i++) m = fmaxf(m, shm[i]);
  for (int c = tid; c < nch; c += HD) ex[c] = exp((double)(rec[c * (HD + 4) + HD] - m));
  __syncthreads();
  if (tid == 0) {
    double L = 0.0;
    for (int c = 0; c < nch; c++) L += *reinterpret_cast<const double *>(rec + c * (HD + 4) + HD + 2) * ex[c];
    shL = L;
  }
  __syncthreads();
  const double L = shL;
  for (int c = tid; c < nch; c += HD) wg[c] = (float)(ex[c] / L);
  __syncthreads();
  float o = 0.f;
  for (int c = 0; c < nch; c++) o += rec[c * (HD + 4) + tid] * wg[c];
  out[(int64_t)t * ldo + (int64_t)h * HD + tid] = o;
}

// x[i] *= s: the embedding scale (src/Transformer.cs:94,150) and the logit scale's reciprocal
// (:123).
__global__ void scale_kernel(float *__restrict__ x, int64_t n, float s) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) x[i] *= s;
}

// x[i] += o[i] * rs (src/Transformer.cs:224,231).
__global__ void residual_kernel(float *__restrict__ x, const float *__restrict__ o, int64_t n, float rs) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) x[i] += o[i] * rs;
}

// Greedy sampling (src/Engine.cs:356-360): the first index of the largest logit of each row.
// NaNs never win a comparison, so they are skipped, except at index 0: the reference starts
// from index 0 and nothing compares greater than a NaN there, so such a row gives 0.
// Two launches for long rows: workgroup b of a row reduces the contiguous range
// [b*len, (b+1)*len) to (largest value, its first index); the second launch reduces the ranges
// in order. Ties go to the lower index at every step, so the result is the first maximum.
__device__ __forceinline__ void argmax_block(float bv, int bi, float *sv, int *si) {
  sv[threadIdx.x] = bv;
  si[threadIdx.x] = bi;
  __syncthreads();
  for (int s = blockDim.x / 2; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) {
      const float ov = sv[threadIdx.x + s];
      const int oi = si[threadIdx.x + s];
      if (ov > sv[threadIdx.x] || (ov == sv[threadIdx.x] && oi < si[threadIdx.x])) {
        sv[threadIdx.x] = ov;
        si[threadIdx.x] = oi;
      }
    }
    __syncthreads();
  }
}

__global__ __launch_bounds__(256) void argmax_part_kernel(const float *__restrict__ logits, int64_t n, int64_t len,
                                                          float *__restrict__ pv, int *__restrict__ pi) {
  __shared__ float sv[256];
  __shared__ int si[256];
  const int64_t row = blockIdx.y, lo = (int64_t)blockIdx.x * len;
  const int64_t hi = lo + len < n ? lo + len : n;
  const float *l = logits + row * n;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int64_t i = lo + threadIdx.x; i < hi; i += blockDim.x) {
    const float v = l[i];
    if (v > bv) {  // strictly greater: a thread keeps its first maximum
      bv = v;
      bi = (int)i;
    }
  }
  argmax_block(bv, bi, sv, si);
  if (threadIdx.x == 0) {
    pv[row * gridDim.x + blockIdx.x] = sv[0];
    pi[row * gridDim.x + blockIdx.x] = si[0];
  }
}

__global__ __launch_bounds__(256) void argmax_final_kernel(const float *__restrict__ logits, int64_t n, int parts,
                                                           const float *__restrict__ pv, const int *__restrict__ pi,
                                                           int *__restrict__ out) {
  __shared__ float sv[256];
  __shared__ int si[256];
  const int64_t row = blockIdx.x;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int p = threadIdx.x; p < parts; p += blockDim.x) {
    const float v = pv[row * parts + p];
    const int i = pi[row * parts + p];
    if (v > bv || (v == bv && i < bi)) {
      bv = v;
      bi = i;
    }
  }
  argmax_block(bv, bi, sv, si);
  const float l0 = logits[row * n];
  if (threadIdx.x == 0) out[row] = (si[0] == 0x7fffffff || l0 != l0) ? 0 : si[0];
}

// AddBias (src/Transformer.cs:433-443): y[t][i] += b[i].
// MoeFfn's shared expert (src/Transformer.cs:296-309): o[t][d] += f_t * sh[t][d], with
// f_t = 1 / (1 + exp(-gl[t])) (the exponential in double, cast to float) or 1 without a gate.
__global__ void shared_expert_kernel(float *__restrict__ o, const float *__restrict__ sh, const float *__restrict__ gl,
                                     int64_t n, int64_t dim) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float f = gl ? 1.0f / (1.0f + (float)exp((double)(-gl[i / dim]))) : 1.0f;
  o[i] += f * sh[i];
}

__global__ void bias_kernel(float *__restrict__ y, const float *__restrict__ b, int64_t n, int64_t dim) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] += b[i % dim];
}

// SwiGlu's elementwise pass (src/Transformer.cs:247): g = g / (1 + exp(-g)) * u, exp in double.
__global__ void silu_mul_kernel(float *__restrict__ g, const float *__restrict__ u, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    const float a = g[i];
    g[i] = a / (1.0f + (float)exp((double)(-a))) * u[i];
  }
}

static unsigned blocks_of(int64_t n, int b) { return (unsigned)((n + b - 1) / b); }

hipError_t bias_launch(float *y, const float *b, int64_t rows, int64_t dim, hipStream_t st) {
  const int64_t n = rows * dim;
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(bias_kernel, dim3(blocks_of(n, 256)), dim3(256), 0, st, y, b, n, dim);
  return hipGetLastError();
}

hipError_t silu_mul_launch(float *g, const float *u, int64_t n, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(silu_mul_kernel, dim3(blocks_of(n, 256)), dim3(256), 0, st, g, u, n);
  return hipGetLastError();
}

hipError_t rms_norm_launch(const float *x, int64_t rows, int64_t dim, const float *w, float eps, float *y,
                           hipStream_t st) {
  if (rows <= 0) return hipSuccess;
  int nt = (int)((dim / 4 + 63) / 64 * 64);  // a float4 per thread, 64..1024 threads
  nt = nt < 64 ? 64 : nt > 1024 ? 1024 : nt;
  hipLaunchKernelGGL(rms_norm_kernel, dim3((unsigned)rows), dim3(nt), 0, st, x, dim, w, eps, y);
  return hipGetLastError();
}

hipError_t rope_launch(float *x, int64_t ldx, int T, int heads, int hd, int n, int neox, const int *pos, int pos0,
                       double base, double freq_scale, const float *freqs, hipStream_t st) {
  if (T <= 0) return hipSuccess;
  const int64_t items = (int64_t)heads * (n / 2);
  hipLaunchKernelGGL(rope_qkv_kernel, dim3(blocks_of(items, 256), T), dim3(256), 0, st, x, ldx, heads, nullptr,
                     nullptr, 0, hd, n, neox, pos, pos0, pow(base, -2.0 / n), freq_scale, freqs, nullptr, nullptr,
                     nullptr, (int64_t)0);
  return hipGetLastError();
}

hipError_t rope_kv_launch(float *q, float *k, const float *v, int T, int H, int KH, int hd, int n, int neox,
                          int pos0, double base, double freq_scale, const float *freqs, uint16_t *Kc, uint16_t *Vc,
                          const RowMap &rm, hipStream_t st) {
  if (T <= 0) return hipSuccess;
  const int64_t items = (int64_t)(H + KH) * (n / 2) + (int64_t)KH * hd;
  hipLaunchKernelGGL(rope_qkv_kernel, dim3(blocks_of(items, 256), T), dim3(256), 0, st, q, (int64_t)H * hd, H, k, v,
                     KH, hd, n, neox, rm.pos, pos0, pow(base, -2.0 / n), freq_scale, freqs, Kc, Vc, rm.slot, rm.cap);
  return hipGetLastError();
}

hipError_t kv_store_launch(const float *k, const float *v, int64_t n, uint16_t *K, uint16_t *V, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(kv_store_kernel, dim3(blocks_of(n, 256)), dim3(256), 0, st, k, v, n, K, V);
  return hipGetLastError();
}

// The chunked kernel takes head dims of 64 and 128 with 16-byte aligned cache rows; other
// shapes take attention_kernel.
static bool attention_chunked(int hd, int kv_dim, const uint16_t *K, const uint16_t *V) {
  return (hd == 64 || hd == 128) && kv_dim % 8 == 0 && ((uintptr_t)K & 15) == 0 && ((uintptr_t)V & 15) == 0;
}

int64_t attention_scratch_floats(int T, int heads, int hd, int kv_dim, int max_n, const uint16_t *K,
                                 const uint16_t *V) {
  if (T <= 0) return 0;
  if (!attention_chunked(hd, kv_dim, K, V)) return (int64_t)T * heads * max_n;
  const int chunks = (max_n + kAttP - 1) / kAttP;
  return chunks > 1 ? (int64_t)T * heads * chunks * (hd + 4) : 0;
}

template <int HD, bool ROPE>
static hipError_t attention_chunked_launch(const float *q, int64_t ldq, int T, const uint16_t *K, const uint16_t *V,
                                           int kv_dim, int heads, int kv_heads, int pos0, float scale, float *part,
                                           float *out, int64_t ldo, const RowMap &rm, int max_n, const RopeArgs &ra,
                                           hipStream_t st) {
  const int chunks = (max_n + kAttP - 1) / kAttP;
  hipLaunchKernelGGL((attention_chunk_kernel<HD, ROPE>), dim3(heads, chunks, T), dim3(256), 0, st, q, ldq, K, V,
                     kv_dim, heads, kv_heads, pos0, scale, part, chunks, out, ldo, rm.pos, rm.slot, rm.cap, ra);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || chunks == 1) return e;
  hipLaunchKernelGGL(attention_combine_kernel<HD>, dim3(heads, T), dim3(HD), (size_t)chunks * 12, st, part, chunks,
                     heads, pos0, out, ldo, rm.pos);
  return hipGetLastError();
}

// The decode rows' kernel (attention_group_kernel) and, for rows longer than one chunk, the combine.
template <int HD, bool ROPE>
static hipError_t attention_group_launch(const float *q, int64_t ldq, int T, const uint16_t *K, const uint16_t *V,
                                         int kv_dim, int heads, int kv_heads, int pos0, float scale, float *part,
                                         float *out, int64_t ldo, const RowMap &rm, int max_n, const RopeArgs &ra,
                                         hipStream_t st) {
  const int chunks = (max_n + kAttP - 1) / kAttP, G = heads / kv_heads;
  hipLaunchKernelGGL((attention_group_kernel<HD, ROPE>), dim3(kv_heads, chunks, T), dim3(64 * G), 0, st, q, ldq, K, V,
                     kv_dim, heads, kv_heads, pos0, scale, part, chunks, out, ldo, rm.pos, rm.slot, rm.cap, ra);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || chunks == 1) return e;
  hipLaunchKernelGGL(attention_combine_kernel<HD>, dim3(heads, T), dim3(HD), (size_t)chunks * 12, st, part, chunks,
                     heads, pos0, out, ldo, rm.pos);
  return hipGetLastError();
}

// Rows whose earlier positions are all cached and not written by another row of the call: one
// token of a sequence, or batch rows on distinct slots.
static bool own_rows(int T, const RowMap &rm) { return rm.pos ? rm.slot != nullptr : T == 1; }

hipError_t attention_launch(const float *q, int64_t ldq, int T, const uint16_t *K, const uint16_t *V, int kv_dim,
                            int heads, int kv_heads, int hd, int pos0, float scale, float *scratch, float *out,
                            int64_t ldo, const RowMap &rm, int max_n, hipStream_t st) {
  if (T <= 0) return hipSuccess;
  if (T > 1 && !rm.pos && !rm.slot && attention_chunked(hd, kv_dim, K, V)) {  // a prompt's rows
    const int chunks = (max_n + kAttP - 1) / kAttP;
    constexpr int RW = WL_ATT_ROWS;
    const dim3 grid(heads, chunks, (T + RW - 1) / RW);
    if (hd == 64)
      hipLaunchKernelGGL((attention_rows_kernel<64, RW>), grid, dim3(64 * RW), 0, st, q, ldq, K, V, kv_dim, heads,
                         kv_heads, T, pos0, scale, scratch, chunks, out, ldo);
    else
      hipLaunchKernelGGL((attention_rows_kernel<128, RW>), grid, dim3(64 * RW), 0, st, q, ldq, K, V, kv_dim, heads,
                         kv_heads, T, pos0, scale, scratch, chunks, out, ldo);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || chunks == 1) return e;
    if (hd == 64)
      hipLaunchKernelGGL(attention_combine_kernel<64>, dim3(heads, T), dim3(64), (size_t)chunks * 12, st, scratch,
                         chunks, heads, pos0, out, ldo, (const int *)nullptr);
    else
      hipLaunchKernelGGL(attention_combine_kernel<128>, dim3(heads, T), dim3(128), (size_t)chunks * 12, st, scratch,
                         chunks, heads, pos0, out, ldo, (const int *)nullptr);
    return hipGetLastError();
  }
  if (own_rows(T, rm) && max_n > kAttP && heads / kv_heads <= kAttGroup && attention_chunked(hd, kv_dim, K, V)) {
    const RopeArgs none;
    return hd == 64 ? attention_group_launch<64, false>(q, ldq, T, K, V, kv_dim, heads, kv_heads, pos0, scale, scratch,
                                                        out, ldo, rm, max_n, none, st)
                    : attention_group_launch<128, false>(q, ldq, T, K, V, kv_dim, heads, kv_heads, pos0, scale,
                                                         scratch, out, ldo, rm, max_n, none, st);
  }
  if (attention_chunked(hd, kv_dim, K, V)) {
    const RopeArgs none;
    return hd == 64 ? attention_chunked_launch<64, false>(q, ldq, T, K, V, kv_dim, heads, kv_heads, pos0, scale,
                                                          scratch, out, ldo, rm, max_n, none, st)
                    : attention_chunked_launch<128, false>(q, ldq, T, K, V, kv_dim, heads, kv_heads, pos0, scale,
                                                           scratch, out, ldo, rm, max_n, none, st);
  }
  hipLaunchKernelGGL(attention_kernel, dim3(heads, T), dim3(256), 0, st, q, ldq, K, V, kv_dim, heads, kv_heads, hd,
                     pos0, scale, scratch, (int64_t)max_n, out, ldo, rm.pos, rm.slot, rm.cap);
  return hipGetLastError();
}

hipError_t rope_table_launch(float4 *tab, int lo, int count, int n, double base, double freq_scale,
                             const float *freqs, hipStream_t st) {
  if (count <= 0 || n / 2 > kRopePairs) return count <= 0 ? hipSuccess : hipErrorInvalidValue;
  hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)count), dim3(64), 0, st, tab, lo, n / 2, pow(base, -2.0 / n),
                     freq_scale, freqs);
  return hipGetLastError();
}

bool rope_attention_fused(int T, const RowMap &rm, int hd, int kv_heads, int n, const uint16_t *Kc,
                          const uint16_t *Vc) {
  return own_rows(T, rm) && n / 2 <= kRopePairs && attention_chunked(hd, kv_heads * hd, Kc, Vc);
}

hipError_t rope_attention_launch(float *q, float *k, const float *v, int T, int H, int KH, int hd, int n, int neox,
                                 int pos0, double base, double freq_scale, const float *freqs, const float4 *tab,
                                 uint16_t *Kc, uint16_t *Vc, const RowMap &rm, float scale, float *scratch,
                                 float *out, int max_n, hipStream_t st) {
  if (T <= 0) return hipSuccess;
  const int kv_dim = KH * hd;
  if (!rope_attention_fused(T, rm, hd, KH, n, Kc, Vc) || !tab) {
    hipError_t e = rope_kv_launch(q, k, v, T, H, KH, hd, n, neox, pos0, base, freq_scale, freqs, Kc, Vc, rm, st);
    if (e != hipSuccess) return e;
    return attention_launch(q, (int64_t)H * hd, T, Kc, Vc, kv_dim, H, KH, hd, pos0, scale, scratch, out,
                            (int64_t)H * hd, rm, max_n, st);
  }
  RopeArgs ra;
  ra.k = k;
  ra.v = v;
  ra.n = n;
  ra.neox = neox;
  ra.theta_scale = pow(base, -2.0 / n);
  ra.freq_scale = freq_scale;
  ra.freqs = freqs;
  ra.tab = tab;
  ra.Kc = Kc;
  ra.Vc = Vc;
  const int64_t ld = (int64_t)H * hd;
  if (max_n > kAttP && H / KH <= kAttGroup)  // past one chunk: each KV head's chunk loaded once for its heads
    return hd == 64 ? attention_group_launch<64, true>(q, ld, T, Kc, Vc, kv_dim, H, KH, pos0, scale, scratch, out, ld,
                                                       rm, max_n, ra, st)
                    : attention_group_launch<128, true>(q, ld, T, Kc, Vc, kv_dim, H, KH, pos0, scale, scratch, out,
                                                        ld, rm, max_n, ra, st);
  return hd == 64 ? attention_chunked_launch<64, true>(q, ld, T, Kc, Vc, kv_dim, H, KH, pos0, scale, scratch, out, ld,
                                                       rm, max_n, ra, st)
                  : attention_chunked_launch<128, true>(q, ld, T, Kc, Vc, kv_dim, H, KH, pos0, scale, scratch, out,
                                                        ld, rm, max_n, ra, st);
}

hipError_t shared_expert_launch(float *o, const float *sh, const float *gl, int64_t rows, int64_t dim,
                                hipStream_t st) {
  const int64_t n = rows * dim;
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(shared_expert_kernel, dim3(blocks_of(n, 256)), dim3(256), 0, st, o, sh, gl, n, dim);
  return hipGetLastError();
}

hipError_t scale_launch(float *x, int64_t n, float s, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(scale_kernel, dim3(blocks_of(n, 256)), dim3(256), 0, st, x, n, s);
  return hipGetLastError();
}

hipError_t residual_launch(float *x, const float *o, int64_t n, float rs, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(residual_kernel, dim3(blocks_of(n, 256)), dim3(256), 0, st, x, o, n, rs);
  return hipGetLastError();
}

int argmax_parts(int64_t n) {
  int64_t p = (n + 2047) / 2048;  // at least 2048 values per workgroup
  return (int)(p < 1 ? 1 : p > 64 ? 64 : p);
}

hipError_t argmax_launch(const float *logits, int rows, int64_t n, int *out, float *scratch, hipStream_t st) {
  if (rows <= 0) return hipSuccess;
  const int parts = argmax_parts(n);
  const int64_t len = (n + parts - 1) / parts;
  float *pv = scratch;
  int *pi = reinterpret_cast<int *>(scratch + (int64_t)rows * parts);
  hipLaunchKernelGGL(argmax_part_kernel, dim3(parts, rows), dim3(256), 0, st, logits, n, len, pv, pi);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(argmax_final_kernel, dim3(rows), dim3(256), 0, st, logits, n, parts, pv, pi, out);
  return hipGetLastError();
}

}  // namespace wl
