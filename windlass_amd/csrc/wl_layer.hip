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

// Block-wide sum of doubles over 256 threads (all threads get the result).
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

// RmsNormRows (src/Transformer.cs:446-457): one workgroup per row.
__global__ __launch_bounds__(256) void rms_norm_kernel(const float *x, int64_t dim, const float *__restrict__ w,
                                                       float eps, float *y) {  // x == y allowed
  __shared__ double sh[4];
  const float *xr = x + (int64_t)blockIdx.x * dim;
  float *yr = y + (int64_t)blockIdx.x * dim;
  double s = 0.0;
  for (int64_t i = threadIdx.x; i < dim; i += blockDim.x) s += (double)xr[i] * (double)xr[i];
  s = block_sum_d(s, sh);
  const float mean = (float)(s / (double)dim);
  const float scale = 1.0f / (float)sqrt((double)(mean + eps));
  for (int64_t i = threadIdx.x; i < dim; i += blockDim.x) yr[i] = xr[i] * scale * w[i];
}

// RopeTable (src/Transformer.cs:396-414): cos/sin per rotated pair at each row's position,
// the angle a running product in double as there, divided by the pair's frequency factor when
// the model has them (rope_freqs.weight). One thread per row.
__global__ void rope_table_kernel(const int *__restrict__ pos, int pos0, int T, int n, double theta_scale,
                                  double freq_scale, const float *__restrict__ freqs, float *__restrict__ cs) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= T) return;
  double theta = (double)(pos ? pos[t] : pos0 + t) * freq_scale;
  float *c = cs + (int64_t)t * n;
  for (int i = 0; i < n / 2; i++) {
    const double a = freqs ? theta / (double)freqs[i] : theta;
    c[2 * i] = (float)cos(a);
    c[2 * i + 1] = (float)sin(a);
    theta *= theta_scale;
  }
}

// Rope (src/Transformer.cs:416-431) on row t's `heads` heads: pairs (2i, 2i+1), or (i, i+half)
// for the NeoX layout.
__global__ void rope_kernel(float *__restrict__ x, int64_t ldx, int heads, int hd, int n, int neox,
                            const float *__restrict__ cs) {
  const int t = blockIdx.y;
  const int half = n / 2;
  const int k = blockIdx.x * blockDim.x + threadIdx.x;  // (head, pair)
  if (k >= heads * half) return;
  const int h = k / half, i = k % half;
  float *o = x + (int64_t)t * ldx + (int64_t)h * hd;
  const float c = cs[(int64_t)t * n + 2 * i], s = cs[(int64_t)t * n + 2 * i + 1];
  const int a = neox ? i : 2 * i, b = neox ? i + half : 2 * i + 1;
  const float x0 = o[a], x1 = o[b];
  o[a] = x0 * c - x1 * s;
  o[b] = x0 * s + x1 * c;
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
                                                        float *__restrict__ out, int64_t ldo) {
  __shared__ double shd[4];
  __shared__ float shf[4];
  const int t = blockIdx.y, h = blockIdx.x, kvh = h / (heads / kv_heads);
  const int n = pos0 + t + 1;
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

// x[i] += o[i] * rs (src/Transformer.cs:224,231).
__global__ void residual_kernel(float *__restrict__ x, const float *__restrict__ o, int64_t n, float rs) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) x[i] += o[i] * rs;
}

// Greedy sampling (src/Engine.cs:356-360): the first index of the largest logit of each row.
// NaNs never win a comparison, so they are skipped, except at index 0: the reference starts
// from index 0 and nothing compares greater than a NaN there, so such a row gives 0.
__global__ __launch_bounds__(256) void argmax_kernel(const float *__restrict__ logits, int64_t n,
                                                     int *__restrict__ out) {
  __shared__ float sv[256];
  __shared__ int si[256];
  const float *l = logits + (int64_t)blockIdx.x * n;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
    const float v = l[i];
    if (v > bv) {  // strictly greater: a thread keeps its first maximum
      bv = v;
      bi = (int)i;
    }
  }
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
  if (threadIdx.x == 0) out[blockIdx.x] = (si[0] == 0x7fffffff || l[0] != l[0]) ? 0 : si[0];
}

// AddBias (src/Transformer.cs:433-443): y[t][i] += b[i].
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
  hipLaunchKernelGGL(rms_norm_kernel, dim3((unsigned)rows), dim3(256), 0, st, x, dim, w, eps, y);
  return hipGetLastError();
}

hipError_t rope_launch(float *x, int64_t ldx, int T, int heads, int hd, int n, int neox, const int *pos, int pos0,
                       double base, double freq_scale, const float *freqs, float *cs, hipStream_t st) {
  if (T <= 0) return hipSuccess;
  hipLaunchKernelGGL(rope_table_kernel, dim3(blocks_of(T, 64)), dim3(64), 0, st, pos, pos0, T, n,
                     pow(base, -2.0 / n), freq_scale, freqs, cs);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(rope_kernel, dim3(blocks_of((int64_t)heads * (n / 2), 256), T), dim3(256), 0, st, x, ldx, heads,
                     hd, n, neox, cs);
  return hipGetLastError();
}

hipError_t kv_store_launch(const float *k, const float *v, int64_t n, uint16_t *K, uint16_t *V, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(kv_store_kernel, dim3(blocks_of(n, 256)), dim3(256), 0, st, k, v, n, K, V);
  return hipGetLastError();
}

hipError_t attention_launch(const float *q, int64_t ldq, int T, const uint16_t *K, const uint16_t *V, int kv_dim,
                            int heads, int kv_heads, int hd, int pos0, float scale, float *scores, float *out,
                            int64_t ldo, hipStream_t st) {
  if (T <= 0) return hipSuccess;
  hipLaunchKernelGGL(attention_kernel, dim3(heads, T), dim3(256), 0, st, q, ldq, K, V, kv_dim, heads, kv_heads, hd,
                     pos0, scale, scores, (int64_t)(pos0 + T), out, ldo);
  return hipGetLastError();
}

hipError_t residual_launch(float *x, const float *o, int64_t n, float rs, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(residual_kernel, dim3(blocks_of(n, 256)), dim3(256), 0, st, x, o, n, rs);
  return hipGetLastError();
}

hipError_t argmax_launch(const float *logits, int rows, int64_t n, int *out, hipStream_t st) {
  if (rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(argmax_kernel, dim3((unsigned)rows), dim3(256), 0, st, logits, n, out);
  return hipGetLastError();
}

}  // namespace wl
