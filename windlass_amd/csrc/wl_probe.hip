// wl_probe.hip - a plain streaming read of device memory: the HBM read rate a kernel that does
// nothing but load can reach on this device, the practical ceiling the decode GEMVs are compared
// with (their algorithmic bytes are reads, their writes a few KB).
//
// Each thread walks the buffer in 16-byte loads with a grid stride, four loads in flight per
// iteration, so every wave load instruction reads 1 KB contiguous. The values are folded with
// XOR and stored only if the fold equals a constant no buffer here produces, which keeps every
// load live without a store per thread.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "wl_probe.h"

namespace wl {

__global__ __launch_bounds__(256) void read_peak_kernel(const uint4 *__restrict__ src, int64_t n16,
                                                        uint32_t *__restrict__ out) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint32_t acc = 0;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const uint4 a = src[i], b = src[i + stride], c = src[i + 2 * stride], d = src[i + 3 * stride];
    acc ^= (a.x ^ a.y ^ a.z ^ a.w) ^ (b.x ^ b.y ^ b.z ^ b.w) ^ (c.x ^ c.y ^ c.z ^ c.w) ^ (d.x ^ d.y ^ d.z ^ d.w);
  }
  for (; i < n16; i += stride) {
    const uint4 a = src[i];
    acc ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  if (acc == 0x9E3779B9u) out[0] = acc;
}

hipError_t read_peak_launch(const void *src, int64_t bytes, int workgroups, uint32_t *out, hipStream_t st) {
  if (bytes < 16 || workgroups < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(read_peak_kernel, dim3(workgroups), dim3(256), 0, st, (const uint4 *)src, bytes / 16, out);
  return hipGetLastError();
}

}  // namespace wl
