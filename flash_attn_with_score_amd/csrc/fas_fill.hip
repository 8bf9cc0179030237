// Zero-fill of strided fp32 outputs for degenerate shapes (no query rows or
// no keys).  A kernel rather than hipMemsetAsync so a captured launch
// sequence holds no memset node, and because the outputs may be strided.
#include "fas_launch.hpp"

namespace fas {

__global__ void fill_zero_3d(float* p, int64_t s0, int64_t s1, int64_t s2, int64_t n0, int64_t n1,
                             int64_t n2) {
  const int64_t total = n0 * n1 * n2;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i2 = i % n2;
    const int64_t i1 = (i / n2) % n1;
    const int64_t i0 = i / (n1 * n2);
    p[i0 * s0 + i1 * s1 + i2 * s2] = 0.f;
  }
}

hipError_t launch_fill_zero(float* p, int64_t s0, int64_t s1, int64_t s2, int64_t n0, int64_t n1,
                            int64_t n2, hipStream_t s) {
  const int64_t total = n0 * n1 * n2;
  if (total <= 0) return hipSuccess;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(fill_zero_3d, dim3((unsigned)blocks), dim3(256), 0, s, p, s0, s1, s2, n0, n1,
                     n2);
  return hipGetLastError();
}

}  // namespace fas
