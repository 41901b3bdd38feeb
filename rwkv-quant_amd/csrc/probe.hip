// Bandwidth ceiling probe: streams a buffer with 16-byte loads (the access
// pattern of the GEMV kernels) and folds it into one value per workgroup,
// so the measured rate is the achievable HBM read ceiling on this device.
#include "rwkvq_common.h"

namespace {

__global__ void __launch_bounds__(256)
stream_read(const uint4* __restrict__ p, size_t n16, uint32_t* out) {
  uint32_t acc = 0;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    uint4 a = p[i], b = p[i + stride], c = p[i + 2 * stride],
          d = p[i + 3 * stride];
    acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^
           c.w ^ d.x ^ d.y ^ d.z ^ d.w;
  }
  for (; i < n16; i += stride) {
    uint4 a = p[i];
    acc ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  __shared__ uint32_t red[256];
  red[threadIdx.x] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t s = 0;
    for (int t = 0; t < 256; ++t) s ^= red[t];
    out[blockIdx.x] = s;
  }
}

}  // namespace

extern "C" int rwkvq_probe_stream_read(const void* buf, long bytes,
                                       uint32_t* out, int n_blocks,
                                       void* stream) {
  if (!buf || bytes < 16 || (bytes & 15) || n_blocks <= 0)
    return RWKVQ_ERR_ARG;
  hipLaunchKernelGGL(stream_read, dim3(n_blocks), dim3(256), 0,
                     (hipStream_t)stream, (const uint4*)buf,
                     (size_t)bytes / 16, out);
  return hipGetLastError() == hipSuccess ? RWKVQ_OK : RWKVQ_ERR_LAUNCH;
}
