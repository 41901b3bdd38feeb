// SpQR outliers of the per-row int8 (rtn) format, as CSR per output row:
// row_ptr[rows + 1], cols[nnz], vals[nnz] (bf16, the stored values; the
// codes are 0 at these positions).  Outside the lane-dot GEMV, which sums
// them itself, the tail is added by its own kernel after the GEMV / GEMM.
// (reference: rwkv_quant/backends/metal/quant_linear_v2.py:44-53, 300-321)
#include "rwkvq_common.h"
#include "rwkvq_hip.h"

using namespace rwkvq;

namespace {

__device__ __forceinline__ float bf16_f32(uint16_t u) {
  return __builtin_bit_cast(float, (uint32_t)u << 16);
}

// one wave per (input row n, output row r): lanes stride the row's
// outliers, a fixed-order lane sum, then the epilogue
__global__ void __launch_bounds__(256)
spqr_apply_k(const float* __restrict__ x, long x_ld,
             const int* __restrict__ row_ptr, const int* __restrict__ cols,
             const uint16_t* __restrict__ vals, int rows, int n,
             float* __restrict__ y, int mode) {
  const int lane = threadIdx.x & 63;
  const long item = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= (long)rows * n) return;
  const int r = (int)(item % rows), t = (int)(item / rows);
  const float* xr = x + (size_t)t * x_ld;
  float s = 0.f;
  for (int k = row_ptr[r] + lane; k < row_ptr[r + 1]; k += 64)
    s += bf16_f32(vals[k]) * xr[cols[k]];
  s = wave_sum_dpp(s);
  if (lane) return;
  float v = y[(size_t)t * rows + r] + s;
  switch (mode) {
    case RWKVQ_EPI_RELU2: v = v > 0.f ? v * v : 0.f; break;
    case RWKVQ_EPI_TANH: v = tanhf(v); break;
    case RWKVQ_EPI_SIGMOID: v = 1.f / (1.f + __expf(-v)); break;
    default: break;
  }
  y[(size_t)t * rows + r] = v;
}

__global__ void __launch_bounds__(256)
spqr_scatter_k(const int* __restrict__ row_ptr, const int* __restrict__ cols,
               const uint16_t* __restrict__ vals, int rows,
               float* __restrict__ w, long ld) {
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  for (int k = row_ptr[r] + (threadIdx.x & 63); k < row_ptr[r + 1]; k += 64)
    w[(size_t)r * ld + cols[k]] = bf16_f32(vals[k]);
}

}  // namespace

extern "C" {

int rwkvq_spqr_apply(const float* x, long x_ld, const int* row_ptr,
                     const int* cols, const uint16_t* vals, int rows, int n,
                     float* y, int mode, void* stream) {
  if (!x || !row_ptr || !cols || !vals || !y || rows <= 0 || n <= 0 ||
      x_ld <= 0 || mode < 0 || mode > RWKVQ_EPI_SIGMOID ||
      mode == RWKVQ_EPI_ADD)
    return RWKVQ_ERR_ARG;
  const long items = (long)rows * n;
  hipLaunchKernelGGL(spqr_apply_k, dim3((unsigned)((items + 3) / 4)),
                     dim3(256), 0, (hipStream_t)stream, x, x_ld, row_ptr,
                     cols, vals, rows, n, y, mode);
  return hipGetLastError() == hipSuccess ? RWKVQ_OK : RWKVQ_ERR_LAUNCH;
}

int rwkvq_spqr_scatter(const int* row_ptr, const int* cols,
                       const uint16_t* vals, int rows, float* w, long ld,
                       void* stream) {
  if (!row_ptr || !cols || !vals || !w || rows <= 0 || ld <= 0)
    return RWKVQ_ERR_ARG;
  hipLaunchKernelGGL(spqr_scatter_k, dim3((rows + 3) / 4), dim3(256), 0,
                     (hipStream_t)stream, row_ptr, cols, vals, rows, w, ld);
  return hipGetLastError() == hipSuccess ? RWKVQ_OK : RWKVQ_ERR_LAUNCH;
}

}  // extern "C"
