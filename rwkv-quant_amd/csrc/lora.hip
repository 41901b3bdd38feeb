// Grouped dense-fp16 GEMV for the four low-rank branches (w, a, v, g) of an
// RWKV-7 time-mix layer: one launch runs all down projections, one launch
// all up projections.
//
// The LoRA matrices are the file's exact dequantization (asym gw64 @6 and
// per-row int8, expanded on the device at load) stored in fp16, as the
// reference stores dense 2-D parameters (reference:
// rwkv_quant/backends/metal/quant_model.py:128-154, 462-526).  Inputs are
// rounded to fp16 pairs, products and sums are fp32 (v_dot2_f32_f16).
#include "rwkvq_common.h"

using namespace rwkvq;

namespace {

struct LoraJob {
  const uint16_t* W;   // fp16 [rows, in] row-major
  const float* x;      // x[n * x_ld + c]
  float* y;            // y[n * y_ld + row]
  int rows, in, x_ld, y_ld, epi;
  int wave0;           // first wave index of this job in the grid
};

struct LoraJobs {
  LoraJob j[4];
  int n_jobs, N;
};

__device__ __forceinline__ float epi_apply(float v, int epi) {
  switch (epi) {
    case RWKVQ_EPI_TANH: return tanhf(v);
    case RWKVQ_EPI_SIGMOID: return 1.f / (1.f + __expf(-v));
    case RWKVQ_EPI_RELU2: return v > 0.f ? v * v : 0.f;
    default: return v;
  }
}

// One wave handles 8 rows; each row is split over 8 lanes (in <= 512) or the
// wave walks one row at a time with 64 lanes (wide rows).  N <= 8 inputs.
__global__ void __launch_bounds__(256)
lora_gemv_k(LoraJobs J) {
  const int lane = threadIdx.x & 63;
  const int gw = blockIdx.x * 4 + (threadIdx.x >> 6);     // global wave
  int jb = 0;
#pragma unroll
  for (int q = 1; q < 4; ++q)
    if (q < J.n_jobs && gw >= J.j[q].wave0) jb = q;
  const LoraJob& jo = J.j[jb];
  const int lw = gw - jo.wave0;
  if (jo.in > 512) {
    // wide: 64 lanes per row, 8 rows per wave, lane owns in/64 columns
    const int per = jo.in >> 6;                          // multiple of 2
    for (int rr = 0; rr < 8; ++rr) {
      const int row = lw * 8 + rr;
      if (row >= jo.rows) break;
      const uint32_t* wr = reinterpret_cast<const uint32_t*>(
          jo.W + (size_t)row * jo.in + lane * per);
      for (int n = 0; n < J.N; ++n) {
        const float* xp = jo.x + (size_t)n * jo.x_ld + lane * per;
        float acc = 0.f;
        for (int c = 0; c < per; c += 2)
          acc = dot2(wr[c >> 1], pack_h2(xp[c], xp[c + 1]), acc);
        acc = wave_sum_dpp(acc);
        if (lane == 0)
          jo.y[(size_t)n * jo.y_ld + row] = epi_apply(acc, jo.epi);
      }
    }
  } else {
    // narrow: 8 lanes per row, lane owns in/8 columns
    const int sub = lane & 7, row = lw * 8 + (lane >> 3);
    const int per = jo.in >> 3;                          // even
    const bool live = row < jo.rows;
    const uint32_t* wr = reinterpret_cast<const uint32_t*>(
        jo.W + (size_t)(live ? row : 0) * jo.in + sub * per);
    for (int n = 0; n < J.N; ++n) {
      const float* xp = jo.x + (size_t)n * jo.x_ld + sub * per;
      float acc = 0.f;
      for (int c = 0; c < per; c += 2)
        acc = dot2(wr[c >> 1], pack_h2(xp[c], xp[c + 1]), acc);
      acc += dpp_f<0xB1>(acc);
      acc += dpp_f<0x4E>(acc);
      acc += dpp_f<0x141>(acc);
      if (live && sub == 0)
        jo.y[(size_t)n * jo.y_ld + row] = epi_apply(acc, jo.epi);
    }
  }
}

}  // namespace

extern "C" int rwkvq_lora_gemv(int n_jobs, const void* const* W,
                               const float* const* x, const int* x_ld,
                               float* const* y, const int* y_ld,
                               const int* rows, const int* in, const int* epi,
                               int N, void* stream) {
  if (n_jobs <= 0 || n_jobs > 4 || N <= 0 || N > 8) return RWKVQ_ERR_ARG;
  LoraJobs J{};
  J.n_jobs = n_jobs;
  J.N = N;
  int waves = 0;
  for (int q = 0; q < n_jobs; ++q) {
    if (rows[q] <= 0 || in[q] <= 0 || in[q] % 16 ||
        (in[q] > 512 && in[q] % 128) || x_ld[q] < in[q] || y_ld[q] < rows[q])
      return RWKVQ_ERR_ARG;
    LoraJob& j = J.j[q];
    j.W = static_cast<const uint16_t*>(W[q]);
    j.x = x[q]; j.y = y[q];
    j.rows = rows[q]; j.in = in[q]; j.x_ld = x_ld[q]; j.y_ld = y_ld[q];
    j.epi = epi[q];
    j.wave0 = waves;
    waves += (rows[q] + 7) / 8;
  }
  hipLaunchKernelGGL(lora_gemv_k, dim3((waves + 3) / 4), dim3(256), 0,
                     (hipStream_t)stream, J);
  return hipGetLastError() == hipSuccess ? RWKVQ_OK : RWKVQ_ERR_LAUNCH;
}
