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

// One wave handles 4 (wide) or 8 (narrow) rows of one branch.
// Wide rows (in = 64 * PER, PER in {32, 40}): the 64 lanes split each row,
// lane owns PER columns; 4 rows are decoded together so their weight loads
// are in flight at once, x is read once per (wave, input row).
// Narrow rows (in <= 512): 8 lanes per row, lane owns in/8 columns.
// All column loops are fully unrolled (guards up to kMaxPer) so every load
// of a row is issued before the first use.
constexpr int kMaxPer = 64;

template <int PER>
__device__ __forceinline__ void lora_wide(const LoraJob& jo, int N, int lw,
                                          int lane) {
  // 4 rows per wave, all their weight loads in flight at once; lane l owns
  // the 8-column chunks l + 64 q (q < PER / 8), so consecutive lanes read
  // consecutive 16 bytes of a row (1 KiB per instruction)
  constexpr int PQ = PER / 8;
  float res[8][4];                             // stores deferred to the end
  uint4 wv[4][PQ];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = min(lw * 4 + j, jo.rows - 1);
    const uint4* wr = reinterpret_cast<const uint4*>(jo.W + (size_t)row * jo.in);
#pragma unroll
    for (int q = 0; q < PQ; ++q) wv[j][q] = wr[lane + 64 * q];
  }
#pragma unroll
  for (int n = 0; n < 8; ++n) {
    if (n >= N) break;
    const float4* xp =
        reinterpret_cast<const float4*>(jo.x + (size_t)n * jo.x_ld);
    uint4 xh[PQ];
#pragma unroll
    for (int q = 0; q < PQ; ++q) {
      const float4 f0 = xp[2 * (lane + 64 * q)], f1 = xp[2 * (lane + 64 * q) + 1];
      xh[q] = make_uint4(pack_h2(f0.x, f0.y), pack_h2(f0.z, f0.w),
                         pack_h2(f1.x, f1.y), pack_h2(f1.z, f1.w));
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float a = 0.f;
#pragma unroll
      for (int q = 0; q < PQ; ++q) {
        a = dot2(wv[j][q].x, xh[q].x, a);
        a = dot2(wv[j][q].y, xh[q].y, a);
        a = dot2(wv[j][q].z, xh[q].z, a);
        a = dot2(wv[j][q].w, xh[q].w, a);
      }
      res[n][j] = wave_sum_dpp(a);
    }
  }
  if (lane < 4) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = lw * 4 + j;
      if (j != lane || row >= jo.rows) continue;
#pragma unroll
      for (int n = 0; n < 8; ++n)
        if (n < N)
          jo.y[(size_t)n * jo.y_ld + row] = epi_apply(res[n][j], jo.epi);
    }
  }
}

__device__ __forceinline__ void lora_narrow(const LoraJob& jo, int N, int lw, int lane) {
  // 8 lanes per row; lane sub owns fp16 pairs p = sub + 8 q
  const int sub = lane & 7, row = lw * 8 + (lane >> 3);
  const int pairs = jo.in >> 1;
  const bool live = row < jo.rows;
  const uint32_t* wr = reinterpret_cast<const uint32_t*>(
      jo.W + (size_t)(live ? row : 0) * jo.in);
  uint32_t wv[kMaxPer / 2];
#pragma unroll
  for (int q = 0; q < kMaxPer / 2; ++q) {
    const int p = sub + 8 * q;
    wv[q] = p < pairs ? wr[p] : 0u;
  }
  float res[8];
#pragma unroll
  for (int n = 0; n < 8; ++n) {
    res[n] = 0.f;
    if (n >= N) continue;
    const float2* xp =
        reinterpret_cast<const float2*>(jo.x + (size_t)n * jo.x_ld);
    float acc = 0.f;
#pragma unroll
    for (int q = 0; q < kMaxPer / 2; ++q) {
      const int p = sub + 8 * q;
      if (p < pairs) {
        const float2 f = xp[p];
        acc = dot2(wv[q], pack_h2(f.x, f.y), acc);
      }
    }
    acc += dpp_f<0xB1>(acc);
    acc += dpp_f<0x4E>(acc);
    acc += dpp_f<0x141>(acc);
    res[n] = acc;
  }
  if (live && sub == 0) {
#pragma unroll
    for (int n = 0; n < 8; ++n)
      if (n < N) jo.y[(size_t)n * jo.y_ld + row] = epi_apply(res[n], jo.epi);
  }
}

__device__ __forceinline__ void lora_run(const LoraJob& jo, int N, int gw,
                                         int lane) {
  const int lw = gw - jo.wave0;
  if (jo.in == 64 * 32 || jo.in == 64 * 40) {
    if (lw * 4 >= jo.rows) return;
    if (jo.in == 64 * 32) lora_wide<32>(jo, N, lw, lane);
    else lora_wide<40>(jo, N, lw, lane);
  } else {
    if (lw * 8 >= jo.rows) return;
    lora_narrow(jo, N, lw, lane);
  }
}

__global__ void __launch_bounds__(256)
lora_gemv_k(LoraJobs J) {
  const int lane = threadIdx.x & 63;
  const int gw = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(
                                      threadIdx.x >> 6);
  // the job is wave-uniform; each case reads the kernel-argument table
  // with constant offsets (a dynamic index would copy it to scratch)
  int jb = 0;
  if (J.n_jobs > 1 && gw >= J.j[1].wave0) jb = 1;
  if (J.n_jobs > 2 && gw >= J.j[2].wave0) jb = 2;
  if (J.n_jobs > 3 && gw >= J.j[3].wave0) jb = 3;
  switch (jb) {
    case 0: lora_run(J.j[0], J.N, gw, lane); break;
    case 1: lora_run(J.j[1], J.N, gw, lane); break;
    case 2: lora_run(J.j[2], J.N, gw, lane); break;
    default: lora_run(J.j[3], J.N, gw, lane); break;
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
    const bool wide = in[q] == 64 * 32 || in[q] == 64 * 40;
    if (rows[q] <= 0 || in[q] <= 0 || in[q] % 16 ||
        (!wide && in[q] > 8 * kMaxPer) || x_ld[q] < in[q] ||
        (wide && (((uintptr_t)x[q] & 15) || x_ld[q] % 4)) ||   // float4 x
        y_ld[q] < rows[q])
      return RWKVQ_ERR_ARG;
    LoraJob& j = J.j[q];
    j.W = static_cast<const uint16_t*>(W[q]);
    j.x = x[q]; j.y = y[q];
    j.rows = rows[q]; j.in = in[q]; j.x_ld = x_ld[q]; j.y_ld = y_ld[q];
    j.epi = epi[q];
    j.wave0 = waves;
    waves += wide ? (rows[q] + 3) / 4 : (rows[q] + 7) / 8;
  }
  hipLaunchKernelGGL(lora_gemv_k, dim3((waves + 3) / 4), dim3(256), 0,
                     (hipStream_t)stream, J);
  return hipGetLastError() == hipSuccess ? RWKVQ_OK : RWKVQ_ERR_LAUNCH;
}
