// Next-token negative log-likelihood per logits row, for the perplexity
// harness: nll[r] = logsumexp(logits[r, :]) - logits[r, target[r]].
//
// One workgroup per row.  Each thread keeps an online (max, scaled sum)
// pair over its strided share of the row (one pass over the logits, read
// with 16-byte loads), the pairs are merged in a fixed tree order in LDS,
// so the result is deterministic.  A target outside [0, V) gives NaN
// instead of a read out of bounds; NaN logits give NaN.
// (reference: rwkv_quant/calibration/ablation.py:21-69 -- logsumexp minus
// the gathered target logit, without materialising log_softmax)
#include "rwkvq_common.h"
#include "rwkvq_hip.h"

namespace {

constexpr int kNllThreads = 256;

__device__ __forceinline__ void merge(float& m, float& s, float m2,
                                      float s2) {
  if (m2 > m) {
    s = s * __expf(m - m2) + s2;
    m = m2;
  } else if (m2 > -INFINITY) {
    s += s2 * __expf(m2 - m);
  }
}

__global__ void __launch_bounds__(kNllThreads)
nll_rows_k(const float* __restrict__ logits, long ld,
           const int64_t* __restrict__ target, int V,
           float* __restrict__ nll) {
  const float* row = logits + (size_t)blockIdx.x * ld;
  float m = -INFINITY, s = 0.f;
  const int v4 = V >> 2;
  for (int i = threadIdx.x; i < v4; i += kNllThreads) {
    const float4 f = reinterpret_cast<const float4*>(row)[i];
    const float lm = fmaxf(fmaxf(f.x, f.y), fmaxf(f.z, f.w));
    const float ls = __expf(f.x - lm) + __expf(f.y - lm) +
                     __expf(f.z - lm) + __expf(f.w - lm);
    merge(m, s, lm, ls);
    if (isnan(f.x + f.y + f.z + f.w)) s = NAN;   // NaN logits propagate
  }
  for (int i = 4 * v4 + threadIdx.x; i < V; i += kNllThreads) {
    merge(m, s, row[i], 1.f);
    if (isnan(row[i])) s = NAN;
  }
  __shared__ float sm[kNllThreads], ss[kNllThreads];
  sm[threadIdx.x] = m;
  ss[threadIdx.x] = s;
  __syncthreads();
  for (int w = kNllThreads / 2; w > 0; w >>= 1) {
    if (threadIdx.x < w) {
      float a = sm[threadIdx.x], b = ss[threadIdx.x];
      merge(a, b, sm[threadIdx.x + w], ss[threadIdx.x + w]);
      sm[threadIdx.x] = a;
      ss[threadIdx.x] = b;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const int64_t t = target[blockIdx.x];
    const float lse = sm[0] + __logf(ss[0]);
    nll[blockIdx.x] = (t >= 0 && t < V) ? lse - row[t] : NAN;
  }
}

}  // namespace

extern "C" int rwkvq_nll_rows(const float* logits, long ld,
                              const int64_t* target, int rows, int V,
                              float* nll, void* stream) {
  if (!logits || !target || !nll || rows <= 0 || V <= 0 || ld < V ||
      (ld & 3) || (reinterpret_cast<uintptr_t>(logits) & 15))
    return RWKVQ_ERR_ARG;
  hipLaunchKernelGGL(nll_rows_k, dim3(rows), dim3(kNllThreads), 0,
                     (hipStream_t)stream, logits, ld, target, V, nll);
  return hipGetLastError() == hipSuccess ? RWKVQ_OK : RWKVQ_ERR_LAUNCH;
}
