// RWKV-7 time-mix / channel-mix kernels around the quantized GEMVs:
// layer norm + token shift + lerps, the per-channel WKV inputs, the WKV-7
// recurrence and the fused group-norm/bonus/gate tail.
//
// Math (reference: rwkv_quant/models/rwkv7_ref.py:184-255,
//                  rwkv_quant/backends/metal/quant_model.py:264-301, 638-728,
//                  803-809; rwkv_quant/backends/metal/fused_tail.py:43-77):
//   xn  = LN(x) (eps 1e-5);  xx = shift(xn) - xn;  x_c = xn + xx * coef_c
//   w   = exp(-0.606531 * sigmoid(y_w + w0))        (= exp(-exp(-softplus(
//                                                    -(y_w+w0)) - 0.5)))
//   a   = sigmoid(y_a + a0);  kk = l2norm_head(k * k_k)
//   k'  = k * (1 + (a - 1) * k_a)
//   v'  = v (layer 0, becomes v_first) | v + (v_first - v) * sigmoid(y_v+v0)
//   S_t = S_{t-1} diag(w) + (S_{t-1} a_t) b_t^T + v_t k_t^T, a = -kk,
//         b = kk * a;  y_t = S_t r_t      (S[i][j]: i value row, j key col)
//   out = ((GN(y) * ln_x_w + ln_x_b) + (sum_head r * k' * r_k) * v') * g
//         (group norm per head, two-pass, eps 64e-5)
#include "rwkvq_common.h"

using namespace rwkvq;

namespace {

constexpr int kHead = 64;   // head size N (kernels below assume 64)

// block-wide sum of one value per thread (blockDim.x multiple of 64, <= 1024)
__device__ __forceinline__ float block_sum(float v, float* sh) {
  v = wave_sum_dpp(v);
  const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh[w] = v;
  __syncthreads();
  float s = 0.f;
  for (int i = 0; i < nw; ++i) s += sh[i];
  return s;
}

// Mean and rstd of one row of D floats (two-pass, as the reference).
__device__ __forceinline__ void row_stats(const float* row, int D, float eps,
                                          float* sh, float& mean,
                                          float& rstd) {
  float s = 0.f;
  for (int c = threadIdx.x; c < D; c += blockDim.x) s += row[c];
  mean = block_sum(s, sh) / (float)D;
  float q = 0.f;
  for (int c = threadIdx.x; c < D; c += blockDim.x) {
    float d = row[c] - mean;
    q += d * d;
  }
  float var = block_sum(q, sh) / (float)D;
  rstd = 1.f / sqrtf(var + eps);
}

// y = LN(x) row-wise (x and y may alias)
__global__ void __launch_bounds__(256)
layer_norm_k(const float* x, const float* w, const float* b, float* y, int D,
             float eps) {
  __shared__ float sh[16];
  const float* xr = x + (size_t)blockIdx.x * D;
  float mean, rstd;
  row_stats(xr, D, eps, sh, mean, rstd);
  float* yr = y + (size_t)blockIdx.x * D;
  for (int c = threadIdx.x; c < D; c += blockDim.x)
    yr[c] = (xr[c] - mean) * rstd * w[c] + b[c];
}

// LN + token shift + ncoef lerps for one token row (b, t):
//   out[(b*T+t), k, :] = xn + (shift - xn) * coef[k, :]
// shift = xn of (b, t-1), or prev[b] (zeros when prev is null) at t = 0.
// new_prev[b] = xn of (b, T-1).  ln_out (optional) receives xn.
__global__ void __launch_bounds__(256)
shift_lerp_k(const float* x, const float* lw, const float* lb,
             const float* prev, const float* coef, int ncoef, float* out,
             float* new_prev, int T, int D) {
  __shared__ float sh[16];
  const int row = blockIdx.x;           // b * T + t
  const int t = row % T, bb = row / T;
  const float* xr = x + (size_t)row * D;
  float mean, rstd;
  row_stats(xr, D, 1e-5f, sh, mean, rstd);
  float pmean = 0.f, prstd = 0.f;
  if (t > 0) row_stats(xr - D, D, 1e-5f, sh, pmean, prstd);
  for (int c = threadIdx.x; c < D; c += blockDim.x) {
    const float xn = (xr[c] - mean) * rstd * lw[c] + lb[c];
    float sv;
    if (t > 0) sv = (xr[c - D] - pmean) * prstd * lw[c] + lb[c];
    else sv = prev ? prev[(size_t)bb * D + c] : 0.f;
    const float xx = sv - xn;
    for (int k = 0; k < ncoef; ++k)
      out[((size_t)row * ncoef + k) * D + c] = xn + xx * coef[(size_t)k * D + c];
    if (t == T - 1 && new_prev) new_prev[(size_t)bb * D + c] = xn;
  }
}

__device__ __forceinline__ float sigm(float v) { return 1.f / (1.f + __expf(-v)); }

// Per-channel WKV inputs.  One wave = one (token, head).
//   rkv [N, 3, D] (r, k, v);  yw, ya, yv, g [N, D] (LoRA outputs; yv may be
//   null on layer 0);  vfirst [N, D] written on layer 0, read otherwise.
//   outputs w, kp, vp, aa, bb [N, D]
__global__ void __launch_bounds__(256)
wkv_prep_k(const float* rkv, const float* yw, const float* ya, const float* yv,
           const float* w0, const float* a0, const float* v0, const float* k_k,
           const float* k_a, float* vfirst, int layer0, float* wo, float* kpo,
           float* vpo, float* aao, float* bbo, int D) {
  const int n = blockIdx.y;
  const int c = blockIdx.x * blockDim.x + threadIdx.x;    // channel
  const size_t e = (size_t)n * D + c;
  const float k = rkv[((size_t)n * 3 + 1) * D + c];
  float v = rkv[((size_t)n * 3 + 2) * D + c];
  const float wv = __expf(-0.606531f * sigm(yw[e] + w0[c]));
  const float av = sigm(ya[e] + a0[c]);
  const float kkr = k * k_k[c];
  const float ss = wave_sum_dpp(kkr * kkr);               // head = one wave
  const float kk = kkr / sqrtf(ss + 1e-12f);
  const float kp = k * (1.f + (av - 1.f) * k_a[c]);
  if (layer0) {
    vfirst[e] = v;
  } else {
    const float vf = vfirst[e];
    v = v + (vf - v) * sigm(yv[e] + v0[c]);
  }
  wo[e] = wv;
  kpo[e] = kp;
  vpo[e] = v;
  aao[e] = -kk;
  bbo[e] = kk * av;
}

// WKV-7 recurrence.  Block = RB rows of one (batch, head) x L lanes per row;
// lane (row i, part p) keeps S[i][p*C .. p*C+C) in registers (C = 64 / L).
// The (S a) and (S r) row sums meet over the L lanes with DPP.
template <int L>
__global__ void __launch_bounds__(128)
wkv_scan_k(const float* r, long r_ld, const float* w, const float* k,
           const float* v, const float* aa, const float* bb, long ld,
           const float* state_in, float* state, float* y, long y_ld, int T,
           int H, int RB) {
  constexpr int C = kHead / L;
  const int nblk = kHead / RB;
  const int bh = blockIdx.x / nblk, rb = blockIdx.x % nblk;
  const int bi = bh / H, h = bh % H;
  const int part = threadIdx.x % L;
  const int i = rb * RB + threadIdx.x / L;                 // value row
  const size_t soff = (((size_t)bi * H + h) * kHead + i) * kHead + part * C;
  float* Sp = state + soff;
  float S[C];
#pragma unroll
  for (int c = 0; c < C; c += 4) {
    float4 q = *reinterpret_cast<const float4*>(state_in + soff + c);
    S[c] = q.x; S[c + 1] = q.y; S[c + 2] = q.z; S[c + 3] = q.w;
  }
  const size_t col = (size_t)h * kHead + part * C;
  for (int t = 0; t < T; ++t) {
    const size_t tok = (size_t)bi * T + t;
    const float* wp = w + tok * ld + col;
    const float* kp = k + tok * ld + col;
    const float* ap = aa + tok * ld + col;
    const float* bp = bb + tok * ld + col;
    const float* rp = r + tok * r_ld + col;
    const float vi = v[tok * ld + (size_t)h * kHead + i];
    float av[C], bv[C], wv[C], kv[C], rv[C];
#pragma unroll
    for (int c = 0; c < C; c += 4) {
      float4 q;
      q = *reinterpret_cast<const float4*>(ap + c);
      av[c] = q.x; av[c + 1] = q.y; av[c + 2] = q.z; av[c + 3] = q.w;
      q = *reinterpret_cast<const float4*>(bp + c);
      bv[c] = q.x; bv[c + 1] = q.y; bv[c + 2] = q.z; bv[c + 3] = q.w;
      q = *reinterpret_cast<const float4*>(wp + c);
      wv[c] = q.x; wv[c + 1] = q.y; wv[c + 2] = q.z; wv[c + 3] = q.w;
      q = *reinterpret_cast<const float4*>(kp + c);
      kv[c] = q.x; kv[c + 1] = q.y; kv[c + 2] = q.z; kv[c + 3] = q.w;
      q = *reinterpret_cast<const float4*>(rp + c);
      rv[c] = q.x; rv[c + 1] = q.y; rv[c + 2] = q.z; rv[c + 3] = q.w;
    }
    float sa = 0.f;
#pragma unroll
    for (int c = 0; c < C; ++c) sa += S[c] * av[c];
    if (L >= 2) sa += dpp_f<0xB1>(sa);     // xor 1
    if (L >= 4) sa += dpp_f<0x4E>(sa);     // xor 2
    if (L >= 8) sa += dpp_f<0x141>(sa);    // half-row mirror
    float yv = 0.f;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      S[c] = S[c] * wv[c] + sa * bv[c] + vi * kv[c];
      yv += S[c] * rv[c];
    }
    if (L >= 2) yv += dpp_f<0xB1>(yv);
    if (L >= 4) yv += dpp_f<0x4E>(yv);
    if (L >= 8) yv += dpp_f<0x141>(yv);
    if (part == 0) y[tok * y_ld + (size_t)h * kHead + i] = yv;
  }
#pragma unroll
  for (int c = 0; c < C; c += 4)
    *reinterpret_cast<float4*>(Sp + c) = make_float4(S[c], S[c + 1], S[c + 2],
                                                     S[c + 3]);
}

// Group norm per head + bonus + gate.  One wave = one (token, head).
__global__ void __launch_bounds__(256)
wkv_tail_k(const float* y, const float* rkv, const float* kp, const float* vp,
           const float* g, const float* r_k, const float* lnw,
           const float* lnb, float* out, int D) {
  const int n = blockIdx.y;
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  const size_t e = (size_t)n * D + c;
  const float yv = y[e];
  const float mean = wave_sum_dpp(yv) * (1.f / kHead);
  const float dv = yv - mean;
  const float var = wave_sum_dpp(dv * dv) * (1.f / kHead);
  const float nrm = dv / sqrtf(var + 64e-5f);
  const float r = rkv[(size_t)n * 3 * D + c];
  const float dp = wave_sum_dpp(r * kp[e] * r_k[c]);
  out[e] = ((nrm * lnw[c] + lnb[c]) + dp * vp[e]) * g[e];
}

inline int ok_launch() {
  return hipGetLastError() == hipSuccess ? RWKVQ_OK : RWKVQ_ERR_LAUNCH;
}

}  // namespace

extern "C" {

int rwkvq_layer_norm(const float* x, const float* w, const float* b, float* y,
                     int rows, int D, float eps, void* stream) {
  if (rows <= 0 || D <= 0) return RWKVQ_ERR_ARG;
  hipLaunchKernelGGL(layer_norm_k, dim3(rows), dim3(256), 0,
                     (hipStream_t)stream, x, w, b, y, D, eps);
  return ok_launch();
}

int rwkvq_shift_lerp(const float* x, const float* ln_w, const float* ln_b,
                     const float* prev, const float* coef, int ncoef,
                     float* out, float* new_prev, int B, int T, int D,
                     void* stream) {
  if (B <= 0 || T <= 0 || D <= 0 || ncoef <= 0 || ncoef > 8)
    return RWKVQ_ERR_ARG;
  hipLaunchKernelGGL(shift_lerp_k, dim3(B * T), dim3(256), 0,
                     (hipStream_t)stream, x, ln_w, ln_b, prev, coef, ncoef,
                     out, new_prev, T, D);
  return ok_launch();
}

int rwkvq_wkv_prep(const float* rkv, const float* yw, const float* ya,
                   const float* yv, const float* w0, const float* a0,
                   const float* v0, const float* k_k, const float* k_a,
                   float* v_first, int layer0, float* w, float* kp, float* vp,
                   float* a, float* b, int N, int D, int head_size,
                   void* stream) {
  if (N <= 0 || D <= 0 || head_size != kHead || D % 256 ||
      (!layer0 && (!yv || !v0)))
    return RWKVQ_ERR_ARG;
  hipLaunchKernelGGL(wkv_prep_k, dim3(D / 256, N), dim3(256), 0,
                     (hipStream_t)stream, rkv, yw, ya, yv, w0, a0, v0, k_k,
                     k_a, v_first, layer0, w, kp, vp, a, b, D);
  return ok_launch();
}

int rwkvq_wkv7_scan(const float* r, long r_ld, const float* w, const float* k,
                    const float* v, const float* a, const float* b, long ld,
                    const float* state_in, float* state_out, float* y,
                    long y_ld, int B, int T, int H, int head_size,
                    void* stream) {
  if (B <= 0 || T <= 0 || H <= 0 || head_size != kHead || ld < H * kHead ||
      r_ld < H * kHead || y_ld < H * kHead || (r_ld & 3) || (ld & 3))
    return RWKVQ_ERR_ARG;
  constexpr int L = 8, RB = 16;
  hipLaunchKernelGGL((wkv_scan_k<L>), dim3(B * H * (kHead / RB)),
                     dim3(RB * L), 0, (hipStream_t)stream, r, r_ld, w, k, v,
                     a, b, ld, state_in ? state_in : state_out, state_out, y,
                     y_ld, T, H, RB);
  return ok_launch();
}

int rwkvq_wkv_tail(const float* y, const float* rkv, const float* kp,
                   const float* vp, const float* g, const float* r_k,
                   const float* ln_w, const float* ln_b, float* out, int N,
                   int D, int head_size, void* stream) {
  if (N <= 0 || D % 256 || head_size != kHead) return RWKVQ_ERR_ARG;
  hipLaunchKernelGGL(wkv_tail_k, dim3(D / 256, N), dim3(256), 0,
                     (hipStream_t)stream, y, rkv, kp, vp, g, r_k, ln_w, ln_b,
                     out, D);
  return ok_launch();
}

}  // extern "C"
