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
#include "gather_cols.h"

#include <mutex>

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

// Row kernels keep the row in registers: thread t owns columns t + 256 e,
// e < kMaxE, so every load of a row is issued before the first use (a
// loop over dependent global loads would pay the memory latency per
// iteration).  D <= 256 * kMaxE.
constexpr int kRowThreads = 256;
constexpr int kMaxE = 16;

__device__ __forceinline__ void load_row(const float* row, int D,
                                         float (&v)[kMaxE]) {
#pragma unroll
  for (int e = 0; e < kMaxE; ++e) {
    const int c = threadIdx.x + e * kRowThreads;
    v[e] = c < D ? row[c] : 0.f;
  }
}

// Mean and rstd of a register-resident row (two-pass, as the reference).
__device__ __forceinline__ void row_stats(const float (&v)[kMaxE], int D,
                                          float eps, float* sh, float& mean,
                                          float& rstd) {
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < kMaxE; ++e) s += v[e];
  mean = block_sum(s, sh) / (float)D;
  float q = 0.f;
#pragma unroll
  for (int e = 0; e < kMaxE; ++e) {
    const int c = threadIdx.x + e * kRowThreads;
    const float d = c < D ? v[e] - mean : 0.f;
    q += d * d;
  }
  const float var = block_sum(q, sh) / (float)D;
  rstd = 1.f / sqrtf(var + eps);
}

// y = LN(x) row-wise (x and y may alias)
__global__ void __launch_bounds__(kRowThreads)
layer_norm_k(const float* x, const float* __restrict__ w,
             const float* __restrict__ b, float* y, int D, float eps) {
  __shared__ float sh[16];
  float v[kMaxE], cw[kMaxE], cb[kMaxE];
  load_row(x + (size_t)blockIdx.x * D, D, v);
  load_row(w, D, cw);
  load_row(b, D, cb);
  float mean, rstd;
  row_stats(v, D, eps, sh, mean, rstd);
  float* yr = y + (size_t)blockIdx.x * D;
#pragma unroll
  for (int e = 0; e < kMaxE; ++e) {
    const int c = threadIdx.x + e * kRowThreads;
    if (c < D) yr[c] = (v[e] - mean) * rstd * cw[e] + cb[e];
  }
}

// Embedding row gather fused with the LayerNorm after it (ln0): one
// workgroup per output row decodes the row straight from the packed table
// into LDS (8 consecutive columns per thread, the arithmetic of the row
// gather), then runs layer_norm_k's LayerNorm over it with the same column
// ownership and reduction order -- the output equals gather + layer_norm_k
// bit for bit, one launch instead of two.
// KIND 0 = sb6 (aux0 = rec), 1 = sym (aux0 = qs, aux1 = d), 2 = rtn@8
// (aux1 = scale).
template <int KIND>
__global__ void __launch_bounds__(kRowThreads)
gather_ln_k(const uint8_t* q, const uint32_t* hb, const void* aux0,
            const uint16_t* aux1, int bits, int src_rows, int D,
            const int64_t* idx, const float* __restrict__ w,
            const float* __restrict__ b, float* y, float eps) {
  __shared__ float sh[16];
  __shared__ float4 s_row4[kRowThreads * kMaxE / 4];
  float* s_row = reinterpret_cast<float*>(s_row4);
  const int orow = blockIdx.x;
  const int row = src_row(idx, orow, src_rows);
  for (int k = threadIdx.x; k < D / 8; k += kRowThreads) {
    float o[8];
    if constexpr (KIND == 0)
      sb6_cols8(q, hb, static_cast<const uint8_t*>(aux0), bits, D, row, k, o);
    else if constexpr (KIND == 1)
      sym_cols8(q, hb, static_cast<const int8_t*>(aux0), aux1, bits, D, row,
                k, o);
    else
      rtn8_cols8(reinterpret_cast<const int8_t*>(q), aux1, D, row, k, o);
    s_row4[2 * k] = make_float4(o[0], o[1], o[2], o[3]);
    s_row4[2 * k + 1] = make_float4(o[4], o[5], o[6], o[7]);
  }
  float v[kMaxE], cw[kMaxE], cb[kMaxE];
  load_row(w, D, cw);
  load_row(b, D, cb);
  __syncthreads();
#pragma unroll
  for (int e = 0; e < kMaxE; ++e) {
    const int c = threadIdx.x + e * kRowThreads;
    v[e] = c < D ? s_row[c] : 0.f;
  }
  float mean, rstd;
  row_stats(v, D, eps, sh, mean, rstd);
  float* yr = y + (size_t)orow * D;
#pragma unroll
  for (int e = 0; e < kMaxE; ++e) {
    const int c = threadIdx.x + e * kRowThreads;
    if (c < D) yr[c] = (v[e] - mean) * rstd * cw[e] + cb[e];
  }
}

// Row held as float4s: thread t owns columns 4 (t + 256 e) .. +3, e <
// kMaxE4 (D <= 4096, D % 4 == 0) -- a quarter of the load and store
// instructions of the scalar layout, which matters when one workgroup
// carries a whole decode row.
constexpr int kMaxE4 = 4;

__device__ __forceinline__ void load_row4(const float* row, int D,
                                          float4 (&v)[kMaxE4]) {
#pragma unroll
  for (int e = 0; e < kMaxE4; ++e) {
    const int c = 4 * (threadIdx.x + e * kRowThreads);
    v[e] = c < D ? *reinterpret_cast<const float4*>(row + c)
                 : make_float4(0.f, 0.f, 0.f, 0.f);
  }
}

// Mean and rstd of a float4 register row (two-pass, as the reference).
__device__ __forceinline__ void row_stats4(const float4 (&v)[kMaxE4], int D,
                                           float eps, float* sh, float& mean,
                                           float& rstd) {
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < kMaxE4; ++e) s += (v[e].x + v[e].y) + (v[e].z + v[e].w);
  mean = block_sum(s, sh) / (float)D;
  float q = 0.f;
#pragma unroll
  for (int e = 0; e < kMaxE4; ++e) {
    const int c = 4 * (threadIdx.x + e * kRowThreads);
    if (c < D) {
      const float a = v[e].x - mean, b = v[e].y - mean, cc = v[e].z - mean,
                  d = v[e].w - mean;
      q += (a * a + b * b) + (cc * cc + d * d);
    }
  }
  const float var = block_sum(q, sh) / (float)D;
  rstd = 1.f / sqrtf(var + eps);
}

// fp16 stores in a GEMM input pair order (within each 32-column group,
// halves 2i, 2i+1 = columns (c0(i), c1(i)); RWKVQ_ORDER_*).  Lanes holding
// consecutive columns form the groups, so a column's partner is held by the
// lane at a fixed xor distance in the same wave; the lane of the lower
// column writes the pair.  All lanes of a 32-column group must call these.
//   store_pairs4: a lane holds columns c .. c + 3 (c % 4 == 0)
// (the pins keep each value rounded to fp32 before its fp16 rounding, as
// the fp32 output followed by a conversion: without them the compiler may
// fuse the producing multiply-add and the conversion into one mixed-precision
// instruction that rounds once)
template <int ORD>
__device__ __forceinline__ void store_pairs4(uint16_t* row, int c, float4 o) {
  pin(o);
  const uint32_t lo = pack_h2(o.x, o.y), hi = pack_h2(o.z, o.w);
  if constexpr (ORD == RWKVQ_ORDER_PAIRS) {
    *reinterpret_cast<uint2*>(row + c) = make_uint2(lo, hi);
  } else {
    constexpr int m = ORD == RWKVQ_ORDER_SB6 ? 4 : 2;   // partner c + 16 / 8
    const uint32_t plo = __shfl_xor(lo, m, 64), phi = __shfl_xor(hi, m, 64);
    const int cg = c & 31;
    if (((cg >> 2) & m) == 0) {
      const int pos = 2 * cg - (cg >= 16 ? 16 : 0);
      *reinterpret_cast<uint4*>(row + (c - cg) + pos) =
          make_uint4((lo & 0xFFFFu) | (plo << 16), (lo >> 16) | (plo & 0xFFFF0000u),
                     (hi & 0xFFFFu) | (phi << 16), (hi >> 16) | (phi & 0xFFFF0000u));
    }
  }
}
//   store_pairs1: a lane holds column c
template <int ORD>
__device__ __forceinline__ void store_pairs1(uint16_t* row, int c, float v) {
  pin(v);
  constexpr int m = ORD == RWKVQ_ORDER_PAIRS ? 1
                  : ORD == RWKVQ_ORDER_SB6 ? 16 : 8;
  const uint32_t h = __builtin_bit_cast(uint16_t, (_Float16)v);
  const uint32_t ph = __shfl_xor(h, m, 64);
  const int cg = c & 31;
  if ((cg & m) == 0) {
    const int pos = ORD == RWKVQ_ORDER_PAIRS ? cg
                                             : 2 * cg - (cg >= 16 ? 16 : 0);
    *reinterpret_cast<uint32_t*>(row + (c - cg) + pos) = h | (ph << 16);
  }
}

// LN + token shift + ncoef lerps for one token row (b, t):
//   out[(b*T+t), k, :] = xn + (shift - xn) * coef[k, :]
// shift = xn of (b, t-1), or prev[b] (zeros when prev is null) at t = 0.
// new_prev[b] = xn of (b, T-1).
// ORD < 0: fp32 out [N, NC, D]; ORD = RWKVQ_ORDER_*: fp16 out, each
// 32-column group in that pair order (the input of the GEMM that reads it).
template <int NC, int ORD>
__global__ void __launch_bounds__(kRowThreads)
shift_lerp_k(const float* __restrict__ x, const float* __restrict__ lw,
             const float* __restrict__ lb, const float* __restrict__ prev,
             const float* __restrict__ coef, void* __restrict__ out_,
             float* __restrict__ new_prev, int T, int D) {
  float* out = static_cast<float*>(out_);
  uint16_t* oh = static_cast<uint16_t*>(out_);
  __shared__ float sh[16];
  const int row = blockIdx.x;           // b * T + t
  const int t = row % T, bb = row / T;
  const float* xr = x + (size_t)row * D;
  float4 v[kMaxE4], pv[kMaxE4];
  load_row4(xr, D, v);
  if (t > 0) load_row4(xr - D, D, pv);
  else if (prev) load_row4(prev + (size_t)bb * D, D, pv);
  // every load is issued before the first store: on this target the
  // vector-memory counter covers stores too, so a load placed after a
  // store would also wait for that store
  float4 cw[kMaxE4], cb[kMaxE4], cf[NC][kMaxE4];
  load_row4(lw, D, cw);
  load_row4(lb, D, cb);
#pragma unroll
  for (int k = 0; k < NC; ++k) load_row4(coef + (size_t)k * D, D, cf[k]);
  float mean, rstd;
  row_stats4(v, D, 1e-5f, sh, mean, rstd);
  float pmean = 0.f, prstd = 0.f;
  if (t > 0) row_stats4(pv, D, 1e-5f, sh, pmean, prstd);
  auto lane4 = [&](const float4& f, int i) {
    return i == 0 ? f.x : i == 1 ? f.y : i == 2 ? f.z : f.w;
  };
#pragma unroll
  for (int e = 0; e < kMaxE4; ++e) {
    const int c = 4 * (threadIdx.x + e * kRowThreads);
    if (c >= D) continue;
    float xn[4], xx[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float w_ = lane4(cw[e], i), b_ = lane4(cb[e], i);
      xn[i] = (lane4(v[e], i) - mean) * rstd * w_ + b_;
      float sv;
      if (t > 0) sv = (lane4(pv[e], i) - pmean) * prstd * w_ + b_;
      else sv = prev ? lane4(pv[e], i) : 0.f;
      xx[i] = sv - xn[i];
    }
#pragma unroll
    for (int k = 0; k < NC; ++k) {
      float4 o;
      o.x = xn[0] + xx[0] * cf[k][e].x;
      o.y = xn[1] + xx[1] * cf[k][e].y;
      o.z = xn[2] + xx[2] * cf[k][e].z;
      o.w = xn[3] + xx[3] * cf[k][e].w;
      const size_t base = ((size_t)row * NC + k) * D;
      if constexpr (ORD < 0) {
        *reinterpret_cast<float4*>(out + base + c) = o;
      } else {
        store_pairs4<ORD>(oh + base, c, o);
      }
    }
    if (t == T - 1 && new_prev)
      *reinterpret_cast<float4*>(new_prev + (size_t)bb * D + c) =
          make_float4(xn[0], xn[1], xn[2], xn[3]);
  }
}

__device__ __forceinline__ float sigm(float v) { return 1.f / (1.f + __expf(-v)); }

// Per-channel WKV inputs.  One wave = one (token, head).
//   rkv [N, 3, D] (r, k, v);  yw, ya, yv, g [N, D] (LoRA outputs; yv may be
//   null on layer 0);  vfirst [N, D] written on layer 0, read otherwise.
//   outputs w, kp, vp, aa, bb [N, D]
__global__ void __launch_bounds__(256)
wkv_prep_k(const float* __restrict__ rkv, const float* __restrict__ yw,
           const float* __restrict__ ya, const float* __restrict__ yv,
           const float* __restrict__ w0, const float* __restrict__ a0,
           const float* __restrict__ v0, const float* __restrict__ k_k,
           const float* __restrict__ k_a, float* __restrict__ vfirst,
           int layer0, float* __restrict__ wo, float* __restrict__ kpo,
           float* __restrict__ vpo, float* __restrict__ aao,
           float* __restrict__ bbo, int D) {
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
// The per-step vectors r, w, k, a, b of the head (64 columns each) and v of
// the block's rows are staged through LDS in chunks of TC steps: the next
// chunk is fetched into registers while the current one is consumed, so
// the recurrence never waits on global memory.  The (S a) and (S r) row
// sums meet over the L lanes with DPP.
constexpr int kScanL = 16, kScanRB = 16, kScanTC = 32;
constexpr int kScanThreads = kScanL * kScanRB;                 // 256
constexpr int kVecF4 = kScanTC * 5 * (kHead / 4);              // float4 / chunk
constexpr int kVecPerThread = kVecF4 / kScanThreads;           // 10
constexpr int kVPerThread = kScanTC * kScanRB / kScanThreads;  // 2

__global__ void __launch_bounds__(kScanThreads)
wkv_scan_k(const float* __restrict__ r, long r_ld,
           const float* __restrict__ w, const float* __restrict__ k,
           const float* __restrict__ v, const float* __restrict__ aa,
           const float* __restrict__ bb, long ld, const float* state_in,
           float* state, float* __restrict__ y, long y_ld, int T, int H) {
  constexpr int L = kScanL, C = kHead / L, RB = kScanRB, TC = kScanTC;
  __shared__ float4 sv4[2][TC][5][kHead / 4];                   // 80 KiB
  __shared__ float svv[2][TC][RB];
  const int nblk = kHead / RB;
  const int bh = blockIdx.x / nblk, rb = blockIdx.x % nblk;
  const int bi = bh / H, h = bh % H;
  const int tid = threadIdx.x;
  const int part = tid % L;
  const int il = tid / L;
  const int i = rb * RB + il;                                  // value row
  const size_t soff = (((size_t)bi * H + h) * kHead + i) * kHead + part * C;
  float S[C];
  {
    float4 q = *reinterpret_cast<const float4*>(state_in + soff);
    S[0] = q.x; S[1] = q.y; S[2] = q.z; S[3] = q.w;
  }
  const float* base[5] = {r, w, k, aa, bb};
  const long lds[5] = {r_ld, ld, ld, ld, ld};
  const size_t col0 = (size_t)h * kHead;
  float4 stg[kVecPerThread];
  float stv[kVPerThread];

  auto fetch = [&](int t0) {
#pragma unroll
    for (int m = 0; m < kVecPerThread; ++m) {
      const int e = tid + m * kScanThreads;          // over [TC][5][16]
      const int f4 = e % (kHead / 4), q = (e / (kHead / 4)) % 5,
                tt = e / (5 * (kHead / 4));
      const int t = min(t0 + tt, T - 1);
      const size_t tok = (size_t)bi * T + t;
      stg[m] = *reinterpret_cast<const float4*>(base[q] + tok * lds[q] +
                                                col0 + 4 * f4);
    }
#pragma unroll
    for (int m = 0; m < kVPerThread; ++m) {
      const int e = tid + m * kScanThreads;          // over [TC][RB]
      const int rr = e % RB, tt = e / RB;
      const int t = min(t0 + tt, T - 1);
      stv[m] = v[((size_t)bi * T + t) * ld + col0 + rb * RB + rr];
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int m = 0; m < kVecPerThread; ++m) {
      const int e = tid + m * kScanThreads;
      const int f4 = e % (kHead / 4), q = (e / (kHead / 4)) % 5,
                tt = e / (5 * (kHead / 4));
      sv4[buf][tt][q][f4] = stg[m];
    }
#pragma unroll
    for (int m = 0; m < kVPerThread; ++m) {
      const int e = tid + m * kScanThreads;
      svv[buf][e / RB][e % RB] = stv[m];
    }
  };

  // one recurrence step from LDS slot (buf, tt); returns y = S_t r_t of the
  // row (all L lanes hold it after the reduction)
  auto step = [&](int bsel, int tt) {
    const float4 rv = sv4[bsel][tt][0][part], wv = sv4[bsel][tt][1][part],
                 kv = sv4[bsel][tt][2][part], av = sv4[bsel][tt][3][part],
                 bv = sv4[bsel][tt][4][part];
    const float vi = svv[bsel][tt][il];
    float sa = (S[0] * av.x + S[1] * av.y) + (S[2] * av.z + S[3] * av.w);
    sa += dpp_f<0xB1>(sa);      // quad_perm [1,0,3,2]
    sa += dpp_f<0x4E>(sa);      // quad_perm [2,3,0,1]
    sa += dpp_f<0x141>(sa);     // row_half_mirror
    sa += dpp_f<0x140>(sa);     // row_mirror
    S[0] = S[0] * wv.x + sa * bv.x + vi * kv.x;
    S[1] = S[1] * wv.y + sa * bv.y + vi * kv.y;
    S[2] = S[2] * wv.z + sa * bv.z + vi * kv.z;
    S[3] = S[3] * wv.w + sa * bv.w + vi * kv.w;
    float yp = (S[0] * rv.x + S[1] * rv.y) + (S[2] * rv.z + S[3] * rv.w);
    yp += dpp_f<0xB1>(yp);
    yp += dpp_f<0x4E>(yp);
    yp += dpp_f<0x141>(yp);
    yp += dpp_f<0x140>(yp);
    return yp;
  };

  fetch(0);
  stash(0);
  __syncthreads();
  int buf = 0;
  for (int t0 = 0; t0 < T; t0 += TC) {
    const bool more = t0 + TC < T;
    if (more) fetch(t0 + TC);                        // in flight meanwhile
    const int n = min(TC, T - t0);
    if (n == TC) {
      // full chunk, unrolled: the step's y reduction overlaps the next
      // step's (S a) reduction, and lane p keeps the y of steps p, p + L
      float ybuf[TC / L];
#pragma unroll
      for (int tt = 0; tt < TC; ++tt) {
        const float yp = step(buf, tt);
        ybuf[tt / L] = part == (tt % L) ? yp : ybuf[tt / L];
      }
#pragma unroll
      for (int j = 0; j < TC / L; ++j)
        y[((size_t)bi * T + t0 + j * L + part) * y_ld + col0 + i] = ybuf[j];
    } else {
      for (int tt = 0; tt < n; ++tt) {
        const float yp = step(buf, tt);
        if (part == 0) y[((size_t)bi * T + t0 + tt) * y_ld + col0 + i] = yp;
      }
    }
    if (more) {
      stash(buf ^ 1);
      __syncthreads();
      buf ^= 1;
    }
  }
  *reinterpret_cast<float4*>(state + soff) = make_float4(S[0], S[1], S[2],
                                                         S[3]);
}

// Group norm per head + bonus + gate.  One wave = one (token, head).
template <int ORD>   // < 0: fp32 out; else fp16 in pair order ORD
__global__ void __launch_bounds__(256)
wkv_tail_k(const float* __restrict__ y, const float* __restrict__ rkv,
           const float* __restrict__ kp, const float* __restrict__ vp,
           const float* __restrict__ g, const float* __restrict__ r_k,
           const float* __restrict__ lnw, const float* __restrict__ lnb,
           void* __restrict__ out, int D) {
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
  const float o = ((nrm * lnw[c] + lnb[c]) + dp * vp[e]) * g[e];
  if constexpr (ORD < 0)
    static_cast<float*>(out)[e] = o;
  else
    store_pairs1<ORD>(static_cast<uint16_t*>(out) + (size_t)n * D, c, o);
}

// Decode (T = 1) time-mix core for one (sequence, head) per block: the
// per-channel WKV inputs, one recurrence step and the group-norm / bonus /
// gate tail in one launch.  256 threads: thread (row i = tid / 4, part
// p = tid % 4) owns S[i][16 p .. 16 p + 16); wave 0 handles the per-channel
// work of the head's 64 channels.
// LoRA up products folded into the decode core: branch k (w, a, v, g) of
// token b is B_k [D, r_k] (fp16) times the down-projection output
// h_k[b, :r_k] (after its nonlinearity), for the head's 64 channels.
struct LoraUp {
  const float* h[4];
  const uint16_t* B[4];
  int r[4];
};
constexpr int kMaxCat = 1024;   // sum of the four ranks

// The up products straight from the file's codes.  A world checkpoint
// stores up factor k as [rank, D] with its quantization blocks along D, 64
// columns = one head: asym (u8 codes, fp32 scale / min per (rank row,
// head)) or per-row int8 (the g branch: fp16 scale per rank row).  At load
// the codes are permuted to [H][rank / 16][64][16] (head, 16-row block,
// channel, row within the block), so lane c of a wave reads the 16 codes
// of channel c for one row block with one 16-byte load (1 KiB contiguous
// per wave), and the asym parameters to [H][rank].  The file's codes,
// scales and mins enter exactly; h stays fp32 and the sum is taken in fp32
// as sum_j q_jc (h_j s_j) + sum_j h_j m_j (two VALU operations per weight:
// byte-to-float conversion and a multiply-add).
struct LoraUpQ {
  const float* h[4];
  const uint8_t* q[4];
  const float* s[4];       // asym scale [H][rank], null for int8
  const float* m[4];       // asym min [H][rank]
  const uint16_t* sc[4];   // int8: fp16 scale [rank]
  int r[4];
};

// LORA: 0 = branch outputs given (yw, ya, yv, g); 1 = up products from
// fp16 factors (lu); 2 = up products from the file's codes (lq).
template <int LORA>
__global__ void __launch_bounds__(256)
wkv_decode_k(const float* __restrict__ rkv, const float* __restrict__ yw,
             const float* __restrict__ ya, const float* __restrict__ yv,
             const float* __restrict__ g, const float* __restrict__ w0,
             const float* __restrict__ a0, const float* __restrict__ v0,
             const float* __restrict__ k_k, const float* __restrict__ k_a,
             const float* __restrict__ r_k, const float* __restrict__ lnw,
             const float* __restrict__ lnb, float* __restrict__ vfirst,
             int layer0, const float* state_in, float* state_out,
             float* __restrict__ out, int H, LoraUp lu, LoraUpQ lq) {
  constexpr int P = 4, C = kHead / P;
  __shared__ float4 s_w[kHead / 4], s_k[kHead / 4], s_a[kHead / 4],
      s_b[kHead / 4], s_r[kHead / 4];
  __shared__ float s_v[kHead], s_y[kHead];
  __shared__ float s_dp;
  const int bi = blockIdx.x / H, h = blockIdx.x % H;
  const int D = H * kHead;
  const int tid = threadIdx.x;
  const int i = tid / P, part = tid % P;
  // state row slice: issue the loads first, they do not depend on phase 1
  const size_t soff = (((size_t)bi * H + h) * kHead + i) * kHead + part * C;
  float S[C];
#pragma unroll
  for (int c = 0; c < C; c += 4) {
    float4 q = *reinterpret_cast<const float4*>(state_in + soff + c);
    S[c] = q.x; S[c + 1] = q.y; S[c + 2] = q.z; S[c + 3] = q.w;
  }
  // per-channel inputs of wave 0, also loaded up front: none depends on
  // the LoRA phase, so their round trip overlaps it
  float r = 0.f, k = 0.f, v = 0.f, w0c = 0.f, a0c = 0.f, kkc = 0.f,
        kac = 0.f, rkc = 0.f, lw = 0.f, lb = 0.f, vf = 0.f, ywe = 0.f,
        yae = 0.f, yve = 0.f, gc = 0.f, v0c = 0.f;
  if (tid < kHead) {
    const int c = h * kHead + tid;
    const size_t e = (size_t)bi * D + c;
    r = rkv[(size_t)bi * 3 * D + c];
    k = rkv[(size_t)bi * 3 * D + D + c];
    v = rkv[(size_t)bi * 3 * D + 2 * D + c];
    w0c = w0[c]; a0c = a0[c]; kkc = k_k[c]; kac = k_a[c]; rkc = r_k[c];
    lw = lnw[c]; lb = lnb[c];
    if (!layer0) {
      vf = vfirst[e]; v0c = v0[c];
      if (!LORA) yve = yv[e];
    }
    if (!LORA) { ywe = yw[e]; yae = ya[e]; gc = g[e]; }
  }
  __shared__ float s_up[4][kHead];
  if constexpr (LORA == 2) {
    // Branch k's output for channel c is
    //   sum_j h_j (q_jc s_j + m_j) = sum_j q_jc (h_j s_j) + sum_j h_j m_j,
    // the second term the same for every channel of the head.  int8 codes
    // are read as unsigned bytes of (q ^ 0x80) = q + 128, their -128 folded
    // into that term.  Staged per (token, head): hs_j = h_j s_j over the
    // concatenated rank axis (w, a, v, g; an absent branch has rank 0) and
    // the per-16-row-block sums of the channel-independent terms.
    __shared__ float4 s_hs4[kMaxCat / 4];
    __shared__ float s_cj[kMaxCat];
    __shared__ float s_bm[kMaxCat / 16];
    __shared__ float s_red[4][4][kHead];
    float* s_hs = reinterpret_cast<float*>(s_hs4);
    const int r0 = lq.r[0], r1 = lq.r[1], r2 = lq.r[2], r3 = lq.r[3];
    const int o1 = r0, o2 = o1 + r1, o3 = o2 + r2, R = o3 + r3;
    // each selection below indexes the argument table with constants (a
    // dynamic index would copy it to scratch)
    auto br = [&](int p) { return p < o1 ? 0 : p < o2 ? 1 : p < o3 ? 2 : 3; };
    auto off = [&](int k) { return k == 0 ? 0 : k == 1 ? o1 : k == 2 ? o2 : o3; };
    auto rk_of = [&](int k) { return k == 0 ? r0 : k == 1 ? r1 : k == 2 ? r2 : r3; };
    auto s_of = [&](int k) { return k == 0 ? lq.s[0] : k == 1 ? lq.s[1]
                                  : k == 2 ? lq.s[2] : lq.s[3]; };
    const int cl = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nb = R >> 4;
    // code blocks of this wave (blocks wv, wv + 4, ...), loads first
    uint4 cv[kMaxCat / 64];
#pragma unroll
    for (int i = 0; i < kMaxCat / 64; ++i) {
      const int b = wv + 4 * i;
      if (b < nb) {
        const int k = br(16 * b);
        const uint8_t* qk = k == 0 ? lq.q[0] : k == 1 ? lq.q[1]
                          : k == 2 ? lq.q[2] : lq.q[3];
        const int rk = rk_of(k), lb = (16 * b - off(k)) >> 4;
        cv[i] = ld16(qk + (((size_t)h * (rk >> 4) + lb) * kHead + cl) * 16);
      }
    }
    // h and the block parameters, branch by branch (pointers and formats
    // are then uniform), rank positions j = tid, tid + 256 (rank <= 512,
    // clamped into the branch for the loads); raw bits first, every load
    // in flight before the first use
    uint32_t hraw[4][2], sraw[4][2], mraw[4][2], craw[4][2];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int rk = lq.r[k];
      if (rk == 0) continue;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int j = min(tid + 256 * t, rk - 1);
        hraw[k][t] = __float_as_uint(lq.h[k][(size_t)bi * rk + j]);
        if (lq.s[k]) {
          sraw[k][t] = __float_as_uint(lq.s[k][(size_t)h * rk + j]);
          mraw[k][t] = __float_as_uint(lq.m[k][(size_t)h * rk + j]);
        } else {
          craw[k][t] = lq.sc[k][j];
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int rk = lq.r[k], o = k == 0 ? 0 : k == 1 ? o1 : k == 2 ? o2 : o3;
      if (rk == 0) continue;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int j = tid + 256 * t;
        if (j < rk) {
          pin(hraw[k][t]);
          const float hv = __uint_as_float(hraw[k][t]);
          if (lq.s[k]) {
            pin(sraw[k][t]);
            pin(mraw[k][t]);
            const float hs = hv * __uint_as_float(sraw[k][t]);
            s_hs[o + j] = hs;
            s_cj[o + j] = hv * __uint_as_float(mraw[k][t]);
          } else {
            pin(craw[k][t]);
            const float hs = hv * f16_bits_to_f32(craw[k][t]);
            s_hs[o + j] = hs;
            s_cj[o + j] = -128.f * hs;
          }
        }
      }
    }
    __syncthreads();
    if (tid < nb) {                            // fixed-order block sums
      float a = 0.f;
#pragma unroll
      for (int e = 0; e < 16; ++e) a += s_cj[16 * tid + e];
      s_bm[tid] = a;
    }
    __syncthreads();
    // each block's channel-independent sum joins the accumulator of the
    // wave that takes the block, so the four waves' partials add up to it
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < kMaxCat / 64; ++i) {
      const int b = wv + 4 * i;
      if (b < nb) {
        const int k = br(16 * b);
        const uint32_t flip = s_of(k) ? 0u : 0x80808080u;
        const uint32_t wd[4] = {cv[i].x ^ flip, cv[i].y ^ flip,
                                cv[i].z ^ flip, cv[i].w ^ flip};
        float d0 = 0.f, d1 = 0.f;
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
          const float4 hs = s_hs4[4 * b + qd];
          const uint32_t w = wd[qd];
          d0 = fmaf((float)(w & 0xFFu), hs.x, d0);
          d1 = fmaf((float)((w >> 8) & 0xFFu), hs.y, d1);
          d0 = fmaf((float)((w >> 16) & 0xFFu), hs.z, d0);
          d1 = fmaf((float)(w >> 24), hs.w, d1);
        }
        const float d = (d0 + d1) + s_bm[b];
        if (k == 0) acc[0] += d;
        else if (k == 1) acc[1] += d;
        else if (k == 2) acc[2] += d;
        else acc[3] += d;
      }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) s_red[wv][k][cl] = acc[k];
    __syncthreads();
    if (tid < kHead) {
#pragma unroll
      for (int k = 0; k < 4; ++k)
        s_up[k][tid] = (s_red[0][k][tid] + s_red[1][k][tid]) +
                       (s_red[2][k][tid] + s_red[3][k][tid]);
    }
  } else if constexpr (LORA == 1) {
    // The four branches' down outputs of token bi, concatenated (w, a, v,
    // g; an absent branch has rank 0) as fp16 pairs (the reference rounds
    // the low-rank activations to fp16 before the up product).
    __shared__ uint32_t s_hp[kMaxCat / 2];
    const uint16_t* B0 = lu.B[0];
    const uint16_t* B1 = lu.B[1];
    const uint16_t* B2 = lu.B[2];
    const uint16_t* B3 = lu.B[3];
    const int r0 = lu.r[0], r1 = lu.r[1], r2 = lu.r[2], r3 = lu.r[3];
    const int o1 = r0, o2 = o1 + r1, o3 = o2 + r2, R = o3 + r3;
    for (int p = tid; 2 * p < R; p += 256) {
      const int o = 2 * p;
      const float* hk = o < o1 ? lu.h[0] : o < o2 ? lu.h[1]
                      : o < o3 ? lu.h[2] : lu.h[3];
      const int rk = o < o1 ? r0 : o < o2 ? r1 : o < o3 ? r2 : r3;
      const int ok = o < o1 ? 0 : o < o2 ? o1 : o < o3 ? o2 : o3;
      const float* src = hk + (size_t)bi * rk + (o - ok);
      s_hp[p] = pack_h2(src[0], src[1]);
    }
    __syncthreads();
    // 4 lanes per channel; lane part j takes the 8-value chunks j, j+4, ...
    // of the concatenated rank axis, so every load of the row is issued
    // before the first product (one memory round trip)
    const int ch = h * kHead + (tid >> 2), j = tid & 3;
    const int nc = R / 8;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    uint4 wv[kMaxCat / 32];
#pragma unroll
    for (int i = 0; i < kMaxCat / 32; ++i) {
      const int q = j + 4 * i;
      if (q < nc) {
        const int o = 8 * q;
        const uint16_t* Bk = o < o1 ? B0 : o < o2 ? B1 : o < o3 ? B2 : B3;
        const int rk = o < o1 ? r0 : o < o2 ? r1 : o < o3 ? r2 : r3;
        const int ok = o < o1 ? 0 : o < o2 ? o1 : o < o3 ? o2 : o3;
        wv[i] = ld16(Bk + (size_t)ch * rk + (o - ok));
      }
    }
#pragma unroll
    for (int i = 0; i < kMaxCat / 32; ++i) {
      const int q = j + 4 * i;
      if (q < nc) {
        const int o = 8 * q;
        float d = dot2(wv[i].x, s_hp[4 * q], 0.f);
        d = dot2(wv[i].y, s_hp[4 * q + 1], d);
        d = dot2(wv[i].z, s_hp[4 * q + 2], d);
        d = dot2(wv[i].w, s_hp[4 * q + 3], d);
        if (o < o1) acc[0] += d;
        else if (o < o2) acc[1] += d;
        else if (o < o3) acc[2] += d;
        else acc[3] += d;
      }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      acc[k] += dpp_f<0xB1>(acc[k]);       // quad_perm [1,0,3,2]
      acc[k] += dpp_f<0x4E>(acc[k]);       // quad_perm [2,3,0,1]
    }
    // lane part j stores branch j of its channel
    s_up[j][tid >> 2] = j == 0 ? acc[0] : j == 1 ? acc[1]
                      : j == 2 ? acc[2] : acc[3];
    __syncthreads();
  }
  float vp = 0.f;
  if (tid < kHead) {
    const int c = h * kHead + tid;
    const size_t e = (size_t)bi * D + c;
    if (LORA) {
      ywe = s_up[0][tid]; yae = s_up[1][tid]; yve = s_up[2][tid];
      gc = s_up[3][tid];
    }
    const float wv = __expf(-0.606531f * sigm(ywe + w0c));
    const float av = sigm(yae + a0c);
    const float kkr = k * kkc;
    const float kk = kkr / sqrtf(wave_sum_dpp(kkr * kkr) + 1e-12f);
    const float kp = k * (1.f + (av - 1.f) * kac);
    if (!layer0)
      v = v + (vf - v) * sigm(yve + v0c);
    else vfirst[e] = v;
    const float dp = wave_sum_dpp(r * kp * rkc);
    reinterpret_cast<float*>(s_w)[tid] = wv;
    reinterpret_cast<float*>(s_k)[tid] = kp;
    reinterpret_cast<float*>(s_a)[tid] = -kk;
    reinterpret_cast<float*>(s_b)[tid] = kk * av;
    reinterpret_cast<float*>(s_r)[tid] = r;
    s_v[tid] = v;
    if (tid == 0) s_dp = dp;
    vp = v;
  }
  __syncthreads();
  const float vi = s_v[i];
  float sa = 0.f;
#pragma unroll
  for (int c = 0; c < C; c += 4) {
    const float4 a4 = s_a[part * (C / 4) + c / 4];
    sa += S[c] * a4.x + S[c + 1] * a4.y + S[c + 2] * a4.z + S[c + 3] * a4.w;
  }
  sa += dpp_f<0xB1>(sa);
  sa += dpp_f<0x4E>(sa);
  float yv2 = 0.f;
#pragma unroll
  for (int c = 0; c < C; c += 4) {
    const int q = part * (C / 4) + c / 4;
    const float4 w4 = s_w[q], b4 = s_b[q], k4 = s_k[q], r4 = s_r[q];
    S[c] = S[c] * w4.x + sa * b4.x + vi * k4.x;
    S[c + 1] = S[c + 1] * w4.y + sa * b4.y + vi * k4.y;
    S[c + 2] = S[c + 2] * w4.z + sa * b4.z + vi * k4.z;
    S[c + 3] = S[c + 3] * w4.w + sa * b4.w + vi * k4.w;
    yv2 += S[c] * r4.x + S[c + 1] * r4.y + S[c + 2] * r4.z + S[c + 3] * r4.w;
  }
  yv2 += dpp_f<0xB1>(yv2);
  yv2 += dpp_f<0x4E>(yv2);
#pragma unroll
  for (int c = 0; c < C; c += 4)
    *reinterpret_cast<float4*>(state_out + soff + c) =
        make_float4(S[c], S[c + 1], S[c + 2], S[c + 3]);
  if (part == 0) s_y[i] = yv2;
  __syncthreads();
  if (tid < kHead) {
    const float yy = s_y[tid];
    const float mean = wave_sum_dpp(yy) * (1.f / kHead);
    const float dv = yy - mean;
    const float var = wave_sum_dpp(dv * dv) * (1.f / kHead);
    const float nrm = dv / sqrtf(var + 64e-5f);
    out[(size_t)bi * D + h * kHead + tid] =
        ((nrm * lw + lb) + s_dp * vp) * gc;
  }
}

// ---------------------------------------------------------------------------
// Chunked WKV-7 scan (prefill).  Per (sequence, head) the recurrence over a
// chunk of L = 16 steps, s_t = s_{t-1} diag(w_t) + (s_{t-1}.a_t) b_t +
// v_t k_t for every value row s (a vector over the key index), is linear in
// the chunk's start state S0 and in its values V:
//   S_end = S0 P + V^T Bq,   Y = S0 Ry + V^T Yq      (Y[i][t] = y_t[i])
// With G[t] the cumulative log decay over the chunk (G[0] = 0), u_t =
// s_{t-1}.a_t solves a unit triangular system, U (I - M^T) = S0 C + V N^T:
//   C[k][t]  = e^{G[t]} a_t                  M[t][j] = b_j.(e^{G[t]-G[j+1]} a_t)
//   N[t][j]  = k_j.(e^{G[t]-G[j+1]} a_t)     (j < t; W = (I - M^T)^-1)
//   Bt[j][t] = b_j.(e^{G[t+1]-G[j+1]} r_t)   Kt[j][t] = k_j.(...r_t)   (j <= t)
//   Bh[j]    = b_j e^{G[L]-G[j+1]}           Kh[j]    = k_j e^{G[L]-G[j+1]}
//   P  = diag(e^{G[L]}) + C W Bh   Bq = N^T W Bh + Kh
//   Ry = e^{G[t+1]} r_t + C W Bt   Yq = N^T W Bt + Kt
// (the WY form of a product of diagonal-plus-rank-one transitions).  One
// launch builds these operators for every chunk in parallel; a second walks
// the chunks in order per 16 value rows: two 64-deep products per chunk on
// the fp32 matrix cores instead of 16 dependent scalar steps.  A ragged last
// chunk is padded with identity steps (w = 1, k = a = b = r = v = 0).
constexpr int kCL = 16;                 // steps per chunk
constexpr int kOpsFloats = 6400;        // operator floats per (b, h, chunk)
constexpr int kPad = 68;                // LDS row stride (floats)

typedef float f32x4c_t __attribute__((ext_vector_type(4)));

// One 16x16x4 fp32 matrix-core step: D = A B + C, lane l holding A[l%16][l/16],
// B[l/16][l%16] and D[4 (l/16) + v][l%16].
__device__ __forceinline__ f32x4c_t mfma4(float a, float b, f32x4c_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Operator block of one chunk, in the register order the scan kernel's
// fp32 MFMAs use.  Lane l = 16 g + m of wave w; the scan's key steps run
// in the order k(s, g) = 16 (s / 4) + 4 g + s % 4, its value steps in the
// order j(s, g) = 4 g + s:
//   [0, 4096)     Pf [w][l][s] = P[k(s, g)][16 w + m]           s < 16
//   [4096, 5120)  Bqf[w][l][s] = Bq[4 g + s][16 w + m]          s < 4
//   [5120, 6144)  Ryf[w][l][s] = Ry[16 w + 4 g + s][m]          s < 4
//   [6144, 6400)  Yqf[l][s]    = Yq[4 g + s][m]                 s < 4
// -- exactly the accumulator registers of the MFMAs that produce them.
// Inputs of the prep step folded into the chunk-operator kernel (prefill:
// rkvq_wkv7_prefill_chunked); unused by the plain chunked scan.
struct PrepIn {
  const float* rkv;          // [N, 3, D] r, k, v
  const float* yw;
  const float* ya;
  const float* yv;           // null on layer 0
  const float* w0;
  const float* a0;
  const float* v0;
  const float* k_k;
  const float* k_a;
  float* vfirst;             // written on layer 0, read otherwise
  int layer0;
  float* kp;                 // out: k' [N, D]
  float* vp;                 // out: v' [N, D]
  int D;
};

template <bool PREP>
__global__ void __launch_bounds__(256)
wkv_chunk_ops_k(const float* __restrict__ r, long r_ld,
                const float* __restrict__ w, const float* __restrict__ k,
                const float* __restrict__ a, const float* __restrict__ b,
                long ld, float* __restrict__ ops, int T, int H, int NC,
                PrepIn pi) {
  const int c = blockIdx.x % NC, bh = blockIdx.x / NC;
  const int h = bh % H, bi = bh / H;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, lg = lane >> 4;
  constexpr int kQ = 20;
  // [step][key channel] rows (stride 68); 16 x 16 matrices (stride 20)
  __shared__ float sEw[kCL][kPad], sK[kCL][kPad], sA[kCL][kPad],
      sB[kCL][kPad], sR[kCL][kPad], sG[kCL + 1][kPad];
  __shared__ float sYa[kCL][kPad], sYr[kCL][kPad], sXb[kCL][kPad],
      sXk[kCL][kPad], sBh[kCL][kPad], sKh[kCL][kPad];
  __shared__ float sM[kCL][kQ], sN[kCL][kQ], sBt[kCL][kQ], sKt[kCL][kQ],
      sW[kCL][kQ], sNW[kCL][kQ], sCW[kHead][kQ];

  // 1. the chunk's inputs (identity steps past T); log decay floored at
  //    -60 so that a decay of exactly 0 stays finite
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int idx = tid + 256 * e, t = idx >> 6, kap = idx & 63;
    const int tg = c * kCL + t;
    float wvl = 1.f, kv = 0.f, av = 0.f, bv = 0.f, rv = 0.f;
    if (tg < T) {                       // (uniform: a wave is one step t)
      const size_t row = (size_t)bi * T + tg, col = (size_t)h * kHead + kap;
      if constexpr (PREP) {
        // the per-channel inputs from r/k/v and the LoRA outputs, as
        // wkv_prep_k; k' and v' also go out for the scan and the tail
        const size_t e = row * pi.D + col;
        const float kr = pi.rkv[(row * 3 + 1) * pi.D + col];
        float vr = pi.rkv[(row * 3 + 2) * pi.D + col];
        rv = pi.rkv[row * 3 * pi.D + col];
        wvl = __expf(-0.606531f * sigm(pi.yw[e] + pi.w0[col]));
        const float aw = sigm(pi.ya[e] + pi.a0[col]);
        const float kkr = kr * pi.k_k[col];
        const float ss = wave_sum_dpp(kkr * kkr);
        const float kk = kkr / sqrtf(ss + 1e-12f);
        kv = kr * (1.f + (aw - 1.f) * pi.k_a[col]);
        av = -kk;
        bv = kk * aw;
        if (pi.layer0) {
          pi.vfirst[e] = vr;
        } else {
          const float vf = pi.vfirst[e];
          vr = vr + (vf - vr) * sigm(pi.yv[e] + pi.v0[col]);
        }
        pi.kp[e] = kv;
        pi.vp[e] = vr;
      } else {
        wvl = w[row * ld + col]; kv = k[row * ld + col];
        av = a[row * ld + col]; bv = b[row * ld + col];
        rv = r[row * r_ld + col];
      }
    }
    const float lw = fmaxf(logf(wvl), -60.f);
    sG[t + 1][kap] = lw;                 // summed in place below
    sEw[t][kap] = __expf(lw);
    sK[t][kap] = kv; sA[t][kap] = av; sB[t][kap] = bv; sR[t][kap] = rv;
  }
  __syncthreads();
  // 2. cumulative log decay per key channel; the factored products below
  //    need e^{-G} finite (G[16] >= -80 on every channel)
  bool ok = true;
  if (tid < kHead) {
    float g = 0.f;
    sG[0][tid] = 0.f;
#pragma unroll
    for (int t = 0; t < kCL; ++t) {
      g += sG[t + 1][tid];
      sG[t + 1][tid] = g;
    }
    ok = g >= -80.f;
  }
  const bool factored = __syncthreads_and(ok);
  // 3. decayed rows: Ya[t] = a_t e^{G[t]}, Yr[t] = r_t e^{G[t+1]} (<= 1),
  //    Xb[j] = b_j e^{-G[j+1]}, Xk[j] = k_j e^{-G[j+1]}, Bh, Kh
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int idx = tid + 256 * e, t = idx >> 6, kap = idx & 63;
    const float g0 = sG[t][kap], g1 = sG[t + 1][kap], gl = sG[kCL][kap];
    sYa[t][kap] = sA[t][kap] * __expf(g0);
    sYr[t][kap] = sR[t][kap] * __expf(g1);
    const float inv = factored ? __expf(-g1) : 0.f;
    sXb[t][kap] = sB[t][kap] * inv;
    sXk[t][kap] = sK[t][kap] * inv;
    const float d = __expf(gl - g1);
    sBh[t][kap] = sB[t][kap] * d;
    sKh[t][kap] = sK[t][kap] * d;
  }
  __syncthreads();
  // 4. M[t][j] = Ya[t].Xb[j] (j < t), N[t][j] = Ya[t].Xk[j] (j < t),
  //    Bt[j][t] = Xb[j].Yr[t], Kt[j][t] = Xk[j].Yr[t] (j <= t): one 16 x 16
  //    x 64 product per wave; exact pairwise decays when e^{-G} would not
  //    be finite
  if (factored) {
    const float(*pA)[kPad] = wv < 2 ? sYa : wv == 2 ? sXb : sXk;
    const float(*pB)[kPad] = wv == 0 ? sXb : wv == 1 ? sXk : sYr;
    f32x4c_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s2 = 0; s2 < 16; ++s2)
      acc = mfma4(pA[li][4 * s2 + lg], pB[li][4 * s2 + lg], acc);
    float(*dst)[kQ] = wv == 0 ? sM : wv == 1 ? sN : wv == 2 ? sBt : sKt;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int row = 4 * lg + q, col = li;   // (t, j) for M, N; (j, t) else
      const bool keep = wv < 2 ? col < row : row <= col;
      dst[row][col] = keep ? acc[q] : 0.f;
    }
  } else {
    const int t = tid >> 4, j = tid & 15;
    float m = 0.f, n = 0.f, bt = 0.f, kt = 0.f;
    const bool lt = j < t, eq = j == t;
    for (int kap = 0; kap < kHead; ++kap) {
      const float d = lt ? __expf(sG[t][kap] - sG[j + 1][kap]) : 0.f;
      const float e1 = d * sA[t][kap];
      const float e2 = (lt ? d * sEw[t][kap] : (eq ? 1.f : 0.f)) * sR[t][kap];
      m += sB[j][kap] * e1; n += sK[j][kap] * e1;
      bt += sB[j][kap] * e2; kt += sK[j][kap] * e2;
    }
    sM[t][j] = m; sN[t][j] = n; sBt[j][t] = bt; sKt[j][t] = kt;
  }
  __syncthreads();
  // 5. W = (I - M^T)^-1 (unit upper triangular), one column per lane:
  //    W[i][cc] = sum_{m > i} M[m][i] W[m][cc], W[cc][cc] = 1
  if (tid < kCL) {
    const int cc = tid;
    float col[kCL];
#pragma unroll
    for (int i = kCL - 1; i >= 0; --i) {
      float sum = 0.f;
#pragma unroll
      for (int m2 = i + 1; m2 < kCL; ++m2) sum += sM[m2][i] * col[m2];
      col[i] = i == cc ? 1.f : (i > cc ? 0.f : sum);
    }
#pragma unroll
    for (int i = 0; i < kCL; ++i) sW[i][cc] = col[i];
  }
  __syncthreads();
  // 6. CW = Ya^T W (wave w: key channels 16w..16w+15), NW = N^T W (wave 0)
  {
    f32x4c_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s2 = 0; s2 < 4; ++s2)
      acc = mfma4(sYa[4 * s2 + lg][16 * wv + li], sW[4 * s2 + lg][li], acc);
#pragma unroll
    for (int q = 0; q < 4; ++q) sCW[16 * wv + 4 * lg + q][li] = acc[q];
    if (wv == 1) {
      f32x4c_t an = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s2 = 0; s2 < 4; ++s2)
        an = mfma4(sN[4 * s2 + lg][li], sW[4 * s2 + lg][li], an);
#pragma unroll
      for (int q = 0; q < 4; ++q) sNW[4 * lg + q][li] = an[q];
    }
  }
  __syncthreads();
  // 7. the operators, accumulated straight into the scan kernel's order
  float* o = ops + ((size_t)bh * NC + c) * kOpsFloats;
  {
    const int mu = 16 * wv + li;
    float pv[16];
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
      f32x4c_t acc;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int kap = 16 * ti + 4 * lg + q;
        acc[q] = kap == mu ? __expf(sG[kCL][kap]) : 0.f;
      }
#pragma unroll
      for (int s2 = 0; s2 < 4; ++s2)
        acc = mfma4(sCW[16 * ti + li][4 * s2 + lg], sBh[4 * s2 + lg][mu], acc);
#pragma unroll
      for (int q = 0; q < 4; ++q) pv[4 * ti + q] = acc[q];
    }
    float4* p4 = reinterpret_cast<float4*>(o + (wv * 64 + lane) * 16);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      p4[q] = make_float4(pv[4 * q], pv[4 * q + 1], pv[4 * q + 2], pv[4 * q + 3]);
    // Bq = Kh + NW Bh (columns 16w..), Ry = Yr^T + CW Bt (rows 16w..)
    f32x4c_t aq, ar;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      aq[q] = sKh[4 * lg + q][mu];
      ar[q] = sYr[li][16 * wv + 4 * lg + q];
    }
#pragma unroll
    for (int s2 = 0; s2 < 4; ++s2) {
      aq = mfma4(sNW[li][4 * s2 + lg], sBh[4 * s2 + lg][mu], aq);
      ar = mfma4(sCW[16 * wv + li][4 * s2 + lg], sBt[4 * s2 + lg][li], ar);
    }
    *reinterpret_cast<float4*>(o + 4096 + (wv * 64 + lane) * 4) =
        make_float4(aq[0], aq[1], aq[2], aq[3]);
    *reinterpret_cast<float4*>(o + 5120 + (wv * 64 + lane) * 4) =
        make_float4(ar[0], ar[1], ar[2], ar[3]);
    if (wv == 0) {     // Yq = Kt + NW Bt
      f32x4c_t ay;
#pragma unroll
      for (int q = 0; q < 4; ++q) ay[q] = sKt[4 * lg + q][li];
#pragma unroll
      for (int s2 = 0; s2 < 4; ++s2)
        ay = mfma4(sNW[li][4 * s2 + lg], sBt[4 * s2 + lg][li], ay);
      *reinterpret_cast<float4*>(o + 6144 + lane * 4) =
          make_float4(ay[0], ay[1], ay[2], ay[3]);
    }
  }
}

// The sequential part: block = 16 value rows of one (sequence, head), 4
// waves; per chunk wave w computes columns 16w..16w+15 of S0 P + V^T Bq and
// key channels 16w..16w+15 of S0 Ry (wave 0 adds V^T Yq); the new rows and
// the partial outputs meet in LDS (double-buffered: one barrier per chunk).
// Each chunk's operators and values are loaded three chunks ahead, into
// three register sets used in turn (compile-time indices, no copies).
struct ChunkOps {
  float4 pf[4];
  float4 bq, ry, yq;
  float vv[4];
};

__global__ void __launch_bounds__(256)
wkv_chunk_scan_k(const float* __restrict__ v, long ld,
                 const float* __restrict__ ops, const float* state_in,
                 float* state_out, float* __restrict__ y, long y_ld, int T,
                 int H, int NC) {
  const int rb = blockIdx.x & 3, bh = blockIdx.x >> 2;
  const int h = bh % H, bi = bh / H;
  const int row0 = rb * 16;
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int li = lane & 15, lg = lane >> 4;
  __shared__ __attribute__((aligned(16))) float sS[2][16][kPad];   // [buf][row][key]
  __shared__ float sY[2][4][4][64];                              // [buf][wave][q][lane]

  // A fragments of the rows in the operators' key order:
  // aS[4 ti + q] = S[row0 + li][16 ti + 4 lg + q]
  float aS[16];
  {
    const float* st = state_in + ((size_t)bh * kHead + row0 + li) * kHead;
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
      const float4 f = *reinterpret_cast<const float4*>(st + 16 * ti + 4 * lg);
      aS[4 * ti] = f.x; aS[4 * ti + 1] = f.y; aS[4 * ti + 2] = f.z; aS[4 * ti + 3] = f.w;
    }
  }
  const float* opsb = ops + (size_t)bh * NC * kOpsFloats;
  auto load_ops = [&](int c, ChunkOps& co) {
    c = min(c, NC - 1);                      // past the end: reloads, unused
    const float* o = opsb + (size_t)c * kOpsFloats;
    const float4* p4 = reinterpret_cast<const float4*>(o + (wv * 64 + lane) * 16);
#pragma unroll
    for (int q = 0; q < 4; ++q) co.pf[q] = p4[q];
    co.bq = *reinterpret_cast<const float4*>(o + 4096 + (wv * 64 + lane) * 4);
    co.ry = *reinterpret_cast<const float4*>(o + 5120 + (wv * 64 + lane) * 4);
    co.yq = *reinterpret_cast<const float4*>(o + 6144 + lane * 4);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      // unconditional load of a clamped step, kept as loaded (zeroed past
      // T where it is used): the compiler's load counting stays exact and
      // nothing waits for the load before its chunk
      const int tg = c * kCL + 4 * lg + s;
      co.vv[s] =
          v[((size_t)bi * T + min(tg, T - 1)) * ld + (size_t)h * kHead + row0 + li];
    }
  };
  auto chunk = [&](int c, const ChunkOps& co) {
    const int p = c & 1;
    const float pfs[16] = {co.pf[0].x, co.pf[0].y, co.pf[0].z, co.pf[0].w,
                           co.pf[1].x, co.pf[1].y, co.pf[1].z, co.pf[1].w,
                           co.pf[2].x, co.pf[2].y, co.pf[2].z, co.pf[2].w,
                           co.pf[3].x, co.pf[3].y, co.pf[3].z, co.pf[3].w};
    const float bqs[4] = {co.bq.x, co.bq.y, co.bq.z, co.bq.w};
    const float rys[4] = {co.ry.x, co.ry.y, co.ry.z, co.ry.w};
    const float yqs[4] = {co.yq.x, co.yq.y, co.yq.z, co.yq.w};
    float vvs[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) vvs[s] = c * kCL + 4 * lg + s < T ? co.vv[s] : 0.f;
    // two accumulators halve the dependent chain
    f32x4c_t accS = {0.f, 0.f, 0.f, 0.f}, accS2 = {0.f, 0.f, 0.f, 0.f};
    f32x4c_t accY = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 16; s += 2) {
      accS = mfma4(aS[s], pfs[s], accS);
      accS2 = mfma4(aS[s + 1], pfs[s + 1], accS2);
    }
#pragma unroll
    for (int s = 0; s < 4; s += 2) {
      accS = mfma4(vvs[s], bqs[s], accS);
      accS2 = mfma4(vvs[s + 1], bqs[s + 1], accS2);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const float av = wv == 0 ? aS[s] : wv == 1 ? aS[4 + s]
                     : wv == 2 ? aS[8 + s] : aS[12 + s];
      accY = mfma4(av, rys[s], accY);
    }
    if (wv == 0) {
#pragma unroll
      for (int s = 0; s < 4; ++s) accY = mfma4(vvs[s], yqs[s], accY);
    }
    // lane holds new S[4 lg + q][16 wv + li] and partial Y[4 lg + q][li]
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      sS[p][4 * lg + q][16 * wv + li] = accS[q] + accS2[q];
      sY[p][wv][q][lane] = accY[q];
    }
    __syncthreads();
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
      const float4 f = *reinterpret_cast<const float4*>(&sS[p][li][16 * ti + 4 * lg]);
      aS[4 * ti] = f.x; aS[4 * ti + 1] = f.y; aS[4 * ti + 2] = f.z; aS[4 * ti + 3] = f.w;
    }
    // output element (row i, step t) of this chunk: C layout lane
    // t + 16 (i / 4), register i % 4
    const int i = threadIdx.x & 15, t = threadIdx.x >> 4;
    const int tg = c * kCL + t;
    const int src = t + 16 * (i >> 2), q = i & 3;
    const float yv = (sY[p][0][q][src] + sY[p][1][q][src]) +
                     (sY[p][2][q][src] + sY[p][3][q][src]);
    if (tg < T)
      y[((size_t)bi * T + tg) * y_ld + (size_t)h * kHead + row0 + i] = yv;
  };
  // NC is a multiple of 3 (identity chunks pad the sequence), so the
  // loop body has no branches and each wait covers only its own set
  ChunkOps o0, o1, o2;
  load_ops(0, o0);
  load_ops(1, o1);
  load_ops(2, o2);
  for (int c = 0; c < NC; c += 3) {
    chunk(c, o0);
    load_ops(c + 3, o0);
    chunk(c + 1, o1);
    load_ops(c + 4, o1);
    chunk(c + 2, o2);
    load_ops(c + 5, o2);
  }
  // final rows, from the last chunk's buffer
  const int pl = (NC - 1) & 1;
  float* so = state_out + ((size_t)bh * kHead + row0) * kHead;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int idx = threadIdx.x + 256 * e, rr = idx >> 6, kk = idx & 63;
    so[(size_t)rr * kHead + kk] = sS[pl][rr][kk];
  }
}

inline int ok_launch() {
  return hipGetLastError() == hipSuccess ? RWKVQ_OK : RWKVQ_ERR_LAUNCH;
}

}  // namespace

namespace {

template <int NC>
void launch_lerp_f16(int order, int rows, hipStream_t s, const float* x,
                     const float* lw, const float* lb, const float* prev,
                     const float* coef, uint16_t* out, float* new_prev, int T,
                     int D) {
  if (order == RWKVQ_ORDER_PAIRS)
    hipLaunchKernelGGL((shift_lerp_k<NC, RWKVQ_ORDER_PAIRS>), dim3(rows),
                       dim3(kRowThreads), 0, s, x, lw, lb, prev, coef, out,
                       new_prev, T, D);
  else if (order == RWKVQ_ORDER_SB6)
    hipLaunchKernelGGL((shift_lerp_k<NC, RWKVQ_ORDER_SB6>), dim3(rows),
                       dim3(kRowThreads), 0, s, x, lw, lb, prev, coef, out,
                       new_prev, T, D);
  else
    hipLaunchKernelGGL((shift_lerp_k<NC, RWKVQ_ORDER_SYM6>), dim3(rows),
                       dim3(kRowThreads), 0, s, x, lw, lb, prev, coef, out,
                       new_prev, T, D);
}

}  // namespace

// Chunk-operator scratch of rwkvq_wkv7_scan_chunked_noalloc: a module-
// global device array (one copy per GPU, alive until the process ends), so
// that entry point allocates nothing.  Host code never passes `scratch`
// itself to a kernel (on the host it names a stand-in, not a device
// address): scratch_base() resolves the current device's copy with
// hipGetSymbolAddress once per device and every launch uses that pointer.
constexpr long kScratchFloats = 16L << 20;      // 64 MiB
static __device__ __align__(256) float scratch[kScratchFloats];

namespace {
float* g_scratch_base[64];
std::once_flag g_scratch_once[64];

int scratch_base(float** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
    return RWKVQ_ERR_LAUNCH;
  std::call_once(g_scratch_once[dev], [dev] {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) == hipSuccess)
      g_scratch_base[dev] = static_cast<float*>(p);
  });
  if (!g_scratch_base[dev]) return RWKVQ_ERR_LAUNCH;
  *out = g_scratch_base[dev];
  return RWKVQ_OK;
}
}  // namespace

extern "C" {

int rwkvq_layer_norm(const float* x, const float* w, const float* b, float* y,
                     int rows, int D, float eps, void* stream) {
  if (rows <= 0 || D <= 0 || D > kRowThreads * kMaxE) return RWKVQ_ERR_ARG;
  hipLaunchKernelGGL(layer_norm_k, dim3(rows), dim3(256), 0,
                     (hipStream_t)stream, x, w, b, y, D, eps);
  return ok_launch();
}

int rwkvq_gather_ln_f32(int kind, int bits, const uint8_t* q,
                        const uint32_t* hb, const void* aux0,
                        const uint16_t* aux1, int src_rows, int in,
                        const int64_t* idx, int n_idx, const float* w,
                        const float* b, float eps, float* out,
                        void* stream) {
  if (n_idx <= 0 || src_rows <= 0 || in <= 0 || !idx || !w || !b || !out ||
      in > kRowThreads * kMaxE || in % 8)
    return RWKVQ_ERR_ARG;
  hipStream_t s = (hipStream_t)stream;
  if (kind == 0) {            // sb6: aux0 = rec
    if (in % 256 || bits < 4 || bits > 6 || (bits > 4 && !hb) || !aux0)
      return RWKVQ_ERR_ARG;
    hipLaunchKernelGGL(gather_ln_k<0>, dim3(n_idx), dim3(kRowThreads), 0, s,
                       q, hb, aux0, aux1, bits, src_rows, in, idx, w, b, out,
                       eps);
  } else if (kind == 1) {     // sym: aux0 = qs, aux1 = d
    if (in % 256 || (bits != 6 && bits != 8) || (bits == 6 && !hb) ||
        !aux0 || !aux1)
      return RWKVQ_ERR_ARG;
    hipLaunchKernelGGL(gather_ln_k<1>, dim3(n_idx), dim3(kRowThreads), 0, s,
                       q, hb, aux0, aux1, bits, src_rows, in, idx, w, b, out,
                       eps);
  } else if (kind == 2) {     // rtn@8: aux1 = scale
    if (!aux1) return RWKVQ_ERR_ARG;
    hipLaunchKernelGGL(gather_ln_k<2>, dim3(n_idx), dim3(kRowThreads), 0, s,
                       q, hb, aux0, aux1, 8, src_rows, in, idx, w, b, out,
                       eps);
  } else {
    return RWKVQ_ERR_ARG;
  }
  return ok_launch();
}

int rwkvq_shift_lerp(const float* x, const float* ln_w, const float* ln_b,
                     const float* prev, const float* coef, int ncoef,
                     float* out, float* new_prev, int B, int T, int D,
                     void* stream) {
  if (B <= 0 || T <= 0 || D <= 0 || D > 4 * kRowThreads * kMaxE4 ||
      D % 4 || (ncoef != 1 && ncoef != 6))
    return RWKVQ_ERR_ARG;
  if (ncoef == 6)
    hipLaunchKernelGGL((shift_lerp_k<6, -1>), dim3(B * T), dim3(kRowThreads),
                       0, (hipStream_t)stream, x, ln_w, ln_b, prev, coef, out,
                       new_prev, T, D);
  else
    hipLaunchKernelGGL((shift_lerp_k<1, -1>), dim3(B * T), dim3(kRowThreads),
                       0, (hipStream_t)stream, x, ln_w, ln_b, prev, coef, out,
                       new_prev, T, D);
  return ok_launch();
}

int rwkvq_shift_lerp_f16(const float* x, const float* ln_w, const float* ln_b,
                         const float* prev, const float* coef, int ncoef,
                         uint16_t* out, int order, float* new_prev, int B,
                         int T, int D, void* stream) {
  if (B <= 0 || T <= 0 || D <= 0 || D > 4 * kRowThreads * kMaxE4 ||
      D % 32 || (ncoef != 1 && ncoef != 6) || order < 0 ||
      order > RWKVQ_ORDER_SYM6 || reinterpret_cast<uintptr_t>(out) % 16)
    return RWKVQ_ERR_ARG;
  hipStream_t s = (hipStream_t)stream;
  if (ncoef == 6)
    launch_lerp_f16<6>(order, B * T, s, x, ln_w, ln_b, prev, coef, out,
                       new_prev, T, D);
  else
    launch_lerp_f16<1>(order, B * T, s, x, ln_w, ln_b, prev, coef, out,
                       new_prev, T, D);
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
  hipLaunchKernelGGL(wkv_scan_k, dim3(B * H * (kHead / kScanRB)),
                     dim3(kScanThreads), 0, (hipStream_t)stream, r, r_ld, w,
                     k, v, a, b, ld, state_in ? state_in : state_out,
                     state_out, y, y_ld, T, H);
  return ok_launch();
}

int rwkvq_wkv7_scan_chunked(const float* r, long r_ld, const float* w,
                            const float* k, const float* v, const float* a,
                            const float* b, long ld, const float* state_in,
                            float* state_out, float* y, long y_ld, int B,
                            int T, int H, int head_size, float* ws,
                            long ws_floats, void* stream) {
  if (B <= 0 || T <= 0 || H <= 0 || head_size != kHead || ld < H * kHead ||
      r_ld < H * kHead || y_ld < H * kHead || !ws || !state_out)
    return RWKVQ_ERR_ARG;
  // chunks padded to a multiple of 3 with identity steps (the sequential
  // kernel walks them three at a time)
  const int NC = ((T + kCL - 1) / kCL + 2) / 3 * 3;
  if (ws_floats < (long)B * H * NC * kOpsFloats || ((uintptr_t)ws & 15))
    return RWKVQ_ERR_ARG;
  hipLaunchKernelGGL(wkv_chunk_ops_k<false>, dim3(B * H * NC), dim3(256), 0,
                     (hipStream_t)stream, r, r_ld, w, k, a, b, ld, ws, T, H,
                     NC, PrepIn{});
  hipLaunchKernelGGL(wkv_chunk_scan_k, dim3(B * H * 4), dim3(256), 0,
                     (hipStream_t)stream, v, ld, ws,
                     state_in ? state_in : state_out, state_out, y, y_ld, T,
                     H, NC);
  return ok_launch();
}

int rwkvq_wkv7_scan_chunked_noalloc(const float* r, long r_ld,
                                    const float* w, const float* k,
                                    const float* v, const float* a,
                                    const float* b, long ld,
                                    const float* state_in, float* state_out,
                                    float* y, long y_ld, int B, int T, int H,
                                    int head_size, void* stream) {
  if (B <= 0 || T <= 0 || H <= 0 || head_size != kHead)
    return RWKVQ_ERR_ARG;
  const long NC = ((T + kCL - 1) / kCL + 2) / 3 * 3;
  if ((long)B * H * NC * kOpsFloats > kScratchFloats) return RWKVQ_ERR_SIZE;
  float* ws = nullptr;
  const int st = scratch_base(&ws);
  if (st) return st;
  // every operator slot the scan reads is written by the operator kernel
  // of the same call, so nothing in the scratch has to start at zero
  return rwkvq_wkv7_scan_chunked(r, r_ld, w, k, v, a, b, ld, state_in,
                                 state_out, y, y_ld, B, T, H, head_size, ws,
                                 kScratchFloats, stream);
}

int rwkvq_wkv7_prefill_chunked(const float* rkv, const float* yw,
                               const float* ya, const float* yv,
                               const float* w0, const float* a0,
                               const float* v0, const float* k_k,
                               const float* k_a, float* v_first, int layer0,
                               float* kp, float* vp, const float* state_in,
                               float* state_out, float* y, int B, int T,
                               int H, int head_size, float* ws,
                               long ws_floats, void* stream) {
  const int D = H * kHead;
  if (B <= 0 || T <= 0 || H <= 0 || head_size != kHead || D % 256 || !rkv ||
      !yw || !ya || !w0 || !a0 || !k_k || !k_a || !v_first || !kp || !vp ||
      !y || !ws || !state_out || (!layer0 && (!yv || !v0)))
    return RWKVQ_ERR_ARG;
  const int NC = ((T + kCL - 1) / kCL + 2) / 3 * 3;
  if (ws_floats < (long)B * H * NC * kOpsFloats || ((uintptr_t)ws & 15))
    return RWKVQ_ERR_ARG;
  const PrepIn pi{rkv, yw, ya, yv, w0, a0, v0, k_k, k_a, v_first, layer0, kp,
                  vp, D};
  hipLaunchKernelGGL(wkv_chunk_ops_k<true>, dim3(B * H * NC), dim3(256), 0,
                     (hipStream_t)stream, nullptr, 0, nullptr, nullptr,
                     nullptr, nullptr, 0, ws, T, H, NC, pi);
  hipLaunchKernelGGL(wkv_chunk_scan_k, dim3(B * H * 4), dim3(256), 0,
                     (hipStream_t)stream, vp, (long)D, ws,
                     state_in ? state_in : state_out, state_out, y, (long)D,
                     T, H, NC);
  return ok_launch();
}

int rwkvq_wkv_tail(const float* y, const float* rkv, const float* kp,
                   const float* vp, const float* g, const float* r_k,
                   const float* ln_w, const float* ln_b, float* out, int N,
                   int D, int head_size, void* stream) {
  if (N <= 0 || D % 256 || head_size != kHead) return RWKVQ_ERR_ARG;
  hipLaunchKernelGGL(wkv_tail_k<-1>, dim3(D / 256, N), dim3(256), 0,
                     (hipStream_t)stream, y, rkv, kp, vp, g, r_k, ln_w, ln_b,
                     out, D);
  return ok_launch();
}

int rwkvq_wkv_tail_f16(const float* y, const float* rkv, const float* kp,
                       const float* vp, const float* g, const float* r_k,
                       const float* ln_w, const float* ln_b, uint16_t* out,
                       int order, int N, int D, int head_size, void* stream) {
  if (N <= 0 || D % 256 || head_size != kHead || order < 0 ||
      order > RWKVQ_ORDER_SYM6 || reinterpret_cast<uintptr_t>(out) % 4)
    return RWKVQ_ERR_ARG;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid(D / 256, N);
  if (order == RWKVQ_ORDER_PAIRS)
    hipLaunchKernelGGL(wkv_tail_k<RWKVQ_ORDER_PAIRS>, grid, dim3(256), 0, s,
                       y, rkv, kp, vp, g, r_k, ln_w, ln_b, out, D);
  else if (order == RWKVQ_ORDER_SB6)
    hipLaunchKernelGGL(wkv_tail_k<RWKVQ_ORDER_SB6>, grid, dim3(256), 0, s, y,
                       rkv, kp, vp, g, r_k, ln_w, ln_b, out, D);
  else
    hipLaunchKernelGGL(wkv_tail_k<RWKVQ_ORDER_SYM6>, grid, dim3(256), 0, s,
                       y, rkv, kp, vp, g, r_k, ln_w, ln_b, out, D);
  return ok_launch();
}

int rwkvq_wkv7_decode(const float* rkv, const float* yw, const float* ya,
                      const float* yv, const float* g, const float* w0,
                      const float* a0, const float* v0, const float* k_k,
                      const float* k_a, const float* r_k, const float* ln_w,
                      const float* ln_b, float* v_first, int layer0,
                      const float* state_in, float* state_out, float* out,
                      int B, int H, int head_size, void* stream) {
  if (B <= 0 || H <= 0 || head_size != kHead || (!layer0 && (!yv || !v0)))
    return RWKVQ_ERR_ARG;
  hipLaunchKernelGGL(wkv_decode_k<0>, dim3(B * H), dim3(256), 0,
                     (hipStream_t)stream, rkv, yw, ya, yv, g, w0, a0, v0, k_k,
                     k_a, r_k, ln_w, ln_b, v_first, layer0,
                     state_in ? state_in : state_out, state_out, out, H,
                     LoraUp{}, LoraUpQ{});
  return ok_launch();
}

int rwkvq_wkv7_decode_lora(const float* rkv, const float* const* h,
                           const void* const* Bup, const int* rank,
                           const float* w0, const float* a0, const float* v0,
                           const float* k_k, const float* k_a,
                           const float* r_k, const float* ln_w,
                           const float* ln_b, float* v_first, int layer0,
                           const float* state_in, float* state_out,
                           float* out, int B, int H, int head_size,
                           void* stream) {
  if (B <= 0 || H <= 0 || head_size != kHead) return RWKVQ_ERR_ARG;
  LoraUp lu{};
  for (int k = 0; k < 4; ++k) {
    const bool need = k != 2 || !layer0;       // no v branch in layer 0
    if (!need) continue;
    if (!h[k] || !Bup[k] || rank[k] <= 0 || rank[k] % 8)
      return RWKVQ_ERR_ARG;
    lu.h[k] = h[k];
    lu.B[k] = static_cast<const uint16_t*>(Bup[k]);
    lu.r[k] = rank[k];
  }
  if (!layer0 && !v0) return RWKVQ_ERR_ARG;
  if (lu.r[0] + lu.r[1] + lu.r[2] + lu.r[3] > kMaxCat) return RWKVQ_ERR_SIZE;
  hipLaunchKernelGGL(wkv_decode_k<1>, dim3(B * H), dim3(256), 0,
                     (hipStream_t)stream, rkv, nullptr, nullptr, nullptr,
                     nullptr, w0, a0, v0, k_k, k_a, r_k, ln_w, ln_b, v_first,
                     layer0, state_in ? state_in : state_out, state_out, out,
                     H, lu, LoraUpQ{});
  return ok_launch();
}

int rwkvq_wkv7_decode_lora_q(const float* rkv, const float* const* h,
                             const uint8_t* const* q, const float* const* s,
                             const float* const* m, const uint16_t* const* sc,
                             const int* rank, const float* w0,
                             const float* a0, const float* v0,
                             const float* k_k, const float* k_a,
                             const float* r_k, const float* ln_w,
                             const float* ln_b, float* v_first, int layer0,
                             const float* state_in, float* state_out,
                             float* out, int B, int H, int head_size,
                             void* stream) {
  if (B <= 0 || H <= 0 || head_size != kHead) return RWKVQ_ERR_ARG;
  LoraUpQ lq{};
  for (int k = 0; k < 4; ++k) {
    const bool need = k != 2 || !layer0;       // no v branch in layer 0
    if (!need) continue;
    const bool i8 = s[k] == nullptr;
    if (!h[k] || !q[k] || rank[k] <= 0 || rank[k] % 16 || rank[k] > 512 ||
        (i8 ? !sc[k] : !m[k]) || (reinterpret_cast<uintptr_t>(q[k]) & 15))
      return RWKVQ_ERR_ARG;
    lq.h[k] = h[k];
    lq.q[k] = q[k];
    lq.s[k] = s[k];
    lq.m[k] = i8 ? nullptr : m[k];
    lq.sc[k] = i8 ? sc[k] : nullptr;
    lq.r[k] = rank[k];
  }
  if (!layer0 && !v0) return RWKVQ_ERR_ARG;
  if (lq.r[0] + lq.r[1] + lq.r[2] + lq.r[3] > kMaxCat) return RWKVQ_ERR_SIZE;
  hipLaunchKernelGGL(wkv_decode_k<2>, dim3(B * H), dim3(256), 0,
                     (hipStream_t)stream, rkv, nullptr, nullptr, nullptr,
                     nullptr, w0, a0, v0, k_k, k_a, r_k, ln_w, ln_b, v_first,
                     layer0, state_in ? state_in : state_out, state_out, out,
                     H, LoraUp{}, lq);
  return ok_launch();
}

}  // extern "C"
