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

// ---- down products straight from the file's codes (decode) -------------
// A world checkpoint stores each down factor as [in, rank] with its
// quantization blocks along the rank axis: asym gw64 (u8 codes, fp32 scale
// and min per 64 ranks of a stored row) or per-row int8 (fp16 scale per
// stored row, the g branch).  At load the codes are transposed to
// [rank, in] (a permutation of the file's bytes) and the asym scale / min
// to [rank / 64, in], so output row r streams one contiguous code row and
// the block parameters of its 64-row group along the same columns; the
// int8 scale is then one value per input column.  Each weight is
// dequantized in registers exactly as rwkvq_dequant_asym_f32 /
// rwkvq_dequant_rtn8_f32 compute it (fp32 code * scale, then + min, no
// contraction); x stays fp32, products and sums are fp32.
struct LoraQJob {
  const uint8_t* q;      // codes [rows, in] (u8 asym / i8 rtn)
  const float* s;        // asym: scale [rows / 64 (ceil), in]; rtn: null
  const float* m;        // asym: min, same layout
  const uint16_t* sc;    // rtn: fp16 scale per input column [in]
  const float* x;        // x[n * x_ld + c]
  float* y;              // y[n * y_ld + r]
  int rows, x_ld, y_ld, epi;
  int wg0;               // first workgroup of this job
};

struct LoraQJobs {
  LoraQJob j[4];
  int n_jobs, N, in;
};

// One weight, rounded as the dequant kernels round it: the product, then
// the sum, each in fp32 (no fused multiply-add).
__device__ __forceinline__ float dq_asym_1(uint32_t code, float s, float m) {
#pragma clang fp contract(off)
  return (float)code * s + m;
}
__device__ __forceinline__ float dq_rtn8_1(uint32_t byte, float s) {
  return (float)(int)(int8_t)byte * s;
}

constexpr int kQRowsPerWave = 2;
constexpr int kQRowsPerWg = 4 * kQRowsPerWave;

// One workgroup = 8 output rows of one job (two per wave, same 64-row
// block group); lane l owns the 4-column chunks l + 64 k (k < KQ,
// in = 256 KQ).  Codes and block parameters are loaded before x is staged
// in LDS, so the two memory round trips overlap; the wave's weights are
// dequantized once into registers, then each input row is one pass of
// fused multiply-adds over them (the row loop is not unrolled, which keeps
// the kernel small).
template <int KQ, bool RTN>
__device__ __forceinline__ void lora_q_rows(const LoraQJob& jo, int N,
                                            int lwg, float* s_x) {
  constexpr int IN = 256 * KQ;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r0 = lwg * kQRowsPerWg + wave * kQRowsPerWave;
  const bool live = r0 < jo.rows;
  const int rr = live ? r0 : jo.rows - kQRowsPerWave;   // in-bounds loads
  uint32_t cq[kQRowsPerWave][KQ];
#pragma unroll
  for (int r = 0; r < kQRowsPerWave; ++r)
#pragma unroll
    for (int k = 0; k < KQ; ++k)
      cq[r][k] = *reinterpret_cast<const uint32_t*>(
          jo.q + (size_t)(rr + r) * IN + 4 * (lane + 64 * k));
  // block parameters as raw bits: nothing consumes them before every load
  // of the thread is in flight
  uint4 sv[KQ], mv[KQ];
  uint2 scv[KQ];
#pragma unroll
  for (int k = 0; k < KQ; ++k) {
    const int c0 = 4 * (lane + 64 * k);
    if constexpr (RTN) {
      scv[k] = *reinterpret_cast<const uint2*>(jo.sc + c0);
    } else {
      const size_t o = (size_t)(rr >> 6) * IN + c0;
      sv[k] = *reinterpret_cast<const uint4*>(jo.s + o);
      mv[k] = *reinterpret_cast<const uint4*>(jo.m + o);
    }
  }
  // x of the job, all N rows, into LDS, eight loads of a thread in flight
  // before their stores (N * in <= 16384 floats: at most 16 float4 per
  // thread, two rounds).  Indices past the rows are clamped to the last
  // element, whose value the thread then also stores (the same bits the
  // owning thread writes), so loads and stores carry no condition.
  constexpr int kXRound = 8;
  const int nx4 = N * (IN / 4);
#pragma unroll
  for (int t0 = 0; t0 < 16384 / 4 / 256; t0 += kXRound) {
    if (256 * t0 >= nx4) break;              // workgroup-uniform
    uint4 xv[kXRound];
    int xi[kXRound];
#pragma unroll
    for (int t = 0; t < kXRound; ++t) {
      xi[t] = min((int)threadIdx.x + 256 * (t0 + t), nx4 - 1);
      const int n = xi[t] / (IN / 4), c4 = xi[t] % (IN / 4);
      xv[t] = *reinterpret_cast<const uint4*>(jo.x + (size_t)n * jo.x_ld +
                                              4 * c4);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < kXRound; ++t) {
      pin(xv[t]);
      reinterpret_cast<uint4*>(s_x)[xi[t]] = xv[t];
    }
  }
  // the wave's weights, exact
  float w[kQRowsPerWave][KQ][4];
#pragma unroll
  for (int k = 0; k < KQ; ++k) {
    float sk[4], mk[4];
    if constexpr (RTN) {
      sk[0] = h2_lo(scv[k].x); sk[1] = h2_hi(scv[k].x);
      sk[2] = h2_lo(scv[k].y); sk[3] = h2_hi(scv[k].y);
    } else {
      sk[0] = __uint_as_float(sv[k].x); sk[1] = __uint_as_float(sv[k].y);
      sk[2] = __uint_as_float(sv[k].z); sk[3] = __uint_as_float(sv[k].w);
      mk[0] = __uint_as_float(mv[k].x); mk[1] = __uint_as_float(mv[k].y);
      mk[2] = __uint_as_float(mv[k].z); mk[3] = __uint_as_float(mv[k].w);
    }
#pragma unroll
    for (int r = 0; r < kQRowsPerWave; ++r)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t b = (cq[r][k] >> (8 * e)) & 0xFFu;
        if constexpr (RTN) w[r][k][e] = dq_rtn8_1(b, sk[e]);
        else w[r][k][e] = dq_asym_1(b, sk[e], mk[e]);
      }
  }
  __syncthreads();
  if (!live) return;
  for (int n = 0; n < N; ++n) {
    const float4* xr = reinterpret_cast<const float4*>(s_x + n * IN);
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int k = 0; k < KQ; ++k) {
      const float4 xv = xr[lane + 64 * k];
      a0 = fmaf(xv.x, w[0][k][0], a0);
      a1 = fmaf(xv.x, w[1][k][0], a1);
      a0 = fmaf(xv.y, w[0][k][1], a0);
      a1 = fmaf(xv.y, w[1][k][1], a1);
      a0 = fmaf(xv.z, w[0][k][2], a0);
      a1 = fmaf(xv.z, w[1][k][2], a1);
      a0 = fmaf(xv.w, w[0][k][3], a0);
      a1 = fmaf(xv.w, w[1][k][3], a1);
    }
    a0 = wave_sum_dpp(a0);
    a1 = wave_sum_dpp(a1);
    if (lane == 0) {
      float* yr = jo.y + (size_t)n * jo.y_ld + r0;
      yr[0] = epi_apply(a0, jo.epi);
      yr[1] = epi_apply(a1, jo.epi);
    }
  }
}

template <int KQ>
__global__ void __launch_bounds__(256)
lora_down_q_k(LoraQJobs J) {
  extern __shared__ float s_xq[];
  // the job is workgroup-uniform: its descriptor is selected field by
  // field with constant indices into the argument table (a dynamic index
  // would copy the table to scratch), and the body is instantiated once
  const int bx = blockIdx.x;
  const int jb = (J.n_jobs > 3 && bx >= J.j[3].wg0) ? 3
               : (J.n_jobs > 2 && bx >= J.j[2].wg0) ? 2
               : (J.n_jobs > 1 && bx >= J.j[1].wg0) ? 1 : 0;
  LoraQJob jo;
  jo.q = jb == 0 ? J.j[0].q : jb == 1 ? J.j[1].q : jb == 2 ? J.j[2].q : J.j[3].q;
  jo.s = jb == 0 ? J.j[0].s : jb == 1 ? J.j[1].s : jb == 2 ? J.j[2].s : J.j[3].s;
  jo.m = jb == 0 ? J.j[0].m : jb == 1 ? J.j[1].m : jb == 2 ? J.j[2].m : J.j[3].m;
  jo.sc = jb == 0 ? J.j[0].sc : jb == 1 ? J.j[1].sc : jb == 2 ? J.j[2].sc : J.j[3].sc;
  jo.x = jb == 0 ? J.j[0].x : jb == 1 ? J.j[1].x : jb == 2 ? J.j[2].x : J.j[3].x;
  jo.y = jb == 0 ? J.j[0].y : jb == 1 ? J.j[1].y : jb == 2 ? J.j[2].y : J.j[3].y;
  jo.rows = jb == 0 ? J.j[0].rows : jb == 1 ? J.j[1].rows : jb == 2 ? J.j[2].rows : J.j[3].rows;
  jo.x_ld = jb == 0 ? J.j[0].x_ld : jb == 1 ? J.j[1].x_ld : jb == 2 ? J.j[2].x_ld : J.j[3].x_ld;
  jo.y_ld = jb == 0 ? J.j[0].y_ld : jb == 1 ? J.j[1].y_ld : jb == 2 ? J.j[2].y_ld : J.j[3].y_ld;
  jo.epi = jb == 0 ? J.j[0].epi : jb == 1 ? J.j[1].epi : jb == 2 ? J.j[2].epi : J.j[3].epi;
  jo.wg0 = jb == 0 ? J.j[0].wg0 : jb == 1 ? J.j[1].wg0 : jb == 2 ? J.j[2].wg0 : J.j[3].wg0;
  if (jo.s) lora_q_rows<KQ, false>(jo, J.N, bx - jo.wg0, s_xq);
  else lora_q_rows<KQ, true>(jo, J.N, bx - jo.wg0, s_xq);
}

}  // namespace

extern "C" int rwkvq_lora_down_q(int n_jobs, const uint8_t* const* q,
                                 const float* const* s, const float* const* m,
                                 const uint16_t* const* sc,
                                 const float* const* x, const int* x_ld,
                                 float* const* y, const int* y_ld,
                                 const int* rows, const int* epi, int in,
                                 int N, void* stream) {
  if (n_jobs <= 0 || n_jobs > 4 || N <= 0 || N > 8 ||
      (in != 2048 && in != 2560 && in != 4096))
    return RWKVQ_ERR_ARG;
  const size_t lds = (size_t)N * in * sizeof(float);
  if (lds > 64 * 1024) return RWKVQ_ERR_SIZE;
  LoraQJobs J{};
  J.n_jobs = n_jobs;
  J.N = N;
  J.in = in;
  int wgs = 0;
  for (int k = 0; k < n_jobs; ++k) {
    const bool rtn = s[k] == nullptr;
    if (!q[k] || !x[k] || !y[k] || rows[k] <= 0 || rows[k] % 16 ||
        (rtn ? !sc[k] : !m[k]) || x_ld[k] < in || x_ld[k] % 4 ||
        (reinterpret_cast<uintptr_t>(x[k]) & 15) || y_ld[k] < rows[k] ||
        (reinterpret_cast<uintptr_t>(q[k]) & 3) ||
        (rtn ? (reinterpret_cast<uintptr_t>(sc[k]) & 7)
             : ((reinterpret_cast<uintptr_t>(s[k]) |
                 reinterpret_cast<uintptr_t>(m[k])) & 15)))
      return RWKVQ_ERR_ARG;
    LoraQJob& j = J.j[k];
    j.q = q[k]; j.s = s[k]; j.m = rtn ? nullptr : m[k];
    j.sc = rtn ? sc[k] : nullptr;
    j.x = x[k]; j.y = y[k];
    j.rows = rows[k]; j.x_ld = x_ld[k]; j.y_ld = y_ld[k]; j.epi = epi[k];
    j.wg0 = wgs;
    wgs += (rows[k] + kQRowsPerWg - 1) / kQRowsPerWg;
  }
  hipStream_t st = (hipStream_t)stream;
  switch (in) {
    case 2048:
      hipLaunchKernelGGL(lora_down_q_k<8>, dim3(wgs), dim3(256), lds, st, J);
      break;
    case 2560:
      hipLaunchKernelGGL(lora_down_q_k<10>, dim3(wgs), dim3(256), lds, st, J);
      break;
    default:
      hipLaunchKernelGGL(lora_down_q_k<16>, dim3(wgs), dim3(256), lds, st, J);
      break;
  }
  return hipGetLastError() == hipSuccess ? RWKVQ_OK : RWKVQ_ERR_LAUNCH;
}

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
