// Bit-exact fp32 dequantization of the device layouts (the checker the
// GEMV/GEMM kernels are compared against, and the load-time expansion of
// LoRA tensors).  Arithmetic follows the format formulas with their fp16
// round trips and with products and sums rounded separately (no FMA
// contraction), exactly as the numpy reference computes them
// (reference: rwkv_quant/formats/codec.py:183-292).
#include "rwkvq_common.h"
#include "gather_cols.h"

// products and sums must round separately, as numpy does: forbid the
// a*b+c -> fma contraction hipcc applies by default
#pragma clang fp contract(off)

using namespace rwkvq;

namespace {

__global__ void dq_sb6(const uint8_t* nib, const uint32_t* hb,
                       const uint8_t* rec, int bits, int rows, int in,
                       float* w, int ld, const int64_t* idx, int src_rows) {
  const int ng = in >> 5, nsb = in >> 8;
  long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (long)rows * ng) return;
  const int orow = (int)(t / ng), g = (int)(t % ng);
  const int row = src_row(idx, orow, src_rows);
  const uint8_t* rp = rec + ((size_t)row * nsb + (g >> 3)) * 16;
  const int kb = g & 7;
  // 6-bit fields of the 48-bit qs stream and the 48-bit qm stream
  uint64_t s0 = 0, s1 = 0;
  for (int b = 0; b < 6; ++b) {
    s0 |= (uint64_t)rp[b] << (8 * b);
    s1 |= (uint64_t)rp[6 + b] << (8 * b);
  }
  const uint32_t qs = (uint32_t)(s0 >> (6 * kb)) & 63u;
  const int qm = (int)((uint32_t)(s1 >> (6 * kb)) & 63u) - 31;
  const float d = f16_bits_to_f32(rp[12] | (rp[13] << 8));
  const float dm = f16_bits_to_f32(rp[14] | (rp[15] << 8));
  const float s = fmaxf(f16_round(((float)qs * d)), 1e-8f);
  const float m = f16_round(((float)qm * dm));
  const uint8_t* np = nib + ((size_t)row * ng + g) * 16;
  float* out = w + (size_t)orow * ld + (size_t)g * 32;
  for (int c = 0; c < 32; ++c) {
    const int i = c & 15, half = c >> 4;
    uint32_t q = half ? (np[i] >> 4) : (np[i] & 15u);
    if (bits == 5) {
      uint32_t hw = hb[(size_t)row * ng + g];
      q |= ((hw >> c) & 1u) << 4;
    } else if (bits == 6) {
      q |= high_bits_crumb(hb + ((size_t)row * ng + g) * 2, i, half) << 4;
    }
    out[c] = (float)q * s + m;
  }
}

// Row gather of sb6 codes (the embedding lookup, a few rows): one thread
// per 8 consecutive columns (sb6_cols8: the group's 16-byte record and the
// thread's 8 code bytes in one load each), the 8 outputs in two float4
// stores (consecutive threads, consecutive columns).
__global__ void gather_sb6(const uint8_t* nib, const uint32_t* hb,
                           const uint8_t* rec, int bits, int n, int in,
                           float* w, const int64_t* idx, int src_rows) {
  const int per_row = in >> 3;
  const long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (long)n * per_row) return;
  const int orow = (int)(t / per_row), k = (int)(t % per_row);
  float o[8];
  sb6_cols8(nib, hb, rec, bits, in, src_row(idx, orow, src_rows), k, o);
  float4* out = reinterpret_cast<float4*>(w + (size_t)orow * in + 8 * k);
  out[0] = make_float4(o[0], o[1], o[2], o[3]);
  out[1] = make_float4(o[4], o[5], o[6], o[7]);
}

__global__ void dq_sym(const uint8_t* codes, const uint32_t* hb,
                       const int8_t* qsp, const uint16_t* dp, int bits,
                       int rows, int in, float* w, int ld, const int64_t* idx,
                       int src_rows) {
  const int ng = in >> 5, nsb = in >> 8;
  long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (long)rows * ng) return;
  const int orow = (int)(t / ng), g = (int)(t % ng);
  const int row = src_row(idx, orow, src_rows);
  const float d = f16_bits_to_f32(dp[(size_t)row * nsb + (g >> 3)]);
  const float sA = f16_round(((float)qsp[(size_t)row * (in >> 4) + 2 * g] * d));
  const float sB = f16_round(((float)qsp[(size_t)row * (in >> 4) + 2 * g + 1] * d));
  float* out = w + (size_t)orow * ld + (size_t)g * 32;
  for (int c = 0; c < 32; ++c) {
    int q;
    if (bits == 8) {
      q = (int)(int8_t)codes[(size_t)row * in + (size_t)g * 32 + c];
    } else {
      // 16-block local split: byte j of block b holds columns j and j + 8
      const int blk = c >> 4, cc = c & 15;
      const int byte = blk * 8 + (cc & 7), half = cc >> 3;
      const uint8_t v = codes[((size_t)row * ng + g) * 16 + byte];
      uint32_t u = half ? (v >> 4) : (v & 15u);
      u |= high_bits_crumb(hb + ((size_t)row * ng + g) * 2, byte, half) << 4;
      q = (int)u - 32;
    }
    out[c] = (float)q * (c < 16 ? sA : sB);
  }
}

// Row gather of sym codes, laid out as gather_sb6 (sym_cols8).
__global__ void gather_sym(const uint8_t* codes, const uint32_t* hb,
                           const int8_t* qsp, const uint16_t* dp, int bits,
                           int n, int in, float* w, const int64_t* idx,
                           int src_rows) {
  const int per_row = in >> 3;
  const long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (long)n * per_row) return;
  const int orow = (int)(t / per_row), k = (int)(t % per_row);
  float o[8];
  sym_cols8(codes, hb, qsp, dp, bits, in, src_row(idx, orow, src_rows), k,
            o);
  float4* out = reinterpret_cast<float4*>(w + (size_t)orow * in + 8 * k);
  out[0] = make_float4(o[0], o[1], o[2], o[3]);
  out[1] = make_float4(o[4], o[5], o[6], o[7]);
}

__global__ void dq_rtn8(const int8_t* codes, const uint16_t* scale, int rows,
                        int in, float* w, int ld, const int64_t* idx,
                        int src_rows) {
  long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (long)rows * in) return;
  const int orow = (int)(t / in), c = (int)(t % in);
  const int row = src_row(idx, orow, src_rows);
  w[(size_t)orow * ld + c] =
      (float)codes[(size_t)row * in + c] * f16_bits_to_f32(scale[row]);
}

__global__ void dq_asym(const uint8_t* codes, const float* scale,
                        const float* mn, int gs, int rows, int in, float* w,
                        int ld) {
  long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (long)rows * in) return;
  const int row = (int)(t / in), c = (int)(t % in);
  const int nb = (in + gs - 1) / gs;
  const size_t b = (size_t)row * nb + c / gs;
  w[(size_t)row * ld + c] = (float)codes[t] * scale[b] + mn[b];
}

// ---- wide dequant for the prefill GEMM operands -------------------------
// One thread per (row, 32-column group): 16-byte loads of the packed fields,
// the same fp32 arithmetic as the bit-exact kernels above, then one
// rounding to the output type and 16-byte stores in natural column order.
// fp16 output is therefore exactly f16(the bit-exact fp32 dequant).
enum DqFmt { DQ_SB6_4 = 0, DQ_SB6_5, DQ_SB6_6, DQ_SYM6, DQ_SYM8, DQ_RTN8 };

template <int FMT>
__device__ __forceinline__ void group_values(
    const uint8_t* __restrict__ q, const uint32_t* __restrict__ hb,
    const uint8_t* __restrict__ rec, const int8_t* __restrict__ qsp,
    const uint16_t* __restrict__ dp, int in, int row, int g, float (&w)[32]) {
  const int ng = in >> 5, nsb = in >> 8;
  if (FMT == DQ_SYM8 || FMT == DQ_RTN8) {
    const uint8_t* p = q + (size_t)row * in + (size_t)g * 32;
    const uint4 a = *reinterpret_cast<const uint4*>(p);
    const uint4 b = *reinterpret_cast<const uint4*>(p + 16);
    const uint32_t wd[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    float sA, sB;
    if (FMT == DQ_RTN8) {
      sA = sB = f16_bits_to_f32(dp[row]);
    } else {
      const float d = f16_bits_to_f32(dp[(size_t)row * nsb + (g >> 3)]);
      const uint16_t q2 =
          *reinterpret_cast<const uint16_t*>(qsp + (size_t)row * (in >> 4) + 2 * g);
      sA = f16_round((float)(int8_t)(q2 & 0xFF) * d);
      sB = f16_round((float)(int8_t)(q2 >> 8) * d);
    }
#pragma unroll
    for (int c = 0; c < 32; ++c) {
      const int8_t code = (int8_t)((wd[c >> 2] >> (8 * (c & 3))) & 0xFF);
      w[c] = (float)code * (c < 16 ? sA : sB);
    }
    return;
  }
  const uint4 nb = *reinterpret_cast<const uint4*>(q + ((size_t)row * ng + g) * 16);
  const uint32_t nw[4] = {nb.x, nb.y, nb.z, nb.w};
  uint32_t h0 = 0, h1 = 0;
  if (FMT == DQ_SB6_5) h0 = hb[(size_t)row * ng + g];
  if (FMT == DQ_SB6_6 || FMT == DQ_SYM6) {
    const uint2 hh = *reinterpret_cast<const uint2*>(hb + ((size_t)row * ng + g) * 2);
    h0 = hh.x; h1 = hh.y;
  }
  int code[32];
#pragma unroll
  for (int i = 0; i < 16; ++i) {            // nibble byte i
    const uint32_t byte = (nw[i >> 2] >> (8 * (i & 3))) & 0xFF;
    int c0, c1;
    if (FMT == DQ_SYM6) { c0 = i < 8 ? i : i + 8; c1 = c0 + 8; }
    else { c0 = i; c1 = i + 16; }
    uint32_t lo = byte & 15, hi = byte >> 4;
    if (FMT == DQ_SB6_5) {
      lo |= ((h0 >> c0) & 1) << 4;
      hi |= ((h0 >> c1) & 1) << 4;
    } else if (FMT == DQ_SB6_6 || FMT == DQ_SYM6) {
      const uint32_t H = i < 8 ? h0 : h1;
      const int sh = 2 * (i & 7);
      lo |= ((H >> sh) & 3) << 4;
      hi |= ((H >> (sh + 16)) & 3) << 4;
    }
    code[c0] = (int)lo;
    code[c1] = (int)hi;
  }
  if (FMT == DQ_SYM6) {
    const float d = f16_bits_to_f32(dp[(size_t)row * nsb + (g >> 3)]);
    const uint16_t q2 =
        *reinterpret_cast<const uint16_t*>(qsp + (size_t)row * (in >> 4) + 2 * g);
    const float sA = f16_round((float)(int8_t)(q2 & 0xFF) * d);
    const float sB = f16_round((float)(int8_t)(q2 >> 8) * d);
#pragma unroll
    for (int c = 0; c < 32; ++c) w[c] = (float)(code[c] - 32) * (c < 16 ? sA : sB);
    return;
  }
  // sb6: superblock record
  const uint4 rc = *reinterpret_cast<const uint4*>(rec + ((size_t)row * nsb + (g >> 3)) * 16);
  const uint64_t s0 = (uint64_t)rc.x | ((uint64_t)(rc.y & 0xFFFF) << 32);
  const uint64_t s1 = (uint64_t)(rc.y >> 16) | ((uint64_t)rc.z << 16);
  const int kb = g & 7;
  const uint32_t qsv = (uint32_t)(s0 >> (6 * kb)) & 63u;
  const int qmv = (int)((uint32_t)(s1 >> (6 * kb)) & 63u) - 31;
  const float d = f16_bits_to_f32(rc.w & 0xFFFF);
  const float dm = f16_bits_to_f32(rc.w >> 16);
  const float sc = fmaxf(f16_round((float)qsv * d), 1e-8f);
  const float mn = f16_round((float)qmv * dm);
#pragma unroll
  for (int c = 0; c < 32; ++c) w[c] = (float)code[c] * sc + mn;
}

template <int FMT, typename OutT>
__global__ void __launch_bounds__(256)
dq_wide_k(const uint8_t* __restrict__ q, const uint32_t* __restrict__ hb,
          const uint8_t* __restrict__ rec, const int8_t* __restrict__ qsp,
          const uint16_t* __restrict__ dp, int rows, int in,
          OutT* __restrict__ out, int ld) {
  const int ng = in >> 5;
  const long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (long)rows * ng) return;
  const int row = (int)(t / ng), g = (int)(t % ng);
  float w[32];
  group_values<FMT>(q, hb, rec, qsp, dp, in, row, g, w);
  OutT* o = out + (size_t)row * ld + (size_t)g * 32;
  if constexpr (sizeof(OutT) == 2) {
    uint32_t pk[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) pk[i] = pack_h2(w[2 * i], w[2 * i + 1]);
#pragma unroll
    for (int v = 0; v < 4; ++v)
      reinterpret_cast<uint4*>(o)[v] =
          make_uint4(pk[4 * v], pk[4 * v + 1], pk[4 * v + 2], pk[4 * v + 3]);
  } else {
#pragma unroll
    for (int v = 0; v < 8; ++v)
      reinterpret_cast<float4*>(o)[v] =
          make_float4(w[4 * v], w[4 * v + 1], w[4 * v + 2], w[4 * v + 3]);
  }
}

template <typename OutT>
int launch_wide(int fmt, const uint8_t* q, const uint32_t* hb,
                const uint8_t* rec, const int8_t* qs, const uint16_t* d,
                int rows, int in, OutT* out, int ld, hipStream_t s) {
  const long n = (long)rows * (in / 32);
  const dim3 grid((unsigned)((n + 255) / 256)), block(256);
  switch (fmt) {
    case DQ_SB6_4: hipLaunchKernelGGL((dq_wide_k<DQ_SB6_4, OutT>), grid, block, 0, s, q, hb, rec, qs, d, rows, in, out, ld); break;
    case DQ_SB6_5: hipLaunchKernelGGL((dq_wide_k<DQ_SB6_5, OutT>), grid, block, 0, s, q, hb, rec, qs, d, rows, in, out, ld); break;
    case DQ_SB6_6: hipLaunchKernelGGL((dq_wide_k<DQ_SB6_6, OutT>), grid, block, 0, s, q, hb, rec, qs, d, rows, in, out, ld); break;
    case DQ_SYM6: hipLaunchKernelGGL((dq_wide_k<DQ_SYM6, OutT>), grid, block, 0, s, q, hb, rec, qs, d, rows, in, out, ld); break;
    case DQ_SYM8: hipLaunchKernelGGL((dq_wide_k<DQ_SYM8, OutT>), grid, block, 0, s, q, hb, rec, qs, d, rows, in, out, ld); break;
    case DQ_RTN8: hipLaunchKernelGGL((dq_wide_k<DQ_RTN8, OutT>), grid, block, 0, s, q, hb, rec, qs, d, rows, in, out, ld); break;
    default: return RWKVQ_ERR_ARG;
  }
  return hipGetLastError() == hipSuccess ? RWKVQ_OK : RWKVQ_ERR_LAUNCH;
}

inline dim3 grid_for(long n, int bs) { return dim3((unsigned)((n + bs - 1) / bs)); }

}  // namespace

extern "C" {

int rwkvq_dequant_sb6_f32(const uint8_t* nib, const uint32_t* hb,
                          const uint8_t* rec, int bits, int rows, int in,
                          float* w, int ld, void* stream) {
  if (rows <= 0 || in <= 0 || in % 256 || ld < in || bits < 4 || bits > 6 ||
      (bits > 4 && !hb))
    return RWKVQ_ERR_ARG;
  long n = (long)rows * (in / 32);
  hipLaunchKernelGGL(dq_sb6, grid_for(n, 256), dim3(256), 0,
                     (hipStream_t)stream, nib, hb, rec, bits, rows, in, w, ld,
                     (const int64_t*)nullptr, rows);
  return hipGetLastError() == hipSuccess ? RWKVQ_OK : RWKVQ_ERR_LAUNCH;
}

int rwkvq_dequant_sym_f32(const uint8_t* codes, const uint32_t* hb,
                          const int8_t* qs, const uint16_t* d, int bits,
                          int rows, int in, float* w, int ld, void* stream) {
  if (rows <= 0 || in <= 0 || in % 256 || ld < in || (bits != 6 && bits != 8) ||
      (bits == 6 && !hb))
    return RWKVQ_ERR_ARG;
  long n = (long)rows * (in / 32);
  hipLaunchKernelGGL(dq_sym, grid_for(n, 256), dim3(256), 0,
                     (hipStream_t)stream, codes, hb, qs, d, bits, rows, in, w, ld,
                     (const int64_t*)nullptr, rows);
  return hipGetLastError() == hipSuccess ? RWKVQ_OK : RWKVQ_ERR_LAUNCH;
}

int rwkvq_dequant_rtn8_f32(const int8_t* codes, const uint16_t* scale,
                           int rows, int in, float* w, int ld, void* stream) {
  if (rows <= 0 || in <= 0 || ld < in) return RWKVQ_ERR_ARG;
  long n = (long)rows * in;
  hipLaunchKernelGGL(dq_rtn8, grid_for(n, 256), dim3(256), 0,
                     (hipStream_t)stream, codes, scale, rows, in, w, ld,
                     (const int64_t*)nullptr, rows);
  return hipGetLastError() == hipSuccess ? RWKVQ_OK : RWKVQ_ERR_LAUNCH;
}

int rwkvq_dequant_asym_f32(const uint8_t* codes, const float* scale,
                           const float* mn, int gs, int rows, int in,
                           float* w, int ld, void* stream) {
  if (rows <= 0 || in <= 0 || gs <= 0 || ld < in) return RWKVQ_ERR_ARG;
  long n = (long)rows * in;
  hipLaunchKernelGGL(dq_asym, grid_for(n, 256), dim3(256), 0,
                     (hipStream_t)stream, codes, scale, mn, gs, rows, in, w, ld);
  return hipGetLastError() == hipSuccess ? RWKVQ_OK : RWKVQ_ERR_LAUNCH;
}

int rwkvq_gather_rows_f32(int kind, int bits, const uint8_t* q,
                          const uint32_t* hb, const void* aux0,
                          const uint16_t* aux1, int src_rows, int in,
                          const int64_t* idx, int n_idx, float* out,
                          void* stream) {
  if (n_idx <= 0 || src_rows <= 0 || in <= 0 || !idx) return RWKVQ_ERR_ARG;
  hipStream_t s = (hipStream_t)stream;
  if (kind == 0) {            // sb6: aux0 = rec
    if (in % 256 || bits < 4 || bits > 6 || (bits > 4 && !hb))
      return RWKVQ_ERR_ARG;
    if (reinterpret_cast<uintptr_t>(out) & 15) return RWKVQ_ERR_ARG;
    long n = (long)n_idx * (in / 8);
    hipLaunchKernelGGL(gather_sb6, grid_for(n, 256), dim3(256), 0, s, q, hb,
                       (const uint8_t*)aux0, bits, n_idx, in, out, idx,
                       src_rows);
  } else if (kind == 1) {     // sym: aux0 = qs, aux1 = d
    if (in % 256 || (bits != 6 && bits != 8) || (bits == 6 && !hb))
      return RWKVQ_ERR_ARG;
    if (reinterpret_cast<uintptr_t>(out) & 15) return RWKVQ_ERR_ARG;
    long n = (long)n_idx * (in / 8);
    hipLaunchKernelGGL(gather_sym, grid_for(n, 256), dim3(256), 0, s, q, hb,
                       (const int8_t*)aux0, aux1, bits, n_idx, in, out, idx,
                       src_rows);
  } else if (kind == 2) {     // rtn@8: aux1 = scale
    long n = (long)n_idx * in;
    hipLaunchKernelGGL(dq_rtn8, grid_for(n, 256), dim3(256), 0, s,
                       (const int8_t*)q, aux1, n_idx, in, out, in, idx,
                       src_rows);
  } else {
    return RWKVQ_ERR_ARG;
  }
  return hipGetLastError() == hipSuccess ? RWKVQ_OK : RWKVQ_ERR_LAUNCH;
}

int rwkvq_dequant_f16(int fmt, const uint8_t* q, const uint32_t* hb,
                      const uint8_t* rec, const int8_t* qs, const uint16_t* d,
                      int rows, int in, uint16_t* out, int ld, void* stream) {
  if (rows <= 0 || in <= 0 || in % 256 || ld < in || (ld & 7) || fmt < 0 ||
      fmt > DQ_RTN8 || ((fmt == DQ_SB6_5 || fmt == DQ_SB6_6 || fmt == DQ_SYM6) && !hb))
    return RWKVQ_ERR_ARG;
  return launch_wide<_Float16>(fmt, q, hb, rec, qs, d, rows, in,
                               reinterpret_cast<_Float16*>(out), ld,
                               (hipStream_t)stream);
}

}  // extern "C"
