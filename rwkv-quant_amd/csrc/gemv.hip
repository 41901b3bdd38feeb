// Fused dequant-GEMV for the packed `.rwkvq` layouts on gfx950.
//
// y[n, row] = sum_c x[n, seg(row), c] * W[row, c]  with W decoded from its
// packed codes in registers; no dequantized copy of W ever exists.
//
// Mapping (wave64): lane <-> one 32-column group of the row.  A wave owns a
// K-slice of 64 groups (2048 columns); the lane keeps its 32 x values in
// 16 VGPRs as fp16 pairs for every row it visits, so x is read once per
// wave while the weights stream from HBM with one or two 16-byte loads per
// lane per row (1 KiB contiguous per wave instruction).  Rows wider than
// 2048 columns are split over the waves of a workgroup (K-slices) and the
// partial sums meet in LDS.
//
// Decode: a code byte pair becomes an fp16 pair 1024 + q with v_perm_b32 +
// v_and_or_b32 (high-bit planes are rotated into bits 4/5 with
// v_alignbit_b32); v_dot2_f32_f16 multiplies by the fp16 x pair and
// accumulates in fp32.  The accumulator starts at -1024 * sum(x), so it
// ends at sum(q * x) exactly up to fp32 rounding.  Block scales follow the
// format: s = f32(f16(qs * d)) (sb6 also m = f32(f16(qm * dm)), s clamped at
// 1e-8), identical to the reference arithmetic
// (reference: rwkv_quant/formats/codec.py:183-257,
//             rwkv_quant/backends/metal/quant_linear_gw.py:491-557,
//             rwkv_quant/backends/metal/quant_linear_sym.py:107-247,
//             rwkv_quant/backends/metal/quant_linear_v2.py:35-84).
#include "rwkvq_common.h"
#include "rwkvq_hip.h"

using namespace rwkvq;

namespace {

enum Fmt { F_SB6_4 = 0, F_SB6_5 = 1, F_SB6_6 = 2, F_SYM6 = 3, F_SYM8 = 4,
           F_RTN8 = 5 };

struct GemvArgs {
  const uint8_t* q;      // nibble plane [rows, NG, 16] or int8 codes [rows, IN]
  const uint32_t* hb;    // high-bit words: sb6@5 [rows, NG], @6/sym6 [rows, NG, 2]
  const uint8_t* rec;    // sb6 superblock records [rows, NSB, 16]
  const int8_t* qs;      // sym block-scale codes [rows, IN/16]
  const uint16_t* d;     // sym: f16 d [rows, NSB]; rtn: f16 row scale [rows]
  const float* x;        // [N, n_seg, IN]
  float* y;              // [N, rows]
  int rows, in, out_per, n_seg, ks, rg, rpw, mode, n;
};

template <int FMT>
__device__ __forceinline__ void x_cols(int i, int& c0, int& c1) {
  if (FMT <= F_SB6_6) { c0 = i; c1 = i + 16; }
  else if (FMT == F_SYM6) { c0 = (i < 8) ? i : i + 8; c1 = c0 + 8; }
  else { c0 = 2 * i; c1 = 2 * i + 1; }
}

template <int FMT>
__device__ __forceinline__ float magic_bias() {
  if (FMT <= F_SB6_6) return 1024.0f;
  if (FMT == F_SYM6) return 1056.0f;    // 1024 + the +32 storage shift
  return 1152.0f;                       // 1024 + 128 (signed byte bias)
}

// Decode one (row, group) into 16 fp16 pairs.
template <int FMT>
__device__ __forceinline__ void decode_group(const GemvArgs& a, size_t row,
                                             int ng, int g, uint32_t h[16]) {
  if (FMT == F_SYM8 || FMT == F_RTN8) {
    const uint8_t* p = a.q + row * (size_t)a.in + (size_t)g * 32;
    uint4 u0 = ld16(p), u1 = ld16(p + 16);
    uint32_t w[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      h[2 * k] = i8_pair<0>(w[k]);
      h[2 * k + 1] = i8_pair<1>(w[k]);
    }
    return;
  }
  uint4 u = ld16(a.q + (row * ng + g) * 16);
  uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    uint32_t ws = w[k] >> 4;
    h[4 * k + 0] = nib_pair<0>(w[k], ws);
    h[4 * k + 1] = nib_pair<1>(w[k], ws);
    h[4 * k + 2] = nib_pair<2>(w[k], ws);
    h[4 * k + 3] = nib_pair<3>(w[k], ws);
  }
  if (FMT == F_SB6_5) {
    uint32_t hw = a.hb[row * ng + g];
#pragma unroll
    for (int i = 0; i < 16; ++i)
      h[i] |= __builtin_amdgcn_alignbit(hw, hw, (uint32_t)((i - 4) & 31)) &
              0x00100010u;
  } else if (FMT == F_SB6_6 || FMT == F_SYM6) {
    uint2 hw = *reinterpret_cast<const uint2*>(a.hb + (row * ng + g) * 2);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      uint32_t H = (i < 8) ? hw.x : hw.y;
      int ip = i & 7;
      h[i] |= __builtin_amdgcn_alignbit(H, H, (uint32_t)((2 * ip - 4) & 31)) &
              0x00300030u;
    }
  }
}

template <int FMT, int NN, int RS>
__global__ void __launch_bounds__(256)
gemv_kernel(GemvArgs a) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int kslice = wave % a.ks;
  const int rgi = wave / a.ks;
  const int ng = a.in >> 5;
  const int g = kslice * 64 + lane;
  const bool active = g < ng;
  const int row_base = (blockIdx.x * a.rg + rgi) * a.rpw;
  const int nsb = a.in >> 8;

  __shared__ float red[4 * 4 * RS * NN];   // [wave][RS*NN], waves <= 4*?
  // (max 16 waves of 64 = 1024 threads is not used; launch caps at 256)

  // ---- lane-resident x: 16 fp16 pairs per column + block sums
  int seg = row_base < a.rows ? row_base / a.out_per : 0;
  uint32_t xh[NN][16];
  float xsa[NN], xsb[NN], xsf[NN];
#pragma unroll
  for (int n = 0; n < NN; ++n) {
    float sa = 0.f, sb = 0.f, sf = 0.f;
    if (active && n < a.n) {
      const float* xp = a.x + ((size_t)n * a.n_seg + seg) * a.in + (size_t)g * 32;
      float xv[32];
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        float4 f = reinterpret_cast<const float4*>(xp)[t];
        xv[4 * t] = f.x; xv[4 * t + 1] = f.y; xv[4 * t + 2] = f.z; xv[4 * t + 3] = f.w;
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        int c0, c1;
        x_cols<FMT>(i, c0, c1);
        uint32_t p = pack_h2(xv[c0], xv[c1]);
        xh[n][i] = p;
        float s = h2_lo(p) + h2_hi(p);
        if (i < 8) sa += s; else sb += s;
      }
#pragma unroll
      for (int c = 0; c < 32; ++c) sf += xv[c];
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) xh[n][i] = 0u;
    }
    xsa[n] = sa; xsb[n] = sb; xsf[n] = sf;
  }

  // per-lane constants for sb6 scale extraction (block k of its superblock)
  const int kb = g & 7;
  const int qs_word = (6 * kb) >> 5, qs_sh = (6 * kb) & 31;
  const int qm_word = (48 + 6 * kb) >> 5, qm_sh = (48 + 6 * kb) & 31;
  const float mb = magic_bias<FMT>();

  for (int r0 = 0; r0 < a.rpw; r0 += RS) {
    float acc[NN][RS];
#pragma unroll
    for (int j = 0; j < RS; ++j) {
      const int row = row_base + r0 + j;
#pragma unroll
      for (int n = 0; n < NN; ++n) acc[n][j] = 0.f;
      if (!active || row >= a.rows) continue;
      uint32_t h[16];
      decode_group<FMT>(a, (size_t)row, ng, g, h);
      float dA[NN], dB[NN];
#pragma unroll
      for (int n = 0; n < NN; ++n) {
        float ca = -mb * xsa[n], cb = -mb * xsb[n];
#pragma unroll
        for (int i = 0; i < 8; ++i) ca = dot2(h[i], xh[n][i], ca);
#pragma unroll
        for (int i = 8; i < 16; ++i) cb = dot2(h[i], xh[n][i], cb);
        dA[n] = ca; dB[n] = cb;
      }
      if (FMT <= F_SB6_6) {
        uint4 rc = ld16(a.rec + ((size_t)row * nsb + (g >> 3)) * 16);
        uint32_t r[4] = {rc.x, rc.y, rc.z, rc.w};
        uint32_t lo = qs_word == 0 ? r[0] : r[1];
        uint32_t hi = qs_word == 0 ? r[1] : r[2];
        uint32_t qsv = __builtin_amdgcn_alignbit(hi, lo, (uint32_t)qs_sh) & 63u;
        lo = qm_word == 1 ? r[1] : r[2];
        hi = qm_word == 1 ? r[2] : r[3];
        uint32_t qmv = __builtin_amdgcn_alignbit(hi, lo, (uint32_t)qm_sh) & 63u;
        float d = f16_bits_to_f32(r[3] & 0xFFFFu);
        float dm = f16_bits_to_f32(r[3] >> 16);
        float s = fmaxf(f16_round((float)qsv * d), 1e-8f);
        float m = f16_round((float)((int)qmv - 31) * dm);
#pragma unroll
        for (int n = 0; n < NN; ++n) acc[n][j] = s * (dA[n] + dB[n]) + m * xsf[n];
      } else if (FMT == F_SYM6 || FMT == F_SYM8) {
        uint32_t q2 = *reinterpret_cast<const uint16_t*>(
            a.qs + (size_t)row * (a.in >> 4) + 2 * g);
        float d = f16_bits_to_f32(a.d[(size_t)row * nsb + (g >> 3)]);
        float sA = f16_round((float)(int8_t)(q2 & 0xFFu) * d);
        float sB = f16_round((float)(int8_t)(q2 >> 8) * d);
#pragma unroll
        for (int n = 0; n < NN; ++n) acc[n][j] = sA * dA[n] + sB * dB[n];
      } else {
#pragma unroll
        for (int n = 0; n < NN; ++n) acc[n][j] = dA[n] + dB[n];
      }
    }
    // ---- reduce over the 64 lanes, then over K-slices through LDS
#pragma unroll
    for (int n = 0; n < NN; ++n)
#pragma unroll
      for (int j = 0; j < RS; ++j) acc[n][j] = wave_sum(acc[n][j]);
    if (a.ks > 1) {
      if (lane == 0) {
#pragma unroll
        for (int n = 0; n < NN; ++n)
#pragma unroll
          for (int j = 0; j < RS; ++j) red[(wave * NN + n) * RS + j] = acc[n][j];
      }
      __syncthreads();
      if (kslice == 0) {
#pragma unroll
        for (int n = 0; n < NN; ++n)
#pragma unroll
          for (int j = 0; j < RS; ++j) {
            float s = 0.f;
            for (int k = 0; k < a.ks; ++k)
              s += red[((wave + k) * NN + n) * RS + j];
            acc[n][j] = s;
          }
      }
      __syncthreads();
    }
    if (kslice == 0 && lane < RS) {
#pragma unroll
      for (int j = 0; j < RS; ++j) {
        const int row = row_base + r0 + j;
        if (j != lane || row >= a.rows) continue;
#pragma unroll
        for (int n = 0; n < NN; ++n) {
          if (n >= a.n) continue;
          float v = acc[n][j];
          if (FMT == F_RTN8) v *= f16_bits_to_f32(a.d[row]);
          float* yp = a.y + (size_t)n * a.rows + row;
          switch (a.mode) {
            case RWKVQ_EPI_ADD: v += *yp; break;
            case RWKVQ_EPI_RELU2: v = v > 0.f ? v * v : 0.f; break;
            case RWKVQ_EPI_TANH: v = tanhf(v); break;
            case RWKVQ_EPI_SIGMOID: v = 1.f / (1.f + __expf(-v)); break;
            default: break;
          }
          *yp = v;
        }
      }
    }
  }
}

constexpr int kRS = 4;

template <int FMT, int NN>
void launch_nn(const GemvArgs& a, dim3 grid, dim3 block, hipStream_t s) {
  hipLaunchKernelGGL((gemv_kernel<FMT, NN, kRS>), grid, block, 0, s, a);
}

template <int FMT>
int launch_fmt(GemvArgs a, hipStream_t s) {
  const int ng = a.in / 32;
  a.ks = (ng + 63) / 64;
  if (a.ks > 4) return RWKVQ_ERR_SIZE;          // IN > 8192 not tiled here
  a.rg = 4 / a.ks;
  if (a.rg < 1) a.rg = 1;
  const int waves = a.ks * a.rg;
  // rows per wave: aim for >= 2048 waves in flight, at least kRS rows
  long rows_waves = (long)a.rows * a.ks;
  int rpw = (int)(rows_waves / 4096);
  rpw = rpw < kRS ? kRS : (rpw / kRS) * kRS;
  if (rpw > 32) rpw = 32;
  // a wave's rows share one x segment
  while (a.out_per % rpw) rpw -= kRS;
  if (rpw < kRS) return RWKVQ_ERR_ARG;
  a.rpw = rpw;
  const int rows_per_wg = a.rg * rpw;
  dim3 grid((a.rows + rows_per_wg - 1) / rows_per_wg);
  dim3 block(64 * waves);
  for (int n0 = 0; n0 < a.n; n0 += 4) {
    GemvArgs b = a;
    b.x = a.x + (size_t)n0 * a.n_seg * a.in;
    b.y = a.y + (size_t)n0 * a.rows;
    b.n = a.n - n0 < 4 ? a.n - n0 : 4;
    switch (b.n) {
      case 1: launch_nn<FMT, 1>(b, grid, block, s); break;
      case 2: launch_nn<FMT, 2>(b, grid, block, s); break;
      case 3: launch_nn<FMT, 3>(b, grid, block, s); break;
      default: launch_nn<FMT, 4>(b, grid, block, s); break;
    }
  }
  return hipGetLastError() == hipSuccess ? RWKVQ_OK : RWKVQ_ERR_LAUNCH;
}

int check_common(int rows, int in, int out_per, int n, int mode) {
  if (rows <= 0 || in <= 0 || n <= 0 || out_per <= 0) return RWKVQ_ERR_ARG;
  if (in % 256) return RWKVQ_ERR_ARG;
  if (rows % out_per || out_per % 4) return RWKVQ_ERR_ARG;
  if (mode < 0 || mode > RWKVQ_EPI_SIGMOID) return RWKVQ_ERR_ARG;
  return RWKVQ_OK;
}

}  // namespace

extern "C" {

int rwkvq_gemv_sb6(const uint8_t* nib, const uint32_t* hb, const uint8_t* rec,
                   int bits, int rows, int in, int out_per, const float* x,
                   float* y, int n, int mode, void* stream) {
  int st = check_common(rows, in, out_per, n, mode);
  if (st) return st;
  if (bits < 4 || bits > 6 || (bits > 4 && !hb)) return RWKVQ_ERR_ARG;
  GemvArgs a{};
  a.q = nib; a.hb = hb; a.rec = rec; a.x = x; a.y = y;
  a.rows = rows; a.in = in; a.out_per = out_per; a.n_seg = rows / out_per;
  a.mode = mode; a.n = n;
  hipStream_t s = (hipStream_t)stream;
  if (bits == 4) return launch_fmt<F_SB6_4>(a, s);
  if (bits == 5) return launch_fmt<F_SB6_5>(a, s);
  return launch_fmt<F_SB6_6>(a, s);
}

int rwkvq_gemv_sym(const uint8_t* codes, const uint32_t* hb, const int8_t* qs,
                   const uint16_t* d, int bits, int rows, int in, int out_per,
                   const float* x, float* y, int n, int mode, void* stream) {
  int st = check_common(rows, in, out_per, n, mode);
  if (st) return st;
  if ((bits != 6 && bits != 8) || (bits == 6 && !hb)) return RWKVQ_ERR_ARG;
  GemvArgs a{};
  a.q = codes; a.hb = hb; a.qs = qs; a.d = d; a.x = x; a.y = y;
  a.rows = rows; a.in = in; a.out_per = out_per; a.n_seg = rows / out_per;
  a.mode = mode; a.n = n;
  hipStream_t s = (hipStream_t)stream;
  return bits == 6 ? launch_fmt<F_SYM6>(a, s) : launch_fmt<F_SYM8>(a, s);
}

int rwkvq_gemv_rtn8(const int8_t* codes, const uint16_t* scale, int rows,
                    int in, int out_per, const float* x, float* y, int n,
                    int mode, void* stream) {
  int st = check_common(rows, in, out_per, n, mode);
  if (st) return st;
  GemvArgs a{};
  a.q = reinterpret_cast<const uint8_t*>(codes); a.d = scale; a.x = x; a.y = y;
  a.rows = rows; a.in = in; a.out_per = out_per; a.n_seg = rows / out_per;
  a.mode = mode; a.n = n;
  return launch_fmt<F_RTN8>(a, (hipStream_t)stream);
}

}  // extern "C"
