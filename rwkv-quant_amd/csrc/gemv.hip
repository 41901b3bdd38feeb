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
// v_alignbit_b32), and one packed fp16 subtraction (exact) leaves the
// signed integer codes.  x is staged per 32-column group as an fp16 hi +
// lo pair of x * 2^e (a power of two per group, so no fp16 range limit):
// two v_dot2_f32_f16 per code pair multiply the codes by hi and by lo with
// exact products and fp32 sums, so the block sums carry x to about 22 bits
// (fp32 x within the fp32 rounding of the sums).  The int8 formats (rtn8,
// sym8) and sb6@4 / @5 (unsigned codes) take x instead as three int8
// digits under the group's power of two (about 21 bits) and multiply the
// codes with exact int32 v_dot4_i32_i8: int8 codes as stored (rtn8 head
// 29.6 -> 28.3 us), sb6 nibbles masked into bytes with the fifth bit
// spread in (1.5B COMPRESSION decode 1.256 -> 1.185 ms).  Block scales follow the
// format: s = f32(f16(qs * d)) (sb6 also m = f32(f16(qm * dm)), s clamped at
// 1e-8), identical to the reference arithmetic
// (reference: rwkv_quant/formats/codec.py:183-257,
//             rwkv_quant/backends/metal/quant_linear_gw.py:491-557,
//             rwkv_quant/backends/metal/quant_linear_sym.py:107-247,
//             rwkv_quant/backends/metal/quant_linear_v2.py:35-84).
//
// One or two input rows take this lane-dot kernel; three or more take the
// matrix-core kernel further down (bgemv_kernel), which carries the
// format's fp32 weights and x each as fp16 hi + lo through the MFMAs.
#include "qfmt.h"
#include "rwkvq_hip.h"
#include "xdig.h"

using namespace rwkvq;

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

#ifndef RWKVQ_BG_NB2
#define RWKVQ_BG_NB2 1
#endif

namespace {

struct GemvArgs {
  const uint8_t* q;      // nibble plane [rows, NG, 16] or int8 codes [rows, IN]
  const uint32_t* hb;    // high-bit words: sb6@5 [rows, NG], @6/sym6 [rows, NG, 2]
  const uint8_t* rec;    // sb6 superblock records [rows, NSB, 16]
  const int8_t* qs;      // sym block-scale codes [rows, IN/16]
  const uint16_t* d;     // sym: f16 d [rows, NSB]; rtn: f16 row scale [rows]
  const float* x;        // x[n * x_ld + seg * IN + c]
  float* y;              // [N, rows]
  long x_ld;
  int rows, in, out_per, n_seg, ks, rg, rpw, mode, n;
  // segment table (matrix-core kernel, rwkvq_gemv_f16_seg): segment j
  // holds rows [seg_end[j-1], seg_end[j]), reads x at x + j * in and writes
  // seg_y[j] [n, rows of j]; 0 segments = uniform out_per segments
  int nseg_tab, seg_modes;
  int seg_end[8];
  float* seg_y[8];
  // matrix-core kernel, split-K across workgroups: `split` workgroups
  // share a row tile, each over its own K slices; partials go to ws,
  // cnt[tile] counts arrivals (the GEMMs' registered workspace)
  int split;
  float* ws;
  int* cnt;
  // lane-dot kernel, rtn8 with SpQR outliers: CSR per output row (row
  // pointers into columns / bf16 values); null without outliers
  const int* sp_ptr;
  const int* sp_col;
  const uint16_t* sp_val;
};

#ifndef RWKVQ_GEMV_I8DOT
#define RWKVQ_GEMV_I8DOT 1
#endif
#ifndef RWKVQ_GEMV_I8SB6
#define RWKVQ_GEMV_I8SB6 1
#endif
#ifndef RWKVQ_GEMV_I8SYM6
#define RWKVQ_GEMV_I8SYM6 1
#endif
// int8 codes (rtn8, sym8) and the 4- / 5-bit sb6 codes (unsigned, so they
// fit an int8 as they are) take x as three int8 digits instead of fp16
// hi + lo: the code products are then exact int32 dot products
// (v_dot4_i32_i8, four columns per instruction).
template <int FMT>
constexpr bool kI8 =
    RWKVQ_GEMV_I8DOT &&
    (FMT == F_RTN8 || FMT == F_SYM8 ||
     (RWKVQ_GEMV_I8SB6 && (FMT == F_SB6_4 || FMT == F_SB6_5)) ||
     (RWKVQ_GEMV_I8SYM6 && FMT == F_SYM6));

// Convert one lane's 32 x values of group g into the format's pair order
// as an fp16 hi + lo split of x * 2^e: hi = f16(x 2^e), lo = f16(x 2^e - hi),
// so hi + lo holds x to about 22 bits.  The power of two 2^e (exact) puts
// the group's largest |x| in [2^14, 2^15): no fp16 overflow whatever the
// range of x, and lo stays a normal fp16 down to 2^-17 of that maximum.
// dst: 16 hi pairs, then 16 lo pairs; sums: the fp32 sum of x (the sb6
// min term), 2^-e and 0.  int8-digit formats: the digit words of x_digits
// instead (hi = first and second digits, lo[0..7] = third) and the sums of
// columns 0..15 and 16..31.
template <int FMT, bool DIG = kI8<FMT>>
__device__ __forceinline__ void x_group_regs(const float* __restrict__ xp,
                                             uint32_t hi[16], uint32_t lo[16],
                                             float& sum, float& isc,
                                             float& sum_b) {
  float xv[32];
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    float4 f = reinterpret_cast<const float4*>(xp)[t];
    xv[4 * t] = f.x; xv[4 * t + 1] = f.y; xv[4 * t + 2] = f.z;
    xv[4 * t + 3] = f.w;
  }
  if constexpr (DIG) {
    uint32_t w[24];
    x_digits(xv, w, isc, sum, sum_b);
#pragma unroll
    for (int i = 0; i < 16; ++i) hi[i] = w[i];
#pragma unroll
    for (int i = 0; i < 8; ++i) { lo[i] = w[16 + i]; lo[8 + i] = 0u; }
    return;
  }
  float amax = 0.f, sf = 0.f;
#pragma unroll
  for (int c = 0; c < 32; ++c) {
    amax = fmaxf(amax, fabsf(xv[c]));
    sf += xv[c];
  }
  // inf / nan (amax not finite) keep e = 0 and propagate through the dot
  int e = 0;
  if (amax > 0.f && amax <= 3.0e38f) e = min(14 - ilogbf(amax), 100);
  const float sc = ldexpf(1.f, e);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    int c0, c1;
    x_cols<FMT>(i, c0, c1);
    const float a0 = xv[c0] * sc, a1 = xv[c1] * sc;
    hi[i] = pack_h2(a0, a1);
    lo[i] = pack_h2(a0 - h2_lo(hi[i]), a1 - h2_hi(hi[i]));
  }
  sum = sf;
  sum_b = 0.f;
  isc = ldexpf(1.f, -e);
}

template <int FMT>
__device__ __forceinline__ void x_group(const float* __restrict__ xp,
                                        uint32_t* __restrict__ dst,
                                        float* __restrict__ sums) {
  uint32_t hi[16], lo[16];
  x_group_regs<FMT, false>(xp, hi, lo, sums[0], sums[1], sums[2]);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    reinterpret_cast<uint4*>(dst)[q] =
        make_uint4(hi[4 * q], hi[4 * q + 1], hi[4 * q + 2], hi[4 * q + 3]);
    reinterpret_cast<uint4*>(dst)[4 + q] =
        make_uint4(lo[4 * q], lo[4 * q + 1], lo[4 * q + 2], lo[4 * q + 3]);
  }
}

constexpr int kXWords = 32;   // staged words per (input row, group)
constexpr int kXSums = 3;     // staged floats per (input row, group):
                              // sum (cols 0..15 or all), 2^-e, sum 16..31

// ILV: interleaved row order (the heads); otherwise blocked rows.  The
// sb6 codes are read with non-temporal loads (1.5B COMPRESSION decode
// B = 1 1.213 -> 1.169 ms for the blocked rows, the sb6@5 head included
// 1.118 ms); for the sym / rtn formats (the rtn8 head 28.1 -> 31.6 us) and
// the batched kernel they were slower (measured).
// XD: x loaded and converted per lane (no LDS staging, no barrier) --
// faster for rows wider than a wave's 2048-column slice, where every
// workgroup would otherwise stage the whole row (measured: 8192-wide sym6
// 9.8 -> 9.4 us; slower for 2048-wide rows and the heads).
template <int FMT, int NN, int RS, bool ILV = false,
          bool NT = FMT <= F_SB6_6, bool XD = false>
__global__ void __launch_bounds__(512)
gemv_kernel(GemvArgs a) {
  const int lane = threadIdx.x & 63;
  // wave-uniform values live in SGPRs: row addressing becomes scalar and
  // only the lane's group offset is a VGPR
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kslice = wave % a.ks;
  const int rgi = wave / a.ks;
  const int ng = a.in >> 5;
  const int g = kslice * 64 + lane;
  const bool active = g < ng;
  const int gl = active ? g : 0;               // in-bounds group for loads
  const int wg_row0 = blockIdx.x * a.rg * a.rpw;
  const int row_base = wg_row0 + rgi * a.rpw;
  const int nsb = a.in >> 8;

  // x of this workgroup's segment, staged once per workgroup as fp16
  // hi / lo pairs [NN][ng][32] followed by the sums [NN][ng][2] (dynamic LDS)
  extern __shared__ uint32_t smem[];
  uint32_t* s_xh = smem;
  float* s_xs = reinterpret_cast<float*>(smem + NN * ng * kXWords);
  __shared__ float red[8 * RS * NN];

  // first weight batch in flight before x is fetched: the two memory round
  // trips overlap.  Loads are unconditional (row index clamped into the
  // matrix) so the compiler can count them and wait only for the batch it
  // consumes.
  const int nrows = min(a.rpw, a.rows - row_base);   // rows of this wave
  // loads past the wave's own rows are clamped to its last row (an L2 hit
  // of data it has just read) rather than to the matrix's last row: the
  // rows after them belong to another wave, possibly on another XCD, and
  // reading them there costs a second HBM fetch
  const int last = max(min(row_base + a.rpw, a.rows) - 1, 0);
  // interleaved order (one segment, grid covering the rows exactly): batch
  // b of row-wave w holds rows b * bstride + w * RS + j, so that at any
  // moment the grid's waves stream one contiguous stretch of the matrix
  // instead of points a whole wave's share (rpw rows) apart
  const int wrow = blockIdx.x * a.rg + rgi;
  const int bstride = gridDim.x * a.rg * RS;
  auto row_of = [&](int r) {
    return ILV ? (r / RS) * bstride + wrow * RS + r % RS : row_base + r;
  };
  Raw cur[RS], nxt[RS];
#pragma unroll
  for (int j = 0; j < RS; ++j)
    load_raw<FMT, NT>(a, ILV ? row_of(j) : min(row_base + j, last), ng,
                        nsb, gl, cur[j]);

  const int seg = !ILV && wg_row0 < a.rows ? wg_row0 / a.out_per : 0;
  // the int8-digit products for one or two input rows (more rows would not
  // fit the registers) with x staged in LDS: converted per lane (XD), the
  // digits cost more than they save (8192-wide sym6 value GEMV 9.4 -> 10.7
  // us; 1.5B sb6 decode 1.190 ms with hi + lo there, 1.202 ms with digits)
  constexpr bool kDig = kI8<FMT> && NN <= 2 && !XD;
  uint32_t xh[NN][16], xl[NN][16];
  float xsf[NN], xsc[NN], xsb[NN];
  if constexpr (XD) {
  // each lane converts its own group of x straight from global memory
  // (L2 after the first wave): no LDS round trip, no barrier before the
  // first row
#pragma unroll
  for (int n = 0; n < NN; ++n) {
    if (n < a.n) {
      x_group_regs<FMT, kDig>(a.x + (size_t)n * a.x_ld + (size_t)seg * a.in +
                            (size_t)gl * 32,
                        xh[n], xl[n], xsf[n], xsc[n], xsb[n]);
      if constexpr (!kDig) xsb[n] = 0.f;
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) xh[n][i] = xl[n][i] = 0u;
      xsf[n] = 0.f;
      xsc[n] = 1.f;
      xsb[n] = 0.f;
    }
  }
  } else {
  if constexpr (kDig) {
    // digits: 8 threads per (input row, group), 4 columns each; the
    // group's largest |x| through three butterflies over those 8 lanes
    for (int it = threadIdx.x; it < NN * ng * 8; it += blockDim.x) {
      const int item = it >> 3, k = it & 7;
      const int n = item / ng, gg = item % ng;
      float4 f = make_float4(0.f, 0.f, 0.f, 0.f);
      if (n < a.n)
        f = reinterpret_cast<const float4*>(
            a.x + (size_t)n * a.x_ld + (size_t)seg * a.in + (size_t)gg * 32)[k];
      const float xv4[4] = {f.x, f.y, f.z, f.w};
      float amax = fmaxf(fmaxf(fabsf(f.x), fabsf(f.y)),
                         fmaxf(fabsf(f.z), fabsf(f.w)));
      int bad = !(fabsf(f.x) <= 3.4e38f) | !(fabsf(f.y) <= 3.4e38f) |
                !(fabsf(f.z) <= 3.4e38f) | !(fabsf(f.w) <= 3.4e38f);
      float sf = (f.x + f.y) + (f.z + f.w);
#pragma unroll
      for (int m = 1; m < 8; m <<= 1) {
        amax = fmaxf(amax, __shfl_xor(amax, m, 64));
        bad |= __shfl_xor(bad, m, 64);
        if (m < 4) sf += __shfl_xor(sf, m, 64);   // sum of the half
      }
      const int e = digit_exp(amax);
      uint32_t w0 = 0u, w1 = 0u, w2 = 0u;
#pragma unroll
      for (int bb = 0; bb < 4; ++bb) {
        uint32_t b0, b1, b2;
        x_digit3(bad ? 0.f : xv4[bb], e, b0, b1, b2);
        w0 |= b0 << (8 * bb);
        w1 |= b1 << (8 * bb);
        w2 |= b2 << (8 * bb);
      }
      uint32_t* dst = s_xh + (size_t)item * kXWords;
      dst[k] = w0;
      dst[8 + k] = w1;
      dst[16 + k] = w2;
      if (k == 0) {
        s_xs[item * kXSums] = sf;
        s_xs[item * kXSums + 1] = bad ? __builtin_nanf("") : ldexpf(1.f, -e);
      }
      if (k == 4) s_xs[item * kXSums + 2] = sf;
    }
  } else {
  for (int item = threadIdx.x; item < NN * ng; item += blockDim.x) {
    const int n = item / ng, gg = item % ng;
    if (n < a.n) {
      x_group<FMT>(a.x + (size_t)n * a.x_ld + (size_t)seg * a.in +
                       (size_t)gg * 32,
                   s_xh + (size_t)item * kXWords,
                   s_xs + (size_t)item * kXSums);
    } else {
#pragma unroll
      for (int q = 0; q < kXWords; ++q) s_xh[(size_t)item * kXWords + q] = 0u;
      s_xs[item * kXSums] = 0.f;
      s_xs[item * kXSums + 1] = 1.f;
      s_xs[item * kXSums + 2] = 0.f;
    }
  }
  }
  __syncthreads();
#pragma unroll
  for (int n = 0; n < NN; ++n) {
    const uint4* src =
        reinterpret_cast<const uint4*>(s_xh + (n * ng + gl) * kXWords);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint4 v = src[q];
      xh[n][4 * q] = v.x; xh[n][4 * q + 1] = v.y;
      xh[n][4 * q + 2] = v.z; xh[n][4 * q + 3] = v.w;
      v = src[4 + q];
      xl[n][4 * q] = v.x; xl[n][4 * q + 1] = v.y;
      xl[n][4 * q + 2] = v.z; xl[n][4 * q + 3] = v.w;
    }
    xsf[n] = s_xs[(n * ng + gl) * kXSums];
    xsc[n] = s_xs[(n * ng + gl) * kXSums + 1];
    xsb[n] = kDig ? s_xs[(n * ng + gl) * kXSums + 2] : 0.f;
  }
  }
  // sym6: the digits once more in the order of the crumb words, whose
  // (W >> 2t) & 0x03030303 holds the high bits of columns t, 4 + t, 8 + t,
  // 12 + t of a 16-column half: xc[8 d + 4 h + t] (digit d, half h)
  constexpr bool kCrumbDot = kDig && FMT == F_SYM6;
  uint32_t xc[NN][kCrumbDot ? 24 : 1];
  if constexpr (kCrumbDot) {
#pragma unroll
    for (int n = 0; n < NN; ++n)
#pragma unroll
      for (int d = 0; d < 3; ++d)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const uint32_t* src = d < 2 ? &xh[n][8 * d + 4 * hh] : &xl[n][4 * hh];
          byte_transpose4(src[0], src[1], src[2], src[3], &xc[n][8 * d + 4 * hh]);
        }
  }
  // the decoder's fp16 pairs hold 1024 + code (+ the storage bias):
  // subtracting it in fp16 is exact and leaves the signed integer codes
  const _Float16 mbh = (_Float16)magic_bias<FMT>();
  const h2_t bias2 = {mbh, mbh};

  // per-lane constants for sb6 scale extraction (block k of its superblock)
  const int kb = g & 7;
  const int qs_word = (6 * kb) >> 5, qs_sh = (6 * kb) & 31;
  const int qm_word = (48 + 6 * kb) >> 5, qm_sh = (48 + 6 * kb) & 31;


  for (int r0 = 0; r0 < a.rpw; r0 += RS) {
    // prefetch the next batch before touching this one
#pragma unroll
    for (int j = 0; j < RS; ++j)
      load_raw<FMT, NT>(a,
                    !ILV ? min(row_base + r0 + RS + j, last)
                    : r0 + RS < a.rpw ? row_of(r0 + RS + j) : row_of(a.rpw - 1),
                    ng, nsb, gl, nxt[j]);

    float acc[NN][RS];
#pragma unroll
    for (int j = 0; j < RS; ++j) {
      float dA[NN], dB[NN];
      if constexpr (kDig) {
      // block sums of code * digit: exact int32 dot products, three digits
      // per 4 columns.  int8 formats: the stored codes as they are; sb6:
      // byte j of the nibble plane holds columns j (low nibble) and j + 16
      // (high), so masking gives columns 0..15 and 16..31 in order, and the
      // fifth bits (bit c of the group's word = column c) are spread in
      uint32_t cw[8];
      if constexpr (FMT == F_SYM6) {
        // byte i of the nibble plane holds columns (i, i + 8) for i < 8 and
        // (i + 8, i + 16) from 8 on: low nibbles of bytes 0..3 / 4..7 are
        // columns 0..3 / 4..7, their high nibbles 8..11 / 12..15, and the
        // same for bytes 8..15 and columns 16..31
        const uint32_t nw[4] = {cur[j].a.x, cur[j].a.y, cur[j].a.z, cur[j].a.w};
        cw[0] = nw[0] & 0x0F0F0F0Fu;         cw[1] = nw[1] & 0x0F0F0F0Fu;
        cw[2] = (nw[0] >> 4) & 0x0F0F0F0Fu;  cw[3] = (nw[1] >> 4) & 0x0F0F0F0Fu;
        cw[4] = nw[2] & 0x0F0F0F0Fu;         cw[5] = nw[3] & 0x0F0F0F0Fu;
        cw[6] = (nw[2] >> 4) & 0x0F0F0F0Fu;  cw[7] = (nw[3] >> 4) & 0x0F0F0F0Fu;
      } else if constexpr (FMT == F_RTN8 || FMT == F_SYM8) {
        cw[0] = cur[j].a.x; cw[1] = cur[j].a.y; cw[2] = cur[j].a.z;
        cw[3] = cur[j].a.w; cw[4] = cur[j].b.x; cw[5] = cur[j].b.y;
        cw[6] = cur[j].b.z; cw[7] = cur[j].b.w;
      } else {
        const uint32_t nw[4] = {cur[j].a.x, cur[j].a.y, cur[j].a.z, cur[j].a.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          cw[k] = nw[k] & 0x0F0F0F0Fu;
          cw[4 + k] = (nw[k] >> 4) & 0x0F0F0F0Fu;
          if constexpr (FMT == F_SB6_5) {
            const uint32_t H = cur[j].h.x;
            cw[k] |= spread4((H >> (4 * k)) & 15u) << 4;
            cw[4 + k] |= spread4((H >> (16 + 4 * k)) & 15u) << 4;
          }
        }
      }
#pragma unroll
      for (int n = 0; n < NN; ++n) {
        int a0 = 0, a1 = 0, a2 = 0, b0 = 0, b1 = 0, b2 = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          a0 = __builtin_amdgcn_sdot4((int)cw[k], (int)xh[n][k], a0, false);
          a1 = __builtin_amdgcn_sdot4((int)cw[k], (int)xh[n][8 + k], a1, false);
          a2 = __builtin_amdgcn_sdot4((int)cw[k], (int)xl[n][k], a2, false);
          b0 = __builtin_amdgcn_sdot4((int)cw[4 + k], (int)xh[n][4 + k], b0, false);
          b1 = __builtin_amdgcn_sdot4((int)cw[4 + k], (int)xh[n][12 + k], b1, false);
          b2 = __builtin_amdgcn_sdot4((int)cw[4 + k], (int)xl[n][4 + k], b2, false);
        }
        if constexpr (kCrumbDot) {
          // stored code u = nibble + 16 crumb = q + 32
          const uint32_t W0 = cur[j].h.x, W1 = cur[j].h.y;
          int ca0 = 0, ca1 = 0, ca2 = 0, cb0 = 0, cb1 = 0, cb2 = 0;
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const int c0 = (int)((W0 >> (2 * t)) & 0x03030303u);
            const int c1 = (int)((W1 >> (2 * t)) & 0x03030303u);
            ca0 = __builtin_amdgcn_sdot4(c0, (int)xc[n][t], ca0, false);
            ca1 = __builtin_amdgcn_sdot4(c0, (int)xc[n][8 + t], ca1, false);
            ca2 = __builtin_amdgcn_sdot4(c0, (int)xc[n][16 + t], ca2, false);
            cb0 = __builtin_amdgcn_sdot4(c1, (int)xc[n][4 + t], cb0, false);
            cb1 = __builtin_amdgcn_sdot4(c1, (int)xc[n][12 + t], cb1, false);
            cb2 = __builtin_amdgcn_sdot4(c1, (int)xc[n][20 + t], cb2, false);
          }
          a0 += ca0 << 4; a1 += ca1 << 4; a2 += ca2 << 4;
          b0 += cb0 << 4; b1 += cb1 << 4; b2 += cb2 << 4;
          dA[n] = digit_sum(a0, a1, a2) * xsc[n] - 32.f * xsf[n];
          dB[n] = digit_sum(b0, b1, b2) * xsc[n] - 32.f * xsb[n];
        } else {
        dA[n] = digit_sum(a0, a1, a2) * xsc[n];
        dB[n] = digit_sum(b0, b1, b2) * xsc[n];
        }
      }
      } else {
      uint32_t h[16];
      decode_raw<FMT>(cur[j], h);
#pragma unroll
      for (int i = 0; i < 16; ++i) h[i] = h2_bits(as_h2(h[i]) - bias2);
      // block sums of code * x (scaled by 2^e): the products are exact in
      // fp32, four independent chains
#pragma unroll
      for (int n = 0; n < NN; ++n) {
        float ah = 0.f, al = 0.f, bh = 0.f, bl = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          ah = dot2(h[i], xh[n][i], ah);
          al = dot2(h[i], xl[n][i], al);
        }
#pragma unroll
        for (int i = 8; i < 16; ++i) {
          bh = dot2(h[i], xh[n][i], bh);
          bl = dot2(h[i], xl[n][i], bl);
        }
        dA[n] = (ah + al) * xsc[n];
        dB[n] = (bh + bl) * xsc[n];
      }
      }
      if (FMT <= F_SB6_6) {
        const uint32_t rr[4] = {cur[j].b.x, cur[j].b.y, cur[j].b.z,
                                cur[j].b.w};
        uint32_t lo = qs_word == 0 ? rr[0] : rr[1];
        uint32_t hi = qs_word == 0 ? rr[1] : rr[2];
        uint32_t qsv = __builtin_amdgcn_alignbit(hi, lo, (uint32_t)qs_sh) & 63u;
        lo = qm_word == 1 ? rr[1] : rr[2];
        hi = qm_word == 1 ? rr[2] : rr[3];
        uint32_t qmv = __builtin_amdgcn_alignbit(hi, lo, (uint32_t)qm_sh) & 63u;
        float d = f16_bits_to_f32(rr[3] & 0xFFFFu);
        float dm = f16_bits_to_f32(rr[3] >> 16);
        float s = fmaxf(f16_round((float)qsv * d), 1e-8f);
        float m = f16_round((float)((int)qmv - 31) * dm);
#pragma unroll
        for (int n = 0; n < NN; ++n)
          acc[n][j] = active ? s * (dA[n] + dB[n]) + m * (xsf[n] + xsb[n])
                             : 0.f;
      } else if (FMT == F_SYM6 || FMT == F_SYM8) {
        float d = f16_bits_to_f32(cur[j].dd);
        float sA = f16_round((float)(int8_t)(cur[j].s & 0xFFu) * d);
        float sB = f16_round((float)(int8_t)((cur[j].s >> 8) & 0xFFu) * d);
#pragma unroll
        for (int n = 0; n < NN; ++n)
          acc[n][j] = active ? sA * dA[n] + sB * dB[n] : 0.f;
      } else {
#pragma unroll
        for (int n = 0; n < NN; ++n) acc[n][j] = active ? dA[n] + dB[n] : 0.f;
      }
    }
    // ---- reduce over the 64 lanes (uniform result), then K-slices in LDS
#pragma unroll
    for (int n = 0; n < NN; ++n)
#pragma unroll
      for (int j = 0; j < RS; ++j) acc[n][j] = wave_sum_dpp(acc[n][j]);
    // SpQR tail of the int8 rows (after the row scale): the row's outliers
    // strided over the lanes of K-slice 0, x read in fp32
    float osum[NN][RS];
#pragma unroll
    for (int n = 0; n < NN; ++n)
#pragma unroll
      for (int j = 0; j < RS; ++j) osum[n][j] = 0.f;
    if (FMT == F_RTN8 && a.sp_ptr && kslice == 0) {
#pragma unroll
      for (int j = 0; j < RS; ++j) {
        const int row = row_of(r0 + j);
        const bool live = r0 + j < nrows;
        const int k0 = live ? a.sp_ptr[row] : 0;
        const int k1 = live ? a.sp_ptr[row + 1] : 0;
        for (int k = k0 + lane; k < k1; k += 64) {
          const int c = a.sp_col[k];
          const float val = __builtin_bit_cast(
              float, (uint32_t)a.sp_val[k] << 16);
#pragma unroll
          for (int n = 0; n < NN; ++n)
            if (n < a.n)
              osum[n][j] += val * a.x[(size_t)n * a.x_ld +
                                      (size_t)seg * a.in + c];
        }
#pragma unroll
        for (int n = 0; n < NN; ++n) osum[n][j] = wave_sum_dpp(osum[n][j]);
      }
    }
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
            float s2 = 0.f;
            for (int k = 0; k < a.ks; ++k)
              s2 += red[((wave + k) * NN + n) * RS + j];
            acc[n][j] = s2;
          }
      }
      __syncthreads();
    }
    if (kslice == 0 && lane < RS * NN) {
      // lane (n * RS + j) writes row r0 + j of column n
#pragma unroll
      for (int n = 0; n < NN; ++n)
#pragma unroll
        for (int j = 0; j < RS; ++j) {
          const int row = row_of(r0 + j);
          if (lane != n * RS + j || n >= a.n || r0 + j >= nrows) continue;
          float v = acc[n][j];
          if (FMT == F_RTN8) v = v * f16_bits_to_f32(a.d[row]) + osum[n][j];
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
#pragma unroll
    for (int j = 0; j < RS; ++j) cur[j] = nxt[j];
  }
}

// ---------------------------------------------------------------------------
// Small batches (2..16 input rows per launch) on the matrix cores.
//
// v_mfma_f32_16x16x32_f16 with A = W (16 weight rows x 32 k) and B = x^T
// (32 k x 16 input rows): lane l = i + 16 q holds A[i][8 q + e] and
// B[8 q + e][i] (e = 0..7) and receives D[4 q + v][i] (v = 0..3).  In a
// 128-column step, quarter q of the wave decodes group 4 s + q of weight
// row i into the fp16 weights the format's dequant rounds to (the values
// the reference's batched path multiplies,
// reference: rwkv_quant/backends/metal/quant_linear_gw.py:821-849,
//            rwkv_quant/backends/metal/quant_linear_sym.py:433-484) and
// loads the 32 x values of that group for input row i; both go in the
// decoder's pair order, and MFMA j of the step takes pairs 4j..4j+3 of
// every quarter, so the four MFMAs of a step sum the 128 columns exactly
// once.  The k-reduction happens inside the matrix core: no lane
// reductions, and the batch costs one B operand per step instead of one
// dot product per input row.
//
// Workgroup = `ks` waves = ks slices of K over the same 16 * RT weight rows;
// a wave runs `rpw` consecutive steps of its slice, with the weights (HBM)
// and x (L2) of step s + 1 loaded before the MFMAs of step s.  The slices
// meet in LDS in a fixed order (deterministic); each output element
// depends only on its own input row, so a row's result does not depend on
// the other rows of the batch.
// NB blocks of 16 input rows share each decoded weight fragment (NB = 2:
// batches of 17..32 rows in one pass over the weights).
template <int FMT, int RT, int NS, int KSMAX, int NB = 1>
__global__ void __launch_bounds__(64 * KSMAX)
bgemv_kernel(GemvArgs a) {
  using RawT = typename RawOf<FMT>::T;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int i = lane & 15, q = lane >> 4;
  const int ng = a.in >> 5, nsb = a.in >> 8;
  const int tile = blockIdx.x / a.split, sp = blockIdx.x % a.split;
  const int row0 = tile * 16 * RT;
  // segment of this tile: uniform out_per, or the table (constant-index
  // reads and value selects only)
  int seg = row0 / a.out_per, s_lo = 0;
  float* s_y = a.y;
  if (a.nseg_tab > 0) {
    seg = 0;
    s_y = a.seg_y[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) {
      const bool past = j < a.nseg_tab && row0 >= a.seg_end[j - 1];
      seg = past ? j : seg;
      s_lo = past ? a.seg_end[j - 1] : s_lo;
      s_y = past ? a.seg_y[j] : s_y;
    }
  }
  // first group of the wave's K slice (slices of all split workgroups of
  // the tile in order)
  const int gw = (sp * a.ks + wave) * a.rpw * 4;
  bool xon[NB];
  const float* xr[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    xon[b] = i + 16 * b < a.n;
    xr[b] = a.x + (size_t)(xon[b] ? i + 16 * b : 0) * a.x_ld +
            (size_t)seg * a.in + q * 32;
  }

  auto load_w = [&](int g, RawT (&dst)[RT]) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
      load_raw<FMT, false>(a, row0 + 16 * rt + i, ng, nsb, g, dst[rt]);
  };
  // unconditional loads (lanes past the batch read input row 0 and zero
  // their B operand later): no branches, so the compiler's load counting
  // stays exact and a wait covers only the step it feeds
  auto load_x = [&](int g0, float4 (&dst)[NB][8]) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float4* p =
          reinterpret_cast<const float4*>(xr[b] + (size_t)g0 * 32);
#pragma unroll
      for (int t = 0; t < 8; ++t) dst[b][t] = p[t];
    }
  };

  f32x4_t acc[NB][RT];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) acc[b][rt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // One 128-column step: x of the step (per input row, scaled by a power of
  // two that puts its largest |x| in [2^14, 2^15), so fp16 cannot
  // overflow) and the weights, each as fp16 hi + lo; per sub-step the
  // products hi.hi + hi.lo + lo.hi go through the matrix core (lo.lo,
  // below 2^-22 of the product, is dropped), the step's sum is unscaled
  // and added to the fp32 accumulator.
#ifndef RWKVQ_BG_WLO
#define RWKVQ_BG_WLO 1
#endif
  constexpr bool kWLo = RWKVQ_BG_WLO && FMT != F_RTN8 && FMT != F_F16;
  auto mma_step = [&](int st, RawT (&w_raw)[RT], float4 (&xv)[NB][8]) {
    half8_t bh[NB][4], bl[NB][4];
    float isc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      float amax = 0.f;
#pragma unroll
      for (int t = 0; t < 8; ++t)
        amax = fmaxf(fmaxf(fmaxf(amax, fabsf(xv[b][t].x)), fabsf(xv[b][t].y)),
                     fmaxf(fabsf(xv[b][t].z), fabsf(xv[b][t].w)));
      // the step's four groups of input row i sit in lanes i + 16 q
      amax = fmaxf(amax, __shfl_xor(amax, 16));
      amax = fmaxf(amax, __shfl_xor(amax, 32));
      int e = 0;
      if (amax > 0.f && amax <= 3.0e38f) e = min(14 - ilogbf(amax), 100);
      const float sc = ldexpf(1.f, e);
      isc[b] = ldexpf(1.f, -e);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        int ca, cb;
        step_cols<FMT>(j, ca, cb);
        float4 A = xv[b][ca >> 2], B = xv[b][cb >> 2];
        A.x *= sc; A.y *= sc; A.z *= sc; A.w *= sc;
        B.x *= sc; B.y *= sc; B.z *= sc; B.w *= sc;
        const float4 Ah = make_float4(f16_round(A.x), f16_round(A.y),
                                      f16_round(A.z), f16_round(A.w));
        const float4 Bh = make_float4(f16_round(B.x), f16_round(B.y),
                                      f16_round(B.z), f16_round(B.w));
        uint4 xh = x_pairs<FMT>(Ah, Bh);
        uint4 xl = x_pairs<FMT>(
            make_float4(A.x - Ah.x, A.y - Ah.y, A.z - Ah.z, A.w - Ah.w),
            make_float4(B.x - Bh.x, B.y - Bh.y, B.z - Bh.z, B.w - Bh.w));
        if (!xon[b]) xh = xl = make_uint4(0u, 0u, 0u, 0u);
        bh[b][j] = __builtin_bit_cast(half8_t, xh);
        bl[b][j] = __builtin_bit_cast(half8_t, xl);
      }
    }
    const int kb = (gw + 4 * st + q) & 7;   // group within its superblock
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      uint32_t wh[16], wl[16];
      if (kWLo || FMT == F_RTN8 || FMT == F_F16) {
        dequant_group_hilo<FMT>(w_raw[rt], kb, wh, wl);
      } else {                 // fp16 weights (the format's one rounding)
        dequant_group<FMT>(w_raw[rt], kb, wh);
#pragma unroll
        for (int i = 0; i < 16; ++i) wl[i] = 0u;
      }
      f32x4_t d[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) d[b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const half8_t ah = __builtin_bit_cast(
            half8_t, make_uint4(wh[4 * j], wh[4 * j + 1], wh[4 * j + 2],
                                wh[4 * j + 3]));
        const half8_t al = __builtin_bit_cast(
            half8_t, make_uint4(wl[4 * j], wl[4 * j + 1], wl[4 * j + 2],
                                wl[4 * j + 3]));
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          d[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh[b][j], d[b],
                                                        0, 0, 0);
          d[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl[b][j], d[b],
                                                        0, 0, 0);
          if (kWLo)
            d[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh[b][j], d[b],
                                                          0, 0, 0);
        }
      }
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[b][rt][v] += d[b][v] * isc[b];
    }
  };

  if (NS == 2) {
    // both steps' loads in flight at once
    RawT wa[RT], wb[RT];
    float4 xa[NB][8], xb[NB][8];
    load_w(gw + q, wa);
    load_x(gw, xa);
    load_w(gw + 4 + q, wb);
    load_x(gw + 4, xb);
    // keep the second step's loads ahead of the first step's MFMAs: left
    // to itself the scheduler sinks them next to their use
    __builtin_amdgcn_sched_barrier(0);
    mma_step(0, wa, xa);
    __builtin_amdgcn_sched_barrier(0);
    mma_step(1, wb, xb);
  } else if (NS > 2) {
    // straight-line: step s + 1 loads while step s multiplies, in two
    // register sets (compile-time indices, no copies)
    RawT w2[2][RT];
    float4 x2[2][NB][8];
    load_w(gw + q, w2[0]);
    load_x(gw, x2[0]);
#pragma unroll
    for (int st = 0; st < NS; ++st) {
      if (st + 1 < NS) {
        load_w(gw + 4 * (st + 1) + q, w2[(st + 1) & 1]);
        load_x(gw + 4 * (st + 1), x2[(st + 1) & 1]);
      }
      __builtin_amdgcn_sched_barrier(0);
      mma_step(st, w2[st & 1], x2[st & 1]);
      __builtin_amdgcn_sched_barrier(0);
    }
  } else {
    // any step count: the same two register sets in a loop.  Loads past
    // the slice's last step are clamped to it (L2 hits, never used).
    RawT wa[RT], wb[RT];
    float4 xa[NB][8], xb[NB][8];
    const int last = a.rpw - 1;
    load_w(gw + q, wa);
    load_x(gw, xa);
    for (int st = 0; st < a.rpw; st += 2) {
      load_w(gw + 4 * min(st + 1, last) + q, wb);
      load_x(gw + 4 * min(st + 1, last), xb);
      __builtin_amdgcn_sched_barrier(0);
      mma_step(st, wa, xa);
      __builtin_amdgcn_sched_barrier(0);
      if (st + 1 > last) break;
      load_w(gw + 4 * min(st + 2, last) + q, wa);
      load_x(gw + 4 * min(st + 2, last), xa);
      __builtin_amdgcn_sched_barrier(0);
      mma_step(st + 1, wb, xb);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // ---- K slices meet in LDS: red[wave][b][rt][v][lane]
  __shared__ float red[KSMAX * NB * RT * 256];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        red[((wave * NB + b) * RT + rt) * 256 + v * 64 + lane] = acc[b][rt][v];
  __syncthreads();
  constexpr int kRows = 16 * RT;
  const int mode = a.mode == RWKVQ_EPI_PER_SEG ? (a.seg_modes >> (4 * seg)) & 15
                                               : a.mode;
  int seg_hi = a.rows;
  if (a.nseg_tab > 0) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      seg_hi = j == seg ? a.seg_end[j] : seg_hi;
  }
  auto slice_sum = [&](int idx) {
    const int n = idx / kRows, r = idx % kRows;
    const int e = ((n >> 4) * RT + (r >> 4)) * 256 + (r & 3) * 64 + (n & 15) +
                  16 * ((r & 15) >> 2);
    float v = 0.f;
    for (int k = 0; k < a.ks; ++k) v += red[k * NB * RT * 256 + e];
    return v;
  };
  constexpr int TE = kRows * 16 * NB;        // outputs of a row tile
  if (a.split > 1) {
    // Every workgroup stores its partial sums and counts itself in; the
    // last to arrive adds the partials in split order 0, 1, ... (the same
    // sum whichever finishes last), applies the epilogue and re-arms the
    // counter.  Agent-scope relaxed atomics are coherent across the XCDs'
    // L2s without a cache flush.
    float* part = a.ws + (size_t)tile * a.split * TE;
    for (int idx = threadIdx.x; idx < TE; idx += a.ks * 64) {
      if (idx / kRows >= a.n) break;
      __hip_atomic_store(part + (size_t)sp * TE + idx, slice_sum(idx),
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __shared__ int s_last;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0)
      s_last = __hip_atomic_fetch_add(a.cnt + tile, 1, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT) ==
               a.split - 1;
    __syncthreads();
    if (!s_last) return;
    if (threadIdx.x == 0)
      __hip_atomic_store(a.cnt + tile, 0, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }
  for (int idx = threadIdx.x; idx < kRows * 16 * NB; idx += a.ks * 64) {
    const int n = idx / kRows, r = idx % kRows;   // rows fastest: coalesced
    if (n >= a.n) break;
    float v;
    if (a.split > 1) {
      const float* part = a.ws + (size_t)tile * a.split * TE + idx;
      v = 0.f;
      for (int q = 0; q < a.split; ++q)
        v += q == sp ? slice_sum(idx)
                     : __hip_atomic_load(part + (size_t)q * TE,
                                         __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
    } else {
      v = slice_sum(idx);
    }
    const int row = row0 + r;
    if (FMT == F_RTN8) v *= f16_bits_to_f32(a.d[row]);
    float* yp = a.nseg_tab > 0
                    ? s_y + (size_t)n * (seg_hi - s_lo) + (row - s_lo)
                    : a.y + (size_t)n * a.rows + row;
    switch (mode) {
      case RWKVQ_EPI_ADD: v += *yp; break;
      case RWKVQ_EPI_RELU2: v = v > 0.f ? v * v : 0.f; break;
      case RWKVQ_EPI_TANH: v = tanhf(v); break;
      case RWKVQ_EPI_SIGMOID: v = 1.f / (1.f + __expf(-v)); break;
      default: break;
    }
    *yp = v;
  }
}

// Split K across workgroups (halving each wave's steps) until the launch
// has >= RWKVQ_BG_SPLIT_WGS workgroups, where the workspace allows; one
// 16-row block only (measured: 1.5B decode B = 8 2.15 -> 2.04 ms per step;
// with two blocks, 2.9B B = 32, 7.47 -> 7.78 ms, so not there).
#ifndef RWKVQ_BG_SPLIT_WGS
#define RWKVQ_BG_SPLIT_WGS 256
#endif

template <int FMT, int RT, int KSMAX, int NB = 1>
int launch_bg_rt(GemvArgs a, hipStream_t s) {
  const long tiles = a.rows / (16 * RT);
  a.split = 1;
  float* ws;
  long ws_bytes;
  int* cnt;
  int ncnt;
  if (NB == 1 && split_workspace(&ws, &ws_bytes, &cnt, &ncnt) &&
      tiles <= ncnt) {
    const long te = 16L * RT * 16 * NB;
    while (tiles * a.split < RWKVQ_BG_SPLIT_WGS && a.rpw % 2 == 0 &&
           tiles * 2 * a.split * te * (long)sizeof(float) <= ws_bytes) {
      a.split *= 2;
      a.rpw /= 2;
    }
    a.ws = ws;
    a.cnt = cnt;
  }
  dim3 grid(tiles * a.split), block(64 * a.ks);
  for (int n0 = 0; n0 < a.n; n0 += 16 * NB) {
    GemvArgs b = a;
    b.x = a.x + (size_t)n0 * a.x_ld;
    b.y = a.y + (size_t)n0 * a.rows;
    b.n = a.n - n0 < 16 * NB ? a.n - n0 : 16 * NB;
    if (a.rpw == 2)
      hipLaunchKernelGGL((bgemv_kernel<FMT, RT, 2, KSMAX, NB>), grid, block, 0, s, b);
    else if (a.rpw == 4)
      hipLaunchKernelGGL((bgemv_kernel<FMT, RT, 4, KSMAX, NB>), grid, block, 0, s, b);
    else
      hipLaunchKernelGGL((bgemv_kernel<FMT, RT, 0, KSMAX, NB>), grid, block, 0, s, b);
  }
  return hipGetLastError() == hipSuccess ? RWKVQ_OK : RWKVQ_ERR_LAUNCH;
}

// K slices: two 128-column steps per wave where up to 8 waves cover K,
// else the largest divisor <= 8 of the step count.  Row tiles are the
// widest that keep >= 256 workgroups and divide a segment.
template <int FMT>
int launch_bg(GemvArgs a, hipStream_t s) {
  const int steps = a.in / 128;
  // at most 8 K slices: the hi / lo operands need more than the 128 VGPRs
  // a lane of a 16-wave workgroup has
  int ks;
  if (steps % 2 == 0 && steps / 2 <= 8) {
    ks = steps / 2;
  } else {
    ks = 8;
    while (steps % ks) --ks;
  }
  if (RWKVQ_BG_NB2 && a.n > 16) {
    // 17+ rows: two 16-row blocks per pass (each decoded weight feeds both;
    // the second block's x doubles the registers, so at most 8 K slices)
    ks = 8;
    while (steps % ks) --ks;
    a.ks = ks;
    a.rpw = steps / ks;
    if (a.out_per % 32 == 0 && a.rows / 32 >= 256)
      return launch_bg_rt<FMT, 2, 8, 2>(a, s);
    return launch_bg_rt<FMT, 1, 8, 2>(a, s);
  }
  a.ks = ks;
  a.rpw = steps / ks;
  // 64-row tiles only pay for the int8 formats (measured: sb6 heads are
  // faster with 32-row tiles, int8 heads with 64)
  constexpr bool kWide = FMT == F_SYM8 || FMT == F_RTN8;
  if (kWide && a.out_per % 64 == 0 && a.rows / 64 >= 256)
    return launch_bg_rt<FMT, kWide ? 4 : 2, 8>(a, s);
  if (a.out_per % 32 == 0 && a.rows / 32 >= 256)
    return launch_bg_rt<FMT, 2, 8>(a, s);
  return launch_bg_rt<FMT, 1, 8>(a, s);
}

#ifndef RWKVQ_TARGET_WAVES
#define RWKVQ_TARGET_WAVES 4096
#endif
#ifndef RWKVQ_GEMV_ILV
#define RWKVQ_GEMV_ILV 1
#endif
#ifndef RWKVQ_MAX_RPW
#define RWKVQ_MAX_RPW 32
#endif

template <int FMT, int RS>
int launch_rs(GemvArgs a, hipStream_t s) {
  // rows per wave: aim for RWKVQ_TARGET_WAVES waves, at least RS rows; the
  // rows of a workgroup share one x segment (out_per multiple of them)
  // (matrices up to 16384 row-slices: aim for half that many waves --
  // measured faster, each workgroup's x staging then serves more rows)
  long rows_waves = (long)a.rows * a.ks;
  int rpw = (int)(rows_waves / (rows_waves <= 16384 ? RWKVQ_TARGET_WAVES / 2
                                                    : RWKVQ_TARGET_WAVES));
  rpw = rpw < RS ? RS : (rpw / RS) * RS;
  if (rpw > RWKVQ_MAX_RPW) rpw = RWKVQ_MAX_RPW;
  while (a.rg > 1 && a.out_per % (a.rg * RS)) a.rg >>= 1;
  while (rpw > RS && a.out_per % (a.rg * rpw)) rpw -= RS;
  if (a.out_per % (a.rg * rpw)) return RWKVQ_ERR_ARG;
  a.rpw = rpw;
  const int rows_per_wg = a.rg * rpw;
  dim3 grid((a.rows + rows_per_wg - 1) / rows_per_wg);
  dim3 block(64 * a.ks * a.rg);
  // interleaved row order for large one-segment matrices only (the heads:
  // 28.4 vs 29.6 us for 2048->65536 int8); below 16384 row-slices it was
  // slower (measured)
  // (4-row batches, one or two input rows)
  const bool ilv = RWKVQ_GEMV_ILV && RS == 4 && a.n <= 2 && a.n_seg == 1 &&
                   rows_waves > 16384 &&
                   (long)grid.x * rows_per_wg == (long)a.rows;
  const int ng = a.in / 32;
  // up to 4 input rows per launch (each weight read once per chunk; the
  // hi / lo x of 8 rows would not fit the VGPRs); the staged x must fit
  // the LDS budget of 96 KiB per workgroup
  int chunk = 4;
  while (chunk > 1 &&
         (size_t)chunk * ng * (kXWords + kXSums) * 4 > 96 * 1024)
    chunk >>= 1;
  for (int n0 = 0; n0 < a.n; n0 += chunk) {
    GemvArgs b = a;
    b.x = a.x + (size_t)n0 * a.x_ld;
    b.y = a.y + (size_t)n0 * a.rows;
    b.n = a.n - n0 < chunk ? a.n - n0 : chunk;
    const int nn = b.n <= 1 ? 1 : b.n <= 2 ? 2 : b.n <= 4 ? 4 : 8;
    // (the interleaved-row kernels always stage x in LDS)
    const bool xd = a.ks > 1 && !ilv;
    const size_t lds = xd ? 0 : (size_t)nn * ng * (kXWords + kXSums) * 4;
    constexpr bool NT = FMT <= F_SB6_6;
    switch (nn) {
      case 1:
        if (ilv)
          hipLaunchKernelGGL((gemv_kernel<FMT, 1, RS, RS == 4>), grid, block, lds, s, b);
        else if (xd)
          hipLaunchKernelGGL((gemv_kernel<FMT, 1, RS, false, NT, true>), grid, block, lds, s, b);
        else
          hipLaunchKernelGGL((gemv_kernel<FMT, 1, RS>), grid, block, lds, s, b);
        break;
      case 2:
        if (ilv)
          hipLaunchKernelGGL((gemv_kernel<FMT, 2, RS, RS == 4>), grid, block, lds, s, b);
        else if (xd)
          hipLaunchKernelGGL((gemv_kernel<FMT, 2, RS, false, NT, true>), grid, block, lds, s, b);
        else
          hipLaunchKernelGGL((gemv_kernel<FMT, 2, RS>), grid, block, lds, s, b);
        break;
      default: hipLaunchKernelGGL((gemv_kernel<FMT, 4, RS>), grid, block, lds, s, b); break;
    }
  }
  return hipGetLastError() == hipSuccess ? RWKVQ_OK : RWKVQ_ERR_LAUNCH;
}

template <int FMT>
int launch_fmt(GemvArgs a, hipStream_t s) {
  // three or more input rows: the matrix-core kernel (16-row weight
  // tiles); at two the lane-dot kernel is as fast or faster (measured)
  if (a.n >= 3 && a.rows % 16 == 0 && a.out_per % 16 == 0)
    return launch_bg<FMT>(a, s);
  const int ng = a.in / 32;
  a.ks = (ng + 63) / 64;
  if (a.ks > 8) return RWKVQ_ERR_SIZE;             // IN <= 16384
  a.rg = a.ks >= 8 ? 1 : 8 / a.ks;  // <= 8 waves per workgroup share x
  // small matrices: 2-row batches keep more waves in flight; large ones
  // amortise the lane-resident x over 4-row batches
  if ((long)a.rows * a.ks <= 8192 || a.out_per % 4 || a.n > 2)
    return launch_rs<FMT, 2>(a, s);
  return launch_rs<FMT, 4>(a, s);
}

int check_common(int rows, int in, int out_per, int n, int mode) {
  if (rows <= 0 || in <= 0 || n <= 0 || out_per <= 0) return RWKVQ_ERR_ARG;
  if (in % 256) return RWKVQ_ERR_ARG;
  if (rows % out_per || out_per % 2) return RWKVQ_ERR_ARG;
  if (mode < 0 || mode > RWKVQ_EPI_SIGMOID) return RWKVQ_ERR_ARG;
  return RWKVQ_OK;
}

}  // namespace

extern "C" {

int rwkvq_gemv_sb6(const uint8_t* nib, const uint32_t* hb, const uint8_t* rec,
                   int bits, int rows, int in, int out_per, const float* x,
                   long x_ld, float* y, int n, int mode, void* stream) {
  int st = check_common(rows, in, out_per, n, mode);
  if (st) return st;
  if (bits < 4 || bits > 6 || (bits > 4 && !hb)) return RWKVQ_ERR_ARG;
  GemvArgs a{};
  a.q = nib; a.hb = hb; a.rec = rec; a.x = x; a.y = y;
  a.rows = rows; a.in = in; a.out_per = out_per; a.n_seg = rows / out_per;
  a.mode = mode; a.n = n;
  a.x_ld = x_ld > 0 ? x_ld : (long)a.n_seg * in;
  if (a.x_ld < (long)a.n_seg * in) return RWKVQ_ERR_ARG;
  hipStream_t s = (hipStream_t)stream;
  if (bits == 4) return launch_fmt<F_SB6_4>(a, s);
  if (bits == 5) return launch_fmt<F_SB6_5>(a, s);
  return launch_fmt<F_SB6_6>(a, s);
}

int rwkvq_gemv_sym(const uint8_t* codes, const uint32_t* hb, const int8_t* qs,
                   const uint16_t* d, int bits, int rows, int in, int out_per,
                   const float* x, long x_ld, float* y, int n, int mode,
                   void* stream) {
  int st = check_common(rows, in, out_per, n, mode);
  if (st) return st;
  if ((bits != 6 && bits != 8) || (bits == 6 && !hb)) return RWKVQ_ERR_ARG;
  GemvArgs a{};
  a.q = codes; a.hb = hb; a.qs = qs; a.d = d; a.x = x; a.y = y;
  a.rows = rows; a.in = in; a.out_per = out_per; a.n_seg = rows / out_per;
  a.mode = mode; a.n = n;
  a.x_ld = x_ld > 0 ? x_ld : (long)a.n_seg * in;
  if (a.x_ld < (long)a.n_seg * in) return RWKVQ_ERR_ARG;
  hipStream_t s = (hipStream_t)stream;
  return bits == 6 ? launch_fmt<F_SYM6>(a, s) : launch_fmt<F_SYM8>(a, s);
}

int rwkvq_gemv_rtn8(const int8_t* codes, const uint16_t* scale, int rows,
                    int in, int out_per, const float* x, long x_ld, float* y,
                    int n, int mode, void* stream) {
  int st = check_common(rows, in, out_per, n, mode);
  if (st) return st;
  GemvArgs a{};
  a.q = reinterpret_cast<const uint8_t*>(codes); a.d = scale; a.x = x; a.y = y;
  a.rows = rows; a.in = in; a.out_per = out_per; a.n_seg = rows / out_per;
  a.mode = mode; a.n = n;
  a.x_ld = x_ld > 0 ? x_ld : (long)a.n_seg * in;
  if (a.x_ld < (long)a.n_seg * in) return RWKVQ_ERR_ARG;
  return launch_fmt<F_RTN8>(a, (hipStream_t)stream);
}

int rwkvq_gemv_rtn8_spqr(const int8_t* codes, const uint16_t* scale,
                         const int* row_ptr, const int* cols,
                         const uint16_t* vals, int rows, int in,
                         const float* x, long x_ld, float* y, int n,
                         int mode, void* stream) {
  int st = check_common(rows, in, rows, n, mode);
  if (st) return st;
  if (!codes || !scale || !row_ptr || !cols || !vals || !x || !y)
    return RWKVQ_ERR_ARG;
  if (x_ld <= 0) x_ld = in;
  if (x_ld < in) return RWKVQ_ERR_ARG;
  hipStream_t s = (hipStream_t)stream;
  if (n > 2) {
    // the matrix-core rows: GEMV (store / accumulate), then the outlier
    // tail and the epilogue in rwkvq_spqr_apply
    st = rwkvq_gemv_rtn8(codes, scale, rows, in, rows, x, x_ld, y, n,
                         mode == RWKVQ_EPI_ADD ? RWKVQ_EPI_ADD
                                               : RWKVQ_EPI_STORE,
                         stream);
    if (st) return st;
    return rwkvq_spqr_apply(x, x_ld, row_ptr, cols, vals, rows, n, y,
                            mode == RWKVQ_EPI_ADD ? RWKVQ_EPI_STORE : mode,
                            stream);
  }
  GemvArgs a{};
  a.q = reinterpret_cast<const uint8_t*>(codes); a.d = scale; a.x = x; a.y = y;
  a.rows = rows; a.in = in; a.out_per = rows; a.n_seg = 1;
  a.mode = mode; a.n = n; a.x_ld = x_ld;
  a.sp_ptr = row_ptr; a.sp_col = cols; a.sp_val = vals;
  return launch_fmt<F_RTN8>(a, s);
}

int rwkvq_gemv_f16_seg(const uint16_t* w, int nseg, const int* seg_rows,
                       int in, const float* x, long x_ld,
                       float* const* seg_y, int n, int seg_modes,
                       void* stream) {
  // one launch covers the batch: 16 rows, or 32 with the two-block kernel
  if (!w || !x || nseg < 1 || nseg > 8 || in <= 0 || in % 128 || n < 1 ||
      n > (RWKVQ_BG_NB2 ? 32 : 16))
    return RWKVQ_ERR_ARG;
  GemvArgs a{};
  int rows = 0;
  for (int j = 0; j < nseg; ++j) {
    const int m = (seg_modes >> (4 * j)) & 15;
    if (seg_rows[j] <= 0 || seg_rows[j] % 16 || !seg_y[j] ||
        m > RWKVQ_EPI_SIGMOID)
      return RWKVQ_ERR_ARG;
    rows += seg_rows[j];
    a.seg_end[j] = rows;
    a.seg_y[j] = seg_y[j];
  }
  a.q = reinterpret_cast<const uint8_t*>(w);
  a.x = x; a.y = seg_y[0];
  a.rows = rows; a.in = in; a.out_per = 16; a.n_seg = nseg; a.n = n;
  a.nseg_tab = nseg; a.mode = RWKVQ_EPI_PER_SEG; a.seg_modes = seg_modes;
  a.x_ld = x_ld > 0 ? x_ld : (long)nseg * in;
  if (a.x_ld < (long)nseg * in) return RWKVQ_ERR_ARG;
  return launch_bg<F_F16>(a, (hipStream_t)stream);
}

}  // extern "C"
