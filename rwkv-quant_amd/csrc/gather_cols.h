// Column decoders of the packed row gathers (the embedding lookup): 8
// consecutive columns of one row per call -- columns 8 k .. 8 k + 7, i.e.
// quarter k & 3 of the 32-column group k >> 2 -- with the arithmetic of the
// full-matrix dequant kernels (fp16 round trips, products and sums rounded
// separately), so a gathered row equals that row of the dequantized matrix
// bit for bit (reference: rwkv_quant/formats/codec.py:183-292).
#pragma once
#include "rwkvq_common.h"

namespace rwkvq {

// code bits 4/5 of column (pair i, half) of a 32-column group from the
// device high-bit words
__device__ __forceinline__ uint32_t high_bits_crumb(const uint32_t* hw, int i,
                                                    int half) {
  uint32_t H = hw[i >> 3];
  int sh = 2 * (i & 7) + 16 * half;
  return (H >> sh) & 3u;
}

// `idx` (optional) gathers rows: output row o is source row
// min(max(idx[o], 0), src_rows - 1)
__device__ __forceinline__ int src_row(const int64_t* idx, int o,
                                       int src_rows) {
  if (!idx) return o;
  long v = idx[o];
  return (int)(v < 0 ? 0 : (v >= src_rows ? src_rows - 1 : v));
}

// sb6 (4/5/6-bit codes, one 16-byte record per 256 columns): columns
// 8 qq .. 8 qq + 7 of group g are code bytes i0 .. i0 + 7 (i0 = 8 (qq & 1)),
// low nibbles for qq < 2, high for qq >= 2
__device__ __forceinline__ void sb6_cols8(const uint8_t* nib,
                                          const uint32_t* hb,
                                          const uint8_t* rec, int bits,
                                          int in, int row, int k,
                                          float (&o)[8]) {
#pragma clang fp contract(off)
  const int g = k >> 2, qq = k & 3;
  const int ng = in >> 5, nsb = in >> 8;
  // record bytes 0..5: the 6-bit qs fields, 6..11: the qm fields,
  // 12..13: d, 14..15: dm (fp16)
  const uint4 r4 = *reinterpret_cast<const uint4*>(
      rec + ((size_t)row * nsb + (g >> 3)) * 16);
  const uint64_t s0 = (uint64_t)r4.x | ((uint64_t)(r4.y & 0xFFFFu) << 32);
  const uint64_t s1 = (uint64_t)(r4.y >> 16) | ((uint64_t)r4.z << 16);
  const int kb = g & 7;
  const uint32_t qs = (uint32_t)(s0 >> (6 * kb)) & 63u;
  const int qm = (int)((uint32_t)(s1 >> (6 * kb)) & 63u) - 31;
  const float d = f16_bits_to_f32(r4.w & 0xFFFFu);
  const float dm = f16_bits_to_f32(r4.w >> 16);
  const float s = fmaxf(f16_round(((float)qs * d)), 1e-8f);
  const float m = f16_round(((float)qm * dm));
  const int i0 = (qq & 1) * 8, half = qq >> 1;
  const size_t gi = (size_t)row * ng + g;
  const uint2 nb = *reinterpret_cast<const uint2*>(nib + gi * 16 + i0);
  const uint32_t hw5 = bits == 5 ? hb[gi] : 0u;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int i = i0 + j, c = half * 16 + i;
    const uint32_t byte = ((j < 4 ? nb.x : nb.y) >> (8 * (j & 3))) & 0xFFu;
    uint32_t q = half ? (byte >> 4) : (byte & 15u);
    if (bits == 5) {
      q |= ((hw5 >> c) & 1u) << 4;
    } else if (bits == 6) {
      q |= high_bits_crumb(hb + gi * 2, i, half) << 4;
    }
    o[j] = (float)q * s + m;
  }
}

// sym (6/8-bit codes, int8 sub-scales per 16 columns, fp16 d per 256):
// int8 codes: bytes 8 qq .. 8 qq + 7 of the group; 6-bit codes: bytes
// 8 (qq >> 1) .. + 7 of the group's 16, low nibbles for even qq, high for
// odd (byte j of 16-column block b holds columns j and j + 8 of the block)
__device__ __forceinline__ void sym_cols8(const uint8_t* codes,
                                          const uint32_t* hb,
                                          const int8_t* qsp,
                                          const uint16_t* dp, int bits,
                                          int in, int row, int k,
                                          float (&o)[8]) {
#pragma clang fp contract(off)
  const int g = k >> 2, qq = k & 3;
  const int ng = in >> 5, nsb = in >> 8;
  const float d = f16_bits_to_f32(dp[(size_t)row * nsb + (g >> 3)]);
  const float sc = f16_round(
      ((float)qsp[(size_t)row * (in >> 4) + 2 * g + (qq >> 1)] * d));
  const size_t gi = (size_t)row * ng + g;
  if (bits == 8) {
    const uint2 cb = *reinterpret_cast<const uint2*>(
        codes + (size_t)row * in + (size_t)g * 32 + 8 * qq);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t byte = ((j < 4 ? cb.x : cb.y) >> (8 * (j & 3))) & 0xFFu;
      o[j] = (float)(int)(int8_t)byte * sc;
    }
  } else {
    const int b0 = (qq >> 1) * 8, half = qq & 1;
    const uint2 cb = *reinterpret_cast<const uint2*>(codes + gi * 16 + b0);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t v = ((j < 4 ? cb.x : cb.y) >> (8 * (j & 3))) & 0xFFu;
      uint32_t u = half ? (v >> 4) : (v & 15u);
      u |= high_bits_crumb(hb + gi * 2, b0 + j, half) << 4;
      o[j] = (float)((int)u - 32) * sc;
    }
  }
}

// rtn@8 (int8 codes, fp16 scale per row)
__device__ __forceinline__ void rtn8_cols8(const int8_t* codes,
                                           const uint16_t* scale, int in,
                                           int row, int k, float (&o)[8]) {
  const float s = f16_bits_to_f32(scale[row]);
  const uint2 cb = *reinterpret_cast<const uint2*>(
      codes + (size_t)row * in + 8 * k);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t byte = ((j < 4 ? cb.x : cb.y) >> (8 * (j & 3))) & 0xFFu;
    o[j] = (float)(int)(int8_t)byte * s;
  }
}

}  // namespace rwkvq
