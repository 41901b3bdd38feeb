// x as int8 digits for the exact integer-dot GEMV paths (lane-dot GEMV
// and the persistent decode kernel): x 2^e = d0 + d1 / 128 + d2 / 16384 +
// r per value, the group's largest |x| 2^e in [63.75, 127.5), multiplied
// with the stored codes by v_dot4_i32_i8.
#pragma once
#include "rwkvq_common.h"

namespace rwkvq {

// 4 x 4 byte transpose: out[t] byte b = in[b] byte t (eight v_perm_b32).
__device__ __forceinline__ void byte_transpose4(uint32_t a, uint32_t b,
                                                uint32_t c, uint32_t d,
                                                uint32_t out[4]) {
  const uint32_t t0 = __builtin_amdgcn_perm(b, a, 0x05010400u);  // a0 b0 a1 b1
  const uint32_t t1 = __builtin_amdgcn_perm(b, a, 0x07030602u);  // a2 b2 a3 b3
  const uint32_t t2 = __builtin_amdgcn_perm(d, c, 0x05010400u);  // c0 d0 c1 d1
  const uint32_t t3 = __builtin_amdgcn_perm(d, c, 0x07030602u);  // c2 d2 c3 d3
  out[0] = __builtin_amdgcn_perm(t2, t0, 0x05040100u);
  out[1] = __builtin_amdgcn_perm(t2, t0, 0x07060302u);
  out[2] = __builtin_amdgcn_perm(t3, t1, 0x05040100u);
  out[3] = __builtin_amdgcn_perm(t3, t1, 0x07060302u);
}

// Four bits b (bits 0..3) spread to bit 0 of bytes 0..3: the partial
// products of the 24-bit multiply land 7 bits apart, so nothing carries.
__device__ __forceinline__ uint32_t spread4(uint32_t b) {
  return __umul24(b, 0x204081u) & 0x01010101u;
}

// Power of two for the int8 digits of a group whose largest |x| is amax:
// amax 2^e in [63.75, 127.5), so the first digit fits [-127, 127].
__device__ __forceinline__ int digit_exp(float amax) {
  if (!(amax > 0.f)) return 0;
  int e = 6 - ilogbf(amax);
  if (ldexpf(amax, e) >= 127.5f) --e;
  return min(e, 126);
}

// Digits of one value: x 2^e = d0 + d1 / 128 + d2 / 16384 + r, |r| <= 2^-15
// (each step exact in fp32), d0 in [-127, 127], d1 and d2 in [-64, 64];
// relative to the group's largest |x| about 21 bits.  Returned as bytes.
__device__ __forceinline__ void x_digit3(float x, int e, uint32_t& b0,
                                         uint32_t& b1, uint32_t& b2) {
  const float a = ldexpf(x, e);
  const float d0 = rintf(a);
  const float r1 = (a - d0) * 128.f;
  const float d1 = rintf(r1);
  const float d2 = rintf((r1 - d1) * 128.f);
  b0 = (uint32_t)(int)d0 & 0xFFu;
  b1 = (uint32_t)(int)d1 & 0xFFu;
  b2 = (uint32_t)(int)d2 & 0xFFu;
}

// One lane's 32 values of a group as digit words: w[0..7] first digits,
// w[8..15] second, w[16..23] third (bytes in column order, word k = columns
// 4k..4k+3); isc = 2^-e, NaN when the group holds a non-finite x (the
// result is then NaN rather than a finite number); sum_a / sum_b = the fp32
// sums of columns 0..15 / 16..31 (the sb6 min and sym6 storage-shift terms).
__device__ __forceinline__ void x_digits(const float xv[32], uint32_t w[24],
                                         float& isc, float& sum_a,
                                         float& sum_b) {
  float amax = 0.f, sa = 0.f, sb = 0.f;
  bool bad = false;
#pragma unroll
  for (int c = 0; c < 32; ++c) {
    amax = fmaxf(amax, fabsf(xv[c]));
    bad |= !(fabsf(xv[c]) <= 3.4e38f);
    if (c < 16) sa += xv[c]; else sb += xv[c];
  }
  sum_a = sa;
  sum_b = sb;
  const int e = digit_exp(amax);
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    uint32_t w0 = 0u, w1 = 0u, w2 = 0u;
#pragma unroll
    for (int bb = 0; bb < 4; ++bb) {
      uint32_t b0, b1, b2;
      x_digit3(bad ? 0.f : xv[4 * k + bb], e, b0, b1, b2);
      w0 |= b0 << (8 * bb);
      w1 |= b1 << (8 * bb);
      w2 |= b2 << (8 * bb);
    }
    w[k] = w0;
    w[8 + k] = w1;
    w[16 + k] = w2;
  }
  isc = bad ? __builtin_nanf("") : ldexpf(1.f, -e);
}

// Sum of the three digit dot products, unscaled: s0 + s1 / 128 + s2 / 16384.
__device__ __forceinline__ float digit_sum(int s0, int s1, int s2) {
  return fmaf(fmaf((float)s2, 0.0078125f, (float)s1), 0.0078125f, (float)s0);
}

}  // namespace rwkvq
