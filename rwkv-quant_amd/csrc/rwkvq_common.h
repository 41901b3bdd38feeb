// Shared device helpers for the gfx950 (CDNA4) kernels of librwkvq_hip.
//
// Wave64 everywhere: one wavefront = 64 lanes; reductions use DPP/permute
// across the full wave.  No packed-fp32 instructions are written by hand.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rwkvq_hip.h"

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

namespace rwkvq {

// The split-K workspace registered on the current device with
// rwkvq_gemm_workspace (partial tiles + arrival counters), shared by the
// GEMMs and the batched GEMV; false when none is registered.  Host side.
bool split_workspace(float** ws, long* bytes, int** cnt, int* ncnt);

__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

// float32(float16(v)) with round-to-nearest-even, the fp16 round trip the
// format uses for block scales.
__device__ __forceinline__ float f16_round(float v) {
  return (float)(_Float16)v;
}

// DPP move of a float within rows of 16 lanes (bound_ctrl: out-of-row
// sources read 0, never used by the patterns below).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                         0xF, 0xF, true));
}

// Sum over all 64 lanes, result uniform (in every lane).  Butterflies
// inside each 16-lane row with DPP (quad_perm xor1, xor2, row_half_mirror,
// row_mirror), then the four row sums through v_readlane.
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp_f<0xB1>(v);    // quad_perm [1,0,3,2]
  v += dpp_f<0x4E>(v);    // quad_perm [2,3,0,1]
  v += dpp_f<0x141>(v);   // row_half_mirror
  v += dpp_f<0x140>(v);   // row_mirror
  const int b = __builtin_bit_cast(int, v);
  float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
  float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
  float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
  float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
  return (r0 + r1) + (r2 + r3);
}

__device__ __forceinline__ float wave_sum(float v) {
  v += __shfl_xor(v, 32, 64);
  v += __shfl_xor(v, 16, 64);
  v += __shfl_xor(v, 8, 64);
  v += __shfl_xor(v, 4, 64);
  v += __shfl_xor(v, 2, 64);
  v += __shfl_xor(v, 1, 64);
  return v;
}

// 16-byte global load as four dwords.
__device__ __forceinline__ uint4 ld16(const void* p) {
  return *reinterpret_cast<const uint4*>(p);
}

#ifndef RWKVQ_NT_LOADS
#define RWKVQ_NT_LOADS 1
#endif
typedef unsigned int u32x4_nt_t __attribute__((ext_vector_type(4)));
// 16-byte load of packed weight codes.  NT: a non-temporal (streaming)
// load (the codes are read once per launch).
template <bool NT>
__device__ __forceinline__ uint4 ld16_w(const void* p) {
  if constexpr (NT && RWKVQ_NT_LOADS) {
    u32x4_nt_t v =
        __builtin_nontemporal_load(reinterpret_cast<const u32x4_nt_t*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
  } else {
    return ld16(p);
  }
}

// Nibble byte pair -> two fp16 lanes holding 1024 + code:
// result low half = 0x6400 | (lo nibble of byte j of w) [| high bits],
// high half = 0x6400 | (hi nibble of byte j of w).
// `ws` must be w >> 4.  v_perm_b32 picks byte j of w and of ws, zeroing the
// other two bytes; v_and_or_b32 keeps the nibbles and sets the exponent.
template <int J>
__device__ __forceinline__ uint32_t nib_pair(uint32_t w, uint32_t ws) {
  constexpr uint32_t sel = (uint32_t)J | (0x0Cu << 8) | ((4u + J) << 16) |
                           (0x0Cu << 24);
  uint32_t t = __builtin_amdgcn_perm(ws, w, sel);
  return (t & 0x000F000Fu) | 0x64006400u;
}

// Signed byte pair (bytes 2P, 2P+1 of w) -> two fp16 lanes holding
// 1024 + 128 + code  (code in -128..127).
template <int P>
__device__ __forceinline__ uint32_t i8_pair(uint32_t w) {
  constexpr uint32_t sel = (uint32_t)(2 * P) | (0x0Cu << 8) |
                           ((uint32_t)(2 * P + 1) << 16) | (0x0Cu << 24);
  uint32_t t = __builtin_amdgcn_perm(0u, w, sel);
  return t ^ 0x64806480u;
}

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, a),
                                __builtin_bit_cast(h2_t, b), c, false);
}

__device__ __forceinline__ uint32_t pack_h2(float lo, float hi) {
  _Float16 a = (_Float16)lo, b = (_Float16)hi;
  return (uint32_t)__builtin_bit_cast(uint16_t, a) |
         ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

// Register pin: an empty volatile asm that "rewrites" v.  Placed after a
// scheduling barrier, it keeps every consumer of a prefetched register (and
// the wait for its load) behind that point.
__device__ __forceinline__ void pin(uint32_t& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void pin(float& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void pin(uint4& v) { pin(v.x); pin(v.y); pin(v.z); pin(v.w); }
__device__ __forceinline__ void pin(float4& v) { pin(v.x); pin(v.y); pin(v.z); pin(v.w); }

__device__ __forceinline__ float h2_lo(uint32_t u) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(u & 0xFFFFu));
}
__device__ __forceinline__ float h2_hi(uint32_t u) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(u >> 16));
}

}  // namespace rwkvq
