// Packed-format decode shared by the GEMV and GEMM kernels.
//
// Formats (device layouts from rwkv_quant/backends/hip/repack.py):
//   F_SB6_4/5/6  nibble plane [rows, NG, 16] (byte j of a 32-column group =
//                column j low nibble, column j+16 high nibble), high-bit
//                words, 16-byte superblock records qs|qm(6-bit)|d|dm
//   F_SYM6       nibble plane + high-bit crumbs, int8 block scales per 16
//                columns, fp16 d per 256 columns
//   F_SYM8       int8 codes, same scales
//   F_RTN8       int8 codes, fp16 scale per row
// A lane decodes one (row, 32-column group) into 16 fp16 pairs holding
// 1024 + code (+ the storage bias); pair i covers columns x_cols(i).
#pragma once
#include "rwkvq_common.h"

namespace rwkvq {

enum Fmt { F_SB6_4 = 0, F_SB6_5 = 1, F_SB6_6 = 2, F_SYM6 = 3, F_SYM8 = 4,
           F_RTN8 = 5,
           F_F16 = 6 };   // dense fp16 rows (GEMM only)

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

// Raw bytes of one (row, group): issued as loads one row batch ahead of
// the arithmetic that consumes them.
struct Raw {
  uint4 a;        // nibbles, or codes 0..15 (int8 formats)
  uint4 b;        // sb6 superblock record, or codes 16..31 (int8 formats)
  uint2 h;        // high-bit words
  uint32_t s;     // sym: qs pair (two int8 block scales, low 16 bits)
  uint32_t dd;    // sym: fp16 d bits
  // loaded values are kept as loaded (no arithmetic at load time), so a
  // consumer's wait is for its own loads, not for the whole batch
};

template <int FMT, class Args>
__device__ __forceinline__ void load_raw(const Args& a, int row, int ng,
                                         int nsb, int g, Raw& r) {
  if (FMT == F_SYM8 || FMT == F_RTN8) {
    const uint8_t* p = a.q + (size_t)row * a.in;     // wave-uniform
    r.a = ld16(p + g * 32);
    r.b = ld16(p + g * 32 + 16);
  } else {
    const uint8_t* p = a.q + (size_t)row * ng * 16;  // wave-uniform
    r.a = ld16(p + g * 16);
  }
  if (FMT <= F_SB6_6)
    r.b = ld16(a.rec + (size_t)row * nsb * 16 + (g >> 3) * 16);
  if (FMT == F_SB6_5) r.h.x = a.hb[(size_t)row * ng + g];
  if (FMT == F_SB6_6 || FMT == F_SYM6)
    r.h = *reinterpret_cast<const uint2*>(a.hb + (size_t)row * ng * 2 + g * 2);
  if (FMT == F_SYM6 || FMT == F_SYM8) {
    r.s = *reinterpret_cast<const uint16_t*>(
        a.qs + (size_t)row * (a.in >> 4) + 2 * g);
    r.dd = a.d[(size_t)row * nsb + (g >> 3)];
  }
}

// Raw bytes -> 16 fp16 pairs (1024 + code, offset by the storage bias).
template <int FMT>
__device__ __forceinline__ void decode_raw(const Raw& r, uint32_t h[16]) {
  if (FMT == F_SYM8 || FMT == F_RTN8) {
    uint32_t w[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      h[2 * k] = i8_pair<0>(w[k]);
      h[2 * k + 1] = i8_pair<1>(w[k]);
    }
    return;
  }
  uint32_t w[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    uint32_t ws = w[k] >> 4;
    h[4 * k + 0] = nib_pair<0>(w[k], ws);
    h[4 * k + 1] = nib_pair<1>(w[k], ws);
    h[4 * k + 2] = nib_pair<2>(w[k], ws);
    h[4 * k + 3] = nib_pair<3>(w[k], ws);
  }
  if (FMT == F_SB6_5) {
    uint32_t hw = r.h.x;
#pragma unroll
    for (int i = 0; i < 16; ++i)
      h[i] |= __builtin_amdgcn_alignbit(hw, hw, (uint32_t)((i - 4) & 31)) &
              0x00100010u;
  } else if (FMT == F_SB6_6 || FMT == F_SYM6) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      uint32_t H = (i < 8) ? r.h.x : r.h.y;
      int ip = i & 7;
      h[i] |= __builtin_amdgcn_alignbit(H, H, (uint32_t)((2 * ip - 4) & 31)) &
              0x00300030u;
    }
  }
}

}  // namespace rwkvq
