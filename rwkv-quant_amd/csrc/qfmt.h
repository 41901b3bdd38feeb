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

template <int FMT, bool NT = true, class Args>
__device__ __forceinline__ void load_raw(const Args& a, int row, int ng,
                                         int nsb, int g, Raw& r) {
  if (FMT == F_SYM8 || FMT == F_RTN8) {
    const uint8_t* p = a.q + (size_t)row * a.in;     // wave-uniform
    r.a = ld16_w<NT>(p + g * 32);
    r.b = ld16_w<NT>(p + g * 32 + 16);
  } else {
    const uint8_t* p = a.q + (size_t)row * ng * 16;  // wave-uniform
    r.a = ld16_w<NT>(p + g * 16);
  }
  if (FMT <= F_SB6_6)
    r.b = ld16_w<NT>(a.rec + (size_t)row * nsb * 16 + (g >> 3) * 16);
  if (FMT == F_SB6_5) r.h.x = a.hb[(size_t)row * ng + g];
  if (FMT == F_SB6_6 || FMT == F_SYM6)
    r.h = *reinterpret_cast<const uint2*>(a.hb + (size_t)row * ng * 2 + g * 2);
  if (FMT == F_SYM6 || FMT == F_SYM8) {
    r.s = *reinterpret_cast<const uint16_t*>(
        a.qs + (size_t)row * (a.in >> 4) + 2 * g);
    r.dd = a.d[(size_t)row * nsb + (g >> 3)];
  }
}

// Dense fp16 rows (F_F16): one lane's 32-column group is 64 bytes, held
// as loaded; the pair order is the natural one.
struct RawF16 {
  uint4 q[4];
};
template <int FMT> struct RawOf { using T = Raw; };
template <> struct RawOf<F_F16> { using T = RawF16; };

template <int FMT, bool NT = true, class Args>
__device__ __forceinline__ void load_raw(const Args& a, int row, int ng,
                                         int nsb, int g, RawF16& r) {
  const uint8_t* p = a.q + ((size_t)row * a.in + g * 32) * 2;
#pragma unroll
  for (int i = 0; i < 4; ++i) r.q[i] = ld16(p + 16 * i);
}

// Pin the fields of a Raw that the format loads (pinning an unused one
// would keep its registers alive).
template <int FMT>
__device__ __forceinline__ void pin_raw(Raw& r) {
  pin(r.a);
  if (FMT != F_SYM6) pin(r.b);
  if (FMT == F_SB6_5) pin(r.h.x);
  if (FMT == F_SB6_6 || FMT == F_SYM6) { pin(r.h.x); pin(r.h.y); }
  if (FMT == F_SYM6 || FMT == F_SYM8) { pin(r.s); pin(r.dd); }
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

// fp16 pair <-> its 32-bit register image
__device__ __forceinline__ uint32_t h2_bits(h2_t v) {
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ h2_t as_h2(uint32_t u) {
  return __builtin_bit_cast(h2_t, u);
}

// fp16 weights of one (row, group) in the decoder's pair order.
template <int FMT>
__device__ __forceinline__ void dequant_group(const Raw& r, int kb,
                                              uint32_t w[16]) {
  decode_raw<FMT>(r, w);
  if (FMT <= F_SB6_6) {
    const uint32_t rr[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
    const int qs_word = (6 * kb) >> 5, qs_sh = (6 * kb) & 31;
    const int qm_word = (48 + 6 * kb) >> 5, qm_sh = (48 + 6 * kb) & 31;
    uint32_t lo = qs_word == 0 ? rr[0] : rr[1];
    uint32_t hi = qs_word == 0 ? rr[1] : rr[2];
    const uint32_t qsv = __builtin_amdgcn_alignbit(hi, lo, (uint32_t)qs_sh) & 63u;
    lo = qm_word == 1 ? rr[1] : rr[2];
    hi = qm_word == 1 ? rr[2] : rr[3];
    const uint32_t qmv = __builtin_amdgcn_alignbit(hi, lo, (uint32_t)qm_sh) & 63u;
    const float d = f16_bits_to_f32(rr[3] & 0xFFFFu);
    const float dm = f16_bits_to_f32(rr[3] >> 16);
    const _Float16 s = (_Float16)fmaxf(f16_round((float)qsv * d), 1e-8f);
    const _Float16 m = (_Float16)((float)((int)qmv - 31) * dm);
    const h2_t s2 = {s, s}, m2 = {m, m}, bias = {(_Float16)1024.f, (_Float16)1024.f};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const h2_t q = as_h2(w[i]) - bias;                      // exact
      w[i] = h2_bits(__builtin_elementwise_fma(q, s2, m2));  // one rounding
    }
  } else if (FMT == F_SYM6 || FMT == F_SYM8) {
    const float d = f16_bits_to_f32(r.dd);
    const _Float16 sa = (_Float16)((float)(int8_t)(r.s & 0xFFu) * d);
    const _Float16 sb = (_Float16)((float)(int8_t)((r.s >> 8) & 0xFFu) * d);
    const _Float16 mb = (_Float16)magic_bias<FMT>();
    const h2_t bias = {mb, mb}, a2 = {sa, sa}, b2 = {sb, sb};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const h2_t q = as_h2(w[i]) - bias;                      // exact
      w[i] = h2_bits(q * (i < 8 ? a2 : b2));                  // one rounding
    }
  } else {
    const h2_t bias = {(_Float16)1152.f, (_Float16)1152.f};
#pragma unroll
    for (int i = 0; i < 16; ++i) w[i] = h2_bits(as_h2(w[i]) - bias);
  }
}

// dequant_group a quad (4 pairs) at a time, for kernels that spread one
// group's decode over several matrix-core rounds: dq_scale once per group,
// then dq_quad(qd) for qd = 0..3 gives pairs 4 qd .. 4 qd + 3, bit for bit
// those of dequant_group.
struct DqScale {
  h2_t a, b;      // sb6: scale, min; sym: scales of pairs 0-7 and 8-15
};

template <int FMT>
__device__ __forceinline__ DqScale dq_scale(const Raw& r, int kb) {
  DqScale sc;
  if (FMT <= F_SB6_6) {
    const uint32_t rr[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
    const int qs_word = (6 * kb) >> 5, qs_sh = (6 * kb) & 31;
    const int qm_word = (48 + 6 * kb) >> 5, qm_sh = (48 + 6 * kb) & 31;
    uint32_t lo = qs_word == 0 ? rr[0] : rr[1];
    uint32_t hi = qs_word == 0 ? rr[1] : rr[2];
    const uint32_t qsv = __builtin_amdgcn_alignbit(hi, lo, (uint32_t)qs_sh) & 63u;
    lo = qm_word == 1 ? rr[1] : rr[2];
    hi = qm_word == 1 ? rr[2] : rr[3];
    const uint32_t qmv = __builtin_amdgcn_alignbit(hi, lo, (uint32_t)qm_sh) & 63u;
    const float d = f16_bits_to_f32(rr[3] & 0xFFFFu);
    const float dm = f16_bits_to_f32(rr[3] >> 16);
    const _Float16 s = (_Float16)fmaxf(f16_round((float)qsv * d), 1e-8f);
    const _Float16 m = (_Float16)((float)((int)qmv - 31) * dm);
    sc.a = h2_t{s, s};
    sc.b = h2_t{m, m};
  } else if (FMT == F_SYM6 || FMT == F_SYM8) {
    const float d = f16_bits_to_f32(r.dd);
    const _Float16 sa = (_Float16)((float)(int8_t)(r.s & 0xFFu) * d);
    const _Float16 sb = (_Float16)((float)(int8_t)((r.s >> 8) & 0xFFu) * d);
    sc.a = h2_t{sa, sa};
    sc.b = h2_t{sb, sb};
  } else {
    sc.a = h2_t{(_Float16)0.f, (_Float16)0.f};
    sc.b = sc.a;
  }
  return sc;
}

template <int FMT>
__device__ __forceinline__ void dq_quad(const Raw& r, const DqScale& sc,
                                        int qd, uint32_t w[16]) {
  uint32_t h[4];
  if (FMT == F_SYM8 || FMT == F_RTN8) {
    const uint32_t u0 = qd == 0 ? r.a.x : qd == 1 ? r.a.z : qd == 2 ? r.b.x : r.b.z;
    const uint32_t u1 = qd == 0 ? r.a.y : qd == 1 ? r.a.w : qd == 2 ? r.b.y : r.b.w;
    h[0] = i8_pair<0>(u0); h[1] = i8_pair<1>(u0);
    h[2] = i8_pair<0>(u1); h[3] = i8_pair<1>(u1);
  } else {
    const uint32_t u = qd == 0 ? r.a.x : qd == 1 ? r.a.y : qd == 2 ? r.a.z : r.a.w;
    const uint32_t us = u >> 4;
    h[0] = nib_pair<0>(u, us); h[1] = nib_pair<1>(u, us);
    h[2] = nib_pair<2>(u, us); h[3] = nib_pair<3>(u, us);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = 4 * qd + j;
      if (FMT == F_SB6_5) {
        const uint32_t hw = r.h.x;
        h[j] |= __builtin_amdgcn_alignbit(hw, hw, (uint32_t)((i - 4) & 31)) &
                0x00100010u;
      } else if (FMT == F_SB6_6 || FMT == F_SYM6) {
        const uint32_t H = (i < 8) ? r.h.x : r.h.y;
        const int ip = i & 7;
        h[j] |= __builtin_amdgcn_alignbit(H, H, (uint32_t)((2 * ip - 4) & 31)) &
                0x00300030u;
      }
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = 4 * qd + j;
    if (FMT <= F_SB6_6) {
      const h2_t bias = {(_Float16)1024.f, (_Float16)1024.f};
      const h2_t q = as_h2(h[j]) - bias;                       // exact
      w[i] = h2_bits(__builtin_elementwise_fma(q, sc.a, sc.b)); // one rounding
    } else if (FMT == F_SYM6 || FMT == F_SYM8) {
      const _Float16 mb = (_Float16)magic_bias<FMT>();
      const h2_t bias = {mb, mb};
      const h2_t q = as_h2(h[j]) - bias;                       // exact
      w[i] = h2_bits(q * (i < 8 ? sc.a : sc.b));               // one rounding
    } else {
      const h2_t bias = {(_Float16)1152.f, (_Float16)1152.f};
      w[i] = h2_bits(as_h2(h[j]) - bias);
    }
  }
}

// The format's fp32 weights of one (row, group) split into fp16 hi + lo
// pairs (hi = f16(w), lo = f16(w - hi): w to about 22 bits), in the
// decoder's pair order.  sb6 w = q s + m, sym w = q s (s, m the fp32
// values of the format's fp16 block scales); rtn8 and dense fp16 weights
// are fp16 already (lo = 0).  Returns false where lo is identically 0.
template <int FMT>
__device__ __forceinline__ bool dequant_group_hilo(const Raw& r, int kb,
                                                   uint32_t whi[16],
                                                   uint32_t wlo[16]) {
  decode_raw<FMT>(r, whi);
  const _Float16 mbh = (_Float16)magic_bias<FMT>();
  const h2_t bias = {mbh, mbh};
#pragma unroll
  for (int i = 0; i < 16; ++i) whi[i] = h2_bits(as_h2(whi[i]) - bias);
  if (FMT == F_RTN8) {                 // the int8 codes; row scale later
#pragma unroll
    for (int i = 0; i < 16; ++i) wlo[i] = 0u;
    return false;
  }
  float s0, s1, m = 0.f;
  if (FMT <= F_SB6_6) {
    const uint32_t rr[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
    const int qs_word = (6 * kb) >> 5, qs_sh = (6 * kb) & 31;
    const int qm_word = (48 + 6 * kb) >> 5, qm_sh = (48 + 6 * kb) & 31;
    uint32_t lo = qs_word == 0 ? rr[0] : rr[1];
    uint32_t hi = qs_word == 0 ? rr[1] : rr[2];
    const uint32_t qsv = __builtin_amdgcn_alignbit(hi, lo, (uint32_t)qs_sh) & 63u;
    lo = qm_word == 1 ? rr[1] : rr[2];
    hi = qm_word == 1 ? rr[2] : rr[3];
    const uint32_t qmv = __builtin_amdgcn_alignbit(hi, lo, (uint32_t)qm_sh) & 63u;
    const float d = f16_bits_to_f32(rr[3] & 0xFFFFu);
    const float dm = f16_bits_to_f32(rr[3] >> 16);
    s0 = s1 = fmaxf(f16_round((float)qsv * d), 1e-8f);
    m = f16_round((float)((int)qmv - 31) * dm);
  } else {                             // sym6 / sym8: two 16-column blocks
    const float d = f16_bits_to_f32(r.dd);
    s0 = f16_round((float)(int8_t)(r.s & 0xFFu) * d);
    s1 = f16_round((float)(int8_t)((r.s >> 8) & 0xFFu) * d);
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float s = i < 8 ? s0 : s1;
    const float wa = fmaf(h2_lo(whi[i]), s, m);
    const float wb = fmaf(h2_hi(whi[i]), s, m);
    whi[i] = pack_h2(wa, wb);
    wlo[i] = pack_h2(wa - h2_lo(whi[i]), wb - h2_hi(whi[i]));
  }
  return true;
}

template <int FMT>
__device__ __forceinline__ bool dequant_group_hilo(const RawF16& r, int,
                                                   uint32_t whi[16],
                                                   uint32_t wlo[16]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    whi[4 * i] = r.q[i].x; whi[4 * i + 1] = r.q[i].y;
    whi[4 * i + 2] = r.q[i].z; whi[4 * i + 3] = r.q[i].w;
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) wlo[i] = 0u;
  return false;
}

// Dense fp16 rows: the stored values are the weights.
template <int FMT>
__device__ __forceinline__ void dequant_group(const RawF16& r, int,
                                              uint32_t w[16]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    w[4 * i] = r.q[i].x; w[4 * i + 1] = r.q[i].y;
    w[4 * i + 2] = r.q[i].z; w[4 * i + 3] = r.q[i].w;
  }
}

// Columns (within a group) of the two float4s that sub-step s of the pair
// order reads: pairs 4s..4s+3.
template <int FMT>
__device__ __forceinline__ void step_cols(int s, int& ca, int& cb) {
  if (FMT <= F_SB6_6) { ca = 4 * s; cb = 4 * s + 16; }
  else if (FMT == F_SYM6) { ca = (s < 2 ? 4 * s : 4 * s + 8); cb = ca + 8; }
  else { ca = 8 * s; cb = 8 * s + 4; }
}

// 8 x values of one (token, group, sub-step) -> 4 fp16 pairs in pair order.
template <int FMT>
__device__ __forceinline__ uint4 x_pairs(float4 A, float4 B) {
  if (FMT == F_SYM8 || FMT == F_RTN8 || FMT == F_F16)   // pairs (2i, 2i+1)
    return make_uint4(pack_h2(A.x, A.y), pack_h2(A.z, A.w),
                      pack_h2(B.x, B.y), pack_h2(B.z, B.w));
  return make_uint4(pack_h2(A.x, B.x), pack_h2(A.y, B.y),   // (c0, c1)
                    pack_h2(A.z, B.z), pack_h2(A.w, B.w));
}

}  // namespace rwkvq
