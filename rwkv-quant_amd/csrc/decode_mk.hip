// Persistent decode step: every layer of one batch-1 decode step in one
// launch of 256 workgroups (one per CU), the phases separated by grid
// barriers instead of kernel boundaries.
//
// Per layer (reference: rwkv_quant/backends/metal/quant_model.py:638-728,
// 803-809, the same math as the per-kernel decode path of this library):
//   P1  LayerNorm 1 + token shift + lerp, folded into each consumer
//       workgroup (each computes the row statistics itself), then the
//       r/k/v GEMV rows (workgroups 0..191) and the LoRA down products from
//       the file's codes (the next 36..64 workgroups)
//   P2  WKV step per head (LoRA up products from the codes, per-channel
//       prep, one recurrence step, group norm / bonus / gate tail)
//   P3  output projection GEMV, += residual
//   P4  LayerNorm 2 + shift + lerp folded in, key GEMV, relu^2
//   P5  value GEMV (8192 wide), += residual
// Five phases instead of eight launches.  Each workgroup issues the loads
// of its next phase's weights (and WKV state) between its barrier arrival
// and its wait, so the HBM round trip and the streaming of those bytes
// overlap the barrier instead of following it.  (Issued earlier, during the
// current phase's compute, they measured slower: the issue of ~36 KB of
// loads per workgroup stalls the wave's instruction stream, and the
// vector-memory counter is in order.)
//
// Activations crossing workgroups (residual, r/k/v, LoRA down outputs, the
// WKV output, the key output, v_first) are written and read with
// agent-scope relaxed atomics, which are coherent across the XCDs' L2s
// without a cache flush; a barrier arrival is issued only after the
// workgroup's stores have completed (s_waitcnt vmcnt(0)).
//
// Barrier: arrival counters per group of 32 workgroups; the last arriver of
// a group raises the group's flag, and the first wave of every workgroup
// polls the 8 flags with one load (lane g reads flag g).  Measured on
// MI355X at 256 workgroups: 1.57 us per barrier; with a top counter and
// per-group release words 1.8 us; one counter polled by all 6.7 us.  Every
// wait is bounded: past the spin limit the workgroup records an error and
// stops waiting, so a launch that is not co-resident ends with an error
// flag instead of hanging.  The last workgroup to finish resets every word
// for the next launch.
//
// GEMV rows use the exact integer-digit dot products of the lane-dot GEMV
// (codes times three int8 digits of x under a per-group power of two) and
// the format's block scales in fp32; the LoRA down products multiply the
// dequantized fp32 weights (bit-exact with the dequant kernels) by fp32 x.
#include <mutex>
#include <type_traits>

#include "qfmt.h"
#include "rwkvq_hip.h"
#include "xdig.h"

using namespace rwkvq;

namespace {

constexpr int kT = 256;            // threads per workgroup (4 waves)
constexpr int kG = 256;            // workgroups per launch
constexpr int kW = kG * 4;         // waves per launch
constexpr int kHd = 64;            // head size
constexpr int kBarGroup = 32;      // workgroups per arrival counter
constexpr int kNGrp = kG / kBarGroup;
constexpr int kSpinLimit = 1 << 20;  // default polls per barrier wait
constexpr int kRkvWgs = 192;       // P1 workgroups on the r/k/v rows
constexpr int kMkCv = 10;          // 16-row LoRA-up code blocks per wave
constexpr int kMkMaxCat = 4 * 16 * kMkCv;   // sum of the four ranks (640)
constexpr int kBarWords = 2048;    // barrier workspace (uint32 words)

// Descriptor pointers are typed global: read from the LDS copy of the
// table, a pointer without an address space compiles to flat
// instructions, which also count in the LDS counter (every LDS wait would
// then also wait for the weight prefetch).
// (host compilation parses the same structs with the default address
// space; the layout is the same 64-bit pointers)
#if defined(__HIP_DEVICE_COMPILE__)
#define GLB __attribute__((address_space(1)))
#else
#define GLB
#endif

struct MkMat {                     // a packed matrix (load_raw's fields)
  const GLB uint8_t* q;
  const GLB uint32_t* hb;
  const GLB uint8_t* rec;
  const GLB int8_t* qs;
  const GLB uint16_t* d;
  int rows, in;
};

struct MkDown {                    // one LoRA down product from the codes
  const GLB uint8_t* q;                // u8 asym / i8 codes [rows, D]
  const GLB float* s;                  // asym scale [rows / 64, D]; null: int8
  const GLB float* m;                  // asym min
  const GLB uint16_t* sc;              // int8: fp16 scale per input column [D]
  GLB float* y;                        // [rows]
  int rows, slot, epi, wg0;        // lerp slot; first P1 workgroup (rel.)
};

struct MkUp {                      // LoRA up products (rwkvq_wkv7_decode_lora_q)
  const GLB float* h[4];               // the branches' down outputs (w a v g)
  const GLB uint8_t* q[4];
  const GLB float* s[4];
  const GLB float* m[4];
  const GLB uint16_t* sc[4];
  int r[4];
};

struct MkLayer {
  MkMat rkv, o, key, val;
  const GLB float* ln1_w;
  const GLB float* ln1_b;
  const GLB float* coef;               // [6, D] lerp coefficients r k v w a g
  const GLB float* tshift_in;          // [D] or null (zero shift)
  GLB float* tshift_out;
  const GLB float* ln2_w;
  const GLB float* ln2_b;
  const GLB float* xk;                 // [D]
  const GLB float* cshift_in;
  GLB float* cshift_out;
  MkDown down[4];
  MkUp up;
  const GLB float* w0;
  const GLB float* a0;
  const GLB float* v0;
  const GLB float* k_k;
  const GLB float* k_a;
  const GLB float* r_k;
  const GLB float* lnx_w;
  const GLB float* lnx_b;
  const GLB float* state_in;           // [H, 64, 64]
  GLB float* state_out;
  int n_down, layer0, lora_wgs, pad;
};

// Activations live in an arena with one region per (layer, phase output):
// rkv [3 D], the WKV output [D], x after the output projection [D], the key
// output [F], x after the value GEMV [D] (the last layer's goes to x).  The
// WKV and key outputs are stored already as the consumer GEMV's int8
// digits, 32 words per 32-column group (same size as the fp32 values), by
// the workgroup that produces the group, so the consumers load them
// instead of each converting the whole vector again.  A region is
// written once per launch and read only after the barrier that follows
// its writes, so no L2 of any XCD can hold an older copy of it (every L2 is
// invalidated at kernel start): the readers use ordinary loads, and the
// 32 workgroups of an XCD share one L2 fetch of a broadcast input instead
// of each reading it from memory.  The writers store with agent-scope
// (write-through) stores.
static_assert(sizeof(MkLayer) % 16 == 0, "descriptor copied as 16-byte words");
static_assert(kNGrp <= 64 && (2 * kNGrp + 1) * 32 <= kBarWords, "barrier words");

struct MkArgs {
  const MkLayer* layers;
  float* x;        // residual [D]: the input of layer 0, the output of L-1
  float* act;      // arena, act_stride floats per layer
  float* vfirst;   // [D]
  unsigned* bar;   // kBarWords words, zero between launches
  int* err;        // set to 1 when a barrier wait ran past its limit
  int L, H, act_stride;
  int spin_limit;  // polls per barrier wait before the error is recorded
};

// ---- activations shared across workgroups (agent-scope, no L2 flush)
__device__ __forceinline__ float act_ld(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float4 act_ld4(const float* p) {
  const uint64_t* q = reinterpret_cast<const uint64_t*>(p);
  const uint64_t a = __hip_atomic_load(q, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
  const uint64_t b = __hip_atomic_load(q + 1, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
  return make_float4(__uint_as_float((uint32_t)a),
                     __uint_as_float((uint32_t)(a >> 32)),
                     __uint_as_float((uint32_t)b),
                     __uint_as_float((uint32_t)(b >> 32)));
}
__device__ __forceinline__ void act_st(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float sigm(float v) {
  return 1.f / (1.f + __expf(-v));
}

// Workgroup barrier for LDS traffic only: the LDS operations complete, then
// s_barrier.  __syncthreads() adds a workgroup-scope release fence, which
// here waits for every outstanding vector-memory operation -- the next
// phase's weight prefetch included -- so every phase would wait for its
// successor's weights at its first barrier.
__device__ __forceinline__ void lds_sync() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// ---- grid barrier (see the header comment)
struct GridBar {
  unsigned* w;
  int k = 0;          // barriers passed
  bool bad = false;   // a wait ran past its limit (this workgroup stops waiting)
  __device__ unsigned* cnt(int g) const { return w + g * 32; }
  __device__ unsigned* flag(int g) const { return w + (kNGrp + g) * 32; }
  __device__ unsigned* exitc() const { return w + 2 * kNGrp * 32; }

  // every wave's stores complete, then thread 0 counts the workgroup in;
  // the group's last arriver raises the group's flag
  __device__ void arrive() {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
      const int g = blockIdx.x / kBarGroup;
      const unsigned old = __hip_atomic_fetch_add(
          cnt(g), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (old == (unsigned)((k + 1) * kBarGroup - 1))
        __hip_atomic_store(flag(g), (unsigned)(k + 1), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  // wave 0 polls every group's flag at once (lane g reads flag g)
  __device__ void wait(int* err, int spin_limit) {
    if (threadIdx.x < 64) {
      const int lane = threadIdx.x;
      int spins = 0;
      while (!bad) {
        const bool ok =
            lane >= kNGrp ||
            __hip_atomic_load(flag(lane < kNGrp ? lane : 0), __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT) >= (unsigned)(k + 1);
        if (__all(ok)) break;
        __builtin_amdgcn_s_sleep(1);
        if (++spins >= spin_limit) {
          if (lane == 0)
            __hip_atomic_store(err, 1, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
          bad = true;
        }
      }
    }
    ++k;
    lds_sync();
  }
  // after the last wait: the last workgroup out re-arms every word
  __device__ void finish() {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
      const unsigned e = __hip_atomic_fetch_add(
          exitc(), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (e == (unsigned)gridDim.x - 1) {
        for (int i = 0; i < kNGrp; ++i) {
          __hip_atomic_store(cnt(i), 0u, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(flag(i), 0u, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
        }
        __hip_atomic_store(exitc(), 0u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
};

// ---- block reductions (256 threads)
// sh: 4 floats no wave reads or writes until every wave has passed the
// barrier inside (each phase begins after the grid barrier's workgroup
// barrier; the two sums of one LayerNorm use separate slots)
__device__ __forceinline__ float block_sum(float v, float* sh) {
  v = wave_sum_dpp(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) sh[w] = v;
  lds_sync();
  float s = 0.f;
  for (int i = 0; i < kT / 64; ++i) s += sh[i];
  return s;
}

// LN + token shift + one lerp of the decode row, into LDS (fp32), in two
// halves (ln_load, ln_finish):
//   xn = LN(x);  out = xn + (prev - xn) * coef   (prev null: zero shift)
// and, where shift_out is given, shift_out = xn (the next step's shift).
// Thread t owns columns 4 (t + 256 e); sums in the order of the per-kernel
// shift/lerp path (float4 pair sums, then the block sum), so the row
// statistics are those of that path bit for bit.
template <int KE>
struct LnIn {
  float4 v[KE], cw[KE], cb[KE], pv[KE], cf[KE];
};

// The loads of the LN + lerp.
template <int KE>
__device__ __forceinline__ void ln_load(LnIn<KE>& in, const float* x,
                                        const float* lw, const float* lb,
                                        const float* prev,
                                        const float* coef) {
#pragma unroll
  for (int e = 0; e < KE; ++e) {
    const int c = 4 * (threadIdx.x + e * kT);
    in.v[e] = *reinterpret_cast<const float4*>(x + c);
    in.cw[e] = *reinterpret_cast<const float4*>(lw + c);
    in.cb[e] = *reinterpret_cast<const float4*>(lb + c);
    in.cf[e] = *reinterpret_cast<const float4*>(coef + c);
    in.pv[e] = prev ? *reinterpret_cast<const float4*>(prev + c)
                    : make_float4(0.f, 0.f, 0.f, 0.f);
  }
}

// s_out: the row into LDS (null: not stored); keep: the thread's KE float4s
// of it in registers (null: not kept) -- columns 4 (t + 256 e), the lane
// layout of the digit staging, so a GEMV phase stages from registers
template <int KE>
__device__ __forceinline__ void ln_finish(const LnIn<KE>& in, float* s_out,
                                          float* shift_out, float* sh,
                                          float4* keep = nullptr) {
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < KE; ++e)
    s += (in.v[e].x + in.v[e].y) + (in.v[e].z + in.v[e].w);
  constexpr int D = 4 * kT * KE;
  const float mean = block_sum(s, sh) / (float)D;
  float q = 0.f;
#pragma unroll
  for (int e = 0; e < KE; ++e) {
    const float a = in.v[e].x - mean, b = in.v[e].y - mean,
                cc = in.v[e].z - mean, d = in.v[e].w - mean;
    q += (a * a + b * b) + (cc * cc + d * d);
  }
  const float var = block_sum(q, sh + 4) / (float)D;
  const float rstd = 1.f / sqrtf(var + 1e-5f);
#pragma unroll
  for (int e = 0; e < KE; ++e) {
    const int c = 4 * (threadIdx.x + e * kT);
    const float4 v = in.v[e], cw = in.cw[e], cb = in.cb[e], pv = in.pv[e],
                 cf = in.cf[e];
    float4 xn, o;
    xn.x = (v.x - mean) * rstd * cw.x + cb.x;
    xn.y = (v.y - mean) * rstd * cw.y + cb.y;
    xn.z = (v.z - mean) * rstd * cw.z + cb.z;
    xn.w = (v.w - mean) * rstd * cw.w + cb.w;
    o.x = xn.x + (pv.x - xn.x) * cf.x;
    o.y = xn.y + (pv.y - xn.y) * cf.y;
    o.z = xn.z + (pv.z - xn.z) * cf.z;
    o.w = xn.w + (pv.w - xn.w) * cf.w;
    if (s_out) *reinterpret_cast<float4*>(s_out + c) = o;
    if (keep) keep[e] = o;
    if (shift_out) *reinterpret_cast<float4*>(shift_out + c) = xn;
  }
}

// x of a GEMV phase (NG groups of 32 columns) as int8 digit words in LDS:
// per group 24 words (first, second, third digits, bytes in column order)
// and three floats (sum of columns 0..15, 2^-e or NaN for a non-finite
// group, sum of columns 16..31); 8 threads per group, 4 columns each.
template <int NG>
struct StageIn {
  static constexpr int NIT = NG * 8 / kT;     // float4s per thread
  static_assert(NIT * kT == NG * 8, "stage shape");
  float4 fv[NIT];
};

// every load of the thread in flight before the first use
template <int NG>
__device__ __forceinline__ void stage_load(StageIn<NG>& in, const float* src) {
#pragma unroll
  for (int i = 0; i < StageIn<NG>::NIT; ++i)
    in.fv[i] = reinterpret_cast<const float4*>(src)[threadIdx.x + kT * i];
}

// One 32-column group as digits, computed by 8 consecutive lanes (aligned
// to 8) holding 4 columns each (lane k: columns 4k .. 4k + 3): the group's
// largest |x| and non-finite flag over all 8 lanes and the sums of each
// half by DPP within the lane row (no LDS trip).  Returns the lane's three
// digit words (columns 4k .. 4k + 3 of the first, second, third digit), the
// half sum (lanes 0..3: columns 0..15, lanes 4..7: 16..31) and 2^-e (NaN
// for a non-finite group).
__device__ __forceinline__ void group_digits(float4 f, uint32_t& w0,
                                             uint32_t& w1, uint32_t& w2,
                                             float& sf, float& isc) {
  const float xv4[4] = {f.x, f.y, f.z, f.w};
  float amax = fmaxf(fmaxf(fabsf(f.x), fabsf(f.y)),
                     fmaxf(fabsf(f.z), fabsf(f.w)));
  float fb = (!(fabsf(f.x) <= 3.4e38f) | !(fabsf(f.y) <= 3.4e38f) |
              !(fabsf(f.z) <= 3.4e38f) | !(fabsf(f.w) <= 3.4e38f))
                 ? 1.f : 0.f;
  sf = (f.x + f.y) + (f.z + f.w);
  amax = fmaxf(amax, dpp_f<0xB1>(amax));      // quad_perm [1,0,3,2]
  fb = fmaxf(fb, dpp_f<0xB1>(fb));
  sf += dpp_f<0xB1>(sf);
  amax = fmaxf(amax, dpp_f<0x4E>(amax));      // quad_perm [2,3,0,1]
  fb = fmaxf(fb, dpp_f<0x4E>(fb));
  sf += dpp_f<0x4E>(sf);
  amax = fmaxf(amax, dpp_f<0x141>(amax));     // row_half_mirror: the
  fb = fmaxf(fb, dpp_f<0x141>(fb));           // other quad of the 8
  const bool bad = fb > 0.f;
  const int e = digit_exp(amax);
  w0 = w1 = w2 = 0u;
#pragma unroll
  for (int bb = 0; bb < 4; ++bb) {
    uint32_t b0, b1, b2;
    x_digit3(bad ? 0.f : xv4[bb], e, b0, b1, b2);
    w0 |= b0 << (8 * bb);
    w1 |= b1 << (8 * bb);
    w2 |= b2 << (8 * bb);
  }
  isc = bad ? __builtin_nanf("") : ldexpf(1.f, -e);
}

template <int NG>
__device__ __forceinline__ void stage_digits(const StageIn<NG>& in,
                                             uint32_t* s_xh, float* s_xs) {
  constexpr int NIT = StageIn<NG>::NIT;
#pragma unroll
  for (int i = 0; i < NIT; ++i) {
    const int it = threadIdx.x + kT * i;
    const int gg = it >> 3, k = it & 7;
    uint32_t w0, w1, w2;
    float sf, isc;
    group_digits(in.fv[i], w0, w1, w2, sf, isc);
    uint32_t* dst = s_xh + gg * 24;
    dst[k] = w0;
    dst[8 + k] = w1;
    dst[16 + k] = w2;
    if (k == 0) {
      s_xs[gg * 3] = sf;
      s_xs[gg * 3 + 1] = isc;
    }
    if (k == 4) s_xs[gg * 3 + 2] = sf;
  }
}

// A producer's groups stored in global memory in the staged form: 32 words
// per group (24 digit words, the sum of columns 0..15, 2^-e, the sum of
// columns 16..31, 5 unused), written by the 8 lanes of the group.
__device__ __forceinline__ void store_group_digits(float* g32, int k,
                                                   uint32_t w0, uint32_t w1,
                                                   uint32_t w2, float sf,
                                                   float isc) {
  act_st(g32 + k, __uint_as_float(w0));
  act_st(g32 + 8 + k, __uint_as_float(w1));
  act_st(g32 + 16 + k, __uint_as_float(w2));
  if (k == 0) {
    act_st(g32 + 24, sf);
    act_st(g32 + 25, isc);
  }
  if (k == 4) act_st(g32 + 26, sf);
}

// Consumer: NG groups in that form (global) into the LDS staging layout.
template <int NG>
struct DigIn {
  static constexpr int NIT = NG * 7 / kT + ((NG * 7) % kT != 0);
  uint4 v[NIT];
};

template <int NG>
__device__ __forceinline__ void dig_load(DigIn<NG>& in, const float* src) {
#pragma unroll
  for (int i = 0; i < DigIn<NG>::NIT; ++i) {
    const int it = min((int)threadIdx.x + kT * i, NG * 7 - 1);
    const int g = it / 7, q = it - 7 * (it / 7);
    in.v[i] = reinterpret_cast<const uint4*>(src + g * 32)[q];
  }
}

template <int NG>
__device__ __forceinline__ void dig_store(const DigIn<NG>& in,
                                          uint32_t* s_xh, float* s_xs) {
#pragma unroll
  for (int i = 0; i < DigIn<NG>::NIT; ++i) {
    const int it = (int)threadIdx.x + kT * i;
    if (it >= NG * 7) break;
    const int g = it / 7, q = it - 7 * (it / 7);
    const uint4 v = in.v[i];
    if (q < 6) {
      *reinterpret_cast<uint4*>(s_xh + g * 24 + 4 * q) = v;
    } else {
      s_xs[g * 3] = __uint_as_float(v.x);
      s_xs[g * 3 + 1] = __uint_as_float(v.y);
      s_xs[g * 3 + 2] = __uint_as_float(v.z);
    }
  }
}

// One lane's x digits of group g (registers), and for sym6 the digits in
// the order of the crumb words.
template <int FMT>
struct XDig {
  uint32_t h[16];
  uint32_t l[8];
  uint32_t c[FMT == F_SYM6 ? 24 : 1];
  float sa, sc, sb;
};

template <int FMT>
__device__ __forceinline__ void xdig_load(XDig<FMT>& x, const uint32_t* s_xh,
                                          const float* s_xs, int g) {
  const uint4* src = reinterpret_cast<const uint4*>(s_xh + g * 24);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint4 v = src[q];
    x.h[4 * q] = v.x; x.h[4 * q + 1] = v.y;
    x.h[4 * q + 2] = v.z; x.h[4 * q + 3] = v.w;
  }
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const uint4 v = src[4 + q];
    x.l[4 * q] = v.x; x.l[4 * q + 1] = v.y;
    x.l[4 * q + 2] = v.z; x.l[4 * q + 3] = v.w;
  }
  x.sa = s_xs[g * 3];
  x.sc = s_xs[g * 3 + 1];
  x.sb = s_xs[g * 3 + 2];
  if constexpr (FMT == F_SYM6) {
#pragma unroll
    for (int d = 0; d < 3; ++d)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const uint32_t* s = d < 2 ? &x.h[8 * d + 4 * hh] : &x.l[4 * hh];
        byte_transpose4(s[0], s[1], s[2], s[3], &x.c[8 * d + 4 * hh]);
      }
  }
}

// Lane partial of one (row, group): the block sums of code * x as exact
// int32 digit dot products, then the format's block scales in fp32
// (rtn8: the row scale is applied by the caller).
template <int FMT>
__device__ __forceinline__ float group_dot(const Raw& r, const XDig<FMT>& x,
                                           int g) {
  uint32_t cw[8];
  if constexpr (FMT == F_SYM6) {
    const uint32_t nw[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
    cw[0] = nw[0] & 0x0F0F0F0Fu;         cw[1] = nw[1] & 0x0F0F0F0Fu;
    cw[2] = (nw[0] >> 4) & 0x0F0F0F0Fu;  cw[3] = (nw[1] >> 4) & 0x0F0F0F0Fu;
    cw[4] = nw[2] & 0x0F0F0F0Fu;         cw[5] = nw[3] & 0x0F0F0F0Fu;
    cw[6] = (nw[2] >> 4) & 0x0F0F0F0Fu;  cw[7] = (nw[3] >> 4) & 0x0F0F0F0Fu;
  } else if constexpr (FMT == F_RTN8 || FMT == F_SYM8) {
    cw[0] = r.a.x; cw[1] = r.a.y; cw[2] = r.a.z; cw[3] = r.a.w;
    cw[4] = r.b.x; cw[5] = r.b.y; cw[6] = r.b.z; cw[7] = r.b.w;
  } else {
    const uint32_t nw[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      cw[k] = nw[k] & 0x0F0F0F0Fu;
      cw[4 + k] = (nw[k] >> 4) & 0x0F0F0F0Fu;
      if constexpr (FMT == F_SB6_5) {
        const uint32_t H = r.h.x;
        cw[k] |= spread4((H >> (4 * k)) & 15u) << 4;
        cw[4 + k] |= spread4((H >> (16 + 4 * k)) & 15u) << 4;
      }
    }
  }
  int a0 = 0, a1 = 0, a2 = 0, b0 = 0, b1 = 0, b2 = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    a0 = __builtin_amdgcn_sdot4((int)cw[k], (int)x.h[k], a0, false);
    a1 = __builtin_amdgcn_sdot4((int)cw[k], (int)x.h[8 + k], a1, false);
    a2 = __builtin_amdgcn_sdot4((int)cw[k], (int)x.l[k], a2, false);
    b0 = __builtin_amdgcn_sdot4((int)cw[4 + k], (int)x.h[4 + k], b0, false);
    b1 = __builtin_amdgcn_sdot4((int)cw[4 + k], (int)x.h[12 + k], b1, false);
    b2 = __builtin_amdgcn_sdot4((int)cw[4 + k], (int)x.l[4 + k], b2, false);
  }
  float dA, dB;
  if constexpr (FMT == F_SYM6) {
    // stored code u = nibble + 16 crumb = q + 32
    const uint32_t W0 = r.h.x, W1 = r.h.y;
    int ca0 = 0, ca1 = 0, ca2 = 0, cb0 = 0, cb1 = 0, cb2 = 0;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int c0 = (int)((W0 >> (2 * t)) & 0x03030303u);
      const int c1 = (int)((W1 >> (2 * t)) & 0x03030303u);
      ca0 = __builtin_amdgcn_sdot4(c0, (int)x.c[t], ca0, false);
      ca1 = __builtin_amdgcn_sdot4(c0, (int)x.c[8 + t], ca1, false);
      ca2 = __builtin_amdgcn_sdot4(c0, (int)x.c[16 + t], ca2, false);
      cb0 = __builtin_amdgcn_sdot4(c1, (int)x.c[4 + t], cb0, false);
      cb1 = __builtin_amdgcn_sdot4(c1, (int)x.c[12 + t], cb1, false);
      cb2 = __builtin_amdgcn_sdot4(c1, (int)x.c[20 + t], cb2, false);
    }
    a0 += ca0 << 4; a1 += ca1 << 4; a2 += ca2 << 4;
    b0 += cb0 << 4; b1 += cb1 << 4; b2 += cb2 << 4;
    dA = digit_sum(a0, a1, a2) * x.sc - 32.f * x.sa;
    dB = digit_sum(b0, b1, b2) * x.sc - 32.f * x.sb;
  } else {
    dA = digit_sum(a0, a1, a2) * x.sc;
    dB = digit_sum(b0, b1, b2) * x.sc;
  }
  if constexpr (FMT <= F_SB6_6) {
    const int kb = g & 7;
    const int qs_word = (6 * kb) >> 5, qs_sh = (6 * kb) & 31;
    const int qm_word = (48 + 6 * kb) >> 5, qm_sh = (48 + 6 * kb) & 31;
    const uint32_t rr[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
    uint32_t lo = qs_word == 0 ? rr[0] : rr[1];
    uint32_t hi = qs_word == 0 ? rr[1] : rr[2];
    const uint32_t qsv = __builtin_amdgcn_alignbit(hi, lo, (uint32_t)qs_sh) & 63u;
    lo = qm_word == 1 ? rr[1] : rr[2];
    hi = qm_word == 1 ? rr[2] : rr[3];
    const uint32_t qmv = __builtin_amdgcn_alignbit(hi, lo, (uint32_t)qm_sh) & 63u;
    const float d = f16_bits_to_f32(rr[3] & 0xFFFFu);
    const float dm = f16_bits_to_f32(rr[3] >> 16);
    const float s = fmaxf(f16_round((float)qsv * d), 1e-8f);
    const float m = f16_round((float)((int)qmv - 31) * dm);
    return s * (dA + dB) + m * (x.sa + x.sb);
  } else if constexpr (FMT == F_SYM6 || FMT == F_SYM8) {
    const float d = f16_bits_to_f32(r.dd);
    const float sA = f16_round((float)(int8_t)(r.s & 0xFFu) * d);
    const float sB = f16_round((float)(int8_t)((r.s >> 8) & 0xFFu) * d);
    return sA * dA + sB * dB;
  } else {
    return dA + dB;
  }
}

// Row results of a wave, one per row j, gathered into lane j.
template <int R>
__device__ __forceinline__ float gather_rows(const float (&acc)[R]) {
  const int lane = threadIdx.x & 63;
  float out = 0.f;
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const float s = wave_sum_dpp(acc[j]);
    if (lane == j) out = s;
  }
  return out;
}

// One weight, rounded as the dequant kernels round it.
__device__ __forceinline__ float dq_asym_1(uint32_t code, float s, float m) {
#pragma clang fp contract(off)
  return (float)code * s + m;
}

__device__ __forceinline__ float epi_apply(float v, int epi) {
  switch (epi) {
    case RWKVQ_EPI_TANH: return tanhf(v);
    case RWKVQ_EPI_SIGMOID: return 1.f / (1.f + __expf(-v));
    default: return v;
  }
}

template <int FP, int FC, int KQ>
__global__ void __launch_bounds__(kT)
decode_mk_k(MkArgs A) {
  constexpr int D = 256 * KQ;          // model width
  constexpr int NGD = D / 32;          // groups per D-wide row (64)
  constexpr int F = 4 * D;             // channel-mix width
  constexpr int NGF = F / 32;
  constexpr int KGF = NGF / 64;        // groups per lane of a F-wide row
  constexpr int KE = D / (4 * kT);     // float4s per thread of a row
  constexpr int RPW1 = 3 * D / (kRkvWgs * 4);   // r/k/v rows per wave
  constexpr int RPG1 = 4 * RPW1;
  constexpr int RPW3 = D / kW;         // o / value rows per wave
  constexpr int RPW4 = F / kW;         // key rows per wave
  constexpr bool NTP = FP <= F_SB6_6, NTC = FC <= F_SB6_6;
  static_assert(NGD == 64 && RPW3 >= 1 && RPG1 * kRkvWgs == 3 * D &&
                D % RPG1 == 0, "decode kernel shape");
  // a key workgroup's rows are one 32-column group of the value input
  static_assert(4 * RPW4 == 32 && NGF == kG, "key rows per workgroup");
  // the LayerNorm's registers are the digit staging's input
  static_assert(StageIn<NGD>::NIT == KE, "LN / staging lane layout");

  extern __shared__ uint32_t smem[];
  // the layer descriptors, copied once: fields are then LDS reads instead
  // of scalar loads that miss the scalar cache on every layer
  const MkLayer* s_tab = reinterpret_cast<const MkLayer*>(smem);
  {
    constexpr int kW4 = (int)(sizeof(MkLayer) / 16);
    const uint4* src = reinterpret_cast<const uint4*>(A.layers);
    uint4* dst = reinterpret_cast<uint4*>(smem);
    for (int i = threadIdx.x; i < A.L * kW4; i += kT) dst[i] = src[i];
    __syncthreads();
  }
  uint32_t* const smem2 = smem + A.L * (int)(sizeof(MkLayer) / 4);
  float* s_row = reinterpret_cast<float*>(smem2);          // [D] fp32
  uint32_t* s_xh = smem2 + D;                             // [NGF * 24]
  float* s_xs = reinterpret_cast<float*>(s_xh + NGF * 24);  // [NGF * 3]
  __shared__ float sh[16];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wg = blockIdx.x;
  const int gw = wg * 4 + wave;
  GridBar bar{A.bar};

  // prefetched operands, one phase ahead
  Raw r1[RPW1];                        // P1 r/k/v rows
  uint32_t cq[2][KQ];                  // P1 LoRA down codes (2 rows / wave)
  uint4 smv[KQ / 2];                   // P1 the workgroup's block scales /
                                       // mins (asym) or column scales (int8)
  int jb = -1;                         // P1 LoRA job of this workgroup
  float S[16];                         // P2 state row slice
  uint4 cv[kMkCv];                     // P2 LoRA up code blocks
  float4 pc0, pc1;                     // P2 per-channel constants
  float4 psv, pmv;                     // P2 LoRA up scale / min per rank
  Raw r3[RPW3], r4[RPW4], r5[RPW3][KGF];

  // The role of a workgroup in P1 / P2 is a run-time condition: every
  // prefetch register is (re)defined on every path, so that its live range
  // runs from its phase's prefetch to its use and not around the layer loop.
  auto pf1 = [&](const MkLayer& Ly) {
#pragma unroll
    for (int j = 0; j < RPW1; ++j) r1[j] = Raw{};
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int k = 0; k < KQ; ++k) cq[r][k] = 0u;
#pragma unroll
    for (int q = 0; q < KQ / 2; ++q) smv[q] = make_uint4(0u, 0u, 0u, 0u);
    if (wg < kRkvWgs) {
      const int row0 = wg * RPG1 + wave * RPW1;
#pragma unroll
      for (int j = 0; j < RPW1; ++j)
        load_raw<FP, NTP>(Ly.rkv, row0 + j, NGD, D / 256, lane, r1[j]);
      return;
    }
    const int lw = wg - kRkvWgs;
    jb = -1;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (j < Ly.n_down && lw >= Ly.down[j].wg0 &&
          lw < Ly.down[j].wg0 + (Ly.down[j].rows + 7) / 8)
        jb = j;
    if (jb < 0) return;
    const MkDown& dn = jb == 0 ? Ly.down[0] : jb == 1 ? Ly.down[1]
                     : jb == 2 ? Ly.down[2] : Ly.down[3];
    const int r0 = (lw - dn.wg0) * 8 + wave * 2;
    const int rr = min(r0, dn.rows - 2);
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int k = 0; k < KQ; ++k)
        cq[r][k] = *reinterpret_cast<const GLB uint32_t*>(
            dn.q + (size_t)(rr + r) * D + 4 * (lane + 64 * k));
    // the block parameters of the workgroup's 8 rows (one 64-row block),
    // once per workgroup: D scales and D mins (asym) or D fp16 column
    // scales (int8), KQ / 2 16-byte words per thread
    if (dn.s) {
      const GLB uint4* sp = reinterpret_cast<const GLB uint4*>(
          dn.s + (size_t)(rr >> 6) * D);
      const GLB uint4* mp = reinterpret_cast<const GLB uint4*>(
          dn.m + (size_t)(rr >> 6) * D);
#pragma unroll
      for (int q = 0; q < KQ / 4; ++q) {
        smv[q] = sp[threadIdx.x + kT * q];
        smv[KQ / 4 + q] = mp[threadIdx.x + kT * q];
      }
    } else {
      const GLB uint4* cp = reinterpret_cast<const GLB uint4*>(dn.sc);
#pragma unroll
      for (int q = 0; q < KQ / 8; ++q) smv[q] = cp[threadIdx.x + kT * q];
    }
  };
  auto pf2 = [&](const MkLayer& Ly) {
#pragma unroll
    for (int c = 0; c < 16; ++c) S[c] = 0.f;
#pragma unroll
    for (int q = 0; q < kMkCv; ++q) cv[q] = make_uint4(0u, 0u, 0u, 0u);
    pc0 = pc1 = psv = pmv = make_float4(0.f, 0.f, 0.f, 0.f);
    if (wg >= A.H) return;
    const int h = wg, tid = threadIdx.x;
    // the head's constants: per-channel parameters and the LoRA up block
    // scales / mins of rank position tid
    if (tid < kHd) {
      const int c = h * kHd + tid;
      pc0 = make_float4(Ly.w0[c], Ly.a0[c], Ly.k_k[c],
                        Ly.k_a[c]);
      pc1 = make_float4(Ly.r_k[c], Ly.lnx_w[c], Ly.lnx_b[c],
                        Ly.layer0 ? 0.f : Ly.v0[c]);
    }
    const MkUp& u = Ly.up;
    auto sm = [&](const float* sk, const float* mk, const uint16_t* sck,
                  int rk, float& sv, float& mv) {
      if (tid >= rk) return;
      if (sk) {
        sv = sk[(size_t)h * rk + tid];
        mv = mk[(size_t)h * rk + tid];
      } else {
        sv = f16_bits_to_f32(sck[tid]);
      }
    };
    sm(u.s[0], u.m[0], u.sc[0], u.r[0], psv.x, pmv.x);
    sm(u.s[1], u.m[1], u.sc[1], u.r[1], psv.y, pmv.y);
    sm(u.s[2], u.m[2], u.sc[2], u.r[2], psv.z, pmv.z);
    sm(u.s[3], u.m[3], u.sc[3], u.r[3], psv.w, pmv.w);
    const int i = tid >> 2, part = tid & 3;
    const GLB float* sp = Ly.state_in + ((size_t)h * kHd + i) * kHd + part * 16;
#pragma unroll
    for (int c = 0; c < 16; c += 4) {
      const float4 q = *reinterpret_cast<const GLB float4*>(sp + c);
      S[c] = q.x; S[c + 1] = q.y; S[c + 2] = q.z; S[c + 3] = q.w;
    }
    const int o1 = u.r[0], o2 = o1 + u.r[1], o3 = o2 + u.r[2];
    const int nb = (o3 + u.r[3]) >> 4;
#pragma unroll
    for (int q = 0; q < kMkCv; ++q) {
      const int b = wave + 4 * q;
      if (b < nb) {
        const int p = 16 * b;
        const int k = p < o1 ? 0 : p < o2 ? 1 : p < o3 ? 2 : 3;
        const uint8_t* qk = k == 0 ? u.q[0] : k == 1 ? u.q[1]
                          : k == 2 ? u.q[2] : u.q[3];
        const int rk = k == 0 ? u.r[0] : k == 1 ? u.r[1]
                     : k == 2 ? u.r[2] : u.r[3];
        const int off = k == 0 ? 0 : k == 1 ? o1 : k == 2 ? o2 : o3;
        const int lb = (p - off) >> 4;
        cv[q] = ld16(qk + (((size_t)h * (rk >> 4) + lb) * kHd + lane) * 16);
      }
    }
  };
  auto pf3 = [&](const MkLayer& Ly) {
#pragma unroll
    for (int j = 0; j < RPW3; ++j)
      load_raw<FP, NTP>(Ly.o, gw * RPW3 + j, NGD, D / 256, lane, r3[j]);
  };
  auto pf4 = [&](const MkLayer& Ly) {
#pragma unroll
    for (int j = 0; j < RPW4; ++j)
      load_raw<FC, NTC>(Ly.key, gw * RPW4 + j, NGD, D / 256, lane, r4[j]);
  };
  auto pf5 = [&](const MkLayer& Ly) {
#pragma unroll
    for (int j = 0; j < RPW3; ++j)
#pragma unroll
      for (int kg = 0; kg < KGF; ++kg)
        load_raw<FC, NTC>(Ly.val, gw * RPW3 + j, NGF, F / 256,
                          lane + 64 * kg, r5[j][kg]);
  };

  pf1(s_tab[0]);
  for (int l = 0; l < A.L; ++l) {
    const MkLayer& Ly = s_tab[l];
    float* const a_rkv = A.act + (size_t)l * A.act_stride;
    float* const a_o = a_rkv + 3 * D;
    float* const a_xm = a_o + D;
    float* const a_hk = a_xm + D;
    float* const a_xo = l == A.L - 1 ? A.x : a_hk + F;
    const float* const a_xi = l == 0 ? A.x : A.act + (size_t)(l - 1) * A.act_stride + 5 * D + F;
    if (l > 0) {
      bar.arrive();
      pf1(Ly);
      bar.wait(A.err, A.spin_limit);
    }
    // ---------------- P1: LN1 + lerp, r/k/v rows, LoRA down products
    if (wg < kRkvWgs) {
      const int row0 = wg * RPG1;
      const int slot = row0 / D;
      LnIn<KE> li;
      ln_load<KE>(li, a_xi, Ly.ln1_w, Ly.ln1_b, Ly.tshift_in,
                  Ly.coef + slot * D);
      {
        StageIn<NGD> si;
        ln_finish<KE>(li, nullptr, wg == 0 ? Ly.tshift_out : nullptr, sh,
                      si.fv);
        stage_digits<NGD>(si, s_xh, s_xs);
      }
      lds_sync();
      XDig<FP> xd;
      xdig_load<FP>(xd, s_xh, s_xs, lane);
      float acc[RPW1];
#pragma unroll
      for (int j = 0; j < RPW1; ++j) acc[j] = group_dot<FP>(r1[j], xd, lane);
      const float v = gather_rows<RPW1>(acc);
      if (lane < RPW1) act_st(a_rkv + row0 + wave * RPW1 + lane, v);
    } else if (jb >= 0) {
      const MkDown& dn = jb == 0 ? Ly.down[0] : jb == 1 ? Ly.down[1]
                       : jb == 2 ? Ly.down[2] : Ly.down[3];
      // the prefetched block parameters into LDS (the digit area is free in
      // this role); visible after the LN's first barrier
      float* s_sm = reinterpret_cast<float*>(s_xh);
#pragma unroll
      for (int q = 0; q < KQ / 2; ++q)
        reinterpret_cast<uint4*>(s_sm)[threadIdx.x + kT * q] = smv[q];
      LnIn<KE> li;
      ln_load<KE>(li, a_xi, Ly.ln1_w, Ly.ln1_b, Ly.tshift_in,
                  Ly.coef + dn.slot * D);
      ln_finish<KE>(li, s_row, nullptr, sh);
      lds_sync();
      const int lw = wg - kRkvWgs;
      const int r0 = (lw - dn.wg0) * 8 + wave * 2;
      const float4* xr = reinterpret_cast<const float4*>(s_row);
      float a0 = 0.f, a1 = 0.f;
      // one body per code format, chosen by a wave-uniform (scalar) test:
      // asym codes (fp32 scale and min per column) or int8 codes (fp16
      // scale per column); each weight is the format's dequantized value
      auto down_dot = [&](auto asym) {
        // every LDS operand first (one wait), then the arithmetic
        float4 sv[KQ], mv[KQ], xv[KQ];
#pragma unroll
        for (int k = 0; k < KQ; ++k) {
          const int c0 = 4 * (lane + 64 * k);
          if constexpr (decltype(asym)::value) {
            sv[k] = *reinterpret_cast<const float4*>(s_sm + c0);
            mv[k] = *reinterpret_cast<const float4*>(s_sm + D + c0);
          } else {
            const uint2 scv = *reinterpret_cast<const uint2*>(
                reinterpret_cast<const uint16_t*>(s_sm) + c0);
            sv[k] = make_float4(h2_lo(scv.x), h2_hi(scv.x), h2_lo(scv.y),
                                h2_hi(scv.y));
            mv[k] = make_float4(0.f, 0.f, 0.f, 0.f);
          }
          xv[k] = xr[lane + 64 * k];
        }
#pragma unroll
        for (int k = 0; k < KQ; ++k) {
          const float sk[4] = {sv[k].x, sv[k].y, sv[k].z, sv[k].w};
          const float mk[4] = {mv[k].x, mv[k].y, mv[k].z, mv[k].w};
          const float xe[4] = {xv[k].x, xv[k].y, xv[k].z, xv[k].w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t b0 = (cq[0][k] >> (8 * e)) & 0xFFu;
            const uint32_t b1 = (cq[1][k] >> (8 * e)) & 0xFFu;
            float w0, w1;
            if constexpr (decltype(asym)::value) {
              w0 = dq_asym_1(b0, sk[e], mk[e]);
              w1 = dq_asym_1(b1, sk[e], mk[e]);
            } else {
              w0 = (float)(int)(int8_t)b0 * sk[e];
              w1 = (float)(int)(int8_t)b1 * sk[e];
            }
            a0 = fmaf(xe[e], w0, a0);
            a1 = fmaf(xe[e], w1, a1);
          }
        }
      };
      if (__builtin_amdgcn_readfirstlane(dn.s != nullptr ? 1 : 0))
        down_dot(std::integral_constant<bool, true>{});
      else
        down_dot(std::integral_constant<bool, false>{});
      a0 = wave_sum_dpp(a0);
      a1 = wave_sum_dpp(a1);
      if (r0 < dn.rows && lane < 2)
        act_st(dn.y + r0 + lane, epi_apply(lane == 0 ? a0 : a1, dn.epi));
    }
    bar.arrive();
    pf2(Ly);
    bar.wait(A.err, A.spin_limit);

    // ---------------- P2: WKV step of head wg
    if (wg < A.H) {
      __shared__ float4 s_w[kHd / 4], s_k[kHd / 4], s_a[kHd / 4],
          s_b[kHd / 4], s_r[kHd / 4];
      __shared__ float s_v[kHd], s_y[kHd];
      __shared__ float s_dp;
      __shared__ float s_up[4][kHd];
      __shared__ float4 s_hs4[kMkMaxCat / 4];
      __shared__ float s_bm[kMkMaxCat / 16];
      __shared__ float s_red[4][4][kHd];
      float* s_hs = reinterpret_cast<float*>(s_hs4);
      const int h = wg, tid = threadIdx.x;
      const int i = tid >> 2, part = tid & 3;
      const MkUp& u = Ly.up;
      const int layer0 = Ly.layer0;
      float r = 0.f, k = 0.f, v = 0.f, vf = 0.f;
      const float w0c = pc0.x, a0c = pc0.y, kkc = pc0.z, kac = pc0.w,
                  rkc = pc1.x, lw = pc1.y, lb = pc1.z, v0c = pc1.w;
      if (tid < kHd) {
        const int c = h * kHd + tid;
        r = a_rkv[c];
        k = a_rkv[D + c];
        v = a_rkv[2 * D + c];
        if (!layer0) vf = act_ld(A.vfirst + c);
      }
      const int o1 = u.r[0], o2 = o1 + u.r[1], o3 = o2 + u.r[2];
      const int nb = (o3 + u.r[3]) >> 4;
      // h_j s_j and h_j m_j (int8: -128 h_j s_j) over the concatenated
      // rank axis w, a, v, g (an absent branch has rank 0; ranks <= 256, one
      // position per thread): every load issued before the first use
      float hv[4];
#pragma unroll
      for (int kb2 = 0; kb2 < 4; ++kb2) {
        const int rk = u.r[kb2];
        hv[kb2] = 0.f;
        if (tid >= rk) continue;
        const float* hp = kb2 == 0 ? u.h[0] : kb2 == 1 ? u.h[1]
                        : kb2 == 2 ? u.h[2] : u.h[3];
        hv[kb2] = hp[tid];
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int kb2 = 0; kb2 < 4; ++kb2) {
        const int rk = u.r[kb2];
        const int off = kb2 == 0 ? 0 : kb2 == 1 ? o1 : kb2 == 2 ? o2 : o3;
        const bool asym = (kb2 == 0 ? u.s[0] : kb2 == 1 ? u.s[1]
                           : kb2 == 2 ? u.s[2] : u.s[3]) != nullptr;
        const float svk = kb2 == 0 ? psv.x : kb2 == 1 ? psv.y
                        : kb2 == 2 ? psv.z : psv.w;
        const float mvk = kb2 == 0 ? pmv.x : kb2 == 1 ? pmv.y
                        : kb2 == 2 ? pmv.z : pmv.w;
        const float hs = hv[kb2] * svk;
        // the block term of each 16-rank code block: ranks are multiples
        // of 16, so a block's positions are the 16 lanes of one DPP row
        // (all active or all past the rank)
        float bm = asym ? hv[kb2] * mvk : -128.f * hs;
        bm += dpp_f<0xB1>(bm);
        bm += dpp_f<0x4E>(bm);
        bm += dpp_f<0x141>(bm);
        bm += dpp_f<0x140>(bm);
        if (tid < rk) {
          s_hs[off + tid] = hs;
          if ((tid & 15) == 0) s_bm[(off + tid) >> 4] = bm;
        }
      }
      lds_sync();
      // Branch-free over the code blocks of the wave (blocks wave, wave + 4,
      // ...), so the LDS reads of all blocks can be issued together: a block
      // past the last one reads block 0 and adds nothing.  The branch of a
      // block, its int8 flip and the accumulator it joins are selects.
      const uint32_t amask = (u.s[0] ? 1u : 0u) | (u.s[1] ? 2u : 0u) |
                             (u.s[2] ? 4u : 0u) | (u.s[3] ? 8u : 0u);
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
      auto up_blocks = [&](auto q0c, auto q1c) {
        constexpr int Q0 = decltype(q0c)::value, Q1 = decltype(q1c)::value;
        constexpr int NQ = Q1 - Q0;
        // every LDS read of the chunk in flight before the first use
        float4 hsv[NQ][4];
        float bmv[NQ];
#pragma unroll
        for (int q = Q0; q < Q1; ++q) {
          const int b = wave + 4 * q;
          const int bc = b < nb ? b : 0;
#pragma unroll
          for (int qd = 0; qd < 4; ++qd) hsv[q - Q0][qd] = s_hs4[4 * bc + qd];
          bmv[q - Q0] = s_bm[bc];
        }
#pragma unroll
        for (int q = Q0; q < Q1; ++q) {
          const int b = wave + 4 * q;
          // 1 for a live block, 0 past the last one; opaque to the
          // compiler, which would otherwise branch around each block
          float lm = b < nb ? 1.f : 0.f;
          asm volatile("" : "+v"(lm));
          const int p = 16 * b;
          const int kb2 = (p >= o1) + (p >= o2) + (p >= o3);
          const uint32_t flip = ((amask >> kb2) & 1u) ? 0u : 0x80808080u;
          const uint32_t wd[4] = {cv[q].x ^ flip, cv[q].y ^ flip,
                                  cv[q].z ^ flip, cv[q].w ^ flip};
          float d0 = 0.f, d1 = 0.f;
#pragma unroll
          for (int qd = 0; qd < 4; ++qd) {
            const float4 hs = hsv[q - Q0][qd];
            const uint32_t wv = wd[qd];
            d0 = fmaf((float)(wv & 0xFFu), hs.x, d0);
            d1 = fmaf((float)((wv >> 8) & 0xFFu), hs.y, d1);
            d0 = fmaf((float)((wv >> 16) & 0xFFu), hs.z, d0);
            d1 = fmaf((float)(wv >> 24), hs.w, d1);
          }
          const float d = ((d0 + d1) + bmv[q - Q0]) * lm;
          acc[0] += kb2 == 0 ? d : 0.f;
          acc[1] += kb2 == 1 ? d : 0.f;
          acc[2] += kb2 == 2 ? d : 0.f;
          acc[3] += kb2 == 3 ? d : 0.f;
        }
      };
      // chunks of 4, 4 and 2 blocks per wave: 32 blocks (ranks 512) run
      // exactly two chunks, no dead slot
      static_assert(kMkCv == 10, "up-product chunks");
      up_blocks(std::integral_constant<int, 0>{},
                std::integral_constant<int, 4>{});
      if (nb > 16)
        up_blocks(std::integral_constant<int, 4>{},
                  std::integral_constant<int, 8>{});
      if (nb > 32)
        up_blocks(std::integral_constant<int, 8>{},
                  std::integral_constant<int, 10>{});
#pragma unroll
      for (int q = 0; q < 4; ++q) s_red[wave][q][lane] = acc[q];
      lds_sync();
      float vp = 0.f;
      if (tid < kHd) {
        float up[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
          up[q] = (s_red[0][q][tid] + s_red[1][q][tid]) +
                  (s_red[2][q][tid] + s_red[3][q][tid]);
        const int c = h * kHd + tid;
        const float wv = __expf(-0.606531f * sigm(up[0] + w0c));
        const float av = sigm(up[1] + a0c);
        const float kkr = k * kkc;
        const float kk = kkr / sqrtf(wave_sum_dpp(kkr * kkr) + 1e-12f);
        const float kp = k * (1.f + (av - 1.f) * kac);
        if (!layer0) v = v + (vf - v) * sigm(up[2] + v0c);
        else act_st(A.vfirst + c, v);
        const float dp = wave_sum_dpp(r * kp * rkc);
        reinterpret_cast<float*>(s_w)[tid] = wv;
        reinterpret_cast<float*>(s_k)[tid] = kp;
        reinterpret_cast<float*>(s_a)[tid] = -kk;
        reinterpret_cast<float*>(s_b)[tid] = kk * av;
        reinterpret_cast<float*>(s_r)[tid] = r;
        s_v[tid] = v;
        s_up[3][tid] = up[3];
        if (tid == 0) s_dp = dp;
        vp = v;
      }
      lds_sync();
      const float vi = s_v[i];
      float sa = 0.f;
#pragma unroll
      for (int c = 0; c < 16; c += 4) {
        const float4 a4 = s_a[part * 4 + c / 4];
        sa += S[c] * a4.x + S[c + 1] * a4.y + S[c + 2] * a4.z + S[c + 3] * a4.w;
      }
      sa += dpp_f<0xB1>(sa);
      sa += dpp_f<0x4E>(sa);
      float yv2 = 0.f;
#pragma unroll
      for (int c = 0; c < 16; c += 4) {
        const int q = part * 4 + c / 4;
        const float4 w4 = s_w[q], b4 = s_b[q], k4 = s_k[q], r4 = s_r[q];
        S[c] = S[c] * w4.x + sa * b4.x + vi * k4.x;
        S[c + 1] = S[c + 1] * w4.y + sa * b4.y + vi * k4.y;
        S[c + 2] = S[c + 2] * w4.z + sa * b4.z + vi * k4.z;
        S[c + 3] = S[c + 3] * w4.w + sa * b4.w + vi * k4.w;
        yv2 += S[c] * r4.x + S[c + 1] * r4.y + S[c + 2] * r4.z + S[c + 3] * r4.w;
      }
      yv2 += dpp_f<0xB1>(yv2);
      yv2 += dpp_f<0x4E>(yv2);
      float* so = Ly.state_out + ((size_t)h * kHd + i) * kHd + part * 16;
#pragma unroll
      for (int c = 0; c < 16; c += 4)
        *reinterpret_cast<float4*>(so + c) =
            make_float4(S[c], S[c + 1], S[c + 2], S[c + 3]);
      if (part == 0) s_y[i] = yv2;
      lds_sync();
      if (tid < kHd) {
        const float yy = s_y[tid];
        const float mean = wave_sum_dpp(yy) * (1.f / kHd);
        const float dv = yy - mean;
        const float var = wave_sum_dpp(dv * dv) * (1.f / kHd);
        const float nrm = dv / sqrtf(var + 64e-5f);
        s_row[tid] = ((nrm * lw + lb) + s_dp * vp) * s_up[3][tid];
      }
      // the head's 64 outputs = two groups of the output projection's
      // input, stored once as digits (lanes 0..7 and 8..15 of wave 0);
      // wave 0 wrote all 64 and reads its own LDS writes (in order)
      if (wave == 0) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        const float4 f = reinterpret_cast<const float4*>(s_row)[lane & 15];
        uint32_t w0, w1, w2;
        float sf, isc;
        group_digits(f, w0, w1, w2, sf, isc);
        if (lane < 16)
          store_group_digits(a_o + (2 * h + (lane >> 3)) * 32, lane & 7, w0,
                             w1, w2, sf, isc);
      }
    }
    bar.arrive();
    pf3(Ly);
    bar.wait(A.err, A.spin_limit);

    // ---------------- P3: output projection, += residual
    {
      const int xr = gw * RPW3 + min(lane, RPW3 - 1);
      const float xres = a_xi[xr];         // in flight with the staging
      DigIn<NGD> di;
      dig_load<NGD>(di, a_o);
      dig_store<NGD>(di, s_xh, s_xs);
      lds_sync();
      XDig<FP> xd;
      xdig_load<FP>(xd, s_xh, s_xs, lane);
      float acc[RPW3];
#pragma unroll
      for (int j = 0; j < RPW3; ++j) acc[j] = group_dot<FP>(r3[j], xd, lane);
      const float v = gather_rows<RPW3>(acc);
      if (lane < RPW3) act_st(a_xm + xr, v + xres);
    }
    bar.arrive();
    pf4(Ly);
    bar.wait(A.err, A.spin_limit);

    // ---------------- P4: LN2 + lerp, key rows, relu^2
    {
      LnIn<KE> li;
      ln_load<KE>(li, a_xm, Ly.ln2_w, Ly.ln2_b, Ly.cshift_in,
                  Ly.xk);
      {
        StageIn<NGD> si;
        ln_finish<KE>(li, nullptr, wg == 0 ? Ly.cshift_out : nullptr, sh,
                      si.fv);
        stage_digits<NGD>(si, s_xh, s_xs);
      }
      lds_sync();
      XDig<FC> xd;
      xdig_load<FC>(xd, s_xh, s_xs, lane);
      float acc[RPW4];
#pragma unroll
      for (int j = 0; j < RPW4; ++j) acc[j] = group_dot<FC>(r4[j], xd, lane);
      float v = gather_rows<RPW4>(acc);
      v = v > 0.f ? v * v : 0.f;
      // the workgroup's 32 rows are one group of the value product's input:
      // stored once as digits (lanes 0..7 of wave 0)
      if (lane < RPW4) s_row[wave * RPW4 + lane] = v;
      lds_sync();
      if (wave == 0) {
        const float4 f = reinterpret_cast<const float4*>(s_row)[lane & 7];
        uint32_t w0, w1, w2;
        float sf, isc;
        group_digits(f, w0, w1, w2, sf, isc);
        if (lane < 8)
          store_group_digits(a_hk + wg * 32, lane, w0, w1, w2, sf, isc);
      }
    }
    bar.arrive();
    pf5(Ly);
    bar.wait(A.err, A.spin_limit);

    // ---------------- P5: value rows (F wide), += residual
    {
      const int xr = gw * RPW3 + min(lane, RPW3 - 1);
      const float xres = a_xm[xr];
      DigIn<NGF> di;
      dig_load<NGF>(di, a_hk);
      dig_store<NGF>(di, s_xh, s_xs);
      lds_sync();
      float acc[RPW3];
#pragma unroll
      for (int j = 0; j < RPW3; ++j) acc[j] = 0.f;
#pragma unroll
      for (int kg = 0; kg < KGF; ++kg) {
        XDig<FC> xd;
        xdig_load<FC>(xd, s_xh, s_xs, lane + 64 * kg);
#pragma unroll
        for (int j = 0; j < RPW3; ++j)
          acc[j] += group_dot<FC>(r5[j][kg], xd, lane + 64 * kg);
      }
      const float v = gather_rows<RPW3>(acc);
      if (lane < RPW3) act_st(a_xo + xr, v + xres);
    }
  }
  bar.finish();
}

constexpr int kMaxLayers = 32;
constexpr size_t mk_lds_bytes(int KQ, int L) {
  return (size_t)(256 * KQ + 32 * KQ * 24 + 32 * KQ * 3) * 4 +
         (size_t)L * sizeof(MkLayer);
}

template <int FP, int FC>
int launch_mk(const MkArgs& a, hipStream_t st) {
  constexpr int KQ = 8;
  hipLaunchKernelGGL((decode_mk_k<FP, FC, KQ>), dim3(kG), dim3(kT),
                     mk_lds_bytes(KQ, a.L), st, a);
  return hipGetLastError() == hipSuccess ? RWKVQ_OK : RWKVQ_ERR_LAUNCH;
}

// Occupancy of each instantiation on the current device (launch needs
// every workgroup resident at once): checked once per device.
template <int FP, int FC>
bool mk_resident() {
  int dev = 0, cus = 0, occ = 0;
  if (hipGetDevice(&dev) != hipSuccess) return false;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount,
                            dev) != hipSuccess)
    return false;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &occ, decode_mk_k<FP, FC, 8>, kT, mk_lds_bytes(8, kMaxLayers)) !=
      hipSuccess)
    return false;
  return (long)cus * occ >= kG;
}

}  // namespace

// Polls per barrier wait (host setting, read at each launch).
int g_spin_limit = kSpinLimit;

extern "C" {

int rwkvq_decode_mk_spin_limit(int limit) {
  if (limit < 0) return RWKVQ_ERR_ARG;
  g_spin_limit = limit == 0 ? kSpinLimit : limit;
  return RWKVQ_OK;
}

int rwkvq_decode_mk_info(int* layer_bytes, int* bar_words, int* wgs,
                         int* max_cat) {
  if (layer_bytes) *layer_bytes = (int)sizeof(MkLayer);
  if (bar_words) *bar_words = kBarWords;
  if (wgs) *wgs = kG;
  if (max_cat) *max_cat = kMkMaxCat;
  return RWKVQ_OK;
}

int rwkvq_decode_mk(const void* layers, int L, int fmt_proj, int fmt_cmix,
                    int D, int F, int H, float* x, float* act,
                    long act_floats, float* vfirst, unsigned* bar, int* err,
                    void* stream) {
  const long stride = 6L * D + F;
  if (!layers || L <= 0 || L > kMaxLayers || !x || !act || !vfirst ||
      !bar || !err ||
      D != 2048 || F != 4 * D || H != D / kHd || H > kG ||
      act_floats < (long)L * stride ||
      ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(act)) &
       127))
    return RWKVQ_ERR_ARG;
  MkArgs a{};
  a.layers = static_cast<const MkLayer*>(layers);
  a.x = x; a.act = act; a.vfirst = vfirst;
  a.bar = bar; a.err = err; a.L = L; a.H = H; a.act_stride = (int)stride;
  a.spin_limit = g_spin_limit;
  hipStream_t st = (hipStream_t)stream;
  static std::once_flag once;
  static bool ok_c = false, ok_r = false;
  std::call_once(once, [] {
    ok_c = mk_resident<F_SB6_5, F_SB6_4>();
    ok_r = mk_resident<F_SYM8, F_SYM6>();
  });
  if (fmt_proj == F_SB6_5 && fmt_cmix == F_SB6_4)
    return ok_c ? launch_mk<F_SB6_5, F_SB6_4>(a, st) : RWKVQ_ERR_SIZE;
  if (fmt_proj == F_SYM8 && fmt_cmix == F_SYM6)
    return ok_r ? launch_mk<F_SYM8, F_SYM6>(a, st) : RWKVQ_ERR_SIZE;
  return RWKVQ_ERR_ARG;
}

}  // extern "C"
