// Prefill GEMM with the dequantization fused into the operand load, on the
// gfx950 matrix cores (v_mfma_f32_32x32x16_f16).
//
//   y[t, n] = epi( sum_k x[t, seg(n) * K + k] * W[n, k] )
//
// x is fp32 [M, x_ld] (tokens), W one of the packed `.rwkvq` device layouts,
// y fp32 [M, N].  The reference runs this step as a dense fp16 dequant of W
// followed by an fp16 matmul with fp32 output
// (reference: rwkv_quant/backends/metal/quant_linear_gw.py:821-849,
//             rwkv_quant/backends/metal/quant_linear_sym.py:433-484,
//             rwkv_quant/backends/metal/quant_linear_v2.py:322-351);
// here no dense copy of W exists: each lane decodes its codes into the fp16
// weight the reference's dequant would give and feeds them straight to the
// MFMA as the A operand, so W is read from HBM once per token tile.
//
// Roles in the 32x32x16 MFMA: A = W (row i <-> output n), B = x^T (column
// j <-> token t).  Lane l holds A[i = l % 32][k = 8 * (l / 32) + e] and
// B[k = 8 * (l / 32) + e][j = l % 32], e = 0..7; D[i][j] lands in lane
// l = j + 32 * ((i / 4) % 2), register v = 4 * (i / 8) + i % 4.
//
// The k order inside a 32-column quant group is the decoder's pair order
// (x_cols): x is written to LDS in that same order, so both operands walk k
// identically and the sum is the plain dot product.
//
// Tiling: a workgroup of 4 waves covers BN = 4 * 32 * WN output rows and
// BM = 32 * WM tokens.  A wave owns 32 * WN rows (its W fragments stay in
// registers, nothing of W goes through LDS) and all BM tokens.  The K loop
// takes 128 columns per step: lane half h decodes groups 2h and 2h+1 of
// the step; x of the step (BM x 128, fp16, pair order) is staged in LDS,
// double-buffered, one barrier per step.  x of step c + 1 is loaded into
// registers at the start of step c, weights two steps ahead; each group's
// decode is spread over the MFMA rounds before the ones that use it.
//
// Weight values (fp16, exactly as the format's dequant rounded once):
//   sb6   w = fma(q, f16(s), f16(m))   (s = max(f32(f16(qs*d)), 1e-8))
//   sym   w = q * f16(qs * d)
//   rtn8  w = q, the fp32 row scale multiplies the fp32 sum
#include <type_traits>

#include "qfmt.h"
#include "rwkvq_hip.h"

using namespace rwkvq;


typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

namespace {

struct GemmArgs {
  const uint8_t* q;
  const uint32_t* hb;
  const uint8_t* rec;
  const int8_t* qs;
  const uint16_t* d;
  const float* x;        // x[t * x_ld + seg * K + k]
  float* y;              // y[t * N + n]
  long x_ld;
  int M, N, in, out_per, mode;
  int seg_modes;         // mode RWKVQ_EPI_PER_SEG: 4 bits per segment
  int nt, mt;            // tile counts along N and M
  // segment table (rwkvq_gemm_f16_seg): segment j holds rows
  // [seg_end[j-1], seg_end[j]) and reads x at x + j * in; 0 = uniform
  int nseg_tab;
  int seg_end[8];
  // split-K: `split` workgroups share an output tile, each taking an equal
  // run of the K steps; partial tiles go to ws, cnt[tile] counts arrivals
  int split;
  float* ws;
  int* cnt;
  int xh;                // x is fp16 in the format's pair order
  int yord;              // -1: fp32 y; else fp16 y in pair order yord
  int nosplit;           // never split K (caller runs GEMMs concurrently)
  long ldy;              // row stride of y (elements)
  // grouped launch (rwkvq_gemm_f16_grouped): segment j (rows of the segment
  // table) is a matrix of its own
  int grouped;
  const uint8_t* gq[8];
  const float* gx[8];
  long gxld[8];
  float* gy[8];
  int gin[8], gin_rows[8];
};

constexpr int kStepK = 128;                 // columns per K step
constexpr int kRowH = kStepK + 8;           // LDS row stride in halves

// Raw bytes of one row's two consecutive groups (2j, 2j+1) -- one lane's
// share of a K step -- in as few, wide loads as the layout allows: the two
// groups share their superblock record / d, and their high-bit words and
// block scales are adjacent.
struct Raw2 {
  uint4 q[8];     // nibbles: q[0], q[1]; int8 codes: q[0..1], q[2..3];
                  // fp16: q[0..3], q[4..7]
  uint4 hb;       // high-bit words of both groups
  uint4 rec;      // sb6 superblock record
  uint32_t qs;    // sym: the 4 int8 block scales
  uint32_t d;     // sym: fp16 d bits
};

// only the fields the format loads (pinning an unused one would keep its
// registers alive)
template <int FMT>
__device__ __forceinline__ void pin_raw2(Raw2& r) {
  constexpr int NQ = FMT == F_F16 ? 8
                   : (FMT == F_SYM8 || FMT == F_RTN8) ? 4 : 2;
#pragma unroll
  for (int i = 0; i < NQ; ++i) pin(r.q[i]);
  if (FMT == F_SB6_5) { pin(r.hb.x); pin(r.hb.y); }
  if (FMT == F_SB6_6 || FMT == F_SYM6) pin(r.hb);
  if (FMT <= F_SB6_6) pin(r.rec);
  if (FMT == F_SYM6 || FMT == F_SYM8) { pin(r.qs); pin(r.d); }
}

template <int FMT>
__device__ __forceinline__ void load_raw2(const GemmArgs& a, int row, int ng,
                                          int nsb, int g, Raw2& r) {
  if (FMT == F_F16) {
    const uint8_t* p = a.q + ((size_t)row * a.in + g * 32) * 2;
#pragma unroll
    for (int i = 0; i < 8; ++i) r.q[i] = ld16(p + 16 * i);
    return;
  }
  if (FMT == F_SYM8 || FMT == F_RTN8) {
    const uint8_t* p = a.q + (size_t)row * a.in + g * 32;
#pragma unroll
    for (int i = 0; i < 4; ++i) r.q[i] = ld16(p + 16 * i);
  } else {
    const uint8_t* p = a.q + ((size_t)row * ng + g) * 16;
    r.q[0] = ld16(p);
    r.q[1] = ld16(p + 16);
  }
  if (FMT <= F_SB6_6)
    r.rec = ld16(a.rec + ((size_t)row * nsb + (g >> 3)) * 16);
  if (FMT == F_SB6_5) {
    const uint2 v = *reinterpret_cast<const uint2*>(a.hb + (size_t)row * ng + g);
    r.hb.x = v.x; r.hb.y = v.y;
  }
  if (FMT == F_SB6_6 || FMT == F_SYM6)
    r.hb = ld16(a.hb + ((size_t)row * ng + g) * 2);
  if (FMT == F_SYM6 || FMT == F_SYM8) {
    r.qs = *reinterpret_cast<const uint32_t*>(a.qs + (size_t)row * (a.in >> 4) + 2 * g);
    r.d = a.d[(size_t)row * nsb + (g >> 3)];
  }
}

// Group gi (0, 1) of a Raw2 in the single-group form the decoder takes.
template <int FMT>
__device__ __forceinline__ Raw group_of(const Raw2& w, int gi) {
  Raw r;
  if (FMT == F_SYM8 || FMT == F_RTN8) {
    r.a = w.q[2 * gi];
    r.b = w.q[2 * gi + 1];
  } else {
    r.a = w.q[gi];
  }
  if (FMT <= F_SB6_6) r.b = w.rec;
  if (FMT == F_SB6_5) r.h.x = gi ? w.hb.y : w.hb.x;
  if (FMT == F_SB6_6 || FMT == F_SYM6)
    r.h = gi ? make_uint2(w.hb.z, w.hb.w) : make_uint2(w.hb.x, w.hb.y);
  r.s = gi ? (w.qs >> 16) : (w.qs & 0xFFFFu);
  r.dd = w.d;
  return r;
}

// fp16 weights of group gi of a Raw2 in the decoder's pair order, a quad
// (4 pairs) at a time: the group's scales, then pairs 4 qd .. 4 qd + 3
// (dense fp16 rows: the stored values, natural order).
template <int FMT>
__device__ __forceinline__ DqScale scale_of(const Raw2& r2, int gi, int kb) {
  if constexpr (FMT == F_F16) return DqScale{};
  else return dq_scale<FMT>(group_of<FMT>(r2, gi), kb);
}
template <int FMT>
__device__ __forceinline__ void quad_of(const Raw2& r2, int gi,
                                        const DqScale& sc, int qd,
                                        uint32_t w[16]) {
  if constexpr (FMT == F_F16) {
    const uint4 v = r2.q[4 * gi + qd];
    w[4 * qd] = v.x; w[4 * qd + 1] = v.y; w[4 * qd + 2] = v.z; w[4 * qd + 3] = v.w;
  } else {
    dq_quad<FMT>(group_of<FMT>(r2, gi), sc, qd, w);
  }
}

// The workgroup's x staging buffers: KG groups x 2 steps x BM rows.
template <int WM, int KG>
using XStage = _Float16[KG][2][32 * WM * kRowH];

// One workgroup's tile (bid: its index in the launch).  KG groups of NW
// waves share the tile and split its K steps (group g takes steps g,
// g + KG, ...): KG waves per SIMD hide each other's latency without a
// smaller tile; the groups' sums meet in LDS at the end.
template <int FMT, int WN, int WM, int KG, bool XH, int NW>
__device__ __forceinline__ void gemm_tile(const GemmArgs& a0, const int bid,
                                          XStage<WM, KG>& sx) {
  GemmArgs a = a0;     // (grouped launches substitute the segment's fields)
  constexpr int BM = 32 * WM;
  constexpr int BN = 32 * NW * WN;           // NW waves along N
  constexpr int NT = 64 * NW;                // threads of a K group
  constexpr int XI = BM * 16 / NT;           // staging items per thread

  const int lane = threadIdx.x & 63;
  const int wave_all = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kg = wave_all / NW, wave = wave_all % NW;
  const int tid = threadIdx.x % NT;          // thread index in the group
  const int r = lane & 31, h = lane >> 5;
  // Tile order: workgroup b runs on XCD b % 8 (round-robin dispatch).  The
  // M tiles of one N tile go to the same XCD back to back, so that XCD's L2
  // serves the W tile to all of them after one HBM read; N tiles are dealt
  // across the XCDs.
  // With split-K, index j = nt * split + sp stands in for nt: the M tiles
  // of one (N tile, K run) share an XCD, the runs of a tile spread out.
  int j, mt;
  if (((a.nt * a.split) & 7) == 0) {
    const int slot = bid >> 3;
    mt = slot % a.mt;
    j = (slot / a.mt) * 8 + (bid & 7);
  } else {
    mt = bid % a.mt;
    j = bid / a.mt;
  }
  const int nt = j / a.split, sp = j % a.split;
  int n0 = nt * BN;
  const int m0 = mt * BM;
  int seg = n0 / a.out_per;
  if (a.nseg_tab > 0) {                    // constant-index reads only
    seg = 0;
#pragma unroll
    for (int j = 0; j < 7; ++j)
      seg += (j + 1 < a.nseg_tab && n0 >= a.seg_end[j]) ? 1 : 0;
  }
  int xseg = seg;                          // x segment offset (seg * in)
  if (a.grouped) {
    // segment j is its own matrix: weights, K, x, y (row stride = its rows);
    // chosen by selects over constant indices (kernel arguments stay in
    // SGPRs)
    const uint8_t* q = a0.gq[0];
    const float* x = a0.gx[0];
    float* y = a0.gy[0];
    long xld = a0.gxld[0];
    int in = a0.gin[0], ldy = a0.gin_rows[0], off = 0;
#pragma unroll
    for (int j = 1; j < 8; ++j) {
      const bool m = j == seg;
      q = m ? a0.gq[j] : q;
      x = m ? a0.gx[j] : x;
      y = m ? a0.gy[j] : y;
      xld = m ? a0.gxld[j] : xld;
      in = m ? a0.gin[j] : in;
      ldy = m ? a0.gin_rows[j] : ldy;
      off = m ? a0.seg_end[j - 1] : off;
    }
    a.q = q; a.x = x; a.y = y; a.x_ld = xld; a.in = in; a.ldy = ldy;
    n0 -= off;
    xseg = 0;
  }
  const int ng = a.in >> 5, nsb = a.in >> 8;
  const int nrun = a.in / kStepK / a.split;   // K steps of this workgroup
  const int c0 = sp * nrun;
  const float* xb = a.x + (size_t)xseg * a.in;
  // fp16 x (XH): already in pair order, x_ld in halves
  const uint16_t* xh = reinterpret_cast<const uint16_t*>(a.x) + (size_t)xseg * a.in;

  // ---- x staging: item = (token, group of the step, sub-step)
  float4 xa[XH ? 1 : XI], xbv[XH ? 1 : XI];
  uint4 xq[XH ? XI : 1];
  auto load_x = [&](int c) {
#pragma unroll
    for (int p = 0; p < XI; ++p) {
      const int it = tid + NT * p;
      const int t = min(m0 + (it >> 4), a.M - 1);
      if constexpr (XH) {
        xq[p] = ld16(xh + (size_t)t * a.x_ld + c * kStepK + (it & 15) * 8);
      } else {
        const int gq = (it >> 2) & 3, s = it & 3;
        int ca, cb;
        step_cols<FMT>(s, ca, cb);
        const float* src = xb + (size_t)t * a.x_ld + c * kStepK + gq * 32;
        xa[p] = *reinterpret_cast<const float4*>(src + ca);
        xbv[p] = *reinterpret_cast<const float4*>(src + cb);
      }
    }
  };
  auto store_x = [&](int buf) {
#pragma unroll
    for (int p = 0; p < XI; ++p) {
      const int it = tid + NT * p;
      const int tl = it >> 4, gq = (it >> 2) & 3, s = it & 3;
      *reinterpret_cast<uint4*>(&sx[kg][buf][tl * kRowH + gq * 32 + s * 8]) =
          XH ? xq[p] : x_pairs<FMT>(xa[p], xbv[p]);
    }
  };

  // ---- weights: WN rows x 2 groups per lane per step, in registers
  int rows[WN];
#pragma unroll
  for (int ni = 0; ni < WN; ++ni)
    rows[ni] = n0 + wave * 32 * WN + ni * 32 + r;
  auto load_w = [&](int c, Raw2 (&dst)[WN]) {
#pragma unroll
    for (int ni = 0; ni < WN; ++ni)
      load_raw2<FMT>(a, rows[ni], ng, nsb, c * 4 + 2 * h, dst[ni]);
  };

  f32x16_t acc[WM][WN];
#pragma unroll
  for (int mi = 0; mi < WM; ++mi)
#pragma unroll
    for (int ni = 0; ni < WN; ++ni)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[mi][ni][v] = 0.f;

  // Weights are fetched two steps ahead, into ping-pong register sets: the
  // set of step i is refilled with step i + 2 as soon as its second group
  // is decoded, so an HBM fetch has about a step and a half to land.  x is
  // fetched one step ahead (it comes from L2).
  const int clast = c0 + nrun - KG + kg;       // the group's last step
  Raw2 wset[2][WN];
  load_w(c0 + kg, wset[0]);
  load_w(min(c0 + KG + kg, clast), wset[1]);
  load_x(c0 + kg);
  store_x(0);
  __syncthreads();

  const int nsg = nrun / KG;                   // steps of each group
  // Decode pipelined into the MFMA rounds: round k (k = 0..7) of a step
  // multiplies with quad k % 4 of group k / 4 and decodes one quad of the
  // next group due -- group 1 of the step in rounds 0-3, group 0 of the
  // following step in rounds 4-7 -- so every MFMA has decode VALU work
  // beside it instead of a block of decode in front of the rounds.
  uint32_t w[2][WN][16];
  {
    const int c = c0 + kg;
#pragma unroll
    for (int ni = 0; ni < WN; ++ni) {
      const DqScale sc = scale_of<FMT>(wset[0][ni], 0, (c * 4 + 2 * h) & 7);
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) quad_of<FMT>(wset[0][ni], 0, sc, qd, w[0][ni]);
    }
  }
  auto step = [&](int i, auto set_tag) __attribute__((always_inline)) {
    constexpr int S = decltype(set_tag)::value;   // register set of step i
    const int c = c0 + i * KG + kg;
    const int cn = min(c + KG, clast), cnn = min(c + 2 * KG, clast);
    load_x(cn);
    __builtin_amdgcn_sched_barrier(0);
    const _Float16* xs = sx[kg][i & 1];
    auto read_bx = [&](int k, half8_t (&b)[WM]) {
      const int gi = k >> 2, ss = k & 3;
#pragma unroll
      for (int mi = 0; mi < WM; ++mi)
        b[mi] = *reinterpret_cast<const half8_t*>(
            xs + (mi * 32 + r) * kRowH + (2 * h + gi) * 32 + ss * 8);
    };
    half8_t bx[2][WM];
    read_bx(0, bx[0]);
    DqScale sc[WN];
#pragma unroll
    for (int ni = 0; ni < WN; ++ni)
      sc[ni] = scale_of<FMT>(wset[S][ni], 1, (c * 4 + 2 * h + 1) & 7);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int gi = k >> 2, ss = k & 3;
      if (k == 4) {
        // group 1 of the step is decoded: refill its set with step c + 2 KG
        load_w(cnn, wset[S]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ni = 0; ni < WN; ++ni)
          sc[ni] = scale_of<FMT>(wset[1 - S][ni], 0, (cn * 4 + 2 * h) & 7);
      }
      if (k + 1 < 8) read_bx(k + 1, bx[(k + 1) & 1]);
#pragma unroll
      for (int ni = 0; ni < WN; ++ni) {
        const uint4 wa = make_uint4(w[gi][ni][4 * ss], w[gi][ni][4 * ss + 1],
                                    w[gi][ni][4 * ss + 2],
                                    w[gi][ni][4 * ss + 3]);
        const half8_t av = __builtin_bit_cast(half8_t, wa);
#pragma unroll
        for (int mi = 0; mi < WM; ++mi)
          acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
              av, bx[k & 1][mi], acc[mi][ni], 0, 0, 0);
      }
#pragma unroll
      for (int ni = 0; ni < WN; ++ni) {
        if (k < 4) quad_of<FMT>(wset[S][ni], 1, sc[ni], k, w[1][ni]);
        else quad_of<FMT>(wset[1 - S][ni], 0, sc[ni], k - 4, w[0][ni]);
      }
      // one MFMA, one x read, a share of the decode, ...
#pragma unroll
      for (int j = 0; j < WM * WN; ++j) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (k + 1 < 8 && j < WM) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 7, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int p = 0; p < XI; ++p) {
      if constexpr (XH) pin(xq[p]);
      else { pin(xa[p]); pin(xbv[p]); }
    }
    store_x((i + 1) & 1);
    __syncthreads();
  };
  // two steps per iteration and an odd last step after the loop (a path
  // from the first step back to the loop head would carry that step's
  // weight loads in flight and make every iteration wait for all loads at
  // its head)
  int i = 0;
  for (; i + 1 < nsg; i += 2) {
    step(i, std::integral_constant<int, 0>());
    step(i + 1, std::integral_constant<int, 1>());
  }
  if (i < nsg) step(i, std::integral_constant<int, 0>());

  if constexpr (KG > 1) {
    // group 1 hands its sums to group 0 through the x buffers (free: the
    // loop ended on a barrier); 4 waves x 16 WM WN floats x 64 lanes
    // fits them for every tile of this kernel
    constexpr int NA = WM * WN * 16;
    static_assert(NW * NA * 64 * 4 <= (int)sizeof(sx), "reduction buffer");
    float* red = reinterpret_cast<float*>(&sx[0][0][0]);
    if (kg == 1) {
#pragma unroll
      for (int mi = 0; mi < WM; ++mi)
#pragma unroll
        for (int ni = 0; ni < WN; ++ni)
#pragma unroll
          for (int v = 0; v < 16; ++v)
            red[(wave * NA + (mi * WN + ni) * 16 + v) * 64 + lane] =
                acc[mi][ni][v];
    }
    __syncthreads();
    if (kg == 0) {
#pragma unroll
      for (int mi = 0; mi < WM; ++mi)
#pragma unroll
        for (int ni = 0; ni < WN; ++ni)
#pragma unroll
          for (int v = 0; v < 16; ++v)
            acc[mi][ni][v] += red[(wave * NA + (mi * WN + ni) * 16 + v) * 64 + lane];
    }
  }

  if (a.split > 1) {
    // Every run stores its partial tile (lane-major, coalesced) and counts
    // itself in; the last to arrive adds the partials in run order 0, 1,
    // ... (the same sum whichever run finishes last), applies the
    // epilogue and re-arms the counter for the next launch.  Partials and
    // counter move by agent-scope relaxed atomics, which are coherent
    // across the XCDs' L2s by themselves; a device-scope fence instead
    // would write back and invalidate the whole L2 in every workgroup.
    constexpr int NA = WM * WN * 16;
    constexpr int TE = NW * NA * 64;           // floats per partial tile
    const int tile = nt * a.mt + mt;
    float* part = a.ws + (size_t)tile * a.split * TE;
    if (kg == 0) {
#pragma unroll
      for (int mi = 0; mi < WM; ++mi)
#pragma unroll
        for (int ni = 0; ni < WN; ++ni)
#pragma unroll
          for (int v = 0; v < 16; ++v)
            __hip_atomic_store(
                part + (size_t)sp * TE +
                    (wave * NA + (mi * WN + ni) * 16 + v) * 64 + lane,
                acc[mi][ni][v], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __shared__ int s_last;
    // this wave's partial stores are complete before the barrier, so all
    // of them are before the count goes up
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0)
      s_last = __hip_atomic_fetch_add(a.cnt + tile, 1, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT) ==
               a.split - 1;
    __syncthreads();
    if (!s_last) return;
    if (kg == 0) {
      float sum[WM][WN][16];
#pragma unroll
      for (int mi = 0; mi < WM; ++mi)
#pragma unroll
        for (int ni = 0; ni < WN; ++ni)
#pragma unroll
          for (int v = 0; v < 16; ++v) sum[mi][ni][v] = 0.f;
      for (int q = 0; q < a.split; ++q) {
        if (q == sp) {                         // (uniform branch)
#pragma unroll
          for (int mi = 0; mi < WM; ++mi)
#pragma unroll
            for (int ni = 0; ni < WN; ++ni)
#pragma unroll
              for (int v = 0; v < 16; ++v) sum[mi][ni][v] += acc[mi][ni][v];
          continue;
        }
        // one run's partial tile at a time: all its loads in flight at once
        float p[WM][WN][16];
        const float* pq = part + (size_t)q * TE + wave * NA * 64 + lane;
#pragma unroll
        for (int mi = 0; mi < WM; ++mi)
#pragma unroll
          for (int ni = 0; ni < WN; ++ni)
#pragma unroll
            for (int v = 0; v < 16; ++v)
              p[mi][ni][v] = __hip_atomic_load(
                  pq + ((mi * WN + ni) * 16 + v) * 64, __ATOMIC_RELAXED,
                  __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int mi = 0; mi < WM; ++mi)
#pragma unroll
          for (int ni = 0; ni < WN; ++ni)
#pragma unroll
            for (int v = 0; v < 16; ++v) sum[mi][ni][v] += p[mi][ni][v];
      }
#pragma unroll
      for (int mi = 0; mi < WM; ++mi)
#pragma unroll
        for (int ni = 0; ni < WN; ++ni)
#pragma unroll
          for (int v = 0; v < 16; ++v) acc[mi][ni][v] = sum[mi][ni][v];
      if (threadIdx.x == 0)
        __hip_atomic_store(a.cnt + tile, 0, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if (kg != 0) return;

  // ---- epilogue: lane holds tokens m0 + 32 mi + r, rows 4 at a time
  // (rows 8 q + 4 h + e of each 32-row block in acc[.][.][4 q + e])
  const int mode = a.mode == RWKVQ_EPI_PER_SEG
                       ? (a.seg_modes >> (4 * seg)) & 15 : a.mode;
#pragma unroll
  for (int mi = 0; mi < WM; ++mi) {
    const int t = m0 + mi * 32 + r;
    if (t >= a.M) continue;
    float* yrow = a.y + (size_t)t * a.ldy;
#pragma unroll
    for (int ni = 0; ni < WN; ++ni) {
      const int nb = n0 + wave * 32 * WN + ni * 32;   // 32-row block
      float4 v4[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = nb + 8 * q + 4 * h;
        float4 v = make_float4(acc[mi][ni][4 * q], acc[mi][ni][4 * q + 1],
                               acc[mi][ni][4 * q + 2], acc[mi][ni][4 * q + 3]);
        if (FMT == F_RTN8) {
          const uint2 sc = *reinterpret_cast<const uint2*>(a.d + n);
          v.x *= f16_bits_to_f32(sc.x & 0xFFFFu);
          v.y *= f16_bits_to_f32(sc.x >> 16);
          v.z *= f16_bits_to_f32(sc.y & 0xFFFFu);
          v.w *= f16_bits_to_f32(sc.y >> 16);
        }
        switch (mode) {
          case RWKVQ_EPI_ADD: {
            const float4 o = *reinterpret_cast<const float4*>(yrow + n);
            v.x += o.x; v.y += o.y; v.z += o.z; v.w += o.w;
            break;
          }
          case RWKVQ_EPI_RELU2:
            v.x = v.x > 0.f ? v.x * v.x : 0.f; v.y = v.y > 0.f ? v.y * v.y : 0.f;
            v.z = v.z > 0.f ? v.z * v.z : 0.f; v.w = v.w > 0.f ? v.w * v.w : 0.f;
            break;
          case RWKVQ_EPI_TANH:
            v.x = tanhf(v.x); v.y = tanhf(v.y); v.z = tanhf(v.z); v.w = tanhf(v.w);
            break;
          case RWKVQ_EPI_SIGMOID:
            v.x = 1.f / (1.f + __expf(-v.x)); v.y = 1.f / (1.f + __expf(-v.y));
            v.z = 1.f / (1.f + __expf(-v.z)); v.w = 1.f / (1.f + __expf(-v.w));
            break;
          default: break;
        }
        v4[q] = v;
      }
      if (a.yord < 0) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<float4*>(yrow + nb + 8 * q + 4 * h) = v4[q];
        continue;
      }
      // fp16 output in the pair order of the consuming GEMM: the block's 32
      // rows are that GEMM's 32-column group, half 2i / 2i+1 = columns
      // (c0(i), c1(i)); a lane's rows pair up with rows it holds itself
      uint16_t* yh = reinterpret_cast<uint16_t*>(a.y) + (size_t)t * a.ldy + nb;
      // rounded to fp32 first, as the fp32 output (no fused mixed-precision
      // multiply-add + conversion)
#pragma unroll
      for (int q = 0; q < 4; ++q) pin(v4[q]);
      auto h2 = [](float lo, float hi) { return pack_h2(lo, hi); };
      if (a.yord == RWKVQ_ORDER_PAIRS) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<uint2*>(yh + 8 * q + 4 * h) =
              make_uint2(h2(v4[q].x, v4[q].y), h2(v4[q].z, v4[q].w));
      } else {
        // sb6: (c, c + 16) = rows of q and q + 2; sym6: (c, c + 8) = rows
        // of q and q + 1, c in [0, 8) or [16, 24)
        const bool sb = a.yord == RWKVQ_ORDER_SB6;
        const float4 l0 = v4[0], p0 = sb ? v4[2] : v4[1];
        const float4 l1 = sb ? v4[1] : v4[2], p1 = v4[3];
        *reinterpret_cast<uint4*>(yh + 8 * h) =
            make_uint4(h2(l0.x, p0.x), h2(l0.y, p0.y), h2(l0.z, p0.z),
                       h2(l0.w, p0.w));
        *reinterpret_cast<uint4*>(yh + 16 + 8 * h) =
            make_uint4(h2(l1.x, p1.x), h2(l1.y, p1.y), h2(l1.z, p1.z),
                       h2(l1.w, p1.w));
      }
    }
  }
}

template <int FMT, int WN, int WM, int KG, bool XH, int NW>
__global__ void __launch_bounds__(64 * NW * KG)
gemm_kernel(GemmArgs a) {
  __shared__ __attribute__((aligned(16))) XStage<WM, KG> sx;
  gemm_tile<FMT, WN, WM, KG, XH, NW>(a, blockIdx.x, sx);
}

// Two GEMMs of the same tile shape in one launch: workgroups [0, grid_a)
// run GEMM a (format FA), the rest GEMM b (format FB) -- the prefill r/k/v
// projection and the LoRA down products, which read the same lerp outputs
// and have the same K, so the few down tiles run on the CUs the r/k/v
// tiles leave free instead of after them.
template <int FA, int FB, int WN, int WM, int KG, bool XH, int NW>
__global__ void __launch_bounds__(64 * NW * KG)
gemm_dual_kernel(GemmArgs a, GemmArgs b, int grid_a) {
  __shared__ __attribute__((aligned(16))) XStage<WM, KG> sx;
  if ((int)blockIdx.x < grid_a)
    gemm_tile<FA, WN, WM, KG, XH, NW>(a, blockIdx.x, sx);
  else
    gemm_tile<FB, WN, WM, KG, XH, NW>(b, blockIdx.x - grid_a, sx);
}

#ifndef RWKVQ_GEMM_KG
#define RWKVQ_GEMM_KG 2
#endif
#ifndef RWKVQ_GEMM_SPLIT
#define RWKVQ_GEMM_SPLIT 1
#endif
// split-K: runs of >= kMinRun steps, until the launch has >= RWKVQ_SPLIT_WGS
// workgroups (the 128 x 128 tile is used from that count on)
#ifndef RWKVQ_SPLIT_WGS
#define RWKVQ_SPLIT_WGS 192
#endif
constexpr int kMinRun = 8;
#ifndef RWKVQ_GEMM_LONG_RUN
#define RWKVQ_GEMM_LONG_RUN 32
#endif
constexpr int kLongRun = RWKVQ_GEMM_LONG_RUN;

// Split-K workspace registered by the caller (rwkvq_gemm_workspace), one
// per device.
struct SplitWs {
  float* ws;
  long bytes;
  int* cnt;
  int ncnt;
};
SplitWs g_split_ws[64];

const SplitWs* current_ws() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  return g_split_ws[dev].ws ? &g_split_ws[dev] : nullptr;
}

// The launch shape of one GEMM: wave tile 32 * wn rows x 32 * wm tokens,
// nw waves along N (4, or 8 for the 256 x 128 tile), K split across
// `split` workgroups per output tile, `one_group` = no second K group
// inside the workgroup (two independent 4-wave workgroups per CU instead).
struct GemmPlan {
  int wn, wm, nw, split;
  bool one_group;
};

// K groups inside a workgroup: two (8 waves) wherever the tile's registers
// allow two waves per SIMD (all tiles but 256 x 128) and the step count of
// a split run is even.
int plan_kgroups(const GemmPlan& p, int in) {
  const bool two = RWKVQ_GEMM_KG == 2 && p.wn * p.wm <= 4 && p.nw == 4;
  return (two && !p.one_group && (in / kStepK / p.split) % 2 == 0) ? 2 : 1;
}

template <int FMT, int WN, int WM, int NW = 4>
int launch_tile(const GemmArgs& a, hipStream_t s, const GemmPlan& p,
                const SplitWs* ws) {
  GemmArgs b = a;
  b.nt = a.N / (32 * NW * WN);
  b.mt = (a.M + 32 * WM - 1) / (32 * WM);
  b.split = p.split;
  if (p.split > 1) { b.ws = ws->ws; b.cnt = ws->cnt; }
  const int grid = b.nt * b.mt * p.split;
  constexpr bool two = RWKVQ_GEMM_KG == 2 && WN * WM <= 4 && NW == 4;
  constexpr int KG2 = two ? 2 : 1;
  if (two && plan_kgroups(p, a.in) == 2) {
    if (a.xh)
      hipLaunchKernelGGL((gemm_kernel<FMT, WN, WM, KG2, true, NW>),
                         dim3(grid), dim3(64 * NW * KG2), 0, s, b);
    else
      hipLaunchKernelGGL((gemm_kernel<FMT, WN, WM, KG2, false, NW>),
                         dim3(grid), dim3(64 * NW * KG2), 0, s, b);
  } else {
    if (a.xh)
      hipLaunchKernelGGL((gemm_kernel<FMT, WN, WM, 1, true, NW>), dim3(grid),
                         dim3(64 * NW), 0, s, b);
    else
      hipLaunchKernelGGL((gemm_kernel<FMT, WN, WM, 1, false, NW>),
                         dim3(grid), dim3(64 * NW), 0, s, b);
  }
  return hipGetLastError() == hipSuccess ? RWKVQ_OK : RWKVQ_ERR_LAUNCH;
}

// Tile choice: 256 x 128 (8 waves of 32 rows x 128 tokens) where that
// alone gives >= 256 workgroups; else 128 x 128 (4 waves of 32 rows x 128
// tokens, each decoded weight feeds 4 MFMAs), split along K where that
// fills the chip; else the largest smaller tile that still gives >= 256
// workgroups.
// N tiles of 256 rows need out_per % 256 == 0; segment tables take 128-row
// tiles (their segments are multiples of 128 rows).
GemmPlan plan_gemm(const GemmArgs& a, const SplitWs* ws) {
  auto wgs = [&](int bn, int bm) {
    return (long)(a.N / bn) * ((a.M + bm - 1) / bm);
  };
  const int nsteps = a.in / kStepK;
  const bool wide = a.out_per % 256 == 0 && a.nseg_tab == 0;
  if (wide && wgs(256, 128) >= 256) return {1, 4, 8, 1, true};
  if (RWKVQ_GEMM_SPLIT && a.M > 64) {
    // Two 4-wave workgroups per CU (each with its own barrier, so the two
    // waves of a SIMD drift out of phase and overlap decode with MFMA)
    // where the launch has >= 512 of them, splitting K only into runs of
    // >= kLongRun steps (the partial tiles cost more than they save on
    // shorter runs).
    const long t = wgs(128, 128);
    int split = 1;
    while (t * split < 512 && split < 8 && nsteps % (2 * split) == 0 &&
           nsteps / (2 * split) >= kLongRun && ws && t <= ws->ncnt &&
           t * 2 * split * 128 * 128 * (long)sizeof(float) <= ws->bytes)
      split *= 2;
    if (t * split >= 512) return {1, 4, 4, split, true};
  }
  if (RWKVQ_GEMM_SPLIT && a.M > 64 && nsteps % 2 == 0) {
    const long t = wgs(128, 128);
    int split = 1;
    while (t * split < RWKVQ_SPLIT_WGS && split < 8 &&
           nsteps % (2 * kMinRun * split) == 0 && ws && t <= ws->ncnt &&
           t * 2 * split * 128 * 128 * (long)sizeof(float) <= ws->bytes)
      split *= 2;
    if (t * split >= RWKVQ_SPLIT_WGS) return {1, 4, 4, split, false};
  }
  if (wide && wgs(256, 64) >= 256) return {2, 2, 4, 1, false};
  if (wgs(128, 64) >= 256) return {1, 2, 4, 1, false};
  if (RWKVQ_GEMM_SPLIT && wgs(128, 32) < 256 && a.M > 32 && nsteps >= 4 &&
      ws) {
    // few output tiles even at 128 x 32 (e.g. the LoRA down products):
    // 128 x 64 tiles split into runs of >= 2 steps
    const long t = wgs(128, 64);
    int split = 1;
    while (t * split < 256 && split < 8 && nsteps % (4 * split) == 0 &&
           t <= ws->ncnt &&
           t * 2 * split * 128 * 64 * (long)sizeof(float) <= ws->bytes)
      split *= 2;
    if (split > 1 && t * split >= 192) return {1, 2, 4, split, false};
  }
  return {1, 1, 4, 1, false};
}

const SplitWs* gemm_ws(const GemmArgs& a) {
  return a.nosplit ? nullptr : current_ws();
}

template <int FMT>
int launch_gemm(const GemmArgs& a, hipStream_t s) {
  const SplitWs* ws = gemm_ws(a);
  const GemmPlan p = plan_gemm(a, ws);
  if (p.nw == 8) return launch_tile<FMT, 1, 4, 8>(a, s, p, ws);
  if (p.wn == 1 && p.wm == 4) return launch_tile<FMT, 1, 4>(a, s, p, ws);
  if (p.wn == 2 && p.wm == 2) return launch_tile<FMT, 2, 2>(a, s, p, ws);
  if (p.wn == 1 && p.wm == 2) return launch_tile<FMT, 1, 2>(a, s, p, ws);
  return launch_tile<FMT, 1, 1>(a, s, p, ws);
}

int check_gemm(int rows, int in, int out_per, int M, long x_ld, int mode,
               int k_mult = 256) {
  if (mode & ~(15 | RWKVQ_X_F16 | RWKVQ_Y_F16 | (3 << RWKVQ_Y_ORDER_SHIFT) |
               RWKVQ_NO_SPLIT))
    return RWKVQ_ERR_ARG;
  if (mode & RWKVQ_Y_F16) {                   // fp16 y: no residual add
    if (((mode >> RWKVQ_Y_ORDER_SHIFT) & 3) > RWKVQ_ORDER_SYM6 ||
        (mode & 15) == RWKVQ_EPI_ADD)
      return RWKVQ_ERR_ARG;
  }
  mode &= 15;
  if (rows <= 0 || in <= 0 || M <= 0 || out_per <= 0) return RWKVQ_ERR_ARG;
  if (in % k_mult) return RWKVQ_ERR_ARG;
  if (rows % out_per || out_per % 128) return RWKVQ_ERR_ARG;
  if (x_ld < (long)(rows / out_per) * in) return RWKVQ_ERR_ARG;
  if (mode < 0 || mode > RWKVQ_EPI_SIGMOID) return RWKVQ_ERR_ARG;
  return RWKVQ_OK;
}

// x rows are read 16 bytes at a time
int check_x(const void* x, long x_ld, int xh) {
  if (reinterpret_cast<uintptr_t>(x) % 16 || x_ld % (xh ? 8 : 4))
    return RWKVQ_ERR_ARG;
  return RWKVQ_OK;
}

GemmArgs make_args(int rows, int in, int out_per, const float* x, long x_ld,
                   float* y, int M, int mode) {
  GemmArgs a{};
  a.split = 1;
  a.xh = (mode & RWKVQ_X_F16) != 0;
  a.yord = (mode & RWKVQ_Y_F16) ? (mode >> RWKVQ_Y_ORDER_SHIFT) & 3 : -1;
  a.nosplit = (mode & RWKVQ_NO_SPLIT) != 0;
  mode &= 15;
  a.x = x; a.y = y; a.M = M; a.N = rows; a.in = in; a.out_per = out_per;
  a.ldy = rows;
  a.mode = mode;
  a.x_ld = x_ld > 0 ? x_ld : (long)(rows / out_per) * in;
  return a;
}

// fp32 x -> fp16 x in the pair order of a weight format: thread = one
// 8-half chunk (token t, 32-column group, sub-step s) of the GEMM's LDS rows.
template <int FMT>
__global__ void __launch_bounds__(256)
x16_kernel(const float* __restrict__ x, long x_ld, uint16_t* __restrict__ out,
           long out_ld, int M, int cols) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  const int per = cols >> 3;                  // chunks per token
  if (i >= (long)M * per) return;
  const int t = (int)(i / per), c = (int)(i % per);
  const int g = c >> 2, s = c & 3;
  int ca, cb;
  step_cols<FMT>(s, ca, cb);
  const float* src = x + (size_t)t * x_ld + g * 32;
  const uint4 v = x_pairs<FMT>(*reinterpret_cast<const float4*>(src + ca),
                               *reinterpret_cast<const float4*>(src + cb));
  *reinterpret_cast<uint4*>(out + (size_t)t * out_ld + c * 8) = v;
}

}  // namespace

namespace rwkvq {
bool split_workspace(float** ws, long* bytes, int** cnt, int* ncnt) {
  const SplitWs* w = current_ws();
  if (!w) return false;
  *ws = w->ws;
  *bytes = w->bytes;
  *cnt = w->cnt;
  *ncnt = w->ncnt;
  return true;
}
}  // namespace rwkvq

extern "C" {

int rwkvq_x16(const float* x, long x_ld, int cols, int M, int order,
              uint16_t* out, long out_ld, void* stream) {
  if (!x || !out || M <= 0 || cols <= 0 || cols % 32 || x_ld < cols ||
      out_ld < cols || check_x(x, x_ld, 0) || check_x(out, out_ld, 1) ||
      order < 0 || order > 2)
    return RWKVQ_ERR_ARG;
  const long n = (long)M * (cols / 8);
  const dim3 grid((unsigned)((n + 255) / 256));
  hipStream_t s = (hipStream_t)stream;
  if (order == RWKVQ_ORDER_PAIRS)
    hipLaunchKernelGGL(x16_kernel<F_SYM8>, grid, dim3(256), 0, s, x, x_ld,
                       out, out_ld, M, cols);
  else if (order == RWKVQ_ORDER_SB6)
    hipLaunchKernelGGL(x16_kernel<F_SB6_4>, grid, dim3(256), 0, s, x, x_ld,
                       out, out_ld, M, cols);
  else
    hipLaunchKernelGGL(x16_kernel<F_SYM6>, grid, dim3(256), 0, s, x, x_ld,
                       out, out_ld, M, cols);
  return hipGetLastError() == hipSuccess ? RWKVQ_OK : RWKVQ_ERR_LAUNCH;
}

int rwkvq_gemm_workspace(void* ws, long ws_bytes, int* counters,
                         int n_counters) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
    return RWKVQ_ERR_ARG;
  if (!ws || !counters) {
    g_split_ws[dev] = SplitWs{nullptr, 0, nullptr, 0};
    return RWKVQ_OK;
  }
  if (ws_bytes <= 0 || n_counters <= 0 ||
      reinterpret_cast<uintptr_t>(ws) % 16)
    return RWKVQ_ERR_ARG;
  g_split_ws[dev] = SplitWs{static_cast<float*>(ws), ws_bytes, counters,
                            n_counters};
  return RWKVQ_OK;
}

int rwkvq_gemm_sb6(const uint8_t* nib, const uint32_t* hb, const uint8_t* rec,
                   int bits, int rows, int in, int out_per, const float* x,
                   long x_ld, float* y, int M, int mode, void* stream) {
  GemmArgs a = make_args(rows, in, out_per, x, x_ld, y, M, mode);
  int st = check_gemm(rows, in, out_per, M, a.x_ld, mode);
  if (!st) st = check_x(x, a.x_ld, a.xh);
  if (st) return st;
  if (bits < 4 || bits > 6 || (bits > 4 && !hb)) return RWKVQ_ERR_ARG;
  a.q = nib; a.hb = hb; a.rec = rec;
  hipStream_t s = (hipStream_t)stream;
  if (bits == 4) return launch_gemm<F_SB6_4>(a, s);
  if (bits == 5) return launch_gemm<F_SB6_5>(a, s);
  return launch_gemm<F_SB6_6>(a, s);
}

int rwkvq_gemm_sym(const uint8_t* codes, const uint32_t* hb, const int8_t* qs,
                   const uint16_t* d, int bits, int rows, int in, int out_per,
                   const float* x, long x_ld, float* y, int M, int mode,
                   void* stream) {
  GemmArgs a = make_args(rows, in, out_per, x, x_ld, y, M, mode);
  int st = check_gemm(rows, in, out_per, M, a.x_ld, mode);
  if (!st) st = check_x(x, a.x_ld, a.xh);
  if (st) return st;
  if ((bits != 6 && bits != 8) || (bits == 6 && !hb)) return RWKVQ_ERR_ARG;
  a.q = codes; a.hb = hb; a.qs = qs; a.d = d;
  hipStream_t s = (hipStream_t)stream;
  return bits == 6 ? launch_gemm<F_SYM6>(a, s) : launch_gemm<F_SYM8>(a, s);
}

int rwkvq_gemm_rtn8(const int8_t* codes, const uint16_t* scale, int rows,
                    int in, int out_per, const float* x, long x_ld, float* y,
                    int M, int mode, void* stream) {
  GemmArgs a = make_args(rows, in, out_per, x, x_ld, y, M, mode);
  int st = check_gemm(rows, in, out_per, M, a.x_ld, mode);
  if (!st) st = check_x(x, a.x_ld, a.xh);
  if (st) return st;
  a.q = reinterpret_cast<const uint8_t*>(codes); a.d = scale;
  return launch_gemm<F_RTN8>(a, (hipStream_t)stream);
}

int rwkvq_gemm_f16(const uint16_t* w, int rows, int in, int out_per,
                   const float* x, long x_ld, float* y, int M, int mode,
                   int seg_modes, void* stream) {
  const int flags = mode & ~15;
  mode &= 15;
  GemmArgs a = make_args(rows, in, out_per, x, x_ld, y, M,
                         (mode == RWKVQ_EPI_PER_SEG ? 0 : mode) | flags);
  int st = check_gemm(rows, in, out_per, M, a.x_ld,
                      (mode == RWKVQ_EPI_PER_SEG ? 0 : mode) | flags, kStepK);
  if (!st) st = check_x(x, a.x_ld, a.xh);
  if (st) return st;
  if (mode == RWKVQ_EPI_PER_SEG) {
    for (int j = 0; j < rows / out_per; ++j) {
      const int m = (seg_modes >> (4 * j)) & 15;
      if (m > RWKVQ_EPI_SIGMOID || j >= 8 ||
          (a.yord >= 0 && m == RWKVQ_EPI_ADD))
        return RWKVQ_ERR_ARG;
    }
    a.mode = mode;
    a.seg_modes = seg_modes;
  }
  a.q = reinterpret_cast<const uint8_t*>(w);
  return launch_gemm<F_F16>(a, (hipStream_t)stream);
}

int rwkvq_gemm_f16_seg(const uint16_t* w, int nseg, const int* seg_rows,
                       int in, const float* x, long x_ld, float* y, int M,
                       int seg_modes, int flags, void* stream) {
  if (!w || !x || !y || nseg < 1 || nseg > 8 || in <= 0 || in % kStepK ||
      M <= 0 || (flags & 15) ||
      check_gemm(128, 128, 128, 1, 128, flags, kStepK))
    return RWKVQ_ERR_ARG;
  int rows = 0;
  GemmArgs a = make_args(128, 128, 128, x, x_ld, y, M, flags);
  for (int j = 0; j < nseg; ++j) {
    const int m = (seg_modes >> (4 * j)) & 15;
    if (seg_rows[j] <= 0 || seg_rows[j] % 128 || m > RWKVQ_EPI_SIGMOID ||
        (a.yord >= 0 && m == RWKVQ_EPI_ADD))
      return RWKVQ_ERR_ARG;
    rows += seg_rows[j];
    a.seg_end[j] = rows;
  }
  a.x = x; a.y = y; a.M = M; a.N = rows; a.in = in; a.out_per = rows;
  a.ldy = rows;
  a.x_ld = x_ld > 0 ? x_ld : (long)nseg * in;
  if (a.x_ld < (long)nseg * in || check_x(x, a.x_ld, a.xh))
    return RWKVQ_ERR_ARG;
  a.mode = RWKVQ_EPI_PER_SEG;
  a.seg_modes = seg_modes;
  a.nseg_tab = nseg;
  a.q = reinterpret_cast<const uint8_t*>(w);
  return launch_gemm<F_F16>(a, (hipStream_t)stream);
}

int rwkvq_gemm_dual_f16seg(int kind, int bits, const void* p0, const void* p1,
                           const void* p2, const void* p3, int rows, int in,
                           int out_per, const void* x, long x_ld, float* y,
                           int mode, const uint16_t* w, int nseg,
                           const int* seg_rows, const void* xb, long xb_ld,
                           float* yb, int seg_modes, int flags_b, int M,
                           void* stream) {
  hipStream_t s = (hipStream_t)stream;
  // GEMM a: the quantized projection, as rwkvq_gemm_{sb6,sym,rtn8}
  GemmArgs a = make_args(rows, in, out_per, static_cast<const float*>(x),
                         x_ld, y, M, mode);
  int st = check_gemm(rows, in, out_per, M, a.x_ld, mode);
  if (!st) st = check_x(x, a.x_ld, a.xh);
  if (st) return st;
  int fa;
  if (kind == 0) {                               // sb6: nib, hb, rec
    if (bits < 4 || bits > 6 || (bits > 4 && !p1) || !p0 || !p2)
      return RWKVQ_ERR_ARG;
    a.q = static_cast<const uint8_t*>(p0);
    a.hb = static_cast<const uint32_t*>(p1);
    a.rec = static_cast<const uint8_t*>(p2);
    fa = bits == 4 ? F_SB6_4 : bits == 5 ? F_SB6_5 : F_SB6_6;
  } else if (kind == 1) {                        // sym: codes, hb, qs, d
    if ((bits != 6 && bits != 8) || (bits == 6 && !p1) || !p0 || !p2 || !p3)
      return RWKVQ_ERR_ARG;
    a.q = static_cast<const uint8_t*>(p0);
    a.hb = static_cast<const uint32_t*>(p1);
    a.qs = static_cast<const int8_t*>(p2);
    a.d = static_cast<const uint16_t*>(p3);
    fa = bits == 6 ? F_SYM6 : F_SYM8;
  } else if (kind == 2) {                        // rtn8: codes, scale
    if (bits != 8 || !p0 || !p3) return RWKVQ_ERR_ARG;
    a.q = static_cast<const uint8_t*>(p0);
    a.d = static_cast<const uint16_t*>(p3);
    fa = F_RTN8;
  } else {
    return RWKVQ_ERR_ARG;
  }
  // GEMM b: the segmented fp16 GEMM, as rwkvq_gemm_f16_seg
  if (!w || !xb || !yb || nseg < 1 || nseg > 8 || in % kStepK ||
      (flags_b & 15) || check_gemm(128, 128, 128, 1, 128, flags_b, kStepK))
    return RWKVQ_ERR_ARG;
  GemmArgs b = make_args(128, 128, 128, static_cast<const float*>(xb), xb_ld,
                         yb, M, flags_b);
  int rows_b = 0;
  for (int j = 0; j < nseg; ++j) {
    const int m = (seg_modes >> (4 * j)) & 15;
    if (seg_rows[j] <= 0 || seg_rows[j] % 128 || m > RWKVQ_EPI_SIGMOID ||
        (b.yord >= 0 && m == RWKVQ_EPI_ADD))
      return RWKVQ_ERR_ARG;
    rows_b += seg_rows[j];
    b.seg_end[j] = rows_b;
  }
  b.x = static_cast<const float*>(xb); b.y = yb; b.N = rows_b; b.in = in;
  b.out_per = rows_b; b.ldy = rows_b;
  b.x_ld = xb_ld > 0 ? xb_ld : (long)nseg * in;
  if (b.x_ld < (long)nseg * in || check_x(xb, b.x_ld, b.xh))
    return RWKVQ_ERR_ARG;
  b.mode = RWKVQ_EPI_PER_SEG;
  b.seg_modes = seg_modes;
  b.nseg_tab = nseg;
  b.q = reinterpret_cast<const uint8_t*>(w);

  // One launch of 128 x 128 tiles (two K groups, no split) when GEMM a
  // leaves CUs free; otherwise the two GEMMs as separate launches.
  const long mt = (M + 127) / 128;
  const long ta = (rows / 128) * mt, tb = (rows_b / 128) * mt;
  const bool dual = a.xh && b.xh && M > 64 && (in / kStepK) % 2 == 0 &&
                    ta < 256;
  if (!dual) {
    auto one = [&](int f, const GemmArgs& g) {
      switch (f) {
        case F_SB6_4: return launch_gemm<F_SB6_4>(g, s);
        case F_SB6_5: return launch_gemm<F_SB6_5>(g, s);
        case F_SB6_6: return launch_gemm<F_SB6_6>(g, s);
        case F_SYM6: return launch_gemm<F_SYM6>(g, s);
        case F_SYM8: return launch_gemm<F_SYM8>(g, s);
        case F_RTN8: return launch_gemm<F_RTN8>(g, s);
        default: return launch_gemm<F_F16>(g, s);
      }
    };
    st = one(fa, a);
    return st ? st : one(F_F16, b);
  }
  // GEMM b's tiles take as long as a's at half the steps (fp16 weights are
  // twice the bytes): split b's K in two where the workspace allows
  a.split = b.split = 1;
  const SplitWs* ws = (flags_b & RWKVQ_NO_SPLIT) ? nullptr : current_ws();
  if (ws && (in / kStepK) % 4 == 0 && tb <= ws->ncnt &&
      tb * 2 * 128 * 128 * (long)sizeof(float) <= ws->bytes) {
    b.split = 2;
    b.ws = ws->ws;
    b.cnt = ws->cnt;
  }
  a.nt = rows / 128; b.nt = rows_b / 128;
  a.mt = b.mt = (int)mt;
  const dim3 grid((unsigned)(ta + tb * b.split)), block(512);
  switch (fa) {
#define RWKVQ_DUAL(F)                                                        \
  case F:                                                                    \
    hipLaunchKernelGGL((gemm_dual_kernel<F, F_F16, 1, 4, 2, true, 4>), grid, \
                       block, 0, s, a, b, (int)ta);                          \
    break;
    RWKVQ_DUAL(F_SB6_4)
    RWKVQ_DUAL(F_SB6_5)
    RWKVQ_DUAL(F_SB6_6)
    RWKVQ_DUAL(F_SYM6)
    RWKVQ_DUAL(F_SYM8)
    RWKVQ_DUAL(F_RTN8)
#undef RWKVQ_DUAL
    default: return RWKVQ_ERR_ARG;
  }
  return hipGetLastError() == hipSuccess ? RWKVQ_OK : RWKVQ_ERR_LAUNCH;
}

int rwkvq_gemm_f16_grouped(int nseg, const uint16_t* const* w,
                           const int* rows, const int* in,
                           const void* const* x, const long* x_ld,
                           float* const* y, int M, int seg_modes, int flags,
                           void* stream) {
  if (nseg < 1 || nseg > 8 || !w || !rows || !in || !x || !x_ld || !y ||
      M <= 0 || (flags & 15) ||
      check_gemm(128, 128, 128, 1, 128, flags, kStepK))
    return RWKVQ_ERR_ARG;
  GemmArgs a = make_args(128, 128, 128, nullptr, 0, nullptr, M, flags);
  a.split = 1;
  int tot = 0;
  for (int j = 0; j < nseg; ++j) {
    const int m = (seg_modes >> (4 * j)) & 15;
    if (!w[j] || !x[j] || !y[j] || rows[j] <= 0 || rows[j] % 128 ||
        in[j] <= 0 || in[j] % kStepK || x_ld[j] < in[j] ||
        check_x(x[j], x_ld[j], a.xh) || m > RWKVQ_EPI_SIGMOID ||
        (a.yord >= 0 && m == RWKVQ_EPI_ADD))
      return RWKVQ_ERR_ARG;
    a.gq[j] = reinterpret_cast<const uint8_t*>(w[j]);
    a.gx[j] = static_cast<const float*>(x[j]);
    a.gxld[j] = x_ld[j];
    a.gy[j] = y[j];
    a.gin[j] = in[j];
    a.gin_rows[j] = rows[j];
    tot += rows[j];
    a.seg_end[j] = tot;
  }
  a.grouped = 1;
  a.nseg_tab = nseg;
  a.mode = RWKVQ_EPI_PER_SEG;
  a.seg_modes = seg_modes;
  a.N = tot; a.out_per = tot; a.in = kStepK;   // (per segment in the kernel)
  a.q = a.gq[0]; a.x = a.gx[0]; a.y = a.gy[0];
  hipStream_t s = (hipStream_t)stream;
  // one workgroup per (128-row tile, token tile), one K group: the
  // segments' step counts differ
  auto wgs = [&](int bm) { return (long)(tot / 128) * ((M + bm - 1) / bm); };
  if (wgs(128) >= 256)
    return launch_tile<F_F16, 1, 4>(a, s, {1, 4, 4, 1, true}, nullptr);
  if (wgs(64) >= 256)
    return launch_tile<F_F16, 1, 2>(a, s, {1, 2, 4, 1, true}, nullptr);
  return launch_tile<F_F16, 1, 1>(a, s, {1, 1, 4, 1, true}, nullptr);
}

int rwkvq_gemm_plan(int rows, int in, int out_per, int M, int mode,
                    int* plan) {
  if (!plan) return RWKVQ_ERR_ARG;
  const int st = check_gemm(rows, in, out_per, M, (long)(rows / out_per) * in,
                            mode, kStepK);
  if (st) return st;
  GemmArgs a = make_args(rows, in, out_per, nullptr, 0, nullptr, M, mode);
  const GemmPlan p = plan_gemm(a, gemm_ws(a));
  plan[0] = 32 * p.nw * p.wn;
  plan[1] = 32 * p.wm;
  plan[2] = p.nw;
  plan[3] = plan_kgroups(p, in);
  plan[4] = p.split;
  plan[5] = (rows / plan[0]) * ((M + plan[1] - 1) / plan[1]) * p.split;
  return RWKVQ_OK;
}

}  // extern "C"
