/* librwkvq_hip -- C ABI of the MI355X (gfx950) kernels of the rwkv_quant
 * HIP backend.
 *
 * Every entry point takes device pointers, sizes and a hipStream_t passed
 * as void*, allocates nothing, launches asynchronously on that stream and
 * returns an int status: 0 (RWKVQ_OK), a RWKVQ_ERR_* code for arguments
 * rejected before launch, or RWKVQ_ERR_LAUNCH when the launch failed.
 *
 * Buffer layouts are the device ("HBM") layouts produced by the host
 * repack (rwkv_quant/backends/hip/repack.py); every one is a byte
 * permutation of the canonical `.rwkvq` fields, with the same byte count:
 *
 *   sb6 (gs 32, sb 8, bits 4/5/6)
 *     nib  u8 [rows, IN/32, 16]  canonical codes_packed (block-local nibbles)
 *     hb   u32 [rows, IN/32]      bits 5: canonical gw_qh word of the block
 *          u32 [rows, IN/32, 2]   bits 6: bits 4,5 of code for columns
 *                                 (i, i+16) at bits (2i', 2i'+1) and
 *                                 (16+2i', 17+2i') of word i/8, i' = i%8
 *     rec  u8 [rows, IN/256, 16]  gw_qsqm (12 B) ++ gw_d (f16) ++ gw_dm (f16)
 *   sym (gs 16, sb 16, bits 6/8)
 *     codes u8 [rows, IN/32, 16] (bits 6, canonical codes_packed) or
 *           i8 [rows, IN] (bits 8, canonical codes)
 *     hb   u32 [rows, IN/32, 2]   bits 6: as sb6@6 with the 16-block pairing
 *                                 (byte i of the group holds columns c and
 *                                 c + 8, c = i < 8 ? i : i + 8)
 *     qs   i8 [rows, IN/16]       canonical gw_qs
 *     d    f16 [rows, IN/256]     canonical gw_d
 *   rtn@8  codes i8 [rows, IN], scale f16 [rows]          (canonical)
 *   asym   codes u8 [rows, IN], scale/min f32 [rows, ceil(IN/gs)] (canonical)
 */
#ifndef RWKVQ_HIP_H
#define RWKVQ_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RWKVQ_OK 0
#define RWKVQ_ERR_ARG 1001
#define RWKVQ_ERR_LAUNCH 1002
#define RWKVQ_ERR_SIZE 1003

/* GEMV epilogues applied to each output element */
#define RWKVQ_EPI_STORE 0    /* y = acc */
#define RWKVQ_EPI_ADD 1      /* y += acc (residual) */
#define RWKVQ_EPI_RELU2 2    /* y = relu(acc)^2 (channel-mix key) */
#define RWKVQ_EPI_TANH 3     /* y = tanh(acc) */
#define RWKVQ_EPI_SIGMOID 4  /* y = sigmoid(acc) */

/* ---------------------------------------------------------------- GEMV
 * y[n, r] = epi( sum_c x[n, r / out_per, c] * W[r, c] ),  n < n_cols.
 * x is fp32 [n_cols, rows / out_per, IN]; y is fp32 [n_cols, rows].
 * out_per == rows is the plain GEMV; out_per < rows runs K = rows/out_per
 * row-concatenated matrices with their own inputs in one launch (the fused
 * r/k/v projection).  IN % 256 == 0, IN <= 8192, out_per % 4 == 0.
 * Inputs are rounded to fp16 pairs; products and sums are fp32.
 *
 * Replaces:
 *   GwQuantLinear._gemv1 / _gemv_nb / GwQuantLinearFused.__call__
 *     (reference: rwkv_quant/backends/metal/quant_linear_gw.py:873-930,
 *      983-1020; kernels :491-557, :658-744)
 *   SymQuantLinear._gemv / SymQuantLinearFused.__call__
 *     (reference: rwkv_quant/backends/metal/quant_linear_sym.py:498-574;
 *      kernels :107-247)
 *   QuantLinearV2.__call__ int8 path
 *     (reference: rwkv_quant/backends/metal/quant_linear_v2.py:322-351;
 *      kernel :35-84)
 */
int rwkvq_gemv_sb6(const uint8_t* nib, const uint32_t* hb, const uint8_t* rec,
                   int bits, int rows, int in, int out_per, const float* x,
                   float* y, int n_cols, int epilogue, void* stream);
int rwkvq_gemv_sym(const uint8_t* codes, const uint32_t* hb, const int8_t* qs,
                   const uint16_t* d, int bits, int rows, int in, int out_per,
                   const float* x, float* y, int n_cols, int epilogue,
                   void* stream);
int rwkvq_gemv_rtn8(const int8_t* codes, const uint16_t* scale, int rows,
                    int in, int out_per, const float* x, float* y, int n_cols,
                    int epilogue, void* stream);

/* ------------------------------------------------------ dequant to fp32
 * Bit-exact with the format's dequant formula: w = q * s + m with
 * s = max(f32(f16(qs * d)), 1e-8), m = f32(f16(qm * dm)) (sb6);
 * w = q * f32(f16(qs * d)) (sym); w = codes * f32(scale) (rtn);
 * w = q * scale[blk] + min[blk] (asym).  Output fp32 [rows, IN] row-major
 * with leading dimension ld (>= IN).
 *
 * Replaces:
 *   codec.dequant_sb6 / dequant_sym / dequant_rtn / dequant_asym
 *     (reference: rwkv_quant/formats/codec.py:183-292)
 *   SymQuantLinear._dequant_w(dtype=float32)
 *     (reference: rwkv_quant/backends/metal/quant_linear_sym.py:433-452)
 */
int rwkvq_dequant_sb6_f32(const uint8_t* nib, const uint32_t* hb,
                          const uint8_t* rec, int bits, int rows, int in,
                          float* w, int ld, void* stream);
int rwkvq_dequant_sym_f32(const uint8_t* codes, const uint32_t* hb,
                          const int8_t* qs, const uint16_t* d, int bits,
                          int rows, int in, float* w, int ld, void* stream);
int rwkvq_dequant_rtn8_f32(const int8_t* codes, const uint16_t* scale,
                           int rows, int in, float* w, int ld, void* stream);
int rwkvq_dequant_asym_f32(const uint8_t* codes, const float* scale,
                           const float* mn, int gs, int rows, int in,
                           float* w, int ld, void* stream);

#ifdef __cplusplus
}
#endif
#endif
