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
#define RWKVQ_EPI_PER_SEG 5  /* rwkvq_gemm_f16: mode of segment j in bits
                                4j..4j+3 of seg_modes */

/* GEMM flags, or-ed into the epilogue of rwkvq_gemm_*:
 *   RWKVQ_X_F16  x is fp16 in the pair order of the weight format
 *                (rwkvq_x16), x_ld in halves;
 *   RWKVQ_Y_F16 | (order << RWKVQ_Y_ORDER_SHIFT)  y is written as fp16
 *                [M, rows] in pair order `order` (the input of a GEMM over
 *                a format of that order); not with RWKVQ_EPI_ADD. */
#define RWKVQ_X_F16 16
#define RWKVQ_Y_F16 32
#define RWKVQ_Y_ORDER_SHIFT 6
/* GEMM flag: do not split K (the split-K workspace serves one stream; a
 * GEMM launched concurrently on another stream passes this) */
#define RWKVQ_NO_SPLIT 256
/* Pair orders of fp16 GEMM inputs: within each 32-column group, halves
 * 2i, 2i+1 hold columns (c0(i), c1(i)) -- the order in which the format's
 * decoder pairs its weights. */
#define RWKVQ_ORDER_PAIRS 0  /* (2i, 2i+1): sym8, rtn8, dense fp16 */
#define RWKVQ_ORDER_SB6 1    /* (i, i+16): sb6 int4/5/6 */
#define RWKVQ_ORDER_SYM6 2   /* (i, i+8) for i < 8, (i+8, i+16) else: sym6 */

/* ---------------------------------------------------------------- GEMV
 * y[n, r] = epi( sum_c x[n, r / out_per, c] * W[r, c] ),  n < n_cols.
 * x is fp32 with element (n, seg, c) at x[n * x_ld + seg * IN + c]
 * (x_ld = 0 means packed: (rows / out_per) * IN); y is fp32 [n_cols, rows].
 * out_per == rows is the plain GEMV; out_per < rows runs K = rows/out_per
 * row-concatenated matrices with their own inputs in one launch (the fused
 * r/k/v projection).  IN % 256 == 0, IN <= 16384, out_per % 2 == 0.
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
                   long x_ld, float* y, int n_cols, int epilogue, void* stream);
int rwkvq_gemv_sym(const uint8_t* codes, const uint32_t* hb, const int8_t* qs,
                   const uint16_t* d, int bits, int rows, int in, int out_per,
                   const float* x, long x_ld, float* y, int n_cols,
                   int epilogue, void* stream);
int rwkvq_gemv_rtn8(const int8_t* codes, const uint16_t* scale, int rows,
                    int in, int out_per, const float* x, long x_ld, float* y,
                    int n_cols, int epilogue, void* stream);

/* SpQR outliers of the per-row int8 format as CSR per output row:
 * row_ptr [rows + 1], cols [nnz] (int32), vals [nnz] (bf16 bits, the
 * stored outlier values; the codes are 0 there).
 *
 * rwkvq_gemv_rtn8_spqr: y = epi(x . W^T) with W = codes * scale + the
 * outliers (out_per = rows).  One or two input rows sum the row's
 * outliers inside the GEMV (after the row scale, x in fp32); three or
 * more run the matrix-core GEMV, then rwkvq_spqr_apply.
 * Replaces: QuantLinearV2.__call__ with outliers and its kernel's CSR loop
 *   (reference: quant_linear_v2.py:35-84, 322-351).
 * rwkvq_spqr_apply: y[t, r] = epi(y[t, r] + sum_k vals[k] x[t, cols[k]]),
 * k over row r's outliers (the tail after a GEMM / GEMV that stored or
 * accumulated the int8 part); mode RWKVQ_EPI_STORE (plain add), RELU2,
 * TANH or SIGMOID.
 * rwkvq_spqr_scatter: w[r, cols[k]] = vals[k] (the dense dequant's
 * outlier overwrite, codec.py:279-292). */
int rwkvq_gemv_rtn8_spqr(const int8_t* codes, const uint16_t* scale,
                         const int* row_ptr, const int* cols,
                         const uint16_t* vals, int rows, int in,
                         const float* x, long x_ld, float* y, int n,
                         int mode, void* stream);
int rwkvq_spqr_apply(const float* x, long x_ld, const int* row_ptr,
                     const int* cols, const uint16_t* vals, int rows, int n,
                     float* y, int mode, void* stream);
int rwkvq_spqr_scatter(const int* row_ptr, const int* cols,
                       const uint16_t* vals, int rows, float* w, long ld,
                       void* stream);

/* ------------------------------------------------------ prefill GEMM
 * y[t, :] = epilogue(x[t] @ W^T) for t < M tokens, on the matrix cores
 * (v_mfma_f32_32x32x16_f16), W decoded from the same device layouts as the
 * GEMV entry points; same arguments as rwkvq_gemv_* with M in place of
 * n_cols.  Operands are fp16 exactly as the reference's prefill uses them
 * (x rounded once; W = the format's dequant rounded once to fp16; rtn8
 * multiplies the fp32 sum of x * code by its row scale), fp32 accumulate,
 * fp32 out.  Output rows per input segment (out_per) must be a multiple of
 * 128.  No dense copy of W is made.
 *
 * Replaces the reference's prefill path of the same linears, a dense fp16
 * dequant followed by an fp16 matmul:
 *   GwQuantLinear.__call__ / _dequant_w + mx.matmul
 *       (rwkv_quant/backends/metal/quant_linear_gw.py:821-849)
 *   SymQuantLinear.__call__ GEMM branch
 *       (rwkv_quant/backends/metal/quant_linear_sym.py:433-484)
 *   QuantLinearV2.__call__ GEMM branch
 *       (rwkv_quant/backends/metal/quant_linear_v2.py:322-351)
 */
int rwkvq_gemm_sb6(const uint8_t* nib, const uint32_t* hb, const uint8_t* rec,
                   int bits, int rows, int in, int out_per, const float* x,
                   long x_ld, float* y, int M, int epilogue, void* stream);
int rwkvq_gemm_sym(const uint8_t* codes, const uint32_t* hb, const int8_t* qs,
                   const uint16_t* d, int bits, int rows, int in, int out_per,
                   const float* x, long x_ld, float* y, int M, int epilogue,
                   void* stream);
int rwkvq_gemm_rtn8(const int8_t* codes, const uint16_t* scale, int rows,
                    int in, int out_per, const float* x, long x_ld, float* y,
                    int M, int epilogue, void* stream);

/* fp32 x [M, x_ld] -> fp16 out [M, out_ld] (round to nearest even), the
 * first `cols` columns (a multiple of 32) in pair order `order`
 * (RWKVQ_ORDER_*): the GEMMs' RWKVQ_X_F16 input.  x, out 16-byte aligned,
 * x_ld % 4 == 0, out_ld % 8 == 0.  No counterpart in the reference (its
 * matmul rounds x to fp16 itself: x.astype(mx.float16)). */
int rwkvq_x16(const float* x, long x_ld, int cols, int M, int order,
              uint16_t* out, long out_ld, void* stream);

/* Split-K workspace of the GEMMs on the current device: ws (16-byte
 * aligned, ws_bytes) holds partial output tiles, counters[n_counters]
 * (int32, zero when registered) count the workgroups that finished a tile;
 * every launch leaves the counters at zero again.  Without a workspace
 * (the default, or ws == NULL) no GEMM splits K.  Launches that use it
 * must not overlap (one stream at a time).  No counterpart in the
 * reference (its matmul library keeps its own scratch). */
int rwkvq_gemm_workspace(void* ws, long ws_bytes, int* counters,
                         int n_counters);

/* The launch shape rwkvq_gemm_sb6 / _sym / _rtn8 choose for a GEMM of
 * these arguments on the current device (with the split-K workspace that
 * is registered there), without launching anything: plan[0] output rows
 * per workgroup tile, plan[1] tokens per tile, plan[2] waves along the
 * rows, plan[3] K groups inside a workgroup (1 or 2), plan[4] workgroups
 * splitting K per tile, plan[5] workgroups of the launch.  mode as for the
 * GEMMs (RWKVQ_NO_SPLIT changes the plan).  No counterpart in the
 * reference (its matmul library picks its own kernel); for tests and
 * profiles that must know which kernel variant ran. */
int rwkvq_gemm_plan(int rows, int in, int out_per, int M, int mode,
                    int* plan);

/* The same GEMM over dense fp16 rows W [rows, in] (in % 128 == 0): the
 * prefill LoRA products.  With epilogue RWKVQ_EPI_PER_SEG each input
 * segment j (rows j*out_per ..) applies the mode in bits 4j..4j+3 of
 * seg_modes (up to 8 segments), so the down products of the branches
 * (tanh / none / sigmoid) run as one launch.
 * Replaces: QuantTMix._lora at B*T > 1, fp16 matmuls of the dense LoRA
 * factors (reference: quant_model.py:462-526). */
int rwkvq_gemm_f16(const uint16_t* w, int rows, int in, int out_per,
                   const float* x, long x_ld, float* y, int M, int epilogue,
                   int seg_modes, void* stream);

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

/* Dense fp16 expansion for the prefill GEMM: out[r, c] = f16(dequant(W)[r, c])
 * where dequant is the bit-exact fp32 formula above (one rounding).
 * fmt 0/1/2 = sb6@4/5/6 (q = nib, hb, rec), 3/4 = sym@6/8 (q = codes, hb,
 * qs, d), 5 = rtn@8 (q = codes, d = scale).  ld % 8 == 0.
 * Replaces: GwQuantLinear._dequant_w / SymQuantLinear._dequant_w(fp16)
 *   (reference: quant_linear_gw.py:821-840; quant_linear_sym.py:275-363). */
int rwkvq_dequant_f16(int fmt, const uint8_t* q, const uint32_t* hb,
                      const uint8_t* rec, const int8_t* qs, const uint16_t* d,
                      int rows, int in, uint16_t* out, int ld, void* stream);

/* Row gather of a packed matrix into fp32 (the embedding lookup):
 * out[o, :] = dequant(W)[min(max(idx[o], 0), src_rows - 1), :], o < n_idx.
 * kind 0 = sb6 (q = nib, hb, aux0 = rec), 1 = sym (q = codes, hb,
 * aux0 = qs, aux1 = d), 2 = rtn@8 (q = codes, aux1 = scale).  Values are
 * bit-exact with the dequant entry points above.  Kinds 0 and 1 need
 * `out` 16-byte aligned (RWKVQ_ERR_ARG otherwise).
 * Replaces: the emb gather on the dense table
 *   (reference: rwkv_quant/backends/metal/quant_model.py:853, 975). */
int rwkvq_gather_rows_f32(int kind, int bits, const uint8_t* q,
                          const uint32_t* hb, const void* aux0,
                          const uint16_t* aux1, int src_rows, int in,
                          const int64_t* idx, int n_idx, float* out,
                          void* stream);

/* The row gather above fused with the LayerNorm that follows it (ln0):
 * out[o, :] = LN(gather(o)) with weight w, bias b, eps -- bit-exact with
 * rwkvq_gather_rows_f32 followed by rwkvq_layer_norm, in one launch (one
 * workgroup per output row).  in <= 4096, in % 8 == 0 (kinds 0 and 1:
 * in % 256 == 0).
 * Replaces: emb gather + ln0 of the first block
 *   (reference: rwkv_quant/backends/metal/quant_model.py:853-857, 975-976). */
int rwkvq_gather_ln_f32(int kind, int bits, const uint8_t* q,
                        const uint32_t* hb, const void* aux0,
                        const uint16_t* aux1, int src_rows, int in,
                        const int64_t* idx, int n_idx, const float* w,
                        const float* b, float eps, float* out, void* stream);

/* ------------------------------------------------------- RWKV-7 blocks
 * Row layer norm (two-pass mean/variance): y = (x - mean) / sqrt(var + eps)
 * * w + b over rows of D (x and y may alias).
 * Replaces: _layer_norm (reference: quant_model.py:281-284). */
int rwkvq_layer_norm(const float* x, const float* w, const float* b, float* y,
                     int rows, int D, float eps, void* stream);

/* LN (eps 1e-5) + token shift + ncoef lerps for x [B, T, D]:
 * out[(b*T+t), c, :] = xn + (shift - xn) * coef[c, :], shift = xn of the
 * previous token or prev[b] (zeros if prev is NULL) at t = 0;
 * new_prev[b] = xn of the last token (may be NULL).  ncoef is 1 or 6;
 * D <= 4096 and a multiple of 4.
 * Replaces: _token_shift_stateful + the six lerps of the time mix and the
 * one of the channel mix (reference: quant_model.py:292-301, 643-650,
 * 803-809). */
int rwkvq_shift_lerp(const float* x, const float* ln_w, const float* ln_b,
                     const float* prev, const float* coef, int ncoef,
                     float* out, float* new_prev, int B, int T, int D,
                     void* stream);
/* The same with fp16 out [B*T, ncoef, D] (round to nearest even), each
 * 32-column group in pair order `order` (RWKVQ_ORDER_*): the RWKVQ_X_F16
 * input of the prefill GEMMs.  D % 32 == 0, out 16-byte aligned. */
int rwkvq_shift_lerp_f16(const float* x, const float* ln_w, const float* ln_b,
                         const float* prev, const float* coef, int ncoef,
                         uint16_t* out, int order, float* new_prev, int B,
                         int T, int D, void* stream);

/* Per-channel WKV inputs from rkv [N, 3, D] and the LoRA outputs yw, ya,
 * yv (NULL on layer 0) [N, D]: w = exp(-0.606531 * sigmoid(yw + w0)),
 * a = sigmoid(ya + a0), kk = l2norm_head(k * k_k), k' = k (1 + (a-1) k_a),
 * v' = v + (v_first - v) sigmoid(yv + v0) (layer 0: v_first = v);
 * outputs w, k', v', a_wkv = -kk, b_wkv = kk * a, all [N, D].
 * Replaces: reference quant_model.py:693-712. */
int rwkvq_wkv_prep(const float* rkv, const float* yw, const float* ya,
                   const float* yv, const float* w0, const float* a0,
                   const float* v0, const float* k_k, const float* k_a,
                   float* v_first, int layer0, float* w, float* kp, float* vp,
                   float* a, float* b, int N, int D, int head_size,
                   void* stream);

/* WKV-7 recurrence over T tokens for B sequences, H heads of 64:
 * S = S diag(w_t) + (S a_t) b_t^T + v_t k_t^T;  y_t = S r_t  (fp32).
 * Inputs [B, T, H*64] with token stride ld (r: r_ld); state [B, H, 64, 64]
 * (row = value index, column = key index) is read from state_in (or
 * state_out when NULL) and the final state written to state_out;
 * y [B, T, ...] with token stride y_ld.
 * Replaces: rwkv_metal wkv7_infer / wkv7_train (reference call sites
 * quant_model.py:118-125, 394, 714; math rwkv7_ref.py:236-255). */
int rwkvq_wkv7_scan(const float* r, long r_ld, const float* w, const float* k,
                    const float* v, const float* a, const float* b, long ld,
                    const float* state_in, float* state_out, float* y,
                    long y_ld, int B, int T, int H, int head_size,
                    void* stream);

/* rwkvq_wkv7_scan in 16-step chunks: per (sequence, head, chunk) the
 * chunk's transition is built in parallel in WY form (S_end = S0 P +
 * V^T Bq, Y = S0 Ry + V^T Yq, from the cumulative log decay and a 16 x 16
 * unit triangular solve), then the chunks are applied in order on the
 * fp32 matrix cores.  ws: device workspace of at least
 * B * H * NC * 6400 floats (ws_floats), NC = ceil(T / 16) rounded up to a
 * multiple of 3, 16-byte aligned; decays are floored at e^-60.  Same result as the step-by-step scan to fp32
 * rounding (the float64 oracle bar, 1e-5 relative, holds for both).
 * Replaces: rwkv_metal.wkv7_infer for T > 1 (reference: quant_model.py:
 * 118-125, 714; math rwkv7_ref.py:236-255). */
int rwkvq_wkv7_scan_chunked(const float* r, long r_ld, const float* w,
                            const float* k, const float* v, const float* a,
                            const float* b, long ld, const float* state_in,
                            float* state_out, float* y, long y_ld, int B,
                            int T, int H, int head_size, float* ws,
                            long ws_floats, void* stream);

/* rwkvq_wkv7_scan_chunked without a workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, serving
 * loops, harnesses that forbid hipMalloc).  No counterpart in the
 * reference.  The chunk operators live in a library-owned device array of
 * 64 MiB per GPU (allocated with the code object, held until the process
 * ends): B * H * NC * 6400 floats must fit in it (NC = ceil(T / 16)
 * rounded up to a multiple of 3), i.e. B * H * NC <= 2621 (1.5B: T <= 1296
 * at B = 1; 2.9B: T <= 1008), else RWKVQ_ERR_SIZE.  Calls on one GPU share
 * that array: calls that overlap in time (different streams) race; calls
 * in one stream are ordered.  Nothing in it needs to start at zero (each
 * call writes every operator it reads).  Same results as
 * rwkvq_wkv7_scan_chunked, bit for bit. */
int rwkvq_wkv7_scan_chunked_noalloc(const float* r, long r_ld,
                                    const float* w, const float* k,
                                    const float* v, const float* a,
                                    const float* b, long ld,
                                    const float* state_in, float* state_out,
                                    float* y, long y_ld, int B, int T, int H,
                                    int head_size, void* stream);

/* Prefill time-mix core from the projections: the per-channel inputs of
 * rwkvq_wkv_prep (w, k' -> kp, v' -> vp, a, b; v_first written on layer 0,
 * read otherwise) computed inside the chunk-operator kernel, then the
 * chunked scan of rwkvq_wkv7_scan_chunked (r from rkv, v = v'); y, kp, vp
 * are [B*T, H*64].  Equals rwkvq_wkv_prep + rwkvq_wkv7_scan_chunked with
 * two launches instead of three and no w / a / b round trip through HBM.
 * Replaces: the prep, the recurrence and its call site in the reference's
 * prefill (quant_model.py:638-712, 118-125; rwkv7_ref.py:236-255). */
int rwkvq_wkv7_prefill_chunked(const float* rkv, const float* yw,
                               const float* ya, const float* yv,
                               const float* w0, const float* a0,
                               const float* v0, const float* k_k,
                               const float* k_a, float* v_first, int layer0,
                               float* kp, float* vp, const float* state_in,
                               float* state_out, float* y, int B, int T,
                               int H, int head_size, float* ws,
                               long ws_floats, void* stream);

/* Time-mix tail per head: out = ((GN(y) ln_w + ln_b) + (sum r k' r_k) v') g
 * with a two-pass group norm (eps 64e-5); r is rkv[:, 0, :].
 * Replaces: wkv_tail (reference: fused_tail.py:43-110) and the unfused
 * group_norm + bonus (quant_model.py:269-278, 722-728). */
int rwkvq_wkv_tail(const float* y, const float* rkv, const float* kp,
                   const float* vp, const float* g, const float* r_k,
                   const float* ln_w, const float* ln_b, float* out, int N,
                   int D, int head_size, void* stream);
/* The same with fp16 out [N, D] in pair order `order` (RWKVQ_ORDER_*): the
 * RWKVQ_X_F16 input of the output projection's GEMM. */
int rwkvq_wkv_tail_f16(const float* y, const float* rkv, const float* kp,
                       const float* vp, const float* g, const float* r_k,
                       const float* ln_w, const float* ln_b, uint16_t* out,
                       int order, int N, int D, int head_size, void* stream);

/* Decode (T = 1) time-mix core in one launch per (sequence, head):
 * rwkvq_wkv_prep + one rwkvq_wkv7_scan step + rwkvq_wkv_tail for
 * rkv [B, 3, D] and LoRA outputs [B, D]; state_in -> state_out (may alias).
 * Replaces: the decode path of _forward_stateful_fused from the LoRA
 * outputs to the o_proj input (reference: quant_model.py:693-720). */
int rwkvq_wkv7_decode(const float* rkv, const float* yw, const float* ya,
                      const float* yv, const float* g, const float* w0,
                      const float* a0, const float* v0, const float* k_k,
                      const float* k_a, const float* r_k, const float* ln_w,
                      const float* ln_b, float* v_first, int layer0,
                      const float* state_in, float* state_out, float* out,
                      int B, int H, int head_size, void* stream);

/* Decode core with the LoRA up products folded in: as rwkvq_wkv7_decode,
 * with the branch outputs computed per head from the down outputs
 * h[k] [B, rank[k]] (after their nonlinearity) and the up matrices
 * Bup[k] fp16 [D, rank[k]], k = 0..3 for w, a, v, g (v unused in layer 0,
 * may be null there).  h is rounded to fp16 pairs, products fp32.
 * rank[k] % 8 == 0, rank[k] <= 512.
 * Replaces: the decode path of _forward_stateful_fused from the LoRA down
 * outputs to the o_proj input, including QuantTMix._lora's up products
 * (reference: quant_model.py:462-526, 693-720). */
int rwkvq_wkv7_decode_lora(const float* rkv, const float* const* h,
                           const void* const* Bup, const int* rank,
                           const float* w0, const float* a0, const float* v0,
                           const float* k_k, const float* k_a,
                           const float* r_k, const float* ln_w,
                           const float* ln_b, float* v_first, int layer0,
                           const float* state_in, float* state_out,
                           float* out, int B, int H, int head_size,
                           void* stream);

/* As rwkvq_wkv7_decode_lora, with the up factors read straight from the
 * file's codes of a world checkpoint (stored [rank, D], blocks of 64
 * columns = one head).  Branch k: q[k] the codes permuted to
 * [H][rank / 16][64][16] (head, 16-row block, channel, row); asym: s[k],
 * m[k] the fp32 scale / min as [H][rank]; per-row int8 (s[k] null):
 * sc[k] the fp16 row scales [rank].  Codes, scales and mins enter
 * exactly; h fp32, the sum fp32 as sum_j q_jc (h_j s_j) + sum_j h_j m_j.
 * rank[k] % 16 == 0, rank[k] <= 512, sum of ranks <= 1024, q[k]
 * 16-byte aligned.
 * Replaces: as rwkvq_wkv7_decode_lora, reading the LoRA codes the file
 * stores (reference: quant_model.py:462-526, codec.py:260-292). */
int rwkvq_wkv7_decode_lora_q(const float* rkv, const float* const* h,
                             const uint8_t* const* q, const float* const* s,
                             const float* const* m, const uint16_t* const* sc,
                             const int* rank, const float* w0,
                             const float* a0, const float* v0,
                             const float* k_k, const float* k_a,
                             const float* r_k, const float* ln_w,
                             const float* ln_b, float* v_first, int layer0,
                             const float* state_in, float* state_out,
                             float* out, int B, int H, int head_size,
                             void* stream);

/* rwkvq_gemm_f16 over up to 8 segments of unequal height (seg_rows[j] a
 * multiple of 128) of one matrix w [sum rows, in]: segment j reads
 * x[t * x_ld + j * in + c] and writes columns [sum_{i<j} rows_i, ...) of
 * y [M, sum rows] with epilogue field j of seg_modes.  in % 128 == 0.
 * flags: RWKVQ_X_F16 / RWKVQ_Y_F16 as for rwkvq_gemm_f16 (0: fp32 x, y).
 * Replaces: the down products of QuantTMix._lora in prefill, all
 * branches in one launch, each padded only to 128 rows (reference:
 * quant_model.py:462-526). */
int rwkvq_gemm_f16_seg(const uint16_t* w, int nseg, const int* seg_rows,
                       int in, const float* x, long x_ld, float* y, int M,
                       int seg_modes, int flags, void* stream);

/* A quantized GEMM (as rwkvq_gemm_sb6 / _sym / _rtn8: kind 0 sb6 with p0..p2
 * = nib, hb, rec; kind 1 sym with p0..p3 = codes, hb, qs, d; kind 2 rtn8
 * with p0 = codes, p3 = scale) and a segmented fp16 GEMM of the same K
 * (as rwkvq_gemm_f16_seg: w, nseg, seg_rows, xb, xb_ld, yb, seg_modes,
 * flags_b) over the same M tokens, in one launch when the first leaves CUs
 * free (both inputs RWKVQ_X_F16), else as two launches.  Replaces: the
 * prefill r/k/v projections and the LoRA down products of the time mix,
 * which read the same lerp outputs (reference: quant_model.py:462-526,
 * 643-650). */
int rwkvq_gemm_dual_f16seg(int kind, int bits, const void* p0, const void* p1,
                           const void* p2, const void* p3, int rows, int in,
                           int out_per, const void* x, long x_ld, float* y,
                           int mode, const uint16_t* w, int nseg,
                           const int* seg_rows, const void* xb, long xb_ld,
                           float* yb, int seg_modes, int flags_b, int M,
                           void* stream);

/* Up to 8 independent dense fp16 GEMMs in one launch: segment j computes
 * y[j][t * rows[j] + r] = epi_j(sum_c x_j[t * x_ld[j] + c] * w[j][r * in[j]
 * + c]) for t < M, r < rows[j] (a multiple of 128), c < in[j] (a multiple
 * of 128); epi_j = 4-bit field j of seg_modes.  flags as for
 * rwkvq_gemm_f16_seg (RWKVQ_X_F16: x_j fp16 in natural pair order).
 * Replaces: the up products of QuantTMix._lora in prefill, one matmul per
 * branch in the reference (quant_model.py:462-526), here one launch. */
int rwkvq_gemm_f16_grouped(int nseg, const uint16_t* const* w,
                           const int* rows, const int* in,
                           const void* const* x, const long* x_ld,
                           float* const* y, int M, int seg_modes, int flags,
                           void* stream);

/* Dense fp16 rows in up to 8 segments of one matrix w [sum rows, in], for
 * 1..32 input rows, on the matrix cores: segment j (rows seg_rows[j], a
 * multiple of 16) reads x[n * x_ld + j * in + c] and writes
 * seg_y[j][n * seg_rows[j] + r] = epi_j(sum_c x . w), epi_j = 4-bit field
 * j of seg_modes (RWKVQ_EPI_*).  in % 128 == 0.
 * Replaces: the down products of QuantTMix._lora for a decode batch, all
 * branches in one launch (reference: quant_model.py:462-526). */
int rwkvq_gemv_f16_seg(const uint16_t* w, int nseg, const int* seg_rows,
                       int in, const float* x, long x_ld,
                       float* const* seg_y, int n, int seg_modes,
                       void* stream);

/* Grouped dense-fp16 GEMV of up to 4 low-rank branches in one launch:
 * y_j[n, r] = epi_j( sum_c x_j[n * x_ld_j + c] * W_j[r, c] ), n < N <= 8.
 * in_j % 16 == 0 and in_j <= 512, or in_j in {2048, 2560} (then x_j
 * 16-byte aligned and x_ld_j % 4 == 0).
 * Replaces: QuantTMix._lora down/up products (reference:
 * quant_model.py:462-526). */
int rwkvq_lora_gemv(int n_jobs, const void* const* W, const float* const* x,
                    const int* x_ld, float* const* y, const int* y_ld,
                    const int* rows, const int* in, const int* epi, int N,
                    void* stream);


/* Down products of up to 4 low-rank branches straight from the file's
 * codes of a world checkpoint (stored [in, rank], blocks along the rank):
 * y_j[n * y_ld_j + r] = epi_j( sum_c x_j[n * x_ld_j + c] * W_j[r, c] ),
 * n < N <= 8, with q[j] the codes transposed to [rank, in] and either
 * asym (s[j], m[j]: fp32 scale / min as [ceil(rank / 64), in]) or
 * per-row int8 (s[j] null, sc[j]: fp16 scale per input column [in]).
 * Weights are dequantized exactly as rwkvq_dequant_asym_f32 / _rtn8_f32
 * give them; x fp32, products and sums fp32.  in in {2048, 2560, 4096},
 * N * in <= 16384, rank % 16 == 0, x 16-byte aligned with x_ld % 4 == 0,
 * q 4-byte, s / m 16-byte, sc 8-byte aligned.
 * Replaces: QuantTMix._lora down products at decode, reading the LoRA
 * codes the file stores (reference: quant_model.py:462-526,
 * codec.py:260-292). */
int rwkvq_lora_down_q(int n_jobs, const uint8_t* const* q,
                      const float* const* s, const float* const* m,
                      const uint16_t* const* sc, const float* const* x,
                      const int* x_ld, float* const* y, const int* y_ld,
                      const int* rows, const int* epi, int in, int N,
                      void* stream);

/* ------------------------------------------------- persistent decode
 * Every layer of one batch-1 decode step in one launch of 256 workgroups
 * (one per CU), five phases per layer separated by grid barriers: LN1 +
 * token shift + lerp folded into the r/k/v GEMV rows and the LoRA down
 * products (from the file's codes); the WKV step per head with the LoRA up
 * products; the output projection (+= x); LN2 + shift + lerp folded into
 * the key GEMV (relu^2); the value GEMV (+= x).  Each workgroup loads its
 * next phase's weights while it waits at a barrier.
 * layers: device array of L layer descriptors (the MkLayer struct of
 * csrc/decode_mk.hip; its size from rwkvq_decode_mk_info); x [D] the
 * residual stream after ln0, replaced by the last layer's output; act: the
 * activation arena, act_floats >= L (6 D + F) floats (one region per layer
 * and phase output, so each is written once per launch); x and act
 * 128-byte aligned; vfirst [D]; the LoRA down outputs go to the regions
 * the descriptors name (one 128-byte aligned region per layer); bar: bar_words uint32
 * barrier words, zero before the first launch (every launch leaves them
 * zero); err: set to 1 when a barrier wait ran past its spin limit (the
 * results are then invalid).  Formats (fmt_proj, fmt_cmix): (1, 0) =
 * sb6@5 projections / sb6@4 channel mix, (4, 3) = sym8 / sym6; D = 2048,
 * F = 4 D, H = D / 64.  RWKVQ_ERR_SIZE when the device cannot hold all
 * the workgroups at once.  Launches on one bar array must not overlap.
 * Replaces: the per-layer decode body, one token per sequence (reference:
 *   rwkv_quant/backends/metal/quant_model.py:638-728, 803-809). */
int rwkvq_decode_mk(const void* layers, int L, int fmt_proj, int fmt_cmix,
                    int D, int F, int H, float* x, float* act,
                    long act_floats, float* vfirst, unsigned* bar, int* err,
                    void* stream);

/* Failed polls of one barrier wait of rwkvq_decode_mk before it records the error
 * flag and stops waiting (0 restores the default, 2^20).  A small limit
 * forces the error path from the host: every wait then ends at once, the
 * launch completes with invalid results and the flag set.
 * Replaces: no reference function (a bound on this kernel's own waits). */
int rwkvq_decode_mk_spin_limit(int limit);

/* Layout facts of rwkvq_decode_mk: the layer descriptor size in bytes,
 * the barrier words, the workgroups per launch, the largest sum of LoRA
 * ranks.  Any pointer may be null.
 * Replaces: no reference function (the descriptor is this library's). */
int rwkvq_decode_mk_info(int* layer_bytes, int* bar_words, int* wgs,
                         int* max_cat);

/* ------------------------------------------------------ perplexity
 * nll[r] = logsumexp(logits[r, :V]) - logits[r, target[r]] for r < rows
 * (one pass over each row, fixed reduction order); a target outside
 * [0, V) or a NaN logit gives NaN.  logits 16-byte aligned, ld % 4 == 0.
 * Replaces: the per-batch NLL of calibration.ablation.perplexity
 *   (reference: rwkv_quant/calibration/ablation.py:21-69). */
int rwkvq_nll_rows(const float* logits, long ld, const int64_t* target,
                   int rows, int V, float* nll, void* stream);

/* ------------------------------------------------------------- probes
 * HBM read ceiling: stream `bytes` (multiple of 16) with 16-byte loads
 * from n_blocks workgroups of 256 threads; out[n_blocks] receives a
 * checksum per workgroup.  The measured rate is the roofline reference
 * next to the 8 TB/s datasheet peak.
 * Replaces: the reference's stream-read ceiling probe
 *   (reference: tests/bench_membw.py; NEXT_SESSION.md:2961-2996).
 */
int rwkvq_probe_stream_read(const void* buf, long bytes, uint32_t* out,
                            int n_blocks, void* stream);

#ifdef __cplusplus
}
#endif
#endif
