"""Quantized Linear layers of the HIP backend.

Same contract as the reference Metal classes
(reference: rwkv_quant/backends/metal/quant_linear_gw.py:747-1020,
            rwkv_quant/backends/metal/quant_linear_sym.py:372-574,
            rwkv_quant/backends/metal/quant_linear_v2.py:282-351):

  Linear(qt)                   load-time repack of the canonical buffers
                               into the device layout (memory 1x)
  .in_features / .out_features
  __call__(x [..., IN])        -> [..., OUT] float32 on the GPU
  _dequant_w(dtype)            dense [OUT, IN] (float32 is bit-exact with
                               the format's dequant)
  Fused(lins)(xstack [K, IN])  -> [K, out_per]: the K row-concatenated
                               matrices in one launch

Batches of up to GEMM_MIN_BATCH_NB - 1 rows take the GEMV kernels (fp32
x and exact weights to about 22 bits, like the reference's k3 / k3nb
kernels; the batched one reads each weight once per 16 or 32 rows);
larger batches (prefill) take the MFMA GEMM with the dequantization fused
into its operand load and fp16 operands, as the reference's prefill
matmul.  Every path runs a HIP kernel of librwkvq_hip; nothing here
computes on the CPU.
"""
import ctypes

import numpy as np
import torch

from . import _lib
from .repack import rtn8_device, sb6_device, sym_device

GEMM_MIN_BATCH_NB = 128          # reference: quant_linear_gw.py:153
GEMM_ROW_TILE = 128              # output rows per MFMA GEMM tile
# Below GEMM_MIN_BATCH_NB rows the fp16-operand MFMA GEMM is faster than
# the batched GEMV from 33 rows on every 2.9B shape, and from 17 rows where
# the output has at least GEMM_WIDE_ROWS rows (measured on MI355X), but it
# rounds x and W to fp16 (the reference keeps fp32 x below 128 rows).
# GEMM_MID_BATCH / GEMM_WIDE_BATCH = GEMM_MIN_BATCH_NB keep the precise
# GEMV for every decode batch; lowering them trades that precision for
# speed (33 / 17 were the measured cross-over points).
GEMM_MID_BATCH = GEMM_MIN_BATCH_NB
GEMM_WIDE_BATCH = GEMM_MIN_BATCH_NB
GEMM_WIDE_ROWS = 4096


def _np(t):
    return None if t is None else t.detach().cpu().contiguous().numpy()


def _dev(a, device):
    if a is None:
        return None
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def _flat_x(x, in_features):
    if not x.is_cuda:
        raise ValueError("HIP linear: input must be a GPU tensor")
    lead = x.shape[:-1]
    x2 = x.reshape(-1, in_features)
    if x2.dtype != torch.float32:
        x2 = x2.float()
    return lead, x2.contiguous()


class _HipLinearBase:
    out_features: int
    in_features: int
    device: torch.device

    def _kargs(self):
        """(entry-point suffix, leading arguments) of this format's GEMV /
        GEMM entry points; both take the same argument list."""
        raise NotImplementedError

    def _run(self, kind, x2, y, out_per=None, mode=_lib.EPI_STORE, n=None,
             x_ld=0):
        k = 1 if out_per is None else self.out_features // out_per
        suffix, lead = self._kargs()
        _lib.call(f"rwkvq_{kind}_{suffix}", *lead, self.out_features,
                  self.in_features, out_per or self.out_features,
                  _lib.ptr(x2), x_ld, _lib.ptr(y),
                  n if n is not None else x2.shape[0] // k, mode,
                  _lib.stream_handle())

    def _gemv(self, x2, y, out_per=None, mode=_lib.EPI_STORE, n=None,
              x_ld=0):
        self._run("gemv", x2, y, out_per, mode, n, x_ld)

    def gemm_ok(self, out_per=None):
        """The MFMA GEMM tiles output rows by 128 per input segment."""
        return (out_per or self.out_features) % GEMM_ROW_TILE == 0

    def _apply(self, x2, y, out_per=None, mode=_lib.EPI_STORE, n=None,
               x_ld=0):
        rows = n if n is not None else x2.shape[0]
        if rows < GEMM_MIN_BATCH_NB and self.gemm_ok(out_per) and (
                rows >= GEMM_MID_BATCH or (rows >= GEMM_WIDE_BATCH and
                                           self.out_features >= GEMM_WIDE_ROWS)):
            self._run("gemm", x2, y, out_per, mode, n, x_ld)
        elif rows < GEMM_MIN_BATCH_NB:
            self._gemv(x2, y, out_per, mode, n, x_ld)
        elif self.gemm_ok(out_per):
            self._run("gemm", x2, y, out_per, mode, n, x_ld)
        else:
            # output rows off the MFMA GEMM's 128-row tiles: the GEMV
            # kernels take any number of input rows (in launches of up to
            # 32), exact weights and fp32 x
            self._gemv(x2, y, out_per, mode, n, x_ld)

    def __call__(self, x, mode=_lib.EPI_STORE):
        lead, x2 = _flat_x(x, self.in_features)
        n = x2.shape[0]
        y = torch.empty((n, self.out_features), dtype=torch.float32,
                        device=x2.device)
        self._apply(x2, y, mode=mode)
        return y.reshape(*lead, self.out_features)

    def gemv_into(self, x2, y, mode=_lib.EPI_STORE, n=None, x_ld=0):
        """y [N, OUT] (preallocated) <- epi(x2 [N, IN] @ W^T) with the GEMV
        kernel.  With x_ld, row n of the input starts at element n * x_ld of
        x2 (a strided view); n is then the number of rows."""
        self._gemv(x2, y, mode=mode, n=n, x_ld=x_ld)
        return y

    def apply_into(self, x2, y, mode=_lib.EPI_STORE, n=None, x_ld=0):
        """As gemv_into, with the kernel chosen by the row count: GEMV below
        GEMM_MIN_BATCH_NB rows, the MFMA GEMM from there on."""
        self._apply(x2, y, mode=mode, n=n, x_ld=x_ld)
        return y

    def _dequant_w(self, dtype=torch.float16):
        """Dense [OUT, IN]; float32 is bit-exact with the format's dequant,
        float16 is exactly its one rounding (rwkvq_dequant_f16)."""
        if dtype == torch.float16 and self._f16_args() is not None:
            w = torch.empty((self.out_features, self.in_features),
                            dtype=torch.float16, device=self.device)
            fmt, q, hb, rec, qs, d = self._f16_args()
            _lib.call("rwkvq_dequant_f16", fmt, _lib.ptr(q), _lib.ptr(hb),
                      _lib.ptr(rec), _lib.ptr(qs), _lib.ptr(d),
                      self.out_features, self.in_features, _lib.ptr(w),
                      self.in_features, _lib.stream_handle())
            return w
        w = torch.empty((self.out_features, self.in_features),
                        dtype=torch.float32, device=self.device)
        self._dequant_into(w)
        return w if dtype == torch.float32 else w.to(dtype)

    def _f16_args(self):
        return None

    # pair order of the fp16 GEMM input (RWKVQ_X_F16); None: fp32 only
    x16_order = None


class GwQuantLinear(_HipLinearBase):
    """sb6 tensor (gs 32, sb 8, bits 4/5/6)."""

    def __init__(self, qt, device="cuda"):
        assert qt.gw_mode == "sb6", qt.gw_mode
        assert qt.gw_gs == 32 and qt.gw_sb == 8, (qt.gw_gs, qt.gw_sb)
        self.out_features, self.in_features = qt.shape
        self.bits = int(qt.bits)
        self.xbits = self.bits - 4
        self.has_qh = self.xbits >= 1
        self.device = torch.device(device)
        lay = sb6_device(_np(qt.codes_packed), _np(qt.gw_qsqm), _np(qt.gw_d),
                         _np(qt.gw_dm), shape=qt.shape, bits=self.bits,
                         qh=_np(qt.gw_qh), qh2=_np(qt.gw_qh2))
        self._set(lay)

    def _set(self, lay):
        self.nib = _dev(lay["nib"], self.device)
        self.hb = _dev(lay["hb"], self.device) if lay["hb"] is not None \
            else None
        self.rec = _dev(lay["rec"], self.device)

    def _kargs(self):
        return "sb6", (_lib.ptr(self.nib), _lib.ptr(self.hb),
                       _lib.ptr(self.rec), self.bits)

    x16_order = _lib.ORDER_SB6

    def _f16_args(self):
        return (self.bits - 4, self.nib, self.hb, self.rec, None, None)

    def _dequant_into(self, w):
        _lib.call("rwkvq_dequant_sb6_f32", _lib.ptr(self.nib),
                  _lib.ptr(self.hb), _lib.ptr(self.rec), self.bits,
                  self.out_features, self.in_features, _lib.ptr(w),
                  self.in_features, _lib.stream_handle())


class SymQuantLinear(_HipLinearBase):
    """sym tensor (Q6_K style, gs 16, sb 16, bits 6/8)."""

    def __init__(self, qt, device="cuda"):
        assert qt.gw_mode == "sym", qt.gw_mode
        assert qt.gw_gs == 16 and qt.gw_sb == 16, (qt.gw_gs, qt.gw_sb)
        self._build(shape=qt.shape, bits=qt.bits, codes=_np(qt.codes),
                    codes_packed=_np(qt.codes_packed), qh=_np(qt.gw_qh),
                    qh2=_np(qt.gw_qh2), qs=_np(qt.gw_qs), d=_np(qt.gw_d),
                    device=device)

    @classmethod
    def from_buffers(cls, *, shape, bits, qs, d, codes=None,
                     codes_packed=None, qh=None, qh2=None, device="cuda"):
        """Torch-free construction from numpy buffers
        (reference: quant_linear_sym.py:392-405)."""
        obj = cls.__new__(cls)
        obj._build(shape=shape, bits=bits, codes=codes,
                   codes_packed=codes_packed, qh=qh, qh2=qh2, qs=qs, d=d,
                   device=device)
        return obj

    def _build(self, *, shape, bits, codes, codes_packed, qh, qh2, qs, d,
               device):
        self.out_features, self.in_features = shape
        assert self.in_features % 256 == 0, \
            f"sym kernel: IN={self.in_features} is not a multiple of 256"
        self.bits = int(bits)
        self.device = torch.device(device)
        lay = sym_device(qs, d, shape=shape, bits=self.bits, codes=codes,
                         codes_packed=codes_packed, qh=qh, qh2=qh2)
        self.codes = _dev(lay["codes"], self.device)
        self.hb = _dev(lay["hb"], self.device) if lay["hb"] is not None \
            else None
        self.qs = _dev(lay["qs"], self.device)
        self.d = _dev(lay["d"].view(np.uint16), self.device)

    def can_fuse_with(self, other):
        return (self.bits == other.bits
                and self.in_features == other.in_features
                and self.out_features == other.out_features)

    def _kargs(self):
        return "sym", (_lib.ptr(self.codes), _lib.ptr(self.hb),
                       _lib.ptr(self.qs), _lib.ptr(self.d), self.bits)

    @property
    def x16_order(self):
        return _lib.ORDER_SYM6 if self.bits == 6 else _lib.ORDER_PAIRS

    def _f16_args(self):
        return (3 if self.bits == 6 else 4, self.codes, self.hb, None,
                self.qs, self.d)

    def _dequant_into(self, w):
        _lib.call("rwkvq_dequant_sym_f32", _lib.ptr(self.codes),
                  _lib.ptr(self.hb), _lib.ptr(self.qs), _lib.ptr(self.d),
                  self.bits, self.out_features, self.in_features,
                  _lib.ptr(w), self.in_features, _lib.stream_handle())


class QuantLinearV2(_HipLinearBase):
    """Per-row RTN int8 (+ optional SpQR outliers)."""

    def __init__(self, qt, device="cuda"):
        assert qt.bits < 16
        if qt.codes is None:
            raise NotImplementedError("HIP rtn kernel: packed int4 rtn is "
                                      "not supported (no preset uses it)")
        self.out_features, self.in_features = qt.shape
        assert self.in_features % 256 == 0, \
            f"rtn kernel: IN={self.in_features} is not a multiple of 256"
        self.device = torch.device(device)
        lay = rtn8_device(_np(qt.codes), _np(qt.scale), shape=qt.shape)
        self.codes = _dev(lay["codes"], self.device)
        self.scale = _dev(lay["scale"].view(np.uint16), self.device)
        self.has_outliers = (qt.outlier_indices is not None
                             and qt.outlier_indices.numel() > 0)
        if self.has_outliers:
            self.sp_ptr, self.sp_col, self.sp_val = spqr_csr(qt, self.device)

    def _kargs(self):
        return "rtn8", (_lib.ptr(self.codes), _lib.ptr(self.scale))

    @property
    def x16_order(self):
        # the outlier correction reads x in fp32
        return None if self.has_outliers else _lib.ORDER_PAIRS

    def _run(self, kind, x2, y, out_per=None, mode=_lib.EPI_STORE, n=None,
             x_ld=0):
        if not self.has_outliers:
            return super()._run(kind, x2, y, out_per, mode, n, x_ld)
        if (out_per not in (None, self.out_features) or mode & ~15
                or mode > _lib.EPI_SIGMOID):
            raise NotImplementedError("SpQR outliers: one segment, fp32 "
                                      "x and y")
        rows = n if n is not None else x2.shape[0]
        ld = x_ld or self.in_features
        P = _lib.ptr
        csr = (P(self.sp_ptr), P(self.sp_col), P(self.sp_val))
        if kind == "gemv":
            _lib.call("rwkvq_gemv_rtn8_spqr", P(self.codes), P(self.scale),
                      *csr, self.out_features, self.in_features, P(x2), ld,
                      P(y), rows, mode, _lib.stream_handle())
            return
        # the MFMA GEMM stores (or accumulates) the int8 part; the outlier
        # tail and the epilogue follow in rwkvq_spqr_apply (x fp32)
        add = mode == _lib.EPI_ADD
        super()._run(kind, x2, y, None, _lib.EPI_ADD if add else
                     _lib.EPI_STORE, n, x_ld)
        _lib.call("rwkvq_spqr_apply", P(x2), ld, *csr, self.out_features,
                  rows, P(y), _lib.EPI_STORE if add else mode,
                  _lib.stream_handle())

    def _f16_args(self):
        if self.has_outliers:
            return None
        return (5, self.codes, None, None, None, self.scale)

    def _dequant_into(self, w):
        _lib.call("rwkvq_dequant_rtn8_f32", _lib.ptr(self.codes),
                  _lib.ptr(self.scale), self.out_features, self.in_features,
                  _lib.ptr(w), self.in_features, _lib.stream_handle())
        if self.has_outliers:
            _lib.call("rwkvq_spqr_scatter", _lib.ptr(self.sp_ptr),
                      _lib.ptr(self.sp_col), _lib.ptr(self.sp_val),
                      self.out_features, _lib.ptr(w), self.in_features,
                      _lib.stream_handle())


def spqr_csr(qt, device):
    """The SpQR outliers of an rtn tensor, (row, col) pairs + bf16 values,
    as CSR per row on the device: row_ptr int32 [rows + 1], cols int32,
    vals bf16 bits (reference: quant_linear_v2.py:282-321 builds the same
    row offsets at load)."""
    rows = int(qt.shape[0])
    oi = qt.outlier_indices.long().reshape(-1, 2)
    order = torch.argsort(oi[:, 0] * (1 << 32) + oi[:, 1], stable=True)
    r, c = oi[order, 0], oi[order, 1]
    vals = qt.outlier_values.reshape(-1)[order].contiguous().view(torch.int16)
    counts = torch.bincount(r, minlength=rows)
    ptr = torch.zeros(rows + 1, dtype=torch.int64, device=oi.device)
    ptr[1:] = torch.cumsum(counts, 0)
    to = lambda t, dt: t.to(dtype=dt).to(device).contiguous()
    return to(ptr, torch.int32), to(c, torch.int32), to(vals, torch.int16)


class _FusedBase:
    """K row-concatenated linears of one kind and shape, one launch."""

    def __init__(self, lins, cls):
        l0 = lins[0]
        assert all(isinstance(l, cls) for l in lins)
        assert all(l.in_features == l0.in_features
                   and l.out_features == l0.out_features for l in lins)
        self.K = len(lins)
        self.out_per = l0.out_features
        self.out_features = self.out_per * self.K
        self.in_features = l0.in_features

    @property
    def x16_order(self):
        return self._cat.x16_order

    def gemv_into(self, x, y, n, x_ld, mode=_lib.EPI_STORE):
        """y [n, K * out_per] <- the K matrices applied to their own inputs:
        input (row t, matrix k) starts at element t * x_ld + k * IN of x."""
        self._cat._gemv(x, y, out_per=self.out_per, mode=mode, n=n,
                        x_ld=x_ld)
        return y

    def apply_into(self, x, y, n, x_ld, mode=_lib.EPI_STORE):
        """As gemv_into, GEMV below GEMM_MIN_BATCH_NB rows, MFMA GEMM from
        there on."""
        self._cat._apply(x, y, out_per=self.out_per, mode=mode, n=n,
                         x_ld=x_ld)
        return y

    def __call__(self, xstack, mode=_lib.EPI_STORE):
        lead, x2 = _flat_x(xstack, self.in_features)
        assert x2.shape[0] % self.K == 0
        n = x2.shape[0] // self.K
        y = torch.empty((n, self.out_features), dtype=torch.float32,
                        device=x2.device)
        self._cat._apply(x2, y, out_per=self.out_per, mode=mode)
        return y.reshape(n * self.K, self.out_per) if n > 1 else \
            y.reshape(self.K, self.out_per)


class GwQuantLinearFused(_FusedBase):
    def __init__(self, lins):
        super().__init__(lins, GwQuantLinear)
        assert len({l.bits for l in lins}) == 1
        cat = GwQuantLinear.__new__(GwQuantLinear)
        cat.out_features, cat.in_features = self.out_features, self.in_features
        cat.bits, cat.xbits, cat.has_qh = lins[0].bits, lins[0].xbits, \
            lins[0].has_qh
        cat.device = lins[0].device
        cat.nib = torch.cat([l.nib for l in lins])
        cat.hb = None if lins[0].hb is None else torch.cat([l.hb for l in lins])
        cat.rec = torch.cat([l.rec for l in lins])
        self._cat = cat
        self.bits = cat.bits


class SymQuantLinearFused(_FusedBase):
    def __init__(self, lins):
        super().__init__(lins, SymQuantLinear)
        assert all(lins[0].can_fuse_with(l) for l in lins)
        cat = SymQuantLinear.__new__(SymQuantLinear)
        cat.out_features, cat.in_features = self.out_features, self.in_features
        cat.bits, cat.device = lins[0].bits, lins[0].device
        cat.codes = torch.cat([l.codes for l in lins])
        cat.hb = None if lins[0].hb is None else torch.cat([l.hb for l in lins])
        cat.qs = torch.cat([l.qs for l in lins])
        cat.d = torch.cat([l.d for l in lins])
        self._cat = cat
        self.bits = cat.bits


def make_linear(qt, device="cuda"):
    """QuantizedTensor [out, in] -> HIP linear (reference: quant_model.py:245-262)."""
    if qt.bits >= 16:
        return DenseLinear(qt.dense.to(torch.float16), device)
    if qt.gw_mode == "sb6":
        return GwQuantLinear(qt, device)
    if qt.gw_mode == "sym":
        return SymQuantLinear(qt, device)
    if qt.gw_mode == "":
        return QuantLinearV2(qt, device)
    raise NotImplementedError(f"HIP linear for gw_mode={qt.gw_mode!r}")


class DenseLinear:
    """Unquantized [out, in] weight kept in fp16 (reference:
    quant_model.py:202-210), multiplied by the fp16 kernels of librwkvq_hip:
    below GEMM_MIN_BATCH_NB input rows the matrix-core GEMV
    (rwkvq_gemv_f16_seg, up to 32 rows per launch; fp32 x carried as fp16
    hi + lo), from there the MFMA GEMM (rwkvq_gemm_f16_seg, fp16 x, as the
    reference's fp16 matmul).  in % 128 == 0 and out % 16 == 0 (the GEMM
    also out % 128); other shapes raise at construction."""

    def __init__(self, w, device="cuda"):
        self.w = w.to(device=device, dtype=torch.float16).contiguous()
        self.out_features, self.in_features = self.w.shape
        self.device = self.w.device
        if self.in_features % 128 or self.out_features % 16:
            raise NotImplementedError(
                f"fp16 linear {tuple(self.w.shape)}: needs in % 128 == 0 and "
                f"out % 16 == 0")

    def apply_into(self, x2, y, mode=_lib.EPI_STORE, n=None, x_ld=0):
        rows = n if n is not None else x2.shape[0]
        ld = x_ld or self.in_features
        rows_arr = (ctypes.c_int * 1)(self.out_features)
        if rows >= GEMM_MIN_BATCH_NB and self.out_features % GEMM_ROW_TILE == 0:
            _lib.call("rwkvq_gemm_f16_seg", _lib.ptr(self.w), 1, rows_arr,
                      self.in_features, _lib.ptr(x2), ld, _lib.ptr(y), rows,
                      mode, 0, _lib.stream_handle())
            return y
        for n0 in range(0, rows, 32):
            nn = min(32, rows - n0)
            ys = (ctypes.c_void_p * 1)(y.data_ptr() + 4 * n0 * self.out_features)
            _lib.call("rwkvq_gemv_f16_seg", _lib.ptr(self.w), 1, rows_arr,
                      self.in_features, x2.data_ptr() + 4 * n0 * ld, ld, ys,
                      nn, mode, _lib.stream_handle())
        return y

    def __call__(self, x, mode=_lib.EPI_STORE):
        lead, x2 = _flat_x(x, self.in_features)
        y = torch.empty((x2.shape[0], self.out_features), dtype=torch.float32,
                        device=x2.device)
        self.apply_into(x2, y, mode=mode)
        return y.reshape(*lead, self.out_features)
