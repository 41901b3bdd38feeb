"""GPU parity of the dequant and GEMV kernels against the CPU oracle.

Bars: device dequant == oracle dequant bit for bit (fp32 bytes);
GEMV relmax < 1e-3 against float64 x . dequant(W)^T (BASELINE tolerance,
tighter than the reference's 3e-3 gate, tests/test_gw_kernel.py:29), and
the kernels' own bar, relmax < 1e-5: x is carried as an fp16 hi + lo split
under a power-of-two scale (about 22 bits, no fp16 range limit), the
codes exactly and the weights of the matrix-core batches as fp16 hi + lo,
so the result is the fp32 GEMV of the reference's k3 / k3nb kernels
(quant_linear_gw.py:520-546, 658-744) up to fp32 summation order.  Fused
r/k/v == three separate launches bit for bit; each row's result is
independent of the rest of the batch, bit for bit."""
import numpy as np
import pytest
import torch

from oracle import codec_ref as cr
from rwkv_quant.backends.hip import _lib
from rwkv_quant.backends.hip.quant_linear import (
    GwQuantLinear, GwQuantLinearFused, QuantLinearV2, SymQuantLinear,
    SymQuantLinearFused)

from _util import act, qt_for, relmax, weights

pytestmark = pytest.mark.gpu

LIN = {"sb6": GwQuantLinear, "sym": SymQuantLinear, "rtn": QuantLinearV2}
FORMATS = [("sb6", 4), ("sb6", 5), ("sb6", 6), ("sym", 6), ("sym", 8),
           ("rtn", 8)]


def _assert_same_bits(dev, ref):
    a = np.ascontiguousarray(dev, np.float32).view(np.uint32)
    b = np.ascontiguousarray(ref, np.float32).view(np.uint32)
    bad = int((a != b).sum())
    assert a.shape == b.shape and bad == 0, f"{bad} of {a.size} differ"


def _w(rows, cols, seed, degenerate=False, outliers=0):
    w = weights(rows, cols, seed=seed, outlier_cols=outliers)
    if degenerate:
        w[3] = 0.0
        w[5] = 1e-9
        w[6, :256] = 0.0
    return w


@pytest.mark.parametrize("kind,bits", FORMATS)
@pytest.mark.parametrize("shape", [(64, 512), (40, 2560)])
def test_dequant_bit_exact(kind, bits, shape):
    print(f"dequant {kind}@{bits} {shape}", flush=True)
    w = _w(*shape, seed=11, degenerate=True, outliers=3)
    qt = qt_for(kind, bits, w)
    lin = LIN[kind](qt)
    dev = lin._dequant_w(torch.float32).cpu().numpy()
    ref = cr.dequant_qt(qt)
    _assert_same_bits(dev, ref)


@pytest.mark.parametrize("kind,bits", FORMATS)
def test_dequant_f16_is_one_rounding_of_f32(kind, bits):
    w = _w(72, 2560, seed=13, degenerate=True, outliers=3)
    lin = LIN[kind](qt_for(kind, bits, w))
    w32 = lin._dequant_w(torch.float32)
    w16 = lin._dequant_w(torch.float16)
    assert torch.equal(w16, w32.half())


def test_dequant_asym_bit_exact():
    w = weights(96, 2048, seed=5)
    qt = qt_for("asym", 6, w)
    out = torch.empty(96, 2048, device="cuda")
    codes = qt.codes.cuda()
    sc, mn = qt.gw_scale.cuda(), qt.gw_min.cuda()
    _lib.call("rwkvq_dequant_asym_f32", _lib.ptr(codes), _lib.ptr(sc),
              _lib.ptr(mn), 64, 96, 2048, _lib.ptr(out), 2048,
              _lib.stream_handle())
    ref = cr.dequant_qt(qt)
    _assert_same_bits(out.cpu().numpy(), ref)


@pytest.mark.parametrize("kind,bits", FORMATS)
@pytest.mark.parametrize("shape", [(2048, 2048), (8192, 2048), (2048, 8192),
                                   (512, 2560), (256, 10240), (96, 6144)])
@pytest.mark.parametrize("n", [1, 2, 3, 8, 20, 40])
def test_gemv_relmax(kind, bits, shape, n):
    print(f"gemv {kind}@{bits} {shape} n={n}", flush=True)
    w = _w(*shape, seed=shape[0] + bits, outliers=2)
    qt = qt_for(kind, bits, w)
    lin = LIN[kind](qt)
    x = act(n, shape[1], seed=n)
    y = lin(x.cuda()).cpu().numpy()
    ref = cr.gemv_ref(x.numpy(), cr.dequant_qt(qt))
    assert relmax(y, ref) < 1e-3
    # degenerate-reference control: the check must be able to fail
    assert relmax(y, ref * 1.01) > 1e-3
    assert relmax(y, ref) < 1e-5


@pytest.mark.parametrize("kind,bits", FORMATS)
@pytest.mark.parametrize("shape", [(20480, 2048), (4096, 10240)])
@pytest.mark.parametrize("n", [1, 2])
def test_gemv_relmax_interleaved_rows(kind, bits, shape, n):
    """Beyond 16384 row-slices the lane-dot kernel takes the interleaved
    row order (a wave's row batches one grid-stride apart), with one K
    slice per wave (20480 rows) and five (K = 10240)."""
    test_gemv_relmax(kind, bits, shape, n)


@pytest.mark.parametrize("kind,bits", FORMATS)
@pytest.mark.parametrize("n", [1, 2, 8, 20])
@pytest.mark.parametrize("scale", [1.0, 1e-4, 1e5])
def test_gemv_full_mantissa_and_range(kind, bits, n, scale):
    """fp32 x with full mantissas (not bf16-valued), tiny and large
    magnitudes (|x| up to ~5e5, beyond fp16's 65504, as relu^2 outputs can
    be), a few exact zeros and a heavy-tailed row: relmax < 1e-5 against
    the float64 oracle in both the lane-dot (1-2 rows) and the matrix-core
    (3+ rows) kernel."""
    print(f"gemv precision {kind}@{bits} n={n} scale={scale}", flush=True)
    w = _w(2048, 2048, seed=bits + 7, outliers=2)
    qt = qt_for(kind, bits, w)
    lin = LIN[kind](qt)
    g = torch.Generator().manual_seed(n)
    x = torch.randn(n, 2048, generator=g) * scale
    x[0, :5] = 0.0
    x[-1] *= torch.exp(torch.randn(2048, generator=g) * 2)   # heavy tails
    y = lin(x.cuda()).cpu().numpy()
    ref = cr.gemv_ref(x.numpy(), cr.dequant_qt(qt))
    assert np.isfinite(y).all()
    assert relmax(y, ref) < 1e-5


@pytest.mark.parametrize("kind,bits", FORMATS)
@pytest.mark.parametrize("n", [1, 2])
def test_gemv_nonfinite_x_gives_nan(kind, bits, n):
    """A NaN or inf in x makes the outputs it reaches NaN or inf, as in the
    fp32 product, instead of a finite number (the int8 formats carry x as
    integer digits, whose group scale then turns NaN)."""
    lin = LIN[kind](qt_for(kind, bits, _w(256, 2048, seed=41)))
    x = act(n, 2048, seed=42)
    x[0, 100] = float("nan")
    if n > 1:
        x[1, 1000] = float("inf")
    y = lin(x.cuda()).cpu().numpy()
    assert not np.isfinite(y[0]).any()
    if n > 1:
        assert not np.isfinite(y[1]).any()


@pytest.mark.parametrize("kind,bits", [("sb6", 5), ("sym", 6), ("rtn", 8)])
def test_batched_rows_independent_of_batch(kind, bits):
    """A row's output is the same bits whatever else is in the batch and
    wherever it sits in it, for batches of one kernel class: 3-16 rows
    (one 16-row block, K split across workgroups) and 17-32 rows (two
    blocks per pass); between the classes the K partition of the fp32 sum
    differs (within 1e-6)."""
    lin = LIN[kind](qt_for(kind, bits, _w(2048, 2048, seed=31)))
    x = act(32, 2048, seed=32).cuda()
    y16 = lin(x[:16].contiguous())
    y5 = lin(x[[13, 3, 9, 0, 12]].contiguous())
    assert torch.equal(y5, y16[[13, 3, 9, 0, 12]])
    y32 = lin(x)
    y20 = lin(x[[17, 3, 9, 0, 12, 30, 21, 5, 1, 2, 4, 6, 7, 8, 10, 11, 14,
                 15, 16, 31]].contiguous())
    assert torch.equal(y20[:6], y32[[17, 3, 9, 0, 12, 30]])
    assert float((y32[:16] - y16).abs().max()) <= 1e-6 * float(
        y16.abs().max())


@pytest.mark.parametrize("kind,bits", [("sb6", 5), ("sym", 8), ("sb6", 4)])
def test_fused_rkv_equals_separate(kind, bits):
    lins = [LIN[kind](qt_for(kind, bits, _w(2048, 2048, seed=s)))
            for s in range(3)]
    fused = (GwQuantLinearFused if kind == "sb6" else SymQuantLinearFused)(lins)
    x = act(3, 2048, seed=7).cuda()
    yf = fused(x)
    ys = torch.stack([lins[i](x[i:i + 1])[0] for i in range(3)])
    assert torch.equal(yf, ys)


@pytest.mark.parametrize("mode", [_lib.EPI_ADD, _lib.EPI_RELU2, _lib.EPI_TANH,
                                  _lib.EPI_SIGMOID])
def test_gemv_epilogues(mode):
    lin = GwQuantLinear(qt_for("sb6", 4, _w(1024, 2048, seed=3)))
    x = act(2, 2048, seed=4).cuda()
    base = torch.empty(2, 1024, device="cuda")
    lin.gemv_into(x, base)
    y0 = torch.randn(2, 1024, device="cuda")
    y = y0.clone()
    lin.gemv_into(x, y, mode=mode)
    expect = {_lib.EPI_ADD: y0 + base, _lib.EPI_RELU2: torch.relu(base) ** 2,
              _lib.EPI_TANH: torch.tanh(base),
              _lib.EPI_SIGMOID: torch.sigmoid(base)}[mode]
    assert torch.allclose(y, expect, rtol=1e-5, atol=1e-6)


def test_shape_errors_raise():
    lin = GwQuantLinear(qt_for("sb6", 4, _w(64, 512, seed=1)))
    with pytest.raises(_lib.HipKernelError):
        _lib.call("rwkvq_gemv_sb6", _lib.ptr(lin.nib), None,
                  _lib.ptr(lin.rec), 4, 64, 500, 64, None, 0, None, 1, 0,
                  _lib.stream_handle())


@pytest.mark.parametrize("kind,bits", [("sb6", 4), ("sb6", 5), ("sb6", 6),
                                       ("sym", 6), ("sym", 8), ("rtn", 8)])
@pytest.mark.parametrize("n_idx", [1, 8, 37])
def test_gather_rows_bit_exact(kind, bits, n_idx):
    """The embedding gather (rwkvq_gather_rows_f32) == rows of the oracle
    dequant bit for bit, indices clamped into the table."""
    print(f"gather {kind}@{bits} n_idx {n_idx}", flush=True)
    w = _w(40, 2560, seed=17, degenerate=True, outliers=3)
    qt = qt_for(kind, bits, w)
    lin = LIN[kind](qt)
    if kind == "sb6":
        args = (0, bits, lin.nib, lin.hb, lin.rec, None)
    elif kind == "sym":
        args = (1, bits, lin.codes, lin.hb, lin.qs, lin.d)
    else:
        args = (2, 8, lin.codes, None, None, lin.scale)
    rng = np.random.default_rng(n_idx)
    ids = rng.integers(0, 40, size=n_idx)
    ids[0] = 39
    if n_idx > 2:
        ids[1], ids[2] = -5, 1000          # clamped to 0 and 39
    idx = torch.from_numpy(ids.astype(np.int64)).cuda()
    out = torch.full((n_idx, 2560), float("nan"), device="cuda")
    _lib.call("rwkvq_gather_rows_f32", args[0], args[1],
              *[_lib.ptr(t) for t in args[2:]], 40, 2560,
              _lib.ptr(idx), n_idx, _lib.ptr(out), _lib.stream_handle())
    ref = cr.dequant_qt(qt)[np.clip(ids, 0, 39)]
    _assert_same_bits(out.cpu().numpy(), ref)


@pytest.mark.parametrize("kind,bits", [("sb6", 4), ("sb6", 5), ("sb6", 6),
                                       ("sym", 6), ("sym", 8), ("rtn", 8)])
@pytest.mark.parametrize("n_idx", [1, 37])
def test_gather_ln_equals_gather_then_layer_norm(kind, bits, n_idx):
    """rwkvq_gather_ln_f32 (the embedding gather fused with ln0) ==
    rwkvq_gather_rows_f32 followed by rwkvq_layer_norm, bit for bit."""
    print(f"gather+ln {kind}@{bits} n_idx {n_idx}", flush=True)
    D = 2560
    w = _w(40, D, seed=19, outliers=3)
    qt = qt_for(kind, bits, w)
    lin = LIN[kind](qt)
    if kind == "sb6":
        args = (0, bits, lin.nib, lin.hb, lin.rec, None)
    elif kind == "sym":
        args = (1, bits, lin.codes, lin.hb, lin.qs, lin.d)
    else:
        args = (2, 8, lin.codes, None, None, lin.scale)
    g = torch.Generator().manual_seed(n_idx)
    lw = (1 + 0.1 * torch.randn(D, generator=g)).cuda()
    lb = (0.1 * torch.randn(D, generator=g)).cuda()
    ids = np.random.default_rng(n_idx).integers(-2, 45, size=n_idx)
    idx = torch.from_numpy(ids.astype(np.int64)).cuda()
    ptrs = [_lib.ptr(t) for t in args[2:]]
    ref = torch.empty(n_idx, D, device="cuda")
    _lib.call("rwkvq_gather_rows_f32", args[0], args[1], *ptrs, 40, D,
              _lib.ptr(idx), n_idx, _lib.ptr(ref), _lib.stream_handle())
    _lib.call("rwkvq_layer_norm", _lib.ptr(ref), _lib.ptr(lw), _lib.ptr(lb),
              _lib.ptr(ref), n_idx, D, 1e-5, _lib.stream_handle())
    out = torch.full((n_idx, D), float("nan"), device="cuda")
    _lib.call("rwkvq_gather_ln_f32", args[0], args[1], *ptrs, 40, D,
              _lib.ptr(idx), n_idx, _lib.ptr(lw), _lib.ptr(lb), 1e-5,
              _lib.ptr(out), _lib.stream_handle())
    assert torch.equal(out, ref)
