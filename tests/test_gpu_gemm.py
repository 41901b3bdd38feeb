"""GPU parity of the MFMA prefill GEMM (dequantization fused into the
operand load) against the CPU oracle.

Bars: relmax < 1e-3 against float64 x . dequant(W)^T (BASELINE tolerance
for GEMV/GEMM; the reference gated its prefill GEMM at 2e-3 against fp16
operands, tests/test_gemm_prefill.py:32-49), and relmax < 2e-5 against the
float64 product of the operands the reference's prefill feeds its fp16
matmul (x rounded to fp16, W = the format's fp16 dequant; rtn8: the codes,
with the fp32 row scale applied to the sum) -- so the pairing of x and W
along k, the per-group scales and the tile bookkeeping are pinned, not just
the overall magnitude."""
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


def _w(rows, cols, seed, degenerate=False, outliers=2):
    w = weights(rows, cols, seed=seed, outlier_cols=outliers)
    if degenerate:
        w[3] = 0.0
        w[5] = 1e-9
        w[6, :256] = 0.0
    return w


def _gemm(lin, x, mode=_lib.EPI_STORE, y=None):
    M = x.shape[0]
    if y is None:
        y = torch.empty(M, lin.out_features, device="cuda")
    lin._run("gemm", x, y, mode=mode, n=M)
    return y


def _operand_ref(kind, lin, qt, x):
    """float64 product of the fp16 operands of the reference's prefill."""
    x16 = x.half().double().numpy()
    if kind == "rtn":
        q = qt.codes.double().numpy()
        s = qt.scale.float().double().numpy().reshape(1, -1)
        return (x16 @ q.T) * s
    w16 = lin._dequant_w(torch.float16).cpu().double().numpy()
    return x16 @ w16.T


@pytest.mark.parametrize("kind,bits", FORMATS)
@pytest.mark.parametrize("shape", [(2048, 2048), (8192, 2048), (2048, 8192),
                                   (384, 2560)])
@pytest.mark.parametrize("M", [128, 200, 512])
def test_gemm_relmax(kind, bits, shape, M):
    print(f"gemm {kind}@{bits} {shape} M={M}", flush=True)
    w = _w(*shape, seed=shape[0] + bits, degenerate=(M == 200))
    qt = qt_for(kind, bits, w)
    lin = LIN[kind](qt)
    x = act(M, shape[1], seed=M)
    y = _gemm(lin, x.cuda()).cpu().numpy()
    ref = cr.gemv_ref(x.numpy(), cr.dequant_qt(qt))
    assert relmax(y, ref) < 1e-3
    assert relmax(y, ref * 1.01) > 1e-3      # the check can fail
    assert relmax(y, _operand_ref(kind, lin, qt, x)) < 2e-5


@pytest.mark.parametrize("kind,bits", [("sb6", 5), ("sym", 6), ("rtn", 8)])
@pytest.mark.parametrize("mode", [_lib.EPI_ADD, _lib.EPI_RELU2, _lib.EPI_TANH,
                                  _lib.EPI_SIGMOID])
def test_gemm_epilogues(kind, bits, mode):
    lin = LIN[kind](qt_for(kind, bits, _w(1024, 2048, seed=3)))
    x = act(160, 2048, seed=4).cuda()
    base = _gemm(lin, x)
    y0 = torch.randn(160, 1024, device="cuda")
    y = _gemm(lin, x, mode=mode, y=y0.clone())
    expect = {_lib.EPI_ADD: y0 + base, _lib.EPI_RELU2: torch.relu(base) ** 2,
              _lib.EPI_TANH: torch.tanh(base),
              _lib.EPI_SIGMOID: torch.sigmoid(base)}[mode]
    assert torch.allclose(y, expect, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("kind,bits", [("sb6", 5), ("sym", 8), ("sb6", 4)])
def test_gemm_fused_rkv_equals_separate(kind, bits):
    """Three matrices on three input segments of a strided x (the model's
    [T, 6, C] lerp buffer) in one launch == three launches (to 1e-5: the
    launches may split K differently, which reorders the fp32 sums)."""
    lins = [LIN[kind](qt_for(kind, bits, _w(2048, 2048, seed=s)))
            for s in range(3)]
    fused = (GwQuantLinearFused if kind == "sb6" else SymQuantLinearFused)(lins)
    T = 192
    xs = act(T * 6, 2048, seed=9).reshape(T, 6, 2048).cuda()
    y = torch.empty(T, 3 * 2048, device="cuda")
    fused.apply_into(xs, y, T, 6 * 2048)
    for j, lin in enumerate(lins):
        yj = _gemm(lin, xs[:, j].contiguous())
        assert torch.allclose(y[:, j * 2048:(j + 1) * 2048], yj, rtol=1e-5,
                              atol=1e-5)


def test_linear_call_takes_gemm_from_128_rows():
    """__call__ switches to the GEMM at GEMM_MIN_BATCH_NB rows; both paths
    agree with the oracle."""
    qt = qt_for("sym", 6, _w(2048, 2048, seed=21))
    lin = SymQuantLinear(qt)
    ref_w = cr.dequant_qt(qt)
    for M in (127, 128):
        x = act(M, 2048, seed=M)
        y = lin(x.cuda()).cpu().numpy()
        assert relmax(y, cr.gemv_ref(x.numpy(), ref_w)) < 1e-3


def test_gemm_shape_errors_raise():
    lin = GwQuantLinear(qt_for("sb6", 4, _w(192, 512, seed=1)))
    x = torch.zeros(128, 512, device="cuda")
    y = torch.empty(128, 192, device="cuda")
    with pytest.raises(_lib.HipKernelError):       # 192 rows: not 128-tiled
        lin._run("gemm", x, y, n=128)
    with pytest.raises(_lib.HipKernelError):       # IN not a multiple of 256
        _lib.call("rwkvq_gemm_sb6", _lib.ptr(lin.nib), None,
                  _lib.ptr(lin.rec), 4, 128, 500, 128, _lib.ptr(x), 0,
                  _lib.ptr(y), 128, 0, _lib.stream_handle())


@pytest.mark.parametrize("M", [24, 200, 512])
def test_gemm_f16_dense(M):
    """Dense fp16 rows (the prefill LoRA factors): against the float64
    product of the fp16-rounded operands."""
    g = torch.Generator().manual_seed(M)
    W = (torch.randn(384, 2048, generator=g) * 0.02).half()
    x = torch.randn(M, 2048, generator=g)
    y = torch.empty(M, 384, device="cuda")
    Wd, xd = W.cuda(), x.cuda()
    _lib.call("rwkvq_gemm_f16", _lib.ptr(Wd), 384, 2048, 384, _lib.ptr(xd),
              0, _lib.ptr(y), M, _lib.EPI_STORE, 0, _lib.stream_handle())
    ref = x.half().double().numpy() @ W.double().numpy().T
    assert relmax(y.cpu().numpy(), ref) < 2e-5


def test_gemm_f16_per_segment_epilogue():
    """Three segments of 128 rows on three input slices, modes tanh / store
    / sigmoid (the LoRA down products of one layer in one launch)."""
    g = torch.Generator().manual_seed(5)
    M, K, R = 160, 256, 128
    W = (torch.randn(3 * R, K, generator=g) * 0.1).half().cuda()
    xs = torch.randn(M, 6, K, generator=g).cuda()
    y = torch.empty(M, 3 * R, device="cuda")
    modes = _lib.EPI_TANH | (_lib.EPI_STORE << 4) | (_lib.EPI_SIGMOID << 8)
    _lib.call("rwkvq_gemm_f16", _lib.ptr(W), 3 * R, K, R,
              _lib.ptr(xs[:, 2]), 6 * K, _lib.ptr(y), M, _lib.EPI_PER_SEG,
              modes, _lib.stream_handle())
    for j, f in enumerate((torch.tanh, lambda v: v, torch.sigmoid)):
        ref = f(xs[:, 2 + j].half().float() @ W[j * R:(j + 1) * R].float().t())
        assert torch.allclose(y[:, j * R:(j + 1) * R], ref, rtol=1e-4,
                              atol=1e-5)


@pytest.mark.parametrize("n", [1, 3, 8, 16, 17, 32])
@pytest.mark.parametrize("ranks", [(64, 96, 96, 256), (96, 96, 256)])
def test_gemv_f16_segments(n, ranks):
    """The decode LoRA down products in one launch: segment j of the
    stacked fp16 factors reads input slot j and writes its own output with
    its own epilogue; against the float64 product of the fp16 factors and
    the fp32 x (x is carried as an fp16 hi + lo split)."""
    g = torch.Generator().manual_seed(n + len(ranks))
    K = 2048
    A = [(torch.randn(r, K, generator=g) * 0.05).half() for r in ranks]
    xs = torch.randn(n, 6, K, generator=g)
    modes = [_lib.EPI_STORE, _lib.EPI_TANH, _lib.EPI_STORE, _lib.EPI_SIGMOID]
    modes = modes[-len(ranks):]
    fns = {_lib.EPI_STORE: lambda v: v, _lib.EPI_TANH: np.tanh,
           _lib.EPI_SIGMOID: lambda v: 1 / (1 + np.exp(-v))}
    Ad = torch.cat(A).cuda()
    xd = xs.cuda()
    ys = [torch.empty(n, r, device="cuda") for r in ranks]
    import ctypes
    rows = (ctypes.c_int * len(ranks))(*ranks)
    yp = (ctypes.c_void_p * len(ranks))(*[y.data_ptr() for y in ys])
    sm = sum(m << (4 * j) for j, m in enumerate(modes))
    s0 = 6 - len(ranks)
    _lib.call("rwkvq_gemv_f16_seg", _lib.ptr(Ad), len(ranks), rows, K,
              _lib.ptr(xd[:, s0]), 6 * K, yp, n, sm, _lib.stream_handle())
    for j, (Aj, m) in enumerate(zip(A, modes)):
        ref = fns[m](xs[:, s0 + j].double().numpy()
                     @ Aj.double().numpy().T)
        assert relmax(ys[j].cpu().numpy(), ref) < 1e-5, j


def test_gemv_f16_segments_errors():
    A = torch.zeros(96, 2048, dtype=torch.float16, device="cuda")
    x = torch.zeros(33, 2048, device="cuda")
    y = torch.empty(33, 96, device="cuda")
    import ctypes
    yp = (ctypes.c_void_p * 1)(y.data_ptr())
    for rows, n in ((90, 4), (96, 33), (96, 0)):
        r = (ctypes.c_int * 1)(rows)
        with pytest.raises(_lib.HipKernelError):
            _lib.call("rwkvq_gemv_f16_seg", _lib.ptr(A), 1, r, 2048,
                      _lib.ptr(x), 2048, yp, n, 0, _lib.stream_handle())


@pytest.mark.parametrize("M", [160, 512])
def test_gemm_f16_segment_table(M):
    """The prefill LoRA down products in one launch over segments of
    unequal height (each a multiple of 128): segment j reads input slot j
    and has its own epilogue; equal to one launch per segment (to 1e-5: the
    launches may split K differently), and within 2e-5 of the float64
    product of the fp16 operands."""
    import ctypes
    g = torch.Generator().manual_seed(M)
    K, rows = 2048, [128, 128, 128, 384]
    A = [(torch.randn(r, K, generator=g) * 0.05).half() for r in rows]
    xs = torch.randn(M, 6, K, generator=g)
    modes = [_lib.EPI_STORE, _lib.EPI_TANH, _lib.EPI_STORE, _lib.EPI_SIGMOID]
    Ad, xd = torch.cat(A).cuda(), xs.cuda()
    y = torch.empty(M, sum(rows), device="cuda")
    sm = sum(m << (4 * j) for j, m in enumerate(modes))
    _lib.call("rwkvq_gemm_f16_seg", _lib.ptr(Ad), 4,
              (ctypes.c_int * 4)(*rows), K, _lib.ptr(xd[:, 2]), 6 * K,
              _lib.ptr(y), M, sm, 0, _lib.stream_handle())
    fns = {_lib.EPI_STORE: lambda v: v, _lib.EPI_TANH: np.tanh,
           _lib.EPI_SIGMOID: lambda v: 1 / (1 + np.exp(-v))}
    off = 0
    for j, (Aj, m) in enumerate(zip(A, modes)):
        yj = torch.empty(M, rows[j], device="cuda")
        Ajd = Aj.cuda()        # (held: the launch is asynchronous)
        _lib.call("rwkvq_gemm_f16", _lib.ptr(Ajd), rows[j], K, rows[j],
                  _lib.ptr(xd[:, 2 + j]), 6 * K, _lib.ptr(yj), M, m, 0,
                  _lib.stream_handle())
        assert torch.allclose(y[:, off:off + rows[j]], yj, rtol=1e-5,
                              atol=1e-5), j
        ref = fns[m](xs[:, 2 + j].half().double().numpy()
                     @ Aj.double().numpy().T)
        assert relmax(y[:, off:off + rows[j]].cpu().numpy(), ref) < 2e-5
        off += rows[j]
    with pytest.raises(_lib.HipKernelError):      # a segment off the tiles
        _lib.call("rwkvq_gemm_f16_seg", _lib.ptr(Ad), 2,
                  (ctypes.c_int * 2)(100, 668), K, _lib.ptr(xd[:, 2]),
                  6 * K, _lib.ptr(y), M, 0, 0, _lib.stream_handle())


def _set_split(on):
    """Register (on) or drop (off) the split-K workspace of this device."""
    _lib.ensure_gemm_workspace()
    ws, cnt = _lib._gemm_ws[torch.cuda.current_device()]
    args = ((_lib.ptr(ws), _lib.GEMM_WS_BYTES, _lib.ptr(cnt),
             _lib.GEMM_WS_COUNTERS) if on else (None, 0, None, 0))
    assert _lib.load().rwkvq_gemm_workspace(*args) == 0


@pytest.mark.parametrize("kind,bits,shape", [("sym", 6, (2048, 8192)),
                                             ("sym", 8, (2048, 2048)),
                                             ("sb6", 5, (1024, 2048))])
@pytest.mark.parametrize("mode", [_lib.EPI_STORE, _lib.EPI_ADD,
                                  _lib.EPI_RELU2, _lib.EPI_SIGMOID])
def test_gemm_split_k(kind, bits, shape, mode):
    """Output tiles shared by several K runs (the last run to finish adds
    the partials in run order and applies the epilogue): equal, bit for
    bit, from launch to launch, and to 1e-5 of the unsplit launch."""
    print(f"split-K {kind}@{bits} {shape} mode {mode}", flush=True)
    lin = LIN[kind](qt_for(kind, bits, _w(*shape, seed=5)))
    x = act(512, shape[1], seed=6).cuda()
    y0 = torch.randn(512, shape[0], device="cuda")
    try:
        _set_split(False)
        ref = _gemm(lin, x, mode=mode, y=y0.clone())
        _set_split(True)
        outs = [_gemm(lin, x, mode=mode, y=y0.clone()) for _ in range(3)]
    finally:
        _set_split(True)
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    assert torch.allclose(outs[0], ref, rtol=1e-5, atol=1e-5)
    _, cnt = _lib._gemm_ws[torch.cuda.current_device()]
    assert int(cnt.abs().sum()) == 0             # counters re-armed


def _pair_cols(order):
    """Source column of each fp16 position within a 32-column group."""
    c = []
    for i in range(16):
        if order == _lib.ORDER_SB6:
            c += [i, i + 16]
        elif order == _lib.ORDER_SYM6:
            c0 = i if i < 8 else i + 8
            c += [c0, c0 + 8]
        else:
            c += [2 * i, 2 * i + 1]
    return np.array(c)


def _order_of(kind, bits):
    if kind == "sb6":
        return _lib.ORDER_SB6
    return _lib.ORDER_SYM6 if (kind, bits) == ("sym", 6) else _lib.ORDER_PAIRS


def _to_x16(x, order, cols=None):
    M, C = x.shape[0], cols or x.shape[1]
    xh = torch.empty(M, C, dtype=torch.float16, device="cuda")
    _lib.call("rwkvq_x16", _lib.ptr(x), x.stride(0), C, M, order,
              _lib.ptr(xh), C, _lib.stream_handle())
    return xh


@pytest.mark.parametrize("order", [0, 1, 2])
def test_x16_pair_order(order):
    """fp32 -> fp16 (nearest even) with each 32-column group permuted into
    the pair order of the formats' decoders."""
    x = act(5, 256, seed=order).cuda()
    xh = _to_x16(x, order).cpu().numpy().reshape(5, 8, 32)
    src = x.half().cpu().numpy().reshape(5, 8, 32)
    assert np.array_equal(xh, src[:, :, _pair_cols(order)])


@pytest.mark.parametrize("kind,bits", FORMATS)
@pytest.mark.parametrize("M", [37, 512])
def test_gemm_x16_input_equals_fp32_input(kind, bits, M):
    """The GEMM fed fp16 x in the format's pair order (RWKVQ_X_F16) gives the
    bits of the same GEMM fed fp32 x (which rounds x to fp16 itself)."""
    print(f"x16 gemm {kind}@{bits} M={M}", flush=True)
    lin = LIN[kind](qt_for(kind, bits, _w(2048, 2048, seed=11)))
    x = act(M, 2048, seed=12).cuda()
    ref = _gemm(lin, x)
    xh = _to_x16(x, _order_of(kind, bits))
    y = torch.empty_like(ref)
    lin._run("gemm", xh, y, mode=_lib.X_F16, n=M)
    assert torch.equal(y, ref)


@pytest.mark.parametrize("M", [37, 512])
@pytest.mark.parametrize("x16", [False, True])
def test_gemm_f16_grouped(M, x16):
    """Independent fp16 GEMMs of different K (the prefill LoRA up products,
    ranks padded to 128 / 384) in one launch, each with its own x, y and
    epilogue: within 2e-5 of the float64 product of the fp16 operands."""
    import ctypes
    g = torch.Generator().manual_seed(M + x16)
    ks, rows = [128, 384, 128, 256], [256, 256, 128, 384]
    modes = [_lib.EPI_STORE, _lib.EPI_TANH, _lib.EPI_SIGMOID, _lib.EPI_STORE]
    W = [(torch.randn(r, k, generator=g) * 0.05).half() for r, k in
         zip(rows, ks)]
    xs = [torch.randn(M, k + 32, generator=g) for k in ks]   # x_ld = k + 32
    Wd = [w.cuda() for w in W]
    xd = [(x.half() if x16 else x).cuda() for x in xs]
    ys = [torch.empty(M, r, device="cuda") for r in rows]
    P, n = ctypes.c_void_p, len(ks)
    _lib.call("rwkvq_gemm_f16_grouped", n, (P * n)(*[w.data_ptr() for w in Wd]),
              (ctypes.c_int * n)(*rows), (ctypes.c_int * n)(*ks),
              (P * n)(*[x.data_ptr() for x in xd]),
              (ctypes.c_long * n)(*[k + 32 for k in ks]),
              (P * n)(*[y.data_ptr() for y in ys]), M,
              sum(m << (4 * j) for j, m in enumerate(modes)),
              _lib.X_F16 if x16 else 0, _lib.stream_handle())
    fns = {_lib.EPI_STORE: lambda v: v, _lib.EPI_TANH: np.tanh,
           _lib.EPI_SIGMOID: lambda v: 1 / (1 + np.exp(-v))}
    for j in range(n):
        ref = fns[modes[j]](xs[j][:, :ks[j]].half().double().numpy()
                            @ W[j].double().numpy().T)
        assert relmax(ys[j].cpu().numpy(), ref) < 2e-5, j


def test_gemm_f16_small_output_split():
    """Few output tiles (the LoRA down products at pp512: 640 rows, K 2048)
    take 128 x 64 tiles split along K: within 2e-5 of float64."""
    g = torch.Generator().manual_seed(9)
    A = (torch.randn(640, 2048, generator=g) * 0.05).half()
    x = torch.randn(512, 2048, generator=g)
    y = torch.empty(512, 640, device="cuda")
    Ad, xd = A.cuda(), x.cuda()   # (held: the launch is asynchronous)
    _lib.call("rwkvq_gemm_f16", _lib.ptr(Ad), 640, 2048, 640, _lib.ptr(xd),
              0, _lib.ptr(y), 512, _lib.EPI_STORE, 0, _lib.stream_handle())
    ref = x.half().double().numpy() @ A.double().numpy().T
    assert relmax(y.cpu().numpy(), ref) < 2e-5


@pytest.mark.parametrize("kind,bits", [("sym", 8), ("sb6", 5), ("sym", 6)])
def test_gemm_dual_equals_two_launches(kind, bits):
    """The prefill r/k/v projection and the LoRA down products in one launch
    (rwkvq_gemm_dual_f16seg) == the two GEMMs launched on their own: the
    quantized one bit for bit (same tiles), the fp16 one to 1e-5 (its own
    launch may split K)."""
    import ctypes
    from rwkv_quant.backends.hip.quant_linear import (GwQuantLinearFused,
                                                       SymQuantLinearFused)
    T, C = 512, 2048
    lins = [LIN[kind](qt_for(kind, bits, _w(C, C, seed=40 + s)))
            for s in range(3)]
    fused = (GwQuantLinearFused if kind == "sb6" else SymQuantLinearFused)(lins)
    order = _order_of(kind, bits)
    g = torch.Generator().manual_seed(41)
    xs = torch.randn(T, 6, C, generator=g).cuda()
    xs16 = _to_x16(xs.view(T * 6, C), order).view(T, 6, C)
    rows = [128, 128, 128, 256]
    A = (torch.randn(sum(rows), C, generator=g) * 0.05).half().cuda()
    modes = sum(m << (4 * j) for j, m in enumerate(
        [_lib.EPI_STORE, _lib.EPI_TANH, _lib.EPI_STORE, _lib.EPI_SIGMOID]))
    fl = _lib.X_F16 | _lib.Y_F16 | (_lib.ORDER_PAIRS << _lib.Y_ORDER_SHIFT)
    ra = (ctypes.c_int * 4)(*rows)
    y1 = torch.empty(T, 3 * C, device="cuda")
    h1 = torch.empty(T, sum(rows), dtype=torch.float16, device="cuda")
    k, lead = fused._cat._kargs()
    if k == "sb6":
        kk, (p0, p1, p2, b_), p3 = 0, lead, None
    else:
        kk, (p0, p1, p2, p3, b_) = 1, lead
    _lib.call("rwkvq_gemm_dual_f16seg", kk, b_, p0, p1, p2, p3, 3 * C, C, C,
              _lib.ptr(xs16), 6 * C, _lib.ptr(y1), _lib.X_F16, _lib.ptr(A),
              4, ra, _lib.ptr(xs16[:, 2]), 6 * C, _lib.ptr(h1), modes, fl, T,
              _lib.stream_handle())
    y2 = torch.empty_like(y1)
    fused.apply_into(xs16, y2, T, 6 * C, mode=_lib.X_F16)
    h2 = torch.empty_like(h1)
    _lib.call("rwkvq_gemm_f16_seg", _lib.ptr(A), 4, ra, C,
              _lib.ptr(xs16[:, 2]), 6 * C, _lib.ptr(h2), T, modes, fl,
              _lib.stream_handle())
    assert torch.equal(y1, y2)
    # fp16 outputs: the two launches' fp32 sums may round to adjacent halves
    assert torch.allclose(h1.float(), h2.float(), rtol=2e-3, atol=2e-3)
