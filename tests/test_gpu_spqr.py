"""SpQR outliers of the per-row int8 format on the GPU (reference:
quant_linear_v2.py:35-84, the CSR loop inside the int8 GEMV): the GEMV
with the outlier tail summed in-kernel (1-2 rows), the matrix-core rows
and the prefill GEMM followed by rwkvq_spqr_apply, against the float64
oracle of codes * scale + outliers; the dense dequant with the outlier
overwrite bit for bit."""
import numpy as np
import pytest
import torch

from oracle import codec_ref as cr
from rwkv_quant.backends.hip import _lib
from rwkv_quant.backends.hip.quant_linear import QuantLinearV2
from rwkv_quant.formats import writer

from _util import act, relmax, weights

pytestmark = pytest.mark.gpu


def _spqr(rows, cols, seed, frac=0.01):
    w = weights(rows, cols, seed=seed, outlier_cols=3)
    c, s, oi, ov = writer.rtn_quantize_outliers(w, 8, frac)
    return writer.make_rtn("t", "head", 8, w.shape, c, s, oi, ov)


@pytest.mark.parametrize("shape", [(2048, 2048), (8192, 2048), (2048, 8192),
                                   (65536, 2048)])
@pytest.mark.parametrize("n", [1, 2, 8])
def test_spqr_gemv_matches_oracle(shape, n):
    print(f"spqr gemv {shape} n={n}", flush=True)
    qt = _spqr(*shape, seed=shape[0] % 997 + n)
    lin = QuantLinearV2(qt)
    assert lin.has_outliers
    x = act(n, shape[1], seed=n)
    y = lin(x.cuda()).cpu().numpy()
    W = cr.dequant_qt(qt)
    ref = cr.gemv_ref(x.numpy(), W)
    assert relmax(y, ref) < 1e-5
    # without the outliers the result is clearly off: the tail is pinned
    W0 = W.copy()
    oi = qt.outlier_indices.long().numpy()
    W0[oi[:, 0], oi[:, 1]] = 0.0
    assert relmax(y, cr.gemv_ref(x.numpy(), W0)) > 1e-3


@pytest.mark.parametrize("mode", [_lib.EPI_STORE, _lib.EPI_ADD,
                                  _lib.EPI_RELU2, _lib.EPI_SIGMOID])
@pytest.mark.parametrize("n", [1, 5, 200])
def test_spqr_epilogues(mode, n):
    qt = _spqr(1024, 2048, seed=7)
    lin = QuantLinearV2(qt)
    x = act(n, 2048, seed=3)
    y0 = torch.randn(n, 1024, generator=torch.Generator().manual_seed(4))
    y = y0.clone().cuda()
    lin.apply_into(x.cuda(), y, mode=mode)
    acc = cr.gemv_ref(x.numpy(), cr.dequant_qt(qt))
    ref = {_lib.EPI_STORE: acc, _lib.EPI_ADD: acc + y0.double().numpy(),
           _lib.EPI_RELU2: np.maximum(acc, 0) ** 2,
           _lib.EPI_SIGMOID: 1 / (1 + np.exp(-acc))}[mode]
    # 200 rows run the fp16-operand GEMM for the int8 part
    assert relmax(y.cpu().numpy(), ref) < (1e-3 if n >= 128 else 1e-5)


def test_spqr_dequant_bit_exact():
    qt = _spqr(512, 2048, seed=9)
    w = QuantLinearV2(qt)._dequant_w(torch.float32).cpu().numpy()
    ref = cr.dequant_qt(qt)
    assert np.array_equal(w.view(np.uint32), ref.view(np.uint32))
