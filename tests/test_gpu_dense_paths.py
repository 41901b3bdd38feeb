"""GPU parity of the linear paths that are neither a packed-format GEMV
nor an MFMA-tile GEMM: unquantized (16-bit) matrices in fp16
(DenseLinear: the fp16 matrix-core GEMV, and the fp16 MFMA GEMM from 128
input rows) and packed matrices whose output rows are off the GEMM's
128-row tiles (the GEMV kernels for every batch size).  Every path is a
librwkvq_hip kernel.

Bars: fp16 GEMV (fp32 x as fp16 hi + lo) relmax < 1e-5 and fp16 GEMM
(x rounded to fp16, as the reference's fp16 matmul) relmax < 1e-3 against
float64 products of the fp16 weights; packed GEMV relmax < 1e-5 against
the oracle dequant; a 16-bit model's logits within 1e-2 max-abs of the
float64 oracle (decode and a 130-token prefill)."""
import numpy as np
import pytest
import torch

from oracle import codec_ref as cr
from oracle.rwkv7_ref import RWKV7Oracle
from rwkv_quant.backends.hip import quant_model as qm
from rwkv_quant.backends.hip.quant_linear import DenseLinear, GwQuantLinear
from rwkv_quant.calibration.group_config import QuantConfig
from rwkv_quant.models.synthetic import quantized_model

from _util import act, qt_for, relmax, weights

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n", [1, 3, 40, 130])
def test_dense_linear_paths(n):
    print(f"dense linear n={n}", flush=True)
    w = (weights(512, 256, seed=3, std=0.05)).to(torch.float16)
    lin = DenseLinear(w)
    x = torch.randn(n, 256, generator=torch.Generator().manual_seed(n))
    y = lin(x.cuda()).cpu().numpy()
    ref = x.numpy().astype(np.float64) @ w.float().numpy().astype(np.float64).T
    assert relmax(y, ref) < (1e-3 if n >= 128 else 1e-5)


def test_dense_linear_rejects_off_tile_width():
    with pytest.raises(NotImplementedError):
        DenseLinear(torch.zeros(512, 200, dtype=torch.float16))


@pytest.mark.parametrize("n", [1, 5, 130])
def test_packed_rows_off_gemm_tiles(n):
    """2064 output rows (not a multiple of 128): every batch size runs the
    GEMV kernels, also from 128 input rows on."""
    print(f"sb6 2064 rows n={n}", flush=True)
    w = weights(2064, 2048, seed=11)
    qt = qt_for("sb6", 5, w)
    lin = GwQuantLinear(qt)
    assert not lin.gemm_ok()
    x = act(n, 2048, seed=n)
    y = lin(x.cuda()).cpu().numpy()
    ref = cr.gemv_ref(x.numpy(), cr.dequant_qt(qt))
    assert relmax(y, ref) < 1e-5


@pytest.fixture(scope="module")
def dense_model():
    ck = quantized_model("compression", n_layer=2, n_embd=256, vocab=512,
                         seed=5, config=QuantConfig(), device="cuda",
                         to_cpu=True)
    model = qm.QuantRWKV7(ck)
    assert isinstance(model.blocks[0].tmix.r_proj, DenseLinear)
    return RWKV7Oracle(ck), model


def test_16bit_model_decode_and_prefill(dense_model):
    orc, model = dense_model
    rng = np.random.default_rng(2)
    idx = rng.integers(0, 512, size=(1, 130))
    ro, st_o = orc.forward_stateful(idx, orc.init_state(1))
    lg, st_m = model.forward_stateful(torch.from_numpy(idx),
                                      model.init_state(1))
    assert float(np.abs(lg.cpu().numpy() - ro).max()) < 1e-2
    for t in range(3):
        nxt = rng.integers(0, 512, size=(1, 1))
        ro, st_o = orc.forward_stateful(nxt, st_o)
        lg, st_m = model.step(torch.from_numpy(nxt), st_m)
        assert float(np.abs(lg.cpu().numpy() - ro).max()) < 1e-2
