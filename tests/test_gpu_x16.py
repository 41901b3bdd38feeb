"""GPU checks of the fp16 prefill operands: the producers that write a
GEMM input directly as fp16 in the consuming format's pair order (the
lerp / token-shift kernel, the time-mix tail, the GEMM epilogue) give
exactly the bits of their fp32 output rounded to fp16 (nearest even) and
permuted by rwkvq_x16 -- which test_gpu_gemm pins against numpy and
against the fp32-input GEMM."""
import numpy as np
import pytest
import torch

from rwkv_quant.backends.hip import _lib
from rwkv_quant.backends.hip.quant_linear import (GwQuantLinear,
                                                   QuantLinearV2,
                                                   SymQuantLinear)

from _util import act, qt_for, weights

pytestmark = pytest.mark.gpu

P = _lib.ptr
ORDERS = [_lib.ORDER_PAIRS, _lib.ORDER_SB6, _lib.ORDER_SYM6]


def _x16(x2, order):
    """rwkvq_x16 of a 2-D fp32 tensor (all columns)."""
    M, C = x2.shape
    out = torch.empty(M, C, dtype=torch.float16, device="cuda")
    _lib.call("rwkvq_x16", P(x2), x2.stride(0), C, M, order, P(out), C,
              _lib.stream_handle())
    return out


@pytest.mark.parametrize("order", ORDERS)
@pytest.mark.parametrize("nc,prev", [(6, True), (1, False), (6, False)])
def test_shift_lerp_f16(order, nc, prev):
    g = torch.Generator().manual_seed(order * 10 + nc)
    B, T, D = 2, 9, 2048
    x = torch.randn(B, T, D, generator=g).cuda()
    lw, lb = (torch.randn(D, generator=g).cuda() for _ in range(2))
    pr = torch.randn(B, D, generator=g).cuda() if prev else None
    coef = torch.rand(nc, D, generator=g).cuda()
    s = _lib.stream_handle()
    ref = torch.empty(B * T, nc, D, device="cuda")
    np32, np16 = (torch.empty(B, D, device="cuda") for _ in range(2))
    _lib.call("rwkvq_shift_lerp", P(x), P(lw), P(lb), P(pr), P(coef), nc,
              P(ref), P(np32), B, T, D, s)
    out = torch.empty(B * T, nc, D, dtype=torch.float16, device="cuda")
    _lib.call("rwkvq_shift_lerp_f16", P(x), P(lw), P(lb), P(pr), P(coef),
              nc, P(out), order, P(np16), B, T, D, s)
    assert torch.equal(out.view(-1, D), _x16(ref.view(-1, D), order))
    assert torch.equal(np16, np32)


@pytest.mark.parametrize("order", ORDERS)
def test_wkv_tail_f16(order):
    g = torch.Generator().manual_seed(40 + order)
    N, D = 37, 2048
    t = lambda *s: torch.randn(*s, generator=g).cuda()
    y, rkv, kp, vp, gg = t(N, D), t(N, 3 * D), t(N, D), t(N, D), t(N, D)
    r_k, lnw, lnb = t(D), t(D), t(D)
    s = _lib.stream_handle()
    ref = torch.empty(N, D, device="cuda")
    _lib.call("rwkvq_wkv_tail", P(y), P(rkv), P(kp), P(vp), P(gg), P(r_k),
              P(lnw), P(lnb), P(ref), N, D, 64, s)
    out = torch.empty(N, D, dtype=torch.float16, device="cuda")
    _lib.call("rwkvq_wkv_tail_f16", P(y), P(rkv), P(kp), P(vp), P(gg),
              P(r_k), P(lnw), P(lnb), P(out), order, N, D, 64, s)
    assert torch.equal(out, _x16(ref, order))


@pytest.mark.parametrize("kind,bits", [("sym", 6), ("sb6", 5), ("rtn", 8)])
@pytest.mark.parametrize("order", ORDERS)
@pytest.mark.parametrize("M", [37, 512])
def test_gemm_y16(kind, bits, order, M):
    """The GEMM writing relu^2 of its sums as fp16 in a consumer's pair
    order == its fp32 output through rwkvq_x16, bit for bit."""
    lin = {"sym": SymQuantLinear, "sb6": GwQuantLinear,
           "rtn": QuantLinearV2}[kind](
        qt_for(kind, bits, weights(1024, 2048, seed=bits)))
    x = act(M, 2048, seed=M).cuda()
    ref = torch.empty(M, 1024, device="cuda")
    lin._run("gemm", x, ref, mode=_lib.EPI_RELU2, n=M)
    y16 = torch.empty(M, 1024, dtype=torch.float16, device="cuda")
    lin._run("gemm", x, y16, n=M,
             mode=_lib.EPI_RELU2 | _lib.Y_F16 | (order << _lib.Y_ORDER_SHIFT))
    assert torch.equal(y16, _x16(ref, order))


def test_gemm_y16_rejects_residual_add():
    lin = SymQuantLinear(qt_for("sym", 8, weights(256, 256, seed=1)))
    x = torch.zeros(128, 256, device="cuda")
    y = torch.empty(128, 256, dtype=torch.float16, device="cuda")
    with pytest.raises(_lib.HipKernelError):
        lin._run("gemm", x, y, n=128, mode=_lib.EPI_ADD | _lib.Y_F16)
