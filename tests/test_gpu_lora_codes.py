"""GPU parity of the decode LoRA read straight from the file's codes
(world checkpoints: asym gw64 @6 for w / a / v, per-row int8 for g).

Bars: the down products (rwkvq_lora_down_q) against float64 products of
the format's exact dequantization, relmax < 1e-5 before the activation and
max-abs < 1e-5 x max|pre-activation| after it (tanh and sigmoid are
1-Lipschitz); the fused WKV step with the up products from codes
(rwkvq_wkv7_decode_lora_q) against rwkvq_wkv7_decode fed with the float64
up products rounded to fp32: outputs and states within 1e-5 relative.
Formats and shapes of the presets at D = 2048 and 2560 (ranks 96 / 96 /
64 / 256 and 96 / 96 / 64 / 320)."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import codec_ref as cr
from rwkv_quant.backends.hip import _lib
from rwkv_quant.backends.hip.repack import lora_down_device, lora_up_device
from rwkv_quant.formats import writer

from _util import relmax

pytestmark = pytest.mark.gpu

P = ctypes.c_void_p
EPI = {"w": _lib.EPI_TANH, "a": _lib.EPI_STORE, "v": _lib.EPI_STORE,
       "g": _lib.EPI_SIGMOID}
RANKS = {2048: dict(w=96, a=96, v=64, g=256),
         2560: dict(w=96, a=96, v=64, g=320)}


def _factor(b, shape, seed):
    w = torch.randn(*shape, generator=torch.Generator().manual_seed(seed))
    w = w * 0.05
    if b == "g":
        c, s = writer.rtn_quantize(w, 8)
        return writer.make_rtn("g", "g_lora", 8, w.shape, c, s)
    return writer.pack_asym(b, f"{b}_lora", 6, w, 64)


def _dev(qt, fn):
    n = lambda t: t.numpy()
    if qt.gw_mode == "asym":
        lay = fn(n(qt.codes), tuple(qt.shape), scale=n(qt.gw_scale),
                 mn=n(qt.gw_min))
    else:
        lay = fn(n(qt.codes), tuple(qt.shape), row_scale=n(qt.scale))
    return {k: None if v is None else torch.from_numpy(v).cuda()
            for k, v in lay.items()}


def _ptrs(lays, key):
    return (P * len(lays))(*[None if l is None or l[key] is None
                             else l[key].data_ptr() for l in lays])


def _down(C, branches, N, epi, seed):
    """Run rwkvq_lora_down_q over the branches; return (got, ref_pre)."""
    rk = RANKS[C]
    qts = {b: _factor(b, (C, rk[b]), seed + i) for i, b in
           enumerate(branches)}
    lays = [_dev(qts[b], lora_down_device) for b in branches]
    g = torch.Generator().manual_seed(seed)
    xs = torch.randn(N, 6 * C, generator=g) * 3.0
    xs[:, ::97] = 0.0
    xs_d = xs.cuda()
    ys = [torch.empty(N, rk[b], device="cuda") for b in branches]
    n = len(branches)
    ia = lambda v: (ctypes.c_int * n)(*v)
    _lib.call("rwkvq_lora_down_q", n, _ptrs(lays, "q"), _ptrs(lays, "s"),
              _ptrs(lays, "m"), _ptrs(lays, "sc"),
              (P * n)(*[xs_d[:, k * C:].data_ptr() for k in range(n)]),
              ia([6 * C] * n), (P * n)(*[y.data_ptr() for y in ys]),
              ia([rk[b] for b in branches]), ia([rk[b] for b in branches]),
              ia([epi[b] for b in branches]), C, N, _lib.stream_handle())
    torch.cuda.synchronize()
    x64 = xs.numpy().astype(np.float64)
    refs = [x64[:, k * C:(k + 1) * C] @ cr.dequant_qt(qts[b]).astype(np.float64)
            for k, b in enumerate(branches)]
    return [y.cpu().numpy() for y in ys], refs


@pytest.mark.parametrize("C,N", [(2048, 1), (2048, 2), (2048, 5), (2048, 8),
                                 (2560, 1), (2560, 6)])
def test_down_products_from_codes(C, N):
    print(f"lora down codes C={C} N={N}", flush=True)
    br = ["w", "a", "v", "g"]
    got, ref = _down(C, br, N, {b: _lib.EPI_STORE for b in br}, 100 + N)
    for b, y, r in zip(br, got, ref):
        assert relmax(y, r) < 1e-5, b


def test_down_products_epilogues_and_layer0():
    br = ["w", "a", "g"]                          # layer 0: no v branch
    got, ref = _down(2048, br, 3, EPI, 7)
    act = {"w": np.tanh, "a": lambda v: v, "g": lambda v: 1 / (1 + np.exp(-v))}
    for b, y, r in zip(br, got, ref):
        assert np.abs(y - act[b](r)).max() < 1e-5 * max(1.0, np.abs(r).max())


def test_down_rejects_oversized_batch():
    br = ["w"]
    with pytest.raises(_lib.HipKernelError):
        _down(2560, br, 7, {"w": 0}, 1)       # 7 x 2560 > 16384 staged


def _decode_inputs(B, C, seed):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s, sc=1.0: (torch.randn(*s, generator=g) * sc).cuda()
    H = C // 64
    return dict(rkv=r(B, 3 * C, sc=0.5), w0=r(C, sc=0.5), a0=r(C, sc=0.5),
                v0=r(C, sc=0.5), k_k=r(C, sc=0.5), k_a=r(C, sc=0.5),
                r_k=r(C, sc=0.5), lnw=r(C), lnb=r(C, sc=0.1),
                vf=r(B, C), st=r(B, H, 64, 64, sc=0.3))


@pytest.mark.parametrize("C,B,layer0", [(2048, 1, 0), (2048, 3, 0),
                                        (2048, 2, 1), (2560, 1, 0)])
def test_fused_decode_up_from_codes(C, B, layer0):
    print(f"wkv decode lora codes C={C} B={B} layer0={layer0}", flush=True)
    rk = RANKS[C]
    order = ["w", "a", "v", "g"]
    have = [b != "v" or not layer0 for b in order]
    qts = {b: _factor(b, (rk[b], C), 40 + i) for i, b in enumerate(order)}
    lays = [_dev(qts[b], lora_up_device) if h else None
            for b, h in zip(order, have)]
    gen = torch.Generator().manual_seed(B)
    hs = {b: torch.randn(B, rk[b], generator=gen) for b in order}
    inp = _decode_inputs(B, C, 9 + B)
    H = C // 64
    # the unfused reference: up products in float64, rounded to fp32
    ys = {b: torch.from_numpy(
        hs[b].numpy().astype(np.float64)
        @ cr.dequant_qt(qts[b]).astype(np.float64)).float().cuda()
        for b in order}
    outs = []
    for fused in (False, True):
        vf = inp["vf"].clone()
        st_out = torch.empty_like(inp["st"])
        out = torch.empty(B, C, device="cuda")
        common = [_lib.ptr(inp["w0"]), _lib.ptr(inp["a0"]), _lib.ptr(inp["v0"]),
                  _lib.ptr(inp["k_k"]), _lib.ptr(inp["k_a"]),
                  _lib.ptr(inp["r_k"]), _lib.ptr(inp["lnw"]),
                  _lib.ptr(inp["lnb"]), _lib.ptr(vf), layer0,
                  _lib.ptr(inp["st"]), _lib.ptr(st_out), _lib.ptr(out), B, H,
                  64, _lib.stream_handle()]
        if fused:
            hd = {b: hs[b].cuda() for b in order}
            _lib.call("rwkvq_wkv7_decode_lora_q", _lib.ptr(inp["rkv"]),
                      (P * 4)(*[hd[b].data_ptr() if h else None
                                for b, h in zip(order, have)]),
                      _ptrs(lays, "q"), _ptrs(lays, "s"), _ptrs(lays, "m"),
                      _ptrs(lays, "sc"),
                      (ctypes.c_int * 4)(*[rk[b] if h else 0
                                           for b, h in zip(order, have)]),
                      *common)
        else:
            _lib.call("rwkvq_wkv7_decode", _lib.ptr(inp["rkv"]),
                      _lib.ptr(ys["w"]), _lib.ptr(ys["a"]),
                      None if layer0 else _lib.ptr(ys["v"]),
                      _lib.ptr(ys["g"]), *common)
        torch.cuda.synchronize()
        outs.append((out.cpu().numpy(), st_out.cpu().numpy(),
                     vf.cpu().numpy()))
    (o0, s0, v0), (o1, s1, v1) = outs
    assert np.isfinite(o1).all()
    assert relmax(o1, o0) < 1e-5
    assert relmax(s1, s0) < 1e-5
    assert np.array_equal(v1, v0)
