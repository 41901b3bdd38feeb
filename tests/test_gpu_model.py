"""GPU parity of the RWKV-7 kernels and the HIP model against the CPU
oracle (oracle/rwkv7_ref.py, float64).

Bars: WKV state and outputs within 1e-5
relative; end-to-end logits within 1e-2 max-abs."""
import ctypes

import numpy as np
import pytest
import torch

from oracle.rwkv7_ref import RWKV7Oracle, wkv7
from rwkv_quant.backends.hip import _lib
from rwkv_quant.backends.hip import quant_model as qm
from rwkv_quant.models.synthetic import quantized_model

pytestmark = pytest.mark.gpu


def _wkv_inputs(B, T, H, seed):
    g = torch.Generator().manual_seed(seed)
    N = 64
    r, k, v = (torch.randn(B, T, H, N, generator=g) for _ in range(3))
    kk = torch.nn.functional.normalize(torch.randn(B, T, H, N, generator=g),
                                       dim=-1)
    agate = torch.sigmoid(torch.randn(B, T, H, N, generator=g))
    w = torch.exp(-torch.exp(torch.randn(B, T, H, N, generator=g) * 0.5
                             - 0.5))
    s0 = torch.randn(B, H, N, N, generator=g) * 0.05
    return r, w, k, v, -kk, kk * agate, s0


@pytest.mark.parametrize("B,T,H", [(1, 1, 4), (3, 1, 32), (1, 33, 4),
                                   (2, 17, 8), (1, 128, 32)])
def test_wkv7_scan_matches_oracle(B, T, H):
    print(f"wkv scan B={B} T={T} H={H}", flush=True)
    r, w, k, v, a, b, s0 = _wkv_inputs(B, T, H, seed=B * 100 + T)
    dev = [t.reshape(B, T, H * 64).contiguous().cuda()
           for t in (r, w, k, v, a, b)]
    st_in = s0.cuda().contiguous()
    st_out = torch.empty_like(st_in)
    y = torch.empty(B, T, H * 64, device="cuda")
    D = H * 64
    _lib.call("rwkvq_wkv7_scan", _lib.ptr(dev[0]), D, _lib.ptr(dev[1]),
              _lib.ptr(dev[2]), _lib.ptr(dev[3]), _lib.ptr(dev[4]),
              _lib.ptr(dev[5]), D, _lib.ptr(st_in), _lib.ptr(st_out),
              _lib.ptr(y), D, B, T, H, 64, _lib.stream_handle())
    yr, sr = wkv7(*(t.double().numpy() for t in (r, w, k, v, a, b)),
                  s0.double().numpy())
    yd = y.cpu().double().numpy().reshape(B, T, H, 64)
    sd = st_out.cpu().double().numpy()
    assert np.abs(yd - yr).max() / np.abs(yr).max() < 1e-5
    assert np.abs(sd - sr).max() / np.abs(sr).max() < 1e-5
    assert torch.equal(st_in.cpu(), s0)          # input state untouched


@pytest.mark.parametrize("B,T,nc,prev", [(1, 1, 6, True), (8, 1, 6, True),
                                         (3, 1, 1, False), (1, 5, 6, True),
                                         (2, 300, 1, True)])
def test_shift_lerp_matches_float64(B, T, nc, prev):
    """LN (eps 1e-5, two-pass) + token shift + lerps, over the column
    slicing of few-row launches and the one-workgroup-per-row layout of
    long ones; float64 reference, relative 1e-5."""
    D = 2048
    g = torch.Generator().manual_seed(B * 7 + T)
    x = torch.randn(B, T, D, generator=g) * 3 + 0.5
    lw, lb = torch.rand(D, generator=g) + 0.5, torch.randn(D, generator=g)
    pr = torch.randn(B, D, generator=g) if prev else None
    coef = torch.rand(nc, D, generator=g)
    out = torch.empty(B, T, nc, D, device="cuda")
    new_prev = torch.empty(B, D, device="cuda")
    dev = [t.cuda() if t is not None else None for t in (x, lw, lb, pr, coef)]
    _lib.call("rwkvq_shift_lerp", _lib.ptr(dev[0]), _lib.ptr(dev[1]),
              _lib.ptr(dev[2]), _lib.ptr(dev[3]), _lib.ptr(dev[4]), nc,
              _lib.ptr(out), _lib.ptr(new_prev), B, T, D,
              _lib.stream_handle())
    xd = x.double()
    mu = xd.mean(-1, keepdim=True)
    var = ((xd - mu) ** 2).mean(-1, keepdim=True)
    xn = (xd - mu) / torch.sqrt(var + 1e-5) * lw.double() + lb.double()
    first = pr.double()[:, None] if prev else torch.zeros(B, 1, D,
                                                          dtype=torch.float64)
    shift = torch.cat([first, xn[:, :-1]], 1)
    ref = xn[:, :, None] + (shift - xn)[:, :, None] * coef.double()
    assert float((out.cpu().double() - ref).abs().max()) < 1e-5 * float(
        ref.abs().max())
    assert float((new_prev.cpu().double() - xn[:, -1]).abs().max()) < 1e-5 * float(
        xn.abs().max())


def _scan_chunked(dev, st_in, st_out, y, B, T, H):
    D = H * 64
    nc = -(-(-(-T // 16)) // 3) * 3           # chunks, padded to 3k
    ws = torch.empty(B * H * nc * 6400, device="cuda")
    _lib.call("rwkvq_wkv7_scan_chunked", _lib.ptr(dev[0]), D,
              _lib.ptr(dev[1]), _lib.ptr(dev[2]), _lib.ptr(dev[3]),
              _lib.ptr(dev[4]), _lib.ptr(dev[5]), D, _lib.ptr(st_in),
              _lib.ptr(st_out), _lib.ptr(y), D, B, T, H, 64, _lib.ptr(ws),
              ws.numel(), _lib.stream_handle())


@pytest.mark.parametrize("B,T,H", [(1, 16, 4), (1, 37, 4), (2, 33, 8),
                                   (1, 128, 32), (1, 512, 32)])
def test_wkv7_scan_chunked_matches_oracle(B, T, H):
    """The 16-step chunked scan (WY operators + fp32 matrix-core pass):
    ragged last chunks, several sequences, the prefill length."""
    print(f"wkv chunked B={B} T={T} H={H}", flush=True)
    r, w, k, v, a, b, s0 = _wkv_inputs(B, T, H, seed=B * 1000 + T)
    dev = [t.reshape(B, T, H * 64).contiguous().cuda()
           for t in (r, w, k, v, a, b)]
    st_in = s0.cuda().contiguous()
    st_out = torch.empty_like(st_in)
    y = torch.empty(B, T, H * 64, device="cuda")
    _scan_chunked(dev, st_in, st_out, y, B, T, H)
    yr, sr = wkv7(*(t.double().numpy() for t in (r, w, k, v, a, b)),
                  s0.double().numpy())
    yd = y.cpu().double().numpy().reshape(B, T, H, 64)
    sd = st_out.cpu().double().numpy()
    assert np.abs(yd - yr).max() / np.abs(yr).max() < 1e-5
    assert np.abs(sd - sr).max() / np.abs(sr).max() < 1e-5
    assert torch.equal(st_in.cpu(), s0)          # input state untouched


def test_wkv7_scan_chunked_in_place_and_vs_steps():
    """state_in == state_out (the model's own buffers may alias), and the
    chunked and step-by-step scans agree to fp32 rounding; a zero decay
    (floored at e^-60) stays finite."""
    B, T, H = 1, 48, 8
    r, w, k, v, a, b, s0 = _wkv_inputs(B, T, H, seed=77)
    w[0, 5, 2, :7] = 0.0
    dev = [t.reshape(B, T, H * 64).contiguous().cuda()
           for t in (r, w, k, v, a, b)]
    st = s0.cuda().contiguous()
    y1 = torch.empty(B, T, H * 64, device="cuda")
    _scan_chunked(dev, st, st, y1, B, T, H)
    st2 = torch.empty_like(st)
    y2 = torch.empty_like(y1)
    D = H * 64
    s0d = s0.cuda()            # (held: the launch is asynchronous)
    _lib.call("rwkvq_wkv7_scan", _lib.ptr(dev[0]), D, _lib.ptr(dev[1]),
              _lib.ptr(dev[2]), _lib.ptr(dev[3]), _lib.ptr(dev[4]),
              _lib.ptr(dev[5]), D, _lib.ptr(s0d), _lib.ptr(st2),
              _lib.ptr(y2), D, B, T, H, 64, _lib.stream_handle())
    assert torch.isfinite(y1).all() and torch.isfinite(st).all()
    assert float((y1 - y2).abs().max()) < 1e-5 * float(y2.abs().max())
    assert float((st - st2).abs().max()) < 1e-5 * float(st2.abs().max())
    with pytest.raises(_lib.HipKernelError):     # workspace too small
        _lib.call("rwkvq_wkv7_scan_chunked", _lib.ptr(dev[0]), D,
                  _lib.ptr(dev[1]), _lib.ptr(dev[2]), _lib.ptr(dev[3]),
                  _lib.ptr(dev[4]), _lib.ptr(dev[5]), D, _lib.ptr(st),
                  _lib.ptr(st), _lib.ptr(y1), D, B, T, H, 64, _lib.ptr(y1),
                  100, _lib.stream_handle())


def test_lora_kernel_matches_matmul():
    g = torch.Generator().manual_seed(1)
    ranks = [96, 96, 64, 256]
    W = [(torch.randn(r, 2048, generator=g) * 0.02).half() for r in ranks]
    U = [(torch.randn(2048, r, generator=g) * 0.02).half() for r in ranks]
    x = torch.randn(3, 2048, generator=g)
    h = [torch.empty(3, r, device="cuda") for r in ranks]
    y = [torch.empty(3, 2048, device="cuda") for _ in ranks]
    xd = x.cuda()
    epi = [_lib.EPI_TANH, 0, 0, _lib.EPI_SIGMOID]
    qm.QuantTMix._grouped([w.cuda() for w in W], [xd] * 4, [2048] * 4, h,
                          epi, 3)
    qm.QuantTMix._grouped([u.cuda() for u in U], h, ranks, y, [0] * 4, 3)
    for i in range(4):
        ref = x.double() @ W[i].double().t()
        ref = torch.tanh(ref) if i == 0 else (torch.sigmoid(ref) if i == 3
                                              else ref)
        assert (h[i].cpu().double() - ref).abs().max() < 2e-3 * ref.abs().max()
        ref2 = h[i].cpu().double() @ U[i].double().t()
        assert (y[i].cpu().double() - ref2).abs().max() < \
            2e-3 * ref2.abs().max()


@pytest.fixture(scope="module", params=["compression", "reduction"])
def toy(request):
    ck = quantized_model(request.param, n_layer=2, n_embd=256, vocab=1024,
                         seed=11)
    return ck, RWKV7Oracle(ck), qm.QuantRWKV7(ck)


def _maxabs(a, b):
    return float(np.abs(np.asarray(a, np.float64) - b).max())


def test_prefill_logits_match_oracle(toy):
    ck, orc, model = toy
    idx = np.random.default_rng(2).integers(0, 1024, size=(2, 12))
    ref, _ = orc.forward_stateful(idx, orc.init_state(2))
    out, _ = model.forward_stateful(torch.from_numpy(idx),
                                    model.init_state(2))
    err = _maxabs(out.cpu().numpy(), ref)
    print("prefill max-abs", err, "logit scale", np.abs(ref).max())
    assert err < 1e-2
    assert err < 2e-3 * max(1.0, np.abs(ref).max()) * 10


def test_gemm_prefill_path_matches_oracle(toy):
    """B*T >= 128 takes the GEMM path."""
    ck, orc, model = toy
    idx = np.random.default_rng(3).integers(0, 1024, size=(1, 160))
    ref, st_ref = orc.forward_stateful(idx, orc.init_state(1))
    out, st = model.forward_stateful(torch.from_numpy(idx),
                                     model.init_state(1))
    assert _maxabs(out.cpu().numpy(), ref) < 1e-2
    for (a, b, c), (d, e, f) in zip(st, st_ref):
        assert _maxabs(a.cpu().numpy(), d) < 1e-3 * max(1, np.abs(d).max())


def test_graph_decode_matches_oracle_and_eager(toy):
    ck, orc, model = toy
    B = 3
    idx = np.random.default_rng(4).integers(0, 1024, size=(B, 6))
    st_o = orc.init_state(B)
    st_g = model.init_state(B)
    st_e = model.init_state(B)
    for t in range(6):
        ro, st_o = orc.forward_stateful(idx[:, t:t + 1], st_o)
        lg, st_g = model.step(torch.from_numpy(idx[:, t:t + 1]), st_g)
        le, st_e = model.forward_stateful(torch.from_numpy(idx[:, t:t + 1]),
                                          st_e)
        assert _maxabs(lg.cpu().numpy(), ro) < 1e-2
        # graph replay and eager run the same kernels on the same inputs
        assert torch.equal(lg, le)


def test_decode_continues_prefill_state(toy):
    ck, orc, model = toy
    idx = np.random.default_rng(5).integers(0, 1024, size=(1, 9))
    ref, _ = orc.forward_stateful(idx, orc.init_state(1))
    _, st = model.forward_stateful(torch.from_numpy(idx[:, :8]),
                                   model.init_state(1))
    lg, _ = model.step(torch.from_numpy(idx[:, 8:]), st)
    assert _maxabs(lg.cpu().numpy()[:, 0], ref[:, 8]) < 1e-2


@pytest.mark.parametrize("layer0", [1, 0])
def test_fused_decode_core_equals_three_kernels(layer0):
    """rwkvq_wkv7_decode == wkv_prep + wkv7_scan(T=1) + wkv_tail."""
    B, H = 3, 32
    D = H * 64
    g = torch.Generator().manual_seed(21 + layer0)
    mk = lambda *s, sc=1.0: (torch.randn(*s, generator=g) * sc).cuda()
    rkv, yw, ya, yv, gg = mk(B, 3, D), mk(B, D), mk(B, D), mk(B, D), mk(B, D)
    w0, a0, v0 = mk(D, sc=0.5), mk(D, sc=0.5), mk(D, sc=0.5)
    k_k, k_a, r_k = mk(D).abs(), torch.rand(D).cuda(), mk(D, sc=0.1)
    lnw, lnb = mk(D), mk(D, sc=0.1)
    vf1, vf2 = mk(B, D), None
    vf2 = vf1.clone()
    st0 = mk(B, H, 64, 64, sc=0.05)
    st_a, st_b = torch.empty_like(st0), torch.empty_like(st0)
    out_a, out_b = torch.empty(B, D).cuda(), torch.empty(B, D).cuda()
    P = _lib.ptr
    s = _lib.stream_handle()
    _lib.call("rwkvq_wkv7_decode", P(rkv), P(yw), P(ya), P(yv), P(gg), P(w0),
              P(a0), P(v0), P(k_k), P(k_a), P(r_k), P(lnw), P(lnb), P(vf1),
              layer0, P(st0), P(st_a), P(out_a), B, H, 64, s)
    w, kp, vp, aa, bb, y = (torch.empty(B, D).cuda() for _ in range(6))
    _lib.call("rwkvq_wkv_prep", P(rkv), P(yw), P(ya), P(yv), P(w0), P(a0),
              P(v0), P(k_k), P(k_a), P(vf2), layer0, P(w), P(kp), P(vp),
              P(aa), P(bb), B, D, 64, s)
    _lib.call("rwkvq_wkv7_scan", P(rkv), 3 * D, P(w), P(kp), P(vp), P(aa),
              P(bb), D, P(st0), P(st_b), P(y), D, B, 1, H, 64, s)
    _lib.call("rwkvq_wkv_tail", P(y), P(rkv), P(kp), P(vp), P(gg), P(r_k),
              P(lnw), P(lnb), P(out_b), B, D, 64, s)
    rel = lambda a, b: float((a - b).abs().max() / b.abs().max())
    assert rel(st_a, st_b) < 1e-5
    assert rel(out_a, out_b) < 1e-5
    assert torch.equal(vf1, vf2)


def test_graph_prefill_equals_eager(toy):
    """forward_stateful replays a per-shape graph; it must equal the eager
    launch sequence bit for bit, replay after replay."""
    ck, orc, model = toy
    idx = torch.from_numpy(np.random.default_rng(8).integers(0, 1024, (2, 9)))
    qm.USE_GRAPH = False
    try:
        ref, st_ref = model.forward_stateful(idx, model.init_state(2))
    finally:
        qm.USE_GRAPH = True
    for _ in range(3):
        out, st = model.forward_stateful(idx, model.init_state(2))
        assert torch.equal(out, ref)
        for a, b in zip(st, st_ref):
            for x, y in zip(a, b):
                assert torch.equal(x, y)


@pytest.mark.parametrize("layer0", [1, 0])
@pytest.mark.parametrize("T", [37, 160])
def test_prefill_core_fused_equals_prep_then_chunked(layer0, T):
    """rwkvq_wkv7_prefill_chunked (prep folded into the chunk operators) ==
    rwkvq_wkv_prep + rwkvq_wkv7_scan_chunked: y, state, k', v' and v_first
    to 1e-6 relative (the two kernels may contract the prep arithmetic
    differently)."""
    g = torch.Generator().manual_seed(T + layer0)
    B, H = 2, 4
    D, N = H * 64, 2 * T
    t = lambda *s, sc=1.0: (torch.randn(*s, generator=g) * sc).cuda()
    rkv, yw, ya, yv = t(N, 3 * D), t(N, D), t(N, D), t(N, D)
    w0, a0, v0 = t(D, sc=0.5), t(D), t(D)
    k_k, k_a = t(D).abs(), t(D).abs()
    vf0 = t(N, D)
    st0 = t(B, H, 64, 64, sc=0.1)
    P, s = _lib.ptr, _lib.stream_handle()
    nc = ((-(-T // 16)) + 2) // 3 * 3
    ops = torch.empty(B * H * nc * 6400, device="cuda")
    # reference: prep, then the chunked scan
    w, kp, vp, aa, bb = (torch.empty(N, D, device="cuda") for _ in range(5))
    vf1 = vf0.clone()
    _lib.call("rwkvq_wkv_prep", P(rkv), P(yw), P(ya), None if layer0 else
              P(yv), P(w0), P(a0), None if layer0 else P(v0), P(k_k), P(k_a),
              P(vf1), layer0, P(w), P(kp), P(vp), P(aa), P(bb), N, D, 64, s)
    st1, y1 = torch.empty_like(st0), torch.empty(N, D, device="cuda")
    _lib.call("rwkvq_wkv7_scan_chunked", P(rkv), 3 * D, P(w), P(kp), P(vp),
              P(aa), P(bb), D, P(st0), P(st1), P(y1), D, B, T, H, 64, P(ops),
              ops.numel(), s)
    # fused
    vf2 = vf0.clone()
    kp2, vp2 = torch.empty_like(kp), torch.empty_like(vp)
    st2, y2 = torch.empty_like(st0), torch.empty(N, D, device="cuda")
    _lib.call("rwkvq_wkv7_prefill_chunked", P(rkv), P(yw), P(ya),
              None if layer0 else P(yv), P(w0), P(a0),
              None if layer0 else P(v0), P(k_k), P(k_a), P(vf2), layer0,
              P(kp2), P(vp2), P(st0), P(st2), P(y2), B, T, H, 64, P(ops),
              ops.numel(), s)
    rel = lambda a, b: float((a - b).abs().max() / b.abs().max())
    for a_, b_ in ((y2, y1), (st2, st1), (kp2, kp), (vp2, vp), (vf2, vf1)):
        assert rel(a_, b_) < 1e-6
