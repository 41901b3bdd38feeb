"""The kernel variants bench.py times, at the shapes it times them, against
the CPU oracle ([3], [4]).

GEMM: the 2.9B projections at M = 2048 tokens (pp2048) and the 1.5B sym@8
head at M = 512 (pp512).  rwkvq_gemm_plan names the variant each shape
takes, so the test asserts that the 256 x 128 eight-wave tile, the
two-workgroups-per-CU split-K tile and the 128 x 128 two-K-group tile are
all reached.  Bars as tests/test_gpu_gemm.py: relmax < 1e-3 against the
float64 x . dequant(W)^T, < 2e-5 against the float64 product of the fp16
operands (reference gate: tests/test_gemm_prefill.py:32-49).

GEMV: the decode heads at their full 65536 x 2048 (rtn@8, configs[1];
sb6@5, the compression preset's head), relmax < 1e-3.
WKV: the chunked scan at the pp2048 shape (B = 1, T = 2048, H = 40),
1e-5 relative against the float64 recurrence."""
import numpy as np
import pytest
import torch

from oracle import codec_ref as cr
from oracle.rwkv7_ref import wkv7
from rwkv_quant.backends.hip import _lib
from rwkv_quant.backends.hip.quant_linear import (
    GwQuantLinear, QuantLinearV2, SymQuantLinear, SymQuantLinearFused)

from _util import act, qt_for, relmax, weights

pytestmark = pytest.mark.gpu

LIN = {"sb6": GwQuantLinear, "sym": SymQuantLinear, "rtn": QuantLinearV2}


def _check(y, x, qt, lin, kind):
    """relmax of y against the oracle and the fp16-operand product,
    computed in row chunks of W (the 65536-row head in float64)."""
    W = cr.dequant_qt(qt)
    xd = x.numpy().astype(np.float64)
    x16 = x.half().double().numpy()
    y = np.asarray(y, np.float64)
    err = err16 = ref_max = ref16_max = 0.0
    step = 8192
    for r0 in range(0, W.shape[0], step):
        sl = slice(r0, r0 + step)
        ref = xd @ W[sl].astype(np.float64).T
        if kind == "rtn":
            q = qt.codes[sl].double().numpy()
            s = qt.scale[sl].float().double().numpy().reshape(1, -1)
            ref16 = (x16 @ q.T) * s
        else:
            w16 = lin._dequant_w(torch.float16)[sl].cpu().double().numpy()
            ref16 = x16 @ w16.T
        err = max(err, np.abs(y[:, sl] - ref).max())
        err16 = max(err16, np.abs(y[:, sl] - ref16).max())
        ref_max = max(ref_max, np.abs(ref).max())
        ref16_max = max(ref16_max, np.abs(ref16).max())
    return err / ref_max, err16 / ref16_max


# (name, kind, bits, rows, in, out_per, M, expected plan subset)
GEMM_CASES = [
    # 2.9B pp2048: channel-mix key 2560 -> 10240, 256 x 128 eight-wave tile
    ("2p9b_key_sym6", "sym", 6, 10240, 2560, 10240, 2048,
     dict(tile_rows=256, tile_tokens=128, waves=8, kgroups=1, split=1)),
    # 2.9B pp2048: channel-mix value 10240 -> 2560, two 4-wave workgroups
    # per CU with K split in two runs of 40 steps
    ("2p9b_value_sym6", "sym", 6, 2560, 10240, 2560, 2048,
     dict(tile_rows=128, tile_tokens=128, waves=4, kgroups=1, split=2)),
    # 2.9B pp2048: r/k/v (three 2560 x 2560 sym@8 in one launch)
    ("2p9b_rkv_sym8", "sym", 8, 7680, 2560, 2560, 2048,
     dict(tile_rows=256, waves=8)),
    # 2.9B pp2048: output projection 2560 x 2560, 128 x 128 with two K
    # groups per workgroup
    ("2p9b_o_sym8", "sym", 8, 2560, 2560, 2560, 2048,
     dict(tile_rows=128, tile_tokens=128, kgroups=2, split=1)),
    # 1.5B pp512: head 2048 -> 65536 sym@8, 256 x 128 eight-wave tile
    ("1p5b_head_sym8", "sym", 8, 65536, 2048, 65536, 512,
     dict(tile_rows=256, tile_tokens=128, waves=8)),
    # 1.5B pp512: channel-mix value 8192 -> 2048 sym@6
    ("1p5b_value_sym6", "sym", 6, 2048, 8192, 2048, 512, {}),
    # compression preset prefill at pp2048: sb6@4 key 2560 -> 10240
    ("2p9b_key_sb6_4", "sb6", 4, 10240, 2560, 10240, 2048,
     dict(tile_rows=256, waves=8)),
]


@pytest.mark.parametrize("case", GEMM_CASES, ids=[c[0] for c in GEMM_CASES])
def test_gemm_bench_shape(case):
    name, kind, bits, rows, k_in, out_per, M, want = case
    print(f"gemm {name}: {kind}@{bits} {rows}x{k_in} out_per={out_per} "
          f"M={M}", flush=True)
    plan = _lib.gemm_plan(rows, k_in, out_per, M, _lib.X_F16)
    print("plan", plan, flush=True)
    for key, v in want.items():
        assert plan[key] == v, (key, plan)
    w = weights(rows, k_in, seed=rows + k_in + bits, outlier_cols=2)
    segs = rows // out_per
    if segs > 1:
        lins = [LIN[kind](qt_for(kind, bits, w[j * out_per:(j + 1) * out_per]))
                for j in range(segs)]
        lin = SymQuantLinearFused(lins)
        qts = [qt_for(kind, bits, w[j * out_per:(j + 1) * out_per])
               for j in range(segs)]
    else:
        qt = qt_for(kind, bits, w)
        lin = LIN[kind](qt)
    x = act(M, segs * k_in, seed=M + rows)
    xd = x.cuda()
    y = torch.empty(M, rows, device="cuda")
    # fp16 pair-ordered input, as the model's producers write it
    target = lin._cat if segs > 1 else lin
    order = target.x16_order
    x16 = torch.empty(M, segs * k_in, dtype=torch.float16, device="cuda")
    _lib.call("rwkvq_x16", _lib.ptr(xd), segs * k_in, segs * k_in, M, order,
              _lib.ptr(x16), segs * k_in, _lib.stream_handle())
    if segs > 1:
        lin.apply_into(x16, y, M, segs * k_in, mode=_lib.X_F16)
    else:
        lin.apply_into(x16, y, mode=_lib.X_F16, n=M)
    yc = y.cpu().numpy()
    y32 = torch.empty_like(y)           # the fp32-input launch, same bits
    if segs > 1:
        lin.apply_into(xd, y32, M, segs * k_in)
    else:
        lin.apply_into(xd, y32, n=M)
    assert torch.equal(y, y32)
    if segs > 1:
        for j in range(segs):
            sub = LIN[kind](qts[j])
            e, e16 = _check(yc[:, j * out_per:(j + 1) * out_per],
                            x[:, j * k_in:(j + 1) * k_in], qts[j], sub, kind)
            assert e < 1e-3 and e16 < 2e-5, (j, e, e16)
    else:
        e, e16 = _check(yc, x, qt, lin, kind)
        print(f"relmax {e:.2e}, vs fp16 operands {e16:.2e}", flush=True)
        assert e < 1e-3 and e16 < 2e-5


def test_gemm_split_run_to_run_identical():
    """The split-K launch (two workgroups per CU, K in two runs) is
    deterministic: the last arriver adds the partials in run order."""
    w = weights(2560, 10240, seed=5)
    lin = SymQuantLinear(qt_for("sym", 6, w))
    x = act(2048, 10240, seed=6).cuda()
    y1 = torch.empty(2048, 2560, device="cuda")
    y2 = torch.empty_like(y1)
    lin.apply_into(x, y1, n=2048)
    lin.apply_into(x, y2, n=2048)
    assert torch.equal(y1, y2)


@pytest.mark.parametrize("kind,bits", [("rtn", 8), ("sb6", 5), ("sym", 8)])
@pytest.mark.parametrize("n", [1, 8])
def test_head_gemv_full_vocab(kind, bits, n):
    """The decode head at 65536 x 2048 (the interleaved row order of the
    lane-dot kernel at n = 1, the matrix-core batched GEMV at n = 8)."""
    print(f"head gemv {kind}@{bits} n={n}", flush=True)
    w = weights(65536, 2048, seed=40 + bits, outlier_cols=2)
    qt = qt_for(kind, bits, w)
    lin = LIN[kind](qt)
    x = act(n, 2048, seed=41)
    y = lin(x.cuda()).cpu().numpy()
    W = cr.dequant_qt(qt)
    err = ref_max = 0.0
    for r0 in range(0, 65536, 16384):
        ref = cr.gemv_ref(x.numpy(), W[r0:r0 + 16384])
        err = max(err, np.abs(y[:, r0:r0 + 16384] - ref).max())
        ref_max = max(ref_max, np.abs(ref).max())
    print(f"relmax {err / ref_max:.2e}", flush=True)
    assert err / ref_max < 1e-3


def test_wkv7_scan_chunked_pp2048_shape():
    """B = 1, T = 2048, H = 40 (the 2.9B prefill): 129 chunks."""
    B, T, H = 1, 2048, 40
    print(f"wkv chunked B={B} T={T} H={H}", flush=True)
    g = torch.Generator().manual_seed(2048)
    N = 64
    r, k, v = (torch.randn(B, T, H, N, generator=g) for _ in range(3))
    kk = torch.nn.functional.normalize(torch.randn(B, T, H, N, generator=g),
                                       dim=-1)
    agate = torch.sigmoid(torch.randn(B, T, H, N, generator=g))
    w = torch.exp(-torch.exp(torch.randn(B, T, H, N, generator=g) * 0.5
                             - 0.5))
    a, b = -kk, kk * agate
    s0 = torch.randn(B, H, N, N, generator=g) * 0.05
    D = H * N
    dev = [t.reshape(B, T, D).contiguous().cuda() for t in (r, w, k, v, a, b)]
    st_in = s0.cuda().contiguous()
    st_out = torch.empty_like(st_in)
    y = torch.empty(B, T, D, device="cuda")
    nc = -(-(-(-T // 16)) // 3) * 3
    ws = torch.empty(B * H * nc * 6400, device="cuda")
    _lib.call("rwkvq_wkv7_scan_chunked", _lib.ptr(dev[0]), D,
              _lib.ptr(dev[1]), _lib.ptr(dev[2]), _lib.ptr(dev[3]),
              _lib.ptr(dev[4]), _lib.ptr(dev[5]), D, _lib.ptr(st_in),
              _lib.ptr(st_out), _lib.ptr(y), D, B, T, H, 64, _lib.ptr(ws),
              ws.numel(), _lib.stream_handle())
    yr, sr = wkv7(*(t.double().numpy() for t in (r, w, k, v, a, b)),
                  s0.double().numpy())
    yd = y.cpu().double().numpy().reshape(B, T, H, 64)
    sd = st_out.cpu().double().numpy()
    ey = np.abs(yd - yr).max() / np.abs(yr).max()
    es = np.abs(sd - sr).max() / np.abs(sr).max()
    print(f"y {ey:.2e} state {es:.2e}", flush=True)
    assert ey < 1e-5 and es < 1e-5
