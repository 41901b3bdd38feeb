"""rwkvq_wkv7_scan_chunked_noalloc (the entry point that allocates
nothing: its chunk operators live in a library-owned device array)
against rwkvq_wkv7_scan_chunked with a caller workspace, through the C ABI:
bit-identical outputs and states on two calls in a row, the second with a
smaller input (the array keeps the first call's contents), and a clear
error past the array's size."""
import ctypes

import pytest
import torch

from rwkv_quant.backends.hip import _lib

pytestmark = pytest.mark.gpu

SCRATCH_FLOATS = 16 << 20


def _inputs(B, T, H, seed):
    g = torch.Generator().manual_seed(seed)
    N = 64
    r, k, v = (torch.randn(B, T, H, N, generator=g) for _ in range(3))
    kk = torch.nn.functional.normalize(torch.randn(B, T, H, N, generator=g),
                                       dim=-1)
    agate = torch.sigmoid(torch.randn(B, T, H, N, generator=g))
    w = torch.exp(-torch.exp(torch.randn(B, T, H, N, generator=g) * 0.5
                             - 0.5))
    s0 = torch.randn(B, H, N, N, generator=g) * 0.05
    D = H * N
    dev = [t.reshape(B, T, D).contiguous().cuda()
           for t in (r, w, k, v, -kk, kk * agate)]
    return dev, s0.cuda()


def _run(entry, dev, s0, B, T, H):
    D = H * 64
    st_out = torch.empty_like(s0)
    y = torch.empty(B, T, D, device="cuda")
    P = _lib.ptr
    args = [P(dev[0]), D, P(dev[1]), P(dev[2]), P(dev[3]), P(dev[4]),
            P(dev[5]), D, P(s0), P(st_out), P(y), D, B, T, H, 64]
    if entry == "rwkvq_wkv7_scan_chunked":
        nc = -(-(-(-T // 16)) // 3) * 3
        ws = torch.empty(B * H * nc * 6400, device="cuda")
        args += [P(ws), ws.numel()]
    _lib.call(entry, *args, _lib.stream_handle())
    torch.cuda.synchronize()
    return y, st_out


@pytest.mark.parametrize("shape", [[(1, 512, 32), (2, 40, 4)],
                                   [(2, 100, 8), (1, 17, 2)]])
def test_noalloc_scan_equals_workspace_scan(shape):
    for i, (B, T, H) in enumerate(shape):
        print(f"noalloc call {i}: B={B} T={T} H={H}", flush=True)
        dev, s0 = _inputs(B, T, H, seed=100 * i + T)
        y_ref, s_ref = _run("rwkvq_wkv7_scan_chunked", dev, s0, B, T, H)
        y, s = _run("rwkvq_wkv7_scan_chunked_noalloc", dev, s0, B, T, H)
        assert torch.equal(y, y_ref)
        assert torch.equal(s, s_ref)


def test_noalloc_scan_rejects_sizes_past_its_array():
    """B * H * NC * 6400 floats beyond the 64 MiB array: RWKVQ_ERR_SIZE
    from the host check, before any launch (null pointers are never
    touched)."""
    lib = _lib.load()
    B, H, T = 1, 40, 1024 + 16          # NC = 66: 40 * 66 > 2621 slots
    st = lib.rwkvq_wkv7_scan_chunked_noalloc(
        None, H * 64, None, None, None, None, None, H * 64, None, None,
        None, H * 64, B, T, H, 64, _lib.stream_handle())
    assert st == 1003
    assert B * H * 66 * 6400 > SCRATCH_FLOATS
