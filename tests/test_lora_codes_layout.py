"""CPU: the decode-side LoRA layouts (codes read straight from the file)
are permutations of the stored fields that reproduce the format's
dequantization bit for bit (oracle codec_ref.dequant_qt).  Down factors
(world, stored [in, rank]) are read transposed, up factors (stored
[rank, D]) per (head, 16-row block, channel, row)."""
import numpy as np
import pytest
import torch

from oracle import codec_ref as cr
from rwkv_quant.backends.hip.repack import (lora_codes_ok, lora_down_device,
                                            lora_up_device)
from rwkv_quant.formats import writer


def _asym(shape, seed):
    w = torch.randn(*shape, generator=torch.Generator().manual_seed(seed))
    return writer.pack_asym("blocks.0.att.w1", "w_lora", 6, w * 0.05, 64)


def _rtn(shape, seed):
    w = torch.randn(*shape, generator=torch.Generator().manual_seed(seed))
    c, s = writer.rtn_quantize(w * 0.05, 8)
    return writer.make_rtn("blocks.0.att.g1", "g_lora", 8, w.shape, c, s)


def _fields(qt):
    n = lambda t: t.numpy()
    if qt.gw_mode == "asym":
        return dict(scale=n(qt.gw_scale), mn=n(qt.gw_min))
    return dict(row_scale=n(qt.scale))


def _weights_down(lay, rank, n_in):
    q = lay["q"]                                    # [rank, in] bytes
    if lay["s"] is not None:
        g = np.arange(rank) // 64
        return (q.astype(np.float32) * lay["s"][g]) + lay["m"][g]
    sc = lay["sc"].view(np.float16).astype(np.float32)
    return q.view(np.int8).astype(np.float32) * sc[None, :]


def _weights_up(lay, rank, d):
    H = d // 64
    q = lay["q"].transpose(1, 3, 0, 2).reshape(rank, d)   # back to [rank, D]
    if lay["s"] is not None:
        s = np.repeat(lay["s"].T, 64, axis=1)              # [rank, D]
        m = np.repeat(lay["m"].T, 64, axis=1)
        return (q.astype(np.float32) * s) + m
    sc = lay["sc"].view(np.float16).astype(np.float32)
    return q.view(np.int8).astype(np.float32) * sc[:, None]


@pytest.mark.parametrize("kind", ["asym", "rtn"])
@pytest.mark.parametrize("n_in,rank", [(2048, 96), (2560, 64), (2048, 256)])
def test_down_layout_reproduces_dequant(kind, n_in, rank):
    qt = (_asym if kind == "asym" else _rtn)((n_in, rank), rank)
    assert lora_codes_ok(qt, 1, lambda c: c % 16 == 0)
    lay = lora_down_device(qt.codes.numpy(), tuple(qt.shape), **_fields(qt))
    assert lay["q"].nbytes == qt.codes.numpy().nbytes
    ref = cr.dequant_qt(qt)                          # [in, rank]
    got = _weights_down(lay, rank, n_in)
    assert got.dtype == np.float32
    assert np.array_equal(got.view(np.uint32), ref.T.view(np.uint32))


@pytest.mark.parametrize("kind", ["asym", "rtn"])
@pytest.mark.parametrize("rank,d", [(96, 2048), (64, 2560), (256, 2048)])
def test_up_layout_reproduces_dequant(kind, rank, d):
    qt = (_asym if kind == "asym" else _rtn)((rank, d), rank + 1)
    assert lora_codes_ok(qt, 16, lambda c: c == d)
    lay = lora_up_device(qt.codes.numpy(), tuple(qt.shape), **_fields(qt))
    assert lay["q"].shape == (d // 64, rank // 16, 64, 16)
    ref = cr.dequant_qt(qt)
    got = _weights_up(lay, rank, d)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_ineligible_factors():
    w = torch.randn(2048, 96)
    # blocks of 32 ranks, SpQR outliers, ranks off the 16-row blocks
    assert not lora_codes_ok(writer.pack_asym("k", "w_lora", 6, w, 32), 1,
                             lambda c: True)
    c, s, oi, ov = writer.rtn_quantize_outliers(w, 8, 0.01)
    assert not lora_codes_ok(writer.make_rtn("k", "g_lora", 8, w.shape, c, s,
                                             oi, ov), 1, lambda c: True)
    assert not lora_codes_ok(_asym((72, 2048), 3), 16, lambda c: True)
