"""Shared helpers of the test suite: seeded synthetic tensors and packing."""
import hashlib

import numpy as np
import torch

from rwkv_quant.formats import writer


def weights(rows, cols, seed=0, std=0.02, outlier_cols=0):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(rows, cols, generator=g) * std
    if outlier_cols:
        idx = torch.randperm(cols, generator=g)[:outlier_cols]
        w[:, idx] *= 20.0
    return w


def act(n, cols, seed=1, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(n, cols, generator=g).to(dtype).float()


def qt_for(kind, bits, w, search=False):
    """Pack w into one of the hot-path layouts."""
    if kind == "sb6":
        return writer.pack_sb6("t", "proj", bits, w, 32, search=search)
    if kind == "sym":
        return writer.pack_sym("t", "cmix", bits, w, 16, 16, search=search)
    if kind == "rtn":
        codes, scale = writer.rtn_quantize(w, bits)
        return writer.make_rtn("t", "head", bits, w.shape, codes, scale)
    if kind == "asym":
        return writer.pack_asym("t", "w_lora", bits, w, 64)
    raise ValueError(kind)


def digest(t, nan_bits=None):
    """sha256 of shape + dtype + raw bytes (the reference's golden digest)."""
    a = t.detach().contiguous().cpu()
    arr = a.numpy().copy()
    if nan_bits is not None and arr.dtype == np.float32:
        u = arr.view(np.uint32)
        u[np.isnan(arr)] = nan_bits
    h = hashlib.sha256()
    h.update(str(tuple(a.shape)).encode())
    h.update(str(a.dtype).encode())
    h.update(arr.tobytes())
    return h.hexdigest()


def relmax(y, ref):
    """max|y - ref| / max|ref| (reference: tests/test_gw_kernel.py:26)."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.abs(y - ref).max() / max(np.abs(ref).max(), 1e-30))
