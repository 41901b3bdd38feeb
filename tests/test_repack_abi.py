"""Host-side checks: the device repack is a bit-preserving permutation of
the canonical fields, and librwkvq_hip.so exports every entry point that
include/rwkvq_hip.h declares (no device call is made)."""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

from rwkv_quant.backends.hip import _lib, repack
from rwkv_quant.formats import codec

from _util import qt_for, weights

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _unrepack_crumbs(hb, n_out, n_in, pairs):
    ng = n_in // 32
    b4 = np.zeros((n_out, ng, 32), np.uint8)
    b5 = np.zeros((n_out, ng, 32), np.uint8)
    for i, (lo, hi) in enumerate(pairs):
        H = hb[:, :, i // 8]
        ip = i % 8
        b4[:, :, lo] = (H >> (2 * ip)) & 1
        b5[:, :, lo] = (H >> (2 * ip + 1)) & 1
        b4[:, :, hi] = (H >> (16 + 2 * ip)) & 1
        b5[:, :, hi] = (H >> (17 + 2 * ip)) & 1
    return (codec.pack_bitplane(b4.reshape(n_out, n_in)),
            codec.pack_bitplane(b5.reshape(n_out, n_in)))


@pytest.mark.parametrize("bits", [4, 5, 6])
def test_sb6_repack_is_bit_preserving(bits):
    w = weights(64, 512, seed=bits)
    qt = qt_for("sb6", bits, w)
    lay = repack.sb6_device(qt.codes_packed.numpy(), qt.gw_qsqm.numpy(),
                            qt.gw_d.numpy(), qt.gw_dm.numpy(), shape=qt.shape,
                            bits=bits,
                            qh=None if qt.gw_qh is None else qt.gw_qh.numpy(),
                            qh2=None if qt.gw_qh2 is None else qt.gw_qh2.numpy())
    assert np.array_equal(lay["nib"].reshape(64, 256), qt.codes_packed.numpy())
    rec = lay["rec"]
    assert np.array_equal(rec[..., :12], qt.gw_qsqm.numpy())
    assert np.array_equal(rec[..., 12:14].copy().view(np.float16)[..., 0],
                          qt.gw_d.numpy())
    assert np.array_equal(rec[..., 14:16].copy().view(np.float16)[..., 0],
                          qt.gw_dm.numpy())
    canon = sum(getattr(qt, f).numel() * getattr(qt, f).element_size()
                for f in ("codes_packed", "gw_qsqm", "gw_d", "gw_dm", "gw_qh",
                          "gw_qh2") if getattr(qt, f) is not None)
    dev = sum(a.nbytes for a in lay.values() if a is not None)
    assert canon == dev
    if bits == 5:
        assert np.array_equal(lay["hb"].view(np.uint8).reshape(64, 64),
                              qt.gw_qh.numpy())
    if bits == 6:
        qh, qh2 = _unrepack_crumbs(lay["hb"], 64, 512, repack.SB6_PAIRS)
        assert np.array_equal(qh, qt.gw_qh.numpy())
        assert np.array_equal(qh2, qt.gw_qh2.numpy())


def test_sym6_repack_is_bit_preserving():
    w = weights(32, 768, seed=9)
    qt = qt_for("sym", 6, w)
    lay = repack.sym_device(qt.gw_qs.numpy(), qt.gw_d.numpy(), shape=qt.shape,
                            bits=6, codes_packed=qt.codes_packed.numpy(),
                            qh=qt.gw_qh.numpy(), qh2=qt.gw_qh2.numpy())
    qh, qh2 = _unrepack_crumbs(lay["hb"], 32, 768, repack.SYM_PAIRS)
    assert np.array_equal(qh, qt.gw_qh.numpy())
    assert np.array_equal(qh2, qt.gw_qh2.numpy())
    assert np.array_equal(lay["codes"].reshape(32, 384),
                          qt.codes_packed.numpy())


def _declared_symbols():
    text = open(os.path.join(ROOT, "include", "rwkvq_hip.h")).read()
    return sorted(set(re.findall(r"\bint\s+(rwkvq_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail(f"{_lib.LIB_PATH} not built")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    syms = _declared_symbols()
    assert len(syms) >= 7
    for s in syms:
        assert hasattr(lib, s), s
    # every declared symbol has a ctypes signature and vice versa
    assert set(syms) == set(_lib.SIGNATURES)


def test_persistent_decode_descriptor_layout():
    """The ctypes mirror of the persistent decode kernel's layer descriptor
    has the size the library reports (a host-only call: no device)."""
    from rwkv_quant.backends.hip.decode_mk import MkLayer
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail(f"{_lib.LIB_PATH} not built")
    lb, bw, wgs, mc = (ctypes.c_int() for _ in range(4))
    assert _lib.load().rwkvq_decode_mk_info(
        ctypes.byref(lb), ctypes.byref(bw), ctypes.byref(wgs),
        ctypes.byref(mc)) == 0
    assert lb.value == ctypes.sizeof(MkLayer)
    assert wgs.value in (256, 512)
    assert bw.value >= 2 * (wgs.value // 32) * 32 + 64
    assert mc.value >= 288        # the 1.5B shape's four LoRA ranks


def test_persistent_decode_shape_check(monkeypatch):
    """PersistentDecode's host check (no device): the 1.5B LoRA ranks pass;
    a rank above 256 (the WKV phase stages one rank position per thread)
    or more than 64 down-product workgroups is refused before anything is
    allocated."""
    from types import SimpleNamespace
    from rwkv_quant.backends.hip import decode_mk as dm
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail(f"{_lib.LIB_PATH} not built")
    monkeypatch.setattr(dm, "_fmt", lambda lin: lin)

    def model(ranks):
        tm = SimpleNamespace(rkv_fused=dm.F_SB6_5, o_proj=dm.F_SB6_5,
                             lora_q={b: (r, None, None)
                                     for b, r in zip("wavg", ranks)})
        cm = SimpleNamespace(key=dm.F_SB6_4, value=dm.F_SB6_4)
        return SimpleNamespace(n_embd=2048, ffn=8192, head_size=64,
                               blocks=[SimpleNamespace(tmix=tm, cmix=cm)])

    def why(ranks):
        pd = dm.PersistentDecode.__new__(dm.PersistentDecode)
        pd.model, pd.max_cat = model(ranks), 640
        return pd._check()

    assert why((96, 96, 64, 256)) == ""
    assert why((64, 64, 32, 320)) == "LoRA ranks"
    assert why((96, 96, 64, 40)) == "LoRA ranks"            # not % 16
    assert why((256, 256, 64, 64)) == "LoRA down rows"      # 80 workgroups
    pd = dm.PersistentDecode(model((64, 64, 32, 320)))
    assert not pd.ok and pd.why == "LoRA ranks"


def test_gather_ln_rejects_bad_arguments():
    """rwkvq_gather_ln_f32's host-side checks (no device call): widths the
    row kernel cannot hold, widths off the format's blocks, a missing index
    or LayerNorm vector, an unknown kind -> RWKVQ_ERR_ARG."""
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail(f"{_lib.LIB_PATH} not built")
    f = _lib.load().rwkvq_gather_ln_f32
    P = ctypes.c_void_p
    dummy = P(256)                         # never dereferenced: checks first

    def call(kind, bits, src_rows, width, idx, n, w, b, aux1=dummy):
        return f(kind, bits, dummy, dummy, dummy, aux1, src_rows, width, idx,
                 n, w, b, ctypes.c_float(1e-5), dummy, None)

    ERR = 1001
    assert call(0, 5, 8, 4352, dummy, 1, dummy, dummy) == ERR   # > 4096
    assert call(0, 5, 8, 2050, dummy, 1, dummy, dummy) == ERR   # % 8
    assert call(0, 5, 8, 2056, dummy, 1, dummy, dummy) == ERR   # % 256
    assert call(1, 7, 8, 2048, dummy, 1, dummy, dummy) == ERR   # sym bits
    assert call(0, 5, 8, 2048, None, 1, dummy, dummy) == ERR    # no idx
    assert call(0, 5, 8, 2048, dummy, 0, dummy, dummy) == ERR   # no rows
    assert call(0, 5, 8, 2048, dummy, 1, None, dummy) == ERR    # no weight
    assert call(2, 8, 8, 2048, dummy, 1, dummy, dummy, None) == ERR
    assert call(3, 8, 8, 2048, dummy, 1, dummy, dummy) == ERR   # kind
