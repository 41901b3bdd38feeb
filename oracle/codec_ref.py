"""TEST INFRASTRUCTURE ONLY -- CPU oracle of the `.rwkvq` dequantization.

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of
`bench.py` may import this module, and only as the checker.  The product
(rwkv-quant_amd/) never calls it.

A plain numpy restatement of the reference's normative torch-free codec,
written independently of the product's packers so that a packing mistake
on either side shows up as a mismatch:

  unpack_*        reference: rwkv_quant/formats/codec.py:99-178
  dequant_sb6     reference: codec.py:183-216
  dequant_sym     reference: codec.py:219-257
  dequant_asym    reference: codec.py:260-276
  dequant_rtn     reference: codec.py:279-292
  dequant_qt      reference: codec.py:538-571 (dispatch on kind)

How each is pinned (see tests/test_oracle_golden.py):
  * dequant_sb6 / dequant_sym(6): dequant(pack(parts)) reproduces the
    quantizer's `deq`, whose SHA-256 equals the reference's frozen digest
    (tests/fixtures/gw_golden.json, synth::* entries);
  * dequant_sym(8), dequant_rtn, dequant_asym: closed-form invariants
    (|w - deq| <= s/2 for in-range RTN, exact integer-grid reconstruction,
    byte-flip controls) -- the reference digest for plain asym is not
    reproducible on this platform, so asym's formula is pinned by the
    reconstruction identity only.

Arithmetic keeps the reference's fp16 round-trip points: the block scale is
float32(float16(qs * d)) and, for sb6, clamped below at 1e-8 in float32.
"""
import numpy as np


def _nibbles_block_local(p, gs):
    """u8 [OUT, IN/2] -> u8 codes [OUT, IN]; inside each gs-block byte j holds
    column j in its low nibble and column j + gs/2 in its high nibble."""
    p = np.asarray(p, dtype=np.uint8)
    n_out = p.shape[0]
    h = gs // 2
    nblk = p.shape[1] // h
    out = np.empty((n_out, nblk, gs), dtype=np.uint8)
    pb = p.reshape(n_out, nblk, h)
    out[:, :, :h] = pb & 0x0F
    out[:, :, h:] = pb >> 4
    return out.reshape(n_out, nblk * gs)


def _bitplane(p, n_cols):
    """u8 [OUT, IN/8] -> {0,1} [OUT, IN], column c = bit (c%8) of byte c//8."""
    p = np.asarray(p, dtype=np.uint8)
    cols = np.arange(n_cols)
    return ((p[:, cols // 8] >> (cols % 8).astype(np.uint8)) & 1) \
        .astype(np.uint8)


def _six_bit(b, n):
    """3 bytes -> 4 six-bit values, little-endian bit stream."""
    b = np.asarray(b, dtype=np.uint8).astype(np.uint32)
    t = b.reshape(b.shape[:-1] + (-1, 3))
    v = t[..., 0] + (t[..., 1] << 8) + (t[..., 2] << 16)
    vals = [(v >> (6 * i)) & 63 for i in range(4)]
    return np.stack(vals, axis=-1).reshape(b.shape[:-1] + (-1,))[..., :n]


def _f16_round(x):
    return np.asarray(x, dtype=np.float32).astype(np.float16) \
        .astype(np.float32)


def dequant_sb6(codes_packed, qsqm, d, dm, *, shape, gs=32, sb=8, qh=None,
                qh2=None, nb=None):
    n_out, n_in = shape
    nb = n_in // gs if nb is None else nb
    assert qsqm.shape[-2] * sb == nb
    q = _nibbles_block_local(codes_packed, gs).astype(np.float32)
    if qh is not None:
        q += 16.0 * _bitplane(qh, n_in)
    if qh2 is not None:
        q += 32.0 * _bitplane(qh2, n_in)
    qs = _six_bit(qsqm[..., :6], 8).reshape(n_out, nb).astype(np.float32)
    qm = _six_bit(qsqm[..., 6:], 8).reshape(n_out, nb).astype(np.float32) \
        - np.float32(31)
    dd = np.repeat(np.asarray(d, np.float32), sb, axis=1)
    ddm = np.repeat(np.asarray(dm, np.float32), sb, axis=1)
    s = np.maximum(_f16_round(qs * dd), np.float32(1e-8))
    m = _f16_round(qm * ddm)
    return (q.reshape(n_out, nb, gs) * s[:, :, None] + m[:, :, None]) \
        .reshape(n_out, n_in).astype(np.float32)


def dequant_sym(qs, d, *, shape, gs=16, sb=16, codes=None, codes_packed=None,
                qh=None, qh2=None, nb=None):
    n_out, n_in = shape
    nb = n_in // gs if nb is None else nb
    assert qs.shape[-1] == nb and np.asarray(d).shape[-1] * sb == nb
    if codes is not None:
        q = np.asarray(codes).view(np.int8).astype(np.float32)
    else:
        u = _nibbles_block_local(codes_packed, gs).astype(np.int32)
        if qh is not None:
            u += 16 * _bitplane(qh, n_in).astype(np.int32)
        if qh2 is not None:
            u += 32 * _bitplane(qh2, n_in).astype(np.int32)
        q = (u - 32).astype(np.float32)
    dd = np.repeat(np.asarray(d, np.float32), sb, axis=1)
    s = _f16_round(np.asarray(qs).view(np.int8).astype(np.float32) * dd)
    return (q.reshape(n_out, nb, gs) * s[:, :, None]).reshape(n_out, n_in) \
        .astype(np.float32)


def dequant_asym(codes, scale, mn, *, shape, gs, nb=None):
    n_out, n_in = shape
    nb = -(-n_in // gs) if nb is None else nb
    assert scale.shape[-1] == nb
    q = np.asarray(codes).view(np.uint8).astype(np.float32)
    blk = np.arange(n_in) // gs
    return (q * np.asarray(scale, np.float32)[:, blk]
            + np.asarray(mn, np.float32)[:, blk]).astype(np.float32)


def dequant_rtn(scale, *, shape, codes=None, codes_packed=None,
                outlier_indices=None, outlier_values=None):
    if codes is None:
        p = np.asarray(codes_packed, dtype=np.uint8)
        lo = (p & 0xF).astype(np.int16) - 8
        hi = (p >> 4).astype(np.int16) - 8
        codes = np.concatenate([lo, hi], axis=1)[:, :shape[1]]
    w = np.asarray(codes).astype(np.float32) * np.asarray(scale, np.float32)
    if outlier_indices is not None and len(outlier_indices):
        oi = np.asarray(outlier_indices)
        w[oi[:, 0], oi[:, 1]] = np.asarray(outlier_values, np.float32)
    return w.reshape(shape).astype(np.float32)


def _bf16_bits_to_f32(u16):
    return (np.asarray(u16).view(np.uint16).astype(np.uint32) << 16) \
        .view(np.float32)


def dequant_qt(qt):
    """QuantizedTensor (torch CPU buffers) -> float32 ndarray in its stored
    orientation."""
    def a(name):
        v = getattr(qt, name, None)
        if v is None:
            return None
        if str(v.dtype) == "torch.bfloat16":
            return _bf16_bits_to_f32(v.view(__import__("torch").int16)
                                     .numpy())
        return v.numpy()
    shape = tuple(qt.shape)
    if qt.bits >= 16:
        return a("dense").astype(np.float32).reshape(shape)
    if qt.gw_mode == "sb6":
        return dequant_sb6(a("codes_packed"), a("gw_qsqm"), a("gw_d"),
                           a("gw_dm"), shape=shape, gs=qt.gw_gs, sb=qt.gw_sb,
                           qh=a("gw_qh"), qh2=a("gw_qh2"))
    if qt.gw_mode == "sym":
        return dequant_sym(a("gw_qs"), a("gw_d"), shape=shape, gs=qt.gw_gs,
                           sb=qt.gw_sb, codes=a("codes"),
                           codes_packed=a("codes_packed"), qh=a("gw_qh"),
                           qh2=a("gw_qh2"))
    if qt.gw_mode == "asym":
        return dequant_asym(a("codes"), a("gw_scale"), a("gw_min"),
                            shape=shape, gs=qt.gw_gs)
    return dequant_rtn(a("scale"), shape=shape, codes=a("codes"),
                       codes_packed=a("codes_packed"),
                       outlier_indices=a("outlier_indices"),
                       outlier_values=a("outlier_values"))


def gemv_ref(x, w):
    """y = x . w^T in float64 (the tolerance reference for fp32 kernels)."""
    return np.asarray(x, np.float64) @ np.asarray(w, np.float64).T
