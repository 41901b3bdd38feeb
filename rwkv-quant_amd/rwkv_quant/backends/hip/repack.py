"""Canonical `.rwkvq` fields -> device (HBM) layouts of the HIP kernels.

Every layout is a byte/bit permutation of the canonical fields with the
same byte count (nothing is recomputed, no scale is widened):

  sb6    nib  = codes_packed                         (unchanged)
         hb   = bits 5: the block's gw_qh bytes read as one u32 word
                bits 6: gw_qh/gw_qh2 bits regrouped so that the two high
                bits of the column pair that shares a nibble byte sit side
                by side ("crumbs"), which the kernel rotates into place
                with one v_alignbit_b32
         rec  = gw_qsqm (12 B) ++ gw_d (2 B) ++ gw_dm (2 B) per superblock,
                one 16-byte load
  sym    codes / codes_packed unchanged, hb crumbs as above with the
         16-wide block pairing, gw_qs and gw_d unchanged
  rtn@8  unchanged (scale flattened to [rows])
  LoRA factors of a world checkpoint, read by the decode kernels straight
  from their codes (asym gw64 or per-row int8; stored [in, out]):
    down [in, rank]  codes transposed to [rank, in]; asym scale / min to
                     [rank / 64, in]; int8 row scales [in] unchanged
    up   [rank, D]   codes permuted to [D / 64][rank / 16][64][16] (head,
                     16-row block, channel, row); asym scale / min to
                     [D / 64, rank]; int8 row scales [rank] unchanged

The reference loader performs the analogous interleave for its Metal
kernels (reference: rwkv_quant/formats/codec.py:407-435,
rwkv_quant/backends/metal/quant_linear_gw.py:755-794,
rwkv_quant/backends/metal/quant_linear_sym.py:407-431).
"""
import numpy as np

from ...formats import codec

# nibble byte i of a 32-column group holds (lo column, hi column)
SB6_PAIRS = [(i, i + 16) for i in range(16)]
SYM_PAIRS = [((i if i < 8 else i + 8), (i if i < 8 else i + 8) + 8)
             for i in range(16)]


def _planes(qh, qh2, n_out, n_in):
    b4 = codec.unpack_bitplane(np.asarray(qh), n_in).astype(np.uint32)
    b5 = codec.unpack_bitplane(np.asarray(qh2), n_in).astype(np.uint32)
    ng = n_in // 32
    return b4.reshape(n_out, ng, 32), b5.reshape(n_out, ng, 32)


def crumb_words(qh, qh2, n_out, n_in, pairs):
    """u32 [rows, IN/32, 2]: for nibble byte i of a group (i' = i % 8), bits
    (2i', 2i'+1) of word i // 8 hold code bits (4, 5) of its lo column and
    bits (16+2i', 17+2i') those of its hi column."""
    b4, b5 = _planes(qh, qh2, n_out, n_in)
    out = np.zeros((n_out, n_in // 32, 2), dtype=np.uint32)
    for i, (lo, hi) in enumerate(pairs):
        ip = i % 8
        out[:, :, i // 8] |= ((b4[:, :, lo] << (2 * ip))
                              | (b5[:, :, lo] << (2 * ip + 1))
                              | (b4[:, :, hi] << (16 + 2 * ip))
                              | (b5[:, :, hi] << (17 + 2 * ip)))
    return out


def sb6_device(codes_packed, qsqm, d, dm, *, shape, bits, qh=None, qh2=None):
    """-> dict(nib u8 [rows, NG, 16], hb u32 or None, rec u8 [rows, NSB, 16])."""
    n_out, n_in = shape
    assert n_in % 256 == 0, f"sb6 kernel: IN={n_in} is not a multiple of 256"
    ng, nsb = n_in // 32, n_in // 256
    nib = np.ascontiguousarray(np.asarray(codes_packed, np.uint8)
                               .reshape(n_out, ng, 16))
    hb = None
    if bits == 5:
        hb = np.ascontiguousarray(np.asarray(qh, np.uint8)
                                  .reshape(n_out, ng, 4)).view(np.uint32) \
            .reshape(n_out, ng)
    elif bits == 6:
        hb = crumb_words(qh, qh2, n_out, n_in, SB6_PAIRS)
    rec = np.concatenate(
        [np.asarray(qsqm, np.uint8).reshape(n_out, nsb, 12),
         np.asarray(d, np.float16).reshape(n_out, nsb, 1).view(np.uint8),
         np.asarray(dm, np.float16).reshape(n_out, nsb, 1).view(np.uint8)],
        axis=-1)
    return {"nib": nib, "hb": hb, "rec": np.ascontiguousarray(rec)}


def sym_device(qs, d, *, shape, bits, codes=None, codes_packed=None, qh=None,
               qh2=None):
    """-> dict(codes u8, hb u32 or None, qs i8 [rows, IN/16], d f16)."""
    n_out, n_in = shape
    assert n_in % 256 == 0, f"sym kernel: IN={n_in} is not a multiple of 256"
    if bits == 8:
        q = np.ascontiguousarray(np.asarray(codes).view(np.uint8)
                                 .reshape(n_out, n_in))
        hb = None
    else:
        q = np.ascontiguousarray(np.asarray(codes_packed, np.uint8)
                                 .reshape(n_out, n_in // 32, 16))
        hb = crumb_words(qh, qh2, n_out, n_in, SYM_PAIRS)
    return {"codes": q, "hb": hb,
            "qs": np.ascontiguousarray(np.asarray(qs).view(np.int8)),
            "d": np.ascontiguousarray(np.asarray(d, np.float16))}


def rtn8_device(codes, scale, *, shape):
    n_out, n_in = shape
    return {"codes": np.ascontiguousarray(np.asarray(codes).view(np.int8)
                                          .reshape(n_out, n_in)),
            "scale": np.ascontiguousarray(np.asarray(scale, np.float16)
                                          .reshape(n_out))}


def lora_codes_ok(qt, rows_mult, cols_ok):
    """True when the decode kernels can read this LoRA factor's codes:
    asym with 64-column blocks, or per-row int8 without outliers."""
    if len(qt.shape) != 2 or qt.codes is None:
        return False
    r, c = qt.shape
    if r % rows_mult or not cols_ok(c):
        return False
    if qt.gw_mode == "asym":
        return qt.gw_gs == 64 and qt.bits <= 8
    return (qt.gw_mode == "" and qt.bits == 8 and
            (qt.outlier_indices is None or qt.outlier_indices.numel() == 0))


def lora_down_device(codes, shape, *, scale=None, mn=None, row_scale=None):
    """Down factor stored [in, rank]: asym (scale / min [in, rank / 64])
    or per-row int8 (row_scale [in])."""
    n_in, rank = shape
    q = np.asarray(codes).view(np.uint8).reshape(n_in, rank)
    out = {"q": np.ascontiguousarray(q.T), "s": None, "m": None, "sc": None}
    if scale is not None:
        nb = -(-rank // 64)
        out["s"] = np.ascontiguousarray(
            np.asarray(scale, np.float32).reshape(n_in, nb).T)
        out["m"] = np.ascontiguousarray(
            np.asarray(mn, np.float32).reshape(n_in, nb).T)
    else:
        out["sc"] = np.ascontiguousarray(
            np.asarray(row_scale, np.float16).reshape(n_in).view(np.uint16))
    return out


def lora_up_device(codes, shape, *, scale=None, mn=None, row_scale=None):
    """Up factor stored [rank, D] (64-column blocks = heads): asym
    (scale / min [rank, D / 64]) or per-row int8 (row_scale [rank])."""
    rank, d = shape
    H = d // 64
    q = np.asarray(codes).view(np.uint8).reshape(rank // 16, 16, H, 64)
    out = {"q": np.ascontiguousarray(q.transpose(2, 0, 3, 1)),
           "s": None, "m": None, "sc": None}
    if scale is not None:
        out["s"] = np.ascontiguousarray(
            np.asarray(scale, np.float32).reshape(rank, H).T)
        out["m"] = np.ascontiguousarray(
            np.asarray(mn, np.float32).reshape(rank, H).T)
    else:
        out["sc"] = np.ascontiguousarray(
            np.asarray(row_scale, np.float16).reshape(rank).view(np.uint16))
    return out
