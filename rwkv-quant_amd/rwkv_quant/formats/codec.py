"""Torch-free `.rwkvq` container and bit-layout code (numpy only).

The on-disk layout is the reference's and must stay byte-identical:

  container  safetensors: u64 LE header length, JSON header
             {name: {dtype, shape, data_offsets}, "__metadata__":
             {"rwkvq": <manifest JSON>}}, then raw buffers named
             "<state_dict key>::<field>"            (reference: codec.py:462-511)
  sb6        gs=32 blocks, sb=8 blocks per superblock, bits 4/5/6:
             codes_packed u8[OUT, IN/2]  block-local nibble split,
                          byte j of a block = q[j] | q[j+16] << 4
             gw_qh / gw_qh2 u8[OUT, IN/8]  bit 4 / bit 5 planes,
                          bit (c%8) of byte c/8 = column c
             gw_qsqm u8[OUT, NSB, 12]  pack6(qs[8]) ++ pack6(qm[8] + 31)
             gw_d / gw_dm f16[OUT, NSB]            (reference: codec.py:183-216)
  sym        gs=16, sb=16, bits 6/8 (Q6_K style, signed codes, no min):
             bits 8: codes i8[OUT, IN]
             bits 6: u = q + 32 packed like sb6 but with 16-wide blocks
             gw_qs i8[OUT, IN/16], gw_d f16[OUT, IN/256]
                                                   (reference: codec.py:219-257)
  asym       codes u8[OUT, IN], gw_scale / gw_min f32[OUT, ceil(IN/gs)]
                                                   (reference: codec.py:260-276)
  rtn        per-row: codes i8 (bits >= 5) or biased split nibbles
             (bits <= 4), scale f16[rows, 1], optional sparse outliers
                                                   (reference: codec.py:81-105,
                                                    279-292)

This module packs, unpacks and reads; it does not dequantize.  The device
kernels dequantize (rwkv_quant.backends.hip); the CPU restatement used as
the test oracle lives outside the product package.
"""
import json
import mmap as _mmap
import re

import numpy as np

FORMAT = "rwkvq"
FORMAT_VERSION = 2
MAGIC_ZIP = b"PK\x03\x04"          # torch.save zip container (legacy)

_RAW_LORA_WORLD = re.compile(r"^blocks\.\d+\.att\.[wavg][12]$")

_ST_DTYPE = {
    "BOOL": np.bool_, "U8": np.uint8, "I8": np.int8, "I16": np.int16,
    "U16": np.uint16, "F16": np.float16, "BF16": np.uint16,
    "I32": np.int32, "U32": np.uint32, "F32": np.float32,
    "F64": np.float64, "I64": np.int64, "U64": np.uint64,
}


# ------------------------------------------------------------ bit packing

def pack_int4(codes):
    """int8 [rows, cols] in [-8, 7] -> u8 [rows, ceil(cols/2)]; nibble holds
    code + 8, low nibble of byte i is column i, high nibble is column
    i + ceil(cols/2)  (reference: codec.py:81-96)."""
    codes = np.asarray(codes)
    assert codes.dtype == np.int8
    rows, cols = codes.shape
    if cols % 2:
        codes = np.concatenate([codes, np.zeros((rows, 1), np.int8)], axis=1)
    u = (codes.astype(np.int16) + 8).astype(np.uint8)
    half = u.shape[1] // 2
    return (u[:, :half] | (u[:, half:] << 4)).astype(np.uint8)


def unpack_int4(packed, n_cols):
    packed = np.asarray(packed)
    lo = (packed & 0xF).astype(np.int16) - 8
    hi = (packed >> 4).astype(np.int16) - 8
    return np.ascontiguousarray(
        np.concatenate([lo, hi], axis=1).astype(np.int8)[:, :n_cols])


def pack6(v):
    """Values 0..63, last dim % 4 == 0 -> 3 bytes per 4 values, LSB-first
    bit stream  (reference: codec.py:110-119)."""
    v = np.asarray(v)
    assert v.dtype == np.uint8 and v.shape[-1] % 4 == 0
    x = v.astype(np.uint32).reshape(v.shape[:-1] + (-1, 4))
    word = x[..., 0] | (x[..., 1] << 6) | (x[..., 2] << 12) | (x[..., 3] << 18)
    out = np.stack([word & 0xFF, (word >> 8) & 0xFF, (word >> 16) & 0xFF],
                   axis=-1)
    return out.reshape(v.shape[:-1] + (-1,)).astype(np.uint8)


def unpack6(b, n):
    b = np.asarray(b)
    assert b.dtype == np.uint8 and b.shape[-1] % 3 == 0
    x = b.astype(np.uint32).reshape(b.shape[:-1] + (-1, 3))
    word = x[..., 0] | (x[..., 1] << 8) | (x[..., 2] << 16)
    out = np.stack([(word >> s) & 0x3F for s in (0, 6, 12, 18)], axis=-1)
    return out.reshape(b.shape[:-1] + (-1,))[..., :n].astype(np.uint8)


def pack_nib_block(q, gs=32):
    """Unsigned 0..15 codes [OUT, IN] -> u8 [OUT, IN/2] with the block-local
    split: inside each gs-block, byte j = q[j] | q[j + gs/2] << 4
    (reference: codec.py:136-146)."""
    q = np.asarray(q)
    assert q.dtype == np.uint8
    n_out, n_in = q.shape
    assert n_in % gs == 0
    h = gs // 2
    qb = q.reshape(n_out, n_in // gs, 2, h)
    return np.ascontiguousarray(
        (qb[:, :, 0] | (qb[:, :, 1] << 4)).reshape(n_out, n_in // 2)
        .astype(np.uint8))


def unpack_nib_block(p, gs=32):
    p = np.asarray(p)
    n_out, hb = p.shape
    h = gs // 2
    pb = p.reshape(n_out, hb // h, 1, h)
    return np.ascontiguousarray(
        np.concatenate([pb & 0xF, pb >> 4], axis=2).reshape(n_out, hb * 2))


def pack_bitplane(bit):
    """{0,1} [OUT, IN] -> u8 [OUT, IN/8], bit (c % 8) of byte c // 8 is
    column c  (reference: codec.py:162-169)."""
    bit = np.asarray(bit).astype(np.uint8)
    n_out, n_in = bit.shape
    assert n_in % 8 == 0
    return np.packbits(bit.reshape(n_out, n_in // 8, 8), axis=-1,
                       bitorder="little").reshape(n_out, n_in // 8)


def unpack_bitplane(p, n_cols):
    p = np.asarray(p)
    return np.ascontiguousarray(
        np.unpackbits(p[..., None], axis=-1, bitorder="little")
        .reshape(p.shape[0], -1)[:, :n_cols])


def bf16_to_f32(u16):
    return (np.asarray(u16).astype(np.uint32) << 16).view(np.float32)


# -------------------------------------------------------------- container

def read_safetensors(path):
    """(metadata, {name: read-only ndarray view on an mmap})."""
    with open(path, "rb") as f:
        head8 = f.read(8)
        if head8[:4] == MAGIC_ZIP:
            raise ValueError(f"{path}: pickle (torch.save) container, not "
                             f"safetensors; re-save it as .rwkvq v2")
        n = int.from_bytes(head8, "little")
        header = json.loads(f.read(n))
        mm = _mmap.mmap(f.fileno(), 0, access=_mmap.ACCESS_READ)
    buf = np.frombuffer(mm, dtype=np.uint8)
    base = 8 + n
    meta = header.pop("__metadata__", {})
    arrays = {}
    for name, info in header.items():
        b, e = info["data_offsets"]
        dt = _ST_DTYPE[info["dtype"]]
        shape = tuple(info["shape"])
        a = buf[base + b:base + e]
        arrays[name] = a.view(dt).reshape(shape) if a.size else \
            np.empty(shape, dt)
    return meta, arrays


def check_manifest(manifest, path="<rwkvq>"):
    if manifest.get("format") != FORMAT:
        raise ValueError(f"{path}: format {manifest.get('format')!r}, "
                         f"expected {FORMAT!r}")
    if manifest.get("format_version", 0) > FORMAT_VERSION:
        raise ValueError(f"{path}: format_version "
                         f"{manifest['format_version']} is newer than "
                         f"{FORMAT_VERSION}")
    return manifest


def open_rwkvq(path):
    """(manifest, buffers) of a `.rwkvq` file  (reference: codec.py:496-511)."""
    meta, arrays = read_safetensors(path)
    if "rwkvq" not in meta:
        raise ValueError(f"{path}: not a .rwkvq (no rwkvq manifest)")
    return check_manifest(json.loads(meta["rwkvq"]), path), arrays


def is_raw_lora_world(key):
    return _RAW_LORA_WORLD.match(key) is not None


def is_transposed(manifest, key):
    """World checkpoints store LoRA w/a/v/g 1/2 as [in, out]: dequantize
    first, transpose after  (reference: codec.py:514-535)."""
    m = manifest["tensors"][key]
    if "transposed" in m:
        return bool(m["transposed"])
    return is_raw_lora_world(key) and manifest.get("naming") == "world"


# ------------------------------------------------ relayouts for consumers

def pack_mlx_affine(codes, bits):
    """Codes [..., 32] (0 .. 2^bits - 1) -> u32 [..., bits]: the 32 codes of
    a group as one LSB-first bit stream of 32 * bits bits (code p occupies
    stream bits p*bits .. p*bits + bits - 1, crossing word boundaries), the
    container of MLX's affine `quantized_matmul` with group size 32
    (reference: codec.py:313-329)."""
    codes = np.asarray(codes)
    if codes.shape[-1] != 32:
        raise ValueError("MLX affine groups hold 32 codes")
    lead = codes.shape[:-1]
    c = codes.astype(np.uint32).reshape(-1, 32, 1)
    planes = ((c >> np.arange(bits, dtype=np.uint32)) & 1).astype(np.uint8)
    stream = np.packbits(planes.reshape(-1, 32 * bits), axis=-1,
                         bitorder="little")            # [G, 4 * bits] bytes
    words = stream.view("<u4").astype(np.uint32)
    return words.reshape(lead + (bits,))


def unpack_mlx_affine(words, bits, nb):
    """u32 [..., nb * bits] -> codes [..., nb, 32] (inverse of
    pack_mlx_affine; reference: codec.py:332-346)."""
    w = np.ascontiguousarray(np.asarray(words, dtype=np.uint32))
    lead = w.shape[:-1]
    stream = w.reshape(-1, bits).astype("<u4").view(np.uint8)
    planes = np.unpackbits(stream, axis=-1, bitorder="little")
    planes = planes.reshape(-1, 32, bits).astype(np.uint32)
    codes = (planes << np.arange(bits, dtype=np.uint32)).sum(-1)
    return codes.astype(np.uint32).reshape(lead + (nb, 32))


def _sb6_codes_scales(codes_packed, qsqm, d, dm, shape, gs, sb, nb, qh, qh2):
    """Unsigned codes [OUT, IN] and the per-block fp32 scale / min of an
    sb6 tensor, exactly as the format's dequant forms them:
    s = max(f32(f16(qs * d)), 1e-8), m = f32(f16(qm * dm))."""
    OUT, IN = shape
    NB = IN // gs if nb is None else nb
    q = unpack_nib_block(codes_packed, gs).astype(np.uint32)
    if qh is not None:
        q += unpack_bitplane(qh, IN).astype(np.uint32) << 4
    if qh2 is not None:
        q += unpack_bitplane(qh2, IN).astype(np.uint32) << 5
    qsqm = np.asarray(qsqm)
    qs = unpack6(qsqm[..., :6], 8).reshape(OUT, NB).astype(np.float32)
    qm = unpack6(qsqm[..., 6:], 8).reshape(OUT, NB).astype(np.float32) - 31
    dd = np.repeat(np.asarray(d).astype(np.float32), sb, axis=1)
    ddm = np.repeat(np.asarray(dm).astype(np.float32), sb, axis=1)
    s = np.maximum((qs * dd).astype(np.float16).astype(np.float32),
                   np.float32(1e-8))
    m = (qm * ddm).astype(np.float16)
    return q, s, m, NB


def sb6_to_mlx_affine(codes_packed, qsqm, d, dm, *, shape, gs, sb, nb=None,
                      qh=None, qh2=None):
    """sb6 -> (wq u32 [OUT, NB*bits], scales f16 [OUT, NB], biases f16
    [OUT, NB], bits) for an affine w = q * scale + bias consumer with
    group 32.  The codes are moved, not requantized; scale and bias are the
    format's own per-block values, which are fp16 by construction.  The one
    difference: a block whose scale is the 1e-8 clamp stores scale 0
    (1e-8 is below fp16's smallest subnormal), off by at most 63e-8
    (reference: codec.py:349-387)."""
    if gs != 32:
        raise ValueError(f"the affine relayout takes gs 32, not {gs}")
    OUT, IN = shape
    bits = 4 + (qh is not None) + (qh2 is not None)
    q, s, m, NB = _sb6_codes_scales(codes_packed, qsqm, d, dm, shape, gs, sb,
                                    nb, qh, qh2)
    wq = pack_mlx_affine(q.reshape(OUT, NB, gs), bits).reshape(OUT, NB * bits)
    return wq, s.astype(np.float16), m, bits


def sb6_to_k3(codes_packed, qsqm, d, dm, *, shape, gs, sb, nb=None, qh=None,
              qh2=None):
    """sb6 -> (qblk, qsqm_k3, ddm, xbits), the block-interleaved layout of
    the reference's Metal loader (reference: codec.py:390-435):
      qblk[row]    per block: 16 nibble bytes [+ 4 bytes qh] [+ 4 bytes qh2]
      qsqm_k3[row] per block: qs, qm as int8 (the +31 bias removed)
      ddm[row]     per superblock: d, dm (fp16)
    A byte permutation plus the qs/qm widening (2 bytes per block against
    1.5)."""
    if gs != 32:
        raise ValueError(f"the K3 layout takes gs 32, not {gs}")
    OUT, IN = shape
    NB = IN // gs if nb is None else nb
    blocks = [np.asarray(codes_packed).reshape(OUT, NB, 16)]
    for plane in (qh, qh2):
        if plane is not None:
            blocks.append(np.asarray(plane).reshape(OUT, NB, 4))
    qblk = np.concatenate(blocks, axis=2).reshape(OUT, -1)
    qsqm = np.asarray(qsqm)
    qs = unpack6(qsqm[..., :6], 8).reshape(OUT, NB)
    qm = (unpack6(qsqm[..., 6:], 8).reshape(OUT, NB).astype(np.int8)
          - np.int8(31))
    qsqm_k3 = np.empty((OUT, NB, 2), np.uint8)
    qsqm_k3[..., 0] = qs
    qsqm_k3[..., 1] = qm.view(np.uint8)
    ddm = np.empty((OUT, np.asarray(d).shape[1], 2), np.float16)
    ddm[..., 0] = d
    ddm[..., 1] = dm
    return (np.ascontiguousarray(qblk), qsqm_k3.reshape(OUT, -1),
            ddm.reshape(OUT, -1), len(blocks) - 1)
