"""Real quantization + `.rwkvq` writing.

`quantize_tensor` picks the layout a tensor gets from its group and the
`QuantConfig`, quantizes it with `calibration.groupwise` (or per-row RTN)
and packs the parts into the on-disk fields; `save_rwkvq` writes the
safetensors container with manifest v2.  Dispatch, packing and manifest
follow the reference  (reference: rwkv_quant/formats/writer.py:82-142,
145-155, 236-337, 361-454).
"""
import json

import numpy as np
import torch

from ..calibration import groupwise as _gw
from ..calibration.group_config import QuantConfig
from . import codec
from .schema import QuantizedCheckpoint, QuantizedTensor

# group -> key patterns (reference: calibration/outlier_scan.py:15-29)
GROUP_KEY_PATTERNS = {
    "proj": ["r_proj.weight", "k_proj.weight", "v_proj.weight",
             "o_proj.weight", "att.receptance.weight", "att.key.weight",
             "att.value.weight", "att.output.weight"],
    "w_lora": ["w_lora_A", "w_lora_B", ".w0", ".w1", ".w2"],
    "a_lora": ["a_lora_A", "a_lora_B", ".a0", ".a1", ".a2"],
    "v_lora": ["v_lora_A", "v_lora_B", ".v0", ".v1", ".v2"],
    "g_lora": ["g_lora_A", "g_lora_B", ".g1", ".g2"],
    "small": ["k_k", "k_a", "r_k"],
    "cmix": ["cmix.key.weight", "cmix.value.weight", "ffn.key.weight",
             "ffn.value.weight"],
    "emb": ["emb.weight"],
    "head": ["head.weight"],
}
# LoRA bias terms are never quantized (reference: outlier_scan.py:43-44)
LORA_BIAS_SUFFIXES = (".w_lora_B.bias", ".a_lora_B.bias", ".v_lora_B.bias",
                      ".w0", ".a0", ".v0")

TENSOR_FIELDS = ("codes", "codes_packed", "scale", "dense",
                 "outlier_indices", "outlier_values",
                 "gw_d", "gw_dm", "gw_qsqm", "gw_qh", "gw_qh2", "gw_scale",
                 "gw_min", "gw_qs")


def _np(t):
    return t.detach().cpu().contiguous().numpy()


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a))


# ------------------------------------------------------------------ packers

def pack_sb6(key, group, bits, w, gs=32, search=True, ex2=None):
    """sb6 layout: nibbles + 0..2 bit planes + 6-bit qs/qm against fp16
    d/dm per superblock of 8 blocks  (reference: writer.py:236-269)."""
    assert bits in (4, 5, 6)
    n_out, n_in = w.shape
    assert n_in % gs == 0, f"{key}: IN={n_in} not a multiple of gs={gs}"
    assert (n_in // gs) % 8 == 0, f"{key}: NB={n_in // gs} not a multiple of 8"
    p = _gw.groupwise_fake_dequant(w, bits, gs, sb=8,
                                   sb_bits=(-6 if search else 6), ex2=ex2,
                                   return_parts=True)
    q = _np(p["q"])
    qs = _np(p["qs"]).reshape(n_out, -1, 8)
    qm = (_np(p["qm"]).astype(np.int16) + 31).astype(np.uint8) \
        .reshape(n_out, -1, 8)
    qsqm = np.concatenate([codec.pack6(qs), codec.pack6(qm)], axis=-1)
    qh = codec.pack_bitplane((q >> 4) & 1) if bits >= 5 else None
    qh2 = codec.pack_bitplane((q >> 5) & 1) if bits >= 6 else None
    return QuantizedTensor(
        key=key, group=group, bits=bits, shape=(n_out, n_in),
        codes_packed=_t(codec.pack_nib_block(q & 0xF, gs)),
        gw_mode="sb6", gw_gs=gs, gw_sb=8,
        gw_d=p["d"].contiguous(), gw_dm=p["dm"].contiguous(),
        gw_qsqm=_t(qsqm),
        gw_qh=None if qh is None else _t(qh),
        gw_qh2=None if qh2 is None else _t(qh2))


def pack_sym(key, group, bits, w, gs=16, sb=16, search=True, ex2=None):
    """Q6_K-style symmetric layout; bits 8 keep signed bytes, bits 6 store
    q + 32 as block-local nibbles + two bit planes
    (reference: writer.py:272-323)."""
    assert bits in (6, 8), f"{key}: sym supports 6 and 8 bits, not {bits}"
    n_out, n_in = w.shape
    assert n_in % (gs * sb) == 0, \
        f"{key}: IN={n_in} not a multiple of the superblock {gs * sb}"
    p = _gw.groupwise_sym_fake_dequant(w, bits, gs=gs, sb=sb, ex2=ex2,
                                       search=search, return_parts=True)
    q = _np(p["q"])
    codes = codes_packed = qh = qh2 = None
    if bits == 8:
        codes = _t(q)
    else:
        u = (q.astype(np.int16) + 32).astype(np.uint8)
        qh = _t(codec.pack_bitplane((u >> 4) & 1))
        qh2 = _t(codec.pack_bitplane((u >> 5) & 1))
        codes_packed = _t(codec.pack_nib_block(u & 0xF, gs))
    return QuantizedTensor(
        key=key, group=group, bits=bits, shape=(n_out, n_in),
        codes=codes, codes_packed=codes_packed, gw_mode="sym", gw_gs=gs,
        gw_sb=sb, gw_qs=p["qs"].contiguous(), gw_d=p["d"].contiguous(),
        gw_qh=qh, gw_qh2=qh2)


def pack_asym(key, group, bits, w, gs):
    """Block-asym (LoRA): unsigned codes in a byte container, fp32
    scale/min per block, ceil(IN/gs) blocks  (reference: writer.py:326-337)."""
    n_out, n_in = w.shape
    p = _gw.groupwise_fake_dequant(w, bits, gs, return_parts=True)
    return QuantizedTensor(
        key=key, group=group, bits=bits, shape=(n_out, n_in),
        codes=p["q"].contiguous(), gw_mode="asym", gw_gs=gs,
        gw_scale=p["scale"].squeeze(-1).float().contiguous(),
        gw_min=p["mn"].squeeze(-1).float().contiguous())


def rtn_quantize(w, bits):
    """Per-row symmetric RTN: (codes int8, scale fp16 [rows, 1])
    (reference: writer.py:145-155)."""
    w32 = w.float()
    qmax = 2 ** (bits - 1) - 1
    if w32.dim() >= 2:
        amax = w32.abs().amax(dim=tuple(range(1, w32.dim())),
                              keepdim=True).clamp_min(1e-8)
    else:
        amax = w32.abs().amax().clamp_min(1e-8)
    scale = amax / qmax
    codes = torch.clamp(torch.round(w32 / scale), -qmax - 1, qmax) \
        .to(torch.int8)
    return codes, scale.to(torch.float16)


def rtn_quantize_outliers(w, bits, outlier_frac):
    """SpQR-style per-row RTN: the top-|w| columns of each row are stored
    exactly in a sparse list and get code 0  (reference: writer.py:158-180)."""
    w32 = w.float()
    k = max(1, int(round(w32.shape[1] * outlier_frac)))
    aw = w32.abs()
    kth = torch.topk(aw, k, dim=1, largest=True).values[:, -1:] \
        .clamp_min(1e-8)
    mask = aw >= kth
    body = torch.where(mask, torch.zeros_like(w32), w32)
    qmax = 2 ** (bits - 1) - 1
    scale = body.abs().amax(dim=1, keepdim=True).clamp_min(1e-8) / qmax
    codes = torch.clamp(torch.round(body / scale), -qmax - 1, qmax) \
        .to(torch.int8)
    codes = torch.where(mask, torch.zeros_like(codes), codes)
    rows, cols = torch.where(mask)
    return (codes, scale.to(torch.float16),
            torch.stack([rows, cols], dim=1).to(torch.int32),
            w32[rows, cols].to(torch.bfloat16))


def make_rtn(key, group, bits, shape, codes, scale, oi=None, ov=None):
    if bits <= 4:
        return QuantizedTensor(key=key, group=group, bits=bits,
                               shape=tuple(shape),
                               codes_packed=_t(codec.pack_int4(_np(codes))),
                               scale=scale, outlier_indices=oi,
                               outlier_values=ov)
    return QuantizedTensor(key=key, group=group, bits=bits,
                           shape=tuple(shape), codes=codes, scale=scale,
                           outlier_indices=oi, outlier_values=ov)


# ----------------------------------------------------------------- dispatch

def match_group(key):
    for group, pats in GROUP_KEY_PATTERNS.items():
        if any(key.endswith(p) or p in key for p in pats):
            return group
    return None


def _dense(key, group, w):
    return QuantizedTensor(key=key, group=group or "other", bits=16,
                           shape=tuple(w.shape),
                           dense=w.to(torch.bfloat16).clone().contiguous())


def quantize_tensor(key, w, cfg: QuantConfig, real_gw=True):
    """One state_dict entry -> QuantizedTensor in the layout `cfg` assigns
    (reference: writer.py:372-454).  Only real packing is implemented: the
    fake-quant measurement mode belongs to calibration."""
    if not real_gw:
        raise NotImplementedError("fake-quant output is a calibration tool")
    group = match_group(key)
    if group is None or w.dim() < 2 or key.endswith(LORA_BIAS_SUFFIXES):
        return _dense(key, group, w)
    bits = cfg.bits[group]
    for pat, b in cfg.bits_overrides.items():
        if pat in key:
            bits = b
            break
    sp = cfg.act_stats_path
    gs = cfg.group_scale.get(group)
    if gs and bits < 16:
        mode = cfg.group_scale_mode.get(group, "asym")
        if mode in ("asym_sb6", "asym_sb6_search", "asym_sb6_aw") \
                and bits in (4, 5, 6):
            ex2 = _gw.get_ex2(sp, key, w) if mode == "asym_sb6_aw" else None
            return pack_sb6(key, group, bits, w, gs,
                            search=(mode != "asym_sb6"), ex2=ex2)
        if mode.startswith("sym") and bits in (6, 8):
            if cfg.outlier_fracs.get(group, 0.0):
                raise NotImplementedError(
                    f"sym stores no outliers, but group {group} has "
                    f"outlier_frac={cfg.outlier_fracs[group]} ({key})")
            ex2 = _gw.get_ex2(sp, key, w) if mode.endswith("_aw") else None
            return pack_sym(key, group, bits, w, gs, max(1, 256 // gs),
                            search=not mode.endswith("_plain"), ex2=ex2)
        if mode == "asym" and 5 <= bits <= 8:
            return pack_asym(key, group, bits, w, gs)
        raise NotImplementedError(f"real_gw: mode={mode} bits={bits} ({key})")
    if bits >= 16:
        return _dense(key, group, w)
    if group in cfg.outlier_fracs:
        codes, scale, oi, ov = rtn_quantize_outliers(
            w, bits, cfg.outlier_fracs[group])
        return make_rtn(key, group, bits, w.shape, codes, scale, oi, ov)
    codes, scale = rtn_quantize(w, bits)
    return make_rtn(key, group, bits, w.shape, codes, scale)


def _n_blocks(qt):
    if qt.gw_mode == "sb6":
        return int(qt.gw_qsqm.shape[-2]) * int(qt.gw_sb)
    if qt.gw_mode == "asym":
        return int(qt.gw_scale.shape[-1])
    if qt.gw_mode == "sym":
        return int(qt.gw_qs.shape[-1])
    return 0


def config_to_json(cfg):
    if cfg is None:
        return None
    return {"bits": dict(cfg.bits),
            "clip_percentiles": dict(cfg.clip_percentiles),
            "outlier_fracs": dict(cfg.outlier_fracs),
            "bits_overrides": dict(cfg.bits_overrides),
            "group_scale": dict(cfg.group_scale),
            "group_scale_mode": dict(cfg.group_scale_mode),
            "act_stats_path": cfg.act_stats_path}


def save_rwkvq(ckpt: QuantizedCheckpoint, output_path, config=None,
               tokenizer=None):
    """QuantizedCheckpoint -> `.rwkvq` (safetensors + manifest v2)
    (reference: writer.py:82-142)."""
    tensors, manifest_t = {}, {}
    for key, qt in ckpt.tensors.items():
        fields = []
        for f in TENSOR_FIELDS:
            v = getattr(qt, f, None)
            if v is None or v.numel() == 0:
                continue
            tensors[f"{key}::{f}"] = v.detach().contiguous()
            fields.append(f)
        manifest_t[key] = {
            "kind": qt.kind,
            "shape": [int(x) for x in qt.shape],
            "bits": int(qt.bits),
            "group": qt.group or "other",
            "gw_gs": int(qt.gw_gs), "gw_sb": int(qt.gw_sb),
            "n_blocks": _n_blocks(qt),
            "transposed": (ckpt.naming == "world"
                           and codec.is_raw_lora_world(key)),
            "fields": fields,
        }
    config = config if config is not None else ckpt.config
    manifest = {
        "format": codec.FORMAT, "format_version": codec.FORMAT_VERSION,
        "naming": ckpt.naming, "n_layer": int(ckpt.n_layer),
        "n_embd": int(ckpt.n_embd), "head_size": int(ckpt.head_size),
        "vocab_size": int(ckpt.vocab_size),
        "config_repr": ckpt.config_repr,
        "config": config_to_json(config),
        "tokenizer": tokenizer if tokenizer is not None else ckpt.tokenizer,
        "tensors": manifest_t,
    }
    from safetensors.torch import save_file
    save_file(tensors, output_path, metadata={"rwkvq": json.dumps(manifest)})
    return ckpt


def quantize_state_dict(state_dict, config, *, naming, n_layer, n_embd,
                        head_size, vocab_size):
    """state_dict -> QuantizedCheckpoint in memory (no file)."""
    tensors = {k: quantize_tensor(k, w, config) for k, w in state_dict.items()}
    return QuantizedCheckpoint(naming=naming, n_layer=n_layer,
                               n_embd=n_embd, head_size=head_size,
                               vocab_size=vocab_size, tensors=tensors,
                               config_repr=repr(config), config=config)
