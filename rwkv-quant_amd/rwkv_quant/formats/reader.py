"""`.rwkvq` -> `QuantizedCheckpoint` (reference: rwkv_quant/formats/reader.py:42-111).

Only the safetensors container is read.  The legacy pickle container would
need `torch.load(weights_only=False)`, which executes code from the file;
it is rejected with the same message the torch-free reader gives.
"""
import json

from . import codec
from .schema import QuantizedCheckpoint, QuantizedTensor


def load_raw(path):
    with open(path, "rb") as f:
        head = f.read(4)
    if head == codec.MAGIC_ZIP:
        raise ValueError(f"{path}: pickle (torch.save) container, not "
                         f"safetensors; re-save it as .rwkvq v2")
    from safetensors import safe_open
    with safe_open(path, framework="pt", device="cpu") as f:
        meta = f.metadata() or {}
        if "rwkvq" not in meta:
            raise ValueError(f"{path}: safetensors without an rwkvq manifest")
        m = codec.check_manifest(json.loads(meta["rwkvq"]), path)
        tensors = {}
        for key, t in m["tensors"].items():
            kind = t["kind"]
            qt = QuantizedTensor(
                key=key, group=t["group"], bits=t["bits"],
                shape=tuple(t["shape"]),
                gw_mode=kind if kind in ("sb6", "sym", "asym") else "",
                gw_gs=t["gw_gs"], gw_sb=t["gw_sb"])
            for field in t["fields"]:
                setattr(qt, field, f.get_tensor(f"{key}::{field}"))
            tensors[key] = qt
    return QuantizedCheckpoint(
        naming=m["naming"], n_layer=m["n_layer"], n_embd=m["n_embd"],
        head_size=m["head_size"], vocab_size=m["vocab_size"],
        tensors=tensors, config_repr=m.get("config_repr", ""),
        config=config_from_json(m.get("config")),
        tokenizer=m.get("tokenizer"))


def config_from_json(d):
    """Manifest `config` (writer.config_to_json) -> QuantConfig; None for
    files that carry none (reference: reader.py:96-111)."""
    if d is None:
        return None
    from ..calibration.group_config import QuantConfig
    return QuantConfig(
        clip_percentiles=d.get("clip_percentiles"),
        outlier_fracs=d.get("outlier_fracs"),
        bits_overrides=d.get("bits_overrides"),
        group_scale=d.get("group_scale"),
        group_scale_mode=d.get("group_scale_mode"),
        act_stats_path=d.get("act_stats_path"),
        **d.get("bits", {}))
