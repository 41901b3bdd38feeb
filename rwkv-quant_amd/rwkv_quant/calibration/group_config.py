"""Quantization groups of RWKV-7 parameters and `QuantConfig`.

Same groups, alias and constructor as the reference
(reference: rwkv_quant/calibration/group_config.py:34-113).
"""

GROUPS = ["proj", "w_lora", "a_lora", "v_lora", "g_lora", "small", "cmix",
          "emb", "head"]
GROUP_ALIASES = {"emb_head": ("emb", "head")}


def expand_aliases(d):
    out = {}
    for k, v in (d or {}).items():
        if k not in GROUP_ALIASES:
            out[k] = v
    for k, v in (d or {}).items():
        for g in GROUP_ALIASES.get(k, ()):
            if g not in out:
                out[g] = v
    return out


class QuantConfig:
    def __init__(self, clip_percentiles=None, outlier_fracs=None,
                 bits_overrides=None, group_scale=None, group_scale_mode=None,
                 act_stats_path=None, **bits_per_group):
        self.bits = {g: 16 for g in GROUPS}
        self.bits.update(expand_aliases(bits_per_group))
        self.clip_percentiles = expand_aliases(clip_percentiles)
        self.outlier_fracs = expand_aliases(outlier_fracs)
        self.bits_overrides = dict(bits_overrides or {})
        self.group_scale = expand_aliases(group_scale)
        self.group_scale_mode = expand_aliases(group_scale_mode)
        self.act_stats_path = act_stats_path

    def __repr__(self):
        items = [f"{g}={self.bits[g]}" for g in GROUPS]
        return "QuantConfig(" + ", ".join(items) + ")"
