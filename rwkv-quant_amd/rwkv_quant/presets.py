"""The two shipped presets: bits and block layout per group
(reference: rwkv_quant/presets.py:97-135).

Activation statistics for the `_aw` modes are an offline calibration file;
when it is absent the AW modes quantize with the unweighted search, as the
reference does."""
from .calibration.group_config import QuantConfig

REDUCTION = QuantConfig(
    proj=8, cmix=6, emb=8, head=8,
    w_lora=6, a_lora=6, v_lora=6, g_lora=8, small=16,
    outlier_fracs={},
    group_scale={"proj": 16, "cmix": 16, "emb": 16, "head": 16,
                 "w_lora": 64, "a_lora": 64, "v_lora": 64},
    group_scale_mode={"proj": "sym_aw", "cmix": "sym_aw",
                      "emb": "sym_aw", "head": "sym_aw"},
    act_stats_path=None,
)

COMPRESSION = QuantConfig(
    proj=5, cmix=4, emb_head=5,
    w_lora=6, a_lora=6, v_lora=6, g_lora=8, small=16,
    outlier_fracs={},
    group_scale={"proj": 32, "cmix": 32, "emb_head": 32,
                 "w_lora": 64, "a_lora": 64, "v_lora": 64},
    group_scale_mode={"proj": "asym_sb6_aw", "cmix": "asym_sb6_aw",
                      "emb_head": "asym_sb6_aw"},
    act_stats_path=None,
)

PRESETS = {"reduction": REDUCTION, "compression": COMPRESSION}
