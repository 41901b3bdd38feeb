"""Types that cross the format/backend boundary.

Field meanings follow the reference dataclasses
(reference: rwkv_quant/formats/schema.py:45-97); buffers are torch CPU
tensors as read from the safetensors container.
"""
from dataclasses import dataclass, field

import torch


@dataclass
class QuantizedTensor:
    key: str
    group: str
    bits: int                          # 16 = stored dense as-is
    shape: tuple
    codes: torch.Tensor = None         # int8 codes (rtn bits>=5, sym@8) or
                                       # unsigned codes in int8/uint8 (asym)
    codes_packed: torch.Tensor = None  # nibbles (rtn bits<=4, sb6, sym@6)
    scale: torch.Tensor = None         # fp16 [rows, 1] per-row (rtn)
    dense: torch.Tensor = None         # bf16 as-is (bits >= 16)
    outlier_indices: torch.Tensor = None   # int32 [n, 2] (row, col)
    outlier_values: torch.Tensor = None    # bf16 [n]
    gw_mode: str = ""                  # "" | "sb6" | "asym" | "sym"
    gw_gs: int = 0
    gw_sb: int = 0
    gw_d: torch.Tensor = None          # fp16 [OUT, NSB]
    gw_dm: torch.Tensor = None         # fp16 [OUT, NSB] (sb6)
    gw_qsqm: torch.Tensor = None       # u8 [OUT, NSB, 12] (sb6)
    gw_qh: torch.Tensor = None         # u8 [OUT, IN/8] bit-4 plane
    gw_qh2: torch.Tensor = None        # u8 [OUT, IN/8] bit-5 plane
    gw_scale: torch.Tensor = None      # f32 [OUT, NB] (asym)
    gw_min: torch.Tensor = None        # f32 [OUT, NB] (asym)
    gw_qs: torch.Tensor = None         # i8 [OUT, NB] (sym)

    @property
    def kind(self):
        if self.bits >= 16:
            return "dense"
        return self.gw_mode or "rtn"


@dataclass
class QuantizedCheckpoint:
    naming: str                        # "custom" | "world"
    n_layer: int
    n_embd: int
    head_size: int
    vocab_size: int
    tensors: dict = field(default_factory=dict)
    config_repr: str = ""
    config: object = None
    tokenizer: str = None
