"""rwkv_quant with an MI355X (gfx950) HIP backend.

`rwkv_quant.backends.hip` is the sibling of the reference's Metal backend:
same QuantLinear / QuantRWKV7 interface, kernels in hand-written HIP.
Importing this package does not import torch.
"""
__version__ = "0.1.0"
