"""GPU parity of the fused decode path (LoRA up products folded into the
WKV step) on a model of the 1.5B width (D = 2048, 2 layers).

Bars: end-to-end logits within 1e-2 max-abs of the float64 oracle
with the decode LoRA read from the file's
codes (the default) and from the fp16 copies.  Fused vs the unfused launch
sequence (both on the fp16 copies): the fused kernel sums the up products
in another order, so a WKV input can move by an fp32 rounding and carry
into the later residuals and states: logits within 5e-3 max-abs, states
within 2e-3 (a wrong branch or row moves them by ~1e-1)."""
import numpy as np
import pytest
import torch

from oracle.rwkv7_ref import RWKV7Oracle
from rwkv_quant.backends.hip import quant_model as qm
from rwkv_quant.models.synthetic import quantized_model

pytestmark = pytest.mark.gpu

VOCAB = 1024


@pytest.fixture(scope="module", params=["compression", "reduction"])
def wide(request):
    ck = quantized_model(request.param, n_layer=2, n_embd=2048, vocab=VOCAB,
                         seed=21, device="cuda", to_cpu=True)
    model = qm.QuantRWKV7(ck)
    assert all(b.tmix.decode_fusable for b in model.blocks)
    assert all(b.tmix.lora_q is not None for b in model.blocks)
    return ck, RWKV7Oracle(ck), model


def _maxabs(a, b):
    return float(np.abs(np.asarray(a, np.float64) - b).max())


@pytest.mark.parametrize("B", [1, 4])
def test_fused_graph_decode_matches_oracle(wide, B):
    ck, orc, model = wide
    print(f"fused decode B={B}", flush=True)
    idx = np.random.default_rng(B).integers(0, VOCAB, size=(B, 5))
    st_o, st_m = orc.init_state(B), model.init_state(B)
    for t in range(5):
        ro, st_o = orc.forward_stateful(idx[:, t:t + 1], st_o)
        lg, st_m = model.step(torch.from_numpy(idx[:, t:t + 1]), st_m)
        assert _maxabs(lg.cpu().numpy(), ro) < 1e-2


@pytest.mark.parametrize("B", [1, 8])
def test_lora_from_codes_and_fp16_match_oracle(wide, B):
    """Eager decode steps with the LoRA from the codes and from the fp16
    copies, each against the oracle."""
    ck, orc, model = wide
    print(f"lora codes vs fp16 B={B}", flush=True)
    idx = np.random.default_rng(30 + B).integers(0, VOCAB, size=(B, 3))
    for codes in (True, False):
        qm.LORA_FROM_CODES = codes
        try:
            st_o, st_m = orc.init_state(B), model.init_state(B)
            for t in range(3):
                ro, st_o = orc.forward_stateful(idx[:, t:t + 1], st_o)
                lg, st_m = model.forward_stateful(
                    torch.from_numpy(idx[:, t:t + 1]), st_m)
                assert _maxabs(lg.cpu().numpy(), ro) < 1e-2, codes
        finally:
            qm.LORA_FROM_CODES = True


@pytest.mark.parametrize("B", [1, 3, 8])
def test_fused_equals_unfused_decode(wide, B):
    ck, orc, model = wide
    idx = torch.from_numpy(
        np.random.default_rng(10 + B).integers(0, VOCAB, size=(B, 4)))
    st_f, st_u = model.init_state(B), model.init_state(B)
    qm.LORA_FROM_CODES = False
    try:
        for t in range(4):
            qm.FUSE_DECODE = True
            lf, st_f = model.forward_stateful(idx[:, t:t + 1], st_f)
            qm.FUSE_DECODE = False
            lu, st_u = model.forward_stateful(idx[:, t:t + 1], st_u)
            qm.FUSE_DECODE = True
            d = float((lf - lu).abs().max())
            assert d < 5e-3, d
            for sf, su in zip(st_f, st_u):
                for a, b in zip(sf, su):
                    d = float((a - b).abs().max())
                    assert d < 2e-3 * max(1.0, float(b.abs().max())), d
    finally:
        qm.FUSE_DECODE = True
        qm.LORA_FROM_CODES = True
