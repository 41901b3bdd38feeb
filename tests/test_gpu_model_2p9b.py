"""GPU parity of the HIP model at the 2.9B width (D = 2560, 40 heads of 64,
channel-mix hidden 10240, LoRA ranks 96/96/64/320; 2 layers, vocab 1024)
against the float64 oracle, on the paths configs[4] exercises: decode at
batch 1 (one-row GEMVs, fused decode step) and batch 32 (matrix-core batched
GEMVs in two 16-row launches, LoRA through the GEMM path, unfused decode
core), and a prefill long enough for the GEMM path.

Bar: end-to-end logits within 1e-2 max-abs."""
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
    ck = quantized_model(request.param, n_layer=2, n_embd=2560, ffn=10240,
                         vocab=VOCAB, seed=29, device="cuda", to_cpu=True)
    model = qm.QuantRWKV7(ck)
    assert model.n_head == 40
    return ck, RWKV7Oracle(ck), model


def _maxabs(a, b):
    return float(np.abs(np.asarray(a, np.float64) - b).max())


@pytest.mark.parametrize("B", [1, 32])
def test_decode_2p9b_matches_oracle(wide, B):
    ck, orc, model = wide
    print(f"2.9B-width decode B={B}", flush=True)
    idx = np.random.default_rng(B).integers(0, VOCAB, size=(B, 3))
    st_o, st_m = orc.init_state(B), model.init_state(B)
    for t in range(3):
        ro, st_o = orc.forward_stateful(idx[:, t:t + 1], st_o)
        lg, st_m = model.step(torch.from_numpy(idx[:, t:t + 1]), st_m)
        assert _maxabs(lg.cpu().numpy(), ro) < 1e-2


def test_prefill_2p9b_matches_oracle(wide):
    ck, orc, model = wide
    print("2.9B-width prefill T=160", flush=True)
    idx = np.random.default_rng(7).integers(0, VOCAB, size=(1, 160))
    ref, _ = orc.forward_stateful(idx, orc.init_state(1))
    out, _ = model.forward_stateful(torch.from_numpy(idx),
                                    model.init_state(1))
    assert _maxabs(out.cpu().numpy(), ref) < 1e-2
