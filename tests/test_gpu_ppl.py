"""GPU perplexity harness (reference: rwkv_quant/calibration/ablation.py:
21-69): the per-row NLL kernel against float64 logsumexp, and
perplexity() through the HIP model against the oracle's perplexity on the
same checkpoint (the oracle's perplexity is itself pinned to the
reference's on a fixture, tests/test_reference_fixtures.py)."""
import math

import numpy as np
import pytest
import torch

from oracle import rwkv7_ref as orf
from rwkv_quant.backends.hip import quant_model as qm
from rwkv_quant.calibration import ablation
from rwkv_quant.models.synthetic import quantized_model

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,V,ld,scale", [(7, 65536, 65536, 3.0),
                                             (5, 1000, 1004, 40.0),
                                             (3, 37, 40, 1.0)])
def test_nll_rows_matches_float64(rows, V, ld, scale):
    g = torch.Generator().manual_seed(V)
    buf = torch.randn(rows, ld, generator=g) * scale
    tg = torch.randint(0, V, (rows,), generator=g)
    lg = buf[:, :V]
    ref = (torch.logsumexp(lg.double(), -1)
           - lg.double().gather(-1, tg[:, None])[:, 0]).numpy()
    out = ablation.nll_rows(buf.cuda()[:, :V], tg.cuda()).cpu().numpy()
    assert np.abs(out - ref).max() < 1e-5 * max(1.0, np.abs(ref).max())


def test_nll_rows_bad_target_and_nan_give_nan():
    lg = torch.randn(3, 256).cuda()
    lg[2, 17] = float("nan")
    tg = torch.tensor([5, 256, 3]).cuda()          # 256 is out of range
    out = ablation.nll_rows(lg, tg).cpu()
    assert math.isfinite(float(out[0]))
    assert math.isnan(float(out[1])) and math.isnan(float(out[2]))


@pytest.mark.parametrize("preset", ["compression", "reduction"])
def test_perplexity_through_hip_model_matches_oracle(preset):
    ck = quantized_model(preset, n_layer=2, n_embd=256, vocab=1024, seed=17)
    model = qm.QuantRWKV7(ck)
    orc = orf.RWKV7Oracle(ck)
    data = np.random.default_rng(3).integers(0, 1024, size=(5, 24))
    p_hip = ablation.perplexity(model, torch.from_numpy(data), batch_size=2)
    p_orc = orf.perplexity(orc, data, batch_size=2)
    print(f"{preset}: hip {p_hip:.6f} oracle {p_orc:.6f}", flush=True)
    assert abs(math.log(p_hip) - math.log(p_orc)) < 1e-3


def test_perplexity_refuses_fake_quant_config():
    from rwkv_quant.presets import REDUCTION
    ck = quantized_model("reduction", n_layer=1, n_embd=256, vocab=512,
                         seed=2)
    model = qm.QuantRWKV7(ck)
    with pytest.raises(ValueError):
        ablation.perplexity(model, torch.zeros(1, 4, dtype=torch.long),
                            cfg=REDUCTION)
