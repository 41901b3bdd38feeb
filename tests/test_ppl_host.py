"""Host logic of the perplexity harness (CPU): the degenerate-mean guard
of the reference (calibration/ablation.py:51-69)."""
import math

import pytest

from rwkv_quant.calibration import ablation


def test_finish_is_exp_mean():
    assert abs(ablation.finish(6.0, 3) - math.exp(2.0)) < 1e-12


@pytest.mark.parametrize("total", [0.0, -1.0, float("nan"), float("inf")])
def test_finish_refuses_degenerate_mean(total):
    with pytest.raises(RuntimeError):
        ablation.finish(total, 10)
