"""CPU checks that pin the forward oracle (oracle/rwkv7_ref.py) without
retyping its formulas: streaming invariants, a closed-form special case of
the recurrence, the decay identity and a brute-force recurrence."""
import numpy as np
import pytest
import torch

from oracle.rwkv7_ref import RWKV7Oracle, wkv7
from rwkv_quant.models.synthetic import quantized_model, lora_ranks


def _rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape)


def test_wkv_reduces_to_linear_attention_when_w1_a0_b0():
    """w = 1, a = b = 0: S_t = sum_{s<=t} v_s k_s^T, y_t = S_t r_t."""
    B, T, H, N = 2, 7, 3, 8
    r, k, v = _rand((B, T, H, N), 1), _rand((B, T, H, N), 2), \
        _rand((B, T, H, N), 3)
    z = np.zeros((B, T, H, N))
    y, S = wkv7(r, np.ones_like(r), k, v, z, z, np.zeros((B, H, N, N)))
    for t in range(T):
        St = np.einsum("bshi,bshj->bhij", v[:, :t + 1], k[:, :t + 1])
        assert np.allclose(y[:, t], np.einsum("bhij,bhj->bhi", St, r[:, t]))
    assert np.allclose(S, np.einsum("bshi,bshj->bhij", v, k))


def test_wkv_matches_scalar_brute_force():
    B, T, H, N = 1, 5, 2, 4
    rs = [_rand((B, T, H, N), s) for s in range(6)]
    r, k, v, a, b = rs[:5]
    w = 1.0 / (1.0 + np.exp(-rs[5]))
    S0 = _rand((B, H, N, N), 9)
    y, S = wkv7(r, w, k, v, a, b, S0)
    St = S0.copy()
    for t in range(T):
        for h in range(H):
            for i in range(N):
                sa = sum(St[0, h, i, j] * a[0, t, h, j] for j in range(N))
                for j in range(N):
                    St[0, h, i, j] = (St[0, h, i, j] * w[0, t, h, j]
                                      + sa * b[0, t, h, j]
                                      + v[0, t, h, i] * k[0, t, h, j])
                yy = sum(St[0, h, i, j] * r[0, t, h, j] for j in range(N))
                assert abs(yy - y[0, t, h, i]) < 1e-10
    assert np.allclose(S, St)


def test_decay_identity():
    """exp(-exp(-softplus(-z) - 0.5)) == exp(-e^-0.5 * sigmoid(z)), the
    two forms used by the reference forward and the inference model."""
    z = np.linspace(-20, 20, 4001)
    lhs = np.exp(-np.exp(-np.logaddexp(0.0, -z) - 0.5))
    rhs = np.exp(-0.606531 * (1.0 / (1.0 + np.exp(-z))))
    assert np.max(np.abs(lhs - rhs)) < 1e-6


def test_lora_rank_formula_matches_reference_shapes():
    assert lora_ranks(2048) == {"w": 96, "a": 96, "v": 64, "g": 256}
    assert lora_ranks(2560) == {"w": 96, "a": 96, "v": 64, "g": 320}


@pytest.fixture(scope="module")
def toy():
    ck = quantized_model("compression", n_layer=2, n_embd=256, vocab=512,
                         seed=3)
    return RWKV7Oracle(ck)


def test_streaming_token_by_token_equals_whole_sequence(toy):
    """reference: tests/test_streaming_inference.py:46-82"""
    idx = np.random.default_rng(5).integers(0, 512, size=(2, 6))
    full, st_full = toy.forward_stateful(idx, toy.init_state(2))
    st = toy.init_state(2)
    outs = []
    for t in range(6):
        o, st = toy.forward_stateful(idx[:, t:t + 1], st)
        outs.append(o)
    step = np.concatenate(outs, axis=1)
    assert np.allclose(full, step, rtol=1e-10, atol=1e-10)
    for (a, b, c), (d, e, f) in zip(st_full, st):
        assert np.allclose(a, d) and np.allclose(b, e) and np.allclose(c, f)


def test_chunked_prefill_equals_whole(toy):
    idx = np.random.default_rng(6).integers(0, 512, size=(1, 9))
    full, _ = toy.forward_stateful(idx, toy.init_state(1))
    a, st = toy.forward_stateful(idx[:, :4], toy.init_state(1))
    b, _ = toy.forward_stateful(idx[:, 4:], st)
    assert np.allclose(full, np.concatenate([a, b], axis=1), atol=1e-10)
