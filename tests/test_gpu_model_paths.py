"""The HIP model's entry paths (reference: backends/metal/quant_model.py:
838-990): the `.rwkvq` file -> load_raw -> QuantRWKV7 path, last_only /
tail_only (the speculative-verify slice, quant_model.py:983-990),
forward_hidden, and the captured prefill graphs (shapes sharing one
activation buffer set, the LRU cache of graphs)."""
import numpy as np
import pytest
import torch

from oracle.rwkv7_ref import RWKV7Oracle
from rwkv_quant.backends.hip import _lib
from rwkv_quant.backends.hip import quant_model as qm
from rwkv_quant.formats import reader, writer
from rwkv_quant.models.synthetic import quantized_model

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def toy():
    ck = quantized_model("reduction", n_layer=2, n_embd=256, vocab=1024,
                         seed=13)
    return ck, qm.QuantRWKV7(ck)


def _ids(B, T, seed):
    return torch.from_numpy(
        np.random.default_rng(seed).integers(0, 1024, size=(B, T)))


def _eager(model, idx, **kw):
    old = qm.USE_GRAPH
    qm.USE_GRAPH = False
    try:
        return model.forward_stateful(idx, model.init_state(idx.shape[0]),
                                      **kw)
    finally:
        qm.USE_GRAPH = old


def test_graphs_of_one_token_count_do_not_share_freed_buffers(toy):
    """Capture (1, 512), run (2, 256) (same B*T, more chunk slots), replay
    (1, 512): every result equals the eager run bit for bit."""
    _, model = toy
    a, b = _ids(1, 512, 1), _ids(2, 256, 2)
    ref_a, _ = _eager(model, a)
    ref_b, _ = _eager(model, b)
    out_a, _ = model.forward_stateful(a, model.init_state(1))
    out_b, _ = model.forward_stateful(b, model.init_state(2))
    out_a2, st_a2 = model.forward_stateful(a, model.init_state(1))
    assert torch.equal(out_a, ref_a)
    assert torch.equal(out_b, ref_b)
    assert torch.equal(out_a2, ref_a)
    # eager after the graphs exist still matches too
    ref_a3, _ = _eager(model, a)
    assert torch.equal(ref_a3, ref_a)


def test_seq_graph_cache_is_bounded(toy):
    _, model = toy
    shapes = [(1, 3 + i) for i in range(qm.MAX_SEQ_GRAPHS + 2)]
    first = model.forward_stateful(_ids(*shapes[0], 3),
                                   model.init_state(1))[0]
    for B, T in shapes[1:]:
        model.forward_stateful(_ids(B, T, 4), model.init_state(B))
    assert len(model._seq_graphs) <= qm.MAX_SEQ_GRAPHS
    assert (1, 3, False, 0) not in model._seq_graphs     # evicted (LRU)
    again = model.forward_stateful(_ids(*shapes[0], 3),
                                   model.init_state(1))[0]
    assert torch.equal(first, again)                     # recaptured


@pytest.mark.parametrize("T,k", [(12, 4), (160, 5), (160, 1)])
def test_tail_only_and_last_only_are_slices(toy, T, k):
    """tail_only = k returns the logits of the last k tokens, last_only the
    last one; the states are those of the full run."""
    _, model = toy
    idx = _ids(2, T, 5)
    full, st_f = model.forward_stateful(idx, model.init_state(2))
    tail, st_t = model.forward_stateful(idx, model.init_state(2),
                                        tail_only=k)
    last, st_l = model.forward_stateful(idx, model.init_state(2),
                                        last_only=True)
    assert tail.shape == (2, k, full.shape[-1])
    assert last.shape == (2, 1, full.shape[-1])
    scale = float(full.abs().max())
    # the head runs on fewer rows (possibly another GEMV kernel): within
    # the GEMV tolerance of the full run's rows
    assert float((tail - full[:, -k:]).abs().max()) < 1e-3 * scale
    assert float((last - full[:, -1:]).abs().max()) < 1e-3 * scale
    for a, b, c in zip(st_f, st_t, st_l):
        for x, y, z in zip(a, b, c):
            assert torch.equal(x, y) and torch.equal(x, z)


def test_forward_hidden_feeds_the_head(toy):
    _, model = toy
    idx = _ids(1, 7, 6)
    hid, st_h = model.forward_hidden(idx, model.init_state(1))
    lg, st = _eager(model, idx)
    head = model.head(hid.reshape(7, -1))
    assert torch.equal(head.reshape(lg.shape), lg)
    for a, b in zip(st_h, st):
        for x, y in zip(a, b):
            assert torch.equal(x, y)


def test_rwkvq_file_load_equals_in_memory(toy, tmp_path):
    """save_rwkvq -> load_raw -> QuantRWKV7: the documented user path
    gives the in-memory model's logits bit for bit, prefill and decode."""
    ck, model = toy
    path = str(tmp_path / "toy.rwkvq")
    writer.save_rwkvq(ck, path)
    loaded = qm.QuantRWKV7(reader.load_raw(path))
    idx = _ids(1, 20, 7)
    a, sa = model.forward_stateful(idx, model.init_state(1))
    b, sb = loaded.forward_stateful(idx, loaded.init_state(1))
    assert torch.equal(a, b)
    nxt = _ids(1, 1, 8)
    a2, _ = model.step(nxt, sa)
    b2, _ = loaded.step(nxt, sb)
    assert torch.equal(a2, b2)


def test_rwkvq_file_model_matches_oracle(toy, tmp_path):
    ck, _ = toy
    path = str(tmp_path / "toy2.rwkvq")
    writer.save_rwkvq(ck, path)
    back = reader.load_raw(path)
    model = qm.QuantRWKV7(back)
    orc = RWKV7Oracle(back)
    idx = np.random.default_rng(9).integers(0, 1024, size=(1, 9))
    ref, _ = orc.forward_stateful(idx, orc.init_state(1))
    out, _ = model.forward_stateful(torch.from_numpy(idx),
                                    model.init_state(1))
    assert float(np.abs(out.cpu().numpy() - ref).max()) < 1e-2


@pytest.fixture(scope="module")
def full_depth():
    """The bench's 1.5B-shaped compression model: 24 layers, D 2048,
    vocab 65536, quantized on the GPU."""
    ck = quantized_model("compression", n_layer=24, n_embd=2048,
                         vocab=65536, seed=0, device="cuda")
    return ck, qm.QuantRWKV7(ck)


def test_full_depth_decode_properties(full_depth):
    """24 layers, vocab 65536, B = 1 and 8: logits finite and the captured
    step equals the eager step bit for bit over four tokens (the fused and
    unfused decode paths are each held against the oracle in
    test_full_depth_decode_matches_oracle)."""
    _, model = full_depth
    for B in (1, 8):
        print(f"full depth decode B={B}", flush=True)
        idx = _ids(B, 4, 10 + B) % 65536
        st_g, st_e = model.init_state(B), model.init_state(B)
        for t in range(4):
            tok = idx[:, t:t + 1]
            lg, st_g = model.step(tok, st_g)
            le, st_e = _eager_step(model, tok, st_e)
            assert bool(torch.isfinite(lg).all())
            assert torch.equal(lg, le)
            for a, b in zip(st_g, st_e):
                for x, y in zip(a, b):
                    assert torch.equal(x, y)


def test_full_depth_decode_matches_oracle(full_depth):
    """The 24-layer, vocab-65536 model against the float64 oracle on the
    same (GPU-quantized) checkpoint: three decode steps from a zero state
    at B = 1 and B = 8, the fused (graph) and unfused paths, logits within
    1e-2 max-abs."""
    from rwkv_quant.models.synthetic import checkpoint_to
    ck, model = full_depth
    orc = RWKV7Oracle(checkpoint_to(ck, "cpu"))
    for B in (1, 8):
        idx = (_ids(B, 3, 30 + B) % 65536).numpy()
        st_o, st_g, st_u = orc.init_state(B), model.init_state(B), \
            model.init_state(B)
        for t in range(3):
            ro, st_o = orc.forward_stateful(idx[:, t:t + 1], st_o)
            tok = torch.from_numpy(idx[:, t:t + 1])
            lg, st_g = model.step(tok, st_g)
            lu, st_u = _eager_step(model, tok, st_u, fuse_decode=False)
            eg = float(np.abs(lg.cpu().numpy() - ro).max())
            eu = float(np.abs(lu.cpu().numpy() - ro).max())
            print(f"B={B} step {t}: fused {eg:.2e} unfused {eu:.2e} "
                  f"(logit scale {np.abs(ro).max():.2f})", flush=True)
            assert eg < 1e-2 and eu < 1e-2


def _eager_step(model, tok, st, fuse_decode=True):
    old = (qm.USE_GRAPH, qm.FUSE_DECODE)
    qm.USE_GRAPH, qm.FUSE_DECODE = False, fuse_decode
    try:
        return model.forward_stateful(tok, st)
    finally:
        qm.USE_GRAPH, qm.FUSE_DECODE = old


def test_full_depth_prefill_properties(full_depth):
    """pp512 on the full model: finite, the captured graph equals eager,
    and decoding on from the prefill state equals one longer prefill's
    last logits within tolerance."""
    _, model = full_depth
    idx = _ids(1, 512, 20) % 65536
    g, st = model.forward_stateful(idx, model.init_state(1))
    e, _ = _eager(model, idx)
    assert bool(torch.isfinite(g).all())
    assert torch.equal(g, e)
    nxt = _ids(1, 1, 21) % 65536
    d, _ = model.step(nxt, st)
    longer, _ = model.forward_stateful(torch.cat([idx, nxt], 1),
                                       model.init_state(1), last_only=True)
    scale = float(d.abs().max())
    assert float((d - longer).abs().max()) < 2e-2 * scale
