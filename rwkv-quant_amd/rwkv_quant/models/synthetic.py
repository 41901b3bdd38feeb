"""Seeded random-init RWKV-7 state dicts with the official ("world") key
names and shapes, for tests and benchmarks (no checkpoint is available
offline).

Key list and shapes follow the world checkpoint layout
(reference: tests_local/build_world_ckpt_v2.py:42-99); LoRA ranks follow
the reference's formula max(32, round(c * D^p / 32) * 32) with
(c, p) = (1.8, .5) w, (1.8, .5) a, (1.3, .5) v, (0.6, .8) g
(reference: tests/test_quant_model_smoke.py:25-27), which gives
96/96/64/256 at D = 2048 and 96/96/64/320 at D = 2560.

Weights are N(0, std); decay/gate biases are drawn so that the decay
w = exp(-0.606531 * sigmoid(.)) spans (0, 1) with the spread of a trained
model; LayerNorm weights are 1, biases 0.
"""
import torch

SHAPES = {
    "1.5b": dict(n_layer=24, n_embd=2048, head_size=64, vocab=65536,
                 ffn=8192),
    "2.9b": dict(n_layer=32, n_embd=2560, head_size=64, vocab=65536,
                 ffn=10240),
}


def lora_ranks(d):
    f = lambda c, p: max(32, int(round((c * (d ** p)) / 32) * 32))
    return {"w": f(1.8, 0.5), "a": f(1.8, 0.5), "v": f(1.3, 0.5),
            "g": f(0.6, 0.8)}


def world_state_dict(n_layer, n_embd, head_size=64, vocab=65536, ffn=None,
                     seed=0, std=0.02, dtype=torch.bfloat16, device="cpu"):
    """Random-init state dict with world naming (LoRA stored [in, out]).
    `device` selects where the tensors are drawn (a GPU generator gives a
    different, equally seeded stream)."""
    g = torch.Generator(device=device).manual_seed(seed)
    C, H, N = n_embd, n_embd // head_size, head_size
    ffn = ffn or 4 * C
    r = lora_ranks(C)

    def rn(*shape, s=std):
        return (torch.randn(*shape, generator=g, device=device) * s).to(dtype)

    def uni(*shape, lo=0.0, hi=1.0):
        return (lo + (hi - lo) * torch.rand(*shape, generator=g,
                                            device=device)).to(dtype)

    one = lambda *s: torch.ones(*s, dtype=dtype, device=device)
    zero = lambda *s: torch.zeros(*s, dtype=dtype, device=device)
    sd = {"emb.weight": rn(vocab, C)}
    for i in range(n_layer):
        p = f"blocks.{i}."
        if i == 0:
            sd[p + "ln0.weight"], sd[p + "ln0.bias"] = one(C), zero(C)
        sd[p + "ln1.weight"], sd[p + "ln1.bias"] = one(C), zero(C)
        sd[p + "ln2.weight"], sd[p + "ln2.bias"] = one(C), zero(C)
        a = p + "att."
        for nm in ("x_r", "x_w", "x_k", "x_v", "x_a", "x_g"):
            sd[a + nm] = uni(1, 1, C)
        sd[a + "w1"], sd[a + "w2"] = rn(C, r["w"]), rn(r["w"], C)
        sd[a + "w0"] = (torch.randn(1, 1, C, generator=g, device=device) * 0.5
                        - 0.5).to(dtype)
        sd[a + "a1"], sd[a + "a2"] = rn(C, r["a"]), rn(r["a"], C)
        sd[a + "a0"] = rn(1, 1, C, s=0.5)
        if i > 0:
            sd[a + "v1"], sd[a + "v2"] = rn(C, r["v"]), rn(r["v"], C)
            sd[a + "v0"] = rn(1, 1, C, s=0.5)
        sd[a + "g1"], sd[a + "g2"] = rn(C, r["g"]), rn(r["g"], C)
        sd[a + "k_k"] = uni(1, 1, C, lo=0.5, hi=1.5)
        sd[a + "k_a"] = uni(1, 1, C)
        sd[a + "r_k"] = rn(H, N, s=0.1)
        for nm in ("receptance", "key", "value", "output"):
            sd[a + nm + ".weight"] = rn(C, C)
        sd[a + "ln_x.weight"], sd[a + "ln_x.bias"] = one(C), zero(C)
        f = p + "ffn."
        sd[f + "x_k"] = uni(1, 1, C)
        sd[f + "key.weight"] = rn(ffn, C)
        sd[f + "value.weight"] = rn(C, ffn)
    sd["ln_out.weight"], sd["ln_out.bias"] = one(C), zero(C)
    sd["head.weight"] = rn(vocab, C)
    return sd


def quantized_model(preset, n_layer, n_embd, head_size=64, vocab=65536,
                    ffn=None, seed=0, config=None, device="cpu",
                    to_cpu=False):
    """Random-init model quantized with a preset -> QuantizedCheckpoint.
    With a GPU `device` the weights are drawn and quantized there (the
    quantizer is plain torch); the packed fields stay on that device unless
    `to_cpu` (the CPU oracle needs them on the host)."""
    from ..formats import writer
    from ..presets import PRESETS
    cfg = config if config is not None else PRESETS[preset]
    sd = world_state_dict(n_layer, n_embd, head_size, vocab, ffn, seed,
                          device=device)
    ck = writer.quantize_state_dict(sd, cfg, naming="world", n_layer=n_layer,
                                    n_embd=n_embd, head_size=head_size,
                                    vocab_size=vocab)
    return checkpoint_to(ck, "cpu") if to_cpu else ck


def checkpoint_to(ck, device):
    """Move every tensor field of a QuantizedCheckpoint to `device`."""
    import dataclasses
    for qt in ck.tensors.values():
        for f in dataclasses.fields(qt):
            v = getattr(qt, f.name)
            if torch.is_tensor(v):
                setattr(qt, f.name, v.to(device))
    return ck
