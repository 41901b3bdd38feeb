"""Writes the reference-generated fixtures of this directory.

    python tests/golden/make_reference_goldens.py

Runs only in the build container, where the reference checkout is at
/root/reference (RWKVQ_REFERENCE overrides).  The reference is imported in a
child process whose import path holds the reference and not this
repository (both packages are called `rwkv_quant`); nothing of the reference
is copied: the fixtures hold inputs, outputs and SHA-256 digests only.

Outputs:
  rwkv7_ref_forward.npz  the reference RWKV7Ref forward (fp32, CPU) of a
                         seeded 3-layer world-naming model: logits, the
                         residual stream after every block (`trace`), and
                         the reference `perplexity` of a seeded corpus
                         (reference: rwkv_quant/models/rwkv7_ref.py:184-290,
                         rwkv_quant/calibration/ablation.py:21-69)
  reference_digests.json digests of the reference's quantizer outputs on the
                         frozen synthetic tensors of tests/make_gw_golden.py
                         (computed on this machine), of its writer's packed
                         fields (writer.py:145-338) and of its MLX-affine /
                         K3 relayout (codec.py:313-435)

The model weights are not stored: `forward_model_state_dict()` regenerates
them from the seeds recorded in the .npz.
"""
import hashlib
import json
import os
import subprocess
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REFERENCE = os.environ.get("RWKVQ_REFERENCE", "/root/reference")

# the forward fixture's model and inputs
FWD = dict(n_layer=3, n_embd=128, head_size=64, vocab=256, ffn=512, seed=11,
           std=0.1, ln_seed=12, idx_seed=13, B=2, T=16, ppl_rows=3,
           ppl_len=17)
SYNTH_SEED = 20260810          # tests/make_gw_golden.py:91
MLX_SEED = 5


def forward_model_state_dict(cfg=FWD):
    """The fixture's float32 world state dict (bf16-valued, so a dense
    bf16 checkpoint of it is exact): synthetic.world_state_dict with
    LayerNorm / group-norm affines drawn away from (1, 0)."""
    import torch
    from rwkv_quant.models.synthetic import world_state_dict
    sd = world_state_dict(cfg["n_layer"], cfg["n_embd"], cfg["head_size"],
                          cfg["vocab"], cfg["ffn"], seed=cfg["seed"],
                          std=cfg["std"])
    g = torch.Generator().manual_seed(cfg["ln_seed"])
    for k in sorted(sd):
        if k.endswith(("ln0.weight", "ln1.weight", "ln2.weight",
                       "ln_out.weight", "ln_x.weight")):
            sd[k] = (1 + 0.2 * torch.randn(sd[k].shape, generator=g)) \
                .to(torch.bfloat16)
        elif k.endswith(("ln0.bias", "ln1.bias", "ln2.bias", "ln_out.bias",
                         "ln_x.bias")):
            sd[k] = (0.1 * torch.randn(sd[k].shape, generator=g)) \
                .to(torch.bfloat16)
    return {k: v.float() for k, v in sd.items()}


def forward_inputs(cfg=FWD):
    rng = np.random.default_rng(cfg["idx_seed"])
    idx = rng.integers(0, cfg["vocab"], size=(cfg["B"], cfg["T"]))
    data = rng.integers(0, cfg["vocab"], size=(cfg["ppl_rows"],
                                               cfg["ppl_len"]))
    return idx.astype(np.int64), data.astype(np.int64)


def synth_tensors():
    """tests/make_gw_golden.py:91-95 of the reference."""
    import torch
    g = torch.Generator().manual_seed(SYNTH_SEED)
    gauss = torch.randn(128, 512, generator=g)
    z = torch.randn(64, 256, generator=g)
    z[7] = 0.0
    z[9] = 1e-9
    return {"synth::gauss": gauss, "synth::degenerate": z}


def lora_tensor():
    """A ragged LoRA-shaped factor (world w1 is stored [in, out])."""
    import torch
    g = torch.Generator().manual_seed(21)
    return torch.randn(128, 96, generator=g) * 0.05


def mlx_codes(bits):
    rng = np.random.default_rng(MLX_SEED + bits)
    return rng.integers(0, 1 << bits, size=(16, 4, 32)).astype(np.uint8)


def digest_torch(t):
    """The reference's digest (tests/make_gw_golden.py:52-60)."""
    import torch
    a = t.detach().contiguous().cpu()
    h = hashlib.sha256()
    h.update(str(tuple(a.shape)).encode())
    h.update(str(a.dtype).encode())
    if a.dtype == torch.bfloat16:          # numpy has no bfloat16
        a = a.view(torch.int16)
    h.update(a.numpy().tobytes())
    return h.hexdigest()


def digest_np(a):
    a = np.ascontiguousarray(a)
    h = hashlib.sha256()
    h.update(str(tuple(a.shape)).encode())
    h.update(str(a.dtype).encode())
    h.update(a.tobytes())
    return h.hexdigest()


QT_FIELDS = ("codes", "codes_packed", "scale", "gw_d", "gw_dm", "gw_qsqm",
             "gw_qh", "gw_qh2", "gw_qs", "gw_scale", "gw_min",
             "outlier_indices", "outlier_values")


def qt_digests(qt):
    out = {}
    for f in QT_FIELDS:
        v = getattr(qt, f, None)
        if v is not None:
            out[f] = digest_torch(v)
    return out


def pack_cases():
    """(name, packer kind, bits, args) of the writer-level digests."""
    cases = []
    for bits in (4, 5, 6):
        for search in (False, True):
            cases.append((f"sb6|{bits}|search={int(search)}", "sb6", bits,
                          search))
    for bits in (6, 8):
        for search in (False, True):
            cases.append((f"sym|{bits}|search={int(search)}", "sym", bits,
                          search))
    cases.append(("asym|6|gs64", "asym", 6, None))
    cases.append(("asym|8|gs64", "asym", 8, None))
    cases.append(("rtn|8", "rtn", 8, None))
    cases.append(("rtn|8|spqr0.01", "rtn_spqr", 8, None))
    return cases


# ------------------------------------------------------- reference side

def reference_side(work):
    """Runs with the reference first on sys.path (child process)."""
    import torch
    from rwkv_quant.calibration import QuantConfig
    from rwkv_quant.calibration.ablation import perplexity
    from rwkv_quant.formats import codec, writer
    from rwkv_quant.models.rwkv7_ref import RWKV7Ref

    res = {"gw": {}, "pack": {}, "codec": {}}
    arrays = {}

    # forward + perplexity
    inp = np.load(os.path.join(work, "inputs.npz"))
    model = RWKV7Ref(os.path.join(work, "world.pth"), device="cpu",
                     dtype=torch.float32)
    trace = []
    with torch.no_grad():
        logits = model.forward(torch.from_numpy(inp["idx"]), QuantConfig(),
                               trace=trace)
    arrays["logits"] = logits.float().numpy()
    arrays["trace"] = torch.stack(trace).numpy()
    ppl = perplexity(model, torch.from_numpy(inp["data"]), QuantConfig(),
                     batch_size=2)
    arrays["ppl"] = np.array(ppl, dtype=np.float64)

    # quantizer outputs on the frozen synthetic tensors
    gw = writer._groupwise_fake_dequant
    sym = writer._groupwise_sym_fake_dequant
    mx4 = writer._mxfp4_fake_dequant
    for name, w in synth_tensors().items():
        res["gw"][f"{name}|asym_plain|6"] = digest_torch(gw(w, 6, 64))
        for bits in (5, 6):
            res["gw"][f"{name}|sym_spqr|{bits}"] = digest_torch(
                sym(w, bits, gs=16, sb=16, search=True, outlier_frac=0.01))
        res["gw"][f"{name}|mxfp4"] = digest_torch(mx4(w, 32))
        res["gw"][f"{name}|mxfp4_spqr"] = digest_torch(mx4(w, 32, 0.01))
    w = lora_tensor()
    res["gw"]["lora::ragged|asym_plain|6"] = digest_torch(gw(w, 6, 64))

    # writer-level packed fields
    gauss = synth_tensors()["synth::gauss"]
    for name, kind, bits, search in pack_cases():
        if kind == "sb6":
            qt = writer._make_qt_gw_sb6("t", "proj", bits, gauss, 32, None,
                                        search=search)
        elif kind == "sym":
            qt = writer._make_qt_gw_sym("t", "cmix", bits, gauss, 16, 16,
                                        None, search=search)
        elif kind == "asym":
            qt = writer._make_qt_gw_asym("t", "w_lora", bits, lora_tensor(),
                                         64)
        elif kind == "rtn":
            c, s = writer._real_quantize(gauss, bits)
            qt = writer._make_qt("t", "head", bits, gauss.shape, c, s)
        else:
            c, s, oi, ov = writer._real_quantize_sparse_outlier(gauss, bits,
                                                                0.01)
            qt = writer._make_qt("t", "head", bits, gauss.shape, c, s, oi, ov)
        res["pack"][name] = qt_digests(qt)
        if kind == "sb6" and not search:
            npf = lambda t: None if t is None else t.numpy()
            args = dict(shape=tuple(qt.shape), gs=32, sb=8,
                        qh=npf(qt.gw_qh), qh2=npf(qt.gw_qh2))
            wq, sc, bi, b = codec.sb6_to_mlx_affine(
                qt.codes_packed.numpy(), qt.gw_qsqm.numpy(), qt.gw_d.numpy(),
                qt.gw_dm.numpy(), **args)
            res["codec"][f"sb6_to_mlx_affine|{bits}"] = {
                "wq": digest_np(wq), "scales": digest_np(sc),
                "biases": digest_np(bi), "bits": int(b)}
            qb, qk, ddm, xb = codec.sb6_to_k3(
                qt.codes_packed.numpy(), qt.gw_qsqm.numpy(), qt.gw_d.numpy(),
                qt.gw_dm.numpy(), **args)
            res["codec"][f"sb6_to_k3|{bits}"] = {
                "qblk": digest_np(qb), "qsqm": digest_np(qk),
                "ddm": digest_np(ddm), "xbits": int(xb)}
    for bits in (2, 3, 4, 5, 6, 8):
        words = codec.pack_mlx_affine(mlx_codes(bits), bits)
        res["codec"][f"pack_mlx_affine|{bits}"] = digest_np(words)

    np.savez(os.path.join(work, "out.npz"), **arrays)
    with open(os.path.join(work, "out.json"), "w") as f:
        json.dump(res, f)


# ------------------------------------------------------------ main side

def main():
    sys.path[:0] = [ROOT, os.path.join(ROOT, "rwkv-quant_amd")]
    import torch
    with tempfile.TemporaryDirectory(prefix="rwkvq_gold_") as work:
        torch.save(forward_model_state_dict(), os.path.join(work,
                                                            "world.pth"))
        idx, data = forward_inputs()
        np.savez(os.path.join(work, "inputs.npz"), idx=idx, data=data)
        env = dict(os.environ, PYTHONPATH=REFERENCE)
        subprocess.run([sys.executable, "-I", os.path.abspath(__file__),
                        "--reference-side", work, REFERENCE], check=True,
                       env=env)
        out = dict(np.load(os.path.join(work, "out.npz")))
        with open(os.path.join(work, "out.json")) as f:
            res = json.load(f)
    np.savez_compressed(os.path.join(HERE, "rwkv7_ref_forward.npz"),
                        idx=idx, data=data, config=json.dumps(FWD), **out)
    res["note"] = ("digests of the reference's own functions run on x86-64 "
                   "CPU, torch " + torch.__version__)
    with open(os.path.join(HERE, "reference_digests.json"), "w") as f:
        json.dump(res, f, indent=1, sort_keys=True)
    print("wrote rwkv7_ref_forward.npz and reference_digests.json")


if __name__ == "__main__":
    if len(sys.argv) > 1 and sys.argv[1] == "--reference-side":
        # isolated interpreter (-I): only the reference and this directory
        sys.path.insert(0, sys.argv[3])
        sys.path.insert(0, HERE)
        reference_side(sys.argv[2])
    else:
        main()
