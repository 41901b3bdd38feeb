"""`.rwkvq` container round trip and negative controls (CPU), after the
reference's container gate (tests/test_rwkvq_container.py:46-171):
save_rwkvq -> load_raw keeps every field's dtype, shape and bytes, the
checkpoint metadata and the QuantConfig; the torch-free reader sees the
same buffers; files without a manifest, from a newer format_version or in
the pickle container are rejected."""
import json
import os
import struct

import numpy as np
import pytest
import torch

from oracle import codec_ref
from rwkv_quant.formats import codec, reader, writer
from rwkv_quant.models.synthetic import quantized_model


@pytest.fixture(scope="module")
def saved(tmp_path_factory):
    ck = quantized_model("compression", n_layer=2, n_embd=256, vocab=512,
                         seed=3)
    # an rtn tensor with sparse outliers, which the presets do not produce
    w = torch.randn(64, 256, generator=torch.Generator().manual_seed(4))
    c, s, oi, ov = writer.rtn_quantize_outliers(w, 8, 0.01)
    ck.tensors["extra.spqr"] = writer.make_rtn("extra.spqr", "head", 8,
                                               w.shape, c, s, oi, ov)
    path = str(tmp_path_factory.mktemp("rwkvq") / "m.rwkvq")
    writer.save_rwkvq(ck, path, tokenizer="rwkv_vocab_v20230424")
    return ck, path


def _same(a, b):
    return (a.dtype == b.dtype and tuple(a.shape) == tuple(b.shape)
            and bytes(a.contiguous().view(torch.uint8).numpy())
            == bytes(b.contiguous().view(torch.uint8).numpy()))


def test_roundtrip_bit_equal(saved):
    ck, path = saved
    back = reader.load_raw(path)
    for f in ("naming", "n_layer", "n_embd", "head_size", "vocab_size",
              "config_repr"):
        assert getattr(back, f) == getattr(ck, f), f
    assert back.tokenizer == "rwkv_vocab_v20230424"
    assert set(back.tensors) == set(ck.tensors)
    for key, qt in ck.tensors.items():
        bq = back.tensors[key]
        assert (bq.kind, bq.bits, tuple(bq.shape), bq.gw_gs, bq.gw_sb) == \
            (qt.kind, qt.bits, tuple(qt.shape), qt.gw_gs, qt.gw_sb), key
        for f in writer.TENSOR_FIELDS:
            a, b = getattr(qt, f), getattr(bq, f)
            assert (a is None) == (b is None), (key, f)
            if a is not None:
                assert _same(a, b), (key, f)


def test_config_survives_save_load_save(saved, tmp_path):
    ck, path = saved
    back = reader.load_raw(path)
    assert back.config is not None
    assert writer.config_to_json(back.config) == \
        writer.config_to_json(ck.config)
    again = str(tmp_path / "again.rwkvq")
    writer.save_rwkvq(back, again)
    m1, _ = codec.open_rwkvq(path)
    m2, _ = codec.open_rwkvq(again)
    assert m1 == m2


def test_dequant_unchanged_and_torch_free_reader(saved):
    ck, path = saved
    back = reader.load_raw(path)
    manifest, arrays = codec.open_rwkvq(path)
    assert manifest["format"] == codec.FORMAT
    assert manifest["format_version"] == codec.FORMAT_VERSION
    assert set(manifest["tensors"]) == set(ck.tensors)
    for key, qt in ck.tensors.items():
        a = codec_ref.dequant_qt(qt)
        b = codec_ref.dequant_qt(back.tensors[key])
        assert a.shape == b.shape and np.array_equal(a, b, equal_nan=True)
        for f in manifest["tensors"][key]["fields"]:
            buf = arrays[f"{key}::{f}"]
            src = getattr(qt, f).contiguous()
            assert buf.tobytes() == bytes(src.view(torch.uint8).numpy()), \
                (key, f)
        assert codec.is_transposed(manifest, key) == (
            codec.is_raw_lora_world(key))


def _rewrite_manifest(src, dst, fn):
    with open(src, "rb") as f:
        n = struct.unpack("<Q", f.read(8))[0]
        header = json.loads(f.read(n))
        rest = f.read()
    m = json.loads(header["__metadata__"]["rwkvq"])
    fn(m)
    header["__metadata__"]["rwkvq"] = json.dumps(m)
    hb = json.dumps(header).encode()
    hb += b" " * (-len(hb) % 8)
    with open(dst, "wb") as f:
        f.write(struct.pack("<Q", len(hb)) + hb + rest)


def test_rejects_missing_manifest(tmp_path):
    from safetensors.torch import save_file
    p = str(tmp_path / "plain.safetensors")
    save_file({"x": torch.zeros(4)}, p)
    with pytest.raises(ValueError):
        reader.load_raw(p)
    with pytest.raises(ValueError):
        codec.open_rwkvq(p)


def test_rejects_newer_format_version(saved, tmp_path):
    _, path = saved
    p = str(tmp_path / "future.rwkvq")
    _rewrite_manifest(path, p, lambda m: m.update(
        format_version=codec.FORMAT_VERSION + 1))
    with pytest.raises(ValueError, match="format_version"):
        reader.load_raw(p)
    with pytest.raises(ValueError, match="format_version"):
        codec.open_rwkvq(p)
    # the unmodified bytes of the same file still load
    ok = str(tmp_path / "same.rwkvq")
    _rewrite_manifest(path, ok, lambda m: None)
    assert reader.load_raw(ok).n_layer == 2


def test_rejects_wrong_format_name(saved, tmp_path):
    _, path = saved
    p = str(tmp_path / "other.rwkvq")
    _rewrite_manifest(path, p, lambda m: m.update(format="gguf"))
    with pytest.raises(ValueError):
        reader.load_raw(p)


def test_rejects_pickle_container(tmp_path):
    p = str(tmp_path / "legacy.rwkvq")
    with open(p, "wb") as f:
        f.write(codec.MAGIC_ZIP + b"\0" * 60)
    with pytest.raises(ValueError, match="pickle"):
        reader.load_raw(p)
    with pytest.raises(ValueError, match="pickle"):
        codec.open_rwkvq(p)


def test_spqr_csr_is_the_outlier_set():
    """The device CSR of the SpQR outliers (built on the CPU here) holds
    exactly the stored (row, col, value) triples, rows in order."""
    from rwkv_quant.backends.hip.quant_linear import spqr_csr
    w = torch.randn(64, 256, generator=torch.Generator().manual_seed(5))
    c, s, oi, ov = writer.rtn_quantize_outliers(w, 8, 0.02)
    qt = writer.make_rtn("t", "head", 8, w.shape, c, s, oi, ov)
    ptr, col, val = spqr_csr(qt, "cpu")
    ptr, col = ptr.long().numpy(), col.long().numpy()
    assert ptr[0] == 0 and ptr[-1] == len(col) == oi.shape[0]
    assert (np.diff(ptr) >= 0).all()
    rows = np.repeat(np.arange(64), np.diff(ptr))
    got = {(int(r), int(c_), int(v)) for r, c_, v in
           zip(rows, col, val.numpy().astype(np.int64))}
    ref = {(int(r), int(c_), int(v)) for (r, c_), v in
           zip(oi.long().numpy(), ov.view(torch.int16).numpy()
               .astype(np.int64))}
    assert got == ref
