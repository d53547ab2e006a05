"""Safetensors checkpoints through the C-ABI (host side, no GPU): header parsing, tensor
views, sharded index, EXL3 linear validation, and rejection of malformed files.  Files
are written with the `safetensors` package (the format's own writer) or byte by byte."""
import json
import struct

import numpy as np
import pytest

from exl3moe import CxError
from exl3moe.checkpoint import Checkpoint

sft = pytest.importorskip("safetensors.numpy")


def exl3_tensors(prefix, I, O, bits, rng, marker="mul1"):
    k2 = int(round(bits * 2))
    t = {prefix + ".trellis": rng.integers(-32768, 32768, size=(I // 16, O // 16, 8 * k2), dtype=np.int16),
         prefix + ".suh": rng.standard_normal(I).astype(np.float16),
         prefix + ".svh": rng.standard_normal(O).astype(np.float16)}
    if marker == "mul1":
        t[prefix + ".mul1"] = np.array(-2082680531, dtype=np.int32)
    elif marker == "mcg":
        t[prefix + ".mcg"] = np.array(np.uint32(0xCBAC1FED).view(np.int32), dtype=np.int32)
    return t


def test_single_file_roundtrip(tmp_path):
    rng = np.random.default_rng(1)
    t = exl3_tensors("model.layers.0.mlp.experts.3.gate_proj", 256, 128, 4, rng)
    t["other.bf16"] = rng.integers(0, 65535, size=(3, 5), dtype=np.uint16)
    t["empty"] = np.zeros((0, 4), dtype=np.float32)
    f = tmp_path / "a.safetensors"
    sft.save_file(t, str(f), metadata={"format": "pt"})
    with Checkpoint(str(f)) as ck:
        assert ck.names() == sorted(t)
        for k, v in t.items():
            got = ck.tensor(k)
            assert got.shape == v.shape
            assert got.tobytes() == np.ascontiguousarray(v).tobytes()
        assert ck.linear_info("model.layers.0.mlp.experts.3.gate_proj") == (256, 128, 8, "mul1")


@pytest.mark.parametrize("bits,marker,cb", [(2, "mcg", "mcg"), (3, None, "3inst"), (1.5, "mul1", "mul1"),
                                            (6, "mul1", "mul1")])
def test_linear_info_rates_and_codebooks(tmp_path, bits, marker, cb):
    rng = np.random.default_rng(2)
    f = tmp_path / "b.safetensors"
    sft.save_file(exl3_tensors("p", 128, 256, bits, rng, marker), str(f))
    with Checkpoint(str(f)) as ck:
        assert ck.linear_info("p") == (128, 256, int(round(2 * bits)), cb)


def test_sharded_index(tmp_path):
    rng = np.random.default_rng(3)
    a = exl3_tensors("x.a", 128, 128, 4, rng)
    b = exl3_tensors("x.b", 128, 256, 2, rng)
    sft.save_file(a, str(tmp_path / "model-00001.safetensors"))
    # The second shard also holds a copy of one of the first shard's names: the index
    # decides which copy is used.
    b2 = dict(b)
    b2["x.a.suh"] = np.zeros(128, dtype=np.float16)
    sft.save_file(b2, str(tmp_path / "model-00002.safetensors"))
    wm = {k: "model-00001.safetensors" for k in a}
    wm.update({k: "model-00002.safetensors" for k in b})
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"metadata": {"x": 1}, "weight_map": wm}))
    with Checkpoint(str(tmp_path)) as ck:
        assert ck.names() == sorted(wm)
        np.testing.assert_array_equal(ck.tensor("x.a.suh"), a["x.a.suh"])
        np.testing.assert_array_equal(ck.tensor("x.b.trellis"), b["x.b.trellis"])
        assert ck.linear_info("x.b") == (128, 256, 4, "mul1")


def raw_file(path, header: dict | str, payload: bytes):
    h = header if isinstance(header, str) else json.dumps(header)
    hb = h.encode()
    path.write_bytes(struct.pack("<Q", len(hb)) + hb + payload)


@pytest.mark.parametrize("header,payload,why", [
    ({"t": {"dtype": "F16", "shape": [2], "data_offsets": [0, 8]}}, b"\0" * 8, "do not match"),
    ({"t": {"dtype": "F16", "shape": [4], "data_offsets": [0, 8]}}, b"\0" * 4, "outside the payload"),
    ({"t": {"dtype": "F8", "shape": [4], "data_offsets": [0, 4]}}, b"\0" * 4, "unsupported dtype"),
    ({"t": {"dtype": "F16", "shape": [-1], "data_offsets": [0, 0]}}, b"", "negative"),
    ({"t": {"dtype": "F16", "shape": [1]}}, b"\0" * 2, "missing"),
    ('{"t": {"dtype": "F16", "shape": [1], "data_offsets": [0, 2]},}', b"\0" * 2, "trailing comma"),
    ('{"t": {"dtype": "F16", "shape": [1], "data_offsets": [0, 2]}} x', b"\0" * 2, "trailing data"),
    ('{"t": {"dtype": "F16", "shape": [1], "data_offsets": [0, 2]}, "t": {"dtype": "F16", "shape": [1], '
     '"data_offsets": [0, 2]}}', b"\0" * 2, "duplicate tensor"),
    ({"t": {"dtype": "F16", "shape": [1.5], "data_offsets": [0, 2]}}, b"\0" * 2, "fraction"),
])
def test_malformed_headers(tmp_path, header, payload, why):
    f = tmp_path / "bad.safetensors"
    raw_file(f, header, payload)
    with pytest.raises(CxError) as e:
        Checkpoint(str(f))
    assert e.value.rc == -7 and why in str(e.value), str(e.value)


def test_header_length_and_unicode(tmp_path):
    f = tmp_path / "short.safetensors"
    f.write_bytes(struct.pack("<Q", 1000) + b"{}")
    with pytest.raises(CxError) as e:
        Checkpoint(str(f))
    assert "header length" in str(e.value)
    g = tmp_path / "u.safetensors"
    raw_file(g, '{"\\u00e9\\ud83d\\ude00": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}}', b"\x07")
    with Checkpoint(str(g)) as ck:
        assert ck.names() == ["é\U0001F600"]
        assert ck.tensor("é\U0001F600").tolist() == [7]


@pytest.mark.parametrize("mutate,why", [
    (lambda t: t.pop("p.mul1"), None),  # no marker: 3inst, but K 1.5 needs mul1
    (lambda t: t.__setitem__("p.mul1", np.array(7, dtype=np.int32)), "unknown multiplier"),
    (lambda t: t.__setitem__("p.suh", np.zeros(64, dtype=np.float16)), ".suh must be"),
    (lambda t: t.__setitem__("p.svh", np.zeros(256, dtype=np.float32)), ".svh must be"),
    (lambda t: t.__setitem__("p.trellis", np.zeros((8, 16, 20), dtype=np.int16)), "16 K"),
    (lambda t: t.__setitem__("p.trellis", np.zeros((8, 16, 24), dtype=np.float16)), "I16"),
    (lambda t: t.__setitem__("p.mcg", np.array(np.uint32(0xCBAC1FED).view(np.int32), dtype=np.int32)), "both"),
])
def test_linear_validation(tmp_path, mutate, why):
    rng = np.random.default_rng(4)
    t = exl3_tensors("p", 128, 256, 1.5, rng)
    mutate(t)
    f = tmp_path / "v.safetensors"
    sft.save_file(t, str(f))
    with Checkpoint(str(f)) as ck:
        with pytest.raises(CxError) as e:
            ck.linear_info("p")
        assert e.value.rc == -7
        if why:
            assert why in str(e.value), str(e.value)


def test_index_errors(tmp_path):
    rng = np.random.default_rng(5)
    sft.save_file(exl3_tensors("q", 128, 128, 4, rng), str(tmp_path / "s.safetensors"))
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": {"q.suh": "../s.safetensors"}}))
    with pytest.raises(CxError) as e:
        Checkpoint(str(tmp_path))
    assert "plain file name" in str(e.value)
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": {"q.nope": "s.safetensors"}}))
    with pytest.raises(CxError) as e:
        Checkpoint(str(tmp_path))
    assert "missing from its shard" in str(e.value)
    with pytest.raises(CxError):
        Checkpoint(str(tmp_path / "absent.safetensors"))
