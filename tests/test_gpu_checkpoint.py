"""EXL3 linears loaded from safetensors checkpoints (cx_exl3_load_linear): the device
copy dequantizes bit-exactly to the oracle's reconstruction of the file's trellis and the
linear matches the oracle matvec; a sharded checkpoint loads the same way."""
import json

import numpy as np
import pytest

import oracle as O

torch = pytest.importorskip("torch")
sft = pytest.importorskip("safetensors.numpy")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ck_mod():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from exl3moe import checkpoint
    return checkpoint


def write_linear(path, prefix, I, O, bits, seed, marker="mul1"):
    from exl3moe import synth
    rng = np.random.default_rng(seed)
    tr, suh, svh = synth.linear(rng, I, O, bits)
    t = {prefix + ".trellis": tr.view(np.int16), prefix + ".suh": suh, prefix + ".svh": svh}
    if marker == "mul1":
        t[prefix + ".mul1"] = np.array(-2082680531, dtype=np.int32)
    elif marker == "mcg":
        t[prefix + ".mcg"] = np.array(np.uint32(0xCBAC1FED).view(np.int32), dtype=np.int32)
    sft.save_file(t, str(path))
    return tr, suh, svh


@pytest.mark.parametrize("bits,marker,cb", [(4, "mul1", "mul1"), (2.5, "mul1", "mul1"), (3, None, "3inst"),
                                            (4, "mcg", "mcg")])
def test_load_linear_dequant_and_matvec(ck_mod, tmp_path, bits, marker, cb):
    f = tmp_path / "lin.safetensors"
    tr, suh, svh = write_linear(f, "model.mlp.down_proj", 512, 256, bits, 7, marker)
    with ck_mod.Checkpoint(str(f)) as ck:
        lin = ck.load_linear("model.mlp.down_proj")
    assert (lin.in_features, lin.out_features, lin.k2, lin.codebook) == (512, 256, int(round(2 * bits)), cb)
    w = O.reconstruct_inner(tr, bits, cb)
    np.testing.assert_array_equal(lin.dequant().cpu().numpy().view(np.uint16), w.view(np.uint16))
    x = np.random.default_rng(1).standard_normal((5, 512)).astype(np.float16)
    y = lin(torch.from_numpy(x).cuda()).cpu().numpy()
    ref = O.matvec(x, w, suh, svh, np.float32)
    assert np.linalg.norm(y - ref) <= 1e-3 * np.linalg.norm(ref)


def test_load_from_sharded_checkpoint(ck_mod, tmp_path):
    tr_a, _, _ = write_linear(tmp_path / "model-00001-of-00002.safetensors", "l.0.gate", 256, 128, 4, 1)
    tr_b, _, _ = write_linear(tmp_path / "model-00002-of-00002.safetensors", "l.0.up", 256, 128, 3, 2)
    wm = {f"l.0.gate.{s}": "model-00001-of-00002.safetensors" for s in ("trellis", "suh", "svh", "mul1")}
    wm.update({f"l.0.up.{s}": "model-00002-of-00002.safetensors" for s in ("trellis", "suh", "svh", "mul1")})
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wm}))
    with ck_mod.Checkpoint(str(tmp_path)) as ck:
        a, b = ck.load_linear("l.0.gate"), ck.load_linear("l.0.up")
    np.testing.assert_array_equal(a.dequant().cpu().numpy().view(np.uint16),
                                  O.reconstruct_inner(tr_a, 4).view(np.uint16))
    np.testing.assert_array_equal(b.dequant().cpu().numpy().view(np.uint16),
                                  O.reconstruct_inner(tr_b, 3).view(np.uint16))


def test_load_errors(ck_mod, tmp_path):
    from exl3moe import CxError, Matrix, lib
    f = tmp_path / "lin.safetensors"
    write_linear(f, "p", 128, 128, 4, 3)
    with ck_mod.Checkpoint(str(f)) as ck:
        d = torch.empty(1 << 20, dtype=torch.uint8, device="cuda")
        m = Matrix()
        import ctypes
        rc = lib().cx_exl3_load_linear(ck.handle, b"p", ctypes.byref(m), d.data_ptr(), d.data_ptr(), d.data_ptr(),
                                       d.data_ptr(), 16, None)
        assert rc == -4  # staging smaller than the trellis
        with pytest.raises(CxError) as e:
            ck.load_linear("q")
        assert e.value.rc == -7 and "missing .trellis" in str(e.value)
