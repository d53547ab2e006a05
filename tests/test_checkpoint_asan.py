"""The checkpoint reader's host code under AddressSanitizer and UBSan (CPU only, no GPU):
csrc/checkpoint.hip is compiled for the host with the sanitizers, linked with
tests/asan_checkpoint_driver.cpp, and run over well-formed files, the malformed headers
of tests/test_checkpoint.py and a few thousand seeded random mutations of a valid
file's header and length.  Any out-of-bounds access, use after free, leak or undefined
behaviour fails the test."""
import json
import os
import shutil
import struct
import subprocess
from pathlib import Path

import numpy as np
import pytest

from test_checkpoint import exl3_tensors, raw_file

sft = pytest.importorskip("safetensors.numpy")
ROOT = Path(__file__).resolve().parent.parent
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined"]


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    if not Path(HIPCC).exists():
        pytest.skip("hipcc not available")
    d = tmp_path_factory.mktemp("asan")
    common = ["--offload-host-only", "-x", "hip", "-std=c++20", "-O1", "-g", "-fno-omit-frame-pointer"] + SAN
    for src, obj in ((ROOT / "crucible-strix-halo_amd" / "csrc" / "checkpoint.hip", d / "ck.o"),
                     (ROOT / "tests" / "asan_checkpoint_driver.cpp", d / "drv.o")):
        subprocess.run([HIPCC] + common + ["-c", str(src), "-o", str(obj)], check=True, capture_output=True)
    exe = d / "ckasan"
    subprocess.run([HIPCC] + SAN + ["-o", str(exe), str(d / "ck.o"), str(d / "drv.o")], check=True,
                   capture_output=True)
    return exe


def run(exe, args):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:exitcode=23",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1:exitcode=24")
    env.pop("LD_PRELOAD", None)
    r = subprocess.run([str(exe)] + [str(a) for a in args], capture_output=True, text=True, env=env, timeout=600)
    out = r.stdout + r.stderr
    assert r.returncode == 0 and "AddressSanitizer" not in out and "runtime error" not in out, out[-4000:]
    return out


def corpus(tmp_path):
    rng = np.random.default_rng(11)
    files = []
    t = exl3_tensors("m.gate", 256, 128, 4, rng)
    t["m.other"] = rng.integers(0, 255, size=(3, 5), dtype=np.uint8)
    t["m.empty"] = np.zeros((0, 4), dtype=np.float32)
    f = tmp_path / "good.safetensors"
    sft.save_file(t, str(f), metadata={"format": "pt"})
    files.append(f)
    shard = tmp_path / "sharded"
    shard.mkdir()
    a = exl3_tensors("x.a", 128, 128, 4, rng)
    sft.save_file(a, str(shard / "model-00001.safetensors"))
    (shard / "model.safetensors.index.json").write_text(json.dumps({"weight_map": {k: "model-00001.safetensors"
                                                                                  for k in a}}))
    files.append(shard)
    bad = [({"t": {"dtype": "F16", "shape": [2], "data_offsets": [0, 8]}}, b"\0" * 8),
           ({"t": {"dtype": "F16", "shape": [4], "data_offsets": [0, 8]}}, b"\0" * 4),
           ({"t": {"dtype": "F16", "shape": [-1], "data_offsets": [0, 0]}}, b""),
           ('{"t": {"dtype": "F16", "shape": [1], "data_offsets": [0, 2]},}', b"\0" * 2),
           ('{"t": {"dtype": "F16", "shape": [99999999999, 99999999999], "data_offsets": [0, 2]}}', b"\0" * 2),
           ('{"t": {"dtype": "F16", "shape": [1], "data_offsets": [18446744073709551615, 2]}}', b"\0" * 2),
           ('{"\\ud83d": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}}', b"\x07"),
           ('{"t": {"dtype": "F16", "shape": [' + "[" * 5000 + "]" * 5000 + '], "data_offsets": [0, 2]}}', b"\0" * 2),
           ('"' + "\\" * 3, b"")]
    for i, (h, p) in enumerate(bad):
        g = tmp_path / f"bad{i}.safetensors"
        raw_file(g, h, p)
        files.append(g)
    short = tmp_path / "short.safetensors"
    short.write_bytes(struct.pack("<Q", 1 << 62) + b"{}")
    files.append(short)
    tiny = tmp_path / "tiny.safetensors"
    tiny.write_bytes(b"\x01\x02")
    files.append(tiny)
    return files, f


def test_reader_clean_under_sanitizers(driver, tmp_path):
    files, good = corpus(tmp_path)
    out = run(driver, files)
    assert f"files {len(files)} opened 2 " in out, out  # the two well-formed checkpoints open


def test_reader_mutation_sweep(driver, tmp_path):
    _, good = corpus(tmp_path)
    mut = tmp_path / "m.safetensors"
    shutil.copy(good, mut)
    out = run(driver, ["--mutate", 7, 3000, mut])
    assert "files 3000 " in out, out
