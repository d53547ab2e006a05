"""Kernel resource usage of the built library (CPU test over the compiler's remarks).

The Makefile compiles every object with -Rpass-analysis=kernel-resource-usage and keeps the
remarks in _build/<object>.remarks.  Checked here:
* every function the compiler reports is a __global__ kernel: no device function was left
  out of line (a called body reaches LDS, kernel arguments and its stack through flat
  pointers, and its frame lives in scratch memory);
* no kernel has a dynamically sized stack;
* a kernel's scratch holds register spills only (scratch > 0 only with spilled VGPRs);
* the tall prefill GEMM (Exl3GemmTallKernel) uses no scratch at any rate, and neither does
  any kernel at the rates of the BASELINE configurations (3, 4, 5, 6 bits per weight)."""
import re
from pathlib import Path

import pytest

BUILD = Path(__file__).resolve().parent.parent / "crucible-strix-halo_amd" / "_build"


def _kernels():
    files = sorted(BUILD.glob("*.remarks"))
    if not files:
        pytest.skip("library not built with remarks (make -C crucible-strix-halo_amd)")
    out = []
    for f in files:
        cur = None
        for line in f.read_text().splitlines():
            m = re.search(r"remark: Function Name: (\S+)", line)
            if m:
                cur = {"file": f.name, "name": m.group(1)}
                out.append(cur)
                continue
            m = re.search(r"remark:\s+(ScratchSize \[bytes/lane\]|Dynamic Stack|VGPRs Spill): (\S+)", line)
            if m and cur is not None:
                cur[m.group(1)] = m.group(2)
    return out


def test_only_kernels_no_dynamic_stack():
    ks = _kernels()
    assert len(ks) > 500
    for k in ks:
        assert "Kernel" in k["name"], f"{k['file']}: out-of-line device function {k['name']}"
        assert k.get("Dynamic Stack") == "False", f"{k['file']}: {k['name']} has a dynamic stack"


def test_scratch_is_spills_only():
    for k in _kernels():
        scratch = int(k["ScratchSize [bytes/lane]"])
        if scratch:
            assert int(k["VGPRs Spill"]) > 0, f"{k['file']}: {k['name']} uses {scratch} B/lane of scratch, no spills"


def _rate(name):
    m = re.search(r"Kernel(?:ILi|I)(\d+)E", name)
    return int(m.group(1)) if m else None


def test_tall_gemm_and_config_rates_without_scratch():
    ks = _kernels()
    tall = [k for k in ks if "Exl3GemmTallKernel" in k["name"]]
    assert len(tall) == 33  # 11 rates x 3 codebooks
    for k in ks:
        r = _rate(k["name"]) if "Exl3Gemm" in k["name"] else None
        if "Exl3GemmTallKernel" in k["name"] or r in (6, 8, 10, 12):
            assert k["ScratchSize [bytes/lane]"] == "0", f"{k['file']}: {k['name']}"
