"""CPU-side checks of the C-ABI library: it loads, exports every symbol that
include/crucible_exl3.h declares, and rejects bad arguments before touching the GPU."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "crucible_exl3.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    names = re.findall(r"\b(cx_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def test_header_declares_entry_points():
    names = declared_functions()
    for must in ["cx_exl3_repack", "cx_exl3_dequant", "cx_exl3_linear", "cx_moe_route", "cx_moe_group",
                 "cx_moe_layer_forward"]:
        assert must in names


def test_library_exports_every_declared_symbol():
    import exl3moe
    L = exl3moe.lib()
    missing = [n for n in declared_functions() if not hasattr(L, n)]
    assert not missing, missing
    assert set(exl3moe.EXPORTED) <= set(declared_functions())
    assert b"gfx950" in L.cx_version()


def test_argument_errors_without_gpu():
    import exl3moe
    L = exl3moe.lib()
    m = exl3moe.Matrix(1, 1, 1, 100, 128, 8, 2)  # in_features not a multiple of 128
    assert L.cx_exl3_dequant(ctypes.byref(m), ctypes.c_void_p(1), None) == -2
    m = exl3moe.Matrix(1, 1, 1, 128, 128, 9, 2)  # 4.5 bits: unsupported
    assert L.cx_exl3_dequant(ctypes.byref(m), ctypes.c_void_p(1), None) == -3
    m = exl3moe.Matrix(1, 1, 1, 128, 128, 5, 1)  # half rate needs mul1
    assert L.cx_exl3_dequant(ctypes.byref(m), ctypes.c_void_p(1), None) == -3
    m = exl3moe.Matrix(None, 1, 1, 128, 128, 8, 2)
    assert L.cx_exl3_dequant(ctypes.byref(m), ctypes.c_void_p(1), None) == -1
    assert L.cx_exl3_repack(None, 128, 128, 8, ctypes.c_void_p(1), None) == -1
    assert L.cx_exl3_tile_bytes(2048, 512, 8) == 2048 * 512 * 4 // 8
    m = exl3moe.Matrix(1, 1, 1, 2048, 512, 8, 2)
    assert L.cx_exl3_linear_workspace_size(ctypes.byref(m), 1) > 0
    # transform hooks: stride, dtype and row checks come before any launch
    assert L.cx_exl3_input_transform(ctypes.byref(m), ctypes.c_void_p(1), 1, 2040, 3, ctypes.c_void_p(1), None) == -2
    assert L.cx_exl3_input_transform(ctypes.byref(m), ctypes.c_void_p(1), 7, 2048, 3, ctypes.c_void_p(1), None) == -1
    assert L.cx_exl3_input_transform(ctypes.byref(m), None, 1, 2048, 3, ctypes.c_void_p(1), None) == -1
    assert L.cx_exl3_output_transform(ctypes.byref(m), ctypes.c_void_p(1), 0, ctypes.c_void_p(1), 1, None) == -2
    assert L.cx_exl3_output_transform(ctypes.byref(m), ctypes.c_void_p(1), 2, ctypes.c_void_p(1), 5, None) == -1
    # rows must match the session offsets
    ro = exl3moe.i32_host([0, 2, 5])
    assert L.cx_exl3_linear(ctypes.byref(m), ctypes.c_void_p(256), 0, 2048, 4, ro, 2, ctypes.c_void_p(256), 1,
                            ctypes.c_void_p(256), 1 << 30, None) == -2
    # activation dtype, row stride and alignment are checked before any launch
    ro = exl3moe.i32_host([0, 2, 4])
    assert L.cx_exl3_linear(ctypes.byref(m), ctypes.c_void_p(256), 3, 2048, 4, ro, 2, ctypes.c_void_p(256), 1,
                            ctypes.c_void_p(256), 1 << 30, None) == -1
    assert L.cx_exl3_linear(ctypes.byref(m), ctypes.c_void_p(256), 1, 2044, 4, ro, 2, ctypes.c_void_p(256), 1,
                            ctypes.c_void_p(256), 1 << 30, None) == -2
    assert L.cx_exl3_linear(ctypes.byref(m), ctypes.c_void_p(258), 0, 2048, 4, ro, 2, ctypes.c_void_p(256), 1,
                            ctypes.c_void_p(256), 1 << 30, None) == -2


def test_workspace_alignment_checked_without_gpu():
    # Workspaces are carved into 256-byte aligned pieces: a misaligned one is a shape error,
    # returned before any launch.
    import exl3moe
    L = exl3moe.lib()
    m = exl3moe.Matrix(1, 1, 1, 2048, 512, 8, 2)
    ro = exl3moe.i32_host([0, 2, 4])
    assert L.cx_exl3_linear(ctypes.byref(m), ctypes.c_void_p(256), 0, 2048, 4, ro, 2, ctypes.c_void_p(256), 1,
                            ctypes.c_void_p(256 + 16), 1 << 30, None) == -2
    one = ctypes.c_void_p(256)
    assert L.cx_moe_group(one, 200, 8, 8, one, one, one, one, ctypes.c_void_p(512 + 64), 1 << 30, None) == -2
