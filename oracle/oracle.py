"""ctypes front end of the CPU oracle (oracle/exl3_oracle.c).

TEST INFRASTRUCTURE ONLY.  tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import this module, as the checker or as the timed CPU
baseline; the product path never does.

Every array crossing the boundary is a NumPy array; fp16 data travels as
np.float16 (bit patterns), fp32 as np.float32.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle_exl3.so"
REF_LANE_PATH = HERE / "_ref" / "libref_lane.so"

CODEBOOKS = {"3inst": 0, "mcg": 1, "mul1": 2}
HAD_SCALE = np.float32(0.088388347648)

_lib = None


def build(force: bool = False) -> None:
    """Compile the oracle library (and the reference lane harness when the reference is present)."""
    if force or not LIB_PATH.exists():
        subprocess.run(["make", "-C", str(HERE), "liboracle_exl3.so"], check=True, capture_output=True)
    if Path(os.environ.get("CRUCIBLE_REF", "/root/reference")).exists():
        subprocess.run(["make", "-C", str(HERE), "ref"], check=True, capture_output=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        P = ctypes.c_void_p
        L.or_f32_to_f16.argtypes = [ctypes.c_float]
        L.or_f32_to_f16.restype = ctypes.c_uint16
        L.or_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.or_f16_to_f32.restype = ctypes.c_float
        L.or_decode_states.argtypes = [P, ctypes.c_int, P]
        L.or_codebook.argtypes = [ctypes.c_uint16, ctypes.c_int]
        L.or_codebook.restype = ctypes.c_uint16
        L.or_tc_perm.argtypes = [ctypes.c_int]
        L.or_tc_perm.restype = ctypes.c_int
        L.or_decode_tile.argtypes = [P, ctypes.c_int, ctypes.c_int, P]
        L.or_reconstruct_inner.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, P]
        L.or_hadamard.argtypes = [P, ctypes.c_int, ctypes.c_long, ctypes.c_int, P, P]
        L.or_matvec.argtypes = [P, ctypes.c_long, P, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, P]
        L.or_route.argtypes = [P, ctypes.c_long, ctypes.c_long, ctypes.c_int, ctypes.c_int, P, P, P]
        L.or_dispatch.argtypes = [P, ctypes.c_long, ctypes.c_int, ctypes.c_int, P, P, P, P]
        L.or_dispatch.restype = ctypes.c_int
        L.or_moe_layer.argtypes = [P, P, P, ctypes.c_long, ctypes.c_int, ctypes.c_int, ctypes.c_int, P, P, P]
        L.or_expert_rows.argtypes = [P, P, ctypes.c_long, ctypes.c_int, ctypes.c_int, P]
        L.or_num_threads.restype = ctypes.c_int
        L.or_set_num_threads.argtypes = [ctypes.c_int]
        L.or_set_num_threads.restype = None
        L.or_valid_k2.argtypes = [ctypes.c_int]
        L.or_valid_k2.restype = ctypes.c_int
        _lib = L
    return _lib


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def k2_of(bits: float) -> int:
    """2 x bits per weight, validated like ref/exl3_ref.py:18-26."""
    bits = float(bits)
    if not np.isfinite(bits) or bits * 2 != int(bits * 2):
        raise ValueError("EXL3 bitrate must be integer or half-integer")
    k2 = int(bits * 2)
    if not lib().or_valid_k2(k2):
        raise ValueError("Supported bitrates: 1..8 and 1.5, 2.5, 3.5")
    return k2


def f32_to_f16_bits(x: float) -> int:
    return int(lib().or_f32_to_f16(float(x)))


def decode_states(tile_words: np.ndarray, bits: float) -> np.ndarray:
    """256 uint16 decoder states of one tile (ref/exl3_ref.py:40-65)."""
    k2 = k2_of(bits)
    w = np.ascontiguousarray(tile_words, dtype=np.uint16).reshape(-1)
    if w.size != 8 * k2:
        raise ValueError("Packed word count does not match bitrate")
    out = np.empty(256, dtype=np.uint16)
    lib().or_decode_states(_p(w), k2, _p(out))
    return out


def codebook(states: np.ndarray, cb: str = "mul1") -> np.ndarray:
    L = lib()
    c = CODEBOOKS[cb]
    s = np.asarray(states, dtype=np.uint16).reshape(-1)
    return np.array([L.or_codebook(int(v), c) for v in s], dtype=np.uint16).view(np.float16)


def codebook_table(cb: str = "mul1") -> np.ndarray:
    """All 65,536 codebook values, fp16."""
    return codebook(np.arange(65536, dtype=np.uint16), cb)


def tc_perm() -> np.ndarray:
    L = lib()
    return np.array([L.or_tc_perm(i) for i in range(256)], dtype=np.int64)


def reconstruct_inner(trellis: np.ndarray, bits: float, cb: str = "mul1") -> np.ndarray:
    """fp16 W_hat [I][O] from trellis [I/16][O/16][16K] (ref/exl3_ref.py:110-119)."""
    k2 = k2_of(bits)
    t = np.ascontiguousarray(trellis).view(np.uint16)
    A, B, n = t.shape
    if n != 8 * k2:
        raise ValueError("trellis last dimension does not match bitrate")
    w = np.empty((16 * A, 16 * B), dtype=np.float16)
    lib().or_reconstruct_inner(_p(t), 16 * A, 16 * B, k2, CODEBOOKS[cb], _p(w))
    return w


def hadamard(x: np.ndarray, pre: np.ndarray | None = None, post: np.ndarray | None = None) -> np.ndarray:
    """ref/exl3_ref.py:140-156 on fp16 or fp32 rows."""
    x = np.array(x, copy=True, order="C")
    if x.dtype not in (np.float16, np.float32) or x.shape[-1] % 128:
        raise ValueError("Hadamard input must be fp16/fp32 with 128-divisible width")
    n = x.shape[-1]
    rows = x.size // n
    pre = None if pre is None else np.ascontiguousarray(pre, dtype=np.float16)
    post = None if post is None else np.ascontiguousarray(post, dtype=np.float16)
    lib().or_hadamard(_p(x), int(x.dtype == np.float16), rows, n, _p(pre), _p(post))
    return x


def matvec(x: np.ndarray, w_hat: np.ndarray, suh: np.ndarray, svh: np.ndarray, out_dtype=np.float32) -> np.ndarray:
    """Rows of x fp16 [M][I] through one EXL3 linear with decoded W_hat [I][O]."""
    x = np.ascontiguousarray(x, dtype=np.float16)
    squeeze = x.ndim == 1
    x2 = x.reshape(-1, x.shape[-1])
    I, O = w_hat.shape
    if x2.shape[1] != I:
        raise ValueError("x width does not match the matrix")
    out_f16 = np.dtype(out_dtype) == np.float16
    y = np.empty((x2.shape[0], O), dtype=np.float16 if out_f16 else np.float32)
    lib().or_matvec(_p(x2), x2.shape[0], _p(np.ascontiguousarray(w_hat, dtype=np.float16)),
                    _p(np.ascontiguousarray(suh, dtype=np.float16)), _p(np.ascontiguousarray(svh, dtype=np.float16)),
                    I, O, int(out_f16), _p(y))
    return y[0] if squeeze else y


def route(logits: np.ndarray, E: int, topk: int, shared_logit: np.ndarray | None = None):
    """sel int32 [M][topk], wts fp32 [M][topk+1] (engine/layers/ops.h:683-713)."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    M, ld = lg.shape
    if shared_logit is None and ld < E + 1:
        raise ValueError("need a shared logit column or array")
    sl = None if shared_logit is None else np.ascontiguousarray(shared_logit, dtype=np.float32)
    sel = np.empty((M, topk), dtype=np.int32)
    wts = np.empty((M, topk + 1), dtype=np.float32)
    lib().or_route(_p(lg), ld, M, E, topk, _p(sl), _p(sel), _p(wts))
    return sel, wts


def dispatch(sel: np.ndarray, E: int):
    """counts, offsets, pairs, row_ids (ref/prefill_ref.py:37-45)."""
    s = np.ascontiguousarray(sel, dtype=np.int32)
    if s.ndim != 2:
        raise ValueError("selection must be [M][topk]")
    M, topk = s.shape
    counts = np.empty(E, dtype=np.int32)
    offsets = np.empty(E + 1, dtype=np.int32)
    pairs = np.empty(M * topk, dtype=np.int32)
    rows = np.empty(M * topk, dtype=np.int32)
    if lib().or_dispatch(_p(s), M, E, topk, _p(counts), _p(offsets), _p(pairs), _p(rows)) != 0:
        raise ValueError("expert IDs must be in range")
    return counts, offsets, pairs, rows


class _Expert(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("wg", "wu", "wd", "sg", "su", "sd", "vg", "vu", "vd")]


def _expert_struct(ex: dict, keep: list) -> _Expert:
    vals = []
    for key in ("wg", "wu", "wd", "sg", "su", "sd", "vg", "vu", "vd"):
        a = np.ascontiguousarray(ex[key], dtype=np.float16)
        keep.append(a)
        vals.append(a.ctypes.data)
    return _Expert(*vals)


def moe_layer(experts: list[dict], shared: dict, x: np.ndarray, sel: np.ndarray, wts: np.ndarray) -> np.ndarray:
    """MoE layer output fp32 [M][H].  experts[e] / shared: dicts of decoded W_hat
    (wg, wu, wd) and scales (sg, su, sd = suh; vg, vu, vd = svh)."""
    keep: list = []
    arr = (_Expert * len(experts))(*[_expert_struct(e, keep) for e in experts])
    sh = _expert_struct(shared, keep)
    x = np.ascontiguousarray(x, dtype=np.float16)
    M, H = x.shape
    Ie = np.asarray(shared["wg"]).shape[1]
    topk = sel.shape[1]
    s = np.ascontiguousarray(sel, dtype=np.int32)
    w = np.ascontiguousarray(wts, dtype=np.float32)
    y = np.empty((M, H), dtype=np.float32)
    lib().or_moe_layer(ctypes.cast(arr, ctypes.c_void_p), ctypes.byref(sh), _p(x), M, H, Ie, topk, _p(s), _p(w), _p(y))
    return y


def expert_rows(ex: dict, x: np.ndarray) -> np.ndarray:
    keep: list = []
    st = _expert_struct(ex, keep)
    x = np.ascontiguousarray(x, dtype=np.float16)
    M, H = x.shape
    Ie = np.asarray(ex["wg"]).shape[1]
    y = np.empty((M, H), dtype=np.float32)
    lib().or_expert_rows(ctypes.byref(st), _p(x), M, H, Ie, _p(y))
    return y


def num_threads() -> int:
    return int(lib().or_num_threads())


def set_num_threads(n: int) -> None:
    lib().or_set_num_threads(int(n))


# ---- the reference's own lane-window code (oracle/_ref), when it was built ----

_ref_lane = None


def ref_lane_available() -> bool:
    return REF_LANE_PATH.exists()


def ref_lane_states(k_code: int, t: int, words_u32: np.ndarray):
    """States of lane t computed by the reference's LaneWindow/LaneStates."""
    global _ref_lane
    if _ref_lane is None:
        _ref_lane = ctypes.CDLL(str(REF_LANE_PATH))
        _ref_lane.ref_lane_states.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                              ctypes.c_void_p, ctypes.c_void_p]
        _ref_lane.ref_lane_states.restype = ctypes.c_int
    w = np.ascontiguousarray(words_u32, dtype=np.uint32)
    st = np.zeros(8, dtype=np.uint32)
    d0 = ctypes.c_int()
    sh = ctypes.c_int()
    rc = _ref_lane.ref_lane_states(k_code, t, _p(w), _p(st), ctypes.byref(d0), ctypes.byref(sh))
    if rc:
        raise ValueError("unsupported width code")
    return (st & 0xFFFF).astype(np.uint16), d0.value, sh.value
