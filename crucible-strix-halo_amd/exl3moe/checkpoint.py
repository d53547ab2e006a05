"""Safetensors checkpoints through the C-ABI (cx_checkpoint_*): parsed and validated by
the library on the host, tensors exposed as read-only numpy views of the mapped files,
and EXL3 linears uploaded and repacked into device memory (cx_exl3_load_linear)."""
from __future__ import annotations

import ctypes

import numpy as np

from . import CX_CB, check, lib

DTYPES = {0: np.bool_, 1: np.uint8, 2: np.int8, 3: np.int16, 4: np.uint16, 5: np.float16, 6: None, 7: np.int32,
          8: np.uint32, 9: np.float32, 10: np.int64, 11: np.uint64, 12: np.float64}
CODEBOOK_NAMES = {v: k for k, v in CX_CB.items()}


class Checkpoint:
    """One .safetensors file or a directory with model.safetensors.index.json."""

    def __init__(self, path: str):
        h = ctypes.c_void_p()
        check("cx_checkpoint_open", lib().cx_checkpoint_open(str(path).encode(), ctypes.byref(h)))
        self.handle = h.value

    def close(self):
        if self.handle:
            lib().cx_checkpoint_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def names(self) -> list[str]:
        n = lib().cx_checkpoint_count(self.handle)
        return [lib().cx_checkpoint_name(self.handle, i).decode() for i in range(n)]

    def info(self, name: str):
        """(dtype code, shape, host address, bytes)."""
        dt, rank = ctypes.c_int32(), ctypes.c_int32()
        shape = (ctypes.c_int64 * 8)()
        data, nbytes = ctypes.c_void_p(), ctypes.c_uint64()
        check("cx_checkpoint_tensor", lib().cx_checkpoint_tensor(self.handle, name.encode(), ctypes.byref(dt),
                                                                 ctypes.byref(rank), shape, ctypes.byref(data),
                                                                 ctypes.byref(nbytes)))
        return dt.value, tuple(shape[i] for i in range(rank.value)), data.value, nbytes.value

    def tensor(self, name: str) -> np.ndarray:
        """A copy of the tensor's data (BF16 as raw uint16)."""
        dt, shape, addr, nbytes = self.info(name)
        npdt = DTYPES[dt] or np.uint16
        buf = (ctypes.c_char * nbytes).from_address(addr) if nbytes else b""
        return np.frombuffer(bytes(buf), dtype=npdt).reshape(shape)

    def linear_info(self, prefix: str):
        vals = [ctypes.c_int32() for _ in range(4)]
        check("cx_exl3_linear_info", lib().cx_exl3_linear_info(self.handle, prefix.encode(),
                                                               *[ctypes.byref(v) for v in vals]))
        I, O, k2, cb = (v.value for v in vals)
        return I, O, k2, CODEBOOK_NAMES[cb]

    def load_linear(self, prefix: str, device="cuda"):
        """The linear `prefix` as an ops.DeviceLinear (tiles repacked on the device)."""
        import torch
        from . import Matrix
        from .ops import DeviceLinear
        I, O, k2, cb = self.linear_info(prefix)
        tiles = torch.empty(int(lib().cx_exl3_tile_bytes(I, O, k2)) // 4, dtype=torch.int32, device=device)
        suh = torch.empty(I, dtype=torch.float16, device=device)
        svh = torch.empty(O, dtype=torch.float16, device=device)
        staging = torch.empty(I * O * k2 // 16, dtype=torch.uint8, device=device)
        m = Matrix()
        check("cx_exl3_load_linear", lib().cx_exl3_load_linear(
            self.handle, prefix.encode(), ctypes.byref(m), tiles.data_ptr(), suh.data_ptr(), svh.data_ptr(),
            staging.data_ptr(), staging.numel(), None))
        return DeviceLinear(tiles, suh, svh, I, O, k2, cb)
