"""Host-side mirror of the reference's EXL3 linear and MoE layer interface over the C-ABI.

Names follow the reference engine: an EXL3 linear (`Lin`, engine/model/flashnext/model.h:40-46)
is a `DeviceLinear`; a layer's experts (`Moe` / `ExpertPtrs`, model.h:71-76, ops.h:673-678)
are a `MoePlan`; `linear`, `route`, `group` and `moe_layer` are the LinJob/RunGroup,
MoeRouteKernel, MoeDispatch and BlockMoe entry points.  Errors raise `CxError`.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import (CX_CB, CX_F16, CX_F32, CX_MOE_AUTO, Expert, Layer, Matrix, check, i32_host, lib, ptr,
               stream_ptr)


def _xdtype(x: torch.Tensor) -> int:
    """CX_F16 / CX_F32 of an activation tensor."""
    return CX_F32 if x.dtype == torch.float32 else CX_F16


def _dev(a: np.ndarray, device="cuda") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


class DeviceLinear:
    """One EXL3 linear on the device: repacked tiles plus fp16 suh/svh."""

    def __init__(self, tiles: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor, in_features: int,
                 out_features: int, k2: int, codebook: str = "mul1"):
        self.tiles, self.suh, self.svh = tiles, suh, svh
        self.in_features, self.out_features, self.k2 = in_features, out_features, k2
        self.codebook = codebook
        self.struct = Matrix(tiles.data_ptr(), suh.data_ptr(), svh.data_ptr(), in_features, out_features, k2,
                             CX_CB[codebook])

    @classmethod
    def from_trellis(cls, trellis: np.ndarray | torch.Tensor, suh, svh, bits: float, codebook: str = "mul1",
                     stream=None) -> "DeviceLinear":
        """Upload checkpoint-order trellis [I/16][O/16][16K] int16 and repack it on the device."""
        k2 = int(round(float(bits) * 2))
        tr = trellis if isinstance(trellis, torch.Tensor) else _dev(np.asarray(trellis).view(np.int16))
        A, B, n = tr.shape
        I, O = 16 * A, 16 * B
        tiles = torch.empty(A * B * n // 2, dtype=torch.int32, device=tr.device)
        check("cx_exl3_repack", lib().cx_exl3_repack(ptr(tr), I, O, k2, ptr(tiles), stream_ptr(stream)))
        suh_t = suh if isinstance(suh, torch.Tensor) else _dev(np.asarray(suh, dtype=np.float16), tr.device)
        svh_t = svh if isinstance(svh, torch.Tensor) else _dev(np.asarray(svh, dtype=np.float16), tr.device)
        return cls(tiles, suh_t, svh_t, I, O, k2, codebook)

    def dequant(self, stream=None) -> torch.Tensor:
        w = torch.empty(self.in_features, self.out_features, dtype=torch.float16, device=self.tiles.device)
        check("cx_exl3_dequant", lib().cx_exl3_dequant(ctypes.byref(self.struct), ptr(w), stream_ptr(stream)))
        return w

    def input_transform(self, x: torch.Tensor, stream=None) -> torch.Tensor:
        """xh fp16 [M][I] in the library's MFMA row order (cx_exl3_input_transform)."""
        assert x.dtype in (torch.float16, torch.float32) and x.stride(1) == 1 and x.shape[1] >= self.in_features
        xh = torch.empty(x.shape[0], self.in_features, dtype=torch.float16, device=x.device)
        check("cx_exl3_input_transform", lib().cx_exl3_input_transform(
            ctypes.byref(self.struct), ptr(x), CX_F32 if x.dtype == torch.float32 else CX_F16, x.stride(0),
            x.shape[0], ptr(xh), stream_ptr(stream)))
        return xh

    def output_transform(self, y_raw: torch.Tensor, out_dtype=torch.float32, stream=None) -> torch.Tensor:
        """WHT128(y_raw) * (norm * svh) per 128-block (cx_exl3_output_transform)."""
        assert y_raw.dtype == torch.float32 and y_raw.is_contiguous() and y_raw.shape[1] == self.out_features
        y = torch.empty(y_raw.shape[0], self.out_features, dtype=out_dtype, device=y_raw.device)
        check("cx_exl3_output_transform", lib().cx_exl3_output_transform(
            ctypes.byref(self.struct), ptr(y_raw), y_raw.shape[0], ptr(y),
            CX_F16 if out_dtype == torch.float16 else CX_F32, stream_ptr(stream)))
        return y

    def workspace_size(self, M: int) -> int:
        return int(lib().cx_exl3_linear_workspace_size(ctypes.byref(self.struct), M))

    def __call__(self, x: torch.Tensor, out_dtype=torch.float32, row_offsets=None, workspace=None,
                 stream=None) -> torch.Tensor:
        M = x.shape[0]
        y = torch.empty(M, self.out_features, dtype=out_dtype, device=x.device)
        self.forward_into(x, y, row_offsets, workspace, stream)
        return y

    def forward_into(self, x, y, row_offsets=None, workspace=None, stream=None):
        M = x.shape[0]
        assert x.dtype in (torch.float16, torch.float32) and x.stride(1) == 1 and x.shape[1] >= self.in_features
        if workspace is None:
            workspace = torch.empty(self.workspace_size(M), dtype=torch.uint8, device=x.device)
        ro = i32_host(row_offsets)
        ns = 0 if row_offsets is None else len(row_offsets) - 1
        yd = CX_F16 if y.dtype == torch.float16 else CX_F32
        check("cx_exl3_linear", lib().cx_exl3_linear(ctypes.byref(self.struct), ptr(x), _xdtype(x), x.stride(0), M,
                                                     ro, ns, ptr(y), yd, ptr(workspace), workspace.numel(),
                                                     stream_ptr(stream)))
        return y


def group_workspace_size(lins, M: int) -> int:
    """Workspace bytes of cx_exl3_group for these DeviceLinears over M rows."""
    from . import Job
    arr = (Job * len(lins))()
    for i, lin in enumerate(lins):
        arr[i] = Job(lin.struct, None, CX_F16, lin.in_features, None, CX_F32, lin.out_features)
    return int(lib().cx_exl3_group_workspace_size(arr, len(lins), M))


def linear_group(jobs, row_offsets=None, workspace=None, stream=None):
    """Runs EXL3 linears over the same rows in one group (cx_exl3_group).  jobs: list of
    (DeviceLinear, x [M][>= I] fp16/fp32, y [M][>= O] fp16/fp32), rows contiguous in the
    last dimension."""
    from . import Job
    M = jobs[0][1].shape[0]
    arr = (Job * len(jobs))()
    for i, (lin, x, y) in enumerate(jobs):
        assert x.shape[0] == M and y.shape[0] == M and x.stride(1) == 1 and y.stride(1) == 1
        assert x.dtype in (torch.float16, torch.float32) and y.dtype in (torch.float16, torch.float32)
        arr[i] = Job(lin.struct, ptr(x), CX_F16 if x.dtype == torch.float16 else CX_F32, x.stride(0), ptr(y),
                     CX_F16 if y.dtype == torch.float16 else CX_F32, y.stride(0))
    if workspace is None:
        n = int(lib().cx_exl3_group_workspace_size(arr, len(jobs), M))
        workspace = torch.empty(max(n, 1), dtype=torch.uint8, device=jobs[0][1].device)
    ro = i32_host(row_offsets)
    ns = 0 if row_offsets is None else len(row_offsets) - 1
    check("cx_exl3_group", lib().cx_exl3_group(arr, len(jobs), M, ro, ns, ptr(workspace), workspace.numel(),
                                               stream_ptr(stream)))


def dense_linear(W: torch.Tensor, x: torch.Tensor, y: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """y = x @ W^T for fp16 W [O][I] and fp32 or fp16 x [M][I] (the router GEMV), fp32 y."""
    O, I = W.shape
    M = x.shape[0]
    assert W.dtype == torch.float16 and W.is_contiguous() and x.shape[1] == I and x.stride(1) == 1
    assert x.dtype in (torch.float16, torch.float32)
    if y is None:
        y = torch.empty(M, O, dtype=torch.float32, device=x.device)
    xd = CX_F16 if x.dtype == torch.float16 else CX_F32
    check("cx_dense_linear", lib().cx_dense_linear(ptr(W), O, I, ptr(x), xd, x.stride(0), M, ptr(y), y.stride(0),
                                                   stream_ptr(stream)))
    return y


def route(logits: torch.Tensor, E: int, topk: int, shared_logit: torch.Tensor | None = None, stream=None):
    M, ld = logits.shape
    sel = torch.empty(M, topk, dtype=torch.int32, device=logits.device)
    wts = torch.empty(M, topk + 1, dtype=torch.float32, device=logits.device)
    check("cx_moe_route", lib().cx_moe_route(ptr(logits), ld, M, E, topk, ptr(shared_logit), ptr(sel), ptr(wts),
                                             stream_ptr(stream)))
    return sel, wts


def group(sel: torch.Tensor, E: int, workspace=None, stream=None):
    M, topk = sel.shape
    dev = sel.device
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
    pairs = torch.empty(M * topk, dtype=torch.int32, device=dev)
    rows = torch.empty(M * topk, dtype=torch.int32, device=dev)
    ws = workspace
    if ws is None:
        ws = torch.empty(max(1, int(lib().cx_moe_group_workspace_size(M, E, topk))), dtype=torch.uint8, device=dev)
    check("cx_moe_group", lib().cx_moe_group(ptr(sel), M, E, topk, ptr(counts), ptr(offsets), ptr(pairs), ptr(rows),
                                             ptr(ws), ws.numel(), stream_ptr(stream)))
    return counts, offsets, pairs, rows


class MoePlan:
    """A MoE layer's device expert tables (cx_moe_plan)."""

    def __init__(self, hidden: int, intermediate: int, experts: list[dict], shared: dict, topk: int):
        self.hidden, self.intermediate, self.topk = hidden, intermediate, topk
        self.n_experts = len(experts)
        self._experts = experts
        self._shared = shared
        arr = (Expert * self.n_experts)(*[Expert(e["gate"].struct, e["up"].struct, e["down"].struct) for e in experts])
        self._arr = arr
        layer = Layer(hidden, intermediate, self.n_experts, topk, arr,
                      Expert(shared["gate"].struct, shared["up"].struct, shared["down"].struct))
        h = ctypes.c_void_p()
        check("cx_moe_plan_create", lib().cx_moe_plan_create(ctypes.byref(layer), ctypes.byref(h)))
        self.handle = h

    def __del__(self):
        # At interpreter exit the module globals may already be gone: the process end
        # releases the device tables then.
        if getattr(self, "handle", None) and lib is not None:
            try:
                lib().cx_moe_plan_destroy(self.handle)
            except Exception:
                pass
            self.handle = None

    def workspace_size(self, M: int, mode: int = CX_MOE_AUTO) -> int:
        return int(lib().cx_moe_layer_workspace_size(self.handle, M, mode))

    def __call__(self, x: torch.Tensor, logits: torch.Tensor, shared_logit: torch.Tensor | None = None,
                 row_offsets=None, mode: int = CX_MOE_AUTO, workspace=None, y=None, sel=None, wts=None, stream=None):
        M = x.shape[0]
        assert x.dtype in (torch.float16, torch.float32) and x.stride(1) == 1 and x.shape[1] >= self.hidden
        assert logits.dtype == torch.float32 and logits.is_contiguous()
        if y is None:
            y = torch.empty(M, self.hidden, dtype=torch.float32, device=x.device)
        if workspace is None:
            workspace = torch.empty(self.workspace_size(M, mode), dtype=torch.uint8, device=x.device)
        ro = i32_host(row_offsets)
        ns = 0 if row_offsets is None else len(row_offsets) - 1
        check("cx_moe_layer_forward", lib().cx_moe_layer_forward(
            self.handle, ptr(x), _xdtype(x), x.stride(0), ptr(logits), logits.shape[1], ptr(shared_logit), M, ro,
            ns, ptr(y), ptr(sel),
            ptr(wts), mode, ptr(workspace), workspace.numel(), stream_ptr(stream)))
        return y

    def forward_hc(self, x: torch.Tensor, logits: torch.Tensor, post: torch.Tensor, H: torch.Tensor,
                   shared_logit: torch.Tensor | None = None, row_offsets=None, mode: int = CX_MOE_AUTO,
                   workspace=None, sel=None, wts=None, stream=None) -> torch.Tensor:
        """The layer with the residual write-back: H[r, s, :] += post[r, s] * y[r, :] for
        H of shape [M, n_streams, hidden] (or [M, ldh] with ldh >= n_streams * hidden)."""
        M = x.shape[0]
        assert x.dtype in (torch.float16, torch.float32) and x.stride(1) == 1 and x.shape[1] >= self.hidden
        assert logits.dtype == torch.float32 and logits.is_contiguous()
        assert post.dtype == torch.float32 and post.is_contiguous() and post.shape[0] == M
        assert H.dtype == torch.float32 and H.shape[0] == M and H.stride(-1) == 1
        n_streams = post.shape[1]
        ldh = H.stride(0)
        if workspace is None:
            workspace = torch.empty(self.workspace_size(M, mode), dtype=torch.uint8, device=x.device)
        ro = i32_host(row_offsets)
        ns = 0 if row_offsets is None else len(row_offsets) - 1
        check("cx_moe_layer_forward_hc", lib().cx_moe_layer_forward_hc(
            self.handle, ptr(x), _xdtype(x), x.stride(0), ptr(logits), logits.shape[1], ptr(shared_logit), M, ro, ns,
            ptr(post), n_streams,
            ptr(H), ldh, ptr(sel), ptr(wts), mode, ptr(workspace), workspace.numel(), stream_ptr(stream)))
        return H
