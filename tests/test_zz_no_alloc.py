"""The allocation-free MoE layer entry point (cx_moe_layer_forward_static) against the
workspace entry point (cx_moe_layer_forward): same kernels, so bitwise equal outputs,
on two calls in a row (the second with fewer rows, over the scratch the first left)."""
import ctypes

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import exl3moe
    L = exl3moe.lib()
    P, I32 = ctypes.c_void_p, ctypes.c_int32
    L.cx_moe_layer_forward_static.argtypes = [P, P, I32, I32, P, I32, P, I32, P, I32, P, P, P, I32, P]
    L.cx_moe_layer_forward_static.restype = ctypes.c_int
    return L


def _static(L, plan, x, lg, mode, y, sel, wts, offs=None):
    import exl3moe
    ro = exl3moe.i32_host(offs)
    ns = 0 if offs is None else len(offs) - 1
    return L.cx_moe_layer_forward_static(
        plan.handle, x.data_ptr(), exl3moe.CX_F32 if x.dtype == torch.float32 else exl3moe.CX_F16, x.stride(0),
        lg.data_ptr(), lg.shape[1], None, x.shape[0], ro, ns, y.data_ptr(), sel.data_ptr(), wts.data_ptr(), mode,
        exl3moe.stream_ptr())


def _sessions(M, rng):
    """Ragged session offsets over M rows (1 to 5 rows per session)."""
    cuts = [0]
    while cuts[-1] < M:
        cuts.append(min(M, cuts[-1] + int(rng.integers(1, 6))))
    return cuts


@pytest.mark.parametrize("E,H,Ie,k,sizes,mode,xf32", [
    (512, 2048, 512, 10, (40, 7), 1, False),   # config 3 shape, decode
    (16, 256, 128, 4, (300, 33), 2, False),    # small layer, prefill plan
    # fp32 residual rows with a padded row stride and ragged session offsets (the
    # engine's x_ form of the call), decode and prefill
    (512, 2048, 512, 10, (24, 5), 1, True),
    (16, 256, 128, 4, (300, 33), 2, True),
])
def test_static_matches_workspace_entry(lib, E, H, Ie, k, sizes, mode, xf32):
    from exl3moe import synth
    plan = synth.device_moe_layer(3 if E == 512 else 11, E=E, H=H, Ie=Ie, topk=k)
    rng = np.random.default_rng(E + mode)
    for M in sizes:
        print(f"static entry: E={E} M={M} mode={mode} fp32 x={xf32}", flush=True)
        if xf32:
            xs = torch.from_numpy(rng.standard_normal((M, H + 64)).astype(np.float32)).cuda()
            x = xs[:, :H]  # ldx = H + 64
            offs = _sessions(M, rng)
        else:
            x = torch.from_numpy(rng.standard_normal((M, H)).astype(np.float16)).cuda()
            offs = None
        lg = torch.from_numpy(rng.standard_normal((M, E + 1)).astype(np.float32)).cuda()
        sel0 = torch.empty(M, k, dtype=torch.int32, device="cuda")
        wts0 = torch.empty(M, k + 1, dtype=torch.float32, device="cuda")
        want = plan(x, lg, mode=mode, sel=sel0, wts=wts0, row_offsets=offs)
        y = torch.full((M, H), float("nan"), device="cuda")
        sel = torch.empty_like(sel0)
        wts = torch.empty_like(wts0)
        assert _static(lib, plan, x, lg, mode, y, sel, wts, offs) == 0
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int32), want.view(torch.int32))
        assert torch.equal(sel, sel0) and torch.equal(wts.view(torch.int32), wts0.view(torch.int32))


def test_static_rejects_oversize(lib):
    from exl3moe import CX_MOE_PREFILL, synth
    plan = synth.device_moe_layer(11, E=16, H=256, Ie=128, topk=4)
    M = 8192  # the prefill workspace of 8192 rows exceeds the static scratch
    assert plan.workspace_size(M, CX_MOE_PREFILL) > 24 << 20
    x = torch.zeros(M, 256, dtype=torch.float16, device="cuda")
    lg = torch.zeros(M, 17, dtype=torch.float32, device="cuda")
    y = torch.zeros(M, 256, device="cuda")
    sel = torch.empty(M, 4, dtype=torch.int32, device="cuda")
    wts = torch.empty(M, 5, dtype=torch.float32, device="cuda")
    assert _static(lib, plan, x, lg, CX_MOE_PREFILL, y, sel, wts) == -4
