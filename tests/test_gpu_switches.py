"""Every non-default environment switch of the MoE layer against the oracle.

The switches (CX_PREFILL_NRB, CX_PREFILL_WPG, CX_PREFILL_GEMM, CX_PREFILL_MID,
CX_TALL_SEQMID, CX_DOWN_MID, CX_FUSED_ROUTE, CX_STAGE) are read when a plan is created, so each case
sets them, builds a fresh plan and runs small layers through the kernels they select:
routing indices exact, outputs within rel-L2 <= 1e-3 and max |err| <= 2e-3 * max |y|."""
import numpy as np
import pytest

import oracle as O
from test_gpu_moe import oracle_layer, rel_l2, run_layer

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

ALL = ("CX_PREFILL_NRB", "CX_PREFILL_WPG", "CX_PREFILL_GEMM", "CX_PREFILL_MID", "CX_TALL_SEQMID", "CX_DOWN_MID",
       "CX_FUSED_ROUTE", "CX_STAGE")

# (switches, [(E, topk, M, mode, bits_gu, bits_d)])
PREFILL_RB = [(16, 4, 70, 2, 4, 4), (4, 1, 90, 2, 4, 4), (8, 2, 200, 2, 3, 5)]
TALL = [(8, 2, 500, 2, 3, 5), (4, 2, 300, 2, 2, 8)]
DECODE = [(16, 4, 1, 1, 4, 4), (16, 4, 5, 1, 4, 4), (16, 4, 20, 1, 4, 4), (16, 4, 40, 1, 3, 5)]
CASES = [
    ({"CX_STAGE": "0"}, DECODE),
    ({"CX_STAGE": "0", "CX_DOWN_MID": "1"}, DECODE),
    ({"CX_TALL_SEQMID": "0"}, TALL),
    ({"CX_PREFILL_MID": "0"}, PREFILL_RB),
    ({"CX_PREFILL_NRB": "8"}, PREFILL_RB),
    ({"CX_PREFILL_MID": "0", "CX_PREFILL_WPG": "8"}, PREFILL_RB),
    ({"CX_PREFILL_MID": "0", "CX_PREFILL_WPG": "16"}, PREFILL_RB),
    ({"CX_PREFILL_GEMM": "1"}, PREFILL_RB),
    ({"CX_PREFILL_GEMM": "0"}, TALL),
    ({"CX_DOWN_MID": "0"}, DECODE),
    ({"CX_DOWN_MID": "1"}, DECODE),
    ({"CX_FUSED_ROUTE": "0"}, DECODE),
    ({"CX_FUSED_ROUTE": "1"}, DECODE),
]


@pytest.mark.parametrize("env,cases", CASES, ids=["+".join(f"{k}={v}" for k, v in e.items()) for e, _ in CASES])
def test_switch(monkeypatch, env, cases):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from exl3moe import synth
    for k in ALL:
        monkeypatch.delenv(k, raising=False)
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    for E, k, M, mode, bgu, bd in cases:
        H = Ie = 128 if k == 1 else 256
        plan = synth.device_moe_layer(300 + E + M, E=E, H=H, Ie=Ie, topk=k, bits_gu=bgu, bits_d=bd)
        rng = np.random.default_rng(M + 17 * E)
        x = rng.standard_normal((M, H)).astype(np.float16)
        lg = rng.standard_normal((M, E + 1)).astype(np.float32)
        print(f"switch {env} E={E} k={k} M={M} mode={mode} bits={bgu}/{bd}", flush=True)
        y, sel, wts = run_layer(plan, x, lg, mode)
        rs, rw = O.route(lg, E, k)
        np.testing.assert_array_equal(sel, rs)
        ref = oracle_layer(plan, x, rs, rw)
        e = rel_l2(y, ref)
        print(f"  rel_l2={e:.3e}")
        assert e <= 1e-3
        assert np.abs(y - ref).max() <= 2e-3 * np.abs(ref).max()


@pytest.mark.parametrize("E,H,Ie,k,sizes,bits", [(512, 2048, 512, 10, (1, 3, 8, 17, 24, 40, 64), (4, 4)),
                                                 (16, 256, 256, 4, (1, 5, 33, 64), (4, 4)),
                                                 (3, 128, 128, 2, (50, 64), (4, 4)),
                                                 (512, 2048, 512, 10, (12, 24, 40), (3, 5)),
                                                 (16, 256, 256, 4, (33, 64), (4, 5))])
def test_stage_launch_bitwise(monkeypatch, E, H, Ie, k, sizes, bits):
    """Decode calls with gate/up, mid and down in one launch (the default) against the same
    calls in separate launches: the same GEMM bodies and mid arithmetic, so the outputs,
    selections and weights are bitwise equal; a layer with fewer than 8 routed experts
    leaves some XCDs without entries; down rates above the gate/up rate (3 / 5 and 4 / 5 bits
    per weight) take the mixed-rate instantiations."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from exl3moe import synth
    for key in ALL:
        monkeypatch.delenv(key, raising=False)
    monkeypatch.setenv("CX_STAGE", "0")
    sep = synth.device_moe_layer(500 + E, E=E, H=H, Ie=Ie, topk=k, bits_gu=bits[0], bits_d=bits[1])
    monkeypatch.delenv("CX_STAGE")
    one = synth.device_moe_layer(500 + E, E=E, H=H, Ie=Ie, topk=k, bits_gu=bits[0], bits_d=bits[1])
    rng = np.random.default_rng(E)
    for M in sizes:
        print(f"stage launch E={E} M={M}", flush=True)
        x = rng.standard_normal((M, H)).astype(np.float16)
        lg = rng.standard_normal((M, E + 1)).astype(np.float32)
        if M * (k + 1) > 128:  # the stage launch's range: its counters make the workspace larger
            assert one.workspace_size(M, 1) > sep.workspace_size(M, 1), M
        ya, sa, wa = run_layer(sep, x, lg, 1)
        yb, sb, wb = run_layer(one, x, lg, 1)
        np.testing.assert_array_equal(sa, sb)
        np.testing.assert_array_equal(wa.view(np.uint32), wb.view(np.uint32))
        np.testing.assert_array_equal(ya.view(np.uint32), yb.view(np.uint32))
    # and against the oracle once
    ref = oracle_layer(one, x, sb, wb)
    assert rel_l2(yb, ref) <= 1e-3
