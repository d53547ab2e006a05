"""Every non-default environment switch of the MoE layer against the oracle.

The switches (CX_PREFILL_NRB, CX_PREFILL_WPG, CX_PREFILL_GEMM, CX_PREFILL_MID,
CX_TALL_SEQMID, CX_DOWN_MID, CX_FUSED_ROUTE) are read when a plan is created, so each case
sets them, builds a fresh plan and runs small layers through the kernels they select:
routing indices exact, outputs within rel-L2 <= 1e-3 and max |err| <= 2e-3 * max |y|."""
import numpy as np
import pytest

import oracle as O
from test_gpu_moe import oracle_layer, rel_l2, run_layer

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

ALL = ("CX_PREFILL_NRB", "CX_PREFILL_WPG", "CX_PREFILL_GEMM", "CX_PREFILL_MID", "CX_TALL_SEQMID", "CX_DOWN_MID",
       "CX_FUSED_ROUTE")

# (switches, [(E, topk, M, mode, bits_gu, bits_d)])
PREFILL_RB = [(16, 4, 70, 2, 4, 4), (4, 1, 90, 2, 4, 4), (8, 2, 200, 2, 3, 5)]
TALL = [(8, 2, 500, 2, 3, 5), (4, 2, 300, 2, 2, 8)]
DECODE = [(16, 4, 1, 1, 4, 4), (16, 4, 5, 1, 4, 4), (16, 4, 20, 1, 4, 4), (16, 4, 40, 1, 3, 5)]
CASES = [
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
