"""The library's entry points under HIP graph capture: the MoE layer (decode and prefill)
and an EXL3 linear are recorded into one graph, which is replayed several times with
eager work and synchronizations in between; every replay must match the eager result
bitwise (the entry points record only kernel launches: no allocation, no memset)."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def synth():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from exl3moe import synth as _synth
    return _synth


def test_graph_replays_match_eager(synth):
    from exl3moe import CX_MOE_DECODE, CX_MOE_PREFILL
    plan = synth.device_moe_layer(21, E=64, H=512, Ie=256, topk=8)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5)
    lin = synth.device_linear(gen, 512, 1024, 4)
    rng = np.random.default_rng(8)
    cases = []
    # decode at 13 rows (the mid in the down GEMM's prologue) and at 20 rows (gate/up, mid and
    # down in one stage launch, counters zeroed by the grouping launch), and prefill
    for mode, M in ((CX_MOE_DECODE, 13), (CX_MOE_DECODE, 20), (CX_MOE_PREFILL, 300)):
        x = torch.from_numpy(rng.standard_normal((M, 512)).astype(np.float16)).cuda()
        lg = torch.from_numpy(rng.standard_normal((M, 65)).astype(np.float32)).cuda()
        ws = torch.empty(plan.workspace_size(M, mode), dtype=torch.uint8, device="cuda")
        y = torch.empty(M, 512, dtype=torch.float32, device="cuda")
        sel = torch.empty(M, 8, dtype=torch.int32, device="cuda")
        cases.append((mode, x, lg, ws, y, sel))
    xl = torch.from_numpy(rng.standard_normal((7, 512)).astype(np.float16)).cuda()
    yl = torch.empty(7, 1024, dtype=torch.float32, device="cuda")
    wsl = torch.empty(lin.workspace_size(7), dtype=torch.uint8, device="cuda")
    offs = [0, 2, 3, 7]

    def run_all():
        for mode, x, lg, ws, y, sel in cases:
            plan(x, lg, mode=mode, workspace=ws, y=y, sel=sel)
        lin.forward_into(xl, yl, offs, wsl)

    def outputs():
        return [c[4].clone() for c in cases] + [c[5].clone() for c in cases] + [yl.clone()]

    run_all()
    torch.cuda.synchronize()
    want = [t.cpu().numpy() for t in outputs()]
    # Warm-up on a side stream, as torch's capture requires, then capture.
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run_all()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run_all()
    for rep in range(4):
        for c in cases:  # overwrite outputs and scratch between replays
            c[4].fill_(float("nan"))
            c[5].fill_(-1)
            c[3].fill_(0xAB)
        yl.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = [t.cpu().numpy() for t in outputs()]
        for a, b in zip(got, want):
            np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32), err_msg=f"replay {rep}")
        run_all()  # eager work between replays
        torch.cuda.synchronize()
