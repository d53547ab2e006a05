"""MoE layers of seeded random shapes, rates, codebooks and row counts against the oracle.

Each case draws E (2-96 experts), top-k (1-min(E, 16)), hidden and expert widths (128-1024
in 128 steps), the codebook, the routed experts' gate/up and down rates (2-8 bits per
weight, and 1.5 / 2.5 / 3.5 for mul1), the shared expert's rates (the same or different), the row count (1-400, ragged sessions some of the time)
and the mode (decode, prefill, auto) from a fixed seed, so the kernels' less common
combinations (mixed rates, which take separate shared and routed launches; few experts,
which leave XCDs without entries; short last row blocks) run against the oracle: routing
indices exact, outputs within rel-L2 <= 1e-3 and max |err| <= 2e-3 * max |y|."""
import numpy as np
import pytest

import oracle as O
from test_gpu_moe import oracle_layer, rel_l2

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

RATES = (2, 3, 4, 5, 6, 7, 8)  # bits per weight: the rates every codebook supports
HALF_RATES = (1.5, 2.5, 3.5)  # mul1 only


def _case(seed):
    rng = np.random.default_rng(seed)
    E = int(rng.integers(2, 97))
    k = int(rng.integers(1, min(E, 16) + 1))
    H = 128 * int(rng.integers(1, 9))
    Ie = 128 * int(rng.integers(1, 9))
    cb = str(rng.choice(["mul1", "mul1", "mcg", "3inst"]))
    rates = RATES + HALF_RATES if cb == "mul1" else RATES
    bgu, bd = (float(b) for b in rng.choice(rates, 2))
    mixed = rng.random() < 0.3
    sgu, sd = (float(b) for b in rng.choice(rates, 2)) if mixed else (bgu, bd)
    M = int(rng.integers(1, 401)) if rng.random() < 0.5 else int(rng.integers(1, 41))
    mode = int(rng.choice([0, 1, 2]))  # auto, decode, prefill
    ragged = rng.random() < 0.3
    return dict(E=E, k=k, H=H, Ie=Ie, bgu=bgu, bd=bd, sgu=sgu, sd=sd, cb=cb, M=M, mode=mode, ragged=ragged)


@pytest.mark.parametrize("seed", range(48))
def test_random_layer(seed):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from exl3moe import synth
    c = _case(1000 + seed)
    print(f"random layer seed={seed} {c}", flush=True)
    plan = synth.device_moe_layer(2000 + seed, E=c["E"], H=c["H"], Ie=c["Ie"], topk=c["k"], bits_gu=c["bgu"],
                                  bits_d=c["bd"], shared_bits_gu=c["sgu"], shared_bits_d=c["sd"], codebook=c["cb"])
    rng = np.random.default_rng(seed)
    M = c["M"]
    x = rng.standard_normal((M, c["H"])).astype(np.float16)
    lg = rng.standard_normal((M, c["E"] + 1)).astype(np.float32)
    offs = None
    if c["ragged"] and M >= 2:
        cuts = np.sort(rng.choice(np.arange(1, M), size=min(7, M - 1), replace=False))
        offs = [0] + cuts.tolist() + [M]
    sel = torch.empty(M, c["k"], dtype=torch.int32, device="cuda")
    wts = torch.empty(M, c["k"] + 1, dtype=torch.float32, device="cuda")
    y = plan(torch.from_numpy(x).cuda(), torch.from_numpy(lg).cuda(), row_offsets=offs, mode=c["mode"], sel=sel,
             wts=wts).cpu().numpy()
    rs, rw = O.route(lg, c["E"], c["k"])
    np.testing.assert_array_equal(sel.cpu().numpy(), rs)
    ref = oracle_layer(plan, x, rs, rw)
    e = rel_l2(y, ref)
    print(f"  rel_l2={e:.3e}")
    assert e <= 1e-3
    assert np.abs(y - ref).max() <= 2e-3 * np.abs(ref).max()
