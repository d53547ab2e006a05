"""GPU parity of the MoE path (C-ABI, HIP kernels) against the CPU oracle: routing
indices exact, grouping (counts / offsets / pairs / row ids) exact, layer outputs
rel-L2 <= 1e-3 with max |err| <= 2e-3 * max |y| (BASELINE configs 3-5 and small layers)."""
import numpy as np
import pytest

import oracle as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from exl3moe import ops as _ops
    return _ops


def rel_l2(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def host_lin(lin):
    tr = lin.trellis.cpu().numpy().view(np.uint16)
    bits = lin.k2 / 2
    return O.reconstruct_inner(tr, bits, lin.codebook), lin.suh.cpu().numpy(), lin.svh.cpu().numpy()


def oracle_expert(ex):
    d = {}
    for n, key in (("g", "gate"), ("u", "up"), ("d", "down")):
        w, suh, svh = host_lin(ex[key])
        d["w" + n], d["s" + n], d["v" + n] = w, suh, svh
    return d


def oracle_layer(plan, x, sel, wts):
    """Oracle output for the rows of x (the experts they route to are decoded on demand)."""
    used = sorted(set(sel.ravel().tolist()))
    cache = {e: oracle_expert(plan._experts[e]) for e in used}
    dummy = cache[used[0]]
    experts = [cache.get(e, dummy) for e in range(plan.n_experts)]
    return O.moe_layer(experts, oracle_expert(plan._shared), x, sel, wts)


def test_route_exact(ops):
    rng = np.random.default_rng(0)
    for M, E, k in [(24, 512, 10), (2048, 512, 10), (5, 64, 8), (3, 1000, 16), (7, 1024, 32), (300, 96, 32), (2, 16, 1)]:
        lg = rng.standard_normal((M, E + 1)).astype(np.float32)
        lg[0, 7] = lg[0, 300 % E] = lg[0, 9] = 5.0  # a three-way tie: lower ids first
        sel, wts = ops.route(torch.from_numpy(lg).cuda(), E, k)
        rs, rw = O.route(lg, E, k)
        np.testing.assert_array_equal(sel.cpu().numpy(), rs)
        np.testing.assert_allclose(wts.cpu().numpy(), rw, rtol=2e-6, atol=1e-7)


def test_route_heavy_ties(ops):
    # Logits on a coarse grid: most rounds see several lanes holding the same maximum,
    # so the lowest-id rule decides (standalone router and the fused decode router).
    from exl3moe import synth
    rng = np.random.default_rng(5)
    for M, E, k in [(40, 512, 10), (300, 512, 10), (6, 1000, 16)]:
        lg = (rng.integers(0, 6, size=(M, E + 1)) * 0.5).astype(np.float32)
        lg[:, -1] = rng.standard_normal(M)
        sel, wts = ops.route(torch.from_numpy(lg).cuda(), E, k)
        rs, rw = O.route(lg, E, k)
        np.testing.assert_array_equal(sel.cpu().numpy(), rs)
        np.testing.assert_allclose(wts.cpu().numpy(), rw, rtol=2e-6, atol=1e-7)
    plan = synth.device_moe_layer(13, E=64, H=256, Ie=128, topk=8)
    for M in (1, 17, 64):
        lg = (rng.integers(0, 3, size=(M, 65)) * 1.0).astype(np.float32)
        x = rng.standard_normal((M, 256)).astype(np.float16)
        y, sel, wts = run_layer(plan, x, lg, 1)
        rs, rw = O.route(lg, 64, 8)
        np.testing.assert_array_equal(sel, rs)
        np.testing.assert_allclose(wts, rw, rtol=2e-6, atol=1e-7)
        assert rel_l2(y, oracle_layer(plan, x, rs, rw)) <= 1e-3


def test_route_shared_logit_array(ops):
    rng = np.random.default_rng(1)
    lg = rng.standard_normal((9, 512)).astype(np.float32)
    sh = rng.standard_normal(9).astype(np.float32)
    sel, wts = ops.route(torch.from_numpy(lg).cuda(), 512, 10, torch.from_numpy(sh).cuda())
    rs, rw = O.route(lg, 512, 10, sh)
    np.testing.assert_array_equal(sel.cpu().numpy(), rs)
    np.testing.assert_allclose(wts.cpu().numpy(), rw, rtol=2e-6, atol=1e-7)


def test_group_known_answer(ops):
    # ref/test_prefill.py:31-38
    sel = torch.tensor([[2, 1, 0], [0, 2, 1], [1, 0, 2]], dtype=torch.int32, device="cuda")
    counts, offsets, pairs, rows = ops.group(sel, 4)
    assert counts.tolist() == [3, 3, 3, 0]
    assert offsets.tolist() == [0, 3, 6, 9, 9]
    assert pairs.tolist() == [2, 3, 7, 1, 5, 6, 0, 4, 8]
    assert rows.tolist() == [0, 1, 2, 0, 1, 2, 0, 1, 2]


@pytest.mark.parametrize("M", [1, 8, 40, 204, 205, 2048, 8192])
def test_group_exact(ops, M):
    rng = np.random.default_rng(M)
    E, k = 512, 10
    lg = rng.standard_normal((M, E + 1)).astype(np.float32)
    if M >= 2048:
        from exl3moe import synth
        lg[:, :E] += synth.zipf_bias(rng, E)
    sel, _ = O.route(lg, E, k)
    got = ops.group(torch.from_numpy(sel).cuda(), E)
    want = O.dispatch(sel, E)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g.cpu().numpy(), w)


def run_layer(plan, x, lg, mode, offs=None):
    M = x.shape[0]
    sel = torch.empty(M, plan.topk, dtype=torch.int32, device="cuda")
    wts = torch.empty(M, plan.topk + 1, dtype=torch.float32, device="cuda")
    y = plan(torch.from_numpy(x).cuda(), torch.from_numpy(lg).cuda(), row_offsets=offs, mode=mode, sel=sel, wts=wts)
    return y.cpu().numpy(), sel.cpu().numpy(), wts.cpu().numpy()


@pytest.mark.parametrize("mode", [1, 2])
def test_small_layer(ops, mode):
    from exl3moe import synth
    plan = synth.device_moe_layer(11, E=16, H=256, Ie=128, topk=4)
    rng = np.random.default_rng(2)
    for M in (1, 7, 70):
        x = rng.standard_normal((M, 256)).astype(np.float16)
        lg = rng.standard_normal((M, 17)).astype(np.float32)
        y, sel, wts = run_layer(plan, x, lg, mode)
        rs, rw = O.route(lg, 16, 4)
        np.testing.assert_array_equal(sel, rs)
        ref = oracle_layer(plan, x, rs, rw)
        e = rel_l2(y, ref)
        print(f"small layer mode={mode} M={M} rel_l2={e:.3e}")
        assert e <= 1e-3
        assert np.abs(y - ref).max() <= 2e-3 * np.abs(ref).max()


def test_mixed_rates_layer(ops):
    # Routed gate/up K3 and down K5 (config 5's mix), shared expert at K4 / K6.
    from exl3moe import synth
    plan = synth.device_moe_layer(12, E=8, H=256, Ie=256, topk=2, bits_gu=3, bits_d=5, shared_bits_gu=4,
                                  shared_bits_d=6)
    rng = np.random.default_rng(3)
    for mode, M in ((1, 5), (2, 90)):
        x = rng.standard_normal((M, 256)).astype(np.float16)
        lg = rng.standard_normal((M, 9)).astype(np.float32)
        y, sel, wts = run_layer(plan, x, lg, mode)
        ref = oracle_layer(plan, x, sel, wts)
        assert rel_l2(y, ref) <= 1e-3


@pytest.mark.parametrize("E,k,M,bgu,bd", [(8, 2, 500, 3, 5), (16, 4, 700, 4, 4), (4, 2, 300, 2, 8)])
def test_tall_prefill_layer(ops, E, k, M, bgu, bd):
    # At least 96 rows per expert on average selects the tall prefill GEMM: entries of up to
    # 192 rows (one trellis decode for all of them), partial row blocks at their ends.
    from exl3moe import synth
    plan = synth.device_moe_layer(20 + E, E=E, H=256, Ie=256, topk=k, bits_gu=bgu, bits_d=bd)
    rng = np.random.default_rng(M)
    x = rng.standard_normal((M, 256)).astype(np.float16)
    lg = rng.standard_normal((M, E + 1)).astype(np.float32)
    y, sel, wts = run_layer(plan, x, lg, 2)
    rs, rw = O.route(lg, E, k)
    np.testing.assert_array_equal(sel, rs)
    ref = oracle_layer(plan, x, rs, rw)
    e = rel_l2(y, ref)
    print(f"tall E={E} k={k} M={M} rel_l2={e:.3e}")
    assert e <= 1e-3


def test_smallest_shapes(ops):
    # H = I = 128 (one Hadamard block, the mid rows' LDS at its minimum) and top-1: decode
    # with the mid in the down GEMM's prologue (1, 5 rows) and as a launch of its own (60
    # rows), the register-blocked prefill and the tall prefill, all against the oracle.
    from exl3moe import synth
    for E, k, M, mode in ((4, 1, 1, 1), (4, 1, 5, 1), (4, 1, 60, 1), (4, 1, 90, 2), (2, 1, 300, 2)):
        plan = synth.device_moe_layer(90 + M, E=E, H=128, Ie=128, topk=k)
        rng = np.random.default_rng(M)
        x = rng.standard_normal((M, 128)).astype(np.float16)
        lg = rng.standard_normal((M, E + 1)).astype(np.float32)
        y, sel, wts = run_layer(plan, x, lg, mode)
        rs, rw = O.route(lg, E, k)
        np.testing.assert_array_equal(sel, rs)
        e = rel_l2(y, oracle_layer(plan, x, rs, rw))
        print(f"H=I=128 E={E} k={k} M={M} mode={mode} rel_l2={e:.3e}")
        assert e <= 1e-3


@pytest.mark.parametrize("E,H,Ie,k", [(32, 1024, 1536, 4), (24, 1536, 640, 3)])
def test_uneven_block_counts(ops, E, H, Ie, k):
    # Widths with odd numbers of 128-blocks and column pairs that are not powers of two
    # (I = 1536: 48 gate/up column pairs, above the prologue mid's I <= 1024; I = 640: 5
    # Hadamard blocks; H = 1536: 12 down column blocks): decode with the prologue mid (where
    # it applies), the stage launch and the separate launches, the register-blocked and the
    # tall prefill, every row against the oracle.
    from exl3moe import synth
    plan = synth.device_moe_layer(61 + E, E=E, H=H, Ie=Ie, topk=k)
    rng = np.random.default_rng(E + H)
    for M, mode in ((1, 1), (6, 1), (40, 1), (200, 2), (1200, 2)):
        x = rng.standard_normal((M, H)).astype(np.float16)
        lg = rng.standard_normal((M, E + 1)).astype(np.float32)
        print(f"uneven E={E} H={H} I={Ie} k={k} M={M} mode={mode}", flush=True)
        y, sel, wts = run_layer(plan, x, lg, mode)
        rs, rw = O.route(lg, E, k)
        np.testing.assert_array_equal(sel, rs)
        ref = oracle_layer(plan, x, rs, rw)
        e = rel_l2(y, ref)
        print(f"  rel_l2={e:.3e}")
        assert e <= 1e-3
        assert np.abs(y - ref).max() <= 2e-3 * np.abs(ref).max()


def test_largest_expert_count_and_topk(ops):
    # E = 1024 experts (the library's maximum: 16 logits per routing lane) and top-32 (its
    # maximum top-k, past the row-parallel limits of every kernel), decode (fused routing
    # at <= 16 rows, separate above) and prefill, against the oracle.
    from exl3moe import synth
    plan = synth.device_moe_layer(77, E=1024, H=128, Ie=128, topk=32)
    rng = np.random.default_rng(77)
    for M, mode in ((3, 1), (20, 1), (150, 2)):
        x = rng.standard_normal((M, 128)).astype(np.float16)
        lg = rng.standard_normal((M, 1025)).astype(np.float32)
        print(f"E=1024 k=32 M={M} mode={mode}", flush=True)
        y, sel, wts = run_layer(plan, x, lg, mode)
        rs, rw = O.route(lg, 1024, 32)
        np.testing.assert_array_equal(sel, rs)
        e = rel_l2(y, oracle_layer(plan, x, rs, rw))
        print(f"  rel_l2={e:.3e}")
        assert e <= 1e-3


def test_tall_prefill_mixed_rates(ops):
    # The shared expert at other rates than the routed ones: each GEMM runs as two launches
    # (shared entries, then routed), and the tall gate/up launch computes the mid itself in
    # both.  Every row against the oracle.
    from exl3moe import synth
    E, k, M = 4, 2, 300
    plan = synth.device_moe_layer(41, E=E, H=256, Ie=256, topk=k, bits_gu=3, bits_d=5, shared_bits_gu=4,
                                  shared_bits_d=6)
    rng = np.random.default_rng(5)
    x = rng.standard_normal((M, 256)).astype(np.float16)
    lg = rng.standard_normal((M, E + 1)).astype(np.float32)
    y, sel, wts = run_layer(plan, x, lg, 2)
    rs, rw = O.route(lg, E, k)
    np.testing.assert_array_equal(sel, rs)
    ref = oracle_layer(plan, x, rs, rw)
    e = rel_l2(y, ref)
    print(f"tall mixed rates rel_l2={e:.3e}")
    assert e <= 1e-3


@pytest.mark.parametrize("cb", ["mcg", "3inst"])
def test_layer_other_codebooks(ops, cb):
    # Every matrix of the layer in the mcg or 3inst codebook: decode (4 rows: the mid in the
    # down GEMM's prologue; 40 rows: the mid launch), the register-blocked prefill GEMM
    # (fused mid) and the tall prefill GEMM, against the oracle.
    from exl3moe import synth
    for E, k, M, mode in ((16, 4, 4, 1), (16, 4, 40, 1), (16, 4, 40, 2), (8, 2, 500, 2)):
        plan = synth.device_moe_layer(70 + E, E=E, H=256, Ie=256, topk=k, codebook=cb)
        rng = np.random.default_rng(M + mode)
        x = rng.standard_normal((M, 256)).astype(np.float16)
        lg = rng.standard_normal((M, E + 1)).astype(np.float32)
        y, sel, wts = run_layer(plan, x, lg, mode)
        rs, rw = O.route(lg, E, k)
        np.testing.assert_array_equal(sel, rs)
        e = rel_l2(y, oracle_layer(plan, x, rs, rw))
        print(f"{cb} E={E} k={k} M={M} mode={mode} rel_l2={e:.3e}")
        assert e <= 1e-3


@pytest.fixture(scope="module")
def layer512(ops):
    from exl3moe import synth
    return synth.device_moe_layer(3, E=512, H=2048, Ie=512, topk=10)


def test_decode_rows_invariant_to_batch(ops, layer512):
    # Decode: a row's layer output is bitwise the same whatever other rows share the call
    # (the engine verifies draft rows against rows decoded alone).  Rows are permuted and
    # subsets taken, so the rows' experts group differently in every call.
    rng = np.random.default_rng(44)
    M = 40
    x = rng.standard_normal((M, 2048)).astype(np.float16)
    lg = rng.standard_normal((M, 513)).astype(np.float32)
    full, _, _ = run_layer(layer512, x, lg, 1)
    for rows in ([0], [7, 3], list(range(5, 29)), list(rng.permutation(M)[:17])):
        part, _, _ = run_layer(layer512, np.ascontiguousarray(x[rows]), np.ascontiguousarray(lg[rows]), 1)
        np.testing.assert_array_equal(part.view(np.uint32), full[rows].view(np.uint32))


def test_config3_decode(ops, layer512):
    # 8 ragged sessions of 1..5 rows, hidden fp16 N(0,1), logits fp32 N(0,1).
    from exl3moe import synth
    rng = np.random.default_rng(33)
    offs = synth.sessions(rng, 8, 1, 5)
    M = offs[-1]
    x = rng.standard_normal((M, 2048)).astype(np.float16)
    lg = rng.standard_normal((M, 513)).astype(np.float32)
    y, sel, wts = run_layer(layer512, x, lg, 1, offs)
    rs, rw = O.route(lg, 512, 10)
    np.testing.assert_array_equal(sel, rs)
    ref = oracle_layer(layer512, x, rs, rw)
    e = rel_l2(y, ref)
    print(f"config3 M={M} rel_l2={e:.3e} max_abs={np.abs(y - ref).max():.3e}")
    assert e <= 1e-3
    assert np.abs(y - ref).max() <= 2e-3 * np.abs(ref).max()


def test_config4_prefill(ops, layer512):
    # 2048 tokens with a Zipf(1.1) per-expert router bias; every row against the oracle
    # (about 20 s of OpenMP oracle work on the GPU box's 16 host threads).
    from exl3moe import synth
    rng = np.random.default_rng(44)
    M = 2048
    x = rng.standard_normal((M, 2048)).astype(np.float16)
    lg = rng.standard_normal((M, 513)).astype(np.float32)
    lg[:, :512] += synth.zipf_bias(rng, 512)
    y, sel, wts = run_layer(layer512, x, lg, 2)
    rs, rw = O.route(lg, 512, 10)
    np.testing.assert_array_equal(sel, rs)
    counts = np.bincount(rs.ravel(), minlength=512)
    print(f"config4 expert counts: max={counts.max()} zero={np.sum(counts == 0)}")
    # 0 to ~400 tokens per expert, so experts with no rows are skipped
    assert np.sum(counts == 0) > 0 and 300 <= counts.max() <= 600
    ref = oracle_layer(layer512, x, rs, rw)
    e = rel_l2(y, ref)
    print(f"config4 rel_l2={e:.3e} max_abs={np.abs(y - ref).max():.3e}")
    assert e <= 1e-3
    assert np.abs(y - ref).max() <= 2e-3 * np.abs(ref).max()
    # Row by row too: no single row far off while the whole passes.
    per_row = np.sqrt(((y - ref) ** 2).sum(1) / (ref ** 2).sum(1))
    print(f"config4 worst row rel_l2={per_row.max():.3e}")
    assert per_row.max() <= 2e-3
    # Decode and prefill plans agree on the same rows: they sum K in different fp32 orders,
    # which the fp16 rounding points of the mid step can amplify to ~1e-4, and the prefill
    # keeps the down outputs in fp16 (one rounding, 2^-12 relative rms) as the reference's
    # prefill does (engine/layers/prefill_moe.h:648).
    y2, _, _ = run_layer(layer512, x[:40], lg[:40], 1)
    assert rel_l2(y2, y[:40]) <= 5e-4


@pytest.mark.parametrize("mode", [1, 2])
def test_hc_writeback(ops, mode):
    # H[r, s] += post[r, s] * y[r] over 4 streams, in a strided H (ldh > 4 * hidden), checked
    # against the oracle's layer output on the same routing (engine/layers/moe_rows.h:672-681).
    from exl3moe import synth
    plan = synth.device_moe_layer(13, E=16, H=256, Ie=128, topk=4)
    rng = np.random.default_rng(3)
    M, S, ldh = 37, 4, 4 * 256 + 64
    xh = rng.standard_normal((M, 256)).astype(np.float16)
    lgh = rng.standard_normal((M, 17)).astype(np.float32)
    x = torch.from_numpy(xh).cuda()
    lg = torch.from_numpy(lgh).cuda()
    p = rng.standard_normal((M, S)).astype(np.float32)
    post = torch.from_numpy(p).cuda()
    H0 = rng.standard_normal((M, ldh)).astype(np.float32)
    Hd = torch.from_numpy(H0.copy()).cuda()
    sel = torch.empty(M, 4, dtype=torch.int32, device="cuda")
    wts = torch.empty(M, 5, dtype=torch.float32, device="cuda")
    plan.forward_hc(x, lg, post, Hd, mode=mode, sel=sel, wts=wts)
    got = Hd.cpu().numpy()
    rs, rw = O.route(lgh, 16, 4)
    np.testing.assert_array_equal(sel.cpu().numpy(), rs)
    ref = oracle_layer(plan, xh, rs, rw)
    for s in range(S):
        delta = got[:, s * 256:(s + 1) * 256].astype(np.float64) - H0[:, s * 256:(s + 1) * 256]
        want = p[:, s:s + 1].astype(np.float64) * ref
        assert rel_l2(delta, want) <= 1e-3, s
    np.testing.assert_array_equal(got[:, S * 256:], H0[:, S * 256:])  # padding untouched
    # The write-back is one fp32 multiply-add per element on the plain forward's y.
    y = plan(x, lg, mode=mode).cpu().numpy()
    exp = H0.copy()
    for s in range(S):
        exp[:, s * 256:(s + 1) * 256] += p[:, s:s + 1] * y
    np.testing.assert_allclose(got, exp, rtol=0, atol=1e-5 * float(np.abs(exp).max()))


def test_hc_writeback_config3(ops, layer512):
    # The config-3 shape (E = 512, H = 2048, 24 decode rows) with 2 streams, against the oracle.
    rng = np.random.default_rng(31)
    M, S = 24, 2
    xh = rng.standard_normal((M, 2048)).astype(np.float16)
    lgh = rng.standard_normal((M, 513)).astype(np.float32)
    p = rng.standard_normal((M, S)).astype(np.float32)
    H0 = rng.standard_normal((M, S * 2048)).astype(np.float32)
    Hd = torch.from_numpy(H0.copy()).cuda()
    layer512.forward_hc(torch.from_numpy(xh).cuda(), torch.from_numpy(lgh).cuda(), torch.from_numpy(p).cuda(), Hd,
                        mode=1)
    got = Hd.cpu().numpy().astype(np.float64)
    rs, rw = O.route(lgh, 512, 10)
    ref = oracle_layer(layer512, xh, rs, rw)
    for s in range(S):
        assert rel_l2(got[:, s * 2048:(s + 1) * 2048] - H0[:, s * 2048:(s + 1) * 2048], p[:, s:s + 1] * ref) <= 1e-3


def test_hc_errors(ops):
    from exl3moe import CxError, synth
    plan = synth.device_moe_layer(13, E=16, H=256, Ie=128, topk=4)
    x = torch.zeros(2, 256, dtype=torch.float16, device="cuda")
    lg = torch.zeros(2, 17, dtype=torch.float32, device="cuda")
    post = torch.zeros(2, 4, dtype=torch.float32, device="cuda")
    with pytest.raises(CxError) as e:
        plan.forward_hc(x, lg, post, torch.zeros(2, 3 * 256, device="cuda"))  # ldh < 4 * hidden
    assert e.value.rc == -2
    with pytest.raises(CxError) as e:  # ldh not a multiple of 4 (16-byte rows)
        plan.forward_hc(x, lg, post, torch.zeros(2, 4 * 256 + 2, device="cuda"))
    assert e.value.rc == -2
    with pytest.raises(CxError) as e:  # H not 16-byte aligned
        plan.forward_hc(x, lg, post, torch.zeros(2, 4 * 256 + 5, device="cuda")[:, 1:])
    assert e.value.rc == -2


def test_config5_long_prefill(ops):
    # 8192 tokens through a 512-expert layer with gate/up at 3 bpw and down at 5 bpw
    # (shared expert at the same rates); every row against the oracle.
    from exl3moe import synth
    plan = synth.device_moe_layer(5, E=512, H=2048, Ie=512, topk=10, bits_gu=3, bits_d=5)
    rng = np.random.default_rng(55)
    M = 8192
    x = rng.standard_normal((M, 2048)).astype(np.float16)
    lg = rng.standard_normal((M, 513)).astype(np.float32)
    y, sel, wts = run_layer(plan, x, lg, 2)
    rs, rw = O.route(lg, 512, 10)
    np.testing.assert_array_equal(sel, rs)
    ref = oracle_layer(plan, x, rs, rw)
    e = rel_l2(y, ref)
    print(f"config5 rel_l2={e:.3e} max_abs={np.abs(y - ref).max():.3e}")
    per_row = np.sqrt(((y - ref) ** 2).sum(1) / (ref ** 2).sum(1))
    print(f"config5 worst row rel_l2={per_row.max():.3e}")
    assert per_row.max() <= 2e-3
    assert e <= 1e-3
    assert np.abs(y - ref).max() <= 2e-3 * np.abs(ref).max()


def test_config5_output_head(ops):
    # EXL3 6-bpw head 2048 -> 151936 on the last token of 4 sessions; the output
    # transform works per 128-column block, so every column is checked against the oracle
    # in chunks of 8192 columns (the matching trellis / svh slices).
    from exl3moe import synth
    rng = np.random.default_rng(56)
    tr, suh, svh = synth.linear(rng, 2048, 151936, 6)
    lin = ops.DeviceLinear.from_trellis(tr, suh, svh, 6)
    x = rng.standard_normal((4, 2048)).astype(np.float16)
    y = lin(torch.from_numpy(x).cuda(), row_offsets=[0, 1, 2, 3, 4]).cpu().numpy()
    assert np.all(np.isfinite(y))
    worst = 0.0
    for c0 in range(0, 151936, 8192):
        c1 = min(c0 + 8192, 151936)
        ts = np.ascontiguousarray(tr[:, c0 // 16:c1 // 16])
        ref = O.matvec(x, O.reconstruct_inner(ts, 6), suh, svh[c0:c1], np.float32)
        worst = max(worst, rel_l2(y[:, c0:c1], ref))
    print(f"head worst 8192-column chunk rel_l2={worst:.3e}")
    assert worst <= 1e-3


@pytest.mark.parametrize("mode", [1, 2])
def test_many_experts_layer(ops, mode):
    # E = 600 > 512 (the 16-per-lane router), k = 16: decode (fused group + transforms) and
    # prefill paths on small matrices.
    from exl3moe import synth
    plan = synth.device_moe_layer(17, E=600, H=256, Ie=128, topk=16)
    rng = np.random.default_rng(19)
    for M in (3, 40):
        x = rng.standard_normal((M, 256)).astype(np.float16)
        lg = rng.standard_normal((M, 601)).astype(np.float32)
        y, sel, wts = run_layer(plan, x, lg, mode)
        rs, rw = O.route(lg, 600, 16)
        np.testing.assert_array_equal(sel, rs)
        ref = oracle_layer(plan, x, rs, rw)
        e = rel_l2(y, ref)
        print(f"E=600 k=16 mode={mode} M={M} rel_l2={e:.3e}")
        assert e <= 1e-3


def test_route_nonfinite(ops):
    # NaN ranks and weighs as -inf, +-inf rank as themselves, ids break ties (the oracle's
    # documented order; the reference leaves NaN undefined).
    rng = np.random.default_rng(9)
    for E, k in [(64, 10), (512, 10), (1000, 16)]:
        M = 12
        lg = rng.standard_normal((M, E + 1)).astype(np.float32)
        lg[0, [3, 17, 40]] = np.nan
        lg[1, :] = np.nan
        lg[2, [8, 2]] = np.inf
        lg[3, ::2] = -np.inf
        lg[4, :E - 3] = -np.inf
        lg[5, [1, 5]] = [np.nan, -np.inf]
        lg[6, :] = -np.inf
        lg[7, rng.permutation(E)[:E // 2]] = np.nan
        sel, wts = ops.route(torch.from_numpy(lg).cuda(), E, k)
        rs, rw = O.route(lg, E, k)
        np.testing.assert_array_equal(sel.cpu().numpy(), rs)
        np.testing.assert_allclose(wts.cpu().numpy(), rw, rtol=2e-6, atol=1e-7, equal_nan=True)


@pytest.mark.parametrize("M", [7, 300])
def test_group_drops_out_of_range_ids(ops, M):
    # Ids outside [0, E) are dropped: not counted, no position (offsets[E] < M k shows it);
    # the valid routes keep their stable expert-major order.  Both grouping paths (one
    # workgroup up to 2048 routes, tiled above).
    rng = np.random.default_rng(M)
    E, k = 64, 10
    sel = rng.integers(0, E, size=(M, k)).astype(np.int32)
    bad = rng.random((M, k)) < 0.1
    sel[bad] = rng.choice(np.array([-1, E, E + 7, 1 << 30, -(1 << 31)], dtype=np.int64), size=int(bad.sum()))
    valid = ~bad
    counts, offsets, pairs, rows = [t.cpu().numpy() for t in ops.group(torch.from_numpy(sel).cuda(), E)]
    want_counts = np.bincount(sel[valid], minlength=E)
    np.testing.assert_array_equal(counts, want_counts)
    np.testing.assert_array_equal(offsets, np.concatenate([[0], np.cumsum(want_counts)]))
    flat = sel.ravel()
    idx = np.nonzero(valid.ravel())[0]
    want_pairs = idx[np.argsort(flat[idx], kind="stable")]
    n = int(offsets[E])
    assert n == int(valid.sum()) < M * k
    np.testing.assert_array_equal(pairs[:n], want_pairs)
    np.testing.assert_array_equal(rows[:n], want_pairs // k)


def _poison(ws):
    ws.fill_(0xFF)  # every float in the scratch is a NaN, every int is -1
    return ws


@pytest.mark.parametrize("mode", [1, 2])
def test_workspace_poisoning(ops, layer512, mode):
    # The reference fills scratch with NaN in a debug build (engine/exl3/plans.h:48-62): no
    # output may depend on what the workspace held before the call.
    rng = np.random.default_rng(77)
    M = 24 if mode == 1 else 300
    x = torch.from_numpy(rng.standard_normal((M, 2048)).astype(np.float16)).cuda()
    lg = torch.from_numpy(rng.standard_normal((M, 513)).astype(np.float32)).cuda()
    n = layer512.workspace_size(M, mode)
    clean = layer512(x, lg, mode=mode, workspace=torch.zeros(n, dtype=torch.uint8, device="cuda"))
    for _ in range(2):
        got = layer512(x, lg, mode=mode, workspace=_poison(torch.empty(n, dtype=torch.uint8, device="cuda")))
        assert torch.equal(got.view(torch.int32), clean.view(torch.int32))


def test_workspace_poisoning_linear_group(ops):
    from exl3moe import synth
    rng = np.random.default_rng(78)
    tr, suh, svh = synth.linear(rng, 2048, 4096, 4)
    lin = ops.DeviceLinear.from_trellis(tr, suh, svh, 4)
    for M in (1, 24, 130):
        x = torch.from_numpy(rng.standard_normal((M, 2048)).astype(np.float16)).cuda()
        n = lin.workspace_size(M)
        clean = lin(x, workspace=torch.zeros(n, dtype=torch.uint8, device="cuda"))
        got = lin(x, workspace=_poison(torch.empty(n, dtype=torch.uint8, device="cuda")))
        assert torch.equal(got.view(torch.int32), clean.view(torch.int32))
    sel = torch.from_numpy(rng.integers(0, 512, size=(3000, 10)).astype(np.int32)).cuda()
    want = ops.group(sel, 512)
    got = ops.group(sel, 512, workspace=_poison(torch.empty(1 << 20, dtype=torch.uint8, device="cuda")))
    for a, b in zip(want, got):
        assert torch.equal(a, b)


@pytest.mark.parametrize("mode", [1, 2])
def test_fp32_input(ops, layer512, mode):
    # fp32 hidden states (the engine's x_) in a strided buffer: bitwise the fp16 path on
    # x rounded to fp16, and within tolerance of the oracle.
    rng = np.random.default_rng(90 + mode)
    M = 24 if mode == 1 else 200
    xf = (rng.standard_normal((M, 2048)) * 0.7).astype(np.float32)  # not an fp16 grid
    lgh = rng.standard_normal((M, 513)).astype(np.float32)
    lg = torch.from_numpy(lgh).cuda()
    buf = torch.zeros(M, 2048 + 64, dtype=torch.float32, device="cuda")
    buf[:, :2048] = torch.from_numpy(xf).cuda()
    y32 = layer512(buf[:, :2048], lg, mode=mode).cpu().numpy()
    xh = xf.astype(np.float16)
    y16 = layer512(torch.from_numpy(xh).cuda(), lg, mode=mode).cpu().numpy()
    np.testing.assert_array_equal(y32.view(np.uint32), y16.view(np.uint32))
    rs, rw = O.route(lgh, 512, 10)
    ref = oracle_layer(layer512, xh, rs, rw)
    assert rel_l2(y32, ref) <= 1e-3
