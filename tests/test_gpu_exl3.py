"""GPU parity of the EXL3 decode and linear op (C-ABI, HIP kernels) against the CPU oracle.
Dequantized weights: bit-exact.  Linear outputs: rel-L2 <= 1e-3 (fp32 and fp16 outputs)
and max |err| <= 1e-3 * max |y| reported; rows bitwise invariant to M."""
import numpy as np
import pytest

import oracle as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

RATES = [1, 1.5, 2, 2.5, 3, 3.5, 4, 5, 6, 7, 8]


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


@pytest.mark.parametrize("bits", RATES)
def test_dequant_bit_exact_all_rates(ops, bits):
    from exl3moe import synth
    rng = np.random.default_rng(100 + int(bits * 2))
    tr, suh, svh = synth.linear(rng, 256, 384, bits)
    lin = ops.DeviceLinear.from_trellis(tr, suh, svh, bits)
    got = lin.dequant().cpu().numpy()
    want = O.reconstruct_inner(tr, bits, "mul1")
    np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("bits,cb", [(4, "mcg"), (3, "3inst"), (2, "mcg"), (8, "3inst")])
def test_dequant_bit_exact_other_codebooks(ops, bits, cb):
    from exl3moe import synth
    rng = np.random.default_rng(7)
    tr, suh, svh = synth.linear(rng, 128, 256, bits)
    lin = ops.DeviceLinear.from_trellis(tr, suh, svh, bits, codebook=cb)
    got = lin.dequant().cpu().numpy()
    np.testing.assert_array_equal(got.view(np.uint16), O.reconstruct_inner(tr, bits, cb).view(np.uint16))


def test_config1_linear_2048x512(ops):
    # 2048 -> 512 at 4 bpw, x fp16 [1][2048] ~ N(0, 1).
    from exl3moe import synth
    rng = np.random.default_rng(1)
    tr, suh, svh = synth.linear(rng, 2048, 512, 4)
    lin = ops.DeviceLinear.from_trellis(tr, suh, svh, 4)
    w = O.reconstruct_inner(tr, 4)
    np.testing.assert_array_equal(lin.dequant().cpu().numpy().view(np.uint16), w.view(np.uint16))
    x = rng.standard_normal((1, 2048)).astype(np.float16)
    xt = torch.from_numpy(x).cuda()
    y32 = lin(xt, torch.float32).cpu().numpy()
    y16 = lin(xt, torch.float16).cpu().numpy()
    r32 = O.matvec(x, w, suh, svh, np.float32)
    r16 = O.matvec(x, w, suh, svh, np.float16)
    e32, e16 = rel_l2(y32, r32), rel_l2(y16, r16)
    print(f"config1 rel_l2 f32={e32:.3e} f16={e16:.3e} max_abs f32={np.abs(y32 - r32).max():.3e}")
    assert e32 <= 1e-3 and e16 <= 1e-3
    assert np.abs(y32 - r32).max() <= 1e-3 * np.abs(r32).max()


@pytest.mark.parametrize("I,O_", [(2048, 4096), (4096, 2048)])
def test_config2_ragged_gemv(ops, I, O_):
    # 8 sessions x (1 + d) rows, d ~ U{0..4} -> 8..40 rows, 4 bpw.
    from exl3moe import synth
    rng = np.random.default_rng(2 + I)
    tr, suh, svh = synth.linear(rng, I, O_, 4)
    lin = ops.DeviceLinear.from_trellis(tr, suh, svh, 4)
    w = O.reconstruct_inner(tr, 4)
    offs = synth.sessions(rng, 8, 1, 5)
    M = offs[-1]
    x = rng.standard_normal((M, I)).astype(np.float16)
    y = lin(torch.from_numpy(x).cuda(), torch.float32, row_offsets=offs).cpu().numpy()
    ref = O.matvec(x, w, suh, svh, np.float32)
    e = rel_l2(y, ref)
    print(f"config2 {I}->{O_} M={M} rel_l2={e:.3e} max_abs={np.abs(y - ref).max():.3e}")
    assert e <= 1e-3
    assert np.abs(y - ref).max() <= 1e-3 * np.abs(ref).max()


@pytest.mark.parametrize("I,O_", [(2048, 4096), (4096, 2048)])
def test_config2_fp32_input(ops, I, O_):
    # fp32 activations (LinJob.src, engine/exl3/exl3.h:20-33) in a strided buffer: bitwise
    # the fp16 path on x rounded to fp16, and within tolerance of the oracle.
    from exl3moe import synth
    rng = np.random.default_rng(12 + I)
    tr, suh, svh = synth.linear(rng, I, O_, 4)
    lin = ops.DeviceLinear.from_trellis(tr, suh, svh, 4)
    offs = synth.sessions(rng, 8, 1, 5)
    M = offs[-1]
    xf = (rng.standard_normal((M, I)) * 2.3).astype(np.float32)
    buf = torch.zeros(M, I + 40, dtype=torch.float32, device="cuda")
    buf[:, :I] = torch.from_numpy(xf).cuda()
    y32 = lin(buf[:, :I], torch.float32, row_offsets=offs).cpu().numpy()
    xh = xf.astype(np.float16)
    y16 = lin(torch.from_numpy(xh).cuda(), torch.float32, row_offsets=offs).cpu().numpy()
    np.testing.assert_array_equal(y32.view(np.uint32), y16.view(np.uint32))
    ref = O.matvec(xh, O.reconstruct_inner(tr, 4), suh, svh, np.float32)
    assert rel_l2(y32, ref) <= 1e-3


@pytest.mark.parametrize("bits", [1.5, 2.5, 3, 5, 6, 7, 8])
def test_linear_other_rates(ops, bits):
    from exl3moe import synth
    rng = np.random.default_rng(int(bits * 10))
    tr, suh, svh = synth.linear(rng, 512, 256, bits)
    lin = ops.DeviceLinear.from_trellis(tr, suh, svh, bits)
    x = rng.standard_normal((19, 512)).astype(np.float16)
    y = lin(torch.from_numpy(x).cuda(), torch.float32).cpu().numpy()
    ref = O.matvec(x, O.reconstruct_inner(tr, bits), suh, svh, np.float32)
    assert rel_l2(y, ref) <= 1e-3


@pytest.mark.parametrize("bits,cb", [(4, "mcg"), (3, "3inst"), (2, "mcg"), (6, "3inst")])
def test_linear_other_codebooks(ops, bits, cb):
    # The mcg and 3inst codebooks through the decode GEMM (one and several row blocks).
    from exl3moe import synth
    rng = np.random.default_rng(int(bits * 10) + len(cb))
    tr, suh, svh = synth.linear(rng, 512, 256, bits)
    lin = ops.DeviceLinear.from_trellis(tr, suh, svh, bits, codebook=cb)
    w = O.reconstruct_inner(tr, bits, cb)
    for M in (5, 70):
        x = rng.standard_normal((M, 512)).astype(np.float16)
        y = lin(torch.from_numpy(x).cuda(), torch.float32).cpu().numpy()
        ref = O.matvec(x, w, suh, svh, np.float32)
        assert rel_l2(y, ref) <= 1e-3


def test_rows_invariant_to_batch(ops):
    # A row's output is bitwise the same whatever other rows share the call.
    from exl3moe import synth
    rng = np.random.default_rng(5)
    tr, suh, svh = synth.linear(rng, 2048, 1024, 4)
    lin = ops.DeviceLinear.from_trellis(tr, suh, svh, 4)
    x = torch.from_numpy(rng.standard_normal((70, 2048)).astype(np.float16)).cuda()
    full = lin(x).cpu().numpy()
    for M in (1, 3, 17, 40):
        part = lin(x[:M].contiguous()).cpu().numpy()
        np.testing.assert_array_equal(part.view(np.uint32), full[:M].view(np.uint32))


@pytest.mark.parametrize("I,Ot", [(640, 1536), (1536, 640), (384, 2176)])
def test_linear_uneven_widths(ops, I, Ot):
    # Odd numbers of 128-blocks on either side (K splits of unequal step counts, output
    # column blocks not a power of two): decode and prefill row counts against the oracle,
    # and rows bitwise invariant to the batch.
    from exl3moe import synth
    rng = np.random.default_rng(I + Ot)
    tr, suh, svh = synth.linear(rng, I, Ot, 4)
    lin = ops.DeviceLinear.from_trellis(tr, suh, svh, 4)
    w = O.reconstruct_inner(tr, 4)
    x = rng.standard_normal((300, I)).astype(np.float16)
    xd = torch.from_numpy(x).cuda()
    full = None
    for M in (1, 24, 300):
        y = lin(xd[:M].contiguous(), torch.float32).cpu().numpy()
        ref = O.matvec(x[:M], w, suh, svh, np.float32)
        print(f"linear {I}->{Ot} M={M} rel_l2={rel_l2(y, ref):.3e}")
        assert rel_l2(y, ref) <= 1e-3
        assert np.abs(y - ref).max() <= 1e-3 * np.abs(ref).max()
        if M == 24:
            full = y
        elif M == 1:
            first = y
    np.testing.assert_array_equal(first.view(np.uint32), full[:1].view(np.uint32))


def test_linear_large_m_prefill_rows(ops):
    from exl3moe import synth
    rng = np.random.default_rng(8)
    tr, suh, svh = synth.linear(rng, 1024, 512, 3)
    lin = ops.DeviceLinear.from_trellis(tr, suh, svh, 3)
    x = rng.standard_normal((300, 1024)).astype(np.float16)
    y = lin(torch.from_numpy(x).cuda()).cpu().numpy()
    ref = O.matvec(x, O.reconstruct_inner(tr, 3), suh, svh, np.float32)
    assert rel_l2(y, ref) <= 1e-3


def test_linear_errors(ops):
    from exl3moe import CxError, synth
    rng = np.random.default_rng(9)
    tr, suh, svh = synth.linear(rng, 256, 128, 4)
    lin = ops.DeviceLinear.from_trellis(tr, suh, svh, 4)
    x = torch.zeros(3, 256, dtype=torch.float16, device="cuda")
    with pytest.raises(CxError):
        lin(x, row_offsets=[0, 1, 2])  # offsets end at 2, not 3
    small = torch.empty(16, dtype=torch.uint8, device="cuda")
    with pytest.raises(CxError):
        lin(x, workspace=small)


def test_linear_group(ops):
    # Three linears of different shapes, rates and input / output dtypes over the same
    # ragged rows in one group: each job bitwise equal to its own cx_exl3_linear call
    # (fp32 inputs rounded to fp16 first) and within tolerance of the oracle.
    from exl3moe import synth
    rng = np.random.default_rng(21)
    specs = [(2048, 512, 4, np.float16, torch.float32), (512, 1024, 3, np.float32, torch.float16),
             (1024, 256, 6, np.float32, torch.float32)]
    offs = [0, 3, 4, 9, 13]
    M = offs[-1]
    jobs, singles, refs = [], [], []
    for I, Ot, bits, xdt, ydt in specs:
        tr, suh, svh = synth.linear(rng, I, Ot, bits)
        lin = ops.DeviceLinear.from_trellis(tr, suh, svh, bits)
        xb = rng.standard_normal((M, I + 64)).astype(xdt)
        x = torch.from_numpy(xb).cuda()[:, :I]  # strided rows
        y = torch.full((M, Ot + 8), 3.0, dtype=ydt, device="cuda")[:, :Ot]
        jobs.append((lin, x, y))
        x16 = torch.from_numpy(np.ascontiguousarray(xb[:, :I]).astype(np.float16)).cuda()
        singles.append(lin(x16, ydt, row_offsets=offs).cpu().numpy())
        w = O.reconstruct_inner(tr, bits)
        refs.append(O.matvec(xb[:, :I].astype(np.float16), w, suh, svh,
                             np.float32 if ydt == torch.float32 else np.float16))
    ops.linear_group(jobs, row_offsets=offs)
    for (lin, x, y), single, ref in zip(jobs, singles, refs):
        got = y.cpu().numpy()
        np.testing.assert_array_equal(got, single)
        assert rel_l2(got, ref) <= 1e-3
        assert torch.all(y.as_strided((M, 8), (y.stride(0), 1), y.shape[1]) == 3.0)  # padding untouched


def test_linear_group_one_launch_per_rate(ops):
    # 13 jobs at 4 bpw (mul1) over the same ragged rows share GEMM launches (12 + 1 jobs),
    # beside two 3-bpw jobs (one more launch) and an mcg job (a launch of its own): each
    # job bitwise equal to its own cx_exl3_linear call and within tolerance of the oracle.
    from exl3moe import synth
    rng = np.random.default_rng(33)
    specs = [(128 * int(rng.integers(1, 13)), 128 * int(rng.integers(1, 13)), 4, "mul1") for _ in range(13)]
    specs += [(512, 640, 3, "mul1"), (1024, 256, 3, "mul1"), (256, 384, 4, "mcg")]
    offs = [0, 2, 7, 8, 19]
    M = offs[-1]
    jobs, singles, refs = [], [], []
    for I, Ot, bits, cb in specs:
        tr, suh, svh = synth.linear(rng, I, Ot, bits)
        lin = ops.DeviceLinear.from_trellis(tr, suh, svh, bits, codebook=cb)
        x = torch.from_numpy(rng.standard_normal((M, I)).astype(np.float16)).cuda()
        y = torch.empty(M, Ot, dtype=torch.float32, device="cuda")
        jobs.append((lin, x, y))
        singles.append(lin(x, torch.float32, row_offsets=offs).cpu().numpy())
        refs.append(O.matvec(x.cpu().numpy(), O.reconstruct_inner(tr, bits, cb), suh, svh, np.float32))
    ops.linear_group(jobs, row_offsets=offs)
    for (lin, x, y), single, ref in zip(jobs, singles, refs):
        got = y.cpu().numpy()
        np.testing.assert_array_equal(got.view(np.uint32), single.view(np.uint32))
        assert rel_l2(got, ref) <= 1e-3


def test_linear_group_errors(ops):
    from exl3moe import Job, lib, synth
    import ctypes
    rng = np.random.default_rng(2)
    tr, suh, svh = synth.linear(rng, 128, 128, 4)
    lin = ops.DeviceLinear.from_trellis(tr, suh, svh, 4)
    x = torch.zeros(4, 128, dtype=torch.float16, device="cuda")
    y = torch.zeros(4, 128, device="cuda")
    ws = torch.empty(1 << 20, dtype=torch.uint8, device="cuda")
    jobs = (Job * 17)(*[Job(lin.struct, x.data_ptr(), 0, 128, y.data_ptr(), 1, 128)] * 17)
    assert lib().cx_exl3_group(jobs, 17, 4, None, 0, ws.data_ptr(), ws.numel(), None) == -2  # > 16 jobs
    jobs[0].ldx = 100
    assert lib().cx_exl3_group(jobs, 1, 4, None, 0, ws.data_ptr(), ws.numel(), None) == -2  # ldx < I
    jobs[0].ldx = 128
    jobs[0].x_dtype = 9
    assert lib().cx_exl3_group(jobs, 1, 4, None, 0, ws.data_ptr(), ws.numel(), None) == -1
    jobs[0].x_dtype = 0
    assert lib().cx_exl3_group(jobs, 1, 4, None, 0, ws.data_ptr(), 16, None) == -4


def _natural_order(xh):
    # The library's MFMA row order: natural element e of a 128-block sits at
    # 32 (e >> 5) + p(e & 31) (the header's p); gather it back to natural order.
    r = np.arange(32)
    p = 8 * ((r & 7) >> 1) + 4 * (r >> 4) + (r & 1) + 2 * ((r >> 3) & 1)
    n = xh.shape[1]
    e = np.arange(n)
    return xh[:, (e // 32) * 32 + p[e % 32]]


def _same_values(got, want):
    # Bitwise on every nonzero value; an exactly-zero output may carry either sign of zero.
    got = np.asarray(got)
    want = np.asarray(want)
    np.testing.assert_array_equal(got, want)  # +0 == -0
    nz = want != 0
    bits = np.uint16 if got.dtype == np.float16 else np.uint32
    np.testing.assert_array_equal(got[nz].view(bits), want[nz].view(bits))


def _plain_linear(ops, I, O, suh, svh):
    # Transforms read only suh / svh: the tiles are a zero buffer of the right size.
    t = torch.zeros(I * O * 8 // 16 // 4, dtype=torch.int32, device="cuda")
    return ops.DeviceLinear(t, torch.from_numpy(suh).cuda(), torch.from_numpy(svh).cuda(), I, O, 8)


def test_input_transform_bit_exact(ops):
    # The input transform kernel of cx_exl3_linear against the oracle's fp16 Hadamard
    # with pre-scale (ref/exl3_ref.py:140-156), fp16 and fp32 inputs, general fp16 suh.
    rng = np.random.default_rng(21)
    I = 512
    suh = (rng.standard_normal(I) * 1.5).astype(np.float16)
    lin = _plain_linear(ops, I, 256, suh, np.ones(256, np.float16))
    x = (rng.standard_normal((9, I)) * np.array([1, 1e-3, 30, 1, 1, 1, 1, 1, 1])[:, None]).astype(np.float16)
    x[3] = 0
    x[4, ::3] = 0
    want = O.hadamard(x, pre=suh)
    got = _natural_order(lin.input_transform(torch.from_numpy(x).cuda()).cpu().numpy())
    _same_values(got, want)
    # fp32 rows (a strided view): RoundH(x) first.
    xf = np.zeros((5, I + 64), np.float32)
    xf[:, :I] = rng.standard_normal((5, I)).astype(np.float32)
    got = _natural_order(lin.input_transform(torch.from_numpy(xf).cuda()[:, :I]).cpu().numpy())
    _same_values(got, O.hadamard(xf[:, :I].astype(np.float16), pre=suh))


def test_output_transform_bit_exact(ops):
    # fp32 output: WHT128(y) * (norm * svh).  With svh a power of two the two products
    # round alike whatever the association, so the oracle's (WHT(y) * norm) * svh is
    # bitwise the expected value; general svh within one rounding.
    rng = np.random.default_rng(22)
    O_ = 384
    y = (rng.standard_normal((7, O_)) * 10).astype(np.float32)
    y[2] = 0
    svh_p2 = (rng.choice([0.5, 1.0, 2.0], O_) * rng.choice([-1, 1], O_)).astype(np.float16)
    lin = _plain_linear(ops, 128, O_, np.ones(128, np.float16), svh_p2)
    got = lin.output_transform(torch.from_numpy(y).cuda()).cpu().numpy()
    want = O.hadamard(y) * svh_p2.astype(np.float32)
    _same_values(got, want)
    svh = (rng.standard_normal(O_) + 0.1).astype(np.float16)
    lin = _plain_linear(ops, 128, O_, np.ones(128, np.float16), svh)
    got = lin.output_transform(torch.from_numpy(y).cuda()).cpu().numpy()
    want = (O.hadamard(y).astype(np.float64) * svh.astype(np.float64))
    np.testing.assert_allclose(got, want, rtol=2.5e-7, atol=0)
    # fp16 output: fp16(RoundH(WHT(RoundH(y)) * norm) * svh).
    got = lin.output_transform(torch.from_numpy(y).cuda(), torch.float16).cpu().numpy()
    yh = y.astype(np.float16).astype(np.float32)
    want = (O.hadamard(yh).astype(np.float16).astype(np.float32) * svh.astype(np.float32)).astype(np.float16)
    _same_values(got, want)


@pytest.mark.parametrize("seed", range(32))
def test_random_linear(ops, seed):
    # Seeded random widths (128-2048 in 128 steps on either side), rate, codebook, row
    # count (1-300, ragged sessions some of the time), input and output dtypes, and a
    # strided input: outputs against the oracle, and fp32 inputs bitwise equal to the same
    # values rounded to fp16 first.
    from exl3moe import synth
    rng = np.random.default_rng(5000 + seed)
    I, Ot = 128 * int(rng.integers(1, 17)), 128 * int(rng.integers(1, 17))
    cb = str(rng.choice(["mul1", "mul1", "mcg", "3inst"]))
    bits = float(rng.choice(RATES if cb == "mul1" else [2, 3, 4, 5, 6, 7, 8]))
    M = int(rng.integers(1, 301)) if rng.random() < 0.5 else int(rng.integers(1, 41))
    f32_in, f16_out = bool(rng.random() < 0.4), bool(rng.random() < 0.4)
    offs = None
    if M >= 2 and rng.random() < 0.3:
        cuts = np.sort(rng.choice(np.arange(1, M), size=min(7, M - 1), replace=False))
        offs = [0] + cuts.tolist() + [M]
    print(f"random linear seed={seed} {I}->{Ot} bits={bits} cb={cb} M={M} f32_in={f32_in} f16_out={f16_out} "
          f"ragged={offs is not None}", flush=True)
    tr, suh, svh = synth.linear(rng, I, Ot, bits)
    lin = ops.DeviceLinear.from_trellis(tr, suh, svh, bits, codebook=cb)
    xf = rng.standard_normal((M, I + 32)).astype(np.float32)
    xh = xf[:, :I].astype(np.float16)
    x = torch.from_numpy(xf if f32_in else xf.astype(np.float16)).cuda()[:, :I]  # strided rows
    ydt = torch.float16 if f16_out else torch.float32
    y = lin(x, ydt, row_offsets=offs).cpu().numpy()
    if f32_in:
        y16 = lin(torch.from_numpy(np.ascontiguousarray(xh)).cuda(), ydt, row_offsets=offs).cpu().numpy()
        np.testing.assert_array_equal(y.view(np.uint16 if f16_out else np.uint32),
                                      y16.view(np.uint16 if f16_out else np.uint32))
    ref = O.matvec(xh, O.reconstruct_inner(tr, bits, cb), suh, svh, np.float16 if f16_out else np.float32)
    e = rel_l2(y, ref)
    print(f"  rel_l2={e:.3e}")
    assert e <= 1e-3
    assert np.abs(y.astype(np.float64) - ref).max() <= 1e-3 * np.abs(ref).max() + (2e-3 if f16_out else 0)
