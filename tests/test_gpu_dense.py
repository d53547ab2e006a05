"""GPU parity of the dense fp16-weight linear (the MoE router, cx_dense_linear) against a
binary64 product of the same operands: fp32 x for up to 8 rows (fp32 products), x rounded
to fp16 above that or when given fp16 (MFMA).  Bound: |y - ref| <= 1e-5 * sum |x w| per
output (fp32 accumulation over I <= 4096 terms)."""
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


def check(y, W, x_used):
    w = W.astype(np.float64)
    xs = x_used.astype(np.float64)
    ref = xs @ w.T
    bound = np.abs(xs) @ np.abs(w).T
    err = np.abs(y.astype(np.float64) - ref)
    assert np.all(err <= 1e-5 * bound + 1e-30), float((err / (bound + 1e-30)).max())


@pytest.mark.parametrize("M", [1, 3, 8])
def test_router_gemv_fp32(ops, M):
    rng = np.random.default_rng(M)
    W = (rng.standard_normal((513, 2048)) * 0.05).astype(np.float16)
    x = rng.standard_normal((M, 2048)).astype(np.float32)
    y = ops.dense_linear(torch.from_numpy(W).cuda(), torch.from_numpy(x).cuda()).cpu().numpy()
    check(y, W, x)


@pytest.mark.parametrize("M,dt", [(9, np.float32), (24, np.float32), (200, np.float32), (2048, np.float32),
                                  (1, np.float16), (40, np.float16), (2048, np.float16)])
def test_router_mfma(ops, M, dt):
    rng = np.random.default_rng(M + 7)
    W = (rng.standard_normal((513, 2048)) * 0.05).astype(np.float16)
    x = rng.standard_normal((M, 2048)).astype(dt)
    y = ops.dense_linear(torch.from_numpy(W).cuda(), torch.from_numpy(x).cuda()).cpu().numpy()
    check(y, W, x.astype(np.float16))  # fp16 x, or fp32 x rounded to fp16 as the kernel does


def test_strided_and_small_shapes(ops):
    rng = np.random.default_rng(5)
    W = rng.standard_normal((70, 96)).astype(np.float16)
    xb = rng.standard_normal((20, 128)).astype(np.float32)
    x = torch.from_numpy(xb).cuda()[:, :96]  # ldx = 128
    yb = torch.full((20, 80), 7.0, device="cuda")
    ops.dense_linear(torch.from_numpy(W).cuda(), x, y=yb[:, :70])
    y = yb.cpu().numpy()
    check(y[:, :70], W, xb[:, :96].astype(np.float16))
    assert np.all(y[:, 70:] == 7.0)
    for M in (2, 5):
        ys = ops.dense_linear(torch.from_numpy(W).cuda(), x[:M]).cpu().numpy()
        check(ys, W, xb[:M, :96])


def test_router_then_route(ops):
    # Logits from the router kernel routed on the GPU equal the oracle's routing of the
    # same logits (indices exact).
    rng = np.random.default_rng(9)
    W = (rng.standard_normal((513, 2048)) * 0.05).astype(np.float16)
    x = rng.standard_normal((24, 2048)).astype(np.float32)
    lg = ops.dense_linear(torch.from_numpy(W).cuda(), torch.from_numpy(x).cuda())
    sel, wts = ops.route(lg, 512, 10)
    rs, rw = O.route(lg.cpu().numpy(), 512, 10)
    np.testing.assert_array_equal(sel.cpu().numpy(), rs)
    np.testing.assert_allclose(wts.cpu().numpy(), rw, rtol=1e-5, atol=1e-7)


def test_dense_errors(ops):
    from exl3moe import CxError, lib
    W = torch.zeros(8, 48, dtype=torch.float16, device="cuda")
    x = torch.zeros(2, 48, dtype=torch.float32, device="cuda")
    y = torch.zeros(2, 8, device="cuda")
    rc = lib().cx_dense_linear(W.data_ptr(), 8, 48, x.data_ptr(), 1, 48, 2, y.data_ptr(), 8, None)
    assert rc == -2  # I not a multiple of 32
    rc = lib().cx_dense_linear(W.data_ptr(), 8, 32, x.data_ptr(), 1, 16, 2, y.data_ptr(), 8, None)
    assert rc == -2  # ldx < I
    rc = lib().cx_dense_linear(W.data_ptr(), 8, 32, x.data_ptr(), 5, 48, 2, y.data_ptr(), 8, None)
    assert rc == -1  # dtype
    with pytest.raises(CxError):
        ops.dense_linear(W[:, :32].contiguous(), torch.zeros(2, 32, dtype=torch.float32, device="cuda")[:, :32],
                         y=torch.zeros(2, 4, device="cuda"))  # ldy < O
