"""Pins the CPU oracle's transforms, matvec, routing, dispatch and MoE layer against
closed forms: the dense +-1 Sylvester matrix (docs/EXL3_FORMAT.md:146-150), the exact
linear algebra of docs/EXL3_FORMAT.md:152-158 in binary64, the dispatch known answer of
ref/test_prefill.py:31-38, brute-force stable sorting, and ref/oracle.py:226-239's
layer algebra in binary64."""
import numpy as np
import pytest

import oracle as O


def dense_had(n=128):
    idx = np.arange(n)
    pc = np.vectorize(lambda v: bin(v).count("1"))(idx[:, None] & idx[None, :])
    return (1.0 - 2.0 * (pc & 1)) / np.sqrt(128.0)


def had64(x):
    h = dense_had()
    sh = x.shape
    return (x.reshape(*sh[:-1], sh[-1] // 128, 128) @ h).reshape(sh)


def test_hadamard_dense_and_involution():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, 256)).astype(np.float32)
    y = O.hadamard(x)
    np.testing.assert_allclose(y, had64(x.astype(np.float64)), rtol=0, atol=2e-6)
    # H H = I up to the fp32 normalisation constant.
    z = O.hadamard(y)
    np.testing.assert_allclose(z, x, atol=2e-5)
    # A basis vector maps to a +-1/sqrt(128) row of the Sylvester matrix.
    e = np.zeros((1, 128), dtype=np.float32)
    e[0, 37] = 1
    np.testing.assert_array_equal(O.hadamard(e)[0], (dense_had()[37] * 0 + np.sign(dense_had()[37])).astype(np.float32) * np.float32(0.088388347648))


def test_hadamard_fp16_scales():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 384)).astype(np.float16)
    pre = np.where(rng.random(384) < 0.5, -1, 1).astype(np.float16)
    post = (rng.uniform(0.5, 1.5, 384) * np.where(rng.random(384) < 0.5, -1, 1)).astype(np.float16)
    y = O.hadamard(x, pre, post)
    want = had64(x.astype(np.float64) * pre) * post
    assert y.dtype == np.float16
    np.testing.assert_allclose(y.astype(np.float64), want, rtol=3e-3, atol=3e-3)
    with pytest.raises(ValueError):
        O.hadamard(np.zeros((2, 100), dtype=np.float32))


def random_linear(rng, I, O_, bits):
    k2 = int(bits * 2)
    trellis = rng.integers(0, 1 << 16, size=(I // 16, O_ // 16, 8 * k2), dtype=np.uint64).astype(np.uint16)
    suh = np.where(rng.random(I) < 0.5, -1, 1).astype(np.float16)
    svh = (rng.uniform(0.5, 1.5, O_) * np.where(rng.random(O_) < 0.5, -1, 1)).astype(np.float16)
    return trellis, suh, svh


@pytest.mark.parametrize("bits", [4, 3, 2.5])
def test_matvec_linear_algebra(bits):
    # y = (H_O (W_hat^T H_I (x * suh))) * svh  (docs/EXL3_FORMAT.md:152-158), binary64.
    rng = np.random.default_rng(11)
    I, O_ = 256, 384
    trellis, suh, svh = random_linear(rng, I, O_, bits)
    w = O.reconstruct_inner(trellis, bits)
    x = rng.standard_normal((4, I)).astype(np.float16)
    y32 = O.matvec(x, w, suh, svh, np.float32)
    y16 = O.matvec(x, w, suh, svh, np.float16)
    want = had64(had64(x.astype(np.float64) * suh) @ w.astype(np.float64)) * svh.astype(np.float64)
    rel = lambda a: np.linalg.norm(a.astype(np.float64) - want) / np.linalg.norm(want)
    assert rel(y32) < 1e-3  # only the fp16 rounding of the transformed input differs
    assert rel(y16) < 2e-3
    # fp16 output follows the fp32 output within fp16 precision.
    np.testing.assert_allclose(y16.astype(np.float32), y32, rtol=1e-2, atol=2e-2 * np.abs(y32).max())


def test_route_against_sort():
    rng = np.random.default_rng(2)
    M, E, k = 37, 64, 10
    logits = rng.standard_normal((M, E + 1)).astype(np.float32)
    logits[3, 5] = logits[3, 9] = logits[3, 11] = 3.0  # ties resolve to the lower id
    sel, wts = O.route(logits, E, k)
    for r in range(M):
        order = sorted(range(E), key=lambda e: (-logits[r, e], e))[:k]
        assert sel[r].tolist() == order
        l = logits[r, order].astype(np.float64)
        w = np.exp(l - l.max())
        np.testing.assert_allclose(wts[r, :k], w / w.sum(), rtol=1e-6)
        np.testing.assert_allclose(wts[r, k], 1 / (1 + np.exp(-float(logits[r, E]))), rtol=1e-6)
    assert sel[3, :3].tolist() == [5, 9, 11]
    shared = rng.standard_normal(M).astype(np.float32)
    _, w2 = O.route(logits[:, :E].copy(), E, k, shared)
    np.testing.assert_allclose(w2[:, k], 1 / (1 + np.exp(-shared.astype(np.float64))), rtol=1e-6)


def test_route_nonfinite_against_sort():
    # NaN ranks and weighs as -inf; +-inf rank as themselves (ids break ties).
    rng = np.random.default_rng(9)
    M, E, k = 12, 64, 10
    logits = rng.standard_normal((M, E + 1)).astype(np.float32)
    logits[0, [3, 17, 40]] = np.nan
    logits[1, :] = np.nan
    logits[2, [8, 2]] = np.inf
    logits[3, ::2] = -np.inf
    logits[4, :E - 3] = -np.inf
    logits[5, [1, 5]] = [np.nan, -np.inf]
    sel, wts = O.route(logits, E, k)
    key = np.where(np.isnan(logits), -np.inf, logits).astype(np.float64)
    for r in range(M):
        order = sorted(range(E), key=lambda e: (-key[r, e], e))[:k]
        assert sel[r].tolist() == order, r
        with np.errstate(invalid="ignore"):
            w = np.exp(key[r, order] - key[r, order[0]])
            np.testing.assert_allclose(wts[r, :k], w / w.sum(), rtol=1e-6)
    assert sel[2, :2].tolist() == [2, 8] and np.isnan(wts[2, :k]).all()
    assert sel[1].tolist() == list(range(k))  # all NaN: ids in order


def test_dispatch_known_answer():
    # ref/test_prefill.py:31-38
    counts, offsets, pairs, rows = O.dispatch(np.array([[2, 1, 0], [0, 2, 1], [1, 0, 2]]), 4)
    assert counts.tolist() == [3, 3, 3, 0]
    assert offsets.tolist() == [0, 3, 6, 9, 9]
    assert pairs.tolist() == [2, 3, 7, 1, 5, 6, 0, 4, 8]
    assert rows.tolist() == [0, 1, 2, 0, 1, 2, 0, 1, 2]
    with pytest.raises(ValueError):
        O.dispatch(np.array([[4]]), 4)


def test_dispatch_stable_sort_bruteforce():
    rng = np.random.default_rng(4)
    for M, E, k in [(1, 8, 2), (33, 512, 10), (500, 16, 4)]:
        sel = np.stack([rng.choice(E, size=k, replace=False) for _ in range(M)]).astype(np.int32)
        counts, offsets, pairs, rows = O.dispatch(sel, E)
        flat = sel.ravel()
        np.testing.assert_array_equal(counts, np.bincount(flat, minlength=E))
        np.testing.assert_array_equal(pairs, np.array(sorted(range(flat.size), key=lambda i: (flat[i], i))))
        np.testing.assert_array_equal(rows, pairs // k)
        assert offsets[0] == 0 and offsets[-1] == M * k


def tiny_layer(rng, E, H, Ie, bits=(4, 4, 4)):
    def expert():
        d = {}
        for name, (I, O_), b in (("g", (H, Ie), bits[0]), ("u", (H, Ie), bits[1]), ("d", (Ie, H), bits[2])):
            tr, suh, svh = random_linear(rng, I, O_, b)
            d["w" + name] = O.reconstruct_inner(tr, b)
            d["s" + name] = suh
            d["v" + name] = svh
        return d
    return [expert() for _ in range(E)], expert()


def test_moe_layer_algebra():
    # ref/oracle.py:226-239 in binary64 with dense Hadamards: y = sum_k w_k down(silu(g) u) + sig(s) shared.
    rng = np.random.default_rng(9)
    E, H, Ie, k, M = 8, 256, 128, 3, 5
    experts, shared = tiny_layer(rng, E, H, Ie)
    x = rng.standard_normal((M, H)).astype(np.float16)
    logits = rng.standard_normal((M, E + 1)).astype(np.float32)
    sel, wts = O.route(logits, E, k)
    y = O.moe_layer(experts, shared, x, sel, wts)

    def lin(ex, n, v):
        return had64(had64(v * ex["s" + n].astype(np.float64)) @ ex["w" + n].astype(np.float64)) * ex["v" + n].astype(np.float64)

    silu = lambda v: v / (1 + np.exp(-v))
    for r in range(M):
        xr = x[r].astype(np.float64)
        want = np.zeros(H)
        for kk in range(k + 1):
            ex = experts[sel[r, kk]] if kk < k else shared
            h = silu(lin(ex, "g", xr)) * lin(ex, "u", xr)
            want += float(wts[r, kk]) * lin(ex, "d", h)
        assert np.linalg.norm(y[r] - want) / np.linalg.norm(want) < 2e-3
    # A single expert batch equals the per-row layer pieces.
    one = O.expert_rows(shared, x)
    for r in range(M):
        xr = x[r].astype(np.float64)
        h = silu(lin(shared, "g", xr)) * lin(shared, "u", xr)
        want = lin(shared, "d", h)
        assert np.linalg.norm(one[r] - want) / np.linalg.norm(want) < 2e-3
