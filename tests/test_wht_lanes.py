"""Pins the lane network of the device's 128-point WHT (16 lanes x 8 values, signed
cross-lane stages) in both lane layouts against the oracle's natural-order fp32 butterfly
(ref/exl3_ref.py:140-156): the natural layout (lane j holds elements 8j..8j+7, stride-32
partner lane j ^ 4) and the relabelled one of the prefill input transform (physical lane
L holds the elements of lane e = L ^ 3 when L & 4, so the stride-32 partner is lane L ^ 7,
one DPP pattern).  The emulation does what each instruction does in binary32: v + s * p
with s = +-1 (one rounding), then the scale sign(e) * norm."""
import numpy as np
import pytest

import oracle as O

NORM = np.float32(0.088388347648)


def phi(L):
    return L ^ (3 * ((L >> 2) & 1))


def lane_network(x, relabel):
    """x: [128] float32 block -> [128] float32 in element order, as the kernel stores it."""
    e_of = [phi(L) if relabel else L for L in range(16)]
    v = np.array([x[8 * e_of[L]: 8 * e_of[L] + 8] for L in range(16)], dtype=np.float32)
    for st in (1, 2, 4):  # in-lane strides
        for i in range(8):
            if not i & st:
                lo, hi = v[:, i].copy(), v[:, i + st].copy()
                v[:, i], v[:, i + st] = lo + hi, lo - hi
    partners = (1, 2, 7, 8) if relabel else (1, 2, 4, 8)
    for m, px in zip((1, 2, 4, 8), partners):  # element bit m, physical partner lane L ^ px
        p = v[[L ^ px for L in range(16)]].copy()
        s = np.array([-1.0 if e_of[L] & m else 1.0 for L in range(16)], dtype=np.float32)
        assert all(e_of[L ^ px] == e_of[L] ^ m for L in range(16))
        v = v + s[:, None] * p
    sign = np.array([-1.0 if bin(e_of[L]).count("1") & 1 else 1.0 for L in range(16)], dtype=np.float32)
    v = v * (sign * NORM)[:, None]
    out = np.empty(128, dtype=np.float32)
    for L in range(16):
        out[8 * e_of[L]: 8 * e_of[L] + 8] = v[L]
    return out


@pytest.mark.parametrize("relabel", [False, True])
def test_lane_network_matches_oracle(relabel):
    rng = np.random.default_rng(7)
    # fp16-representable inputs over a wide exponent range (the device inputs are fp16
    # products), so the fp32 butterflies round and the operation order matters.
    x = (rng.standard_normal((64, 128)) * np.exp2(rng.integers(-12, 12, (64, 128)))).astype(np.float16)
    x = x.astype(np.float32)
    want = O.hadamard(x.copy())
    for r in range(x.shape[0]):
        got = lane_network(x[r], relabel)
        nz = want[r] != 0
        np.testing.assert_array_equal(got[nz].view(np.uint32), want[r][nz].view(np.uint32))
        assert np.all(got[~nz] == 0)


def test_relabel_is_an_involution_preserving_quads():
    for L in range(16):
        assert phi(phi(L)) == L and phi(L) >> 2 == L >> 2
