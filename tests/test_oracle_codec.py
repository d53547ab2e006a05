"""Pins the CPU oracle's EXL3 codec (oracle/exl3_oracle.c) against independent checks:
the literal MSB-first bit-ring construction of ref/test_exl3_ref.py:13-31 (rng 91),
the scalar bitcast codebook oracles of ref/test_exl3_ref.py:47-61, the closed forms of
docs/EXL3_FORMAT.md §2-3, exact rational arithmetic for mul1, and the reference's own
lane-window C++ (engine/exl3/kernels/lane_window.h via oracle/_ref) when it was built."""
import struct
from fractions import Fraction

import numpy as np
import pytest

import oracle as O

RATES = [1, 1.5, 2, 2.5, 3, 3.5, 4, 5, 6, 7, 8]


def widths_of(bits):
    return np.full(256, int(bits)) + (np.arange(256) % 2 if bits % 1 else 0)


def literal_pack(symbols, bits):
    """MSB-first symbol stream, MSB-first within uint32, stored as little-endian int16 pairs."""
    stream = "".join(format(int(s), f"0{int(w)}b") for s, w in zip(symbols, widths_of(bits)))
    words = np.array([int(stream[i:i + 32], 2) for i in range(0, len(stream), 32)], dtype="<u4")
    return stream, words.view("<u2")


def literal_states(stream, bits):
    ends = np.cumsum(widths_of(bits))
    n = len(stream)
    return np.array([int("".join(stream[(int(e) - 16 + j) % n] for j in range(16)), 2) for e in ends], dtype=np.uint16)


@pytest.mark.parametrize("bits", RATES)
def test_ring_decode_literal(bits):
    # Same construction as the reference's test_ring_decode (seeded rng 91).
    rng = np.random.default_rng(91)
    symbols = np.array([rng.integers(1 << int(w)) for w in widths_of(bits)])
    stream, words = literal_pack(symbols, bits)
    got = O.decode_states(words, bits)
    np.testing.assert_array_equal(got, literal_states(stream, bits))
    np.testing.assert_array_equal(got & ((1 << widths_of(bits)) - 1), symbols)


@pytest.mark.parametrize("bits", RATES)
def test_ring_decode_random_words(bits):
    # Random storage words (every bit pattern is a valid tile), several tiles per rate,
    # against the literal bit window of docs/EXL3_FORMAT.md:76-84.
    rng = np.random.default_rng(461)
    k2 = int(bits * 2)
    for tile in range(6):
        words = rng.integers(0, 1 << 16, size=8 * k2, dtype=np.uint64).astype(np.uint16)
        if tile == 0:
            words[:] = 0xFFFF
        u32 = words[0::2].astype(np.uint64) | (words[1::2].astype(np.uint64) << 16)
        stream = "".join(format(int(v), "032b") for v in u32)
        np.testing.assert_array_equal(O.decode_states(words, bits), literal_states(stream, bits))


@pytest.mark.skipif(not O.ref_lane_available(), reason="oracle/_ref not built (reference tree absent)")
@pytest.mark.parametrize("bits", RATES)
def test_states_match_reference_lane_window(bits):
    # The reference's own C++ lane window (compiled from its header) must give the same states.
    code = int(bits) if bits % 1 == 0 else int(bits) * 10 + 5
    rng = np.random.default_rng(7)
    k2 = int(bits * 2)
    for _ in range(4):
        words = rng.integers(0, 1 << 16, size=8 * k2, dtype=np.uint64).astype(np.uint16)
        u32 = words[0::2].astype(np.uint32) | (words[1::2].astype(np.uint32) << 16)
        ours = O.decode_states(words, bits)
        for t in range(32):
            st, _, _ = O.ref_lane_states(code, t, u32)
            np.testing.assert_array_equal(st, ours[8 * t:8 * t + 8])


def half_of(bits16):
    return struct.unpack("<e", struct.pack("<H", bits16))[0]


@pytest.mark.parametrize("cb", ["mcg", "3inst"])
def test_other_codebooks_exhaustive(cb):
    # Scalar bitcast oracle of ref/test_exl3_ref.py:47-61 over all 65,536 states.
    states = np.arange(65536, dtype=np.uint64)
    p = (states * (0xCBAC1FED if cb == "mcg" else 89226354) + (0 if cb == "mcg" else 64248484)) & 0xFFFFFFFF
    enc = (p & 0x8FFF8FFF) ^ 0x3B603B60
    lo = (enc & 0xFFFF).astype(np.uint16).view(np.float16).astype(np.float64)
    hi = (enc >> 16).astype(np.uint16).view(np.float16).astype(np.float64)
    want = (lo + hi).astype(np.float16)  # the fp16 sum is exact in binary64: one rounding
    np.testing.assert_array_equal(O.codebook_table(cb).view(np.uint16), want.view(np.uint16))


def test_mul1_exhaustive_exact_rational():
    # mul1 = fp16(h * inv + bias) with ONE rounding (docs/EXL3_FORMAT.md:120-131).
    # Exact rational value, then round-to-nearest-even to fp16 by Python's struct ('e'
    # packing rounds a binary64 correctly; the rational is exactly representable in binary64).
    inv = Fraction(half_of(0x1EEE))
    bias = Fraction(half_of(0xC931))
    table = O.codebook_table("mul1").view(np.uint16)
    for s in range(0, 65536, 1):
        p = (s * 0x83DCD12D) & 0xFFFFFFFF
        b = (p & 255) + ((p >> 8) & 255) + ((p >> 16) & 255) + (p >> 24)
        exact = (1024 + b) * inv + bias
        assert float(exact) == exact
        want = struct.unpack("<H", struct.pack("<e", float(exact)))[0]
        assert table[s] == want, (s, table[s], want)


def test_mul1_known_values():
    # Closed-form spot values: state 0 -> p = 0 -> b = 0 -> fp16(1024 * inv + bias) = -3.453125.
    assert O.codebook(np.array([0], dtype=np.uint16))[0] == np.float16(-3.453125)
    # inv and bias as documented (docs/EXL3_FORMAT.md:123-126).
    assert half_of(0x1EEE) == 0.00676727294921875 and half_of(0xC931) == -10.3828125


def test_tensor_core_perm_closed_form():
    perm = O.tc_perm()
    assert len(np.unique(perm)) == 256
    lane = np.arange(32)
    rows, cols = 2 * (lane % 4), lane // 4
    want = np.stack([rows * 16 + cols, (rows + 1) * 16 + cols, (rows + 8) * 16 + cols, (rows + 9) * 16 + cols,
                     rows * 16 + cols + 8, (rows + 1) * 16 + cols + 8, (rows + 8) * 16 + cols + 8,
                     (rows + 9) * 16 + cols + 8], axis=-1).reshape(256)
    np.testing.assert_array_equal(perm, want)


@pytest.mark.parametrize("bits,cb", [(4, "mul1"), (3, "mul1"), (2.5, "mul1"), (5, "mcg"), (2, "3inst")])
def test_reconstruct_inner_composition(bits, cb):
    # W_hat[16a + r][16b + c] = codebook(state[i]) with (r, c) = perm(i), tiles row-major in (a, b).
    rng = np.random.default_rng(5)
    k2 = int(bits * 2)
    A, B = 3, 5
    trellis = rng.integers(0, 1 << 16, size=(A, B, 8 * k2), dtype=np.uint64).astype(np.uint16)
    w = O.reconstruct_inner(trellis, bits, cb)
    assert w.shape == (48, 80)
    perm = O.tc_perm()
    for a in range(A):
        for b in range(B):
            u32 = trellis[a, b, 0::2].astype(np.uint64) | (trellis[a, b, 1::2].astype(np.uint64) << 16)
            stream = "".join(format(int(v), "032b") for v in u32)
            st = literal_states(stream, bits)
            for i in rng.choice(256, size=24, replace=False):
                r, c = divmod(int(perm[i]), 16)
                want = O.codebook(np.array([st[i]], dtype=np.uint16), cb)[0]
                assert w[16 * a + r, 16 * b + c].view(np.uint16) == want.view(np.uint16)


def test_validation_errors():
    with pytest.raises(ValueError):
        O.decode_states(np.zeros(48, dtype=np.int16), 4)
    for bits in [0, 9, 4.5, 3.2, float("nan")]:
        with pytest.raises(ValueError):
            O.k2_of(bits)


def test_f16_conversion_matches_numpy():
    rng = np.random.default_rng(3)
    vals = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 4000),
        np.array([0.0, -0.0, 65504.0, 65520.0, 65519.99, 6e-8, 3e-8, 2.98e-8, 1e-10, np.inf, -np.inf], dtype=np.float32),
        (np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)),
    ]).astype(np.float32)
    vals = vals[np.isfinite(vals) | np.isinf(vals)]
    ours = np.array([O.f32_to_f16_bits(float(v)) for v in vals], dtype=np.uint16)
    want = vals.astype(np.float16).view(np.uint16)
    nan = np.isnan(vals)
    np.testing.assert_array_equal(ours[~nan], want[~nan])
