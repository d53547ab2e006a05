"""Seeded synthetic EXL3 layers and activations (the BASELINE configurations).

Trellis words are uniform random 16-bit codes, suh random +-1, svh random +-1 times
U(0.5, 1.5), all fp16; activations fp16 N(0, 1); router logits fp32 N(0, 1).
"""
from __future__ import annotations

import numpy as np


def linear(rng: np.random.Generator, I: int, O: int, bits: float):
    k2 = int(round(bits * 2))
    trellis = rng.integers(0, 1 << 16, size=(I // 16, O // 16, 8 * k2), dtype=np.uint16)
    suh = np.where(rng.random(I) < 0.5, -1.0, 1.0).astype(np.float16)
    svh = (rng.uniform(0.5, 1.5, O) * np.where(rng.random(O) < 0.5, -1.0, 1.0)).astype(np.float16)
    return trellis, suh, svh


def expert(rng, H: int, Ie: int, bits_gu: float, bits_d: float):
    return {"gate": linear(rng, H, Ie, bits_gu), "up": linear(rng, H, Ie, bits_gu), "down": linear(rng, Ie, H, bits_d)}


def sessions(rng, n: int, lo: int, hi: int) -> list[int]:
    """Row offsets (exclusive prefix sums) of n sessions of lo..hi rows each."""
    sizes = rng.integers(lo, hi + 1, size=n)
    return [0] + np.cumsum(sizes).tolist()


def zipf_bias(rng, E: int, s: float = 1.1, scale: float = 3.0) -> np.ndarray:
    """Per-expert router bias from Zipf(s) rank weights (a random expert order), scaled so
    expert token counts are skewed (a few hundred tokens on the heaviest experts)."""
    ranks = rng.permutation(E) + 1
    w = ranks.astype(np.float64) ** (-s)
    return (scale * np.log(w / w.mean())).astype(np.float32)
