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


def zipf_bias(rng, E: int, s: float = 1.1, scale: float = 0.23, tail: float = 4.0, knee: float = 0.75) -> np.ndarray:
    """Per-expert router bias from Zipf(s) rank weights (a random expert order): expert token
    counts are skewed from 0 to about 400 at 2048 tokens and top-10.

    scale * log(w / mean w) with w = rank^-s sets the head (the heaviest expert gets ~400-460
    tokens); the ranks past knee * E fall off faster by tail * log(rank / (knee E)), so the
    coldest experts get no tokens at all (~15-20 of 512 at 2048 tokens)."""
    ranks = (rng.permutation(E) + 1).astype(np.float64)
    w = ranks ** (-s)
    b = scale * np.log(w / w.mean()) - tail * np.log(np.maximum(ranks / (knee * E), 1.0))
    return b.astype(np.float32)


def device_linear(gen, I: int, O: int, bits: float, device="cuda", codebook: str = "mul1"):
    """A random EXL3 linear generated on the device (checkpoint-order trellis kept for
    host-side checks), repacked into the library layout."""
    import torch
    from .ops import DeviceLinear
    k2 = int(round(bits * 2))
    tr = torch.randint(-32768, 32768, (I // 16, O // 16, 8 * k2), dtype=torch.int16, device=device, generator=gen)
    suh = (torch.randint(0, 2, (I,), device=device, generator=gen) * 2 - 1).to(torch.float16)
    sign = torch.randint(0, 2, (O,), device=device, generator=gen) * 2 - 1
    svh = ((torch.rand(O, device=device, generator=gen) + 0.5) * sign).to(torch.float16)
    lin = DeviceLinear.from_trellis(tr, suh, svh, bits, codebook)
    lin.trellis = tr
    return lin


def device_moe_layer(seed: int, E: int, H: int, Ie: int, topk: int, bits_gu: float = 4, bits_d: float = 4,
                     shared_bits_gu: float | None = None, shared_bits_d: float | None = None, device="cuda",
                     codebook: str = "mul1"):
    """Seeded synthetic MoE layer on the device: E routed experts plus the shared expert,
    every matrix with the given codebook."""
    import torch
    from .ops import MoePlan
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    sg = bits_gu if shared_bits_gu is None else shared_bits_gu
    sd = bits_d if shared_bits_d is None else shared_bits_d

    def one(bgu, bd):
        return {"gate": device_linear(gen, H, Ie, bgu, device, codebook),
                "up": device_linear(gen, H, Ie, bgu, device, codebook),
                "down": device_linear(gen, Ie, H, bd, device, codebook)}

    experts = [one(bits_gu, bits_d) for _ in range(E)]
    shared = one(sg, sd)
    return MoePlan(H, Ie, experts, shared, topk)


def host_moe_layer(seed: int, E: int, H: int, Ie: int, topk: int, bits_gu: float = 4, bits_d: float = 4):
    """The same kind of layer as device_moe_layer, generated with numpy on the host and
    uploaded: a process built this way runs no GPU kernels but the library's (and the
    uploads), which is what counter-collection runs want."""
    from .ops import DeviceLinear, MoePlan
    rng = np.random.default_rng(seed)

    def lin(I, O, bits):
        tr, suh, svh = linear(rng, I, O, bits)
        d = DeviceLinear.from_trellis(tr.view(np.int16), suh, svh, bits)
        d.trellis = tr  # checkpoint order, kept on the host for host-side checks
        return d

    def one():
        return {"gate": lin(H, Ie, bits_gu), "up": lin(H, Ie, bits_gu), "down": lin(Ie, H, bits_d)}

    experts = [one() for _ in range(E)]
    return MoePlan(H, Ie, experts, one(), topk)
