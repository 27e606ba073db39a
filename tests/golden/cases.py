"""Seeded inputs of the encoder golden vectors (shared by the generator and the tests)."""
from __future__ import annotations

import math

import torch


def lognormal(z: torch.Tensor, sigma: float) -> torch.Tensor:
    """``exp(sigma * z)`` as float32, evaluated per element in float64 by ``math.exp`` and rounded
    once. torch's vectorised ``exp`` picks its kernel by the CPU's vector ISA and can differ in
    the last bit between hosts; this does not, so the inputs (and the golden hashes of what the
    encoder makes of them) are the same on every x86 host."""
    return torch.tensor([math.exp(sigma * v) for v in z.double().tolist()], dtype=torch.float32)


def _lognormal_columns(m: int, k: int, generator: torch.Generator) -> torch.Tensor:
    w = torch.randn((m, k), generator=generator) * 0.02
    return w * lognormal(torch.randn(k, generator=generator), 0.3)[None, :]


def small_cases() -> dict[str, tuple[torch.Tensor, torch.Tensor, int]]:
    """name -> (weight [M, K] f32, hdiag [K] f32, rows_per_chunk)."""
    g = torch.Generator().manual_seed(20260827)
    cases = {}
    cases["lognormal_64x64_h1"] = (_lognormal_columns(64, 64, g), torch.ones(64), 128)
    h = lognormal(torch.randn(256, generator=g), 0.5)
    cases["lognormal_128x256_hvaried_chunk32"] = (_lognormal_columns(128, 256, g), h, 32)
    # edge rows: all zero (scale clamps to 1e-12), constant, one spike, alternating signs,
    # a ramp, tiny and huge magnitudes, and exact palette endpoints
    k = 48
    rows = [
        torch.zeros(k),
        torch.full((k,), 0.5),
        torch.full((k,), -0.25),
        torch.nn.functional.one_hot(torch.tensor(5), k).float() * 3.0,
        torch.tensor([(-1.0) ** i for i in range(k)]),
        torch.linspace(-1.0, 1.0, k),
        torch.linspace(0.0, 1.0, k),
        torch.randn(k, generator=g) * 1e-30,
        torch.randn(k, generator=g) * 1e30,
        torch.tensor([i / 127.0 for i in range(-24, 24)]),
        torch.randn(k, generator=g).sign(),
        torch.randn(k, generator=g) * 0.02,
    ]
    cases["edge_rows_12x48"] = (torch.stack(rows), torch.ones(k), 5)
    hz = torch.ones(k)
    hz[::3] = 0.0   # zero activation moments: singular least-squares systems
    cases["edge_rows_zero_hdiag"] = (torch.stack(rows), hz, 128)
    return cases


def config1_inputs() -> tuple[torch.Tensor, torch.Tensor]:
    """W 4096x4096 ~ N(0, 0.02^2) * LogNormal(0, 0.3) per input channel."""
    g = torch.Generator().manual_seed(20260827)
    return _lognormal_columns(4096, 4096, g), torch.ones(4096)
