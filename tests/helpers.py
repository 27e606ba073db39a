"""Shared input generators for the tests (seeded, CPU-side)."""
from __future__ import annotations

import numpy as np
import torch


def random_blocks(m: int, k: int, seed: int, endpoint_low: int = -128) -> np.ndarray:
    """Uniformly random BC4 blocks ``[M, K/16*8]``: every endpoint byte (including -128) and
    every selector pattern occurs."""
    rng = np.random.default_rng(seed)
    blocks = rng.integers(0, 256, size=(m, (k // 16) * 8), dtype=np.uint8)
    view = blocks.reshape(m, k // 16, 8)
    view[:, :, 0] = rng.integers(endpoint_low, 128, size=view.shape[:2]).astype(np.int8).view(np.uint8)
    view[:, :, 1] = rng.integers(endpoint_low, 128, size=view.shape[:2]).astype(np.int8).view(np.uint8)
    return blocks


def lognormal_scales(m: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return (0.02 * np.exp(0.3 * rng.standard_normal(m))).astype(np.float32)


def bf16_vector(shape, seed: int, scale: float = 1.0) -> torch.Tensor:
    generator = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=generator) * scale).to(torch.bfloat16)


def f16_vector(shape, seed: int, scale: float = 1.0) -> torch.Tensor:
    generator = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=generator) * scale).to(torch.float16)


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def config_weight(m: int, k: int, seed: int) -> torch.Tensor:
    """``W ~ N(0, 0.02^2)`` scaled per input channel by ``LogNormal(0, 0.3)``."""
    generator = torch.Generator().manual_seed(seed)
    w = torch.randn((m, k), generator=generator) * 0.02
    s = torch.exp(0.3 * torch.randn(k, generator=generator))
    return w * s[None, :]


def rel_err(reference: np.ndarray, candidate: np.ndarray) -> float:
    reference = np.asarray(reference, dtype=np.float64)
    candidate = np.asarray(candidate, dtype=np.float64)
    return float(np.linalg.norm(candidate - reference) / max(np.linalg.norm(reference), 1e-300))


def max_rel_err_floor(reference: np.ndarray, candidate: np.ndarray) -> float:
    """Largest per-element error relative to max(|ref|, rms(ref))."""
    reference = np.asarray(reference, dtype=np.float64).reshape(-1)
    candidate = np.asarray(candidate, dtype=np.float64).reshape(-1)
    floor = max(float(np.sqrt(np.mean(reference ** 2))), 1e-30)
    return float(np.max(np.abs(candidate - reference) / np.maximum(np.abs(reference), floor)))
