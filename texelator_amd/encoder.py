"""BC4 post-training encoder (palette LUT, E3 endpoint search, block packing).

Restates ``texelator/encoder.py`` of the reference. The arithmetic of the endpoint search is
kept step for step (same float32 expressions and reductions) so that, on the CPU, the chosen
endpoints and selectors are identical to the reference's for the same LUT; the code is
organised differently (coefficient lookup tables, candidate loop over a fixed offset list).
The encoder runs on whatever device ``lut`` lives on.
"""
from __future__ import annotations

import hashlib
from pathlib import Path

import numpy as np
import torch

PALETTE_FLOATS = 255 * 255 * 8


def load_palette(path: Path, device: torch.device | str = "cuda") -> torch.Tensor:
    """Read ``palette.bin`` (255*255*8 little-endian float32) as ``[255, 255, 8]`` (``encoder.py:11-16``)."""
    raw = np.fromfile(path, dtype="<f4")
    if raw.size != PALETTE_FLOATS:
        raise ValueError(f"palette has {raw.size} floats, expected {PALETTE_FLOATS}: {path}")
    return torch.from_numpy(raw.reshape(255, 255, 8)).to(device)


def actual_palette(lut: torch.Tensor, endpoint0: torch.Tensor, endpoint1: torch.Tensor) -> torch.Tensor:
    """Palette rows ``lut[e1 + 127, e0 + 127]`` (``encoder.py:19-20``)."""
    return lut[(endpoint1 + 127).long(), (endpoint0 + 127).long()]


def nearest(values: torch.Tensor, palette: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Nearest palette entry per value; the lowest index wins ties (``encoder.py:23-31``)."""
    best_distance = torch.full_like(values, float("inf"))
    best_index = torch.zeros(values.shape, device=values.device, dtype=torch.uint8)
    for slot in range(8):
        distance = (values - palette[:, slot:slot + 1]).abs()
        closer = distance < best_distance
        best_distance = torch.where(closer, distance, best_distance)
        best_index = torch.where(closer, torch.full_like(best_index, slot), best_index)
    return best_index, torch.gather(palette, 1, best_index.long())


def _coefficient_tables(device: torch.device) -> dict[str, torch.Tensor]:
    """Per-selector weights (a, b, c) of ``q = a*u + b*z + c`` in both BC4 modes (``encoder.py:53-70``)."""
    a8 = [1.0, 0.0] + [(8 - s) / 7 for s in range(2, 8)]
    b8 = [0.0, 1.0] + [(s - 1) / 7 for s in range(2, 8)]
    a6 = [1.0, 0.0] + [(6 - s) / 5 for s in range(2, 6)] + [0.0, 0.0]
    b6 = [0.0, 1.0] + [(s - 1) / 5 for s in range(2, 6)] + [0.0, 0.0]
    c6 = [0.0] * 6 + [-1.0, 1.0]
    as_tensor = lambda v: torch.tensor(v, dtype=torch.float32, device=device)  # noqa: E731
    return {"a8": as_tensor(a8), "b8": as_tensor(b8), "a6": as_tensor(a6), "b6": as_tensor(b6), "c6": as_tensor(c6)}


_OFFSETS = [(d0, d1) for d0 in (-1, 0, 1) for d1 in (-1, 0, 1)]


@torch.inference_mode()
def endpoint_opt(weight: torch.Tensor, hdiag: torch.Tensor, scale: torch.Tensor,
                 lut: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Activation-weighted (E3) endpoint projection for one row chunk (``encoder.py:35-102``).

    Returns int16 endpoints ``[rows*K/16]`` and uint8 selectors ``[rows*K/16, 16]``.
    """
    rows, k = weight.shape
    if k % 16:
        raise ValueError(f"K={k} is not divisible by one BC4 block (16)")
    values = (weight.float() / scale[:, None]).clamp(-1, 1).reshape(-1, 16)
    h = hdiag.float().reshape(k // 16, 16).repeat(rows, 1)

    # 1. min/max start
    start0 = torch.round(values.max(1).values * 127).clamp(-127, 127).to(torch.int16)
    start1 = torch.round(values.min(1).values * 127).clamp(-127, 127).to(torch.int16)
    start_index, _ = nearest(values, actual_palette(lut, start0, start1))

    # 2. weighted least squares for (u, z) = (e0/127, e1/127) with selectors fixed
    tables = _coefficient_tables(values.device)
    sel = start_index.long()
    eight = (start0 > start1)[:, None]
    a = torch.where(eight, tables["a8"][sel], tables["a6"][sel])
    b = torch.where(eight, tables["b8"][sel], tables["b6"][sel])
    c = torch.where(eight, torch.zeros_like(values), tables["c6"][sel])
    target = values - c
    saa = (h * a * a).sum(1)
    sbb = (h * b * b).sum(1)
    sab = (h * a * b).sum(1)
    say = (h * a * target).sum(1)
    sby = (h * b * target).sum(1)
    det = saa * sbb - sab * sab
    singular = det.abs() < 1e-12
    det = det.clamp_min(1e-12)
    u = ((say * sbb - sby * sab) / det).clamp(-1, 1)
    z = ((sby * saa - say * sab) / det).clamp(-1, 1)
    u = torch.where(singular, start0.float() / 127, u)
    z = torch.where(singular, start1.float() / 127, z)
    center0 = torch.round(u * 127).to(torch.int16)
    center1 = torch.round(z * 127).to(torch.int16)

    # 3. 3x3 integer neighbourhood, weighted squared error, first strict improvement wins
    best_error = torch.full((values.shape[0],), float("inf"), device=values.device)
    best0, best1, best_index = start0, start1, start_index
    for d0, d1 in _OFFSETS:
        cand0 = (center0 + d0).clamp(-127, 127)
        cand1 = (center1 + d1).clamp(-127, 127)
        cand_index, quantized = nearest(values, actual_palette(lut, cand0, cand1))
        error = (h * (values - quantized).square()).sum(1)
        improved = error < best_error
        best_error = torch.where(improved, error, best_error)
        best0 = torch.where(improved, cand0, best0)
        best1 = torch.where(improved, cand1, best1)
        best_index = torch.where(improved[:, None], cand_index, best_index)
    return best0, best1, best_index


def pack_blocks(endpoint0: torch.Tensor, endpoint1: torch.Tensor, indices: torch.Tensor) -> np.ndarray:
    """``[N, 8]`` uint8 blocks: e0, e1, then 48 selector bits little-endian, 3 per position
    (``encoder.py:105-117``)."""
    e0 = endpoint0.cpu().numpy().astype(np.int8).view(np.uint8)
    e1 = endpoint1.cpu().numpy().astype(np.int8).view(np.uint8)
    sel = indices.cpu().numpy().astype(np.uint64) & np.uint64(7)
    shifts = (3 * np.arange(16, dtype=np.uint64))[None, :]
    field = np.bitwise_or.reduce(sel << shifts, axis=1)
    packed = np.empty((sel.shape[0], 8), dtype=np.uint8)
    packed[:, 0] = e0
    packed[:, 1] = e1
    packed[:, 2:] = field.astype("<u8").view(np.uint8).reshape(-1, 8)[:, :6]
    return packed


def pack_blocks_tensor(endpoint0: torch.Tensor, endpoint1: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
    """:func:`pack_blocks` on the endpoints' own device: ``[N, 8]`` uint8 tensor, same bytes."""
    fields = torch.zeros(indices.shape[0], dtype=torch.int64, device=indices.device)
    for position in range(16):
        fields |= (indices[:, position].to(torch.int64) & 7) << (3 * position)
    packed = torch.empty((indices.shape[0], 8), dtype=torch.uint8, device=indices.device)
    packed[:, 0] = endpoint0.to(torch.int16).to(torch.uint8)     # two's complement byte
    packed[:, 1] = endpoint1.to(torch.int16).to(torch.uint8)
    for byte in range(6):
        packed[:, 2 + byte] = ((fields >> (8 * byte)) & 0xFF).to(torch.uint8)
    return packed


@torch.inference_mode()
def encode_matrix_tensor(weight: torch.Tensor, hdiag: torch.Tensor, lut: torch.Tensor,
                         rows_per_chunk: int = 2048) -> tuple[torch.Tensor, torch.Tensor]:
    """:func:`encode_matrix` kept on ``lut``'s device: ``(blocks [M, K/16*8] uint8, scales [M]
    float32)`` tensors, the same bytes (no host round trip, for building large models)."""
    m, k = map(int, weight.shape)
    if k % 16:
        raise ValueError(f"unsupported K={k}; BC4 needs K % 16 == 0")
    hdiag = hdiag.to(lut.device)
    blocks = torch.empty((m, k // 16 * 8), dtype=torch.uint8, device=lut.device)
    scales = torch.empty(m, dtype=torch.float32, device=lut.device)
    for start in range(0, m, rows_per_chunk):
        rows = weight[start:start + rows_per_chunk].detach().float().to(lut.device)
        row_scales = rows.abs().amax(1).clamp_min(1e-12)
        e0, e1, idx = endpoint_opt(rows, hdiag, row_scales, lut)
        blocks[start:start + rows.shape[0]] = pack_blocks_tensor(e0, e1, idx).reshape(rows.shape[0], -1)
        scales[start:start + rows.shape[0]] = row_scales
    return blocks, scales


@torch.inference_mode()
def encode_rows(weight: torch.Tensor, hdiag: torch.Tensor, lut: torch.Tensor,
                rows_per_chunk: int = 128):
    """Encode a matrix chunk by chunk; yields ``(packed_blocks [rows, K/16*8], scales [rows])``.

    Row scale = ``max |W[m, :]|`` clamped at 1e-12 (``encoder.py:140``).
    """
    m, k = map(int, weight.shape)
    if k % 16:
        raise ValueError(f"unsupported K={k}; BC4 needs K % 16 == 0")
    hdiag = hdiag.to(lut.device)
    for start in range(0, m, rows_per_chunk):
        rows = weight[start:start + rows_per_chunk].detach().float().to(lut.device)
        scales = rows.abs().amax(1).clamp_min(1e-12)
        e0, e1, idx = endpoint_opt(rows, hdiag, scales, lut)
        packed = pack_blocks(e0, e1, idx).reshape(rows.shape[0], -1)
        yield packed, scales.cpu().numpy().astype("<f4", copy=False)


def encode_matrix(weight: torch.Tensor, hdiag: torch.Tensor, lut: torch.Tensor,
                  rows_per_chunk: int = 128) -> tuple[np.ndarray, np.ndarray]:
    """In-memory encode: ``(blocks [M, K/16*8] uint8, scales [M] float32)``."""
    blocks, scales = [], []
    for packed, s in encode_rows(weight, hdiag, lut, rows_per_chunk):
        blocks.append(packed)
        scales.append(s)
    return np.concatenate(blocks, axis=0), np.concatenate(scales, axis=0)


def encode_linear_e3(weight: torch.Tensor, hdiag: torch.Tensor, lut: torch.Tensor, blocks_path: Path,
                     scales_path: Path, rows_per_chunk: int = 128) -> dict:
    """Encode to ``.bc4`` / ``.scales.f32`` files and return the metadata entry (``encoder.py:121-157``)."""
    m, k = map(int, weight.shape)
    if k % 16:
        raise ValueError(f"unsupported K={k}; BC4 needs K % 16 == 0")
    blocks_path.parent.mkdir(parents=True, exist_ok=True)
    blocks_hash = hashlib.sha256()
    scales_hash = hashlib.sha256()
    with blocks_path.open("wb") as blocks_file, scales_path.open("wb") as scales_file:
        for packed, scales in encode_rows(weight, hdiag, lut, rows_per_chunk):
            raw_blocks = packed.tobytes()
            raw_scales = scales.tobytes()
            blocks_file.write(raw_blocks)
            scales_file.write(raw_scales)
            blocks_hash.update(raw_blocks)
            scales_hash.update(raw_scales)
    return {
        "M": m,
        "K": k,
        "blocks_file": blocks_path.name,
        "blocks_bytes": blocks_path.stat().st_size,
        "blocks_sha256": blocks_hash.hexdigest(),
        "scales_file": scales_path.name,
        "scales_bytes": scales_path.stat().st_size,
        "scales_sha256": scales_hash.hexdigest(),
    }

