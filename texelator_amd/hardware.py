"""Device palette probe and cache (``texelator/hardware.py`` of the reference).

The reference measures the BC4 palette that NVIDIA's texture unit returns and caches it under
``STATE_HOME/hardware/sm_XY/palette.bin`` (``hardware.py:15-60``). On gfx950 the palette is
produced by this build's register decoder, so the probe must reproduce the defined palette
exactly: ``ensure_hardware`` compares the probed table's SHA-256 with ``PALETTE_SHA256`` and
refuses a device whose decoder disagrees. There is no compiler fallback (the reference's
``nvcc`` path, ``hardware.py:44-60``): the probe lives in ``libtexelator_hip.so``.
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import torch

from .artifacts import device_identity, environment_snapshot, sha256_file, write_json
from .store import STATE_HOME

# SHA-256 of the 255 x 255 x 8 little-endian float32 palette defined by this build's decoder
# (index ((e1+127)*255 + (e0+127))*8 + s). Every artifact's palette gate compares against it.
PALETTE_SHA256 = "bd14120748c07e65ab6da1e4c36ac4de90ab1005e2a3970e9bdc4ddf2be86fdf"
PALETTE_BYTES = 255 * 255 * 8 * 4


def device_key() -> str:
    """Cache key of the visible device: its gfx architecture (``sm_XY`` in the reference)."""
    identity = device_identity()
    if identity is None:
        raise RuntimeError("Texelator requires a ROCm-enabled PyTorch and a visible AMD GPU")
    return identity["arch"]


def probe_palette() -> torch.Tensor:
    """Run the device probe and return ``[65025, 8]`` float32 (CPU)."""
    from .runtime import extension

    return extension().palette_probe().contiguous()


def ensure_hardware(force: bool = False) -> Path:
    """Probe (or reuse) the device palette and return the path of ``palette.bin``.

    Raises ``RuntimeError`` if the probed table differs from the defined palette.
    """
    if not torch.cuda.is_available():
        raise RuntimeError("Texelator requires a ROCm-enabled PyTorch and a visible AMD GPU")
    destination = STATE_HOME / "hardware" / device_key()
    palette = destination / "palette.bin"
    if palette.exists() and not force and sha256_file(palette) == PALETTE_SHA256:
        return palette
    destination.mkdir(parents=True, exist_ok=True)
    print(f"[texelator] probing the BC4 decoder on {torch.cuda.get_device_name()}...", flush=True)
    values = probe_palette()
    raw = values.numpy().astype("<f4", copy=False).tobytes()
    digest = hashlib.sha256(raw).hexdigest()
    if digest != PALETTE_SHA256:
        raise RuntimeError(f"device BC4 decoder palette {digest} differs from the defined palette {PALETTE_SHA256}")
    temporary = palette.with_suffix(".bin.tmp")
    temporary.write_bytes(raw)
    temporary.replace(palette)
    write_json(destination / "palette.json", {
        "device": torch.cuda.get_device_name(),
        "arch": device_key(),
        "endpoint_pairs": 255 * 255,
        "values_per_pair": 8,
        "bytes": len(raw),
    })
    write_json(destination / "environment.json", environment_snapshot())
    return palette


def device_palette(device: torch.device | str = "cuda") -> torch.Tensor:
    """The probed palette as a ``[255, 255, 8]`` tensor on ``device`` (the encoder's LUT)."""
    values = probe_palette()
    digest = hashlib.sha256(values.numpy().astype("<f4", copy=False).tobytes()).hexdigest()
    if digest != PALETTE_SHA256:
        raise RuntimeError(f"device BC4 decoder palette {digest} differs from the defined palette")
    return values.reshape(255, 255, 8).to(device)


def doctor_payload(force: bool = False) -> dict:
    """``texelator doctor`` payload (``hardware.py:63-72``)."""
    palette = ensure_hardware(force=force)
    metadata = json.loads(palette.with_name("palette.json").read_text())
    return {
        "status": "ready",
        "state_home": str(STATE_HOME),
        "palette": str(palette),
        "palette_sha256": sha256_file(palette),
        **metadata,
    }
