"""Python runtime of the BC4 path: native module access, linear modules, packing, install, free.

Mirrors ``texelator/runtime.py`` of the reference (same names and semantics). Differences:
the native module is ``texelator_amd._hip`` over ``libtexelator_hip.so`` (built ahead of time,
never JIT-compiled); the NVFP4 prefill experiment has no gfx950 counterpart and cannot be
enabled; a one-token input always runs the decode GEMV whatever the prefill threshold.
"""
from __future__ import annotations

import gc
import json
import os
from pathlib import Path

import numpy as np
import torch
from torch import nn

from .adapters import resolve_parent

PACKAGE_ROOT = Path(__file__).resolve().parent
_EXTENSION = None
PREFILL_THRESHOLD = int(os.environ.get("TEXELATOR_PREFILL_THRESHOLD", "16"))
PREFILL_TILE_ROWS = int(os.environ.get("TEXELATOR_PREFILL_TILE_ROWS", "1024"))


def extension(verbose: bool = False):
    """The native operator module (``runtime.py:27-63``). Raises if the library is not built."""
    global _EXTENSION
    if _EXTENSION is None:
        from . import _hip, _lib

        _lib.load()
        if verbose:
            print(f"[texelator_amd] loaded {_lib.LIBRARY_PATH}", flush=True)
        _EXTENSION = _hip
    return _EXTENSION


def set_fp4_hybrid(enabled: bool) -> None:
    """The reference's opt-in NVFP4 512-token MLP path (``runtime.py:66-73``) does not exist on gfx950."""
    if enabled:
        raise RuntimeError("the NVFP4 hybrid prefill has no gfx950 counterpart in this build")


def _linear_dispatch(handle: int, x: torch.Tensor) -> torch.Tensor:
    return extension().linear(handle, x)


class TexelatorLinear(nn.Module):
    """Drop-in for ``nn.Linear`` over one or more row-split BC4 handles (``runtime.py:133-145``)."""

    def __init__(self, handles: list[int], bias: nn.Parameter | None = None):
        super().__init__()
        if not handles:
            raise ValueError("TexelatorLinear requires at least one texture handle")
        self.handles = list(handles)
        self.bias = bias

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        contiguous = x.contiguous()
        outputs = [_linear_dispatch(handle, contiguous) for handle in self.handles]
        output = outputs[0] if len(outputs) == 1 else torch.cat(outputs, dim=-1)
        return output if self.bias is None else output + self.bias


class DecodeOnlyLinear(nn.Module):
    """One-token inputs go to the BC4 module, longer ones to the dense original (``runtime.py:148-157``)."""

    def __init__(self, original: nn.Module, quantized: nn.Module):
        super().__init__()
        self.original = original
        self.quantized = quantized

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.numel() == x.shape[-1]:
            return self.quantized(x)
        return self.original(x)


def _cpu_u8(path: Path) -> torch.Tensor:
    return torch.from_numpy(np.fromfile(path, dtype=np.uint8).copy())


def _cpu_f32(path: Path) -> torch.Tensor:
    return torch.from_numpy(np.fromfile(path, dtype="<f4").copy())


def pack_entry(weights: Path, entry: dict, bias: torch.Tensor | None = None, lookahead: int = 1) -> int:
    handle = extension().pack_encoded(
        _cpu_u8(weights / entry["blocks_file"]),
        _cpu_f32(weights / entry["scales_file"]),
        bias,
    )
    extension().set_lookahead(handle, lookahead)
    extension().set_prefill(handle, PREFILL_THRESHOLD, PREFILL_TILE_ROWS)
    return handle


def _host_copy(array: np.ndarray) -> np.ndarray:
    """A contiguous, writable host array (read-only memory maps are copied)."""
    array = np.ascontiguousarray(array)
    return array if array.flags.writeable else array.copy()


def pack_arrays(blocks: np.ndarray, scales: np.ndarray, bias: torch.Tensor | None = None,
                lookahead: int = 1, max_rows: int = 32768) -> list[int]:
    """Pack an in-memory matrix (``[M, K/16*8]`` uint8 blocks, ``[M]`` float32 scales),
    splitting outputs taller than ``max_rows`` into independent handles."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype="<f4")
    m = scales.shape[0]
    blocks = blocks.reshape(m, -1)
    if max_rows <= 0:
        raise ValueError("max_texture_rows must be positive")
    handles: list[int] = []
    try:
        for start in range(0, m, max_rows):
            stop = min(start + max_rows, m)
            handle = extension().pack_encoded(
                torch.from_numpy(_host_copy(blocks[start:stop]).reshape(-1)),
                torch.from_numpy(_host_copy(scales[start:stop])),
                bias[start:stop] if bias is not None else None)
            extension().set_lookahead(handle, lookahead)
            extension().set_prefill(handle, PREFILL_THRESHOLD, PREFILL_TILE_ROWS)
            handles.append(handle)
    except Exception:
        free(handles)
        raise
    return handles


def pack_entry_handles(weights: Path, entry: dict, bias: torch.Tensor | None = None, lookahead: int = 1,
                       max_texture_rows: int = 32768, palette: torch.Tensor | None = None) -> list[int]:
    """Pack one matrix, splitting very tall outputs into independent handles (``runtime.py:179-207``).
    ``palette`` (a device table from :func:`artifact_palette`) switches the handles to LUT mode."""
    m, k = int(entry["M"]), int(entry["K"])
    if max_texture_rows <= 0:
        raise ValueError("max_texture_rows must be positive")
    raw_blocks = np.memmap(weights / entry["blocks_file"], dtype=np.uint8, mode="r", shape=(m, (k // 16) * 8))
    raw_scales = np.memmap(weights / entry["scales_file"], dtype="<f4", mode="r", shape=(m,))
    handles = pack_arrays(raw_blocks, raw_scales, bias=bias, lookahead=lookahead, max_rows=max_texture_rows)
    if palette is not None:
        for handle in handles:
            extension().set_palette_table(handle, palette)
    return handles


def artifact_palette(artifact: Path, device: torch.device | str = "cuda") -> torch.Tensor | None:
    """The palette table an artifact's blocks must be decoded with, or ``None`` when that is this
    build's defined palette (decoded arithmetically).

    An artifact encoded on another GPU (the reference's NVIDIA texture palette) names its palette
    by hash and bundles the table (``manifest["hardware"]["palette"]``, by default
    ``hardware/common/palette.bin``; ``packager.py:185-191``, ``standalone.py:68-70``). The
    reference refuses such an artifact unless this GPU reproduces the palette; here it runs in
    LUT mode instead, bit-exact to that palette."""
    from .artifacts import read_manifest, sha256_file
    from .hardware import PALETTE_SHA256
    from .encoder import load_palette

    artifact = Path(artifact)
    hardware = read_manifest(artifact).get("hardware", {})
    expected = hardware.get("palette_sha256")
    if expected is None or expected == PALETTE_SHA256:
        return None
    bundled = artifact / hardware.get("palette", "hardware/common/palette.bin")
    if not bundled.is_file() or sha256_file(bundled) != expected:
        raise RuntimeError("bundled model palette is missing or corrupt")
    return load_palette(bundled, device).reshape(-1).contiguous()


def install(model: nn.Module, weights: Path, lookahead: int = 1, fp16_prefill: bool = False,
            palette: torch.Tensor | None = None) -> list[int]:
    """Replace the linears listed in ``weights/metadata.json`` (``runtime.py:210-239``); with
    ``palette`` the handles decode in LUT mode (see :func:`artifact_palette`)."""
    metadata = json.loads((weights / "metadata.json").read_text())
    handles: list[int] = []
    for entry in metadata["entries"]:
        parent, child = resolve_parent(model, entry["module_name"])
        original = getattr(parent, child)
        device = original.weight.device
        if device.type != "cuda":
            raise RuntimeError(f"{entry['module_name']} is on {device}; selected linears must be CUDA resident")
        bias = original.bias if getattr(original, "bias", None) is not None else None
        with torch.cuda.device(device):
            entry_handles = pack_entry_handles(weights, entry, bias=bias, lookahead=lookahead, palette=palette)
        quantized = TexelatorLinear(entry_handles)
        replacement = DecodeOnlyLinear(original, quantized) if fp16_prefill else quantized
        setattr(parent, child, replacement)
        handles.extend(entry_handles)
        if not fp16_prefill:
            del original
    gc.collect()
    if torch.cuda.is_available():
        torch.cuda.empty_cache()
    model._texelator_handles = handles
    return handles


def install_standalone(model: nn.Module, weights: Path, entries: list[dict], name_mapper,
                       lookahead: int = 1) -> list[int]:
    """Replace meta-initialised linears without keeping dense weights (``runtime.py:242-263``)."""
    handles: list[int] = []
    try:
        for entry in entries:
            parent, child = resolve_parent(model, name_mapper(entry["module_name"]))
            original = getattr(parent, child)
            entry_handles = pack_entry_handles(weights, entry, lookahead=lookahead)
            setattr(parent, child, TexelatorLinear(entry_handles, bias=getattr(original, "bias", None)))
            handles.extend(entry_handles)
    except Exception:
        free(handles)
        raise
    model._texelator_handles = handles
    return handles


def free(handles: list[int]) -> None:
    """Synchronise, then release every handle (``runtime.py:266-274``)."""
    if torch.cuda.is_available():
        torch.cuda.synchronize()
    for handle in handles:
        extension().free(handle)
