"""Python runtime of the BC4 path: the native module, the linear modules, packing, install, free.

Public names and their meaning follow the reference's ``texelator/runtime.py`` (``extension``
:27-63, ``TexelatorLinear`` :133-145, ``DecodeOnlyLinear`` :148-157, ``pack_entry`` :168-176,
``pack_entry_handles`` :179-207, ``install`` :210-239, ``install_standalone`` :242-263, ``free``
:266-274). The implementation is this build's:

* the native module is ``texelator_amd._hip`` over the prebuilt ``libtexelator_hip.so``; there is
  no JIT build and no fallback, a missing library raises on first use;
* every way of packing (a metadata entry, an in-memory matrix, a memory map) goes through one
  row-chunk packer, :func:`_pack_rows`, which frees what it packed if a later chunk fails;
* both installers go through :func:`_swap_linears`, which resolves every target module before
  packing anything and frees the packed handles if a replacement fails;
* the opt-in FP4 hybrid prefill (``runtime.py:21-23, 66-131``) quantizes to MXFP4, the format
  of gfx950's block-scaled MFMA, where the reference quantizes to NVFP4 for Blackwell; one token
  always runs the decode GEMV, whatever the prefill threshold.
"""
from __future__ import annotations

import gc
import json
import os
from pathlib import Path
from typing import Callable, Iterable, Iterator

import numpy as np
import torch
from torch import nn

from .adapters import resolve_parent

PACKAGE_ROOT = Path(__file__).resolve().parent
PREFILL_THRESHOLD = int(os.environ.get("TEXELATOR_PREFILL_THRESHOLD", "16"))
PREFILL_TILE_ROWS = int(os.environ.get("TEXELATOR_PREFILL_TILE_ROWS", "1024"))
# Rows per handle when a matrix is split (the reference's texture-height limit, kept so that
# handle counts and per-handle shapes match the reference's for the same artifact).
MAX_ROWS_PER_HANDLE = 32768

_native = None


def extension(verbose: bool = False):
    """The native operator module, loaded once. Raises if ``libtexelator_hip.so`` is missing."""
    global _native
    if _native is not None:
        return _native
    from . import _hip, _lib

    library = _lib.load()
    if verbose:
        print(f"[texelator_amd] native library {_lib.LIBRARY_PATH} ({library._name})", flush=True)
    _native = _hip
    return _native


# ---------------------------------------------------------------------------------------------
# FP4 hybrid prefill (opt-in)

# The (M, K) shapes and the token count the hybrid path takes (the reference's MLP shapes).
FP4_HYBRID_SHAPES = frozenset({(5120, 17408), (17408, 5120)})
FP4_HYBRID_TOKENS = 512


class _Fp4State:
    """Whether the hybrid is on, and its staging buffers per (device, tokens, M, K)."""

    enabled = False
    buffers: dict[tuple[int, int, int, int], tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]] = {}


def set_fp4_hybrid(enabled: bool) -> None:
    """Turn the FP4 hybrid prefill on or off (off by default; ``free`` turns it off)."""
    _Fp4State.enabled = bool(enabled)


def _fp4_staging(device: torch.device, tokens: int, m: int, k: int):
    key = (device.index or 0, tokens, m, k)
    staged = _Fp4State.buffers.get(key)
    if staged is None:
        def uint8(*shape):
            return torch.empty(shape, dtype=torch.uint8, device=device)
        staged = (uint8(tokens, k // 2), uint8(tokens, k // 32), uint8(m, k // 2), uint8(m, k // 32))
        _Fp4State.buffers[key] = staged
    return staged


def _fp4_linear(handle: int, x: torch.Tensor, m: int, k: int) -> torch.Tensor:
    """The activation and the handle's weights quantized to MXFP4, then the block-scaled GEMM
    (bf16 output). As on the reference's path, the handle's bias is not added."""
    ext = extension()
    flat = x.reshape(-1, k)
    x_packed, x_scales, w_packed, w_scales = _fp4_staging(x.device, flat.shape[0], m, k)
    ext.quantize_activation_fp4_out(flat, x_packed, x_scales)
    ext.decode_weight_fp4_out(handle, w_packed, w_scales)
    return ext.fp4_gemm(x_packed, x_scales, w_packed, w_scales).reshape(*x.shape[:-1], m)


# ---------------------------------------------------------------------------------------------
# Linear modules


def _linear_dispatch(handle: int, x: torch.Tensor) -> torch.Tensor:
    """One handle's ``x @ W^T (+ its bias)``: the FP4 hybrid for its shapes at 512 tokens when it
    is on, otherwise the native call, which picks the GEMV or the prefill tile."""
    ext = extension()
    if _Fp4State.enabled and x.dtype == torch.bfloat16:
        m, k = ext.shape(handle)
        if x.numel() == FP4_HYBRID_TOKENS * k and (m, k) in FP4_HYBRID_SHAPES:
            return _fp4_linear(handle, x, m, k)
    return ext.linear(handle, x)


def bc4_linear(handles: list[int], x: torch.Tensor) -> torch.Tensor:
    """``x @ W^T`` of a matrix held as row shards (handles in row order)."""
    x = x.contiguous()
    if len(handles) == 1:
        return _linear_dispatch(handles[0], x)
    return torch.cat([_linear_dispatch(handle, x) for handle in handles], dim=-1)


class TexelatorLinear(nn.Module):
    """``nn.Linear`` replacement over one or more row shards of a BC4 matrix.

    A handle may carry its own bias (packed with it); ``bias`` here is a separate parameter
    added after the shards are joined (the standalone loader's meta-initialised modules)."""

    def __init__(self, handles: list[int], bias: nn.Parameter | None = None):
        super().__init__()
        shards = [int(handle) for handle in handles]
        if not shards:
            raise ValueError("TexelatorLinear requires at least one BC4 handle")
        self.handles = shards
        self.bias = bias

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        bias = self.bias
        if (bias is not None and len(self.handles) == 1 and x.is_cuda and x.dtype == torch.bfloat16
                and bias.dtype == torch.bfloat16 and bias.is_contiguous() and x.numel() == x.shape[-1]
                and x.is_contiguous() and x.data_ptr() % 16 == 0):
            # one token: the bias goes into the GEMV's own epilogue, rounded as the add below rounds
            from . import layers

            return layers.linear_add_bias(self.handles[0], x, bias)
        y = bc4_linear(self.handles, x)
        if bias is not None:
            y = y + bias
        return y


class DecodeOnlyLinear(nn.Module):
    """Routes a single token (``numel == shape[-1]``) to the BC4 module and any longer input to
    the dense original it was built from."""

    def __init__(self, original: nn.Module, quantized: nn.Module):
        super().__init__()
        self.original = original
        self.quantized = quantized

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        single_token = x.numel() == x.shape[-1]
        return (self.quantized if single_token else self.original)(x)


# ---------------------------------------------------------------------------------------------
# Packing


def _row_chunks(rows: int, max_rows: int) -> Iterator[tuple[int, int]]:
    if max_rows <= 0:
        raise ValueError("max_texture_rows must be positive")
    for start in range(0, rows, max_rows):
        yield start, min(rows, start + max_rows)


def _host_tensor(array: np.ndarray, dtype) -> torch.Tensor:
    """A CPU tensor over a contiguous, writable copy of ``array`` when it is a read-only map or
    a strided view; otherwise over ``array`` itself."""
    array = np.ascontiguousarray(array, dtype=dtype)
    if not array.flags.writeable:
        array = array.copy()
    return torch.from_numpy(array.reshape(-1))


def _configure(handle: int, lookahead: int, palette: torch.Tensor | None) -> None:
    ext = extension()
    ext.set_lookahead(handle, lookahead)
    ext.set_prefill(handle, PREFILL_THRESHOLD, PREFILL_TILE_ROWS)
    if palette is not None:
        ext.set_palette_table(handle, palette)


def _pack_rows(blocks: np.ndarray, scales: np.ndarray, bias: torch.Tensor | None, lookahead: int,
               max_rows: int, palette: torch.Tensor | None) -> list[int]:
    """Pack ``blocks [M, K/16*8]`` and ``scales [M]`` as shards of at most ``max_rows`` rows."""
    rows = int(scales.shape[0])
    blocks = blocks.reshape(rows, -1)
    packed: list[int] = []
    try:
        for start, stop in _row_chunks(rows, max_rows):
            shard_bias = None if bias is None else bias[start:stop]
            handle = extension().pack_encoded(_host_tensor(blocks[start:stop], np.uint8),
                                              _host_tensor(scales[start:stop], "<f4"), shard_bias)
            packed.append(handle)
            _configure(handle, lookahead, palette)
    except BaseException:
        _release(packed)
        raise
    return packed


def pack_arrays(blocks: np.ndarray, scales: np.ndarray, bias: torch.Tensor | None = None,
                lookahead: int = 1, max_rows: int = MAX_ROWS_PER_HANDLE) -> list[int]:
    """Pack an in-memory matrix (uint8 blocks ``[M, K/16*8]``, float32 scales ``[M]``) into row
    shards of at most ``max_rows`` rows."""
    return _pack_rows(np.asarray(blocks), np.asarray(scales), bias, lookahead, max_rows, None)


def _entry_arrays(weights: Path, entry: dict) -> tuple[np.ndarray, np.ndarray]:
    """Memory maps of an entry's ``.bc4`` and ``.scales.f32`` files (``encoder.py:148-157`` layout)."""
    rows, columns = int(entry["M"]), int(entry["K"])
    blocks = np.memmap(Path(weights) / entry["blocks_file"], dtype=np.uint8, mode="r",
                       shape=(rows, columns // 16 * 8))
    scales = np.memmap(Path(weights) / entry["scales_file"], dtype="<f4", mode="r", shape=(rows,))
    return blocks, scales


def pack_entry_handles(weights: Path, entry: dict, bias: torch.Tensor | None = None, lookahead: int = 1,
                       max_texture_rows: int = MAX_ROWS_PER_HANDLE,
                       palette: torch.Tensor | None = None) -> list[int]:
    """Pack one ``metadata.json`` entry as row shards. ``palette`` (a device table from
    :func:`artifact_palette`) switches the shards to LUT-mode decode."""
    if max_texture_rows <= 0:
        raise ValueError("max_texture_rows must be positive")
    blocks, scales = _entry_arrays(weights, entry)
    return _pack_rows(blocks, scales, bias, lookahead, max_texture_rows, palette)


def pack_entry(weights: Path, entry: dict, bias: torch.Tensor | None = None, lookahead: int = 1) -> int:
    """Pack one entry as a single handle, however tall."""
    (handle,) = pack_entry_handles(weights, entry, bias=bias, lookahead=lookahead,
                                   max_texture_rows=max(1, int(entry["M"])))
    return handle


def artifact_palette(artifact: Path, device: torch.device | str = "cuda") -> torch.Tensor | None:
    """The palette table an artifact's blocks must be decoded with, or ``None`` when that is this
    build's defined palette (decoded arithmetically).

    An artifact encoded on another GPU (the reference's NVIDIA texture palette) names its palette
    by hash and bundles the table (``manifest["hardware"]["palette"]``, by default
    ``hardware/common/palette.bin``; ``packager.py:185-191``, ``standalone.py:68-70``). The
    reference refuses such an artifact unless this GPU reproduces the palette; here it runs in
    LUT mode instead, bit-exact to that palette."""
    from .artifacts import read_manifest, sha256_file
    from .encoder import load_palette
    from .hardware import PALETTE_SHA256

    artifact = Path(artifact)
    hardware = read_manifest(artifact).get("hardware", {})
    expected = hardware.get("palette_sha256")
    if expected is None or expected == PALETTE_SHA256:
        return None
    bundled = artifact / hardware.get("palette", "hardware/common/palette.bin")
    if not bundled.is_file() or sha256_file(bundled) != expected:
        raise RuntimeError("bundled model palette is missing or corrupt")
    return load_palette(bundled, device).reshape(-1).contiguous()


# ---------------------------------------------------------------------------------------------
# Installation into a model


def _swap_linears(model: nn.Module, weights: Path, entries: Iterable[dict], target_name: Callable[[str], str],
                  build: Callable[[nn.Module, dict], tuple[nn.Module, list[int]]]) -> list[int]:
    """Replace the module named by each entry with ``build(original, entry)``'s module.

    Every target is resolved before anything is packed, so a misnamed entry fails without
    touching the GPU; if packing or a replacement fails, the handles packed so far are freed and
    the modules already replaced keep their BC4 replacement (which then must not be called)."""
    targets = []
    for entry in entries:
        parent, child = resolve_parent(model, target_name(entry["module_name"]))
        targets.append((parent, child, entry))
    packed: list[int] = []
    try:
        for parent, child, entry in targets:
            module, handles = build(getattr(parent, child), entry)
            packed.extend(handles)
            setattr(parent, child, module)
    except BaseException:
        _release(packed)
        raise
    model._texelator_handles = packed
    return packed


def install(model: nn.Module, weights: Path, lookahead: int = 1, fp16_prefill: bool = False,
            palette: torch.Tensor | None = None) -> list[int]:
    """Replace the linears listed in ``weights/metadata.json`` of a loaded model.

    The packed shards take the original's bias. With ``fp16_prefill`` the dense original is kept
    for inputs longer than one token (:class:`DecodeOnlyLinear`); otherwise it is dropped and the
    allocator cache emptied. ``palette`` selects LUT-mode decode (see :func:`artifact_palette`)."""
    weights = Path(weights)
    entries = json.loads((weights / "metadata.json").read_text())["entries"]

    def build(original: nn.Module, entry: dict):
        device = original.weight.device
        if device.type != "cuda":
            raise RuntimeError(f"{entry['module_name']} is on {device}; selected linears must be CUDA resident")
        with torch.cuda.device(device):
            handles = pack_entry_handles(weights, entry, bias=getattr(original, "bias", None),
                                         lookahead=lookahead, palette=palette)
        quantized = TexelatorLinear(handles)
        return (DecodeOnlyLinear(original, quantized) if fp16_prefill else quantized), handles

    handles = _swap_linears(model, weights, entries, lambda name: name, build)
    gc.collect()
    if torch.cuda.is_available():
        torch.cuda.empty_cache()
    return handles


def install_standalone(model: nn.Module, weights: Path, entries: list[dict], name_mapper,
                       lookahead: int = 1) -> list[int]:
    """Replace the linears of a meta-initialised model (no dense weights ever materialised).

    ``name_mapper`` maps an artifact module name to the model's; the replacement keeps the
    original module's ``bias`` parameter (loaded by the caller) and adds it after the shards."""
    weights = Path(weights)

    def build(original: nn.Module, entry: dict):
        handles = pack_entry_handles(weights, entry, lookahead=lookahead)
        return TexelatorLinear(handles, bias=getattr(original, "bias", None)), handles

    return _swap_linears(model, weights, entries, name_mapper, build)


def _release(handles: Iterable[int]) -> None:
    ext = extension()
    for handle in handles:
        ext.free(handle)


def free(handles: list[int]) -> None:
    """Wait for all queued GPU work, release every handle, and turn the FP4 hybrid off (dropping
    its staging buffers)."""
    if torch.cuda.is_available():
        torch.cuda.synchronize()
    _release(handles)
    _Fp4State.enabled = False
    _Fp4State.buffers.clear()
