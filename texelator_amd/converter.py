"""Activation-aware BC4 conversion of a loaded model: calibration moments, then a resumable encode.

Follows the reference's ``texelator/converter.py``: per-input-channel second moments ``E[x^2]`` of
every target linear's input are collected with forward pre-hooks over a calibration token stream
(``_collect_moments``, :62-103), each linear is encoded with those moments as the E3 search's
``hdiag`` (``encode_linear_e3``, ``encoder.py:121-157``), and the artifact is written in the
reference's layout (``weights/<key>.bc4``, ``.scales.f32``, ``metadata.json`` with per-entry
SHA-256, ``validation.json``, ``texelator.json``; :172-230), resumably: a finished artifact is
verified and reused, the calibration moments are cached, and entries already encoded (files whose
hashes match ``weights/progress.json``) are skipped (:146-205).

Differences, by design:
- the model is passed in already loaded (this build has no model store or hub access); the
  calibration stream is a local token file, or a local text file with a caller's tokenizer
  (the reference's offline ``--calibration-file`` path; its wikitext download is not reachable);
- moments are accumulated in float64 on the model's device and cached as safetensors (no
  pickle), with their SHA-256 in ``calibration/metadata.json``;
- encoding runs wherever the palette LUT lives (the GPU by default).
"""
from __future__ import annotations

import gc
import json
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch
from torch import nn

from .adapters import DEFAULT_SUFFIXES, discover_linears
from .artifacts import (ARTIFACT_FORMAT, MANIFEST, WEIGHTS_FORMAT, environment_snapshot, sha256_file,
                        validate_encoded, write_json)
from .encoder import encode_linear_e3
from .hardware import PALETTE_SHA256

MOMENTS_FILE = Path("calibration") / "moments.safetensors"
CALIBRATION_METADATA = Path("calibration") / "metadata.json"


def read_token_ids(path: Path, tokens: int, tokenizer=None) -> torch.Tensor:
    """The first ``tokens`` ids of a local calibration source.

    ``.npy``: an integer array (no pickle). Any other file: with ``tokenizer`` (a Hugging Face
    tokenizer), its text tokenized without special tokens; without one, whitespace-separated
    integer ids. Raises if the source holds fewer than ``tokens`` ids."""
    path = Path(path).expanduser()
    if path.suffix == ".npy":
        ids = np.load(path, allow_pickle=False).reshape(-1)
        if not np.issubdtype(ids.dtype, np.integer):
            raise RuntimeError(f"calibration ids in {path} are not integers")
        values = torch.from_numpy(ids.astype(np.int64))
    else:
        text = path.read_text(errors="replace")
        if tokenizer is not None:
            values = tokenizer(text, return_tensors="pt", add_special_tokens=False).input_ids.reshape(-1)
        else:
            values = torch.tensor([int(token) for token in text.split()], dtype=torch.int64)
    if values.numel() < tokens:
        raise RuntimeError(f"calibration source {path} has {values.numel()} tokens, need {tokens}")
    return values[:tokens].clone()


class MomentCollector:
    """Forward pre-hooks that accumulate, per target linear, the sum of squares of each input
    feature and the number of input rows; ``moments()`` gives ``E[x^2]`` per feature."""

    def __init__(self, model: nn.Module, targets: dict[str, str]):
        self._sums: dict[str, torch.Tensor] = {}
        self._rows: dict[str, int] = {}
        self._hooks = [model.get_submodule(name).register_forward_pre_hook(self._hook(key))
                       for name, key in targets.items()]

    def _hook(self, key: str):
        def record(_module, inputs):
            x = inputs[0].detach()
            x = x.reshape(-1, x.shape[-1]).double()
            squares = (x * x).sum(0)
            self._sums[key] = squares if key not in self._sums else self._sums[key] + squares
            self._rows[key] = self._rows.get(key, 0) + x.shape[0]
        return record

    def moments(self) -> dict[str, torch.Tensor]:
        return {key: (total / self._rows[key]).float().cpu().contiguous() for key, total in self._sums.items()}

    def close(self) -> None:
        for hook in self._hooks:
            hook.remove()
        self._hooks = []


@torch.inference_mode()
def collect_moments(model: nn.Module, targets: dict[str, str], ids: torch.Tensor, chunk: int) -> dict[str, torch.Tensor]:
    """``E[x^2]`` of each target's input over ``ids``, run through ``model`` ``chunk`` tokens at a
    time (each chunk one sequence, no KV cache). ``targets`` maps module name -> artifact key."""
    if chunk < 1:
        raise ValueError("calibration chunk must be positive")
    device = next(model.parameters()).device
    collector = MomentCollector(model, targets)
    try:
        for start in range(0, ids.numel(), chunk):
            piece = ids[start:start + chunk].view(1, -1).to(device)
            model(piece, use_cache=False)
            print(f"[texelator] calibration {min(start + chunk, ids.numel())}/{ids.numel()}", flush=True)
    finally:
        collector.close()
    missing = sorted(set(targets.values()) - set(collector._sums))
    if missing:
        raise RuntimeError(f"calibration never reached {len(missing)} target linears, e.g. {missing[0]}")
    return collector.moments()


def _load_moments(path: Path) -> dict[str, torch.Tensor]:
    from safetensors.torch import load_file

    return load_file(str(path), device="cpu")


def _save_moments(path: Path, moments: dict[str, torch.Tensor]) -> None:
    from safetensors.torch import save_file

    path.parent.mkdir(parents=True, exist_ok=True)
    temporary = path.with_suffix(".tmp")
    save_file(moments, str(temporary))
    temporary.replace(path)


@dataclass
class _Progress:
    """``weights/progress.json``: the entries encoded so far, in order."""

    path: Path
    entries: list[dict]

    @classmethod
    def load(cls, path: Path, resume: bool) -> "_Progress":
        entries = json.loads(path.read_text()).get("entries", []) if resume and path.exists() else []
        return cls(path, entries)

    def verified(self, weights: Path, module_name: str) -> dict | None:
        """The recorded entry of ``module_name`` if both its files still hash as recorded."""
        for entry in self.entries:
            if entry["module_name"] != module_name:
                continue
            files = [(weights / entry[f"{kind}_file"], entry[f"{kind}_sha256"]) for kind in ("blocks", "scales")]
            if all(path.exists() and sha256_file(path) == digest for path, digest in files):
                return entry
            self.entries.remove(entry)
            return None
        return None

    def add(self, entry: dict) -> None:
        self.entries.append(entry)
        write_json(self.path, {"entries": self.entries})


def _check_finished(destination: Path, palette_sha256: str, tokens: int, source: str) -> bool:
    """True if ``destination`` holds a finished artifact of the same source, palette and
    calibration size whose files all verify; raises if it holds a different finished one."""
    manifest_path = destination / MANIFEST
    if not (manifest_path.exists() and (destination / "weights" / "metadata.json").exists()):
        return False
    manifest = json.loads(manifest_path.read_text())
    same = (manifest.get("source", {}).get("name") == source
            and manifest.get("hardware", {}).get("palette_sha256") == palette_sha256
            and manifest.get("calibration", {}).get("tokens") == tokens)
    if same and validate_encoded(destination / "weights")["ok"]:
        return True
    raise RuntimeError("the output directory contains a finished artifact with a different source, palette, "
                       "calibration size or checksums; choose a new output directory")


def convert_model(model: nn.Module, destination: Path, ids: torch.Tensor, *, source: str, chunk: int = 2048,
                  rows_per_chunk: int = 128, lut: torch.Tensor | None = None, palette_sha256: str = PALETTE_SHA256,
                  include_regex: str | None = None, name: str | None = None, runtime_dtype: str = "bfloat16",
                  resume: bool = True, calibration_source: str = "token ids",
                  stop_after: int | None = None) -> Path:
    """Calibrate ``model`` on ``ids`` and write its BC4 artifact to ``destination``.

    ``lut`` is the palette table the encoder searches (default: the probed device palette, on
    the GPU); ``palette_sha256`` is the hash recorded for it. ``stop_after`` ends the encode
    loop after that many newly encoded entries (an interrupted run, for resume tests). Returns
    ``destination``; an unfinished run returns it without the manifest."""
    destination = Path(destination).expanduser().resolve()
    tokens = int(ids.numel())
    if _check_finished(destination, palette_sha256, tokens, source):
        print(f"[texelator] verified artifact already ready: {destination}", flush=True)
        return destination
    targets = [spec for spec in discover_linears(model, DEFAULT_SUFFIXES, include_regex) if spec.supported]
    if not targets:
        raise RuntimeError("the model contains no BC4-compatible linear weights")
    weights = destination / "weights"
    weights.mkdir(parents=True, exist_ok=True)

    moments_path = destination / MOMENTS_FILE
    metadata_path = destination / CALIBRATION_METADATA
    calibration = json.loads(metadata_path.read_text()) if resume and metadata_path.exists() else None
    if (calibration and moments_path.exists() and calibration.get("tokens") == tokens
            and calibration.get("sha256") == sha256_file(moments_path)):
        moments = _load_moments(moments_path)
        print("[texelator] using verified calibration cache", flush=True)
    elif calibration and calibration.get("tokens") != tokens:
        raise RuntimeError("existing calibration token count differs; choose a new output directory")
    else:
        moments = collect_moments(model, {spec.module_name: spec.artifact_key for spec in targets}, ids, chunk)
        _save_moments(moments_path, moments)
        calibration = {"tokens": tokens, "chunk": chunk, "source": calibration_source,
                       "sha256": sha256_file(moments_path)}
        write_json(metadata_path, calibration)

    if lut is None:
        from .hardware import device_palette

        lut = device_palette("cuda")
    progress = _Progress.load(weights / "progress.json", resume)
    encoded_now = 0
    for index, spec in enumerate(targets, start=1):
        if progress.verified(weights, spec.module_name):
            print(f"[texelator] skip verified {index}/{len(targets)} {spec.module_name}", flush=True)
            continue
        if stop_after is not None and encoded_now >= stop_after:
            return destination
        weight = model.get_submodule(spec.module_name).weight
        if weight.device.type == "meta":
            raise RuntimeError(f"{spec.module_name} has no materialised weight; conversion needs it on CPU or GPU")
        result = encode_linear_e3(weight.detach(), moments[spec.artifact_key], lut,
                                  weights / f"{spec.artifact_key}.bc4", weights / f"{spec.artifact_key}.scales.f32",
                                  rows_per_chunk)
        progress.add({**spec.to_dict(), **result})
        encoded_now += 1
        print(f"[texelator] encoded {index}/{len(targets)} {spec.module_name}", flush=True)

    order = {spec.module_name: i for i, spec in enumerate(targets)}
    entries = sorted(progress.entries, key=lambda entry: order[entry["module_name"]])
    write_json(weights / "metadata.json", {
        "schema_version": 1,
        "format": WEIGHTS_FORMAT,
        "encoder": "activation-aware E3",
        "palette_sha256": palette_sha256,
        "entries": entries,
        "bc4_bytes": sum(entry["blocks_bytes"] for entry in entries),
        "scale_bytes": sum(entry["scales_bytes"] for entry in entries),
    })
    progress.path.unlink(missing_ok=True)
    validation = validate_encoded(weights)
    write_json(destination / "validation.json", validation)
    if not validation["ok"]:
        raise RuntimeError("encoded artifact checksum validation failed")
    write_json(destination / MANIFEST, {
        "schema_version": 1,
        "format": ARTIFACT_FORMAT,
        "name": name or destination.name,
        "source": {"name": source},
        "runtime_dtype": runtime_dtype,
        "calibration": calibration,
        "hardware": {"palette_sha256": palette_sha256},
        "weights": "weights",
        "validation": "validation.json",
        "linked_source": True,
    })
    write_json(destination / "environment.json", environment_snapshot())
    gc.collect()
    print(f"[texelator] artifact ready: {destination}", flush=True)
    return destination
