"""Decode-GEMV lookahead tuner (``texelator/tuning.py`` of the reference).

``tune_artifact`` packs every linear of an artifact, checks each lookahead candidate against
lookahead 1 on a sample of linears (``max_abs <= 1e-3``, ``tuning.py:66-81``; the gfx950
variants are in fact bitwise equal), times full batch-1 sweeps over all linears with events
(``tuning.py:82-98``) and stores the lowest-median candidate in a profile keyed by the weights'
metadata hash and the device (``tuning.py:17-21``). Here "lookahead" is the number of 1 KiB BC4
tiles each wave keeps in flight; the candidate set and the profile layout are the reference's.
"""
from __future__ import annotations

import json
import statistics
from pathlib import Path

import torch

from .artifacts import read_manifest, sha256_file, weights_dir, write_json
from .hardware import PALETTE_SHA256, device_key, ensure_hardware
from .runtime import extension, free, pack_entry_handles
from .store import STATE_HOME, safe_name

CANDIDATES = (1, 2, 3, 4, 6, 8)
MAX_ABS_TOLERANCE = 1e-3


def _profile_path(artifact: Path) -> Path:
    metadata_hash = sha256_file(weights_dir(artifact) / "metadata.json")
    device = safe_name(torch.cuda.get_device_name())
    return STATE_HOME / "profiles" / metadata_hash[:20] / f"{device_key()}-{device}.json"


def _runtime_dtype(manifest: dict) -> torch.dtype:
    name = manifest.get("runtime_dtype", "float16")
    if name == "bfloat16":
        return torch.bfloat16
    if name == "float16":
        return torch.float16
    raise RuntimeError(f"unsupported Texelator runtime dtype: {name!r}")


def check_palette(artifact: Path) -> str:
    """The artifact's palette hash must be this device's probed palette (``tuning.py:38-41``)."""
    current = sha256_file(ensure_hardware())
    expected = read_manifest(artifact).get("hardware", {}).get("palette_sha256")
    if not expected or expected != current or current != PALETTE_SHA256:
        raise RuntimeError("model BC4 palette does not match this GPU; benchmark aborted")
    return expected


def tune_artifact(artifact: Path, warmup: int = 10, measured: int = 50, runs: int = 3) -> dict:
    if not torch.cuda.is_available():
        raise RuntimeError("tuning requires a visible GPU")
    if warmup < 0 or measured < 1 or runs < 1:
        raise ValueError("warmup must be non-negative; measured and runs must be positive")
    artifact = Path(artifact)
    manifest = read_manifest(artifact)
    runtime_dtype = _runtime_dtype(manifest)
    palette_sha = check_palette(artifact)
    weights = weights_dir(artifact)
    metadata_path = weights / "metadata.json"
    entries = json.loads(metadata_path.read_text())["entries"]
    if not entries:
        raise RuntimeError("artifact contains no encoded linears")
    ext = extension()
    handles: list[int] = []
    handle_groups: list[list[int]] = []
    inputs: list[torch.Tensor] = []
    try:
        generator = torch.Generator(device="cuda").manual_seed(0)
        for entry in entries:
            group = pack_entry_handles(weights, entry, lookahead=1)
            handle_groups.append(group)
            handles.extend(group)
            inputs.append(torch.randn((1, int(entry["K"])), device="cuda", generator=generator).to(runtime_dtype))

        def evaluate(group: list[int], value: torch.Tensor) -> torch.Tensor:
            parts = [ext.linear(handle, value) for handle in group]
            return (parts[0] if len(parts) == 1 else torch.cat(parts, dim=-1)).float()

        paired = list(zip(handle_groups, inputs))
        sample = paired if len(paired) <= 8 else paired[:4] + paired[-4:]
        reference = [evaluate(group, value) for group, value in sample]

        def sweep() -> None:
            for group, value in paired:
                for handle in group:
                    ext.linear(handle, value)

        rows = []
        for candidate in CANDIDATES:
            for handle in handles:
                ext.set_lookahead(handle, candidate)
            values = [evaluate(group, value) for group, value in sample]
            max_abs = max(float((got - want).abs().max().item()) for got, want in zip(values, reference))
            if max_abs > MAX_ABS_TOLERANCE:
                raise RuntimeError(f"lookahead K={candidate} failed correctness: max_abs={max_abs}")
            for _ in range(warmup):
                sweep()
            torch.cuda.synchronize()
            timings = []
            for _ in range(runs):
                start = torch.cuda.Event(enable_timing=True)
                stop = torch.cuda.Event(enable_timing=True)
                start.record()
                for _ in range(measured):
                    sweep()
                stop.record()
                torch.cuda.synchronize()
                timings.append(start.elapsed_time(stop) / measured)
            row = {
                "lookahead": candidate,
                "max_abs_vs_k1": max_abs,
                "sweep_ms_median": statistics.median(timings),
                "sweep_ms_min": min(timings),
                "sweep_ms_max": max(timings),
                "runs": timings,
            }
            rows.append(row)
            print(json.dumps(row), flush=True)
        selected = min(rows, key=lambda row: row["sweep_ms_median"])["lookahead"]
        profile = {
            "schema_version": 1,
            "device": torch.cuda.get_device_name(),
            "arch": device_key(),
            "weights_metadata_sha256": sha256_file(metadata_path),
            "palette_sha256": palette_sha,
            "artifact": str(artifact.resolve()),
            "runtime_dtype": manifest.get("runtime_dtype"),
            "linears": len(entries),
            "warmup_sweeps": warmup,
            "measured_sweeps": measured,
            "independent_runs": runs,
            "selected_lookahead": selected,
            "candidates": rows,
        }
        target = _profile_path(artifact)
        write_json(target, profile)
        print(f"[texelator] selected K={selected}; local benchmark profile saved to {target}", flush=True)
        return profile
    finally:
        free(handles)


def selected_lookahead(artifact: Path) -> tuple[int, Path | None]:
    """The tuned lookahead for an artifact, or (1, None) without a profile (``tuning.py:134-145``)."""
    artifact = Path(artifact)
    target = _profile_path(artifact)
    if not target.exists():
        return 1, None
    profile = json.loads(target.read_text())
    if profile.get("weights_metadata_sha256") != sha256_file(weights_dir(artifact) / "metadata.json"):
        raise RuntimeError("benchmark profile does not match the encoded weights; rerun texelator benchmark")
    if profile.get("palette_sha256") != read_manifest(artifact).get("hardware", {}).get("palette_sha256"):
        raise RuntimeError("benchmark profile does not match the model palette; rerun texelator benchmark")
    return int(profile["selected_lookahead"]), target
