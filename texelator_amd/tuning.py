"""Decode-GEMV lookahead tuner: how many 1 KiB BC4 tiles each wave keeps in flight.

Interface kept from the reference's ``texelator/tuning.py``: the candidates 1, 2, 3, 4, 6, 8
(:14), the palette gate before any work (:38-41), the correctness rule (every candidate within
``max_abs <= 1e-3`` of lookahead 1 on at most eight linears, the first and last four, :66-81),
the timing of whole batch-1 sweeps over every linear (warmup sweeps, then ``runs`` event-timed
groups of ``measured`` sweeps, :82-98), the lowest median winning, and the profile's path and
JSON keys (:17-21, :109-127). The device is named by gfx architecture instead of compute
capability.

How it is organised here: a :class:`_DecodeSweep` owns the artifact's packed handles, one
seeded batch-1 input per linear and the lookahead setting; :func:`tune_artifact` asks it for
probe outputs and sweep timings candidate by candidate (timing helpers in
:mod:`texelator_amd.measure`). On gfx950 every lookahead computes bitwise the same outputs, so
the correctness column reads 0.
"""
from __future__ import annotations

import json
import statistics
from pathlib import Path

import torch

from .artifacts import read_manifest, sha256_file, weights_dir, write_json
from .hardware import PALETTE_SHA256, device_key, ensure_hardware
from .measure import mean_time_ms
from .runtime import bc4_linear, extension, free, pack_entry_handles
from .store import STATE_HOME, safe_name

CANDIDATES = (1, 2, 3, 4, 6, 8)
MAX_ABS_TOLERANCE = 1e-3
_PROBE_LINEARS = 8  # linears whose outputs are compared between candidates
_RUNTIME_DTYPES = {"float16": torch.float16, "bfloat16": torch.bfloat16}


def _profile_path(artifact: Path) -> Path:
    """``STATE_HOME/profiles/<metadata sha[:20]>/<gfx arch>-<device>.json``."""
    key = sha256_file(weights_dir(artifact) / "metadata.json")[:20]
    return STATE_HOME / "profiles" / key / f"{device_key()}-{safe_name(torch.cuda.get_device_name())}.json"


def _runtime_dtype(manifest: dict) -> torch.dtype:
    """The artifact's activation dtype; the reference's default is float16."""
    name = manifest.get("runtime_dtype", "float16")
    if name not in _RUNTIME_DTYPES:
        raise RuntimeError(f"unsupported Texelator runtime dtype: {name!r}")
    return _RUNTIME_DTYPES[name]


def check_palette(artifact: Path) -> str:
    """The artifact's palette hash, which must equal this GPU's probed palette (and so this
    build's defined palette); raises otherwise."""
    probed = sha256_file(ensure_hardware())
    expected = read_manifest(artifact).get("hardware", {}).get("palette_sha256")
    if not expected or {expected, probed} != {PALETTE_SHA256}:
        raise RuntimeError("model BC4 palette does not match this GPU; benchmark aborted")
    return expected


def _probe_indices(count: int) -> list[int]:
    """All linears when there are at most eight, else the first four and the last four."""
    if count <= _PROBE_LINEARS:
        return list(range(count))
    half = _PROBE_LINEARS // 2
    return list(range(half)) + list(range(count - half, count))


class _DecodeSweep:
    """Every linear of an artifact packed (row-split as the runtime splits it), with one seeded
    ``randn(1, K)`` input per linear in the runtime dtype (CUDA generator, seed 0)."""

    def __init__(self, weights: Path, entries: list[dict], dtype: torch.dtype):
        self.groups: list[list[int]] = []
        self.inputs: list[torch.Tensor] = []
        generator = torch.Generator(device="cuda").manual_seed(0)
        try:
            for entry in entries:
                self.groups.append(pack_entry_handles(weights, entry, lookahead=1))
                self.inputs.append(torch.randn((1, int(entry["K"])), device="cuda", dtype=dtype,
                                               generator=generator))
        except BaseException:
            self.close()
            raise

    @property
    def handles(self) -> list[int]:
        return [handle for group in self.groups for handle in group]

    def set_lookahead(self, lookahead: int) -> None:
        ext = extension()
        for handle in self.handles:
            ext.set_lookahead(handle, lookahead)

    def outputs(self, indices: list[int]) -> list[torch.Tensor]:
        return [bc4_linear(self.groups[i], self.inputs[i]).float() for i in indices]

    def run(self) -> None:
        """One batch-1 pass over every linear, outputs discarded."""
        linear = extension().linear
        for group, x in zip(self.groups, self.inputs):
            for handle in group:
                linear(handle, x)

    def close(self) -> None:
        free(self.handles)
        self.groups.clear()


def _time_candidate(sweep: _DecodeSweep, warmup: int, measured: int, runs: int) -> list[float]:
    for _ in range(warmup):
        sweep.run()
    torch.cuda.synchronize()
    return [mean_time_ms(sweep.run, measured) for _ in range(runs)]


def tune_artifact(artifact: Path, warmup: int = 10, measured: int = 50, runs: int = 3) -> dict:
    """Time full decode sweeps at every lookahead candidate and save the fastest in the
    artifact's decode profile."""
    if not torch.cuda.is_available():
        raise RuntimeError("tuning requires a visible GPU")
    if warmup < 0 or measured < 1 or runs < 1:
        raise ValueError("warmup must be non-negative; measured and runs must be positive")
    artifact = Path(artifact)
    manifest = read_manifest(artifact)
    dtype = _runtime_dtype(manifest)
    palette_sha = check_palette(artifact)
    metadata = weights_dir(artifact) / "metadata.json"
    entries = json.loads(metadata.read_text())["entries"]
    if not entries:
        raise RuntimeError("artifact contains no encoded linears")

    sweep = _DecodeSweep(weights_dir(artifact), entries, dtype)
    try:
        probes = _probe_indices(len(entries))
        sweep.set_lookahead(CANDIDATES[0])
        expected = sweep.outputs(probes)
        rows = []
        for lookahead in CANDIDATES:
            sweep.set_lookahead(lookahead)
            deviation = max(float((got - want).abs().max()) for got, want in zip(sweep.outputs(probes), expected))
            if deviation > MAX_ABS_TOLERANCE:
                raise RuntimeError(f"lookahead K={lookahead} failed correctness: max_abs={deviation}")
            timings = _time_candidate(sweep, warmup, measured, runs)
            row = {"lookahead": lookahead, "max_abs_vs_k1": deviation,
                   "sweep_ms_median": statistics.median(timings), "sweep_ms_min": min(timings),
                   "sweep_ms_max": max(timings), "runs": timings}
            rows.append(row)
            print(json.dumps(row), flush=True)
    finally:
        sweep.close()

    best = min(rows, key=lambda row: row["sweep_ms_median"])["lookahead"]
    profile = {
        "schema_version": 1,
        "device": torch.cuda.get_device_name(),
        "arch": device_key(),
        "weights_metadata_sha256": sha256_file(metadata),
        "palette_sha256": palette_sha,
        "artifact": str(artifact.resolve()),
        "runtime_dtype": manifest.get("runtime_dtype"),
        "linears": len(entries),
        "warmup_sweeps": warmup,
        "measured_sweeps": measured,
        "independent_runs": runs,
        "selected_lookahead": best,
        "candidates": rows,
    }
    target = _profile_path(artifact)
    write_json(target, profile)
    print(f"[texelator] selected K={best}; local benchmark profile saved to {target}", flush=True)
    return profile


def selected_lookahead(artifact: Path) -> tuple[int, Path | None]:
    """The tuned lookahead of an artifact and its profile path; ``(1, None)`` when there is no
    profile. Raises when the profile belongs to other weights or another palette."""
    artifact = Path(artifact)
    target = _profile_path(artifact)
    if not target.exists():
        return 1, None
    profile = json.loads(target.read_text())
    if profile.get("weights_metadata_sha256") != sha256_file(weights_dir(artifact) / "metadata.json"):
        raise RuntimeError("benchmark profile does not match the encoded weights; rerun texelator benchmark")
    palette = read_manifest(artifact).get("hardware", {}).get("palette_sha256")
    if profile.get("palette_sha256") != palette:
        raise RuntimeError("benchmark profile does not match the model palette; rerun texelator benchmark")
    return int(profile["selected_lookahead"]), target
