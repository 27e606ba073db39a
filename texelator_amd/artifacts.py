"""File hashing, atomic JSON writes and run environment (``texelator/artifacts.py``)."""
from __future__ import annotations

import datetime
import hashlib
import json
import os
import platform
import subprocess
import sys
from pathlib import Path

import torch


def sha256_file(path: Path) -> str:
    digest = hashlib.sha256()
    with Path(path).open("rb") as handle:
        while chunk := handle.read(8 << 20):
            digest.update(chunk)
    return digest.hexdigest()


def write_json(path: Path, value) -> None:
    """Write via a temporary file and ``replace`` (``artifacts.py:24-28``)."""
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    temporary = path.with_suffix(path.suffix + ".tmp")
    temporary.write_text(json.dumps(value, indent=2, sort_keys=True) + "\n")
    temporary.replace(path)


def _command(args: list[str]) -> str | None:
    try:
        return subprocess.run(args, check=False, text=True, capture_output=True, timeout=20).stdout.strip() or None
    except (OSError, subprocess.TimeoutExpired):
        return None


def device_identity(index: int | None = None) -> dict | None:
    """Name, gfx architecture, CU count and memory of a visible GPU (None without one)."""
    if not torch.cuda.is_available():
        return None
    index = torch.cuda.current_device() if index is None else index
    props = torch.cuda.get_device_properties(index)
    return {
        "name": props.name,
        "arch": getattr(props, "gcnArchName", "unknown").split(":")[0],
        "compute_units": int(props.multi_processor_count),
        "total_memory_bytes": int(props.total_memory),
        "hip_runtime": torch.version.hip,
    }


def environment_snapshot() -> dict:
    return {
        "timestamp_utc": datetime.datetime.now(datetime.timezone.utc).isoformat(),
        "hostname": platform.node(),
        "platform": platform.platform(),
        "python": sys.version,
        "torch": torch.__version__,
        "gpu": device_identity(),
        "cpu_count_affinity": len(os.sched_getaffinity(0)),
        "git_commit": _command(["git", "rev-parse", "HEAD"]),
        "command": sys.argv,
        "cwd": os.getcwd(),
    }


def validate_encoded(encoded: Path) -> dict:
    """Check every entry's file hashes against ``metadata.json`` (``artifacts.py:76-87``)."""
    metadata = json.loads((encoded / "metadata.json").read_text())
    failures = []
    for entry in metadata["entries"]:
        for key in ("blocks", "scales"):
            path = encoded / entry[f"{key}_file"]
            expected = entry[f"{key}_sha256"]
            actual = sha256_file(path)
            if actual != expected:
                failures.append({"module_name": entry["module_name"], "file": str(path),
                                 "expected": expected, "actual": actual})
    return {"ok": not failures, "entries": len(metadata["entries"]), "failures": failures}


MANIFEST = "texelator.json"
ARTIFACT_FORMAT = "texelator-bc4-v1"
WEIGHTS_FORMAT = "BC4_SNORM + one FP32 scale per output row"


def read_manifest(artifact: Path) -> dict:
    """The artifact's ``texelator.json`` (``converter.py:216-230``)."""
    path = Path(artifact) / MANIFEST
    if not path.is_file():
        raise RuntimeError(f"not a Texelator artifact (missing {MANIFEST}): {artifact}")
    return json.loads(path.read_text())


def weights_dir(artifact: Path) -> Path:
    return Path(artifact) / read_manifest(artifact).get("weights", "weights")


def write_artifact(destination: Path, matrices, palette_sha256: str, runtime_dtype: str = "bfloat16",
                   name: str | None = None, extra: dict | None = None) -> Path:
    """Write an encoded artifact in the reference's on-disk layout.

    ``matrices`` yields ``(module_name, blocks, scales)`` with ``blocks`` uint8 ``[M, K/16*8]``
    and ``scales`` float32 ``[M]``. Files: ``weights/<key>.bc4``, ``weights/<key>.scales.f32``,
    ``weights/metadata.json`` with per-entry sha256 (``converter.py:172-215``),
    ``validation.json`` and ``texelator.json`` (``converter.py:216-230``).
    """
    import numpy as np

    from .adapters import artifact_key, layer_index

    destination = Path(destination)
    weights = destination / "weights"
    weights.mkdir(parents=True, exist_ok=True)
    entries = []
    for module_name, blocks, scales in matrices:
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
        scales = np.ascontiguousarray(scales, dtype="<f4")
        m = int(scales.shape[0])
        blocks = blocks.reshape(m, -1)
        k = blocks.shape[1] // 8 * 16
        key = artifact_key(module_name)
        blocks_path = weights / f"{key}.bc4"
        scales_path = weights / f"{key}.scales.f32"
        blocks_path.write_bytes(blocks.tobytes())
        scales_path.write_bytes(scales.tobytes())
        entries.append({
            "module_name": module_name, "artifact_key": key, "layer": layer_index(module_name),
            "op": module_name.rsplit(".", 1)[-1], "M": m, "K": k, "bias": False, "supported": True,
            "reason": "ok",
            "blocks_file": blocks_path.name, "blocks_bytes": blocks_path.stat().st_size,
            "blocks_sha256": sha256_file(blocks_path),
            "scales_file": scales_path.name, "scales_bytes": scales_path.stat().st_size,
            "scales_sha256": sha256_file(scales_path),
        })
    write_json(weights / "metadata.json", {
        "schema_version": 1,
        "format": WEIGHTS_FORMAT,
        "palette_sha256": palette_sha256,
        "entries": entries,
        "bc4_bytes": sum(entry["blocks_bytes"] for entry in entries),
        "scale_bytes": sum(entry["scales_bytes"] for entry in entries),
    })
    validation = validate_encoded(weights)
    write_json(destination / "validation.json", validation)
    manifest = {
        "schema_version": 1,
        "format": ARTIFACT_FORMAT,
        "name": name or destination.name,
        "runtime_dtype": runtime_dtype,
        "hardware": {"palette_sha256": palette_sha256},
        "weights": "weights",
        "validation": "validation.json",
        "linked_source": False,
    }
    manifest.update(extra or {})
    write_json(destination / MANIFEST, manifest)
    return destination
