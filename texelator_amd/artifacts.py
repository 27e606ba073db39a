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
