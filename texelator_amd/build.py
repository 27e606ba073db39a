"""Build recipe for ``libtexelator_hip.so`` (gfx950, in-tree).

The library is compiled with ``hipcc`` directly from ``texelator_amd/csrc/*.hip``; nothing is
JIT-compiled at import time. ``python -m texelator_amd.build`` rebuilds it.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE_ROOT = Path(__file__).resolve().parent
CSRC = PACKAGE_ROOT / "csrc"
LIBRARY = PACKAGE_ROOT / "libtexelator_hip.so"
BUILD_DIR = PACKAGE_ROOT / "_build"
ARCH = os.environ.get("TEXELATOR_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    # Packed fp32 VALU instructions are kept out of every kernel on this pool.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found; the gfx950 library cannot be built")
    return found


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(source: Path, build_dir: Path, defines: tuple[str, ...]) -> Path:
    obj = build_dir / (source.stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, *(f"-D{d}" for d in defines), "-c", str(source), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source.name}:\n{result.stderr}")
    return obj


def build(verbose: bool = False, output: Path | None = None, defines: tuple[str, ...] = ()) -> Path:
    """Compile every HIP source for gfx950 and link ``libtexelator_hip.so`` (or ``output``, with
    extra preprocessor ``defines`` such as ``TX_PREFILL_LA=2``)."""
    library = Path(output) if output is not None else LIBRARY
    build_dir = BUILD_DIR if output is None else library.parent / (library.stem + "_build")
    build_dir.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    workers = min(len(srcs), max(1, (os.cpu_count() or 4)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        objects = list(pool.map(lambda src: _compile(src, build_dir, tuple(defines)), srcs))
    tmp = library.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-ldl", "-o", str(tmp)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"link failed:\n{result.stderr}")
    tmp.replace(library)
    if verbose:
        print(f"[texelator_amd] built {library}", flush=True)
    return library


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
