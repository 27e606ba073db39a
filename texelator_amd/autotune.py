"""Prefill tile autotuner: which gfx950 tile candidate each (token bucket, M, K) should use.

Interface kept from the reference's ``texelator/autotune.py`` so that profiles mean the same
thing: the candidate names and their backend ids 5..9 (``autotune.py:16-22``), the token
buckets and ``dispatch_key`` text (:23, :34-43), the seeded input ``randn(T, K) * 0.125`` with
seed ``seed + T*1009 + shape index`` (:139-143), the gate that every candidate be bitwise equal
to the baseline tile (:150-168), round-robin event timing with the lowest median winning
(:170-193), the profile's JSON keys (:194-241) and the checks of ``apply_profile`` /
``selected_profile`` (:247-286). The device is identified by gfx architecture and CU count
instead of compute capability and SM count.

How it is organised here: :func:`_pack_inventory` packs an artifact once and groups its handles
by shape; :func:`_tune_shape` runs one (tokens, shape) trial through the explicit-candidate entry
point ``_hip.prefill`` (the handle's own backend setting is never touched while tuning) and
returns that trial's profile record; :func:`tune_artifact` assembles the profile. Timing and the
error metrics live in :mod:`texelator_amd.measure`.
"""
from __future__ import annotations

import hashlib
import json
from dataclasses import dataclass, field
from pathlib import Path

import torch

from .artifacts import sha256_file, weights_dir, write_json
from .hardware import device_key
from .measure import output_error, round_robin_medians
from .runtime import PACKAGE_ROOT, extension, free, pack_entry_handles
from .store import STATE_HOME, safe_name

CANDIDATES = {
    "large_256x128x128": 5,
    "medium_128x128x128": 6,
    "wide_512x128x64": 7,
    "medium_64x128x128": 8,
    "small_32x128x128": 9,
}
BASELINE = "large_256x128x128"
TOKEN_BUCKETS = (32, 128, 512, 2048, 8192, 16384, 32768, 65535)
# Rows per handle while tuning (the reference packs with its texture limit, autotune.py:94-97).
_TUNING_MAX_ROWS = 32768


def profile_path(artifact: Path) -> Path:
    """``STATE_HOME/profiles/<metadata sha[:20]>/<gfx arch>-<device>-prefill.json``."""
    key = sha256_file(weights_dir(artifact) / "metadata.json")[:20]
    return STATE_HOME / "profiles" / key / f"{device_key()}-{safe_name(torch.cuda.get_device_name())}-prefill.json"


def token_bucket(tokens: int) -> int:
    """Smallest bucket holding ``tokens`` (1..65535)."""
    if tokens < 1:
        raise ValueError("tokens must be positive")
    for bucket in TOKEN_BUCKETS:
        if tokens <= bucket:
            return bucket
    raise ValueError(f"tokens exceeds the supported prefill range: {tokens}")


def dispatch_key(tokens: int, m: int, k: int) -> str:
    return f"tokens<={token_bucket(tokens)}:M={m}:K={k}"


def kernel_source_sha256() -> str:
    """SHA-256 over the names and bytes of the HIP sources (``csrc/*.hip`` then ``*.h``), so a
    profile is void once the kernels change."""
    sources = PACKAGE_ROOT / "csrc"
    digest = hashlib.sha256()
    for pattern in ("*.hip", "*.h"):
        for path in sorted(sources.glob(pattern)):
            digest.update(path.name.encode())
            digest.update(path.read_bytes())
    return digest.hexdigest()


# The autotuner's comparison metrics (max_abs, mean_abs, relative_rms, cosine, bitwise_equal).
_error = output_error


def _eligible(name: str, m: int, k: int) -> tuple[bool, str | None]:
    """Every gfx950 tile takes any M and any K that is a multiple of 16 (partial tiles are
    masked), so only an empty output or a ragged K is refused."""
    del name  # all candidates share the same limits
    if m < 1:
        return False, "empty output dimension"
    return (True, None) if k % 16 == 0 else (False, "K is not divisible by 16")


@dataclass
class _Inventory:
    """An artifact's packed handles, and per distinct (M, K) the handle tuned for it and how
    many handles share that shape."""

    handles: list[int] = field(default_factory=list)
    by_shape: dict[tuple[int, int], tuple[int, int]] = field(default_factory=dict)

    def shapes(self) -> list[tuple[tuple[int, int], int, int]]:
        return [(shape, handle, count) for shape, (handle, count) in sorted(self.by_shape.items())]


def _pack_inventory(artifact: Path) -> _Inventory:
    weights = weights_dir(artifact)
    inventory = _Inventory()
    ext = extension()
    try:
        for entry in json.loads((weights / "metadata.json").read_text())["entries"]:
            inventory.handles.extend(pack_entry_handles(weights, entry, lookahead=1,
                                                        max_texture_rows=_TUNING_MAX_ROWS))
        for handle in inventory.handles:
            ext.set_prefill(handle, 1, _TUNING_MAX_ROWS)
            shape = ext.shape(handle)
            first, count = inventory.by_shape.get(shape, (handle, 0))
            inventory.by_shape[shape] = (first, count + 1)
    except BaseException:
        free(inventory.handles)
        raise
    return inventory


def _tune_shape(handle: int, m: int, k: int, occurrences: int, tokens: int, input_seed: int,
                warmup: int, measured: int) -> dict:
    """One (tokens, M, K) trial: gate every candidate against the baseline tile bit for bit,
    time the ones that pass, and return the profile record."""
    ext = extension()
    generator = torch.Generator(device="cuda").manual_seed(input_seed)
    x = torch.randn((tokens, k), device="cuda", dtype=torch.bfloat16, generator=generator).mul_(0.125)

    def run(name: str) -> torch.Tensor:
        return ext.prefill(handle, CANDIDATES[name], x)

    with torch.inference_mode():
        baseline = run(BASELINE)
        correctness: dict[str, dict] = {}
        rejected: dict[str, str] = {}
        for name in CANDIDATES:
            ok, reason = _eligible(name, m, k)
            if not ok:
                rejected[name] = reason or "unsupported"
                continue
            correctness[name] = output_error(baseline, run(name))
            if not correctness[name]["bitwise_equal"]:
                metrics = correctness[name]
                rejected[name] = f"correctness: rrms={metrics['relative_rms']:.6g}, cosine={metrics['cosine']:.9g}"
    passing = [name for name in CANDIDATES if name in correctness and name not in rejected]
    if BASELINE not in passing:
        raise RuntimeError(f"baseline failed correctness for M={m},K={k}")
    medians, _ = round_robin_medians({name: (lambda n=name: run(n)) for name in passing}, warmup, measured)
    winner = min(passing, key=medians.__getitem__)
    return {
        "key": dispatch_key(tokens, m, k),
        "tokens_measured": tokens,
        "token_bucket": token_bucket(tokens),
        "M": m,
        "K": k,
        "occurrences": occurrences,
        "winner": winner,
        "backend": CANDIDATES[winner],
        "median_ms": medians[winner],
        "baseline_ms": medians[BASELINE],
        "speedup_vs_baseline": medians[BASELINE] / medians[winner],
        "candidate_median_ms": medians,
        "correctness_vs_baseline": correctness,
        "rejected": rejected,
    }


def _device_record() -> dict:
    index = torch.cuda.current_device()
    properties = torch.cuda.get_device_properties(index)
    return {
        "name": torch.cuda.get_device_name(),
        "arch": device_key(),
        "multiprocessor_count": int(properties.multi_processor_count),
        "total_memory": int(properties.total_memory),
        "torch": torch.__version__,
        "torch_hip": torch.version.hip,
    }


def tune_artifact(artifact: Path, output_path: Path | None, tokens: list[int], warmup: int = 5,
                  measured: int = 30, seed: int = 20260827) -> dict:
    """Tune every distinct shape of an artifact at each of ``tokens`` (one count per bucket) and
    write the profile to ``output_path`` or :func:`profile_path`."""
    if warmup < 3 or measured < 10:
        raise ValueError("autotuning requires at least 3 warmups and 10 samples")
    buckets = [token_bucket(count) for count in tokens]
    if len(set(buckets)) != len(buckets):
        raise ValueError("provide at most one representative token count per dispatch bucket")
    artifact = Path(artifact).resolve()
    metadata = weights_dir(artifact) / "metadata.json"
    ext = extension()
    inventory = _pack_inventory(artifact)
    try:
        rows: list[dict] = []
        for count in tokens:
            for index, ((m, k), handle, occurrences) in enumerate(inventory.shapes()):
                record = _tune_shape(handle, m, k, occurrences, count, seed + count * 1009 + index, warmup, measured)
                rows.append(record)
                print(f"[autotune] tokens={count} M={m} K={k} winner={record['winner']} "
                      f"{record['median_ms']:.4f} ms speedup={record['speedup_vs_baseline']:.3f}x", flush=True)
        profile = {
            "schema_version": 1,
            "status": "complete",
            "artifact": str(artifact),
            "metadata_sha256": sha256_file(metadata),
            "kernel_source_sha256": kernel_source_sha256(),
            "device": _device_record(),
            "protocol": {"tokens": list(tokens), "warmup": warmup, "measured": measured, "seed": seed,
                         "bitwise_correctness_required": True},
            "candidates": dict(CANDIDATES),
            "kernel_info": {name: ext.kernel_info(backend) for name, backend in CANDIDATES.items()},
            "selections": {record["key"]: record for record in rows},
            "rows": rows,
        }
        target = Path(output_path) if output_path else profile_path(artifact)
        write_json(target, profile)
        print(f"[texelator] prefill profile saved to {target}", flush=True)
        return profile
    finally:
        free(inventory.handles)


def check_profile_device(profile: dict) -> None:
    """Raise unless ``profile`` was made by this kernel build on the same kind of GPU."""
    if profile.get("kernel_source_sha256") != kernel_source_sha256():
        raise RuntimeError("autotune profile kernel hash does not match this build")
    recorded = profile.get("device", {})
    if recorded.get("arch") != device_key():
        raise RuntimeError("autotune profile GPU architecture does not match this GPU")
    cus = int(torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count)
    if recorded.get("multiprocessor_count") != cus:
        raise RuntimeError("autotune profile CU count does not match this GPU")


def apply_profile(handles: list[int], tokens: int, profile: dict) -> bool:
    """Give every handle threshold 1 and the profile's tile for ``tokens``; shapes the profile
    does not cover keep the baseline tile and make the result False.

    A one-token call still runs the decode GEMV (the gfx950 dispatch never sends one token to a
    prefill tile)."""
    check_profile_device(profile)
    ext = extension()
    selections = profile.get("selections", {})
    covered = True
    for handle in handles:
        m, k = ext.shape(handle)
        choice = selections.get(dispatch_key(tokens, m, k))
        ext.set_prefill(handle, 1, _TUNING_MAX_ROWS)
        ext.set_prefill_backend(handle, int(choice["backend"]) if choice else CANDIDATES[BASELINE])
        covered = covered and choice is not None
    return covered


def selected_profile(artifact: Path) -> tuple[dict | None, Path]:
    """``(profile or None, its path)``; raises if a saved profile belongs to other weights or
    another kernel build."""
    target = profile_path(Path(artifact))
    if not target.is_file():
        return None, target
    profile = json.loads(target.read_text())
    checks = (("metadata_sha256", sha256_file(weights_dir(artifact) / "metadata.json"),
               "prefill profile does not match the encoded weights; rerun benchmark"),
              ("kernel_source_sha256", kernel_source_sha256(),
               "prefill profile does not match this Texelator build; rerun benchmark"))
    for key, expected, message in checks:
        if profile.get(key) != expected:
            raise RuntimeError(message)
    return profile, target
