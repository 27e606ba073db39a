"""Prefill tile autotuner (``texelator/autotune.py`` of the reference).

For each requested token count and each distinct (M, K) of an artifact, every tile candidate is
run on the same seeded input (``randn * 0.125``, seed ``20260827 + tokens*1009 + shape index``,
``autotune.py:139-143``), must be bitwise equal to the large tile (``autotune.py:150-168``), and
is timed round-robin with events (``autotune.py:170-193``); the lowest median wins. Selections
are stored per ``dispatch_key`` ("tokens<=bucket:M=m:K=k") in a profile gated by the weights'
metadata hash, the kernel-source hash and the device (gfx architecture and CU count instead of
compute capability and SM count, ``autotune.py:247-273``). The candidate ids 5..9 keep the
reference's backend numbering; their tiles are this build's.
"""
from __future__ import annotations

import hashlib
import json
import math
import statistics
from collections import Counter
from pathlib import Path

import torch

from .artifacts import sha256_file, weights_dir
from .hardware import device_key
from .runtime import PACKAGE_ROOT, extension, free, pack_entry_handles
from .store import STATE_HOME, safe_name

CANDIDATES = {
    "large_256x128x128": 5,
    "medium_128x128x128": 6,
    "medium_64x256x128": 7,
    "medium_64x128x128": 8,
    "small_32x128x128": 9,
}
BASELINE = "large_256x128x128"
TOKEN_BUCKETS = (32, 128, 512, 2048, 8192, 16384, 32768, 65535)


def profile_path(artifact: Path) -> Path:
    metadata_hash = sha256_file(weights_dir(artifact) / "metadata.json")
    device = safe_name(torch.cuda.get_device_name())
    return STATE_HOME / "profiles" / metadata_hash[:20] / f"{device_key()}-{device}-prefill.json"


def token_bucket(tokens: int) -> int:
    if tokens < 1:
        raise ValueError("tokens must be positive")
    if tokens > TOKEN_BUCKETS[-1]:
        raise ValueError(f"tokens exceeds the supported prefill range: {tokens}")
    return next(value for value in TOKEN_BUCKETS if tokens <= value)


def dispatch_key(tokens: int, m: int, k: int) -> str:
    return f"tokens<={token_bucket(tokens)}:M={m}:K={k}"


def kernel_source_sha256() -> str:
    """Hash of the HIP sources the library is built from (``autotune.py:54-60``)."""
    root = PACKAGE_ROOT / "csrc"
    digest = hashlib.sha256()
    for path in sorted(root.glob("*.hip")) + sorted(root.glob("*.h")):
        digest.update(path.name.encode())
        digest.update(path.read_bytes())
    return digest.hexdigest()


def _error(reference: torch.Tensor, candidate: torch.Tensor) -> dict:
    """``autotune.py:63-76``."""
    ref, value = reference.float(), candidate.float()
    delta = value - ref
    ref_rms = torch.sqrt(torch.mean(ref.square())).item()
    denominator = math.sqrt(torch.sum(ref.square()).item() * torch.sum(value.square()).item())
    return {
        "max_abs": float(delta.abs().max().item()),
        "mean_abs": float(delta.abs().mean().item()),
        "relative_rms": float(torch.sqrt(torch.mean(delta.square())).item() / max(ref_rms, 1e-30)),
        "cosine": float(torch.sum(ref * value).item() / max(denominator, 1e-30)),
        "bitwise_equal": bool(torch.equal(reference, candidate)),
    }


def _eligible(name: str, m: int, k: int) -> tuple[bool, str | None]:
    """Every gfx950 tile handles any M and any K divisible by 16 (partial tiles are masked)."""
    if m < 1:
        return False, "empty output dimension"
    if k % 16:
        return False, "K is not divisible by 16"
    return True, None


def _inventory(artifact: Path) -> tuple[list[int], dict[tuple[int, int], int], Counter]:
    weights = weights_dir(artifact)
    metadata = json.loads((weights / "metadata.json").read_text())
    handles: list[int] = []
    for entry in metadata["entries"]:
        handles.extend(pack_entry_handles(weights, entry, bias=None, lookahead=1, max_texture_rows=32768))
    ext = extension()
    representative: dict[tuple[int, int], int] = {}
    counts: Counter = Counter()
    for handle in handles:
        m, k = map(int, ext.handle_info(handle)[:2])
        counts[(m, k)] += 1
        representative.setdefault((m, k), handle)
        ext.set_prefill(handle, 1, 32768)
    return handles, representative, counts


def _device_record() -> dict:
    properties = torch.cuda.get_device_properties(torch.cuda.current_device())
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
    if warmup < 3 or measured < 10:
        raise ValueError("autotuning requires at least 3 warmups and 10 samples")
    artifact = Path(artifact).resolve()
    buckets = [token_bucket(value) for value in tokens]
    if len(buckets) != len(set(buckets)):
        raise ValueError("provide at most one representative token count per dispatch bucket")
    metadata_path = weights_dir(artifact) / "metadata.json"
    ext = extension()
    handles, representative, counts = _inventory(artifact)
    try:
        kernel_info = {name: ext.kernel_info(backend) for name, backend in CANDIDATES.items()}
        selections: dict[str, dict] = {}
        all_rows: list[dict] = []
        for token_count in tokens:
            bucket = token_bucket(token_count)
            for shape_index, ((m, k), handle) in enumerate(sorted(representative.items())):
                generator = torch.Generator(device="cuda").manual_seed(seed + token_count * 1009 + shape_index)
                x = torch.randn((token_count, k), device="cuda", dtype=torch.bfloat16, generator=generator)
                x.mul_(0.125)
                ext.set_prefill_backend(handle, CANDIDATES[BASELINE])
                with torch.inference_mode():
                    reference = ext.linear(handle, x)
                valid: list[str] = []
                correctness: dict[str, dict] = {}
                rejected: dict[str, str] = {}
                for name, backend in CANDIDATES.items():
                    supported, reason = _eligible(name, m, k)
                    if not supported:
                        rejected[name] = reason or "unsupported"
                        continue
                    ext.set_prefill_backend(handle, backend)
                    with torch.inference_mode():
                        candidate = ext.linear(handle, x)
                    metrics = _error(reference, candidate)
                    correctness[name] = metrics
                    if metrics["bitwise_equal"]:
                        valid.append(name)
                    else:
                        rejected[name] = f"correctness: rrms={metrics['relative_rms']:.6g}, cosine={metrics['cosine']:.9g}"
                    del candidate
                if BASELINE not in valid:
                    raise RuntimeError(f"baseline failed correctness for M={m},K={k}")
                for name in valid:
                    ext.set_prefill_backend(handle, CANDIDATES[name])
                    with torch.inference_mode():
                        for _ in range(warmup):
                            del_value = ext.linear(handle, x)
                            del del_value
                torch.cuda.synchronize()
                samples: dict[str, list[float]] = {name: [] for name in valid}
                for iteration in range(measured):
                    order = valid[iteration % len(valid):] + valid[:iteration % len(valid)]
                    for name in order:
                        ext.set_prefill_backend(handle, CANDIDATES[name])
                        start = torch.cuda.Event(enable_timing=True)
                        stop = torch.cuda.Event(enable_timing=True)
                        with torch.inference_mode():
                            start.record()
                            value = ext.linear(handle, x)
                            stop.record()
                        stop.synchronize()
                        samples[name].append(float(start.elapsed_time(stop)))
                        del value
                medians = {name: statistics.median(values) for name, values in samples.items()}
                winner = min(valid, key=lambda name: medians[name])
                key = dispatch_key(token_count, m, k)
                record = {
                    "key": key, "tokens_measured": token_count, "token_bucket": bucket, "M": m, "K": k,
                    "occurrences": int(counts[(m, k)]), "winner": winner, "backend": CANDIDATES[winner],
                    "median_ms": medians[winner], "baseline_ms": medians[BASELINE],
                    "speedup_vs_baseline": medians[BASELINE] / medians[winner],
                    "candidate_median_ms": medians, "correctness_vs_baseline": correctness, "rejected": rejected,
                }
                selections[key] = record
                all_rows.append(record)
                print(f"[autotune] tokens={token_count} M={m} K={k} winner={winner} {medians[winner]:.4f} ms "
                      f"speedup={record['speedup_vs_baseline']:.3f}x", flush=True)
                del x, reference
        profile = {
            "schema_version": 1,
            "status": "complete",
            "artifact": str(artifact),
            "metadata_sha256": sha256_file(metadata_path),
            "kernel_source_sha256": kernel_source_sha256(),
            "device": _device_record(),
            "protocol": {"tokens": tokens, "warmup": warmup, "measured": measured, "seed": seed,
                         "bitwise_correctness_required": True},
            "candidates": CANDIDATES,
            "kernel_info": kernel_info,
            "selections": selections,
            "rows": all_rows,
        }
        target = Path(output_path) if output_path else profile_path(artifact)
        target.parent.mkdir(parents=True, exist_ok=True)
        target.write_text(json.dumps(profile, indent=2) + "\n")
        print(f"[texelator] prefill profile saved to {target}", flush=True)
        return profile
    finally:
        free(handles)


def check_profile_device(profile: dict) -> None:
    """Raise unless the profile was made by this kernel build on this kind of device."""
    if profile.get("kernel_source_sha256") != kernel_source_sha256():
        raise RuntimeError("autotune profile kernel hash does not match this build")
    device = profile.get("device", {})
    if device.get("arch") != device_key():
        raise RuntimeError("autotune profile GPU architecture does not match this GPU")
    properties = torch.cuda.get_device_properties(torch.cuda.current_device())
    if device.get("multiprocessor_count") != int(properties.multi_processor_count):
        raise RuntimeError("autotune profile CU count does not match this GPU")


def apply_profile(handles: list[int], tokens: int, profile: dict) -> bool:
    """Set each handle's prefill tile for ``tokens`` from a profile (``autotune.py:247-273``).

    Returns False if some shape has no selection (it keeps the large tile). A one-token call
    still runs the decode GEMV: the gfx950 dispatch never sends one token to the prefill GEMM.
    """
    ext = extension()
    check_profile_device(profile)
    complete = True
    for handle in handles:
        m, k = map(int, ext.handle_info(handle)[:2])
        selection = profile.get("selections", {}).get(dispatch_key(tokens, m, k))
        ext.set_prefill(handle, 1, 32768)
        if selection is None:
            ext.set_prefill_backend(handle, CANDIDATES[BASELINE])
            complete = False
            continue
        ext.set_prefill_backend(handle, int(selection["backend"]))
    return complete


def selected_profile(artifact: Path) -> tuple[dict | None, Path]:
    """The saved profile of an artifact, checked against its weights and this build (``autotune.py:276-286``)."""
    artifact = Path(artifact)
    target = profile_path(artifact)
    if not target.is_file():
        return None, target
    profile = json.loads(target.read_text())
    if profile.get("metadata_sha256") != sha256_file(weights_dir(artifact) / "metadata.json"):
        raise RuntimeError("prefill profile does not match the encoded weights; rerun benchmark")
    if profile.get("kernel_source_sha256") != kernel_source_sha256():
        raise RuntimeError("prefill profile does not match this Texelator build; rerun benchmark")
    return profile, target
