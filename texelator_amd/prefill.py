"""Prefill and decode benchmarks of a BC4 decoder (``texelator/prefill.py`` of the reference).

``benchmark_prefill`` keeps the reference's protocol (``prefill.py:63-131``):
1. Correctness on the first <= 32 prompt tokens. The "scalar" path sends every token through the
   decode GEMV (prefill threshold 1<<30); the hybrid path uses the prefill GEMM (threshold 1).
   Their final hidden states must agree within relative RMS 0.02 (``prefill.py:88-108``).
2. ``warmup`` + ``runs`` timed forwards of each path, as wall-clock and event medians with tokens/s
   (``prefill.py:29-60``).

The prompt is ``randint(0, vocab, (tokens,))`` from a CPU generator seeded 0 (``prefill.py:82-85``).
The model is a :class:`texelator_amd.modeling.BC4Decoder`, either passed in or loaded from an
artifact whose manifest carries a ``decoder`` config.

``benchmark_decode`` times greedy decode steps replayed as HIP graphs, from the prompt length up
to a context length.
"""
from __future__ import annotations

import json
import math
import statistics
import time
from dataclasses import asdict
from pathlib import Path

import numpy as np
import torch

from .artifacts import environment_snapshot, read_manifest, weights_dir, write_json
from .modeling import BC4Decoder, DecoderConfig
from .runtime import PREFILL_THRESHOLD, PREFILL_TILE_ROWS

CORRECTNESS_TOKENS = 32
RRMS_LIMIT = 0.02


def load_decoder(artifact: Path, max_context: int, lookahead: int = 1, seed: int = 0) -> BC4Decoder:
    """A decoder whose linears come from an artifact (``model.layers.{i}.{self_attn|mlp}.*_proj``
    entries) and whose other parameters are seeded random; the manifest's ``decoder`` holds the
    :class:`DecoderConfig` fields."""
    manifest = read_manifest(artifact)
    if "decoder" not in manifest:
        raise RuntimeError("the prefill benchmark requires an artifact with a 'decoder' config")
    config = DecoderConfig(**manifest["decoder"])
    weights = weights_dir(artifact)
    entries = {e["module_name"]: e for e in json.loads((weights / "metadata.json").read_text())["entries"]}

    def source(layer: int, name: str, m: int, k: int):
        entry = entries.get(f"model.layers.{layer}.{name}")
        if entry is None:
            raise RuntimeError(f"artifact has no entry for model.layers.{layer}.{name}")
        if (int(entry["M"]), int(entry["K"])) != (m, k):
            raise RuntimeError(f"model.layers.{layer}.{name} is {entry['M']}x{entry['K']}, expected {m}x{k}")
        blocks = torch.from_numpy(np.fromfile(weights / entry["blocks_file"], dtype=np.uint8)).cuda()
        scales = torch.from_numpy(np.fromfile(weights / entry["scales_file"], dtype="<f4")).cuda()
        return blocks, scales

    return BC4Decoder(config, max_context, lookahead=lookahead, seed=seed, linear_source=source)


def _forward(model: BC4Decoder, ids: torch.Tensor) -> torch.Tensor:
    with torch.inference_mode():
        return model.hidden_states(ids, model.key_positions[:ids.numel()], ids.numel())


def _measure(model: BC4Decoder, ids: torch.Tensor, warmup: int, runs: int) -> dict:
    for _ in range(warmup):
        _forward(model, ids)
    torch.cuda.synchronize()
    wall, gpu = [], []
    for _ in range(runs):
        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)
        before = time.perf_counter()
        start.record()
        _forward(model, ids)
        stop.record()
        torch.cuda.synchronize()
        wall.append(time.perf_counter() - before)
        gpu.append(start.elapsed_time(stop) / 1000.0)
    tokens = int(ids.numel())
    return {
        "tokens": tokens, "warmup": warmup, "runs": runs, "wall_seconds": wall, "gpu_seconds": gpu,
        "wall_seconds_median": statistics.median(wall), "gpu_seconds_median": statistics.median(gpu),
        "wall_tokens_per_second": tokens / statistics.median(wall),
        "gpu_tokens_per_second": tokens / statistics.median(gpu),
    }


def prompt_ids(model: BC4Decoder, tokens: int, seed: int = 0) -> torch.Tensor:
    generator = torch.Generator(device="cpu").manual_seed(seed)
    return torch.randint(0, model.config.vocab, (tokens,), generator=generator, dtype=torch.int64).to(model.device)


def benchmark_prefill(source, tokens: int, warmup: int, runs: int, output: Path | None = None,
                      max_context: int | None = None, rrms_limit: float | None = RRMS_LIMIT) -> dict:
    """``rrms_limit=None`` reports the correctness figures without enforcing the gate."""
    if not torch.cuda.is_available():
        raise RuntimeError("prefill benchmark requires a visible GPU")
    if tokens < PREFILL_THRESHOLD:
        raise ValueError(f"tokens must be at least the hybrid threshold ({PREFILL_THRESHOLD})")
    if warmup < 0 or runs < 1:
        raise ValueError("warmup must be non-negative and runs must be positive")
    owned = not isinstance(source, BC4Decoder)
    model = load_decoder(Path(source), max_context or tokens) if owned else source
    try:
        ids = prompt_ids(model, tokens)
        check_ids = ids[:min(tokens, CORRECTNESS_TOKENS)]
        model.set_prefill(1 << 30, PREFILL_TILE_ROWS)
        reference = _forward(model, check_ids).float()
        model.set_prefill(1, PREFILL_TILE_ROWS)
        candidate = _forward(model, check_ids).float()
        difference = candidate - reference
        reference_rms = float(torch.sqrt(torch.mean(reference * reference)).item())
        correctness = {
            "tokens": int(check_ids.numel()),
            "max_abs": float(difference.abs().max().item()),
            "relative_rms": float(torch.sqrt(torch.mean(difference * difference)).item()) / max(reference_rms, 1e-12),
            "cosine": float(torch.nn.functional.cosine_similarity(reference.reshape(1, -1),
                                                                  candidate.reshape(1, -1)).item()),
        }
        correctness["limit"] = rrms_limit
        if rrms_limit is not None and (not math.isfinite(correctness["relative_rms"])
                                       or correctness["relative_rms"] > rrms_limit):
            raise RuntimeError(f"hybrid prefill correctness failed: {correctness}")
        model.set_prefill(1 << 30, PREFILL_TILE_ROWS)
        scalar = _measure(model, ids, warmup, runs)
        model.set_prefill(1, PREFILL_TILE_ROWS)
        hybrid = _measure(model, ids, warmup, runs)
        result = {
            "schema_version": 1,
            "model": asdict(model.config),
            "prefill_tile_rows": PREFILL_TILE_ROWS,
            "correctness": correctness,
            "scalar_gemv": scalar,
            "fused_bc4_mfma": hybrid,
            "speedup_wall": scalar["wall_seconds_median"] / hybrid["wall_seconds_median"],
            "speedup_gpu": scalar["gpu_seconds_median"] / hybrid["gpu_seconds_median"],
            "environment": environment_snapshot(),
        }
        if output is not None:
            write_json(Path(output), result)
        return result
    finally:
        model.set_prefill(PREFILL_THRESHOLD, PREFILL_TILE_ROWS)
        if owned:
            model.close()


def benchmark_decode(model: BC4Decoder, prompt_tokens: int, context: int, warmup_steps: int = 8,
                     sample_steps: int | None = None) -> dict:
    """Prefill ``prompt_tokens``, then time greedy decode steps (graph replays) until the cache
    holds ``context`` tokens. Returns overall and per-512-bucket tokens/s.

    With ``sample_steps``, each 512-position bucket is timed on its first ``sample_steps`` steps
    only, starting at the bucket's first position; the overall rate is then the step-weighted
    projection over the whole range (``projected``: True). The cache rows skipped this way hold
    stale values, which cost the same to read."""
    if context > model.max_context or prompt_tokens >= context:
        raise ValueError("need prompt_tokens < context <= max_context")
    ids = prompt_ids(model, prompt_tokens)
    for length in sorted({model._bucket(p) for p in range(prompt_tokens, context)}):
        model.capture(length)                     # every bucket the timed steps use, before timing
    model.prefill(ids)
    torch.cuda.synchronize()
    warm = min(warmup_steps, context - prompt_tokens - 1)
    model.decode(warm, prompt_tokens)             # untimed: first replays
    model.prefill(ids)                            # reset the cache state to the prompt
    torch.cuda.synchronize()
    buckets: dict[int, tuple[int, int, float]] = {}
    position = prompt_tokens
    start_all = time.perf_counter()
    while position < context:
        length = model._bucket(position)
        span = min(context, length) - position
        steps = span if sample_steps is None else min(span, sample_steps)
        model.position.fill_(position)
        begin = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        begin.record()
        model.decode(steps, position)
        end.record()
        end.synchronize()
        buckets[length] = (span, steps, begin.elapsed_time(end) / 1000.0)
        position += span
    wall = time.perf_counter() - start_all
    steps_total = context - prompt_tokens
    projected_gpu = sum(span * seconds / steps for span, steps, seconds in buckets.values())
    return {
        "prompt_tokens": prompt_tokens, "context": context, "steps": steps_total,
        "timed_steps": sum(steps for _, steps, _ in buckets.values()), "projected": sample_steps is not None,
        "wall_seconds": wall, "gpu_seconds": projected_gpu,
        "gpu_tokens_per_second": steps_total / projected_gpu,
        "ms_per_token": projected_gpu / steps_total * 1e3,
        "per_bucket": {str(length): {"steps": steps, "tokens_per_second": steps / seconds}
                       for length, (_, steps, seconds) in buckets.items()},
    }
