"""Prefill and decode benchmarks of a BC4 model (``texelator/prefill.py`` of the reference).

``benchmark_prefill`` keeps the reference's protocol (``prefill.py:63-131``), which defines what its
prefill tok/s means:
1. Correctness on the first <= 32 prompt tokens. The "scalar" path sends every token through the
   decode GEMV (prefill threshold 1<<30); the hybrid path uses the prefill GEMM (threshold 1).
   Their final hidden states must agree within relative RMS 0.02 (``prefill.py:88-108``).
2. ``warmup`` + ``runs`` timed forwards of each path, as wall-clock and event medians with tokens/s
   (``prefill.py:29-60``).

The prompt is ``randint(0, vocab, (tokens,))`` from a CPU generator seeded 0 (``prefill.py:82-85``).
The model is either this build's :class:`texelator_amd.modeling.BC4Decoder` or, as in the
reference, a Hugging Face causal LM whose linears are ``TexelatorLinear`` modules
(``runtime.install``, ``runtime.install_standalone``, :func:`texelator_amd.hf.build_qwen2`), whose
forward is ``model.model(input_ids=...)`` (``prefill.py:24-26``).

``benchmark_decode`` times greedy decode steps of a ``BC4Decoder`` replayed as HIP graphs, from the
prompt length up to a context length.
"""
from __future__ import annotations

import math
import statistics
import time
from dataclasses import asdict
from pathlib import Path
from typing import NamedTuple

import torch

from .artifacts import environment_snapshot, write_json
from .modeling import BC4Decoder
from .runtime import PREFILL_THRESHOLD, PREFILL_TILE_ROWS, extension

CORRECTNESS_TOKENS = 32
RRMS_LIMIT = 0.02


class GateFailed(RuntimeError):
    """The hybrid path missed the correctness gate; ``correctness`` holds the figures."""

    def __init__(self, correctness: dict):
        super().__init__(f"hybrid prefill correctness failed: {correctness}")
        self.correctness = correctness


class _Target:
    """What the protocol drives: a forward over one token row returning the final hidden states
    ``[tokens, hidden]``, and the prefill threshold of every BC4 handle of the model."""

    def __init__(self, model):
        if isinstance(model, BC4Decoder):
            self.handles = list(model.handles)
            self.vocab = model.config.vocab
            self.device = model.device
            self.description = asdict(model.config)
            self._forward = lambda ids, cache: model.hidden_states(ids, model.key_positions[:ids.numel()], ids.numel())
            return
        handles = getattr(model, "_texelator_handles", None)
        if not handles or not hasattr(model, "model"):
            raise TypeError("benchmark_prefill needs a BC4Decoder or a causal LM with installed Texelator linears")
        from torch.nn.attention import SDPBackend, sdpa_kernel

        self.handles = list(handles)
        self.vocab = int(model.get_input_embeddings().weight.shape[0])
        self.device = model.get_input_embeddings().weight.device
        self.description = {"hf_class": type(model).__name__, **{
            key: getattr(model.config, key, None) for key in
            ("num_hidden_layers", "hidden_size", "intermediate_size", "num_attention_heads", "num_key_value_heads")}}

        def forward(ids, cache):
            with sdpa_kernel([SDPBackend.FLASH_ATTENTION]):
                out = model.model(input_ids=ids[None, :], use_cache=cache, return_dict=True)
            return out.last_hidden_state[0]

        self._forward = forward

    def set_threshold(self, threshold: int) -> None:
        ext = extension()
        for handle in self.handles:
            ext.set_prefill(handle, threshold, PREFILL_TILE_ROWS)

    def forward(self, ids: torch.Tensor, use_cache: bool = False) -> torch.Tensor:
        """Final hidden states; ``use_cache`` lets a Hugging Face model build its KV cache, as the
        reference's timed forwards do (``prefill.py:29-60``)."""
        with torch.inference_mode():
            return self._forward(ids, use_cache)


class _Sample(NamedTuple):
    wall: float
    gpu: float


def _timed(target: _Target, ids: torch.Tensor, warmup: int, runs: int) -> dict:
    """Median wall-clock and event time of ``runs`` forwards after ``warmup`` untimed ones."""
    for _ in range(warmup):
        target.forward(ids, use_cache=True)
    torch.cuda.synchronize()
    samples: list[_Sample] = []
    while len(samples) < runs:
        begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        started = time.perf_counter()
        begin.record()
        target.forward(ids, use_cache=True)
        end.record()
        torch.cuda.synchronize()
        samples.append(_Sample(time.perf_counter() - started, begin.elapsed_time(end) / 1e3))
    tokens = int(ids.numel())
    wall = statistics.median(s.wall for s in samples)
    gpu = statistics.median(s.gpu for s in samples)
    return {"tokens": tokens, "warmup": warmup, "runs": runs,
            "wall_seconds": [s.wall for s in samples], "gpu_seconds": [s.gpu for s in samples],
            "wall_seconds_median": wall, "gpu_seconds_median": gpu,
            "wall_tokens_per_second": tokens / wall, "gpu_tokens_per_second": tokens / gpu}


def _agreement(reference: torch.Tensor, candidate: torch.Tensor) -> dict:
    """Relative RMS, largest absolute difference and cosine of two hidden-state tensors."""
    ref, cand = reference.float().reshape(-1), candidate.float().reshape(-1)
    ref_rms = float(ref.square().mean().sqrt())
    diff = cand - ref
    return {"max_abs": float(diff.abs().max()),
            "relative_rms": float(diff.square().mean().sqrt()) / max(ref_rms, 1e-12),
            "cosine": float(torch.nn.functional.cosine_similarity(ref[None], cand[None]))}


def prompt_ids(model, tokens: int, seed: int = 0) -> torch.Tensor:
    """The protocol's prompt: ``tokens`` ids uniform over the vocabulary, CPU generator ``seed``."""
    target = model if isinstance(model, _Target) else _Target(model)
    generator = torch.Generator(device="cpu").manual_seed(seed)
    return torch.randint(0, target.vocab, (tokens,), generator=generator, dtype=torch.int64).to(target.device)


def benchmark_prefill(model, tokens: int, warmup: int, runs: int, output: Path | None = None,
                      rrms_limit: float | None = RRMS_LIMIT) -> dict:
    """The reference's prefill benchmark on ``model`` (a ``BC4Decoder`` or a Hugging Face model
    with Texelator linears). Raises if the hybrid path fails the correctness gate; with
    ``rrms_limit=None`` the figures are reported without the gate."""
    if not torch.cuda.is_available():
        raise RuntimeError("prefill benchmark requires a visible GPU")
    if tokens < PREFILL_THRESHOLD:
        raise ValueError(f"tokens must be at least the hybrid threshold ({PREFILL_THRESHOLD})")
    if warmup < 0 or runs < 1:
        raise ValueError("warmup must be non-negative and runs must be positive")
    target = _Target(model)
    try:
        ids = prompt_ids(target, tokens)
        check = ids[:min(tokens, CORRECTNESS_TOKENS)]
        hidden = {}
        for path, threshold in (("scalar", 1 << 30), ("hybrid", 1)):
            target.set_threshold(threshold)
            hidden[path] = target.forward(check).float()
        correctness = {"tokens": int(check.numel()), **_agreement(hidden["scalar"], hidden["hybrid"]),
                       "limit": rrms_limit}
        del hidden
        failed = not math.isfinite(correctness["relative_rms"]) or (
            rrms_limit is not None and correctness["relative_rms"] > rrms_limit)
        if rrms_limit is not None and failed:
            raise GateFailed(correctness)
        timings = {}
        for path, threshold in (("scalar_gemv", 1 << 30), ("fused_bc4_mfma", 1)):
            target.set_threshold(threshold)
            timings[path] = _timed(target, ids, warmup, runs)
        result = {
            "schema_version": 1,
            "model": target.description,
            "prefill_tile_rows": PREFILL_TILE_ROWS,
            "correctness": correctness,
            **timings,
            "speedup_wall": timings["scalar_gemv"]["wall_seconds_median"] / timings["fused_bc4_mfma"]["wall_seconds_median"],
            "speedup_gpu": timings["scalar_gemv"]["gpu_seconds_median"] / timings["fused_bc4_mfma"]["gpu_seconds_median"],
            "environment": environment_snapshot(),
        }
        if output is not None:
            write_json(Path(output), result)
        return result
    finally:
        target.set_threshold(PREFILL_THRESHOLD)


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
