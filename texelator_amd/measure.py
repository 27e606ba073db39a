"""Event timing and output comparison shared by the tuners and the prefill benchmark.

* :func:`round_robin_medians` times several candidates against each other the way the
  reference's tile autotuner does (``autotune.py:170-193``): one sample of each candidate per
  round, the starting candidate rotated every round so that none always runs first, each sample
  bracketed by events on the current stream; the statistic is the median per candidate.
* :func:`mean_time_ms` is the decode tuner's figure (``tuning.py:82-98``): events around
  ``repeats`` back-to-back calls, divided by ``repeats``.
* :func:`output_error` holds the closed-form comparison metrics of ``autotune.py:63-76``.
"""
from __future__ import annotations

import math
import statistics
from typing import Callable, Mapping

import torch


def _event_pair() -> tuple[torch.cuda.Event, torch.cuda.Event]:
    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


def mean_time_ms(fn: Callable[[], object], repeats: int) -> float:
    """Milliseconds per call of ``fn`` over ``repeats`` calls between two events (no sync inside)."""
    if repeats < 1:
        raise ValueError("repeats must be positive")
    begin, end = _event_pair()
    begin.record()
    for _ in range(repeats):
        fn()
    end.record()
    end.synchronize()
    return begin.elapsed_time(end) / repeats


def round_robin_medians(runners: Mapping[str, Callable[[], object]], warmup: int,
                        rounds: int) -> tuple[dict[str, float], dict[str, list[float]]]:
    """``(medians, samples)`` in milliseconds for every runner, ``rounds`` samples each, after
    ``warmup`` untimed calls of each."""
    names = list(runners)
    if not names:
        raise ValueError("nothing to time")
    with torch.inference_mode():
        for name in names:
            for _ in range(warmup):
                runners[name]()
        torch.cuda.synchronize()
        samples: dict[str, list[float]] = {name: [] for name in names}
        for turn in range(rounds):
            shift = turn % len(names)
            for name in names[shift:] + names[:shift]:
                begin, end = _event_pair()
                begin.record()
                runners[name]()
                end.record()
                end.synchronize()
                samples[name].append(float(begin.elapsed_time(end)))
    return {name: statistics.median(values) for name, values in samples.items()}, samples


def output_error(reference: torch.Tensor, candidate: torch.Tensor) -> dict:
    """max/mean absolute difference, relative RMS (against the reference's RMS) and cosine,
    computed in float64, plus bitwise equality of the raw tensors."""
    want = reference.detach().to(torch.float64).reshape(-1)
    got = candidate.detach().to(torch.float64).reshape(-1)
    diff = got - want
    n = max(1, want.numel())
    want_sq = float(torch.dot(want, want))
    got_sq = float(torch.dot(got, got))
    diff_sq = float(torch.dot(diff, diff))
    want_rms = math.sqrt(want_sq / n)
    return {
        "max_abs": float(diff.abs().max()) if diff.numel() else 0.0,
        "mean_abs": float(diff.abs().sum()) / n,
        "relative_rms": math.sqrt(diff_sq / n) / max(want_rms, 1e-30),
        "cosine": float(torch.dot(want, got)) / max(math.sqrt(want_sq * got_sq), 1e-30),
        "bitwise_equal": bool(torch.equal(reference, candidate)),
    }
