"""Numerical gate and paired GPU timing protocol for decode comparisons.

Contract of the reference's ``acceleration_checks.py`` (``numerical_gate`` :7-22,
``stepwise_nrmse`` :25-41, ``paired_cuda_timing`` :44-64): the frozen v1 gate
thresholds (elementwise factor 0.02 against a bf16 reference, 0.002 otherwise;
normalized RMSE limit a quarter of it), the result keys, and the timing schedule
(warm-up per arm, alternating arm order per round, median, 10% stability bound)
are kept so reports from either implementation compare.  The code is organised
around an error-statistics record and a precomputed round schedule.
"""
from __future__ import annotations

import statistics
from dataclasses import dataclass

import torch

GATE_FACTOR = {torch.bfloat16: 0.02}  # elementwise tolerance factor by reference dtype
DEFAULT_GATE_FACTOR = 0.002
STABLE_RELATIVE_RANGE = 0.10


@dataclass(frozen=True)
class _ErrorStats:
    rms: float          # root mean square of the reference
    max_abs: float
    nrmse: float
    within: bool        # every |a - b| <= factor * (rms + |b|) + 1e-6

    @classmethod
    def of(cls, actual: torch.Tensor, expected: torch.Tensor, factor: float) -> "_ErrorStats":
        a = actual.detach().to(torch.float64)
        b = expected.detach().to(torch.float64)
        error = a - b
        rms = float(torch.linalg.vector_norm(b) / b.numel() ** 0.5)
        nrmse = float(torch.linalg.vector_norm(error) / error.numel() ** 0.5) / max(rms, 1e-12)
        within = bool((error.abs() <= factor * (rms + b.abs()) + 1e-6).all())
        return cls(rms, float(error.abs().max()), nrmse, within)


def _finite(*tensors: torch.Tensor) -> bool:
    return all(bool(torch.isfinite(t.detach()).all()) for t in tensors)


def numerical_gate(actual: torch.Tensor, expected: torch.Tensor) -> dict:
    """Combined elementwise + normalized-RMSE gate (frozen v1 thresholds).

    Passes when ``|a - b| <= f * (rms(b) + |b|) + 1e-6`` holds everywhere and
    ``rms(a - b) / rms(b) <= f / 4``, with ``f = 0.02`` for a bf16 ``expected`` and
    ``0.002`` otherwise; statistics in float64.
    """
    if actual.shape != expected.shape:
        return {"passed": False, "reason": "shape mismatch"}
    if not _finite(actual, expected):
        return {"passed": False, "reason": "nonfinite output"}
    factor = GATE_FACTOR.get(expected.dtype, DEFAULT_GATE_FACTOR)
    stats = _ErrorStats.of(actual, expected, factor)
    limit = factor / 4
    return {"passed": stats.within and stats.nrmse <= limit, "max_abs_error": stats.max_abs,
            "reference_rms": stats.rms, "normalized_rmse": stats.nrmse,
            "elementwise_tolerance_factor": factor, "normalized_rmse_limit": limit}


def stepwise_nrmse(actual: torch.Tensor, expected: torch.Tensor):
    """Per-step NRMSE of ``[1, steps, vocab]`` logits (report only); None for any
    other shape, mismatched shapes or non-finite values."""
    if actual.shape != expected.shape or actual.ndim != 3 or actual.shape[0] != 1:
        return None
    if not _finite(actual, expected):
        return None
    a = actual.detach().to(torch.float64)[0]
    b = expected.detach().to(torch.float64)[0]
    width = b.shape[-1] ** 0.5
    error_rms = torch.linalg.vector_norm(a - b, dim=-1) / width
    reference_rms = (torch.linalg.vector_norm(b, dim=-1) / width).clamp_min(1e-12)
    return (error_rms / reference_rms).tolist()


def _round_schedule(names: list[str], rounds: int) -> list[list[str]]:
    """Arm order per round: forward on even rounds, reversed on odd ones (cancels
    a systematic first-arm / last-arm bias)."""
    return [names if r % 2 == 0 else names[::-1] for r in range(rounds)]


def _summary(samples: list[float]) -> dict:
    median = statistics.median(samples)
    spread = (max(samples) - min(samples)) / median if median > 0 else float("inf")
    return {"microseconds_per_call": samples, "median_us": median, "relative_range": spread,
            "stable": spread <= STABLE_RELATIVE_RANGE}


def paired_cuda_timing(functions: dict, *, warmup: int = 20, repeats: int = 100, rounds: int = 7) -> dict:
    """Median microseconds per call of each arm, arms alternated per round.

    Each arm gets ``warmup`` untimed calls; then each round times ``repeats``
    back-to-back calls per arm between two events recorded on the current
    stream.  ``stable`` flags a (max - min) / median spread of at most 10%.
    """
    if warmup < 1 or repeats < 1 or rounds < 3:
        raise ValueError("positive warmup/repeats and at least three rounds required")
    for fn in functions.values():
        for _ in range(warmup):
            fn()
    torch.cuda.synchronize()
    samples: dict[str, list[float]] = {name: [] for name in functions}
    for order in _round_schedule(list(functions), rounds):
        for name in order:
            fn = functions[name]
            begin = torch.cuda.Event(enable_timing=True)
            finish = torch.cuda.Event(enable_timing=True)
            begin.record()
            for _ in range(repeats):
                fn()
            finish.record()
            finish.synchronize()
            samples[name].append(begin.elapsed_time(finish) * 1e3 / repeats)
    return {name: _summary(values) for name, values in samples.items()}
