"""Numerical gate and paired GPU timing protocol for decode comparisons.

Reference: ``acceleration_checks.py`` (``numerical_gate`` :7-22,
``stepwise_nrmse`` :25-41, ``paired_cuda_timing`` :44-64).  Same frozen
thresholds and result keys, so reports from either implementation compare.
"""
from __future__ import annotations

import statistics

import torch


def numerical_gate(actual: torch.Tensor, expected: torch.Tensor) -> dict:
    """Combined elementwise + normalized-RMSE gate (frozen v1 thresholds).

    Elementwise: ``|a - b| <= tol * (rms(b) + |b|) + 1e-6`` everywhere, with
    ``tol = 0.02`` for bf16 references and ``0.002`` otherwise; and
    ``nrmse = rms(a - b) / rms(b) <= tol / 4``.  Computed in float64.
    """
    if actual.shape != expected.shape:
        return {"passed": False, "reason": "shape mismatch"}
    a = actual.detach().double()
    b = expected.detach().double()
    if not bool(torch.isfinite(a).all()) or not bool(torch.isfinite(b).all()):
        return {"passed": False, "reason": "nonfinite output"}
    rms = b.square().mean().sqrt().item()
    error = a - b
    nrmse = error.square().mean().sqrt().item() / max(rms, 1e-12)
    tol = 0.02 if expected.dtype == torch.bfloat16 else 0.002
    elementwise = bool((error.abs() <= tol * (rms + b.abs()) + 1e-6).all())
    return {"passed": elementwise and nrmse <= tol / 4, "max_abs_error": error.abs().max().item(),
            "reference_rms": rms, "normalized_rmse": nrmse, "elementwise_tolerance_factor": tol,
            "normalized_rmse_limit": tol / 4}


def stepwise_nrmse(actual: torch.Tensor, expected: torch.Tensor):
    """Per-step NRMSE of ``[1, steps, vocab]`` logits (report only); None otherwise."""
    if actual.shape != expected.shape or actual.ndim != 3 or actual.shape[0] != 1:
        return None
    a = actual.detach().double()
    b = expected.detach().double()
    if not bool(torch.isfinite(a).all()) or not bool(torch.isfinite(b).all()):
        return None
    rms = b.square().mean(dim=-1).sqrt().clamp_min(1e-12)
    return [float(v) for v in ((a - b).square().mean(dim=-1).sqrt() / rms)[0]]


def paired_cuda_timing(functions: dict, *, warmup: int = 20, repeats: int = 100, rounds: int = 7) -> dict:
    """Median microseconds per call of each function, arms alternated per round.

    Every arm gets ``warmup`` untimed calls; then ``rounds`` rounds, each timing
    ``repeats`` back-to-back calls per arm with GPU events, in forward order on
    even rounds and reversed order on odd rounds to cancel ordering bias.
    ``stable`` flags a (max - min) / median spread of at most 10%.
    """
    if warmup < 1 or repeats < 1 or rounds < 3:
        raise ValueError("positive warmup/repeats and at least three rounds required")
    for fn in functions.values():
        for _ in range(warmup):
            fn()
    torch.cuda.synchronize()
    names = list(functions)
    samples = {name: [] for name in names}
    for index in range(rounds):
        for name in (names if index % 2 == 0 else names[::-1]):
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record()
            for _ in range(repeats):
                functions[name]()
            end.record()
            end.synchronize()
            samples[name].append(start.elapsed_time(end) * 1000 / repeats)
    result = {}
    for name, values in samples.items():
        median = statistics.median(values)
        spread = (max(values) - min(values)) / median if median > 0 else float("inf")
        result[name] = {"microseconds_per_call": values, "median_us": median, "relative_range": spread,
                        "stable": spread <= 0.10}
    return result
