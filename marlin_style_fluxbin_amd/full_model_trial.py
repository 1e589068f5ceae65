"""Dynamic-KV decode trace and trace comparison for HF Qwen3 models with packed Linears.

Contract of the reference's ``full_model_trial.py`` (``packed_modules`` :10-12,
``decode_trace`` :15-78, ``compare_trace`` :81-93, ``validate_routes`` :96-99):
the same arguments, result keys, route expectations and error messages.  The
trace is the oracle side of a decode comparison: the prompt runs once through
the dense fallback, then exactly ``steps`` one-token calls on one growing dynamic
cache must take the packed route (the fallback is switched to ``error`` for
them).

Organisation here: a ``_StageClock`` pairs a wall clock with GPU events for one
timed stage, ``_fallback_policy`` owns the temporary fallback switch and its
restoration, and ``_next_token`` is the one greedy step both stages share.
"""
from __future__ import annotations

import time
from contextlib import contextmanager

import torch

from .acceleration_checks import numerical_gate, stepwise_nrmse
from .deployment import PackedHybridLinear
from .w3_lut_deployment import PackedW3Linear

PACKED_TYPES = (PackedHybridLinear, PackedW3Linear)


def packed_modules(model) -> dict:
    """Every packed Linear of ``model`` (W3 and hybrid two-base), by module name."""
    return {name: module for name, module in model.named_modules() if isinstance(module, PACKED_TYPES)}


class _StageClock:
    """Wall time of a stage plus, on GPU, its device time between two events."""

    def __init__(self, device: torch.device):
        self.device = device
        self.gpu = device.type == "cuda"
        self.wall_ms = 0.0
        self._events = None

    def __enter__(self):
        if self.gpu:
            torch.cuda.synchronize(self.device)
            self._events = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
        self._t0 = time.perf_counter()
        if self.gpu:
            self._events[0].record()
        return self

    def __exit__(self, *exc):
        if self.gpu:
            self._events[1].record()
            torch.cuda.synchronize(self.device)
        self.wall_ms = (time.perf_counter() - self._t0) * 1e3
        return False

    @property
    def device_ms(self):
        return self._events[0].elapsed_time(self._events[1]) if self._events else None


@contextmanager
def _fallback_policy(modules: dict):
    """Reset route counters; yield a setter for every module's fallback; restore
    the original fallbacks on exit, whatever happened."""
    original = {name: module.fallback for name, module in modules.items()}
    for module in modules.values():
        module.reset_route_counts()

    def set_all(policy: str) -> None:
        for module in modules.values():
            module.fallback = policy
    try:
        yield set_all
    finally:
        for name, module in modules.items():
            module.fallback = original[name]


def _next_token(model, input_ids, cache):
    """One forward with the cache; (last logits, greedy token, cache)."""
    output = model(input_ids=input_ids, past_key_values=cache, use_cache=True, logits_to_keep=1)
    logits = output.logits[:, -1, :].detach()
    return logits, logits.argmax(-1, keepdim=True), output.past_key_values


def _cache_length(cache) -> int:
    length = cache.get_seq_length()
    return int(length.item()) if isinstance(length, torch.Tensor) else int(length)


@torch.inference_mode()
def decode_trace(model, input_ids: torch.Tensor, *, steps: int, forced_tokens: torch.Tensor | None = None) -> dict:
    """Prefill once, then exactly ``steps`` M=1 calls on a dynamic KV cache.

    Returns ``steps + 1`` predictions (the prefill's included), the logits, the
    fed tokens, the cache length, wall / device times and per-module routes.
    ``forced_tokens [1, steps]`` feeds a fixed continuation (identical contexts
    across arms); otherwise the greedy token is fed back.
    """
    if input_ids.ndim != 2 or input_ids.shape[0] != 1 or input_ids.shape[1] < 2 or steps < 1:
        raise ValueError("batch1, prompt length>=2 and positive decode steps required")
    if forced_tokens is not None and tuple(forced_tokens.shape) != (1, steps):
        raise ValueError("forced continuation shape must be [1,steps]")
    device = input_ids.device
    feed = None if forced_tokens is None else forced_tokens.to(device)
    modules = packed_modules(model)
    gpu = device.type == "cuda"
    with _fallback_policy(modules) as set_fallback:
        set_fallback("dense")
        with _StageClock(device) as prefill:
            logits, token, cache = _next_token(model, input_ids, None)
        all_logits, predictions, fed, step_events = [logits], [token], [], []
        set_fallback("error")  # every decode step must take the packed route
        with _StageClock(device) as decode:
            for i in range(steps):
                token = token if feed is None else feed[:, i:i + 1]
                fed.append(token)
                events = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) if gpu else None
                if events:
                    events[0].record()
                logits, token, cache = _next_token(model, token, cache)
                if events:
                    events[1].record()
                    step_events.append(events)
                all_logits.append(logits)
                predictions.append(token)
        length = _cache_length(cache)
        if length != input_ids.shape[1] + steps:
            raise RuntimeError("KV cache length drift")
        return {
            "logits": torch.stack(all_logits, dim=1).cpu(),
            "predictions": torch.cat(predictions, dim=1).cpu(),
            "fed_tokens": torch.cat(fed, dim=1).cpu(),
            "cache_length": length,
            "prefill_wall_ms": prefill.wall_ms,
            "decode_wall_ms": decode.wall_ms,
            "prefill_device_ms": prefill.device_ms,
            "decode_device_ms": decode.device_ms,
            "step_device_ms": [begin.elapsed_time(end) for begin, end in step_events],
            "routes": {name: dict(module.route_counts) for name, module in modules.items()},
        }


def compare_trace(candidate: dict, reference: dict, *, logprob_tolerance: float) -> dict:
    """Pass iff the logits gate passes, greedy tokens and fed contexts are equal,
    and the max |log-softmax difference| is finite and within ``logprob_tolerance``."""
    if logprob_tolerance < 0:
        raise ValueError("negative logprob tolerance")
    cand, ref = candidate["logits"], reference["logits"]
    gate = numerical_gate(cand, ref)
    if cand.shape != ref.shape:
        return {"passed": False, "reason": "shape drift"}
    checks = {
        "greedy_tokens_equal": torch.equal(candidate["predictions"], reference["predictions"]),
        "fed_tokens_equal": torch.equal(candidate["fed_tokens"], reference["fed_tokens"]),
    }
    gap = (torch.log_softmax(cand.float(), dim=-1) - torch.log_softmax(ref.float(), dim=-1)).abs()
    worst = float(gap.max())
    passed = (gate["passed"] and all(checks.values()) and bool(torch.isfinite(gap).all())
              and worst <= logprob_tolerance)
    return {"passed": passed, "logits": gate, **checks, "max_abs_logprob_error": worst,
            "logprob_tolerance": logprob_tolerance, "stepwise_normalized_rmse": stepwise_nrmse(cand, ref)}


def validate_routes(trace: dict, *, expected_linears: int, steps: int) -> bool:
    """Every packed Linear served the prompt once -- densely, or on the small-M
    packed route when the module opts into 2..8-row inputs and the prompt is that
    short -- and each decode step packed.  Counters at zero are ignored."""
    wanted = ({"dense_fallback": 1, "packed_m1": steps}, {"packed_small_m": 1, "packed_m1": steps})
    routes = trace["routes"]

    def used(route):
        return {key: count for key, count in route.items() if count}
    return len(routes) == expected_linears and all(used(route) in wanted for route in routes.values())
