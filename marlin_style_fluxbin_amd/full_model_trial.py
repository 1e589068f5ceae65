"""Dynamic-KV decode trace and trace comparison for HF Qwen3 models with packed Linears.

Reference: ``full_model_trial.py`` (``packed_modules`` :10-12, ``decode_trace``
:15-78, ``compare_trace`` :81-93, ``validate_routes`` :96-99).  The trace is the
oracle side of a decode comparison: prefill through the dense fallback, then
``steps`` single-token calls on one growing dynamic cache with the packed route
enforced.
"""
from __future__ import annotations

import time

import torch

from .acceleration_checks import numerical_gate, stepwise_nrmse
from .w3_lut_deployment import PackedW3Linear


def packed_modules(model) -> dict:
    return {name: m for name, m in model.named_modules() if isinstance(m, PackedW3Linear)}


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
    forced = None if forced_tokens is None else forced_tokens.to(input_ids.device)
    modules = packed_modules(model)
    saved = {n: m.fallback for n, m in modules.items()}
    for m in modules.values():
        m.route_counts = {"packed_m1": 0, "dense_fallback": 0}
        m.fallback = "dense"
    cuda = input_ids.is_cuda

    def sync():
        if cuda:
            torch.cuda.synchronize(input_ids.device)

    def event():
        return torch.cuda.Event(enable_timing=True) if cuda else None

    logits, predictions, fed, step_events = [], [], [], []
    try:
        sync()
        wall = time.perf_counter()
        pre_start, pre_end = event(), event()
        if cuda:
            pre_start.record()
        output = model(input_ids=input_ids, use_cache=True, logits_to_keep=1)
        cache = output.past_key_values
        logits.append(output.logits[:, -1, :].detach())
        current = logits[-1].argmax(-1, keepdim=True)
        predictions.append(current)
        if cuda:
            pre_end.record()
        sync()
        prefill_wall = (time.perf_counter() - wall) * 1000
        for m in modules.values():
            m.fallback = "error"  # decode steps must take the packed route
        dec_start, dec_end = event(), event()
        wall = time.perf_counter()
        if cuda:
            dec_start.record()
        for i in range(steps):
            token = current if forced is None else forced[:, i:i + 1]
            fed.append(token)
            begin, end = event(), event()
            if cuda:
                begin.record()
            output = model(input_ids=token, past_key_values=cache, use_cache=True, logits_to_keep=1)
            cache = output.past_key_values
            logits.append(output.logits[:, -1, :].detach())
            current = logits[-1].argmax(-1, keepdim=True)
            predictions.append(current)
            if cuda:
                end.record()
                step_events.append((begin, end))
        if cuda:
            dec_end.record()
        sync()
        decode_wall = (time.perf_counter() - wall) * 1000
        length = cache.get_seq_length()
        length = int(length.item()) if isinstance(length, torch.Tensor) else int(length)
        if length != input_ids.shape[1] + steps:
            raise RuntimeError("KV cache length drift")
        return {
            "logits": torch.stack(logits, dim=1).cpu(),
            "predictions": torch.cat(predictions, dim=1).cpu(),
            "fed_tokens": torch.cat(fed, dim=1).cpu(),
            "cache_length": length,
            "prefill_wall_ms": prefill_wall,
            "decode_wall_ms": decode_wall,
            "prefill_device_ms": pre_start.elapsed_time(pre_end) if cuda else None,
            "decode_device_ms": dec_start.elapsed_time(dec_end) if cuda else None,
            "step_device_ms": [a.elapsed_time(b) for a, b in step_events],
            "routes": {n: dict(m.route_counts) for n, m in modules.items()},
        }
    finally:
        for n, m in modules.items():
            m.fallback = saved[n]


def compare_trace(candidate: dict, reference: dict, *, logprob_tolerance: float) -> dict:
    """Pass iff the logits gate passes, greedy tokens and fed contexts are equal,
    and the max |log-softmax difference| is within ``logprob_tolerance``."""
    if logprob_tolerance < 0:
        raise ValueError("negative logprob tolerance")
    gate = numerical_gate(candidate["logits"], reference["logits"])
    if candidate["logits"].shape != reference["logits"].shape:
        return {"passed": False, "reason": "shape drift"}
    tokens_equal = torch.equal(candidate["predictions"], reference["predictions"])
    contexts_equal = torch.equal(candidate["fed_tokens"], reference["fed_tokens"])
    delta = (candidate["logits"].float().log_softmax(-1) - reference["logits"].float().log_softmax(-1)).abs()
    maximum = float(delta.max())
    finite = bool(torch.isfinite(delta).all())
    return {"passed": gate["passed"] and tokens_equal and contexts_equal and finite and maximum <= logprob_tolerance,
            "logits": gate, "greedy_tokens_equal": tokens_equal, "fed_tokens_equal": contexts_equal,
            "max_abs_logprob_error": maximum, "logprob_tolerance": logprob_tolerance,
            "stepwise_normalized_rmse": stepwise_nrmse(candidate["logits"], reference["logits"])}


def validate_routes(trace: dict, *, expected_linears: int, steps: int) -> bool:
    """Every packed Linear served the prefill densely once and each decode step packed."""
    return len(trace["routes"]) == expected_linears and all(
        r == {"dense_fallback": 1, "packed_m1": steps} for r in trace["routes"].values())
