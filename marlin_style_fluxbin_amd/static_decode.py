"""Prepared static-KV Qwen3 decode, captured as one HIP graph.

Contract of the reference's ``static_decode.py`` (``prepared_linears`` :14-23,
``StaticDecodeSession`` :26-138): the constructor checks and messages, the
``reset`` / ``run`` / ``trace`` / ``audit`` / ``capture`` / ``measure`` methods,
the trace keys (``logits``, ``predictions``, ``fed_tokens``, ``cache_length``,
``routes``) and the timing keys (``wall_ms``, ``device_ms``).  The protocol:
prefill the real prefix into a ``transformers.StaticCache`` sized for prefix +
continuation, keep a copy of the prefix KV, then run a fixed continuation with
static boolean masks and fixed positions; ``capture`` records every decode step
(embedding, attention, LM head and argmax included) into one graph (on ROCm a
``torch.cuda.CUDAGraph`` is a hipGraph) and ``measure`` times one pass.  Prefill
and the prefix restore stay outside the timed region.

Organisation here: ``_PrefixKV`` owns the cache snapshot and its restore (only
the continuation slots are cleared: the prefix is overwritten anyway, and the
masks already hide every later slot); ``_StepInputs`` holds every step's token,
position and mask as slices of three tensors built once; the session drives
them and records the graph.
"""
from __future__ import annotations

import ctypes
import time
from contextlib import contextmanager

import torch

from .full_model_trial import packed_modules


def _loaded_hip_runtime():
    """The HIP runtime already mapped into this process (torch's), opened by its
    exact path so no second runtime gets loaded; None if none is mapped."""
    try:
        with open("/proc/self/maps") as maps:
            paths = sorted({line.split()[-1] for line in maps if "libamdhip64" in line})
    except OSError:
        return None
    paths = [p for p in paths if p.startswith("/")]
    return ctypes.CDLL(paths[0]) if paths else None


_HIP_GRAPH_NODE_KERNEL = 0  # hipGraphNodeTypeKernel


def graph_kernel_count(graph) -> int | None:
    """Kernel nodes of a captured ``torch.cuda.CUDAGraph(keep_graph=True)`` (a
    hipGraph), from the HIP runtime; None if the runtime query is unavailable."""
    try:
        raw = ctypes.c_void_p(graph.raw_cuda_graph())
        hip = _loaded_hip_runtime()
    except (AttributeError, OSError, RuntimeError):
        return None
    if hip is None:
        return None
    count = ctypes.c_size_t(0)
    if hip.hipGraphGetNodes(raw, None, ctypes.byref(count)) != 0:
        return None
    nodes = (ctypes.c_void_p * count.value)()
    if hip.hipGraphGetNodes(raw, nodes, ctypes.byref(count)) != 0:
        return None
    kind = ctypes.c_int(-1)
    kernels = 0
    for node in nodes:
        ok = hip.hipGraphNodeGetType(ctypes.c_void_p(node), ctypes.byref(kind)) == 0
        kernels += int(ok and kind.value == _HIP_GRAPH_NODE_KERNEL)
    return kernels


@contextmanager
def prepared_linears(model, dtype):
    """Bind every packed Linear's allocation-free decode route for the duration;
    every binding is cleared on exit, also after a failure part-way through."""
    modules = packed_modules(model)
    if any(m._decode_binding is not None for m in modules.values()):
        raise ValueError("prepared decode contexts cannot overlap")
    try:
        for module in modules.values():
            module.bind_prepared_decode(dtype)
        yield modules
    finally:
        for module in modules.values():
            module.clear_prepared_decode()


class _PrefixKV:
    """The static cache's prefix keys / values, kept so every pass starts alike."""

    def __init__(self, cache, prefix_length: int):
        self.cache = cache
        self.length = prefix_length
        self.saved = [(layer.keys[:, :, :prefix_length].clone(), layer.values[:, :, :prefix_length].clone())
                      for layer in cache.layers]

    def restore(self) -> None:
        n = self.length
        for layer, (keys, values) in zip(self.cache.layers, self.saved):
            layer.keys[:, :, :n].copy_(keys)
            layer.values[:, :, :n].copy_(values)
            layer.keys[:, :, n:].zero_()
            layer.values[:, :, n:].zero_()
            layer.cumulative_length.fill_(n)


class _StepInputs:
    """Token, position and boolean SDPA mask (True = attend) of every step, as
    views of three tensors built once, so no step reads a device length back."""

    def __init__(self, tokens: torch.Tensor, prefix_length: int):
        device = tokens.device
        self.tokens = tokens
        total = prefix_length + tokens.shape[1]
        self.positions = torch.arange(prefix_length, total, device=device).view(1, -1)
        columns = torch.arange(total, device=device)
        self.masks = (columns.view(1, -1) <= self.positions.view(-1, 1)).view(-1, 1, 1, 1, total)

    def __len__(self) -> int:
        return self.tokens.shape[1]

    def step(self, i: int) -> dict:
        return {"input_ids": self.tokens[:, i:i + 1], "position_ids": self.positions[:, i:i + 1],
                "attention_mask": {"full_attention": self.masks[i]}}


class StaticDecodeSession:
    def __init__(self, model, input_ids: torch.Tensor, forced_tokens: torch.Tensor):
        from transformers import StaticCache

        if input_ids.ndim != 2 or input_ids.shape[0] != 1 or input_ids.shape[1] < 2:
            raise ValueError("batch1 nonempty real prefix required")
        if forced_tokens.ndim != 2 or forced_tokens.shape[0] != 1 or forced_tokens.shape[1] < 1:
            raise ValueError("batch1 continuation required")
        if model.training:
            raise ValueError("eval model required")
        if any(m._decode_binding is not None for m in packed_modules(model).values()):
            raise ValueError("prepare real prefix before binding decode-only linears")
        if set(model.config.layer_types) != {"full_attention"}:
            raise ValueError("this protocol supports full-attention Qwen3 only")
        self.model = model
        self.ids = input_ids
        self.prefix_length = input_ids.shape[1]
        self.inputs = _StepInputs(forced_tokens.to(input_ids.device).contiguous(), self.prefix_length)
        self.tokens = self.inputs.tokens
        self.steps = len(self.inputs)
        self.maximum_length = self.prefix_length + self.steps
        self.cache = StaticCache(config=model.config, max_cache_len=self.maximum_length)
        with torch.inference_mode():
            prefill = model(input_ids=input_ids, past_key_values=self.cache, use_cache=True, logits_to_keep=1)
            self.prefill_logits = prefill.logits[:, -1, :].detach().clone()
        self.prefix = _PrefixKV(self.cache, self.prefix_length)
        self.positions = self.inputs.positions
        self.masks = self.inputs.masks
        self.graph = None
        self.graph_outputs = None
        self.capture_routes = None
        self.kernel_nodes = None

    @torch.inference_mode()
    def reset(self):
        """Restore the prefix KV and the cache length (continuation slots zeroed)."""
        self.prefix.restore()

    @torch.inference_mode()
    def run(self):
        """Every decode step once; a list of (logits [1, V], greedy token [1, 1])."""
        outputs = []
        for i in range(self.steps):
            logits = self.model(past_key_values=self.cache, use_cache=True, logits_to_keep=1,
                                **self.inputs.step(i)).logits[:, -1, :]
            outputs.append((logits, logits.argmax(-1, keepdim=True)))
        return outputs

    def set_audit(self, enabled: bool):
        for module in packed_modules(self.model).values():
            module._decode_audit = enabled
            module.reset_route_counts()

    def routes(self) -> dict:
        return {name: dict(module.route_counts) for name, module in packed_modules(self.model).items()}

    def trace(self, outputs) -> dict:
        length = int(self.cache.get_seq_length())
        if length != self.maximum_length:
            raise RuntimeError("static KV length mismatch")
        step_logits = [self.prefill_logits] + [logits for logits, _ in outputs]
        step_tokens = [self.prefill_logits.argmax(-1, keepdim=True)] + [token for _, token in outputs]
        logits = torch.stack(step_logits, dim=1).detach().cpu()
        if not bool(torch.isfinite(logits).all()):
            raise RuntimeError("nonfinite static decode logits")
        return {"logits": logits, "predictions": torch.cat(step_tokens, dim=1).cpu(),
                "fed_tokens": self.tokens.cpu(), "cache_length": length, "routes": self.routes()}

    @torch.inference_mode()
    def audit(self) -> dict:
        self.reset()
        self.set_audit(True)
        try:
            return self.trace(self.run())
        finally:
            self.set_audit(False)

    @torch.inference_mode()
    def capture(self) -> dict:
        """Record all decode steps into one graph (after two warm-up passes on the
        capture stream), replay it once from the restored prefix, return its trace."""
        if self.ids.device.type != "cuda":
            raise RuntimeError("graph capture requires a CUDA (ROCm HIP) device")
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                self.reset()
                self.run()
        torch.cuda.current_stream().wait_stream(side)
        self.reset()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph(keep_graph=True)
        self.set_audit(True)
        try:
            with torch.cuda.graph(graph, stream=side):
                outputs = self.run()
            self.capture_routes = self.routes()
        finally:
            self.set_audit(False)
        self.kernel_nodes = graph_kernel_count(graph)
        graph.instantiate()
        self.graph, self.graph_outputs = graph, outputs
        self.reset()
        graph.replay()
        torch.cuda.synchronize()
        return self.trace(outputs)

    @torch.inference_mode()
    def measure(self, mode: str):
        """Time one pass of all decode steps (``prepared_eager`` or
        ``sequence_graph``); returns (timing, trace), the checks after the timer."""
        if mode not in ("prepared_eager", "sequence_graph"):
            raise ValueError("unknown mode")
        if mode == "sequence_graph" and self.graph is None:
            raise ValueError("capture first")
        self.reset()
        gpu = self.ids.device.type == "cuda"
        events = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) if gpu else None
        if gpu:
            torch.cuda.synchronize()
        t0 = time.perf_counter()
        if gpu:
            events[0].record()
        if mode == "sequence_graph":
            self.graph.replay()
            outputs = self.graph_outputs
        else:
            outputs = self.run()
        if gpu:
            events[1].record()
            events[1].synchronize()
        timing = {"wall_ms": (time.perf_counter() - t0) * 1e3,
                  "device_ms": events[0].elapsed_time(events[1]) if gpu else None}
        return timing, self.trace(outputs)
