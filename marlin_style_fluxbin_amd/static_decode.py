"""Prepared static-KV Qwen3 decode captured as one HIP graph.

Reference: ``static_decode.py`` (``prepared_linears`` :14-23,
``StaticDecodeSession`` :26-138).  Same protocol: prefill the real prefix into a
``transformers.StaticCache`` sized for prefix + continuation, snapshot the
prefix KV, then run a fixed continuation with static boolean masks and fixed
positions.  ``capture`` records every decode step (embedding, attention, LM head
and argmax included) into one graph -- on ROCm ``torch.cuda.CUDAGraph`` is a
hipGraph -- and ``measure`` times a replay.  Prefill and the prefix restore are
outside the timed region.
"""
from __future__ import annotations

import time
from contextlib import contextmanager

import torch

from .full_model_trial import packed_modules


def _loaded_hip_runtime():
    """The HIP runtime already mapped into this process (torch's), opened by its
    exact path so no second runtime gets loaded; None if none is mapped."""
    import ctypes

    try:
        with open("/proc/self/maps") as maps:
            paths = {line.split()[-1] for line in maps if "libamdhip64" in line}
    except OSError:
        return None
    paths = sorted(p for p in paths if p.startswith("/"))
    return ctypes.CDLL(paths[0]) if paths else None


def graph_kernel_count(graph) -> int | None:
    """Kernel nodes of a captured ``torch.cuda.CUDAGraph(keep_graph=True)`` (a
    hipGraph), from the HIP runtime; None if the runtime query is unavailable."""
    import ctypes

    try:
        raw = graph.raw_cuda_graph()
        hip = _loaded_hip_runtime()
    except (AttributeError, OSError, RuntimeError):
        return None
    if hip is None:
        return None
    count = ctypes.c_size_t(0)
    if hip.hipGraphGetNodes(ctypes.c_void_p(raw), None, ctypes.byref(count)) != 0:
        return None
    nodes = (ctypes.c_void_p * count.value)()
    if hip.hipGraphGetNodes(ctypes.c_void_p(raw), nodes, ctypes.byref(count)) != 0:
        return None
    kind = ctypes.c_int(0)
    kernels = 0
    for node in nodes:
        if hip.hipGraphNodeGetType(ctypes.c_void_p(node), ctypes.byref(kind)) == 0 and kind.value == 0:
            kernels += 1  # hipGraphNodeTypeKernel
    return kernels


@contextmanager
def prepared_linears(model, dtype):
    """Bind every packed Linear's allocation-free decode route for the duration."""
    modules = packed_modules(model)
    if any(m._decode_binding is not None for m in modules.values()):
        raise ValueError("prepared decode contexts cannot overlap")
    try:
        for m in modules.values():
            m.bind_prepared_decode(dtype)
        yield modules
    finally:
        for m in modules.values():
            m.clear_prepared_decode()


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
        self.tokens = forced_tokens.to(input_ids.device).contiguous()
        self.steps = self.tokens.shape[1]
        self.prefix_length = input_ids.shape[1]
        self.maximum_length = self.prefix_length + self.steps
        self.cache = StaticCache(config=model.config, max_cache_len=self.maximum_length)
        with torch.inference_mode():
            out = model(input_ids=input_ids, past_key_values=self.cache, use_cache=True, logits_to_keep=1)
            self.prefill_logits = out.logits[:, -1, :].detach().clone()
            self.prefix = [(layer.keys[:, :, :self.prefix_length].clone(),
                            layer.values[:, :, :self.prefix_length].clone()) for layer in self.cache.layers]
        self.positions = torch.arange(self.prefix_length, self.maximum_length,
                                      device=input_ids.device).view(1, -1)
        # boolean SDPA masks (True = attend), one per step, built once: no step
        # reads a device sequence length back to the host
        columns = torch.arange(self.maximum_length, device=input_ids.device)
        self.masks = [(columns <= p).view(1, 1, 1, -1) for p in range(self.prefix_length, self.maximum_length)]
        self.graph = None
        self.graph_outputs = None
        self.capture_routes = None
        self.kernel_nodes = None

    @torch.inference_mode()
    def reset(self):
        """Restore the prefix KV and the cache length (future slots zeroed)."""
        for layer, (k, v) in zip(self.cache.layers, self.prefix):
            layer.keys.zero_()
            layer.values.zero_()
            layer.keys[:, :, :self.prefix_length].copy_(k)
            layer.values[:, :, :self.prefix_length].copy_(v)
            layer.cumulative_length.fill_(self.prefix_length)

    @torch.inference_mode()
    def run(self):
        outputs = []
        for i in range(self.steps):
            out = self.model(input_ids=self.tokens[:, i:i + 1], past_key_values=self.cache,
                             position_ids=self.positions[:, i:i + 1],
                             attention_mask={"full_attention": self.masks[i]}, use_cache=True, logits_to_keep=1)
            logits = out.logits[:, -1, :]
            outputs.append((logits, logits.argmax(-1, keepdim=True)))
        return outputs

    def set_audit(self, enabled: bool):
        for m in packed_modules(self.model).values():
            m._decode_audit = enabled
            m.route_counts = {"dense_fallback": 0, "packed_m1": 0}

    def routes(self) -> dict:
        return {n: dict(m.route_counts) for n, m in packed_modules(self.model).items()}

    def trace(self, outputs) -> dict:
        length = int(self.cache.get_seq_length())
        if length != self.maximum_length:
            raise RuntimeError("static KV length mismatch")
        logits = torch.stack([self.prefill_logits] + [p[0] for p in outputs], dim=1).detach().cpu()
        predictions = torch.cat([self.prefill_logits.argmax(-1, keepdim=True)] + [p[1] for p in outputs], dim=1).cpu()
        if not bool(torch.isfinite(logits).all()):
            raise RuntimeError("nonfinite static decode logits")
        return {"logits": logits, "predictions": predictions, "fed_tokens": self.tokens.cpu(),
                "cache_length": length, "routes": self.routes()}

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
        """Capture all decode steps into one graph (after two warm-up runs on the
        capture stream), replay it once from the restored prefix, return its trace."""
        if self.ids.device.type != "cuda":
            raise RuntimeError("graph capture requires a GPU")
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            for _ in range(2):
                self.reset()
                self.run()
        torch.cuda.current_stream().wait_stream(stream)
        self.reset()
        torch.cuda.synchronize()
        self.set_audit(True)
        graph = torch.cuda.CUDAGraph(keep_graph=True)
        try:
            with torch.cuda.graph(graph, stream=stream):
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
        """Time one pass of all decode steps: ``prepared_eager`` or ``sequence_graph``."""
        if mode not in ("prepared_eager", "sequence_graph"):
            raise ValueError("unknown mode")
        if mode == "sequence_graph" and self.graph is None:
            raise ValueError("capture first")
        self.reset()
        cuda = self.ids.device.type == "cuda"
        if cuda:
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
        wall = time.perf_counter()
        if cuda:
            start.record()
        if mode == "sequence_graph":
            self.graph.replay()
            outputs = self.graph_outputs
        else:
            outputs = self.run()
        if cuda:
            end.record()
            end.synchronize()
        wall_ms = (time.perf_counter() - wall) * 1000
        trace = self.trace(outputs)  # checks stay outside the timed region
        return {"wall_ms": wall_ms, "device_ms": start.elapsed_time(end) if cuda else None}, trace
