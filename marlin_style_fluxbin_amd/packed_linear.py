"""Shared decode protocol of the packed Linear modules.

Both packed Linear types of the reference -- ``PackedW3Linear``
(``w3_lut_deployment.py:190-359``) and ``PackedHybridLinear``
(``deployment.py:182-297``) -- expose the same contract to their callers
(``StaticDecodeSession``, ``prepared_linears``, ``decode_trace``, the block
replacers):

* ``forward(x)``: a one-row fp16/bf16 GPU input takes the packed route; anything
  else raises ``ValueError`` unless ``fallback='dense'``, which runs ``F.linear``
  on the dequantized weight.  Both routes are counted in ``route_counts``
  (``packed_m1`` / ``dense_fallback``) and named in ``last_route``;
* ``bind_prepared_decode(dtype)``: an allocation-free ``[1, 1, K]`` route whose
  result is a view of one module-owned output buffer, validated once at bind
  time; ``clear_prepared_decode()`` drops it, and any ``.to()`` / ``.cuda()``
  move clears it (captured tensor references would dangle);
* ``_decode_audit``: while set, prepared calls are counted too.

Here that contract is written once.  A subclass supplies the payload-specific
parts: the dense weight, the packed kernel for a row count, and its own
bind-time checks.
"""
from __future__ import annotations

from typing import Callable

import torch
from torch import nn
from torch.nn import functional as F

HALF_DTYPES = (torch.float16, torch.bfloat16)
PACKED_M1, DENSE_FALLBACK, PACKED_SMALL_M = "packed_m1", "dense_fallback", "packed_small_m"

PackedKernel = Callable[[torch.Tensor, torch.Tensor], torch.Tensor]  # (x [rows, K], out [rows, O]) -> out


class PackedLinearBase(nn.Module):
    """Route selection, fallback policy, counters and the prepared binding."""

    max_packed_rows = 1
    # forward's bias add: in place into the output (its dtype kept: PackedW3Linear,
    # w3_lut_deployment.py:357-358) or out of place (type promotion: the hybrid
    # Linear, deployment.py:295-296); the bound decode route adds in place for both
    bias_in_place = True

    def _init_protocol(self, *, fallback: str, bias: torch.Tensor | None) -> None:
        if fallback not in ("error", "dense"):
            raise ValueError("fallback must be error or dense")
        self.fallback = fallback
        self.route_counts = {PACKED_M1: 0, DENSE_FALLBACK: 0}
        if self.max_packed_rows > 1:
            self.route_counts[PACKED_SMALL_M] = 0
        self.last_route = "not_called"
        self._decode_binding = None
        self._decode_audit = False
        self.register_buffer("bias", None if bias is None else bias.detach().clone())
        self.register_buffer("_decode_output", None, persistent=False)

    # ------------------------------------------------------------ subclass hooks
    def _payload_device(self) -> torch.device:
        raise NotImplementedError

    def _dense_weight(self, dtype: torch.dtype) -> torch.Tensor:
        """``[O, K]`` weight of the dense fallback in ``dtype``."""
        raise NotImplementedError

    def _packed_kernel(self, rows: int, device: torch.device) -> PackedKernel:
        """The packed-route callable for ``rows`` activation rows."""
        raise NotImplementedError

    def _check_before_call(self) -> None:
        """Checks every call repeats (e.g. buffers that a cast could have changed)."""

    def _check_before_bind(self, device: torch.device) -> None:
        """Bind-time payload checks beyond the device (contiguity, dtypes, ...)."""

    # ------------------------------------------------------------ protocol
    def clear_prepared_decode(self) -> None:
        self._decode_binding = None
        self._decode_output = None
        self._decode_audit = False

    def _apply(self, fn, recurse=True):
        self.clear_prepared_decode()
        self._forget_kernels()
        return super()._apply(fn, recurse=recurse)

    def _forget_kernels(self) -> None:
        """Drop cached kernel bindings that hold device pointers."""

    def _count(self, route: str) -> None:
        self.route_counts[route] = self.route_counts.get(route, 0) + 1
        self.last_route = route

    def reset_route_counts(self) -> None:
        """Zero every route counter this module keeps (``packed_small_m`` too,
        when the module opts into small-M inputs)."""
        self.route_counts = {key: 0 for key in self.route_counts}
        for key in (PACKED_M1, DENSE_FALLBACK):
            self.route_counts.setdefault(key, 0)

    def bind_prepared_decode(self, dtype: torch.dtype) -> None:
        if self._decode_binding is not None:
            raise ValueError("decode already bound")
        if dtype not in HALF_DTYPES:
            raise ValueError("FP16/BF16 required")
        device = self._payload_device()
        if device.type != "cuda":
            raise ValueError("prepared decode requires CUDA (a ROCm GPU)")
        self._check_before_bind(device)
        kernel = self._packed_kernel(1, device)
        output = torch.empty((1, self.out_features), device=device, dtype=dtype)
        self._decode_output = output
        view = output.view(1, 1, self.out_features)
        flat_in = (1, self.in_features)
        expected = (1, 1, self.in_features)
        bias = self.bias

        def prepared(x: torch.Tensor) -> torch.Tensor:
            if torch.is_grad_enabled():
                raise RuntimeError("prepared decode is inference only")
            if tuple(x.shape) != expected or x.dtype != dtype or x.device != device or not x.is_contiguous():
                raise ValueError("prepared decode input shape/dtype/device/stride mismatch")
            if self._decode_audit:
                self._count(PACKED_M1)
            kernel(x.view(flat_in), output)
            if bias is not None:
                output.add_(bias)
            return view

        self._decode_binding = prepared

    def _packed_rows(self, x: torch.Tensor) -> int:
        """Row count if ``x`` may take the packed route, else 0."""
        rows = x.numel() // self.in_features
        if x.is_cuda and x.dtype in HALF_DTYPES and 1 <= rows <= self.max_packed_rows:
            return rows
        return 0

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self._decode_binding is not None:
            return self._decode_binding(x)
        if torch.is_grad_enabled():
            raise RuntimeError("packed inference requires no_grad/inference_mode")
        if x.ndim < 2 or x.shape[-1] != self.in_features:
            raise ValueError("expected [...,K] input")
        self._check_before_call()
        rows = self._packed_rows(x)
        if rows == 0:
            if self.fallback != "dense":
                raise ValueError("unsupported input; enable explicit dense fallback if needed")
            self._count(DENSE_FALLBACK)
            return F.linear(x, self._dense_weight(x.dtype), self.bias)
        self._count(PACKED_M1 if rows == 1 else PACKED_SMALL_M)
        out = torch.empty((rows, self.out_features), device=x.device, dtype=x.dtype)
        self._packed_kernel(rows, x.device)(x.reshape(rows, self.in_features).contiguous(), out)
        if self.bias is not None:
            out = out.add_(self.bias) if self.bias_in_place else out + self.bias
        return out.reshape(*x.shape[:-1], self.out_features)


def replace_linears_atomically(block: nn.Module, built: list[tuple[str, nn.Module]]) -> list[str]:
    """Install already-built replacements; callers build (and so validate) every
    one of them before calling, so a bad payload never leaves a half-replaced block."""
    for name, module in built:
        parent, attribute = name.rsplit(".", 1)
        setattr(block.get_submodule(parent), attribute, module)
    return [name for name, _ in built]
