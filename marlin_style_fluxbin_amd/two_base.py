"""Rank-one two-base binary-basis GEMV with salient columns (batch 1) on gfx950.

The benchmark's config-4 weight format, the compact relative of the reference's
hybrid two-base deployment format (``deployment.py:18-121``; kernel
``csrc/m1_v5.cu:26-104``):

    W[o, k] = s_r[o] t_c[k] (a1[o] B1[o, k] + a2[o] B2[o, k]) + sum_j [k = idx[j]] sal[o, j]

with ``B1, B2`` in {-1, +1} stored as one bit each.  A layout is a dict of GPU
tensors:

* ``planes`` uint8 ``[K/128, O, 2, 16]``: bit ``k >> 4`` of byte ``k & 15`` of
  ``planes[g, o, b]`` is 1 where ``B_b[o, 128 g + k] = +1``;
* ``coef`` fp16 ``[2, O]`` (a1, a2), ``srow`` fp16 ``[O]``, ``tcol`` fp16 ``[K]``;
* ``salient`` bf16 ``[O, S]`` and ``salient_idx`` int32 ``[S]`` (S may be 0).

:func:`two_base_gemv` is the allocation-free entry (caller-owned output and
workspace, current stream, one launch unless K is split); :class:`TwoBaseGemv`
binds one layout and owns its workspace.  There is no CPU path: the HIP library
must be built.
"""
from __future__ import annotations

import torch

from . import _lib

GROUP = 128
_HALF = (torch.float16, torch.bfloat16)


def pack_rank_one_planes(bases: torch.Tensor) -> torch.Tensor:
    """Signs ``[2, O, K]`` in {-1, +1} -> ``planes`` uint8 ``[K/128, O, 2, 16]``
    (column ``128 g + k`` at bit ``k >> 4`` of byte ``k & 15``)."""
    if bases.ndim != 3 or bases.shape[0] != 2:
        raise ValueError("bases must have shape [2, out_features, in_features]")
    _, o, k = bases.shape
    if k % GROUP:
        raise ValueError("in_features must be a multiple of 128")
    if not torch.all((bases == -1) | (bases == 1)):
        raise ValueError("bases must contain only -1 and +1")
    bits = (bases > 0).to(torch.uint8).reshape(2, o, k // GROUP, 8, 16)
    shifts = torch.arange(8, device=bases.device, dtype=torch.uint8).view(1, 1, 1, 8, 1)
    planes = torch.bitwise_left_shift(bits, shifts).sum(dim=3, dtype=torch.uint8)  # distinct bits: sum == or
    return planes.permute(2, 1, 0, 3).contiguous()


def unpack_rank_one_planes(planes: torch.Tensor) -> torch.Tensor:
    """Inverse of :func:`pack_rank_one_planes` -> int8 signs ``[2, O, K]``."""
    if planes.ndim != 4 or planes.shape[2:] != (2, 16) or planes.dtype != torch.uint8:
        raise ValueError("planes must be uint8 [K/128, O, 2, 16]")
    g, o = planes.shape[:2]
    shifts = torch.arange(8, device=planes.device, dtype=torch.uint8).view(1, 1, 1, 8, 1)
    bits = torch.bitwise_and(torch.bitwise_right_shift(planes.unsqueeze(3), shifts), 1)
    return bits.permute(2, 1, 0, 3, 4).reshape(2, o, g * GROUP).to(torch.int8) * 2 - 1


def validate_rank_one(layout: dict) -> tuple[int, int, int]:
    """Shape / dtype contract of a rank-one layout; returns ``(O, K, S)``."""
    planes = layout["planes"]
    if planes.ndim != 4 or planes.shape[2:] != (2, 16) or planes.dtype != torch.uint8:
        raise ValueError("planes must be uint8 [K/128, O, 2, 16]")
    g, o = planes.shape[:2]
    k = g * GROUP
    for name, shape, dtype in (("coef", (2, o), torch.float16), ("srow", (o,), torch.float16),
                               ("tcol", (k,), torch.float16)):
        t = layout[name]
        if tuple(t.shape) != shape or t.dtype != dtype:
            raise ValueError(f"{name} must be {dtype} {list(shape)}")
    sal, idx = layout.get("salient"), layout.get("salient_idx")
    s = 0 if sal is None else sal.shape[-1]
    if s:
        if sal.dtype != torch.bfloat16 or tuple(sal.shape) != (o, s):
            raise ValueError("salient must be bf16 [O, S]")
        if idx is None or idx.dtype != torch.int32 or tuple(idx.shape) != (s,):
            raise ValueError("salient_idx must be int32 [S]")
    for t in layout.values():
        if t is not None and (t.device != planes.device or not t.is_contiguous()):
            raise ValueError("layout tensors must be contiguous and on one device")
    return o, k, s


def two_base_workspace_bytes(out_features: int, in_features: int) -> int:
    return int(_lib.library().fx_two_base_gemv_workspace_bytes(out_features, in_features))


def two_base_gemv(x: torch.Tensor, layout: dict, out: torch.Tensor, workspace: torch.Tensor | None = None, *,
                  tiling: tuple[int, int, int, int] | None = None) -> torch.Tensor:
    """``out[1, O] = x[1, K] @ W.T`` in the activation dtype, fp32 accumulation.

    ``tiling`` = (waves, prefetch, groups_per_split, tiles) selects an explicit
    kernel configuration (benchmark sweeps); the default picks one per shape."""
    o, k, s = validate_rank_one(layout)
    if x.dtype not in _HALF or not x.is_cuda or x.numel() != k or not x.is_contiguous():
        raise ValueError("x must be a contiguous GPU fp16/bf16 tensor with K elements")
    if out.dtype != x.dtype or out.numel() != o or not out.is_contiguous():
        raise ValueError("out must be a contiguous tensor of O elements in the activation dtype")
    lib = _lib.library()
    ws_ptr = None if workspace is None else workspace.data_ptr()
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    sal = layout.get("salient") if s else None
    idx = layout.get("salient_idx") if s else None
    args = (x.data_ptr(), _lib.dtype_code(x.dtype), layout["planes"].data_ptr(), layout["coef"].data_ptr(),
            layout["srow"].data_ptr(), layout["tcol"].data_ptr(), _lib.ptr(sal), _lib.ptr(idx), s,
            ws_ptr, ws_bytes, out.data_ptr(), o, k)
    if tiling is None:
        _lib.check(lib.fx_two_base_gemv(*args, _lib.stream_handle(x.device)), "fx_two_base_gemv")
    else:
        _lib.check(lib.fx_two_base_gemv_config(*args, *tiling, _lib.stream_handle(x.device)),
                   "fx_two_base_gemv_config")
    return out


class TwoBaseGemv:
    """Bound rank-one two-base GEMV: owns the workspace its K split needs."""

    def __init__(self, layout: dict, *, tiling: tuple[int, int, int, int] | None = None):
        self.out_features, self.in_features, self.salient = validate_rank_one(layout)
        device = layout["planes"].device
        if device.type != "cuda":
            raise ValueError("TwoBaseGemv requires a GPU layout")
        self.layout = layout
        self.tiling = tiling
        lib = _lib.library()
        if tiling is None:
            nbytes = lib.fx_two_base_gemv_workspace_bytes(self.out_features, self.in_features)
        else:
            nbytes = lib.fx_two_base_gemv_config_workspace_bytes(self.out_features, self.in_features, *tiling)
        self.workspace = torch.zeros(max(int(nbytes), 256), dtype=torch.uint8, device=device)

    def __call__(self, x: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
        return two_base_gemv(x, self.layout, out, self.workspace, tiling=self.tiling)


def rank_one_reference_weight(layout: dict, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Dense ``W[O, K]`` of a rank-one layout in fp32 (then ``dtype``): the
    dequantize of a dequantize-then-matmul check, on the layout's device."""
    o, k, s = validate_rank_one(layout)
    signs = unpack_rank_one_planes(layout["planes"]).float()
    coef = layout["coef"].float()
    w = layout["srow"].float()[:, None] * layout["tcol"].float()[None, :] * (
        coef[0][:, None] * signs[0] + coef[1][:, None] * signs[1])
    if s:
        w.index_add_(1, layout["salient_idx"].long(), layout["salient"].float())
    return w.to(dtype)
