"""Hybrid g128/s8 two-base format: payload contract, deployment layout, batch-1 op.

Drop-in for the reference's ``deployment.py`` (maxiu188-afk/Marlin_Style_Fluxbin
``src/fluxbin_style/deployment.py``): the same names, field sets, format strings,
layout shapes, workspace shapes and error types (``FIELDS`` :23-25,
``validate_artifact`` :30-55, ``convert_artifact`` / ``restore_artifact``
:84-115, ``decode_layout`` :118-121, ``workspace_shape`` :158-165, ``m1_out``
:168-179, ``PackedHybridLinear`` :182-297, ``replace_block_linears`` :300-320).

How it is built here:

* The payload contract is a table (``_ARTIFACT_SPEC``: shape as a function of
  ``(O, G)``, dtype rule) checked in one loop.
* The deployment layout is a table too (``_LAYOUT_MAP``): each layout field names
  its payload field and a pair of shape maps (payload -> group-major layout and
  back), so conversion and restoration are one generic walk each and cannot
  drift apart.  The planar form splits each interleaved 2-bit row into two
  1-bit planes (``_to_planes`` / ``_from_planes``).
* The GPU op is one gfx950 kernel (``fx_hybrid_gemv``: sign bits as int8
  matrix-core operands, fp32 per-group scales) reading the planar layout of the
  ``v5_p*`` kernels; interleaved layouts (``v1`` .. ``v5``) are converted to
  planes per call by ``m1_out`` (allocating) and once at construction by
  ``PackedHybridLinear``.  Every kernel name shares the factored fp32
  arithmetic of ``v4`` / ``v5``.
* ``PackedHybridLinear`` is ``packed_linear.PackedLinearBase`` (the route,
  fallback and prepared-binding protocol shared with ``PackedW3Linear``) over
  this payload.

There is no CPU substitute for the packed route: without the HIP library it raises.
"""
from __future__ import annotations

from typing import Callable, Mapping

import torch
from torch import nn

from . import _lib
from .evaluation import materialize_hybrid_s8_weight, tensor_sha256
from .packed_linear import PackedLinearBase, replace_linears_atomically

FORMAT = "fluxbin-hybrid-g128-s8-m1-v1"
PLANAR_FORMAT = "fluxbin-hybrid-g128-s8-m1-planar-v1"
PLANAR_KERNELS = ("v5_p256", "v5_p512", "v5_p1024")
FACTORED_KERNELS = ("v4", "v4_late", "v5") + PLANAR_KERNELS
KERNELS = ("v1", "v2_r1", "v2_r2", "v2", "v3") + FACTORED_KERNELS
FIELDS = ("global_sign_codes", "global_row_scales", "global_column_scales",
          "refinement_indices", "refinement_sign_codes",
          "refinement_row_scales", "refinement_column_scales")
LAYOUT_FIELDS = ("codes", "rows", "columns", "indices", "sparse_codes",
                 "sparse_rows", "sparse_columns", "lookup")
GROUP, REFINED = 128, 8
_INDEX_DTYPES = (torch.int16, torch.int32, torch.int64)

# payload field -> (shape from (O, G), dtype rule)
_ARTIFACT_SPEC: dict[str, tuple[Callable[[int, int], tuple], str]] = {
    "global_sign_codes": (lambda o, g: (o, 32 * g), "codes"),
    "global_row_scales": (lambda o, g: (2, o, g), "scales"),
    "global_column_scales": (lambda o, g: (2, g, GROUP), "scales"),
    "refinement_indices": (lambda o, g: (g, REFINED), "indices"),
    "refinement_sign_codes": (lambda o, g: (o, 2 * g), "codes"),
    "refinement_row_scales": (lambda o, g: (2, o, g), "scales"),
    "refinement_column_scales": (lambda o, g: (2, g, REFINED), "scales"),
}


def validate_artifact(p: Mapping[str, torch.Tensor]) -> tuple[int, int]:
    """Shape / dtype / device contract of the seven payload fields; ``(O, G)``."""
    if set(p) != set(FIELDS):
        raise ValueError("expected exactly seven hybrid payload fields")
    codes = p["global_sign_codes"]
    if codes.ndim != 2 or codes.dtype != torch.uint8:
        raise ValueError("global codes must be uint8 [O,K/4]")
    o, width = codes.shape
    if not (1 <= o <= 65536) or not (32 <= width <= 32768) or width % 32:
        raise ValueError("requires O=1..65536 and K=128..131072 divisible by 128")
    g = width // 32
    for name, (shape_of, rule) in _ARTIFACT_SPEC.items():
        t = p[name]
        if tuple(t.shape) != shape_of(o, g) or t.device != codes.device:
            raise ValueError(f"shape/device mismatch: {name}")
        if rule == "scales" and (t.dtype != torch.float32 or not bool(torch.isfinite(t).all())):
            raise ValueError(f"finite FP32 scales required: {name}")
        if rule == "codes" and t.dtype != torch.uint8:
            raise ValueError("refinement codes must be uint8")
        if rule == "indices":
            if t.dtype not in _INDEX_DTYPES:
                raise ValueError("integer refinement indices required")
            if bool((t < 0).any()) or bool((t >= GROUP).any()) or bool((t[:, 1:] <= t[:, :-1]).any()):
                raise ValueError("indices must be sorted, unique and inside each group")
    return o, g


# ------------------------------------------------------------------ bit planes
def _to_planes(codes: torch.Tensor) -> torch.Tensor:
    """Interleaved bytes ``[..., 2n]`` -> ``[..., 2, n]``: planar byte ``c`` of base
    ``b`` holds columns ``8c .. 8c+7``, which sit at bits ``2(j % 4) + b`` of
    interleaved byte ``2c + j // 4``."""
    lo, hi = codes[..., 0::2].to(torch.int32), codes[..., 1::2].to(torch.int32)
    planes = []
    for b in range(2):
        acc = torch.zeros_like(lo)
        for j in range(4):
            acc |= ((lo >> (2 * j + b)) & 1) << j
            acc |= ((hi >> (2 * j + b)) & 1) << (j + 4)
        planes.append(acc.to(torch.uint8))
    return torch.stack(planes, dim=-2)


def _from_planes(planes: torch.Tensor) -> torch.Tensor:
    """Inverse of :func:`_to_planes`."""
    p0, p1 = planes[..., 0, :].to(torch.int32), planes[..., 1, :].to(torch.int32)
    lo = torch.zeros_like(p0)
    hi = torch.zeros_like(p0)
    for j in range(4):
        lo |= (((p0 >> j) & 1) << (2 * j)) | (((p1 >> j) & 1) << (2 * j + 1))
        hi |= (((p0 >> (j + 4)) & 1) << (2 * j)) | (((p1 >> (j + 4)) & 1) << (2 * j + 1))
    return torch.stack((lo, hi), dim=-1).flatten(-2).to(torch.uint8)


# ------------------------------------------------------------------ layout map
def _group_major(width: int):
    """``[O, G * width]`` <-> ``[G, O, width]`` (row-major groups first)."""
    def forward(t: torch.Tensor) -> torch.Tensor:
        return t.reshape(t.shape[0], -1, width).permute(1, 0, 2)

    def backward(t: torch.Tensor) -> torch.Tensor:
        return t.permute(1, 0, 2).reshape(t.shape[1], -1)
    return forward, backward


def _swap(forward_order: tuple[int, ...]):
    backward_order = tuple(forward_order.index(i) for i in range(len(forward_order)))
    return (lambda t: t.permute(*forward_order)), (lambda t: t.permute(*backward_order))


_IDENTITY = (lambda t: t, lambda t: t)

# layout field -> (payload field, (payload -> layout, layout -> payload))
_LAYOUT_MAP = {
    "codes": ("global_sign_codes", _group_major(32)),
    "rows": ("global_row_scales", _swap((2, 1, 0))),
    "columns": ("global_column_scales", _swap((1, 2, 0))),
    "indices": ("refinement_indices", _IDENTITY),
    "sparse_codes": ("refinement_sign_codes", _group_major(2)),
    "sparse_rows": ("refinement_row_scales", _swap((2, 1, 0))),
    "sparse_columns": ("refinement_column_scales", _swap((1, 2, 0))),
}
_PLANAR_FIELDS = ("codes", "sparse_codes")


def layout_format(layout) -> str:
    return PLANAR_FORMAT if layout["codes"].ndim == 4 else FORMAT


def _lookup_table(indices: torch.Tensor) -> torch.Tensor:
    """``[G, 128]`` int16: the refinement slot of each column of a group, -1 elsewhere."""
    g = indices.shape[0]
    table = torch.full((g, GROUP), -1, dtype=torch.int16, device=indices.device)
    slots = torch.arange(REFINED, dtype=torch.int16, device=indices.device).expand(g, REFINED)
    return table.scatter_(1, indices.long(), slots)


def convert_artifact(p: Mapping[str, torch.Tensor], *, kernel: str = "v1") -> dict[str, torch.Tensor]:
    """Payload -> group-major deployment layout: a lossless permutation of the bytes
    plus the column ``lookup``, with storage of its own (later changes to ``p`` do
    not reach it)."""
    if kernel not in KERNELS:
        raise ValueError("unknown kernel")
    validate_artifact(p)
    layout = {}
    for name, (source, (to_layout, _)) in _LAYOUT_MAP.items():
        value = p[source].to(torch.int16) if name == "indices" else p[source]
        layout[name] = to_layout(value).contiguous().clone()
    layout["lookup"] = _lookup_table(layout["indices"])
    if kernel in PLANAR_KERNELS:
        for name in _PLANAR_FIELDS:
            layout[name] = _to_planes(layout[name]).contiguous()
    return layout


def restore_artifact(layout: Mapping[str, torch.Tensor]) -> dict[str, torch.Tensor]:
    """Inverse of :func:`convert_artifact` (the ``lookup`` is derived, not restored)."""
    planar = layout["codes"].ndim == 4
    payload = {}
    for name, (source, (_, to_payload)) in _LAYOUT_MAP.items():
        value = layout[name]
        if planar and name in _PLANAR_FIELDS:
            value = _from_planes(value)
        payload[source] = to_payload(value).contiguous()
    return payload


def decode_layout(p: Mapping[str, torch.Tensor], dtype=torch.bfloat16) -> torch.Tensor:
    """Dense weight ``[O, K]`` of a layout (the dequantize of the dense fallback)."""
    return materialize_hybrid_s8_weight(**restore_artifact(p), group_size=GROUP, columns_per_group=REFINED,
                                        device=p["codes"].device, output_dtype=dtype)


def conversion_record(source, layout) -> dict:
    return {"format": layout_format(layout),
            "source": {k: tensor_sha256(v) for k, v in source.items()},
            "layout": {k: tensor_sha256(v) for k, v in layout.items()},
            "layout_bytes": sum(v.numel() * v.element_size() for v in layout.values())}


def workspace_shape(out_features: int, in_features: int, groups_per_split=8, *, kernel="v1"):
    """fp32 workspace shape of ``m1_out``: ``[splits, O]`` with ``splits =
    ceil(G / groups_per_split)`` (``v4``/``v4_late``: the reference's flat shape).
    The gfx950 kernel uses no more K splits than this workspace holds."""
    if kernel not in KERNELS:
        raise ValueError("unknown kernel")
    valid = (isinstance(groups_per_split, int) and 1 <= groups_per_split <= 1024
             and 1 <= out_features <= 65536 and 128 <= in_features <= 131072 and in_features % 128 == 0)
    if not valid:
        raise ValueError("invalid group/split dimensions")
    groups = in_features // GROUP
    splits = -(-groups // groups_per_split)
    if kernel in ("v4", "v4_late"):
        return (groups * 272 + splits * out_features,)
    return (splits, out_features)


# ------------------------------------------------------------------ the op
def _check_m1_args(x, out, workspace, o, k):
    if not x.is_cuda or x.dtype not in (torch.float16, torch.bfloat16) or tuple(x.shape) != (1, k) \
            or not x.is_contiguous():
        raise RuntimeError("x must be a contiguous CUDA fp16/bf16 tensor [1, K]")
    if out.dtype != x.dtype or tuple(out.shape) != (1, o) or not out.is_contiguous() or out.device != x.device:
        raise RuntimeError("out must be a contiguous [1, O] tensor in the activation dtype")
    if workspace.dtype != torch.float32 or not workspace.is_contiguous() or workspace.device != x.device:
        raise RuntimeError("workspace must be a contiguous fp32 tensor on the activation device")


class HybridExtension:
    """Object returned by :func:`load_extension`: ``m1_out`` with the reference's
    positional arguments (its ``csrc/m1_v5.cu`` binding), on the C ABI."""

    def __init__(self, kernel: str):
        self.kernel = kernel
        self.lib = _lib.library()

    @staticmethod
    def _sorted_columns(indices_or_lookup: torch.Tensor) -> torch.Tensor:
        """int16 ``[G, 8]`` refinement columns from either indices or a lookup table."""
        if indices_or_lookup.shape[-1] == REFINED:
            return indices_or_lookup.to(torch.int16).contiguous()
        present = indices_or_lookup.to(torch.int32) >= 0
        return torch.argsort(~present, dim=1, stable=True)[:, :REFINED].to(torch.int16).contiguous()

    def m1_out(self, x, codes, rows, columns, sparse_codes, sparse_rows, sparse_columns, indices_or_lookup,
               out, workspace, groups_per_split):
        if codes.ndim != 4:
            codes, sparse_codes = _to_planes(codes).contiguous(), _to_planes(sparse_codes).contiguous()
        indices = self._sorted_columns(indices_or_lookup)
        o, k = codes.shape[1], codes.shape[0] * GROUP
        _check_m1_args(x, out, workspace, o, k)
        _lib.check(self.lib.fx_hybrid_gemv(
            x.data_ptr(), _lib.dtype_code(x.dtype), codes.data_ptr(), rows.data_ptr(), columns.data_ptr(),
            indices.data_ptr(), sparse_codes.data_ptr(), sparse_rows.data_ptr(), sparse_columns.data_ptr(),
            workspace.data_ptr(), workspace.numel() * workspace.element_size(), out.data_ptr(), o, k,
            _lib.stream_handle(x.device)), "fx_hybrid_gemv")
        return out


_EXTENSIONS: dict[str, HybridExtension] = {}


def load_extension(kernel: str = "v1") -> HybridExtension:
    if kernel not in KERNELS:
        raise ValueError(f"kernel must be one of {KERNELS}")
    if not torch.cuda.is_available():
        raise RuntimeError("the two-base M=1 kernel needs a ROCm GPU; there is no CPU substitute")
    return _EXTENSIONS.setdefault(kernel, HybridExtension(kernel))


def m1_out(x, layout, out, workspace, *, groups_per_split=8, kernel="v1"):
    """Engine-neutral batch-1 op: ``out = x @ W.T`` for a hybrid layout, fp32
    accumulation, current stream, caller-owned ``out`` and ``workspace``
    (:func:`workspace_shape`); no allocation for planar layouts.  Workspaces must
    not be shared by overlapping calls on different streams."""
    columns = layout["indices"] if kernel in FACTORED_KERNELS else layout["lookup"]
    return load_extension(kernel).m1_out(x, layout["codes"], layout["rows"], layout["columns"],
                                         layout["sparse_codes"], layout["sparse_rows"], layout["sparse_columns"],
                                         columns, out, workspace, groups_per_split)


# ------------------------------------------------------------------ the module
_SCALE_BUFFERS = ("rows", "columns", "sparse_rows", "sparse_columns")


class PackedHybridLinear(PackedLinearBase):
    """Hybrid two-base Linear for batch-1 decode with an explicit dense fallback.

    Reference: ``deployment.py:182-297``; the route / fallback / binding protocol
    is ``packed_linear.PackedLinearBase``.  Keep the fp32 scale buffers intact
    (move with ``.to(device)``, never ``.half()``): both routes check them.
    """

    bias_in_place = False

    def __init__(self, payload, *, bias=None, fallback="error", groups_per_split=8, kernel="v1"):
        super().__init__()
        if kernel not in KERNELS:
            raise ValueError("unknown kernel")
        self.out_features, groups = validate_artifact(payload)
        self.in_features = groups * GROUP
        workspace_shape(self.out_features, self.in_features, groups_per_split)
        self._init_protocol(fallback=fallback, bias=bias)
        self.kernel = kernel
        self.groups_per_split = groups_per_split
        layout = convert_artifact(payload, kernel=kernel)
        for name, value in layout.items():
            self.register_buffer(name, value)
        # the kernel reads planes: interleaved layouts keep a planar copy (not saved)
        planar = kernel in PLANAR_KERNELS
        for name in _PLANAR_FIELDS:
            copy = None if planar else _to_planes(layout[name]).contiguous()
            self.register_buffer(f"_{name}_planar", copy, persistent=False)
        self.register_buffer("_workspace", None, persistent=False)

    def layout(self):
        return {name: getattr(self, name) for name in LAYOUT_FIELDS}

    def _payload_device(self) -> torch.device:
        return self.codes.device

    def _dense_weight(self, dtype: torch.dtype) -> torch.Tensor:
        return decode_layout(self.layout(), dtype)

    def _check_before_call(self) -> None:
        if any(getattr(self, n).dtype != torch.float32 for n in _SCALE_BUFFERS):
            raise ValueError("FP32 scale buffers were cast; move devices without dtype conversion")

    def _check_before_bind(self, device: torch.device) -> None:
        if any(t.device != device or not t.is_contiguous() for t in self.layout().values()):
            raise ValueError("contiguous same-device layout required")
        self._check_before_call()
        load_extension(self.kernel)

    def _workspace_on(self, device: torch.device) -> torch.Tensor:
        shape = workspace_shape(self.out_features, self.in_features, self.groups_per_split, kernel=self.kernel)
        ws = self._workspace
        if ws is None or ws.device != device or tuple(ws.shape) != shape:
            self._workspace = ws = torch.empty(shape, device=device, dtype=torch.float32)
        return ws

    def _packed_kernel(self, rows: int, device: torch.device):
        codes = self.codes if self._codes_planar is None else self._codes_planar
        sparse = self.sparse_codes if self._sparse_codes_planar is None else self._sparse_codes_planar
        extension = load_extension(self.kernel)
        workspace = self._workspace_on(device)

        def run(x2: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
            return extension.m1_out(x2, codes, self.rows, self.columns, sparse, self.sparse_rows,
                                    self.sparse_columns, self.indices, out, workspace, self.groups_per_split)
        return run


class HybridSegmentsGemv:
    """Hybrid Linears that read the same activation (a decoder layer's q|k|v or
    gate|up) as one launch, ``fx_hybrid_gemv_segments``: the modules' codes, row
    scales, refinement codes and refinement row scales are concatenated along O
    once here; their column scales, refinement indices and refinement column
    scales stay per module.  ``out`` is ``[1, sum(out_features)]``, the modules'
    outputs side by side, each row with the bits of its module's own call when the
    fused launch and that call split K over the same number of workgroups (the
    decode shapes: one split each); where the split counts differ (narrow modules
    at long K, e.g. two 256-row modules at K = 16384: 1 split fused, 4 alone) the
    fp32 partials are summed in another order and rows agree to the output's last
    bit or so.  Raises ``ValueError`` unless 1..4 GPU modules share ``in_features``, carry no
    bias, and (for several) have row counts that are multiples of 16."""

    MAX_SEGMENTS = 4

    def __init__(self, modules):
        import ctypes

        modules = list(modules)
        if not 1 <= len(modules) <= self.MAX_SEGMENTS:
            raise ValueError(f"1..{self.MAX_SEGMENTS} hybrid Linears per launch, got {len(modules)}")
        if not all(isinstance(m, PackedHybridLinear) for m in modules):
            raise ValueError("every module must be a PackedHybridLinear")
        first = modules[0]
        device = first.codes.device
        if device.type != "cuda":
            raise ValueError("fused hybrid GEMV runs on a GPU")
        if any(m.in_features != first.in_features or m.bias is not None or m.codes.device != device
               for m in modules):
            raise ValueError("fused hybrid Linears need one in_features, one device and no bias")
        if len(modules) > 1 and any(m.out_features % 16 for m in modules):
            raise ValueError("concatenated hybrid Linears need row counts that are multiples of 16")
        for m in modules:
            m._check_before_call()

        def planar(m, name):
            copy = getattr(m, f"_{name}_planar")
            return getattr(m, name) if copy is None else copy

        def joined(tensors):  # one module: its own (contiguous) buffer, no copy
            return tensors[0].contiguous() if len(tensors) == 1 else torch.cat(tensors, dim=1).contiguous()

        self.in_features = first.in_features
        self.out_features = sum(m.out_features for m in modules)
        self.codes = joined([planar(m, "codes") for m in modules])
        self.rows = joined([m.rows for m in modules])
        self.sparse_codes = joined([planar(m, "sparse_codes") for m in modules])
        self.sparse_rows = joined([m.sparse_rows for m in modules])
        self._columns = [m.columns.contiguous() for m in modules]
        self._indices = [HybridExtension._sorted_columns(m.indices) for m in modules]
        self._sparse_columns = [m.sparse_columns.contiguous() for m in modules]
        n = len(modules)
        vp = ctypes.c_void_p
        self._n = n
        self._segment_rows = (ctypes.c_int * n)(*[m.out_features for m in modules])
        self._cols_ptrs = (vp * n)(*[t.data_ptr() for t in self._columns])
        self._idx_ptrs = (vp * n)(*[t.data_ptr() for t in self._indices])
        self._scols_ptrs = (vp * n)(*[t.data_ptr() for t in self._sparse_columns])
        self.lib = _lib.library()
        nbytes = self.lib.fx_hybrid_gemv_workspace_bytes(self.out_features, self.in_features)
        self.workspace = torch.empty(max(nbytes, 4) // 4, dtype=torch.float32, device=device) if nbytes else None
        self._workspace_view = (self.workspace if self.workspace is not None
                                else torch.empty(0, dtype=torch.float32, device=device))

    def __call__(self, x: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
        _check_m1_args(x, out, self._workspace_view, self.out_features, self.in_features)
        ws = self.workspace
        _lib.check(self.lib.fx_hybrid_gemv_segments(
            x.data_ptr(), _lib.dtype_code(x.dtype), self._n, self._segment_rows, self.codes.data_ptr(),
            self.rows.data_ptr(), self._cols_ptrs, self._idx_ptrs, self.sparse_codes.data_ptr(),
            self.sparse_rows.data_ptr(), self._scols_ptrs, None if ws is None else ws.data_ptr(),
            0 if ws is None else ws.numel() * 4, out.data_ptr(), self.in_features, _lib.stream_handle(x.device)),
            "fx_hybrid_gemv_segments")
        return out

    def rmsnormed(self, h: torch.Tensor, tile_sumsq: torch.Tensor, weight: torch.Tensor, eps: float,
                  out: torch.Tensor) -> torch.Tensor:
        """The GEMV of RMSNorm(h) (``fx_hybrid_gemv_segments_rmsnormed``): the kernel
        normalises h from ``tile_sumsq``, the fp32 sums of h^2 over its 16-element
        tiles, and the norm ``weight`` [K]."""
        _check_m1_args(h, out, self._workspace_view, self.out_features, self.in_features)
        if (tile_sumsq.dtype != torch.float32 or tile_sumsq.device != h.device or not tile_sumsq.is_contiguous()
                or weight.dtype != h.dtype or weight.device != h.device or not weight.is_contiguous()):
            raise RuntimeError("tile sums must be contiguous fp32 and the norm weight contiguous in h's dtype")
        ws = self.workspace
        _lib.check(self.lib.fx_hybrid_gemv_segments_rmsnormed(
            h.data_ptr(), _lib.dtype_code(h.dtype), self._n, self._segment_rows, self.codes.data_ptr(),
            self.rows.data_ptr(), self._cols_ptrs, self._idx_ptrs, self.sparse_codes.data_ptr(),
            self.sparse_rows.data_ptr(), self._scols_ptrs, tile_sumsq.data_ptr(), tile_sumsq.numel(),
            weight.data_ptr(), eps, None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel() * 4,
            out.data_ptr(), self.in_features, _lib.stream_handle(h.device)), "fx_hybrid_gemv_segments_rmsnormed")
        return out

    def residual(self, x: torch.Tensor, residual: torch.Tensor, tile_sumsq: torch.Tensor,
                 out: torch.Tensor | None = None, swiglu: bool = False) -> torch.Tensor:
        """One module: out = round(residual + round(x @ W.T)) (``out`` None: in
        place) and the fp32 sums of out^2 over 16-row tiles into ``tile_sumsq``
        (``fx_hybrid_gemv_residual``).  ``swiglu``: x is gate | up ``[1, 2K]`` and
        the GEMV reads round(round(silu(gate)) * up), the SwiGLU of Qwen3MLP."""
        if self._n != 1:
            raise ValueError("the residual epilogue takes one hybrid Linear")
        out = residual if out is None else out
        k = self.in_features
        if swiglu:
            if tuple(x.shape) != (1, 2 * k):
                raise RuntimeError("x must be gate | up [1, 2K] for the SwiGLU prologue")
            _check_m1_args(x[:, :k].contiguous(), out, self._workspace_view, self.out_features, k)
            if not x.is_contiguous():
                raise RuntimeError("x must be contiguous")
        else:
            _check_m1_args(x, out, self._workspace_view, self.out_features, k)
        if residual.shape != out.shape or residual.dtype != out.dtype or not residual.is_contiguous():
            raise RuntimeError("residual must match out")
        if (tile_sumsq.dtype != torch.float32 or tile_sumsq.numel() != (self.out_features + 15) // 16
                or not tile_sumsq.is_contiguous() or tile_sumsq.device != x.device):
            raise RuntimeError("tile_sumsq must be contiguous fp32 [ceil(O / 16)]")
        _lib.check(self.lib.fx_hybrid_gemv_residual(
            x.data_ptr(), _lib.dtype_code(x.dtype), self.codes.data_ptr(), self.rows.data_ptr(),
            self._columns[0].data_ptr(), self._indices[0].data_ptr(), self.sparse_codes.data_ptr(),
            self.sparse_rows.data_ptr(), self._sparse_columns[0].data_ptr(), residual.data_ptr(), out.data_ptr(),
            tile_sumsq.data_ptr(), self.out_features, self.in_features, int(swiglu), _lib.stream_handle(x.device)),
            "fx_hybrid_gemv_residual")
        return out


def replace_block_linears(block, layer_payload, *, fallback="error", groups_per_split=8, kernel="v1"):
    """Replace the seven Qwen3 Linears of one block; every payload is validated and
    every replacement built before the block is touched."""
    from .qwen3 import QWEN3_LINEAR_MODULES

    if set(layer_payload) != {f"{m}.{f}" for m in QWEN3_LINEAR_MODULES for f in FIELDS}:
        raise ValueError("layer must contain exactly seven complete hybrid payloads")

    def build(name: str) -> PackedHybridLinear:
        linear = block.get_submodule(name)
        payload = {field: layer_payload[f"{name}.{field}"] for field in FIELDS}
        o, g = validate_artifact(payload)
        if not isinstance(linear, nn.Linear) or (linear.out_features, linear.in_features) != (o, g * GROUP):
            raise ValueError(f"Linear shape/type mismatch: {name}")
        return PackedHybridLinear(payload, bias=linear.bias, fallback=fallback, groups_per_split=groups_per_split,
                                  kernel=kernel).to(linear.weight.device)

    return replace_linears_atomically(block, [(name, build(name)) for name in QWEN3_LINEAR_MODULES])
