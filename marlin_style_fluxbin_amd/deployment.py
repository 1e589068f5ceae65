"""Hybrid g128/s8 two-base layout and the batch-1 GEMV, drop-in for the reference's
``deployment.py`` (``FIELDS`` :23-25, ``validate_artifact`` :30-55, ``_to_planes`` /
``_from_planes`` :59-77, ``convert_artifact`` :84-103, ``restore_artifact`` :106-115,
``decode_layout`` :118-121, ``workspace_shape`` :158-165, ``m1_out`` :168-179,
``PackedHybridLinear`` :182-297, ``replace_block_linears`` :300-320).

The GPU op is one gfx950 kernel (``fx_hybrid_gemv``: sign bits as int8 matrix-core
operands, 16-bit fixed-point activation digits, fp32 per-group scales applied
per batch) reading the planar layout of the ``v5_p*`` kernels.  Layouts of the
interleaved kernels (``v1`` .. ``v5``) are accepted: ``m1_out`` converts their codes
to planes per call (allocating), and ``PackedHybridLinear`` keeps a planar copy so
its packed route never converts.  All kernel names share the factored fp32
arithmetic of ``v4``/``v5`` (the ``v1``..``v3`` kernels round each weight to the
activation dtype first; the difference is within the reference's own gates).
There is no CPU substitute for the packed route: without the HIP library it
raises.
"""
from __future__ import annotations

from typing import Mapping

import torch
from torch import nn
from torch.nn import functional as F

from . import _lib
from .evaluation import materialize_hybrid_s8_weight, tensor_sha256

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


def validate_artifact(p: Mapping[str, torch.Tensor]) -> tuple[int, int]:
    """Shape / dtype / device contract of the seven payload fields; ``(O, G)``."""
    if set(p) != set(FIELDS):
        raise ValueError("expected exactly seven hybrid payload fields")
    codes = p["global_sign_codes"]
    if codes.ndim != 2 or codes.dtype != torch.uint8:
        raise ValueError("global codes must be uint8 [O,K/4]")
    o, width = codes.shape
    if not (1 <= o <= 65536) or width < 32 or width > 32768 or width % 32:
        raise ValueError("requires O=1..65536 and K=128..131072 divisible by 128")
    g = width // 32
    shapes = ((o, width), (2, o, g), (2, g, GROUP), (g, REFINED), (o, g * 2), (2, o, g), (2, g, REFINED))
    for name, shape in zip(FIELDS, shapes):
        t = p[name]
        if tuple(t.shape) != shape or t.device != codes.device:
            raise ValueError(f"shape/device mismatch: {name}")
        if "scales" in name and (t.dtype != torch.float32 or not torch.isfinite(t).all()):
            raise ValueError(f"finite FP32 scales required: {name}")
    if p["refinement_sign_codes"].dtype != torch.uint8:
        raise ValueError("refinement codes must be uint8")
    ix = p["refinement_indices"]
    if ix.dtype not in (torch.int16, torch.int32, torch.int64):
        raise ValueError("integer refinement indices required")
    if (ix < 0).any() or (ix >= GROUP).any() or (ix[:, 1:] <= ix[:, :-1]).any():
        raise ValueError("indices must be sorted, unique and inside each group")
    return o, g


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


def layout_format(layout) -> str:
    return PLANAR_FORMAT if layout["codes"].ndim == 4 else FORMAT


def convert_artifact(p: Mapping[str, torch.Tensor], *, kernel: str = "v1") -> dict[str, torch.Tensor]:
    """Payload -> group-major deployment layout; lossless (a permutation of the
    bytes plus the column ``lookup``), independent of later changes to ``p``."""
    if kernel not in KERNELS:
        raise ValueError("unknown kernel")
    o, g = validate_artifact(p)
    ix = p["refinement_indices"].to(torch.int16)
    lookup = torch.full((g, GROUP), -1, dtype=torch.int16, device=ix.device)
    lookup.scatter_(1, ix.long(), torch.arange(REFINED, dtype=torch.int16, device=ix.device).expand(g, REFINED))
    layout = {
        "codes": p["global_sign_codes"].reshape(o, g, 32).permute(1, 0, 2),
        "rows": p["global_row_scales"].permute(2, 1, 0),
        "columns": p["global_column_scales"].permute(1, 2, 0),
        "indices": ix,
        "sparse_codes": p["refinement_sign_codes"].reshape(o, g, 2).permute(1, 0, 2),
        "sparse_rows": p["refinement_row_scales"].permute(2, 1, 0),
        "sparse_columns": p["refinement_column_scales"].permute(1, 2, 0),
        "lookup": lookup,
    }
    layout = {k: v.contiguous().clone() for k, v in layout.items()}
    if kernel in PLANAR_KERNELS:
        layout["codes"] = _to_planes(layout["codes"]).contiguous()
        layout["sparse_codes"] = _to_planes(layout["sparse_codes"]).contiguous()
    return layout


def restore_artifact(layout: Mapping[str, torch.Tensor]) -> dict[str, torch.Tensor]:
    """Inverse of :func:`convert_artifact`."""
    codes, sparse = layout["codes"], layout["sparse_codes"]
    g, o = codes.shape[:2]
    if codes.ndim == 4:
        codes, sparse = _from_planes(codes), _from_planes(sparse)
    payload = {
        "global_sign_codes": codes.permute(1, 0, 2).reshape(o, g * 32),
        "global_row_scales": layout["rows"].permute(2, 1, 0),
        "global_column_scales": layout["columns"].permute(2, 0, 1),
        "refinement_indices": layout["indices"],
        "refinement_sign_codes": sparse.permute(1, 0, 2).reshape(o, g * 2),
        "refinement_row_scales": layout["sparse_rows"].permute(2, 1, 0),
        "refinement_column_scales": layout["sparse_columns"].permute(2, 0, 1),
    }
    return {k: v.contiguous() for k, v in payload.items()}


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
    if (not isinstance(groups_per_split, int) or not 1 <= groups_per_split <= 1024
            or not 1 <= out_features <= 65536 or not 128 <= in_features <= 131072 or in_features % 128):
        raise ValueError("invalid group/split dimensions")
    splits = (in_features // 128 + groups_per_split - 1) // groups_per_split
    if kernel in ("v4", "v4_late"):
        return (in_features // 128 * 272 + splits * out_features,)
    return (splits, out_features)


class HybridExtension:
    """Object returned by :func:`load_extension`: ``m1_out`` with the reference's
    positional arguments (``csrc/m1_v5.cu`` pybind ``m1_out``), on the C ABI."""

    def __init__(self, kernel: str):
        self.kernel = kernel
        self.lib = _lib.library()

    def m1_out(self, x, codes, rows, columns, sparse_codes, sparse_rows, sparse_columns, indices_or_lookup,
               out, workspace, groups_per_split):
        if codes.ndim != 4:
            codes, sparse_codes = _to_planes(codes).contiguous(), _to_planes(sparse_codes).contiguous()
        if indices_or_lookup.shape[-1] != REFINED:  # a lookup table: recover the sorted columns
            lookup = indices_or_lookup
            indices_or_lookup = torch.argsort(lookup.to(torch.int32) < 0, dim=1, stable=True)[:, :REFINED]
        indices = indices_or_lookup.to(torch.int16).contiguous()
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
    if kernel not in _EXTENSIONS:
        _EXTENSIONS[kernel] = HybridExtension(kernel)
    return _EXTENSIONS[kernel]


def _check_m1_args(x, out, workspace, o, k):
    if not x.is_cuda or x.dtype not in (torch.float16, torch.bfloat16) or tuple(x.shape) != (1, k) \
            or not x.is_contiguous():
        raise RuntimeError("x must be a contiguous CUDA fp16/bf16 tensor [1, K]")
    if out.dtype != x.dtype or tuple(out.shape) != (1, o) or not out.is_contiguous() or out.device != x.device:
        raise RuntimeError("out must be a contiguous [1, O] tensor in the activation dtype")
    if workspace.dtype != torch.float32 or not workspace.is_contiguous() or workspace.device != x.device:
        raise RuntimeError("workspace must be a contiguous fp32 tensor on the activation device")


def m1_out(x, layout, out, workspace, *, groups_per_split=8, kernel="v1"):
    """Engine-neutral batch-1 op: ``out = x @ W.T`` for a hybrid layout, fp32
    accumulation, current stream, caller-owned ``out`` and ``workspace``
    (:func:`workspace_shape`); no allocation for planar layouts.  Workspaces must
    not be shared by overlapping calls on different streams."""
    indices = layout["indices"] if kernel in FACTORED_KERNELS else layout["lookup"]
    return load_extension(kernel).m1_out(x, layout["codes"], layout["rows"], layout["columns"],
                                         layout["sparse_codes"], layout["sparse_rows"], layout["sparse_columns"],
                                         indices, out, workspace, groups_per_split)


class PackedHybridLinear(nn.Module):
    """Hybrid two-base Linear for batch-1 decode with an explicit dense fallback.

    Reference: ``deployment.py:182-297``.  The packed route serves one CUDA fp16 /
    bf16 row; anything else raises unless ``fallback='dense'``.  Keep the fp32
    scale buffers intact (move with ``.to(device)``, never ``.half()``).
    """

    def __init__(self, payload, *, bias=None, fallback="error", groups_per_split=8, kernel="v1"):
        super().__init__()
        if fallback not in ("error", "dense"):
            raise ValueError("fallback must be error or dense")
        if kernel not in KERNELS:
            raise ValueError("unknown kernel")
        self.kernel = kernel
        self.route_counts = {"packed_m1": 0, "dense_fallback": 0}
        self.out_features, g = validate_artifact(payload)
        self.in_features = g * GROUP
        self.fallback, self.groups_per_split = fallback, groups_per_split
        workspace_shape(self.out_features, self.in_features, groups_per_split)
        layout = convert_artifact(payload, kernel=kernel)
        for name, value in layout.items():
            self.register_buffer(name, value)
        # the kernel reads planes; interleaved layouts keep a planar copy (not saved)
        planar = kernel in PLANAR_KERNELS
        self.register_buffer("_codes_planar", None if planar else _to_planes(layout["codes"]).contiguous(),
                             persistent=False)
        self.register_buffer("_sparse_planar", None if planar else _to_planes(layout["sparse_codes"]).contiguous(),
                             persistent=False)
        self.register_buffer("bias", None if bias is None else bias.detach().clone())
        self.register_buffer("_workspace", None, persistent=False)
        self.register_buffer("_decode_output", None, persistent=False)
        self.last_route = "not_called"
        self._decode_binding = None
        self._decode_audit = False

    def clear_prepared_decode(self):
        self._decode_binding = None
        self._decode_output = None
        self._decode_audit = False

    def _apply(self, fn, recurse=True):
        self.clear_prepared_decode()  # a move invalidates captured tensor references
        return super()._apply(fn, recurse=recurse)

    def layout(self):
        return {name: getattr(self, name) for name in LAYOUT_FIELDS}

    def _kernel_fields(self):
        codes = self.codes if self._codes_planar is None else self._codes_planar
        sparse = self.sparse_codes if self._sparse_planar is None else self._sparse_planar
        return codes, sparse

    def _check_scales(self):
        if any(getattr(self, n).dtype != torch.float32 for n in ("rows", "columns", "sparse_rows", "sparse_columns")):
            raise ValueError("FP32 scale buffers were cast; move devices without dtype conversion")

    def _workspace_for(self, device):
        shape = workspace_shape(self.out_features, self.in_features, self.groups_per_split, kernel=self.kernel)
        if self._workspace is None or self._workspace.device != device or tuple(self._workspace.shape) != shape:
            self._workspace = torch.empty(shape, device=device, dtype=torch.float32)
        return self._workspace

    def _run(self, x2, out):
        codes, sparse = self._kernel_fields()
        return load_extension(self.kernel).m1_out(x2, codes, self.rows, self.columns, sparse, self.sparse_rows,
                                                   self.sparse_columns, self.indices, out,
                                                   self._workspace_for(x2.device), self.groups_per_split)

    def bind_prepared_decode(self, dtype):
        """Bind serial ``[1, 1, K]`` inference; outputs alias a reusable module buffer.
        Finish consumers on the same stream before another call; clear the binding
        before modifying or replacing any buffer."""
        if self._decode_binding is not None:
            raise ValueError("decode already bound")
        if dtype not in (torch.float16, torch.bfloat16):
            raise ValueError("FP16/BF16 required")
        device = self.codes.device
        if device.type != "cuda":
            raise ValueError("prepared decode requires CUDA")
        if any(t.device != device or not t.is_contiguous() for t in self.layout().values()):
            raise ValueError("contiguous same-device layout required")
        self._check_scales()
        load_extension(self.kernel)
        self._workspace_for(device)
        self._decode_output = torch.empty((1, self.out_features), device=device, dtype=dtype)
        output = self._decode_output
        shaped = output.view(1, 1, self.out_features)
        expected = (1, 1, self.in_features)

        def apply(x):
            if torch.is_grad_enabled():
                raise RuntimeError("prepared decode is inference only")
            if tuple(x.shape) != expected or x.dtype != dtype or x.device != device or not x.is_contiguous():
                raise ValueError("prepared decode input shape/dtype/device/stride mismatch")
            if self._decode_audit:
                self.route_counts["packed_m1"] += 1
                self.last_route = "packed_m1"
            self._run(x.view(1, self.in_features), output)
            if self.bias is not None:
                output.add_(self.bias)
            return shaped

        self._decode_binding = apply

    def forward(self, x):
        if self._decode_binding is not None:
            return self._decode_binding(x)
        if torch.is_grad_enabled():
            raise RuntimeError("packed inference requires no_grad/inference_mode")
        if x.ndim < 2 or x.shape[-1] != self.in_features:
            raise ValueError("expected [...,K] input")
        self._check_scales()
        m = x.numel() // self.in_features
        if m != 1 or not x.is_cuda or x.dtype not in (torch.float16, torch.bfloat16):
            if self.fallback != "dense":
                raise ValueError("unsupported input; enable explicit dense fallback if needed")
            self.last_route = "dense_fallback"
            self.route_counts["dense_fallback"] += 1
            return F.linear(x, decode_layout(self.layout(), x.dtype), self.bias)
        self.last_route = "packed_m1"
        self.route_counts["packed_m1"] += 1
        y = torch.empty((1, self.out_features), device=x.device, dtype=x.dtype)
        self._run(x.reshape(1, self.in_features).contiguous(), y)
        if self.bias is not None:
            y = y + self.bias
        return y.reshape(*x.shape[:-1], self.out_features)


def replace_block_linears(block, layer_payload, *, fallback="error", groups_per_split=8, kernel="v1"):
    """Replace the seven Qwen3 Linears of one block; every payload is validated and
    every replacement built before the block is touched."""
    from .qwen3 import QWEN3_LINEAR_MODULES

    expected = {f"{module}.{field}" for module in QWEN3_LINEAR_MODULES for field in FIELDS}
    if set(layer_payload) != expected:
        raise ValueError("layer must contain exactly seven complete hybrid payloads")
    built = []
    for name in QWEN3_LINEAR_MODULES:
        old = block.get_submodule(name)
        p = {field: layer_payload[f"{name}.{field}"] for field in FIELDS}
        o, g = validate_artifact(p)
        if not isinstance(old, nn.Linear) or (old.out_features, old.in_features) != (o, g * GROUP):
            raise ValueError(f"Linear shape/type mismatch: {name}")
        built.append((name, PackedHybridLinear(p, bias=old.bias, fallback=fallback, groups_per_split=groups_per_split,
                                               kernel=kernel).to(old.weight.device)))
    for name, module in built:
        parent, attr = name.rsplit(".", 1)
        setattr(block.get_submodule(parent), attr, module)
    return [name for name, _ in built]
