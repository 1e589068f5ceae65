"""W3 LUT Linear on MI355X: functional ops, route policy and ``PackedW3Linear``.

Mirrors the public surface of the reference's ``w3_lut_deployment.py``
(maxiu188-afk/Marlin_Style_Fluxbin ``src/fluxbin_style/w3_lut_deployment.py:15-417``);
every GPU call goes to the hand-written gfx950 kernels in ``libfluxbin_amd.so``
through its C ABI (``include/fluxbin_amd.h``).  There is no CPU substitute on the
packed route: a missing library raises.

Differences from the reference, all deliberate:
* The layout may carry ``zeros`` and fp16 scales (see ``gptq_deployment``).
* ``PackedW3Linear`` with one group per split runs the one-launch MFMA kernel in
  either arithmetic (the same sums, another fp32 order; ``decoded_bf16`` adds the
  +-3 correction as a second MFMA chain); a route that splits K over
  ``groups_per_split > 1`` groups runs the reference's split contract on the table
  kernel.
* ``PackedW3Linear(max_packed_rows=n)`` opts 2..n-row inputs into the packed
  route (config 1's small-M GEMV); by default they take the dense fallback, as
  in the reference.
"""
from __future__ import annotations

from functools import lru_cache

import torch
from torch import nn

from . import _lib
from .packed_linear import PackedLinearBase, replace_linears_atomically
from .gptq_deployment import FIELDS, OPTIONAL_FIELDS, restore_planar_w3, validate_planar_w3

ROW_TILES = (256, 512, 1024)
EXPERIMENTAL_ROW_TILES = ROW_TILES
ARITHMETIC_MODES = ("structural", "decoded_bf16")
MAX_PACKED_ROWS = 8
QWEN3_ROW_TILE_BY_SHAPE = {
    (4096, 4096): 256,
    (1024, 4096): 512,
    (12288, 4096): 1024,
    (4096, 12288): 1024,
}
QWEN3_W3_ROUTE_POLICIES = {
    "structural": {
        shape: {"row_tile": row_tile, "groups_per_split": 1, "arithmetic": "structural"}
        for shape, row_tile in QWEN3_ROW_TILE_BY_SHAPE.items()
    },
    "fast_corrected": {
        shape: {"row_tile": row_tile, "groups_per_split": 1, "arithmetic": "decoded_bf16"}
        for shape, row_tile in QWEN3_ROW_TILE_BY_SHAPE.items()
    },
    "observed_exact": {
        shape: {
            "row_tile": row_tile,
            "groups_per_split": {(4096, 4096): 1, (1024, 4096): 1, (12288, 4096): 4, (4096, 12288): 2}[shape],
            "arithmetic": "decoded_bf16",
        }
        for shape, row_tile in QWEN3_ROW_TILE_BY_SHAPE.items()
    },
}


def _arith_code(arithmetic: str) -> int:
    if arithmetic not in ARITHMETIC_MODES:
        raise ValueError(f"arithmetic must be one of {ARITHMETIC_MODES}")
    return _lib.ARITH_STRUCTURAL if arithmetic == "structural" else _lib.ARITH_DECODED_BF16


class _Extension:
    """Tensor-level view of the C ABI with the reference extension's method names
    (``csrc/w3_lut.cu:334-339``: inline_main, inline_main_bf16_weight, finish, m1_out)."""

    def __init__(self, row_tile: int):
        self.row_tile = row_tile
        self.lib = _lib.library()

    def _main(self, x, planes, scales, perm, partial, arithmetic, zeros=None, groups_per_split=1):
        g, _, o, _ = planes.shape
        m, k = x.shape
        _lib.check(self.lib.fx_w3_inline_main(
            x.data_ptr(), _lib.dtype_code(x.dtype), planes.data_ptr(), scales.data_ptr(),
            _lib.dtype_code(scales.dtype), _lib.ptr(zeros), _lib.ptr(perm), partial.data_ptr(),
            m, o, k, groups_per_split, self.row_tile, arithmetic, _lib.stream_handle(x.device)),
            "fx_w3_inline_main")

    def inline_main(self, x, planes, scales, perm, partial, zeros=None):
        self._main(x, planes, scales, perm, partial, _lib.ARITH_STRUCTURAL, zeros)

    def inline_main_bf16_weight(self, x, planes, scales, perm, partial, zeros=None):
        self._main(x, planes, scales, perm, partial, _lib.ARITH_DECODED_BF16, zeros)

    def finish(self, partial, out):
        splits = partial.shape[0]
        m, o = out.shape
        _lib.check(self.lib.fx_w3_finish(partial.data_ptr(), out.data_ptr(), _lib.dtype_code(out.dtype),
                                         splits, m, o, _lib.stream_handle(out.device)), "fx_w3_finish")

    def m1_out(self, x, planes, scales, perm, partial, out, groups_per_split, dense_bf16_weight_semantics,
               zeros=None):
        g, _, o, _ = planes.shape
        m, k = x.shape
        arith = _lib.ARITH_DECODED_BF16 if dense_bf16_weight_semantics else _lib.ARITH_STRUCTURAL
        _lib.check(self.lib.fx_w3_m1_out(
            x.data_ptr(), _lib.dtype_code(x.dtype), planes.data_ptr(), scales.data_ptr(),
            _lib.dtype_code(scales.dtype), _lib.ptr(zeros), _lib.ptr(perm), partial.data_ptr(),
            out.data_ptr(), m, o, k, groups_per_split, self.row_tile, arith,
            _lib.stream_handle(x.device)), "fx_w3_m1_out")


BUILD_CONTRACT_SCHEMA = 1


def _check_build_request(row_tile: int, uniform_index_probe: bool) -> None:
    if row_tile not in EXPERIMENTAL_ROW_TILES:
        raise ValueError(f"row_tile must be one of {EXPERIMENTAL_ROW_TILES}")
    if uniform_index_probe:
        raise ValueError("the uniform-index probe build is not provided; use rocprof LDS counters")


@lru_cache(maxsize=1)
def _hipcc_identity() -> dict:
    import subprocess

    from .build import hipcc

    try:
        exe = hipcc()
    except RuntimeError:
        return {"executable": "unresolved", "version": "unresolved"}
    try:
        done = subprocess.run([exe, "--version"], capture_output=True, text=True, timeout=30, check=False)
        version = (done.stdout or done.stderr).strip()
    except (OSError, subprocess.TimeoutExpired) as exc:
        version = type(exc).__name__
    return {"executable": exe, "version": version}


def w3_lut_extension_build(row_tile: int, uniform_index_probe: bool = False) -> tuple[dict, dict]:
    """Load description and auditable build contract of the kernel library, as
    the reference's ``w3_lut_extension_build`` (``w3_lut_deployment.py:49-68``,
    ``extension_cache.py:74-149``) returns them for its per-row-tile extension.

    Here every row tile is served by the one prebuilt ``libfluxbin_amd.so``
    (``row_tile`` is a tuning hint), so the contract is the same for all of them:
    the name, every HIP source and header with its SHA-256, the hipcc flags and
    target, the interpreter / torch / HIP runtime and the compiler identity, and
    ``cache_key``, the SHA-256 of those fields in canonical JSON.  Any change of
    a source byte, flag or toolchain changes the key; a documentation change does
    not.  ``library_sha256`` (outside the key) is the built library's digest, or
    None when it is not built."""
    import hashlib
    import json
    import platform
    import sys

    from . import build as _build

    _check_build_request(row_tile, uniform_index_probe)
    sources = sorted(_build.CSRC.glob("*.hip")) + sorted(_build.CSRC.glob("*.h"))
    header = _build.PACKAGE.parent / "include" / "fluxbin_amd.h"
    dependencies = [header] if header.is_file() else []
    contract = {
        "schema_version": BUILD_CONTRACT_SCHEMA,
        "name": "fluxbin_amd",
        "sources": [{"name": p.name, "sha256": hashlib.sha256(p.read_bytes()).hexdigest()}
                    for p in sources + dependencies],
        "extra_hip_cflags": list(_build.HIPCC_FLAGS),
        "target_architecture": _build.ARCH,
        "python": f"{sys.version_info.major}.{sys.version_info.minor}",
        "platform": platform.system(),
        "machine": platform.machine(),
        "torch": torch.__version__,
        "torch_hip_runtime": torch.version.hip,
        "compiler": {"hipcc": _hipcc_identity()},
    }
    encoded = json.dumps(contract, sort_keys=True, separators=(",", ":")).encode()
    contract["cache_key"] = hashlib.sha256(encoded).hexdigest()
    units = {p.name for p in _build.compile_units()}
    contract["compile_sources"] = [p.name for p in sources if p.name in units]
    contract["content_dependencies"] = [p.name for p in sources + dependencies if p.name not in units]
    library = _lib.LIBRARY_PATH
    contract["library_sha256"] = hashlib.sha256(library.read_bytes()).hexdigest() if library.is_file() else None
    kwargs = {"name": contract["name"], "sources": [str(p) for p in sources if p.name in units],
              "library": str(library),
              "extra_hip_cflags": list(_build.HIPCC_FLAGS), "row_tile": row_tile}
    return kwargs, contract


@lru_cache(maxsize=2 * len(EXPERIMENTAL_ROW_TILES))
def load_w3_lut_extension(row_tile: int, uniform_index_probe: bool = False):
    """Return the loaded kernel library for one row tile.

    ``uniform_index_probe`` (the reference's timing-only wrong-result build,
    ``csrc/w3_lut.cu:17-27``) is not offered: LDS bank conflicts are read from
    rocprof counters instead, so no build ever returns wrong values on purpose.
    """
    _check_build_request(row_tile, uniform_index_probe)
    if not torch.cuda.is_available():
        raise RuntimeError("W3 LUT requires a ROCm GPU; there is no CPU substitute")
    return _Extension(row_tile)


def workspace_shape(out_features: int, in_features: int, groups_per_split: int = 1) -> tuple[int, int]:
    if not 1 <= out_features <= 65536 or not 128 <= in_features <= 32767 or in_features % 128:
        raise ValueError("invalid W3 LUT dimensions")
    groups = in_features // 128
    if not isinstance(groups_per_split, int) or not 1 <= groups_per_split <= groups:
        raise ValueError("groups_per_split must be an integer in [1,K/128]")
    return (groups + groups_per_split - 1) // groups_per_split, out_features


def _check_layout_device(layout, *tensors):
    device = layout["planes"].device
    if device.type != "cuda":
        raise ValueError("the W3 LUT kernels require the layout on a ROCm GPU")
    if any(t.device != device for t in tensors) or any(v.device != device for v in layout.values()):
        raise ValueError("x, layout and workspace must share a device")


def inline_main(x: torch.Tensor, layout: dict, workspace: torch.Tensor, *, row_tile: int,
                arithmetic: str = "structural") -> None:
    """fp32 per-group partials ``workspace [K/128, O]`` for ``x [1, K]`` (one split per group)."""
    out_features, in_features = validate_planar_w3(layout, check_values=False)
    if x.shape != (1, in_features):
        raise ValueError("x must have shape [1,K]")
    if arithmetic not in ARITHMETIC_MODES:
        raise ValueError(f"arithmetic must be one of {ARITHMETIC_MODES}")
    if tuple(workspace.shape) != workspace_shape(out_features, in_features) or workspace.dtype != torch.float32:
        raise ValueError("workspace must be FP32 [K/128,O]")
    _check_layout_device(layout, x, workspace)
    ext = load_w3_lut_extension(row_tile)
    fn = ext.inline_main if arithmetic == "structural" else ext.inline_main_bf16_weight
    fn(x, layout["planes"], layout["scales"], layout["perm"], workspace, zeros=layout.get("zeros"))


def finish(workspace: torch.Tensor, out: torch.Tensor, *, row_tile: int) -> torch.Tensor:
    if workspace.ndim != 2 or workspace.dtype != torch.float32:
        raise ValueError("workspace must be FP32 [G,O]")
    if out.shape != (1, workspace.shape[1]) or out.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("out must be FP16/BF16 [1,O]")
    load_w3_lut_extension(row_tile).finish(workspace, out)
    return out


def w3_lut_m1_out(x: torch.Tensor, layout: dict, out: torch.Tensor, workspace: torch.Tensor, *,
                  row_tile: int, groups_per_split: int = 1, arithmetic: str = "structural") -> torch.Tensor:
    """Allocation-free GEMV on the current stream with the reference's split semantics.

    ``x [M, K]`` (M in {1, 2, 4, 8}), ``out [M, O]``, ``workspace`` fp32
    ``[ceil(G/groups_per_split), O]`` for M = 1 (``[splits, M, O]`` otherwise).
    With one split the workspace is left untouched.
    """
    if out.dtype != x.dtype:
        raise ValueError("out dtype must match x dtype")
    code = _arith_code(arithmetic)
    out_features, in_features = validate_planar_w3(layout, check_values=False)
    if x.ndim != 2 or x.shape[1] != in_features or x.shape[0] not in (1, 2, 4, 8):
        raise ValueError("x/out shape mismatch")
    m = x.shape[0]
    if tuple(out.shape) != (m, out_features):
        raise ValueError("x/out shape mismatch")
    splits, _ = workspace_shape(out_features, in_features, groups_per_split)
    expected = (splits, out_features) if m == 1 else (splits, m, out_features)
    if tuple(workspace.shape) != expected or workspace.dtype != torch.float32:
        raise ValueError("workspace must be FP32 [ceil(G/groups_per_split),O]")
    _check_layout_device(layout, x, out, workspace)
    load_w3_lut_extension(row_tile).m1_out(
        x, layout["planes"], layout["scales"], layout["perm"], workspace, out, groups_per_split,
        code == _lib.ARITH_DECODED_BF16, zeros=layout.get("zeros"))
    return out


def qwen3_row_tile(out_features: int, in_features: int) -> int:
    try:
        return QWEN3_ROW_TILE_BY_SHAPE[(out_features, in_features)]
    except KeyError as exc:
        raise ValueError(f"unsupported Qwen3-8B W3 shape: {(out_features, in_features)}") from exc


def qwen3_w3_route(route: str, out_features: int, in_features: int) -> dict:
    if route not in QWEN3_W3_ROUTE_POLICIES:
        raise ValueError(f"unknown Qwen3-8B W3 route: {route}")
    try:
        return dict(QWEN3_W3_ROUTE_POLICIES[route][(out_features, in_features)])
    except KeyError as exc:
        raise ValueError(f"unsupported Qwen3-8B W3 shape: {(out_features, in_features)}") from exc


# --------------------------------------------------------------------------- device helpers
def restore_planar_w3_device(layout: dict, *, dtype: torch.dtype,
                             perm_identity: bool | None = None) -> torch.Tensor:
    """HIP dequantize of a GPU layout into a new dense ``[O, K]`` weight."""
    out_features, in_features = validate_planar_w3(layout, check_values=False)
    weight = torch.empty(out_features, in_features, dtype=dtype, device=layout["planes"].device)
    restore_planar_w3_into(layout, weight, perm_identity=perm_identity)
    return weight


def restore_planar_w3_into(layout: dict, weight: torch.Tensor, *,
                           perm_identity: bool | None = None) -> torch.Tensor:
    """``fx_w3_restore`` into ``weight``.  An identity permutation goes to the
    kernel as NULL (row-ordered 16-byte stores); any other stages whole rows in
    LDS.  ``perm_identity`` None compares the permutation on the device (one
    host synchronisation); callers that know it pass it."""
    out_features, in_features = validate_planar_w3(layout, check_values=False)
    if tuple(weight.shape) != (out_features, in_features) or not weight.is_contiguous():
        raise ValueError("weight must be a contiguous [O,K] tensor")
    _check_layout_device(layout, weight)
    perm = layout["perm"]
    if perm_identity is None:
        perm_identity = bool(torch.equal(perm.long(), torch.arange(in_features, device=perm.device)))
    lib = _lib.library()
    _lib.check(lib.fx_w3_restore(
        layout["planes"].data_ptr(), layout["scales"].data_ptr(), _lib.dtype_code(layout["scales"].dtype),
        _lib.ptr(layout.get("zeros")), None if perm_identity else perm.data_ptr(), weight.data_ptr(),
        _lib.dtype_code(weight.dtype), out_features, in_features, _lib.stream_handle(weight.device)),
        "fx_w3_restore")
    return weight


def gemv_fp32_device(x: torch.Tensor, layout: dict, *, arithmetic: str) -> torch.Tensor:
    """fp32 ``[M, O]`` from the HIP kernel with one K split (no output cast)."""
    out_features, in_features = validate_planar_w3(layout, check_values=False)
    m = x.shape[0]
    if m not in (1, 2, 4, 8):
        raise ValueError("fp32 device GEMV supports M in {1,2,4,8}")
    groups = in_features // 128
    xin = x if x.dtype in (torch.float16, torch.bfloat16) else x.to(torch.bfloat16)
    partial = torch.empty(1, m, out_features, dtype=torch.float32, device=x.device)
    _check_layout_device(layout, x)
    lib = _lib.library()
    _lib.check(lib.fx_w3_inline_main(
        xin.contiguous().data_ptr(), _lib.dtype_code(xin.dtype), layout["planes"].data_ptr(),
        layout["scales"].data_ptr(), _lib.dtype_code(layout["scales"].dtype), _lib.ptr(layout.get("zeros")),
        layout["perm"].data_ptr(), partial.data_ptr(), m, out_features, in_features, groups, 256,
        _arith_code(arithmetic), _lib.stream_handle(x.device)), "fx_w3_inline_main")
    return partial[0]


class W3Gemv:
    """Allocation-free fast path bound to one payload: ``out = x @ W.T`` in one launch.

    Owns the zero-initialised workspace the single-launch K split needs; calls
    sharing it must stay ordered on one stream (the decode graph does).
    """

    def __init__(self, layout: dict, *, arithmetic: str = "structural", max_rows: int = MAX_PACKED_ROWS,
                 perm_identity: bool | None = None):
        self.out_features, self.in_features = validate_planar_w3(layout, check_values=False)
        self.layout = layout
        self.arith = _arith_code(arithmetic)
        device = layout["planes"].device
        if device.type != "cuda":
            raise ValueError("W3Gemv requires a GPU layout")
        self.lib = _lib.library()
        if perm_identity is None:
            perm = layout["perm"]
            perm_identity = bool(torch.equal(perm.long(), torch.arange(self.in_features, device=device)))
        self.perm_ptr = None if perm_identity else layout["perm"].data_ptr()
        self.zeros_ptr = _lib.ptr(layout.get("zeros"))
        self.scale_code = _lib.dtype_code(layout["scales"].dtype)
        self.max_rows = max_rows
        nbytes = max(self.lib.fx_w3_gemv_workspace_bytes(m, self.out_features, self.in_features)
                     for m in range(1, max_rows + 1))
        self.workspace = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=device)

    def __call__(self, x: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
        m = x.shape[0]
        _lib.check(self.lib.fx_w3_gemv(
            x.data_ptr(), _lib.dtype_code(x.dtype), self.layout["planes"].data_ptr(),
            self.layout["scales"].data_ptr(), self.scale_code, self.zeros_ptr, self.perm_ptr,
            self.workspace.data_ptr(), self.workspace.numel(), out.data_ptr(), m, self.out_features,
            self.in_features, self.arith, _lib.stream_handle(x.device)), "fx_w3_gemv")
        return out


class _TableRoute:
    """The reference contract's packed route for one payload: ``fx_w3_m1_out``
    with the module's ``row_tile`` / ``groups_per_split`` and arithmetic (the
    table kernel, fp32 split partials summed in split order), one preallocated
    workspace.  Serves ``decoded_bf16`` and any ``groups_per_split > 1``."""

    def __init__(self, module: "PackedW3Linear", device: torch.device):
        self.module = module
        self.ext = load_w3_lut_extension(module.row_tile)
        shape = workspace_shape(module.out_features, module.in_features, module.groups_per_split)
        self.workspace = torch.empty(shape, device=device, dtype=torch.float32)

    def __call__(self, x: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
        m = self.module
        self.ext.m1_out(x, m.planes, m.scales, m.perm, self.workspace, out, m.groups_per_split,
                        m.arithmetic == "decoded_bf16", zeros=getattr(m, "zeros", None))
        return out


class PackedW3Linear(PackedLinearBase):
    """Decode-oriented W3 Linear with an explicit dense fallback.

    Reference: ``w3_lut_deployment.py:190-359``; the route / fallback / binding
    protocol is ``packed_linear.PackedLinearBase``.  The packed route is the MFMA
    kernel with one group per split (one launch; ``decoded_bf16`` arithmetic --
    the ``fast_corrected`` route -- adds the +-3 correction as a second MFMA chain),
    and the reference's table contract (``w3_lut_m1_out``: ``row_tile``,
    ``groups_per_split``, split partials summed in order) for routes that split K,
    as ``observed_exact`` does at the gate/up and down shapes.  The dense fallback
    dequantizes with the HIP restore kernel on GPU.

    ``max_packed_rows`` (not in the reference; default 1) lets 2..8-row inputs
    take the MFMA kernel too; they are then counted under ``packed_small_m``.
    """

    def __init__(self, layout: dict, *, bias: torch.Tensor | None = None, fallback: str = "error",
                 row_tile: int | None = None, groups_per_split: int = 1, arithmetic: str = "structural",
                 route: str = "structural", max_packed_rows: int = 1):
        super().__init__()
        self.out_features, self.in_features = validate_planar_w3(layout)
        self.row_tile = qwen3_row_tile(self.out_features, self.in_features) if row_tile is None else row_tile
        if self.row_tile not in ROW_TILES:
            raise ValueError(f"row_tile must be one of {ROW_TILES}")
        _arith_code(arithmetic)
        if arithmetic == "decoded_bf16":
            if layout["scales"].dtype != torch.bfloat16:
                raise ValueError("decoded_bf16 arithmetic requires bf16 scales")
            zeros = layout.get("zeros")
            if zeros is not None and not bool(((zeros == 3) | (zeros == 4)).all()):
                raise ValueError("decoded_bf16 arithmetic supports zero-points 3 and 4")
        if not isinstance(max_packed_rows, int) or not 1 <= max_packed_rows <= MAX_PACKED_ROWS:
            raise ValueError(f"max_packed_rows must be an integer in [1,{MAX_PACKED_ROWS}]")
        workspace_shape(self.out_features, self.in_features, groups_per_split)
        self.max_packed_rows = max_packed_rows
        self._init_protocol(fallback=fallback, bias=bias)
        self.groups_per_split = groups_per_split
        self.arithmetic = arithmetic
        self.route = route
        self._table = None
        self._gemv = None
        perm = layout["perm"]
        self._perm_identity = bool(torch.equal(perm.long().cpu(), torch.arange(self.in_features)))
        self._fields = FIELDS + tuple(f for f in OPTIONAL_FIELDS if f in layout)
        for name in self._fields:
            self.register_buffer(name, layout[name].detach().clone())

    @property
    def uses_table_route(self) -> bool:
        """True when the packed route is the reference's table contract (K split
        into groups_per_split-group partials summed in split order) rather than the
        one-launch MFMA kernel, which serves one group per split in both
        arithmetics (decoded_bf16: the +-3 correction as a second MFMA chain)."""
        return self.groups_per_split != 1

    def layout(self) -> dict:
        return {name: getattr(self, name) for name in self._fields}

    def _payload_device(self) -> torch.device:
        return self.planes.device

    def _dense_weight(self, dtype: torch.dtype) -> torch.Tensor:
        return restore_planar_w3(self.layout(), dtype=dtype, perm_identity=self._perm_identity)

    def _check_before_bind(self, device: torch.device) -> None:
        validate_planar_w3(self.layout(), check_values=False)

    def _forget_kernels(self) -> None:
        self._table = None
        self._gemv = None

    def _packed_kernel(self, rows: int, device: torch.device):
        if rows == 1 and self.uses_table_route:
            if self._table is None or self._table.workspace.device != device:
                self._table = _TableRoute(self, device)
            return self._table
        if self._gemv is None or self._gemv.layout["planes"].data_ptr() != self.planes.data_ptr():
            self._gemv = W3Gemv(self.layout(), arithmetic=self.arithmetic, perm_identity=self._perm_identity,
                                max_rows=self.max_packed_rows)
        return self._gemv


def replace_w3_block_linears(block, layer_payload, *, fallback: str = "error",
                             row_tile_by_shape: dict | None = None, route: str = "structural") -> list[str]:
    """Replace exactly the seven Qwen3 Linears of a block (reference
    ``w3_lut_deployment.py:362-417``); every payload is validated and every module
    built before the block is touched."""
    from .qwen3 import QWEN3_LINEAR_MODULES

    zero_names = {name for name in QWEN3_LINEAR_MODULES if f"{name}.zeros" in layer_payload}
    wanted = {f"{name}.{field}" for name in QWEN3_LINEAR_MODULES for field in FIELDS}
    wanted |= {f"{name}.zeros" for name in zero_names}
    if set(layer_payload) != wanted:
        raise ValueError("layer must contain exactly seven complete W3 payloads")
    if route not in QWEN3_W3_ROUTE_POLICIES:
        raise ValueError(f"unknown Qwen3-8B W3 route: {route}")
    tiles = QWEN3_ROW_TILE_BY_SHAPE if row_tile_by_shape is None else row_tile_by_shape

    def build(name: str) -> PackedW3Linear:
        linear = block.get_submodule(name)
        names = FIELDS + (("zeros",) if name in zero_names else ())
        layout = {field: layer_payload[f"{name}.{field}"] for field in names}
        shape = validate_planar_w3(layout)
        if not isinstance(linear, nn.Linear) or (linear.out_features, linear.in_features) != shape:
            raise ValueError(f"Linear shape/type mismatch: {name}")
        if shape not in tiles:
            raise ValueError(f"row-tile policy missing shape: {shape}")
        policy = {"row_tile": tiles[shape], "groups_per_split": 1, "arithmetic": "structural"}
        if row_tile_by_shape is None:
            policy = qwen3_w3_route(route, *shape)
            if policy["row_tile"] != tiles[shape]:
                raise ValueError("route and row-tile policies disagree")
        return PackedW3Linear(layout, bias=linear.bias, fallback=fallback, route=route,
                              **policy).to(linear.weight.device)

    return replace_linears_atomically(block, [(name, build(name)) for name in QWEN3_LINEAR_MODULES])
