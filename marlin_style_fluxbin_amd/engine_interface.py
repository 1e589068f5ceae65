"""Engine-neutral Linear backends: what a serving adapter needs to run a packed format.

Contract of the reference's ``engine_interface.py`` (``LinearContract`` :15-28,
``LinearBackend`` :31-37, ``M1Backend`` :40-60): a backend owns layout conversion
and the batch-1 Linear op; the serving adapter owns weight loading, streams,
workspaces and scheduling.  The ``LinearContract`` fields keep the reference's
names; their values describe this library on MI355X (``minimum_compute_capability``
is the (major, minor) torch reports for gfx950, ``target_arch`` names it).

Two backends implement the protocol here:

* ``M1Backend`` -- the reference's hybrid g128/s8 two-base format
  (``deployment.m1_out``; ``fx_hybrid_gemv``);
* ``W3Backend`` -- the W3 g128 planar format of the hot path: ``convert`` takes raw
  GPTQ int3 tensors to the planar payload (``convert_gptq_w3_to_planar``),
  ``apply_out`` is ``fx_w3_gemv`` (one MFMA launch at the Qwen3-8B shapes), and the
  workspace is the byte buffer that call asks for.

``backend_for_format`` maps a layout's format string to the backend that serves it.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Mapping, Protocol

import torch

from . import _lib
from . import deployment as hybrid
from .gptq_deployment import FORMAT as W3_FORMAT
from .gptq_deployment import REFERENCE_FORMAT as W3_REFERENCE_FORMAT
from .gptq_deployment import convert_gptq_w3_to_planar, validate_planar_w3


@dataclass(frozen=True)
class LinearContract:
    format: str = hybrid.FORMAT
    supported_m: tuple[int, ...] = (1,)
    input_dtypes: tuple[torch.dtype, ...] = (torch.bfloat16, torch.float16)
    accumulation_dtype: torch.dtype = torch.float32
    scale_dtype: torch.dtype = torch.float32
    group_size: int = 128
    sparse_columns: int = 8
    arithmetic: str = "combined_weight_activation_dtype_v1"
    minimum_compute_capability: tuple[int, int] = (9, 5)
    fused_qkv: bool = False
    tensor_parallel: bool = False
    graph_capture_after_warmup: bool = True
    target_arch: str = field(default="gfx950")


class LinearBackend(Protocol):
    contract: LinearContract

    def convert(self, artifact: Mapping[str, torch.Tensor]) -> dict[str, torch.Tensor]: ...
    def workspace_shape(self, out_features: int, in_features: int) -> tuple[int, ...]: ...
    def apply_out(self, x: torch.Tensor, layout: Mapping[str, torch.Tensor],
                  out: torch.Tensor, workspace: torch.Tensor) -> torch.Tensor: ...


class M1Backend:
    """Hybrid g128/s8 two-base backend (``deployment.m1_out``)."""

    contract = LinearContract()

    def __init__(self, groups_per_split=8, *, kernel="v1"):
        if kernel not in hybrid.KERNELS:
            raise ValueError(f"kernel must be one of {hybrid.KERNELS}")
        if not isinstance(groups_per_split, int) or not 1 <= groups_per_split <= 1024:
            raise ValueError("groups_per_split must be 1..1024")
        self.kernel = kernel
        self.groups_per_split = groups_per_split
        if kernel in hybrid.FACTORED_KERNELS:
            planar = kernel in hybrid.PLANAR_KERNELS
            self.contract = LinearContract(arithmetic="factored_fp32_v1",
                                           format=hybrid.PLANAR_FORMAT if planar else hybrid.FORMAT)

    def convert(self, artifact):
        return hybrid.convert_artifact(artifact, kernel=self.kernel)

    def workspace_shape(self, out_features, in_features):
        return hybrid.workspace_shape(out_features, in_features, self.groups_per_split, kernel=self.kernel)

    def apply_out(self, x, layout, out, workspace):
        return hybrid.m1_out(x, layout, out, workspace, groups_per_split=self.groups_per_split, kernel=self.kernel)


class W3Backend:
    """W3 g128 planar backend (``fx_w3_gemv``): structural fp32 arithmetic, 1..8 rows."""

    contract = LinearContract(format=W3_REFERENCE_FORMAT, supported_m=(1, 2, 3, 4, 5, 6, 7, 8),
                              scale_dtype=torch.bfloat16, sparse_columns=0, arithmetic="structural_fp32_v1",
                              fused_qkv=True)

    def __init__(self, *, scale_dtype: torch.dtype = torch.bfloat16, allow_zeros: bool = False):
        self.scale_dtype = scale_dtype
        self.allow_zeros = allow_zeros
        if allow_zeros or scale_dtype != torch.bfloat16:
            self.contract = LinearContract(format=W3_FORMAT, supported_m=W3Backend.contract.supported_m,
                                           scale_dtype=scale_dtype, sparse_columns=0,
                                           arithmetic="structural_fp32_v1", fused_qkv=True)

    def convert(self, artifact):
        """Raw GPTQ int3 tensors (``qweight``, ``qzeros``, ``scales``, ``g_idx``) -> planar payload."""
        return convert_gptq_w3_to_planar(artifact, qzero_format=1, scale_dtype=self.scale_dtype,
                                         allow_zeros=self.allow_zeros)

    def workspace_shape(self, out_features, in_features):
        """Bytes (uint8) of the largest workspace ``apply_out`` needs for up to 8 rows."""
        lib = _lib.library()
        need = max(lib.fx_w3_gemv_workspace_bytes(m, out_features, in_features) for m in range(1, 9))
        return (max(int(need), 256),)

    def apply_out(self, x, layout, out, workspace):
        o, k = validate_planar_w3(layout, check_values=False)
        m = x.shape[0]
        if x.ndim != 2 or x.shape[1] != k or tuple(out.shape) != (m, o) or out.dtype != x.dtype:
            raise ValueError("x [M,K] and out [M,O] in one dtype required")
        perm = layout["perm"]
        _lib.check(_lib.library().fx_w3_gemv(
            x.data_ptr(), _lib.dtype_code(x.dtype), layout["planes"].data_ptr(), layout["scales"].data_ptr(),
            _lib.dtype_code(layout["scales"].dtype), _lib.ptr(layout.get("zeros")), perm.data_ptr(),
            workspace.data_ptr(), workspace.numel() * workspace.element_size(), out.data_ptr(), m, o, k,
            _lib.ARITH_STRUCTURAL, _lib.stream_handle(x.device)), "fx_w3_gemv")
        return out


def backend_for_format(format_name: str, **options):
    """The backend serving a layout format string (``layout_storage()['format']`` for
    W3 payloads, ``deployment.layout_format`` for hybrid layouts)."""
    if format_name in (W3_FORMAT, W3_REFERENCE_FORMAT):
        return W3Backend(**options)
    if format_name == hybrid.PLANAR_FORMAT:
        return M1Backend(kernel=options.pop("kernel", "v5_p1024"), **options)
    if format_name == hybrid.FORMAT:
        return M1Backend(**options)
    raise ValueError(f"no backend for format {format_name!r}")
