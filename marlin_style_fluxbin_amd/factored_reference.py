"""Float64 structural reference of the hybrid g128/s8 layout and its output gate.

Reference: ``factored_reference.py:8-57`` (``structural_reference``,
``structural_gate``, ``REFERENCE``).  A checker for the packed hybrid route, never
a route itself: ``PackedHybridLinear`` and ``fx_hybrid_gemv`` run on the GPU and
raise without the kernel library; trials compare their output with this.

``structural_reference(x, layout)`` reconstructs one 128-column group at a time
in float64 from the deployment layout (interleaved or planar sign codes): per
base ``sign * row * column`` summed over the two bases, the refinement formed the
same way and added at its eight columns, then dotted with the group's slice of
``x`` and summed over groups.  No bf16 rounding of the weights, and no dense copy
of more than one group.

``structural_gate(actual, expected)`` is ``acceleration_checks.numerical_gate``
with, for a bf16 ``actual``, the reference's looser bars against the float64
output: ``|a - e| <= 0.02 (rms(e) + |e|) + 1e-6`` everywhere and a normalised
RMSE of at most 0.005.
"""
from __future__ import annotations

import torch

from .acceleration_checks import numerical_gate
from .deployment import GROUP, REFINED, _from_planes
from .packing import unpack_two_bases

REFERENCE = "hybrid-structural-fp64-v1"
BF16_ELEMENTWISE_FACTOR = 0.02
BF16_NRMSE_LIMIT = 0.005


def _group_weight(codes: torch.Tensor, rows: torch.Tensor, cols: torch.Tensor) -> torch.Tensor:
    """``[O, width]`` float64: sum over bases of sign * row * column for one group
    (``codes`` interleaved ``[O, width / 4]``, rows ``[O, 2]``, columns ``[width, 2]``)."""
    signs = unpack_two_bases(codes).to(torch.float64)  # [2, O, width]
    rows, cols = rows.to(torch.float64), cols.to(torch.float64)
    return signs[0] * rows[:, 0, None] * cols[None, :, 0] + signs[1] * rows[:, 1, None] * cols[None, :, 1]


@torch.no_grad()
def structural_reference(x: torch.Tensor, layout) -> torch.Tensor:
    """float64 ``[1, O]``: ``x @ W.T`` with W rebuilt group by group in float64."""
    codes = layout["codes"]
    g, o = codes.shape[:2]
    if tuple(x.shape) != (1, g * GROUP):
        raise ValueError("expected [1,G*128]")
    planar = codes.ndim == 4
    sparse = layout["sparse_codes"]
    xd = x.to(torch.float64)
    result = torch.zeros(o, dtype=torch.float64, device=x.device)
    for group in range(g):
        main = _from_planes(codes[group]) if planar else codes[group]
        refine = _from_planes(sparse[group]) if planar else sparse[group]
        w = _group_weight(main, layout["rows"][group], layout["columns"][group])
        delta = _group_weight(refine, layout["sparse_rows"][group], layout["sparse_columns"][group])
        w[:, layout["indices"][group].long()] += delta
        result += w @ xd[0, group * GROUP:(group + 1) * GROUP]
    return result[None, :]


def structural_gate(actual: torch.Tensor, expected: torch.Tensor) -> dict:
    """The output gate of a packed hybrid call against :func:`structural_reference`."""
    gate = numerical_gate(actual, expected)
    if actual.dtype == torch.bfloat16 and gate.get("reference_rms") is not None:
        error = (actual.double() - expected).abs()
        within = bool((error <= BF16_ELEMENTWISE_FACTOR * (gate["reference_rms"] + expected.abs()) + 1e-6).all())
        gate.update(elementwise_tolerance_factor=BF16_ELEMENTWISE_FACTOR, normalized_rmse_limit=BF16_NRMSE_LIMIT,
                    passed=within and gate["normalized_rmse"] <= BF16_NRMSE_LIMIT)
    gate["reference"] = REFERENCE
    return gate


__all__ = ["REFERENCE", "structural_reference", "structural_gate"]
