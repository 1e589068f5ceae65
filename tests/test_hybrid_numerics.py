"""The hybrid two-base kernel's activation fixed point, emulated on the CPU.

``fx_hybrid_gemv`` rounds each product ``u = x * cols[g, k, b]`` to an integer
``v = rint(u * 2^F)`` with ``max|u| * 2^F`` in ``[2^13, 2^14)`` and multiplies the
integers exactly on the int8 matrix cores.  The rounding costs at most
``2^-14 max|u|`` per element of the exponent's scope, so row ``o`` of the output is
off by at most ``2^-7 sum_{g,b} |rows[g,o,b]| max_g |u_b|`` (128 elements per group)
when the scope is one (group, base) -- bounded by ``2^-7 B_o`` with
``B_o = sum_{g,b} |rows[g,o,b]| sum_k |u_b[k]|`` (plus the refinement's terms).

With one exponent per four-group batch (the kernel's first form) an outlier in
one group coarsened its neighbours, whose own rows could dominate the output:
the emulation below shows that form breaking the per-element bound on an outlier
activation (one column ~1e3 in a group whose row scales are tiny, the rest
~1e-2) and the per-group form keeping it.  ``tests/test_hybrid_gpu.py`` runs the
same case through the GPU kernel.
"""
from __future__ import annotations

import numpy as np

from oracle import two_base as tb

GROUP, REFINED = 128, 8


def _fixed_point(u: np.ndarray, axis_groups: list[np.ndarray]) -> np.ndarray:
    """u rounded as the kernel does, one exponent per index set in ``axis_groups``."""
    out = np.empty_like(u)
    for idx in axis_groups:
        m = np.abs(u[idx]).max()
        if m == 0:
            out[idx] = 0.0
            continue
        e = int(np.frexp(np.float32(m))[1])       # m in [2^(e-1), 2^e)
        f = min(14 - e, 126)
        out[idx] = np.rint(u[idx] * 2.0 ** f) * 2.0 ** -f
    return out


def emulate(x: np.ndarray, layout: dict, scope: str) -> np.ndarray:
    """float64 y[O] of the kernel's integer arithmetic with exponents per (group,
    base) (``scope='group'``) or per (4-group batch, base) (``'batch'``)."""
    x = np.asarray(x, np.float32)[0]
    codes = layout["codes"]
    g_count, o = codes.shape[:2]
    signs = tb._layout_signs(codes, GROUP)                   # [G, O, 128, 2]
    rsigns = tb._layout_signs(layout["sparse_codes"], REFINED)  # [G, O, 8, 2]
    cols = np.asarray(layout["columns"], np.float32)          # [G, 128, 2]
    scols = np.asarray(layout["sparse_columns"], np.float32)  # [G, 8, 2]
    rows = np.asarray(layout["rows"], np.float64)             # [G, O, 2]
    srows = np.asarray(layout["sparse_rows"], np.float64)
    idx = np.asarray(layout["indices"]).astype(np.int64)
    y = np.zeros(o, np.float64)
    for b in range(2):
        u = np.concatenate([(x[g * GROUP:(g + 1) * GROUP] * cols[g, :, b]).astype(np.float32)
                            for g in range(g_count)]).astype(np.float64)
        ur = np.concatenate([(x[g * GROUP + idx[g]] * scols[g, :, b]).astype(np.float32)
                             for g in range(g_count)]).astype(np.float64)
        if scope == "group":
            sets = [np.arange(g * GROUP, (g + 1) * GROUP) for g in range(g_count)]
            rsets = [np.arange(g * REFINED, (g + 1) * REFINED) for g in range(g_count)]
        else:
            sets = [np.arange(s * GROUP, min(s + 4, g_count) * GROUP) for s in range(0, g_count, 4)]
            rsets = [np.arange(s * REFINED, min(s + 4, g_count) * REFINED) for s in range(0, g_count, 4)]
        v = _fixed_point(u, sets)
        vr = _fixed_point(ur, rsets)
        for g in range(g_count):
            y += rows[g, :, b] * (signs[g, :, :, b] @ v[g * GROUP:(g + 1) * GROUP])
            y += srows[g, :, b] * (rsigns[g, :, :, b] @ vr[g * REFINED:(g + 1) * REFINED])
    return y


def row_bound(x: np.ndarray, layout: dict) -> np.ndarray:
    """2^-7 B_o for every output row (the per-group fixed-point bound)."""
    x = np.asarray(x, np.float64)[0]
    rows = np.abs(np.asarray(layout["rows"], np.float64))
    srows = np.abs(np.asarray(layout["sparse_rows"], np.float64))
    cols = np.abs(np.asarray(layout["columns"], np.float64))
    scols = np.abs(np.asarray(layout["sparse_columns"], np.float64))
    idx = np.asarray(layout["indices"]).astype(np.int64)
    total = np.zeros(rows.shape[1])
    for g in range(rows.shape[0]):
        xg = np.abs(x[g * GROUP:(g + 1) * GROUP])
        for b in range(2):
            total += rows[g, :, b] * float(xg @ cols[g, :, b]) + srows[g, :, b] * float(xg[idx[g]] @ scols[g, :, b])
    return 2.0 ** -7 * total


def outlier_case(o=64, g=4, seed=5):
    """A payload and activation where group 0 holds one ~1e3 outlier but tiny row
    scales, and the other groups hold ~1e-2 activations with ordinary rows."""
    p = tb.make_hybrid_payload(o, g, seed=seed)
    p["global_row_scales"][:, :, 0] *= 1e-6
    p["refinement_row_scales"][:, :, 0] *= 1e-6
    layout = tb.convert_artifact(p, planar=True)
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((1, g * GROUP)) * 1e-2).astype(np.float32)
    x[0, 17] = 1e3
    from oracle.bf16 import round_bf16
    return p, layout, round_bf16(x)


def test_per_group_exponents_keep_the_bound_on_an_outlier():
    _, layout, x = outlier_case()
    exact = tb.structural_reference(x, layout)[0]
    bound = row_bound(x, layout) + 1e-12
    group = emulate(x, layout, "group")
    batch = emulate(x, layout, "batch")
    assert np.all(np.abs(group - exact) <= bound)
    # the batch-wide exponent loses the small groups' bits: far outside the bound
    assert np.max(np.abs(batch - exact) / bound) > 4.0


def test_emulation_is_exact_without_rounding_loss():
    # activations that are small integers times a power of two round exactly in
    # both scopes: the emulation must then equal the float64 structural truth
    p = tb.make_hybrid_payload(16, 4, seed=2)
    p["global_column_scales"][:] = 1.0
    p["refinement_column_scales"][:] = 1.0
    layout = tb.convert_artifact(p, planar=True)
    x = np.random.default_rng(0).integers(-8, 9, (1, 512)).astype(np.float32) * 0.25
    exact = tb.structural_reference(x, layout)[0]
    for scope in ("group", "batch"):
        np.testing.assert_allclose(emulate(x, layout, scope), exact, rtol=1e-12, atol=1e-12)
