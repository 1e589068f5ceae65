"""Seeded synthetic payloads shared by the tests (not a test module).

``synthetic_raw`` follows the generator of the reference's
``tests/test_gptq_w3_planar.py:21-39`` (same seed, same draw order), so the raw
GPTQ tensors equal the ones the reference's own tests use.  ``config_codes``
draws the benchmark configs' distributions (codes U{0..7}, fp16 scales
U[0.005,0.02], zero-points U{3,4}).
"""
from __future__ import annotations

import numpy as np
import torch

from marlin_style_fluxbin_amd.gptq_deployment import pack_gptq_w3_codes


def synthetic_raw(*, k=256, o=64, seed=20260916, zero=4):
    generator = torch.Generator().manual_seed(seed)
    codes = torch.randint(0, 8, (k, o), generator=generator, dtype=torch.uint8)
    groups = k // 128
    zeros = torch.full((groups, o), zero, dtype=torch.uint8)
    scales = (torch.rand((groups, o), generator=generator) * 0.125 + 0.001).half()
    activation_order = torch.randperm(k, generator=generator)
    g_idx = torch.empty(k, dtype=torch.int32)
    g_idx[activation_order] = torch.arange(groups, dtype=torch.int32).repeat_interleave(128)
    raw = {
        "qweight": pack_gptq_w3_codes(codes),
        "qzeros": pack_gptq_w3_codes(((zeros.to(torch.int16) - 1) & 7).to(torch.uint8), packed_axis=1),
        "scales": scales,
        "g_idx": g_idx,
    }
    return raw, codes, zeros


def config_codes(o: int, k: int, *, seed: int = 0, zeros: bool = True, scale_dtype=torch.float16,
                 permute: bool = False):
    """Original-order codes [K,O] uint8, scales [G,O], zeros [G,O] or None, perm or None."""
    generator = torch.Generator().manual_seed(seed)
    groups = k // 128
    codes = torch.randint(0, 8, (k, o), generator=generator, dtype=torch.uint8)
    scales = (torch.rand((groups, o), generator=generator) * 0.015 + 0.005).to(scale_dtype)
    zero = torch.randint(3, 5, (groups, o), generator=generator, dtype=torch.uint8) if zeros else None
    perm = None
    if permute:
        # a desc_act-style permutation: each sorted position reads a scattered column
        perm = torch.randperm(k, generator=generator).to(torch.int16)
    return codes, scales, zero, perm


def outlier_activations(m: int, k: int, *, ratio: float, seed: int, channels, dtype=torch.bfloat16):
    """[m, k] activations N(0, 1) * 1e-2 with `channels` at +-ratio * 1e-2 (sign and
    size varying per row) and the two columns after the first channel exactly
    zero: Qwen3's massive activations sit in a few channels of otherwise small rows."""
    generator = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=generator) * 1e-2
    for i, c in enumerate(channels):
        sign = torch.where(torch.rand(m, generator=generator) < 0.5, -1.0, 1.0)
        x[:, c] = sign * ratio * 1e-2 * (1.0 - 0.25 * (i % 3))
    x[:, channels[0] + 1: channels[0] + 3] = 0.0
    return x.to(dtype)


def silence_columns(codes, zeros, perm, columns, rows) -> None:
    """Make the weights of original columns `columns` exactly zero in output rows
    `rows` (code = the zero-point of the column's sorted group, 4 without
    zero-points), in place on the [K, O] codes."""
    k = codes.shape[0]
    position = np.empty(k, dtype=np.int64)
    order = np.arange(k) if perm is None else perm.numpy().astype(np.int64)
    position[order] = np.arange(k)
    for c in columns:
        g = int(position[c]) // 128
        z = torch.full((len(rows),), 4, dtype=torch.uint8) if zeros is None else zeros[g, rows]
        codes[c, rows] = z


def assert_within_terms(actual, exact, dtype: str, x, scales, factor: float, what: str = "") -> None:
    """Element-wise: |actual - exact| <= half an ulp of the output dtype at exact,
    plus factor * 11 * max(s) * sum_k |x[m, k]| for activation row m.  The kernels
    apply the zero-point as z * sum(x) beside the unsigned dot sum(q x) of each
    (group, row), so their fp32 rounding scales with those terms (bounded by
    11 max(s) sum|x|, q <= 7 and z <= 4), not with |y|: a row whose weights
    cancel an outlier channel is held to its terms' scale, not to the outlier
    rows' max|y|."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(exact, dtype=np.float64)
    mantissa = 7 if dtype == "bf16" else 10
    exponent = np.floor(np.log2(np.maximum(np.abs(e), 1e-30)))
    terms = 11.0 * float(scales.float().abs().max()) * np.abs(x.float().numpy()).sum(axis=1, keepdims=True)
    bound = 2.0 ** (exponent - mantissa - 1) + factor * terms
    excess = np.abs(a - e) - bound
    worst = int(np.argmax(excess))
    assert excess.max() <= 0, (f"{what} element {worst}: |{a.flat[worst]} - {e.flat[worst]}| exceeds "
                               f"bound {bound.flat[worst]:.3g}")


def layout_from_codes(codes, scales, zeros, perm):
    """Planar layout (torch, CPU) for original-order codes.

    The planes come from the oracle's packer (``oracle.w3.planar_from_codes``,
    pinned by brute force over every byte value and code position), not from
    the product's, so a packer mistake in the product cannot hide behind planes
    that both the kernels and the truth read; ``tests/test_gptq_deployment.py``
    pins the product's packer against the oracle separately.
    """
    from oracle import w3

    k = codes.shape[0]
    perm_t = torch.arange(k, dtype=torch.int16) if perm is None else perm
    planes = w3.planar_from_codes(codes.numpy(), perm_t.numpy().astype(np.int64))
    layout = {
        "planes": torch.from_numpy(planes),
        "scales": scales.contiguous(),
        "perm": perm_t.contiguous(),
    }
    if zeros is not None:
        layout["zeros"] = zeros.contiguous()
    return layout


def oracle_layout(layout):
    """numpy view of a torch layout for the oracle."""
    scales = layout["scales"]
    return {
        "planes": layout["planes"].cpu().numpy(),
        "scales": scales.float().cpu().numpy(),
        "scale_dtype": "bf16" if scales.dtype == torch.bfloat16 else "f16",
        "perm": layout["perm"].cpu().numpy(),
        "zeros": None if layout.get("zeros") is None else layout["zeros"].cpu().numpy(),
    }


def max_rel(actual, expected) -> float:
    """Normwise max relative error max|a-b| / max|b| in float64."""
    a = np.asarray(actual, dtype=np.float64)
    b = np.asarray(expected, dtype=np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def assert_rel(actual, expected, tol: float, what: str = "") -> float:
    """Assert the normwise max relative error, with a short failure message."""
    err = max_rel(actual, expected)
    assert err <= tol, f"{what} max_rel {err:.4g} > {tol:.4g}"
    return err


def assert_half_ulp(actual, exact, dtype: str, rel_slack: float = 2e-6, what: str = "") -> None:
    """Element-wise: |actual - exact| <= half an ulp of the output dtype at exact,
    plus rel_slack * max|exact| for the fp32 accumulation before the final cast."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(exact, dtype=np.float64)
    mantissa = 7 if dtype == "bf16" else 10
    exponent = np.floor(np.log2(np.maximum(np.abs(e), 1e-30)))
    bound = 2.0 ** (exponent - mantissa - 1) + rel_slack * np.abs(e).max()
    excess = np.abs(a - e) - bound
    worst = int(np.argmax(excess))
    assert excess.max() <= 0, (f"{what} element {worst}: |{a.flat[worst]} - {e.flat[worst]}| exceeds "
                               f"half-ulp bound {bound.flat[worst]:.3g}")
