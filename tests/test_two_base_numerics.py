"""The rank-one two-base kernel's activation fixed point (config 4), emulated on the CPU.

``fx_two_base_gemv`` rounds ``u = t_c * x`` (fp32 product) to ``v = rint(u * 2^F)``
with one exponent per 512-column batch, ``F = min(14 - e, 126)`` for the batch's
``max|u|`` in ``[2^(e-1), 2^e)``, splits ``v`` into two int8 digits ``256 hi + lo``
and multiplies the digits exactly on the int8 matrix cores.  Element ``k`` of batch
``b`` is therefore off by at most ``2^(e_b - 15)``, and row ``o`` by at most

    bound_o = |s_r[o]| (|a1[o]| + |a2[o]|) sum_k 2^(e_b(k) - 15)

(the salient columns are exact bf16 x bf16 products in fp32).  The GPU kernel is
checked against this emulation and this bound in ``tests/test_two_base_gpu.py``.

On an activation outlier (one column ~1e3 among ~1e-2, Qwen3's massive
activations) the bound is wide: every small value of the outlier's batch rounds to
zero.  The emulation also quantifies what per-group exponents (128 columns, the
hybrid kernel's scope) would buy: about half the error on such a batch -- the
outlier's own group still flushes -- so the rank-one format keeps the batch scope
and states its bound; the reference's fp32 tables (``m1_v5.cu:26-104``) flush nothing.
"""
from __future__ import annotations

import numpy as np

from oracle import two_base as tb
from oracle.bf16 import round_bf16

BATCH, GROUP = 512, 128


def _fixed_point(u: np.ndarray, width: int, coarser: int = 0):
    """u rounded as the kernel does with one exponent per ``width`` columns, and
    each element's rounding bound 2^(e - 15); ``coarser`` plants a mistake (an
    exponent that many steps too small)."""
    out = np.empty_like(u)
    bound = np.empty_like(u)
    for s in range(0, u.size, width):
        block = slice(s, min(s + width, u.size))
        m = np.abs(u[block]).max()
        if m == 0:
            out[block] = 0.0
            bound[block] = 0.0
            continue
        e = int(np.frexp(np.float32(m))[1])       # m in [2^(e-1), 2^e)
        f = min(14 - e, 126)
        out[block] = np.rint(u[block] * 2.0 ** (f - coarser)) * 2.0 ** -(f - coarser)
        bound[block] = 2.0 ** (-f - 1)
    return out, bound


def emulate(x: np.ndarray, p: dict, width: int = BATCH, coarser: int = 0):
    """(float64 y[O] of the kernel's integer arithmetic, the row bound) for one
    activation row; ``width`` the exponent's scope in columns."""
    x = np.asarray(x, np.float32)[0]
    u = (x * np.asarray(p["tcol"], np.float32)).astype(np.float64)   # fp32 product, as the kernel
    v, bound = _fixed_point(u, width, coarser)
    signs = tb.rank_one_signs(p["planes"]).astype(np.float64)
    coef = np.asarray(p["coef"], np.float64)
    srow = np.asarray(p["srow"], np.float64)
    y = srow * (coef[0] * (signs[0] @ v) + coef[1] * (signs[1] @ v))
    idx = np.asarray(p["sal_idx"]).astype(np.int64)
    y += np.asarray(p["sal"], np.float64) @ x.astype(np.float64)[idx]
    return y, np.abs(srow) * (np.abs(coef[0]) + np.abs(coef[1])) * bound.sum()


def outlier_case(o=256, k=2048, seed=5, column=17):
    """Config-4-style payload and one bf16 activation row ~1e-2 with one ~1e3
    column; in the first half of the rows a1 = a2 and B1 = -B2 at that column, so
    the outlier cancels there and the small columns are the whole output."""
    p = tb.make_rank_one_payload(o, k, salient=8, seed=seed)
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((1, k)) * 1e-2).astype(np.float32)
    x[0, column] = 1e3
    bases = p["bases"].copy()
    half = o // 2
    bases[1, :half, column] = -bases[0, :half, column]
    p["coef"][1, :half] = p["coef"][0, :half]
    p["planes"] = tb.rank_one_planes(bases)
    p["bases"] = bases
    return p, round_bf16(x)


def test_digit_split_reconstructs_every_16_bit_value():
    """v = 256 hi + lo with lo the signed low byte and hi the next byte of
    rint(u 2^F) + 128 + 1.5 * 2^23 (the kernel's magic-constant rounding): exact for
    every |v| <= 2^14."""
    v = np.arange(-(2 ** 14), 2 ** 14 + 1, dtype=np.int64)
    word = (np.float32(1.5 * 2 ** 23) + (v + 128).astype(np.float32)).view(np.uint32)
    assert np.array_equal((word & 0xFFFF).astype(np.uint16).view(np.int16).astype(np.int64), v + 128)
    lo = ((word & 0xFF) ^ 0x80).astype(np.uint8).view(np.int8).astype(np.int64)
    hi = ((word >> 8) & 0xFF).astype(np.uint8).view(np.int8).astype(np.int64)
    assert np.array_equal(256 * hi + lo, v)


def test_emulation_is_exact_without_rounding_loss():
    # activations whose products with t_c are small integers times 2^-8 round
    # exactly at every scope: the emulation must equal the float64 truth
    p = tb.make_rank_one_payload(40, 1024, salient=3, seed=2)
    p["tcol"][:] = np.float16(1.0)
    x = np.random.default_rng(0).integers(-64, 65, (1, 1024)).astype(np.float32) * 2.0 ** -8
    exact = tb.rank_one_matvec(x, p)[0]
    for width in (BATCH, GROUP):
        y, _ = emulate(x, p, width)
        np.testing.assert_allclose(y, exact, rtol=1e-12, atol=1e-15)


def test_batch_scope_bound_holds_on_an_outlier_and_is_tight():
    p, x = outlier_case()
    exact = tb.rank_one_matvec(x, p)[0]
    y, bound = emulate(x, p, BATCH)
    err = np.abs(y - exact)
    assert np.all(err <= bound)
    # the outlier's batch flushes its 511 other columns: the rows where the outlier
    # cancels lose most of their value, relative to the sum of their terms
    terms = (np.abs(tb.rank_one_weight(p)) * np.abs(x[0].astype(np.float64))).sum(1)
    half = len(y) // 2
    assert np.max(err[:half] / terms[:half]) > 2 ** -7
    # per element: |u' - u| <= 2^(e_b - 15); a planted mistake (each batch's
    # exponent one step too small: 14 bits become 13) breaks it
    u = (x[0] * np.asarray(p["tcol"], np.float32)).astype(np.float64)
    rounded, per_element = _fixed_point(u, BATCH)
    assert np.all(np.abs(rounded - u) <= per_element)
    planted, _ = _fixed_point(u, BATCH, coarser=1)
    assert np.any(np.abs(planted - u) > per_element)


def test_per_group_scope_only_halves_the_outlier_error():
    """What per-group exponents would buy on the outlier case: the error of the
    outlier's batch falls by about half (three of its four groups keep their bits),
    not to the level of the batches without an outlier."""
    p, x = outlier_case()
    exact = tb.rank_one_matvec(x, p)[0]
    batch = np.abs(emulate(x, p, BATCH)[0] - exact)
    group = np.abs(emulate(x, p, GROUP)[0] - exact)
    ratio = float(np.sqrt(np.mean(batch ** 2) / np.mean(group ** 2)))
    assert 1.3 < ratio < 3.0, ratio
    clean = x.copy()
    clean[0, 17] = np.float32(1e-2)
    floor = np.abs(emulate(clean, p, GROUP)[0] - tb.rank_one_matvec(clean, p)[0])
    assert np.sqrt(np.mean(group ** 2)) > 100 * np.sqrt(np.mean(floor ** 2))
