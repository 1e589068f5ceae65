"""numpy restatement of the two-base binary-basis GEMV formats (config 4).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Two payload formats are covered.

Hybrid g128/s8 (the reference's deployment format, ``deployment.py:18-121``):
global two-base rank-one weight per 128-column group plus an 8-column two-base
refinement per group,

    W[o, 128g + k] = sum_b B_b[o, 128g + k] * rows_b[o, g] * cols_b[g, k]
                     + [k = idx[g, j]] sum_b R_b[o, 8g + j] * srows_b[o, g] * scols_b[g, j]

with ``B, R`` in {-1, +1}.  Packed artifact: ``global_sign_codes`` uint8 ``[O, K/4]``
(two bases interleaved, ``packing.py:14-32``), fp32 scales, int16 sorted indices.
Deployment layout (``convert_artifact``, ``deployment.py:84-103``): groups first,
and for the planar kernels each 32-byte interleaved row becomes two 16-byte bit
planes (``_to_planes``, ``deployment.py:59-67``).

Rank-one two-base with salient columns (the benchmark's config 4):

    W[o, k] = s_r[o] * t_c[k] * (a1[o] * B1[o, k] + a2[o] * B2[o, k])
              + sum_j [k = sal_idx[j]] * sal[o, j]

``a1, a2, s_r, t_c`` fp16, ``sal`` bf16 ``[O, S]``, ``sal_idx`` int32 ``[S]`` distinct.
Signs are stored as ``planes[g, o, b, :]`` (16 bytes per group, row and base) in
stride-16 order: column ``128 g + k`` is bit ``k >> 4`` of byte ``k & 15``
(1 = +1), so each bit position of the 16 bytes holds 16 consecutive columns.

How each function is pinned:

* ``pack_two_bases`` / ``unpack_two_bases``: the reference's bit-order KAT
  ``0b11100100`` (``tests/test_packing.py:23-35``) and round trips.
* ``to_planes`` / ``from_planes``: all 65536 interleaved 16-bit words against the
  bit-by-bit definition (``tests/test_planar_layout.py:14-24``).
* ``materialize_hybrid``: bitwise against a scalar loop that performs the same
  fp32 operations element by element on small shapes, and to fp32 rounding
  against the float64 closed form.
* ``structural_reference``: against the independent factored dot of
  ``tests/test_factored_reference.py:10-25`` (signs x (x * cols) summed, times
  rows) and against the dense materialization in float64.
* ``rank_one_matvec``: against the dense float64 ``rank_one_weight`` @ x and the
  factored closed form s_r * (a1 * (B1 . (t x)) + a2 * (B2 . (t x))) + sal . x[idx].
"""
from __future__ import annotations

import numpy as np

FIELDS = ("global_sign_codes", "global_row_scales", "global_column_scales",
          "refinement_indices", "refinement_sign_codes",
          "refinement_row_scales", "refinement_column_scales")
LAYOUT_FIELDS = ("codes", "rows", "columns", "indices", "sparse_codes",
                 "sparse_rows", "sparse_columns", "lookup")
GROUP = 128
REFINED = 8  # refinement columns per group


# --------------------------------------------------------------------------- packing


def pack_two_bases(bases) -> np.ndarray:
    """[2, O, K] signs in {-1, +1} -> uint8 [O, K/4]; column ``4q + i`` of base ``b``
    is bit ``2i + b`` of byte ``q`` (``packing.py:14-32``)."""
    bases = np.asarray(bases)
    if bases.ndim != 3 or bases.shape[0] != 2:
        raise ValueError("bases must have shape [2, out_features, in_features]")
    if bases.shape[-1] % 4:
        raise ValueError("in_features must be divisible by four")
    if not np.all((bases == -1) | (bases == 1)):
        raise ValueError("bases must contain only -1 and +1")
    o, k = bases.shape[1:]
    bits = (bases > 0).astype(np.uint8).reshape(2, o, k // 4, 4)
    out = np.zeros((o, k // 4), np.uint8)
    for i in range(4):
        out |= bits[0, :, :, i] << (2 * i)
        out |= bits[1, :, :, i] << (2 * i + 1)
    return out


def unpack_two_bases(codes) -> np.ndarray:
    """Inverse of :func:`pack_two_bases` -> int8 ``[2, O, K]`` (``packing.py:35-49``)."""
    codes = np.asarray(codes)
    if codes.ndim != 2 or codes.dtype != np.uint8:
        raise ValueError("codes must be a uint8 array shaped [out_features, K/4]")
    o, q = codes.shape
    out = np.empty((2, o, q, 4), np.int8)
    for i in range(4):
        for b in range(2):
            out[b, :, :, i] = ((codes >> (2 * i + b)) & 1).astype(np.int8) * 2 - 1
    return out.reshape(2, o, 4 * q)


def to_planes(codes) -> np.ndarray:
    """Interleaved bytes ``[..., 2n]`` -> planes ``[..., 2, n]``.

    Planar byte ``c`` of base ``b`` holds columns ``8c .. 8c+7`` (bit ``j`` =
    column ``8c + j``); in the interleaved form column ``8c + j`` is bit
    ``2 (j % 4) + b`` of byte ``2c + j // 4`` (``deployment.py:59-67``)."""
    codes = np.asarray(codes, np.uint8)
    n = codes.shape[-1] // 2
    out = np.zeros(codes.shape[:-1] + (2, n), np.uint8)
    for j in range(8):
        src = codes[..., (j // 4)::2]
        for b in range(2):
            out[..., b, :] |= ((src >> (2 * (j % 4) + b)) & 1) << j
    return out


def from_planes(planes) -> np.ndarray:
    """Inverse of :func:`to_planes` (``deployment.py:70-77``)."""
    planes = np.asarray(planes, np.uint8)
    n = planes.shape[-1]
    out = np.zeros(planes.shape[:-2] + (2 * n,), np.uint8)
    for j in range(8):
        for b in range(2):
            bit = (planes[..., b, :] >> j) & 1
            out[..., (j // 4)::2] |= bit << (2 * (j % 4) + b)
    return out


# --------------------------------------------------------------------------- hybrid format


def validate_artifact(p) -> tuple[int, int]:
    """Shape / dtype contract of the seven payload fields (``deployment.py:30-55``);
    returns ``(O, G)``."""
    if set(p) != set(FIELDS):
        raise ValueError("expected exactly seven hybrid payload fields")
    codes = np.asarray(p["global_sign_codes"])
    if codes.ndim != 2 or codes.dtype != np.uint8:
        raise ValueError("global codes must be uint8 [O,K/4]")
    o, width = codes.shape
    if o < 1 or o > 65536 or width < 32 or width > 32768 or width % 32:
        raise ValueError("requires O=1..65536 and K=128..131072 divisible by 128")
    g = width // 32
    shapes = ((o, width), (2, o, g), (2, g, GROUP), (g, REFINED), (o, g * 2), (2, o, g), (2, g, REFINED))
    for name, shape in zip(FIELDS, shapes):
        t = np.asarray(p[name])
        if t.shape != shape:
            raise ValueError(f"shape mismatch: {name}")
        if "scales" in name and (t.dtype != np.float32 or not np.all(np.isfinite(t))):
            raise ValueError(f"finite FP32 scales required: {name}")
    if np.asarray(p["refinement_sign_codes"]).dtype != np.uint8:
        raise ValueError("refinement codes must be uint8")
    ix = np.asarray(p["refinement_indices"])
    if ix.dtype not in (np.int16, np.int32, np.int64):
        raise ValueError("integer refinement indices required")
    if np.any(ix < 0) or np.any(ix >= GROUP) or np.any(ix[:, 1:] <= ix[:, :-1]):
        raise ValueError("indices must be sorted, unique and inside each group")
    return o, g


def convert_artifact(p, *, planar: bool = True) -> dict:
    """Artifact -> deployment layout (``deployment.py:84-103``): group-major codes
    ``[G, O, 32]`` (planar: ``[G, O, 2, 16]``), rows ``[G, O, 2]``, columns
    ``[G, 128, 2]``, indices int16 ``[G, 8]``, sparse codes ``[G, O, 2]`` (planar
    ``[G, O, 2, 1]``), sparse rows ``[G, O, 2]``, sparse columns ``[G, 8, 2]`` and
    ``lookup`` int16 ``[G, 128]`` (-1 or the refinement slot of each column)."""
    o, g = validate_artifact(p)
    ix = np.asarray(p["refinement_indices"]).astype(np.int16)
    lookup = np.full((g, GROUP), -1, np.int16)
    for gi in range(g):
        lookup[gi, ix[gi].astype(np.int64)] = np.arange(REFINED, dtype=np.int16)
    out = {
        "codes": np.ascontiguousarray(np.asarray(p["global_sign_codes"]).reshape(o, g, 32).transpose(1, 0, 2)),
        "rows": np.ascontiguousarray(np.asarray(p["global_row_scales"]).transpose(2, 1, 0)),
        "columns": np.ascontiguousarray(np.asarray(p["global_column_scales"]).transpose(1, 2, 0)),
        "indices": ix.copy(),
        "sparse_codes": np.ascontiguousarray(np.asarray(p["refinement_sign_codes"]).reshape(o, g, 2).transpose(1, 0, 2)),
        "sparse_rows": np.ascontiguousarray(np.asarray(p["refinement_row_scales"]).transpose(2, 1, 0)),
        "sparse_columns": np.ascontiguousarray(np.asarray(p["refinement_column_scales"]).transpose(1, 2, 0)),
        "lookup": lookup,
    }
    if planar:
        out["codes"] = to_planes(out["codes"])
        out["sparse_codes"] = to_planes(out["sparse_codes"])
    return out


def restore_artifact(layout) -> dict:
    """Inverse of :func:`convert_artifact` (``deployment.py:106-115``)."""
    codes, sparse = np.asarray(layout["codes"]), np.asarray(layout["sparse_codes"])
    g, o = codes.shape[:2]
    if codes.ndim == 4:
        codes, sparse = from_planes(codes), from_planes(sparse)
    return {
        "global_sign_codes": np.ascontiguousarray(codes.transpose(1, 0, 2).reshape(o, g * 32)),
        "global_row_scales": np.ascontiguousarray(np.asarray(layout["rows"]).transpose(2, 1, 0)),
        "global_column_scales": np.ascontiguousarray(np.asarray(layout["columns"]).transpose(2, 0, 1)),
        "refinement_indices": np.asarray(layout["indices"]).copy(),
        "refinement_sign_codes": np.ascontiguousarray(sparse.transpose(1, 0, 2).reshape(o, g * 2)),
        "refinement_row_scales": np.ascontiguousarray(np.asarray(layout["sparse_rows"]).transpose(2, 1, 0)),
        "refinement_column_scales": np.ascontiguousarray(np.asarray(layout["sparse_columns"]).transpose(2, 0, 1)),
    }


def materialize_hybrid(p) -> np.ndarray:
    """Dense fp32 weight ``[O, K]`` with the reference's fp32 operation order
    (``evaluation.py:59-175``): per base ``(sign * row) * col``, the two base terms
    added to a zero start in base order, the refinement formed the same way and
    added at its columns.  Cast with :mod:`oracle.bf16` helpers for bf16 / fp16."""
    o, g = validate_artifact(p)
    bases = unpack_two_bases(np.asarray(p["global_sign_codes"])).reshape(2, o, g, GROUP).astype(np.float32)
    rows = np.asarray(p["global_row_scales"], np.float32)
    cols = np.asarray(p["global_column_scales"], np.float32)
    w = np.zeros((o, g, GROUP), np.float32)
    for b in range(2):
        term = bases[b] * rows[b][:, :, None]
        term = term * cols[b][None, :, :]
        w = w + term
    ref = unpack_two_bases(np.asarray(p["refinement_sign_codes"])).reshape(2, o, g, REFINED).astype(np.float32)
    srows = np.asarray(p["refinement_row_scales"], np.float32)
    scols = np.asarray(p["refinement_column_scales"], np.float32)
    sel = np.zeros((o, g, REFINED), np.float32)
    for b in range(2):
        term = ref[b] * srows[b][:, :, None]
        term = term * scols[b][None, :, :]
        sel = sel + term
    idx = np.asarray(p["refinement_indices"]).astype(np.int64)
    for gi in range(g):
        w[:, gi, idx[gi]] = w[:, gi, idx[gi]] + sel[:, gi, :]
    return w.reshape(o, g * GROUP)


def _layout_signs(codes, width):
    """Signs ``[G, O, width, 2]`` (float64) from interleaved or planar layout codes."""
    codes = np.asarray(codes)
    k = np.arange(width)
    if codes.ndim == 4:
        bits = [(codes[:, :, b, :][:, :, k // 8].astype(np.int64) >> (k % 8)) & 1 for b in range(2)]
    else:
        q = codes[:, :, k // 4].astype(np.int64) >> (2 * (k % 4))
        bits = [q & 1, (q >> 1) & 1]
    return np.stack(bits, axis=-1).astype(np.float64) * 2 - 1


def structural_reference(x, layout) -> np.ndarray:
    """float64 ``y[1, O]`` from the deployment layout (``factored_reference.py:8-42``):
    per group the dense float64 weight (signs x rows x columns, plus the refinement
    at its columns) dotted with x."""
    x = np.asarray(x, np.float64)
    codes = np.asarray(layout["codes"])
    g, o = codes.shape[:2]
    if x.shape != (1, g * GROUP):
        raise ValueError("expected [1,G*128]")
    signs = _layout_signs(codes, GROUP)
    ss = _layout_signs(layout["sparse_codes"], REFINED)
    rows = np.asarray(layout["rows"], np.float64)
    cols = np.asarray(layout["columns"], np.float64)
    srows = np.asarray(layout["sparse_rows"], np.float64)
    scols = np.asarray(layout["sparse_columns"], np.float64)
    idx = np.asarray(layout["indices"]).astype(np.int64)
    y = np.zeros(o, np.float64)
    for gi in range(g):
        w = (signs[gi] * rows[gi][:, None, :] * cols[gi][None, :, :]).sum(-1)
        delta = (ss[gi] * srows[gi][:, None, :] * scols[gi][None, :, :]).sum(-1)
        w[:, idx[gi]] += delta
        y += w @ x[0, gi * GROUP:(gi + 1) * GROUP]
    return y[None, :]


def hybrid_storage_bytes(o: int, k: int) -> int:
    """Bytes the planar kernels read per call, excluding x/y: codes, fp32 rows,
    fp32 columns, int16 indices, refinement codes / rows / columns."""
    g = k // GROUP
    return g * o * 32 + g * o * 8 + g * GROUP * 8 + g * REFINED * 2 + g * o * 2 + g * o * 8 + g * REFINED * 8


def make_hybrid_payload(o: int, g: int, seed: int = 19) -> dict:
    """Random hybrid payload with the distributions of the reference's tests
    (``tests/test_deployment.py:12-22``): random signs, row scales ~N(0, 0.1) /
    N(0, 0.07), column scales ~N(0, 1), sorted distinct refinement columns."""
    rng = np.random.default_rng(seed)

    def signs(k):
        return pack_two_bases(rng.integers(0, 2, (2, o, k)) * 2 - 1)

    idx = np.stack([np.sort(rng.permutation(GROUP)[:REFINED]) for _ in range(g)]).astype(np.int16)
    return {
        "global_sign_codes": signs(g * GROUP),
        "global_row_scales": (rng.standard_normal((2, o, g)) * 0.1).astype(np.float32),
        "global_column_scales": rng.standard_normal((2, g, GROUP)).astype(np.float32),
        "refinement_indices": idx,
        "refinement_sign_codes": signs(g * REFINED),
        "refinement_row_scales": (rng.standard_normal((2, o, g)) * 0.07).astype(np.float32),
        "refinement_column_scales": rng.standard_normal((2, g, REFINED)).astype(np.float32),
    }


# --------------------------------------------------------------------------- rank-one format (config 4)


def rank_one_planes(bases) -> np.ndarray:
    """Signs ``[2, O, K]`` -> ``[G, O, 2, 16]`` uint8: column ``128 g + k`` of base
    ``b`` is bit ``k >> 4`` of byte ``k & 15`` of row ``planes[g, o, b]``."""
    bases = np.asarray(bases)
    _, o, k = bases.shape
    if k % GROUP:
        raise ValueError("K must be a multiple of 128")
    bits = (bases > 0).astype(np.uint8).reshape(2, o, k // GROUP, 8, 16)  # [..., k >> 4, k & 15]
    out = np.zeros((2, o, k // GROUP, 16), np.uint8)
    for i in range(8):
        out |= bits[:, :, :, i, :] << i
    return np.ascontiguousarray(out.transpose(2, 1, 0, 3))


def rank_one_signs(planes) -> np.ndarray:
    """Inverse of :func:`rank_one_planes` -> int8 ``[2, O, K]``."""
    planes = np.asarray(planes, np.uint8)
    g, o = planes.shape[:2]
    bits = np.stack([(planes >> i) & 1 for i in range(8)], axis=-2)  # [G, O, 2, 8 (k >> 4), 16 (k & 15)]
    return (bits.transpose(2, 1, 0, 3, 4).reshape(2, o, g * GROUP).astype(np.int8) * 2 - 1)


def make_rank_one_payload(o: int, k: int, *, salient: int = 32, seed: int = 0) -> dict:
    """Config-4 synthetic payload: random +-1 bases, a1/a2 ~U[0.5, 1.5], s_r
    ~U[0.005, 0.02], t_c ~U[0.8, 1.2] (all fp16), ``salient`` distinct columns with
    bf16 values ~N(0, 0.05).  Returns float arrays holding the exactly
    representable stored values plus the planar signs."""
    from . import bf16

    rng = np.random.default_rng(seed)
    bases = rng.integers(0, 2, (2, o, k)).astype(np.int8) * 2 - 1
    coef = rng.uniform(0.5, 1.5, (2, o)).astype(np.float16)
    srow = rng.uniform(0.005, 0.02, o).astype(np.float16)
    tcol = rng.uniform(0.8, 1.2, k).astype(np.float16)
    sal_idx = np.sort(rng.choice(k, size=salient, replace=False)).astype(np.int32)
    sal = bf16.round_bf16(rng.normal(0.0, 0.05, (o, salient)).astype(np.float32))
    return {"planes": rank_one_planes(bases), "coef": coef, "srow": srow, "tcol": tcol,
            "sal": sal, "sal_idx": sal_idx, "bases": bases}


def rank_one_weight(p) -> np.ndarray:
    """Dense float64 ``W[O, K]`` of the config-4 format."""
    signs = rank_one_signs(p["planes"]).astype(np.float64)
    coef = np.asarray(p["coef"], np.float64)
    srow = np.asarray(p["srow"], np.float64)
    tcol = np.asarray(p["tcol"], np.float64)
    w = srow[:, None] * tcol[None, :] * (coef[0][:, None] * signs[0] + coef[1][:, None] * signs[1])
    sal = np.asarray(p["sal"], np.float64)
    for j, col in enumerate(np.asarray(p["sal_idx"]).astype(np.int64)):
        w[:, col] += sal[:, j]
    return w


def rank_one_matvec(x, p) -> np.ndarray:
    """float64 ``y[M, O]`` of the config-4 format in factored form:
    ``s_r (a1 (B1 . u) + a2 (B2 . u)) + sal . x[idx]`` with ``u = t_c x``."""
    x = np.atleast_2d(np.asarray(x, np.float64))
    signs = rank_one_signs(p["planes"]).astype(np.float64)
    u = x * np.asarray(p["tcol"], np.float64)[None, :]
    coef = np.asarray(p["coef"], np.float64)
    d = np.stack([u @ signs[0].T, u @ signs[1].T])  # [2, M, O]
    y = np.asarray(p["srow"], np.float64)[None, :] * (coef[0][None, :] * d[0] + coef[1][None, :] * d[1])
    idx = np.asarray(p["sal_idx"]).astype(np.int64)
    return y + x[:, idx] @ np.asarray(p["sal"], np.float64).T


def rank_one_storage_bytes(o: int, k: int, salient: int = 32) -> int:
    """Payload bytes: 2 sign bits per weight, a1/a2/s_r fp16 per row, t_c fp16 per
    column, bf16 salient values and int32 indices."""
    return 2 * o * k // 8 + 4 * o + 2 * o + 2 * k + 2 * salient * o + 4 * salient
