"""Pins of the two-base oracle (``oracle/two_base.py``) against the reference's own
known-answer tests and against closed forms that a plausible mistake would fail."""
import numpy as np
import pytest

from oracle import bf16, two_base as tb


def test_pack_known_interleaved_bit_order():
    # tests/test_packing.py:23-35: K0..K3 give bit pairs 00, 01, 10, 11 from the LSB
    bases = np.array([[[-1, 1, -1, 1]], [[-1, -1, 1, 1]]], np.int8)
    codes = tb.pack_two_bases(bases)
    assert codes.shape == (1, 1) and int(codes[0, 0]) == 0b11100100
    assert np.array_equal(tb.unpack_two_bases(codes), bases)


def test_pack_round_trip_and_rejects_non_binary():
    rng = np.random.default_rng(31)
    bases = np.where(rng.random((2, 7, 20)) < 0.5, -1, 1).astype(np.int8)
    codes = tb.pack_two_bases(bases)
    assert codes.dtype == np.uint8 and codes.shape == (7, 5)
    assert np.array_equal(tb.unpack_two_bases(codes), bases)
    with pytest.raises(ValueError):
        tb.pack_two_bases(np.zeros((2, 3, 8), np.int8))


def test_planes_all_65536_words():
    # tests/test_planar_layout.py:14-24: plane b bit k = bit 2k + b of the 16-bit word
    word = np.arange(65536, dtype=np.int64)
    inter = np.stack([word & 255, word >> 8], axis=-1).astype(np.uint8)
    planes = tb.to_planes(inter)
    for basis in range(2):
        expected = np.zeros_like(word)
        for k in range(8):
            expected |= ((word >> (2 * k + basis)) & 1) << k
        assert np.array_equal(planes[:, basis, 0], expected.astype(np.uint8))
    assert np.array_equal(tb.from_planes(planes), inter)


@pytest.mark.parametrize("o,g", [(1, 1), (7, 3), (17, 10)])
def test_convert_restore_round_trip_and_lookup(o, g):
    p = tb.make_hybrid_payload(o, g, seed=o + g)
    for planar in (False, True):
        q = tb.convert_artifact(p, planar=planar)
        if planar:
            assert q["codes"].shape == (g, o, 2, 16) and q["sparse_codes"].shape == (g, o, 2, 1)
        else:
            assert q["codes"].shape == (g, o, 32) and q["sparse_codes"].shape == (g, o, 2)
        back = tb.restore_artifact(q)
        for key in tb.FIELDS:
            assert np.array_equal(back[key], np.asarray(p[key])), key
        lookup = np.full((g, 128), -1, np.int16)
        for gi in range(g):
            for j, col in enumerate(p["refinement_indices"][gi]):
                lookup[gi, col] = j
        assert np.array_equal(q["lookup"], lookup)


def test_validate_fails_closed():
    # tests/test_deployment.py:48-60
    for field, mutate in (
        ("refinement_indices", lambda v: np.full_like(v, 128)),
        ("refinement_indices", lambda v: np.zeros_like(v)),
        ("global_row_scales", lambda v: np.full_like(v, np.nan)),
        ("global_column_scales", lambda v: v.astype(np.float16)),
        ("refinement_sign_codes", lambda v: v.astype(np.int64)),
    ):
        p = tb.make_hybrid_payload(7, 3)
        p[field] = mutate(p[field])
        with pytest.raises(ValueError):
            tb.convert_artifact(p)
    with pytest.raises(ValueError):
        tb.convert_artifact({})


def _scalar_materialize(p):
    """Element-by-element fp32 loop: w = ((s0*r0)*c0 + 0) ... in the reference's order."""
    o, g = tb.validate_artifact(p)
    signs = tb.unpack_two_bases(p["global_sign_codes"])
    ref = tb.unpack_two_bases(p["refinement_sign_codes"])
    f = np.float32
    w = np.zeros((o, g * 128), np.float32)
    for row in range(o):
        for k in range(g * 128):
            gi, kk = divmod(k, 128)
            acc = f(0)
            for b in range(2):
                acc = f(acc + f(f(f(signs[b, row, k]) * p["global_row_scales"][b, row, gi]) *
                                p["global_column_scales"][b, gi, kk]))
            w[row, k] = acc
        for gi in range(g):
            for j, col in enumerate(p["refinement_indices"][gi]):
                sel = f(0)
                for b in range(2):
                    sel = f(sel + f(f(f(ref[b, row, 8 * gi + j]) * p["refinement_row_scales"][b, row, gi]) *
                                    p["refinement_column_scales"][b, gi, j]))
                w[row, 128 * gi + col] = f(w[row, 128 * gi + col] + sel)
    return w


def test_materialize_bitwise_scalar_loop_and_closed_form():
    p = tb.make_hybrid_payload(3, 2, seed=5)
    w = tb.materialize_hybrid(p)
    assert np.array_equal(w, _scalar_materialize(p))
    # float64 closed form agrees to fp32 rounding (a dropped or transposed factor would not)
    o, g = 3, 2
    s = tb.unpack_two_bases(p["global_sign_codes"]).astype(np.float64).reshape(2, o, g, 128)
    exact = np.einsum("bogk,bog,bgk->ogk", s, p["global_row_scales"].astype(np.float64),
                      p["global_column_scales"].astype(np.float64))
    r = tb.unpack_two_bases(p["refinement_sign_codes"]).astype(np.float64).reshape(2, o, g, 8)
    sel = np.einsum("bogj,bog,bgj->ogj", r, p["refinement_row_scales"].astype(np.float64),
                    p["refinement_column_scales"].astype(np.float64))
    for gi in range(g):
        exact[:, gi, p["refinement_indices"][gi].astype(np.int64)] += sel[:, gi]
    exact = exact.reshape(o, g * 128)
    assert np.max(np.abs(w - exact)) <= 4 * np.finfo(np.float32).eps * np.max(np.abs(exact))


@pytest.mark.parametrize("o,g", [(1, 1), (17, 3)])
def test_structural_reference_matches_independent_factored_dot(o, g):
    # tests/test_factored_reference.py:10-25
    p = tb.make_hybrid_payload(o, g, seed=3)
    rng = np.random.default_rng(1)
    x = bf16.round_bf16(rng.standard_normal((1, g * 128)).astype(np.float32)).astype(np.float64)
    xd = x.reshape(g, 128)
    signs = tb.unpack_two_bases(p["global_sign_codes"]).astype(np.float64).reshape(2, o, g, 128)
    z = xd[None] * p["global_column_scales"].astype(np.float64)
    expected = ((signs * z[:, None]).sum(-1) * p["global_row_scales"].astype(np.float64)).sum((0, 2))
    sparse = tb.unpack_two_bases(p["refinement_sign_codes"]).astype(np.float64).reshape(2, o, g, 8)
    sx = np.take_along_axis(xd, p["refinement_indices"].astype(np.int64), axis=1)
    sz = sx[None] * p["refinement_column_scales"].astype(np.float64)
    expected += ((sparse * sz[:, None]).sum(-1) * p["refinement_row_scales"].astype(np.float64)).sum((0, 2))
    for planar in (False, True):
        got = tb.structural_reference(x, tb.convert_artifact(p, planar=planar))
        np.testing.assert_allclose(got, expected[None], rtol=1e-12, atol=1e-12)
    dense = x @ tb.materialize_hybrid(p).astype(np.float64).T
    np.testing.assert_allclose(dense, expected[None], rtol=1e-5, atol=1e-5)


def test_structural_reference_detects_dropped_refinement():
    p = tb.make_hybrid_payload(9, 2, seed=8)
    x = np.random.default_rng(2).standard_normal((1, 256))
    layout = tb.convert_artifact(p)
    broken = dict(layout, sparse_rows=np.zeros_like(layout["sparse_rows"]))
    assert np.max(np.abs(tb.structural_reference(x, layout) - tb.structural_reference(x, broken))) > 1e-3
    with pytest.raises(ValueError):
        tb.structural_reference(np.zeros((1, 1)), layout)


def test_rank_one_planes_bit_positions():
    rng = np.random.default_rng(4)
    o, g = 5, 3
    bases = (rng.integers(0, 2, (2, o, g * 128)) * 2 - 1).astype(np.int8)
    planes = tb.rank_one_planes(bases)
    assert planes.shape == (g, o, 2, 16)
    assert np.array_equal(tb.rank_one_signs(planes), bases)
    # brute force: every single +1 lands on bit k >> 4 of byte k & 15 of its (group, row, base)
    for b in range(2):
        for row in (0, 4):
            for col in (0, 1, 15, 16, 17, 100, 127, 128, 255, 383):
                one = np.full((2, o, g * 128), -1, np.int8)
                one[b, row, col] = 1
                pl = tb.rank_one_planes(one)
                gi, k = divmod(col, 128)
                assert pl[gi, row, b, k & 15] == 1 << (k >> 4) and np.count_nonzero(pl) == 1
    # all-(+1) rows are all-ones bytes
    assert np.all(tb.rank_one_planes(np.ones((2, 1, 128), np.int8)) == 255)


def test_rank_one_matvec_closed_forms():
    p = tb.make_rank_one_payload(24, 384, salient=5, seed=3)
    rng = np.random.default_rng(0)
    x = rng.standard_normal((2, 384))
    w = tb.rank_one_weight(p)
    np.testing.assert_allclose(tb.rank_one_matvec(x, p), x @ w.T, rtol=1e-12, atol=1e-12)
    # basis vectors read single columns; a salient column carries its residual
    col = int(p["sal_idx"][2])
    e = np.zeros((1, 384))
    e[0, col] = 1.0
    s = tb.rank_one_signs(p["planes"]).astype(np.float64)
    expected = (p["srow"].astype(np.float64) * float(p["tcol"][col]) *
                (p["coef"][0].astype(np.float64) * s[0, :, col] + p["coef"][1].astype(np.float64) * s[1, :, col])
                + p["sal"][:, 2].astype(np.float64))
    np.testing.assert_allclose(tb.rank_one_matvec(e, p)[0], expected, rtol=1e-12)
    # all-(+1) bases: W = s_r t_c (a1 + a2)
    q = dict(p, planes=np.full_like(p["planes"], 255), sal=np.zeros_like(p["sal"]))
    ones = np.ones((1, 384))
    closed = p["srow"].astype(np.float64) * (p["coef"][0].astype(np.float64) + p["coef"][1].astype(np.float64)) \
        * p["tcol"].astype(np.float64).sum()
    np.testing.assert_allclose(tb.rank_one_matvec(ones, q)[0], closed, rtol=1e-12)


def test_rank_one_payload_distributions_and_storage():
    p = tb.make_rank_one_payload(64, 256, salient=32, seed=1)
    assert p["coef"].dtype == np.float16 and p["srow"].dtype == np.float16 and p["tcol"].dtype == np.float16
    assert 0.5 <= p["coef"].min() and p["coef"].max() <= 1.5
    assert 0.8 <= p["tcol"].min() and p["tcol"].max() <= 1.2
    assert len(set(p["sal_idx"].tolist())) == 32 and np.all(np.diff(p["sal_idx"]) > 0)
    assert np.array_equal(bf16.round_bf16(p["sal"]), p["sal"])
    # config 4 at the gate shape: payload + x + y = 13,484,160 bytes
    assert tb.rank_one_storage_bytes(12288, 4096) + 2 * 4096 + 2 * 12288 == 13_484_160
