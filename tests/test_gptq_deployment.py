"""The product's payload format layer (``gptq_deployment.py``) pinned bit for bit.

Three kinds of checks, all on the CPU:

* the reference's own known-answer and fail-closed cases
  (``tests/test_gptq_w3_planar.py:43-143`` in maxiu188-afk/Marlin_Style_Fluxbin),
  run against the product functions;
* byte-for-byte agreement with the independently written numpy packer and
  unpacker in ``oracle/w3.py`` on random codes, random permutations, both qzero
  formats, bf16 and fp16 scales and zero-points in {3, 4};
* the committed golden fixtures under ``tests/golden/``.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from marlin_style_fluxbin_amd import gptq_deployment as gd
from oracle import bf16, w3
from tests.golden_data import load_npz
from tests.payloads import synthetic_raw


def _oracle_layout(layout):
    scales = layout["scales"]
    return {"planes": layout["planes"].numpy(), "scales": scales.float().numpy(),
            "scale_dtype": "bf16" if scales.dtype == torch.bfloat16 else "f16",
            "perm": layout["perm"].numpy(),
            "zeros": None if layout.get("zeros") is None else layout["zeros"].numpy()}


# --------------------------------------------------------------------------- reference KATs
def test_boundary_word_known_answer():
    """The 10-1-10-1-10 split of 32 codes over three words (reference :43-60),
    built here from the bit positions, not from the product's packer."""
    codes = torch.arange(32, dtype=torch.uint8).remainder_(8).reshape(32, 1)
    words = [0, 0, 0]
    for i in range(10):
        words[0] |= int(codes[i]) << (3 * i)
    words[0] |= (int(codes[10]) & 3) << 30
    words[1] |= int(codes[10]) >> 2
    for i in range(11, 21):
        words[1] |= int(codes[i]) << (1 + 3 * (i - 11))
    words[1] |= (int(codes[21]) & 1) << 31
    words[2] |= int(codes[21]) >> 1
    for i in range(22, 32):
        words[2] |= int(codes[i]) << (2 + 3 * (i - 22))
    signed = torch.tensor([v if v < 2**31 else v - 2**32 for v in words], dtype=torch.int32).reshape(3, 1)
    assert torch.equal(gd.unpack_gptq_w3_qweight(signed), codes)
    assert torch.equal(gd.pack_gptq_w3_codes(codes), signed)


def test_canonical_pack_unpack_and_qzero_formats():
    raw, codes, zeros = synthetic_raw()
    assert torch.equal(gd.unpack_gptq_w3_qweight(raw["qweight"]), codes)
    assert torch.equal(gd.unpack_gptq_w3_qzeros(raw["qzeros"], qzero_format=1), zeros)
    v2 = gd.pack_gptq_w3_codes(zeros, packed_axis=1)
    assert torch.equal(gd.unpack_gptq_w3_qzeros(v2, qzero_format=2), zeros)


def test_desc_act_canonicalization_is_exact():
    raw, codes, _ = synthetic_raw()
    facts = gd.inspect_gptq_checkpoint(raw, qzero_format=1)
    assert facts["decoded_zero_unique"] == [4]
    assert facts["permutation_identity"] is False
    assert (facts["in_features"], facts["out_features"], facts["groups"]) == (256, 64, 2)
    assert facts["qweight_shape"] == [24, 64] and facts["qzeros_shape"] == [2, 6]
    layout = gd.convert_gptq_w3_to_planar(raw, qzero_format=1)
    assert set(layout) == {"planes", "scales", "perm"}
    assert layout["perm"].dtype == torch.int16 and layout["scales"].dtype == torch.bfloat16
    assert torch.equal(layout["scales"], raw["scales"].to(torch.bfloat16))
    assert torch.equal(gd.decode_planar_w3_codes(layout), codes)


def test_bf16_restore_matches_gptq_semantics_bitwise():
    raw, codes, zeros = synthetic_raw()
    layout = gd.convert_gptq_w3_to_planar(raw, qzero_format=1)
    g = raw["g_idx"].long()
    expected = (raw["scales"].to(torch.bfloat16)[g] * (codes.to(torch.int16) - zeros[g])).T.contiguous()
    assert torch.equal(gd.restore_planar_w3(layout), expected)


def test_structural_matvec_matches_direct_formula():
    raw, codes, zeros = synthetic_raw()
    layout = gd.convert_gptq_w3_to_planar(raw, qzero_format=1)
    x = torch.randn(1, codes.shape[0], generator=torch.Generator().manual_seed(9), dtype=torch.bfloat16)
    g = raw["g_idx"].long()
    direct = torch.sum(x.float().T * raw["scales"].to(torch.bfloat16)[g].float()
                       * (codes.to(torch.int16) - zeros[g]).float(), dim=0).unsqueeze(0)
    torch.testing.assert_close(gd.structural_w3_matvec(x, layout), direct, rtol=2e-6, atol=2e-5)


def test_bf16_weight_semantics_equals_materialized_weight():
    raw, codes, _ = synthetic_raw(k=512, o=256, seed=17)
    layout = gd.convert_gptq_w3_to_planar(raw, qzero_format=1)
    x = torch.randn(1, codes.shape[0], generator=torch.Generator().manual_seed(23), dtype=torch.bfloat16)
    corrected = gd.bf16_weight_semantics_w3_matvec(x, layout)
    dense = F.linear(x.float(), gd.restore_planar_w3(layout).float())
    assert torch.equal(corrected.bfloat16(), dense.bfloat16())
    assert float((gd.structural_w3_matvec(x, layout) - dense).abs().max()) > 0.0


def test_layout_storage_includes_permutation():
    raw, _, _ = synthetic_raw()
    record = gd.layout_storage(gd.convert_gptq_w3_to_planar(raw, qzero_format=1))
    assert record["format"] == gd.REFERENCE_FORMAT
    expected = 3 * 256 * 64 // 8 + 2 * 64 * 2 + 2 * 256
    assert record["total_bytes"] == expected
    assert record["bits_per_weight"] == pytest.approx(expected * 8 / (256 * 64))
    # the zeros extension adds one byte per (group, row) and names the extended format
    raw3, _, _ = synthetic_raw(zero=3)
    with_zeros = gd.convert_gptq_w3_to_planar(raw3, qzero_format=1, allow_zeros=True)
    record = gd.layout_storage(with_zeros)
    assert record["format"] == gd.FORMAT and record["total_bytes"] == expected + 2 * 64
    assert record["total_bytes"] == w3.layout_storage_bytes(_oracle_layout(with_zeros))


def test_non_constant_zero_rejected_by_default():
    raw, _, _ = synthetic_raw(zero=3)
    with pytest.raises(ValueError, match="requires decoded zero=4"):
        gd.convert_gptq_w3_to_planar(raw, qzero_format=1)


def test_runtime_validation_skips_only_value_checks():
    raw, _, _ = synthetic_raw()
    layout = gd.convert_gptq_w3_to_planar(raw, qzero_format=1)
    layout["perm"] = torch.zeros_like(layout["perm"])
    with pytest.raises(ValueError, match="bijection"):
        gd.validate_planar_w3(layout)
    assert gd.validate_planar_w3(layout, check_values=False) == (64, 256)


# --------------------------------------------------------------------------- product vs oracle
@pytest.mark.parametrize("k,o,seed", [(128, 1, 0), (256, 7, 1), (384, 64, 2), (1024, 33, 3)])
@pytest.mark.parametrize("permute", [False, True])
def test_planar_from_codes_matches_oracle_packer(k, o, seed, permute):
    g = torch.Generator().manual_seed(seed)
    codes = torch.randint(0, 8, (k, o), generator=g, dtype=torch.uint8)
    perm = torch.randperm(k, generator=g) if permute else None
    product = gd.planar_from_codes(codes, perm)
    oracle_planes = w3.planar_from_codes(codes.numpy(), None if perm is None else perm.numpy())
    assert product.dtype == torch.uint8 and tuple(product.shape) == (k // 128, 3, o, 16)
    np.testing.assert_array_equal(product.numpy(), oracle_planes)


@pytest.mark.parametrize("k,o", [(128, 32), (256, 96), (640, 5)])
def test_gptq_words_match_oracle(k, o):
    codes = torch.randint(0, 8, (k, o), generator=torch.Generator().manual_seed(k + o), dtype=torch.uint8)
    words = gd.pack_gptq_w3_codes(codes)
    np.testing.assert_array_equal(words.numpy(), w3.pack_gptq_w3_codes(codes.numpy(), packed_axis=0))
    np.testing.assert_array_equal(gd.unpack_gptq_w3_qweight(words).numpy(), w3.unpack_gptq_w3(words.numpy(), 0))
    zeros = torch.randint(0, 8, (k // 128, 3 * 32), generator=torch.Generator().manual_seed(1), dtype=torch.uint8)
    packed = gd.pack_gptq_w3_codes(zeros, packed_axis=1)
    np.testing.assert_array_equal(packed.numpy(), w3.pack_gptq_w3_codes(zeros.numpy(), packed_axis=1))
    for fmt in (1, 2):
        np.testing.assert_array_equal(gd.unpack_gptq_w3_qzeros(packed, qzero_format=fmt).numpy(),
                                      w3.unpack_gptq_w3_qzeros(packed.numpy(), fmt))


@pytest.mark.parametrize("zero", [3, 4, "mixed"])
@pytest.mark.parametrize("scale_dtype", [torch.bfloat16, torch.float16])
def test_convert_matches_oracle(zero, scale_dtype):
    raw, codes, zeros = synthetic_raw(k=384, o=64, seed=5, zero=4 if zero == "mixed" else zero)
    if zero == "mixed":
        zeros = torch.randint(3, 5, zeros.shape, generator=torch.Generator().manual_seed(6), dtype=torch.uint8)
        raw["qzeros"] = gd.pack_gptq_w3_codes(((zeros.to(torch.int16) - 1) & 7).to(torch.uint8), packed_axis=1)
    product = gd.convert_gptq_w3_to_planar(raw, qzero_format=1, scale_dtype=scale_dtype, allow_zeros=True)
    oracle_layout = w3.convert_gptq_w3_to_planar(
        raw["qweight"].numpy(), raw["qzeros"].numpy(), raw["scales"].float().numpy(), raw["g_idx"].numpy(),
        qzero_format=1, scale_dtype="bf16" if scale_dtype == torch.bfloat16 else "f16", allow_zeros=True)
    np.testing.assert_array_equal(product["planes"].numpy(), oracle_layout["planes"])
    np.testing.assert_array_equal(product["perm"].numpy(), oracle_layout["perm"])
    np.testing.assert_array_equal(product["scales"].float().numpy(), oracle_layout["scales"])
    if zero == 4:
        assert "zeros" not in product and oracle_layout["zeros"] is None
    else:
        np.testing.assert_array_equal(product["zeros"].numpy(), oracle_layout["zeros"])
        np.testing.assert_array_equal(product["zeros"].numpy(), zeros.numpy())
    # decode in both orders against the oracle's unpacker and against the drawn codes
    np.testing.assert_array_equal(gd.decode_planar_w3_codes(product).numpy(), codes.numpy())
    np.testing.assert_array_equal(gd.decode_planar_w3_codes(product, original_order=False).numpy(),
                                  w3.codes_from_planar(oracle_layout["planes"]))


@pytest.mark.parametrize("zero_mode", ["none", "mixed", "wide"])
@pytest.mark.parametrize("scale_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
def test_cpu_restore_matches_oracle_bitwise(zero_mode, scale_dtype, out_dtype):
    k, o = 384, 48
    g = torch.Generator().manual_seed(11)
    codes = torch.randint(0, 8, (k, o), generator=g, dtype=torch.uint8)
    perm = torch.randperm(k, generator=g)
    layout = {"planes": gd.planar_from_codes(codes, perm),
              "scales": (torch.rand(k // 128, o, generator=g) * 0.3 + 0.001).to(scale_dtype),
              "perm": perm.to(torch.int16)}
    if zero_mode == "mixed":
        layout["zeros"] = torch.randint(3, 5, (k // 128, o), generator=g, dtype=torch.uint8)
    elif zero_mode == "wide":
        layout["zeros"] = torch.randint(0, 8, (k // 128, o), generator=g, dtype=torch.uint8)
    got = gd.restore_planar_w3(layout, dtype=out_dtype).float().numpy()
    want = w3.restore_weight(_oracle_layout(layout), "bf16" if out_dtype == torch.bfloat16 else "f16")
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("m", [1, 3])
def test_cpu_matvecs_match_oracle(m):
    k, o = 512, 80
    g = torch.Generator().manual_seed(12)
    codes = torch.randint(0, 8, (k, o), generator=g, dtype=torch.uint8)
    perm = torch.randperm(k, generator=g)
    layout = {"planes": gd.planar_from_codes(codes, perm),
              "scales": (torch.rand(k // 128, o, generator=g) * 0.015 + 0.005).to(torch.bfloat16),
              "perm": perm.to(torch.int16),
              "zeros": torch.randint(3, 5, (k // 128, o), generator=g, dtype=torch.uint8)}
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    ol = _oracle_layout(layout)
    exact = w3.matvec_exact(x.float().numpy(), ol)
    structural = gd.structural_w3_matvec(x, layout).numpy()
    assert np.abs(structural - exact).max() <= 1e-5 * np.abs(exact).max()
    decoded = w3.matvec_decoded(x.float().numpy(), ol, "bf16")
    semantics = gd.bf16_weight_semantics_w3_matvec(x, layout).numpy()
    assert np.abs(semantics - decoded).max() <= 1e-5 * np.abs(decoded).max()
    # the two arithmetics differ by exactly the +-3 rounding the correction carries
    assert np.abs(decoded - exact).max() > 1e-4 * np.abs(exact).max()


def test_oracle_comparison_detects_layout_mistakes():
    """A plausible packer mistake -- MSB-first bytes, an un-inverted plane 2, a
    swapped plane pair -- planted in a copy of the oracle's output, is caught by the
    byte comparison the tests above use."""
    codes = torch.randint(0, 8, (256, 16), generator=torch.Generator().manual_seed(3), dtype=torch.uint8)
    product = gd.planar_from_codes(codes).numpy()
    good = w3.planar_from_codes(codes.numpy())
    assert np.array_equal(product, good)
    msb_first = np.unpackbits(good, axis=-1, bitorder="little")
    msb_first = np.packbits(msb_first, axis=-1, bitorder="big")
    plane2_plain = good.copy()
    plane2_plain[:, 2] ^= 0xFF
    swapped = good[:, [1, 0, 2]]
    for bad in (msb_first, plane2_plain, swapped):
        assert not np.array_equal(product, bad)


# --------------------------------------------------------------------------- fail-closed contracts
def _good_layout():
    raw, _, _ = synthetic_raw(k=256, o=32)
    return gd.convert_gptq_w3_to_planar(raw, qzero_format=1)


@pytest.mark.parametrize("mutate,message", [
    (lambda l: l.pop("perm"), "expected exactly"),
    (lambda l: l.__setitem__("extra", torch.zeros(1)), "expected exactly"),
    (lambda l: l.__setitem__("planes", l["planes"].to(torch.int16)), "planes must be uint8"),
    (lambda l: l.__setitem__("planes", l["planes"][:, :2].contiguous()), "planes must be uint8"),
    (lambda l: l.__setitem__("scales", l["scales"].float()), "bfloat16 or float16"),
    (lambda l: l.__setitem__("scales", l["scales"][:, :-1].contiguous()), "bfloat16 or float16"),
    (lambda l: l.__setitem__("perm", l["perm"].to(torch.int32)), "perm must be int16"),
    (lambda l: l.__setitem__("zeros", torch.zeros(2, 31, dtype=torch.uint8)), "zeros must be uint8"),
    (lambda l: l.__setitem__("scales", l["scales"].t().contiguous().t()), "contiguous"),
])
def test_validate_rejects_malformed_layouts(mutate, message):
    layout = _good_layout()
    mutate(layout)
    with pytest.raises(ValueError, match=message):
        gd.validate_planar_w3(layout, check_values=False)


@pytest.mark.parametrize("mutate,message", [
    (lambda l: l["scales"].__setitem__((0, 0), float("inf")), "finite"),
    (lambda l: l["scales"].__setitem__((1, 3), float("nan")), "finite"),
    (lambda l: l.__setitem__("zeros", torch.full((2, 32), 8, dtype=torch.uint8)), r"\[0,7\]"),
    (lambda l: l["perm"].__setitem__(0, 1), "bijection"),
])
def test_validate_value_checks(mutate, message):
    layout = _good_layout()
    mutate(layout)
    with pytest.raises(ValueError, match=message):
        gd.validate_planar_w3(layout)
    gd.validate_planar_w3(layout, check_values=False)


def test_validate_rejects_k_beyond_int16():
    planes = torch.zeros(256, 3, 1, 16, dtype=torch.uint8)  # K = 32768
    layout = {"planes": planes, "scales": torch.ones(256, 1, dtype=torch.bfloat16),
              "perm": torch.zeros(32768, dtype=torch.int16)}
    with pytest.raises(ValueError, match="int16"):
        gd.validate_planar_w3(layout, check_values=False)


@pytest.mark.parametrize("mutate,message", [
    (lambda r: r.pop("g_idx"), "expected exactly"),
    (lambda r: r.__setitem__("qweight", r["qweight"].to(torch.int64)), "qweight must be CPU int32"),
    (lambda r: r.__setitem__("qweight", r["qweight"][:-1].contiguous()), "divisible by three"),
    (lambda r: r.__setitem__("qzeros", r["qzeros"][:, :-1].contiguous()), "divisible by three"),
    (lambda r: r.__setitem__("scales", r["scales"].float()), "float16"),
    (lambda r: r["scales"].__setitem__((0, 0), float("inf")), "finite"),
    (lambda r: r.__setitem__("scales", r["scales"][:1].contiguous()), "shape does not match"),
    (lambda r: r.__setitem__("g_idx", r["g_idx"][:-1].contiguous()), "g_idx shape or range"),
    (lambda r: r["g_idx"].__setitem__(0, 5), "g_idx shape or range"),
    (lambda r: r["g_idx"].copy_((torch.arange(256, dtype=torch.int32) >= 129).int()), "exactly 128"),
])
def test_inspect_fails_closed(mutate, message):
    raw, _, _ = synthetic_raw()
    mutate(raw)
    with pytest.raises(ValueError, match=message):
        gd.inspect_gptq_checkpoint(raw, qzero_format=1)


def test_inspect_rejects_unknown_qzero_format():
    raw, _, _ = synthetic_raw()
    with pytest.raises(ValueError, match="qzero_format"):
        gd.inspect_gptq_checkpoint(raw, qzero_format=3)


def test_inspect_reports_identity_and_zero_set():
    raw, _, _ = synthetic_raw(zero=3)
    raw["g_idx"] = torch.arange(256, dtype=torch.int32) // 128
    facts = gd.inspect_gptq_checkpoint(raw, qzero_format=1)
    assert facts["permutation_identity"] is True and facts["decoded_zero_unique"] == [3]


# --------------------------------------------------------------------------- golden fixtures
@pytest.mark.parametrize("name", ["w3_gptq_64x256.npz", "w3_gptq_288x384.npz"])
def test_product_reproduces_golden_payloads(name):
    f = load_npz(name)
    raw = {"qweight": torch.from_numpy(f["qweight"]), "qzeros": torch.from_numpy(f["qzeros"]),
           "scales": torch.from_numpy(f["scales_f16_bits"].view(np.float16)),
           "g_idx": torch.from_numpy(f["g_idx"])}
    codes = torch.from_numpy(f["codes"])
    assert torch.equal(gd.pack_gptq_w3_codes(codes), raw["qweight"])
    assert torch.equal(gd.unpack_gptq_w3_qweight(raw["qweight"]), codes)
    layout = gd.convert_gptq_w3_to_planar(raw, qzero_format=1)
    np.testing.assert_array_equal(layout["planes"].numpy(), f["planes"])
    np.testing.assert_array_equal(layout["perm"].numpy(), f["perm"])
    np.testing.assert_array_equal(bf16.f32_to_bf16_bits(layout["scales"].float().numpy()), f["scales_bf16_bits"])
    restored = gd.restore_planar_w3(layout).view(torch.int16).numpy().view(np.uint16)
    import hashlib
    assert hashlib.sha256(np.ascontiguousarray(restored).tobytes()).hexdigest() == str(f["restored_bf16_sha256"])
    x = torch.from_numpy(f["x_bf16_bits"].view(np.int16)).view(torch.bfloat16)
    y = gd.structural_w3_matvec(x, layout).numpy()
    assert np.abs(y - f["y_exact_bf16x"]).max() <= 1e-5 * np.abs(f["y_exact_bf16x"]).max()
    yd = gd.bf16_weight_semantics_w3_matvec(x, layout).numpy()
    assert np.abs(yd - f["y_decoded_bf16x"]).max() <= 1e-5 * np.abs(f["y_decoded_bf16x"]).max()
