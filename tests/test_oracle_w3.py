"""Pins for the W3 oracle (CPU): reference KATs, brute force, closed forms.

A plausible mistake in the oracle (bit order, inverted plane, zero handling,
scale rounding point, permutation direction) fails at least one test here.
"""
import numpy as np
import pytest
import torch

from oracle import w3
from oracle.bf16 import f32_to_bf16_bits, round_bf16
from oracle.kernel_order import load_kernel_order, load_reference_lut, lut_unsigned, w3_kernel_order
from tests.payloads import synthetic_raw


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    values = np.concatenate([
        rng.standard_normal(10000).astype(np.float32) * np.float32(10.0) ** rng.integers(-30, 30, 10000),
        np.array([0.0, -0.0, 1.0, 1.00390625, 1.0078125, 65504.0, 3.0e38, 1e-40, -2.5], np.float32),
        # exact ties: mantissa low half 0x8000 with even and odd upper halves
        np.array([0x3F808000, 0x3F818000, 0xBF808000], np.uint32).view(np.float32),
    ]).astype(np.float32)
    expected = torch.from_numpy(values).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(f32_to_bf16_bits(values), expected)


def test_gptq_boundary_word_kat():
    """Reference tests/test_gptq_w3_planar.py:43-60: 32 codes across three words."""
    codes = (np.arange(32) % 8).astype(np.uint8).reshape(32, 1)
    words = [0, 0, 0]
    for i in range(10):
        words[0] |= int(codes[i, 0]) << (3 * i)
    words[0] |= (int(codes[10, 0]) & 3) << 30
    words[1] |= int(codes[10, 0]) >> 2
    for i in range(11, 21):
        words[1] |= int(codes[i, 0]) << (1 + 3 * (i - 11))
    words[1] |= (int(codes[21, 0]) & 1) << 31
    words[2] |= int(codes[21, 0]) >> 1
    for i in range(22, 32):
        words[2] |= int(codes[i, 0]) << (2 + 3 * (i - 22))
    signed = np.array([w if w < 2**31 else w - 2**32 for w in words], dtype=np.int64).astype(np.int32).reshape(3, 1)
    assert np.array_equal(w3.unpack_gptq_w3(signed, 0), codes)
    assert np.array_equal(w3.pack_gptq_w3_codes(codes, 0), signed)


def test_gptq_roundtrip_and_qzero_formats():
    rng = np.random.default_rng(1)
    codes = rng.integers(0, 8, (256, 48), dtype=np.uint8)
    assert np.array_equal(w3.unpack_gptq_w3(w3.pack_gptq_w3_codes(codes, 0), 0), codes)
    zeros = rng.integers(0, 8, (2, 96), dtype=np.uint8)
    v2 = w3.pack_gptq_w3_codes(zeros, 1)
    assert np.array_equal(w3.unpack_gptq_w3_qzeros(v2, 2), zeros)
    v1 = w3.pack_gptq_w3_codes(((zeros.astype(np.int16) - 1) & 7).astype(np.uint8), 1)
    assert np.array_equal(w3.unpack_gptq_w3_qzeros(v1, 1), zeros)


def test_reference_synthetic_raw_matches_torch_packer():
    """The reference-seeded fixture: our numpy packer equals the product's torch packer."""
    raw, codes, zeros = synthetic_raw()
    assert np.array_equal(w3.unpack_gptq_w3(raw["qweight"].numpy(), 0), codes.numpy())
    assert np.array_equal(w3.unpack_gptq_w3_qzeros(raw["qzeros"].numpy(), 1), zeros.numpy())


def test_pack_bytes_every_byte_value():
    values = np.arange(256, dtype=np.uint8)
    bits = ((values[:, None] >> np.arange(8)) & 1).astype(np.uint8)     # [256, 8]
    row = np.tile(bits, (1, 16))                                         # [256, 128]
    packed = w3.pack_bytes_lsb(row)
    assert np.array_equal(packed, np.repeat(values[:, None], 16, axis=1))
    assert np.array_equal(w3.unpack_bytes_lsb(packed), row)


def test_planar_every_code_at_every_position():
    """Row o = code o at column position k_pos: check the stored bits by definition."""
    for position in (0, 1, 7, 8, 63, 127):
        codes = np.zeros((128, 8), dtype=np.uint8)
        for q in range(8):
            codes[:, q] = (q + 1) % 8          # background code
            codes[position, q] = q
        planes = w3.planar_from_codes(codes)
        chunk, bit = divmod(position, 8)
        for q in range(8):
            got = [(planes[0, p, q, chunk] >> bit) & 1 for p in range(3)]
            assert got == [q & 1, (q >> 1) & 1, 1 - ((q >> 2) & 1)], (position, q)
        assert np.array_equal(w3.codes_from_planar(planes), codes)


def test_permutation_direction():
    rng = np.random.default_rng(2)
    codes = rng.integers(0, 8, (256, 4), dtype=np.uint8)
    perm = rng.permutation(256)
    planes = w3.planar_from_codes(codes, perm)
    # sorted position s stores original column perm[s]
    sorted_codes = w3.codes_from_planar(planes)
    assert np.array_equal(sorted_codes, codes[perm])
    assert np.array_equal(w3.codes_from_planar(planes, perm), codes)


def _torch_direct_restore(codes, scales16, zeros, g_idx, scale_dtype):
    """The reference's direct formula (tests/test_gptq_w3_planar.py:83-90), extended to zeros."""
    s = scales16.to(scale_dtype)[g_idx.long()]
    return (s * (codes.to(torch.int16) - zeros[g_idx.long()].to(torch.int16))).T.contiguous()


@pytest.mark.parametrize("zero_mode", ["four", "three_four"])
@pytest.mark.parametrize("scale_dtype", ["bf16", "f16"])
def test_restore_matches_direct_formula_bitwise(zero_mode, scale_dtype):
    raw, codes, _ = synthetic_raw()
    g = codes.shape[0] // 128
    gen = torch.Generator().manual_seed(5)
    zeros = (torch.full((g, codes.shape[1]), 4, dtype=torch.uint8) if zero_mode == "four"
             else torch.randint(3, 5, (g, codes.shape[1]), generator=gen, dtype=torch.uint8))
    g_idx = raw["g_idx"]
    perm = np.argsort(g_idx.numpy(), kind="stable")
    tdtype = torch.bfloat16 if scale_dtype == "bf16" else torch.float16
    layout = {
        "planes": w3.planar_from_codes(codes.numpy(), perm),
        "scales": raw["scales"].to(tdtype).float().numpy(),
        "scale_dtype": scale_dtype,
        "perm": perm.astype(np.int16),
        "zeros": None if zero_mode == "four" else zeros.numpy(),
    }
    got = w3.restore_weight(layout, scale_dtype)
    expected = _torch_direct_restore(codes, raw["scales"], zeros, g_idx, tdtype).float().numpy()
    assert np.array_equal(got, expected)


def test_convert_gptq_to_planar_zero_contract():
    raw, codes, _ = synthetic_raw()
    layout = w3.convert_gptq_w3_to_planar(raw["qweight"].numpy(), raw["qzeros"].numpy(),
                                          raw["scales"].numpy(), raw["g_idx"].numpy())
    assert layout["zeros"] is None
    assert np.array_equal(w3.codes_from_planar(layout["planes"], layout["perm"]), codes.numpy())
    raw3, _, _ = synthetic_raw(zero=3)
    with pytest.raises(ValueError, match="zero=4"):
        w3.convert_gptq_w3_to_planar(raw3["qweight"].numpy(), raw3["qzeros"].numpy(),
                                     raw3["scales"].numpy(), raw3["g_idx"].numpy())
    kept = w3.convert_gptq_w3_to_planar(raw3["qweight"].numpy(), raw3["qzeros"].numpy(),
                                        raw3["scales"].numpy(), raw3["g_idx"].numpy(), allow_zeros=True)
    assert (kept["zeros"] == 3).all()


def _tiny_layout(o=3, k=256, seed=3, zeros=True):
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 8, (k, o), dtype=np.uint8)
    perm = rng.permutation(k)
    g = k // 128
    scales = round_bf16(rng.uniform(0.005, 0.02, (g, o)).astype(np.float32))
    z = rng.integers(3, 5, (g, o), dtype=np.uint8) if zeros else None
    layout = {"planes": w3.planar_from_codes(codes, perm), "scales": scales, "scale_dtype": "bf16",
              "perm": perm.astype(np.int16), "zeros": z}
    return layout, codes, perm, scales, z


def test_matvec_exact_brute_force_loops():
    layout, codes, perm, scales, z = _tiny_layout()
    rng = np.random.default_rng(4)
    x = round_bf16(rng.standard_normal((2, 256)).astype(np.float32))
    expected = np.zeros((2, 3))
    inverse = np.empty_like(perm)
    inverse[perm] = np.arange(256)
    for m in range(2):
        for o in range(3):
            total = 0.0
            for k in range(256):
                g = inverse[k] // 128          # group of original column k
                total += float(x[m, k]) * float(scales[g, o]) * (int(codes[k, o]) - int(z[g, o]))
            expected[m, o] = total
    assert np.allclose(w3.matvec_exact(x, layout), expected, rtol=1e-12, atol=1e-12)


def test_matvec_exact_basis_vectors_and_linearity():
    layout, codes, perm, scales, z = _tiny_layout(o=5, zeros=False)
    dense = w3.dequant_exact(layout)
    eye = np.eye(256)
    assert np.array_equal(w3.matvec_exact(eye, layout), dense.T)
    rng = np.random.default_rng(6)
    a, b = rng.standard_normal((2, 256))
    lhs = w3.matvec_exact((2 * a - 3 * b)[None], layout)
    rhs = 2 * w3.matvec_exact(a[None], layout) - 3 * w3.matvec_exact(b[None], layout)
    assert np.allclose(lhs, rhs, rtol=1e-12, atol=1e-12)


def test_decoded_semantics_reference_kat():
    """Reference tests/test_gptq_w3_planar.py:105-122 (seeds 17/23): the bf16-weight
    matvec equals dense F.linear on the restored bf16 weight after a bf16 cast,
    and differs from the structural (exact-scale) value."""
    raw, codes, _ = synthetic_raw(k=512, o=256, seed=17)
    perm = np.argsort(raw["g_idx"].numpy(), kind="stable")
    layout = {"planes": w3.planar_from_codes(codes.numpy(), perm),
              "scales": raw["scales"].to(torch.bfloat16).float().numpy(), "scale_dtype": "bf16",
              "perm": perm.astype(np.int16), "zeros": None}
    x = torch.randn(1, 512, generator=torch.Generator().manual_seed(23), dtype=torch.bfloat16)
    dense = torch.nn.functional.linear(x.float(), torch.from_numpy(w3.restore_weight(layout, "bf16")))
    decoded = w3.matvec_decoded(x.float().numpy(), layout)
    assert np.array_equal(round_bf16(decoded.astype(np.float32)), dense.bfloat16().float().numpy())
    assert np.abs(w3.matvec_exact(x.float().numpy(), layout) - decoded).max() > 0


def test_storage_bytes_kat():
    """Reference tests/test_gptq_w3_planar.py:124-130: 3KO/8 + 2*2*G*O... for K=256, O=64."""
    layout, *_ = _tiny_layout(o=64, zeros=False)
    assert w3.layout_storage_bytes(layout) == 3 * 256 * 64 // 8 + 2 * 64 * 2 + 2 * 256


def test_c_lut_matches_reference_header_and_closed_form():
    lib = load_kernel_order()
    ref = load_reference_lut()
    rng = np.random.default_rng(29)
    for trial in range(100):
        v = rng.uniform(-32, 32, 8).astype(np.float32)
        table = lut_unsigned(lib, v)
        exact = np.array([sum(float(v[b]) for b in range(8) if (p >> b) & 1) for p in range(256)])
        assert np.all(np.abs(table - exact) <= 2e-6 * np.abs(v).sum() + 1e-7)
        if ref is not None:
            import ctypes
            other = np.full(256, np.nan, dtype=np.float32)
            ref.ref_build_unsigned_table(v.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                        other.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
            assert np.array_equal(table.view(np.uint32), other.view(np.uint32))


def test_kernel_order_close_to_exact():
    layout, *_ = _tiny_layout(o=37, k=384, zeros=False)
    rng = np.random.default_rng(7)
    x = round_bf16(rng.standard_normal(384).astype(np.float32))
    got = w3_kernel_order(x, layout)
    exact = w3.matvec_exact(x[None], layout)[0]
    bound = 1e-5 * np.abs(exact).max()
    assert np.abs(got - exact).max() <= bound
    decoded = w3_kernel_order(x, layout, decoded=True)
    assert np.abs(decoded - w3.matvec_decoded(x[None], layout)[0]).max() <= bound


def test_field_layout_known_answer():
    """Hand-built word images of the field layout (32 columns of one group row,
    the rest zero): column 0 code 5 -> member 0 bits 0-2; column 1 (second half
    of register 0) code 3 -> member 0 bits 16-18; column 8 (register 4 = member 0
    field 4, low half) code 7 -> member 0 bits 12-14; column 10 (register 5 =
    member 1 field 0) code 2 -> member 1 bits 0-2; column 30 code 6 = 0b110 ->
    bit 15 of members 1 and 2; column 31 code 1 -> bit 31 of member 0."""
    codes = np.zeros((128, 1), dtype=np.uint8)
    codes[0, 0], codes[1, 0], codes[8, 0], codes[10, 0], codes[30, 0], codes[31, 0] = 5, 3, 7, 2, 6, 1
    words = w3.fields_from_sorted_codes(codes).view("<u4").reshape(1, 3, 1, 4)
    assert words[0, 0, 0, 0] == 5 | (3 << 16) | (7 << 12) | (1 << 31)
    assert words[0, 1, 0, 0] == 2 | (1 << 15)
    assert words[0, 2, 0, 0] == 1 << 15
    assert not words[0, :, 0, 1:].any()


def test_field_layout_bijection_and_roundtrip():
    """Every one of the 96 bits of a word triple carries exactly one code bit,
    so the layout keeps three bits per code; codes and planes round-trip."""
    slots = [pos for t in w3.field_slots() for pos in t]
    assert len(slots) == 96 and len(set(slots)) == 96
    rng = np.random.default_rng(3)
    codes = rng.integers(0, 8, (384, 21)).astype(np.uint8)
    fields = w3.fields_from_sorted_codes(codes)
    assert fields.shape == (3, 3, 21, 16)
    assert np.array_equal(w3.sorted_codes_from_fields(fields), codes)
    assert np.array_equal(w3.fields_from_planar(w3.planar_from_codes(codes)), fields)


@pytest.mark.parametrize("permute", [False, True])
@pytest.mark.parametrize("ratio", [10.0, 1e3, 1e4, 2.0 ** 20])
def test_outlier_case_quiet_rows_and_sensitivity(permute, ratio):
    """The outlier parity case of the GPU suites: silenced rows do not depend on
    the outlier channels at all, and a kernel that flushed the small elements of
    an outlier's group (a per-batch or normal-only fp16 exponent would) misses the
    terms-scaled bar those suites hold every row to, so the bar can see the loss."""
    from tests.payloads import (assert_within_terms, config_codes, layout_from_codes, oracle_layout,
                                outlier_activations, silence_columns)

    o, k = 96, 1024
    codes, scales, zeros, perm = config_codes(o, k, seed=11, zeros=True, permute=permute)
    channels = [5, 300, 301, 777]
    quiet = np.arange(0, o, 2)
    silence_columns(codes, zeros, perm, channels, quiet)
    layout = oracle_layout(layout_from_codes(codes, scales, zeros, perm))
    x = outlier_activations(3, k, ratio=ratio, seed=3, channels=channels)
    exact = w3.matvec_exact(x.float().numpy(), layout)
    cut = x.clone()
    cut[:, channels] = 0
    assert np.array_equal(exact[:, quiet], w3.matvec_exact(cut.float().numpy(), layout)[:, quiet])
    # the exact values pass their own bar at the loosest factor the suites use
    assert_within_terms(exact, exact, "bf16", x, scales, 2.0 ** -18)
    # planted loss: the outlier groups' other elements flushed to zero
    flushed = x.float().clone()
    position = np.empty(k, dtype=np.int64)
    position[np.arange(k) if perm is None else perm.numpy().astype(np.int64)] = np.arange(k)
    for c in channels:
        group = position // 128 == position[c] // 128
        keep = flushed[:, c].clone()
        flushed[:, torch.from_numpy(group)] = 0
        flushed[:, c] = keep
    lossy = w3.matvec_exact(flushed.numpy(), layout)
    with pytest.raises(AssertionError):
        assert_within_terms(lossy, exact, "bf16", x, scales, 2.0 ** -18)


def test_fp6_layout_bijection_round_trip_and_expansion():
    """The fp6 layout: every lane's 96 stored bits carry exactly its 32 codes' bits,
    codes survive the round trip, and the kernel's six-register expansion puts each
    code in the mantissa of the field that meets its column (the instruction's
    measured pairing), with sign and exponent bits zero."""
    slots = w3._fp6_slots()
    for kb in range(4):
        assert sorted(slots[kb].reshape(-1)) == list(range(96))
        assert sorted(w3.fp6_column(kb, e) for e in range(32)) == sorted(
            32 * (2 * (kb % 2) + h) + 16 * (kb // 2) + i for h in range(2) for i in range(16))
    assert sorted(w3.fp6_column(kb, e) for kb in range(4) for e in range(32)) == list(range(128))
    rng = np.random.default_rng(5)
    codes = rng.integers(0, 8, size=(1024, 40)).astype(np.uint8)
    f = w3.fp6_from_sorted_codes(codes)
    assert f.shape == (8, 3, 40, 16) and f.nbytes == w3.planar_from_codes(codes).nbytes
    assert np.array_equal(w3.sorted_codes_from_fp6(f), codes)
    assert np.array_equal(w3.fp6_from_planar(w3.planar_from_codes(codes)), f)
    words = f.view("<u4").reshape(2, 40, 4, 4, 3)
    for bt, o, kb, b in ((0, 0, 0, 0), (1, 39, 3, 3), (0, 17, 1, 2), (1, 5, 2, 1)):
        regs = w3.fp6_expand(*[int(v) for v in words[bt, o, kb, b]])
        bits = sum(r << (32 * i) for i, r in enumerate(regs))
        for e in range(32):
            assert (bits >> (6 * e)) & 63 == codes[(4 * bt + b) * 128 + w3.fp6_column(kb, e), o]
    # known answer: one code 7 at sorted column 128 * 4 + 16 (batch 1, slot 0) of row 2:
    # lane block 2 (16 (kb // 2) = 16), field 0, i.e. bits 0..2 of register 0 = stored word 0
    one = np.zeros((1024, 4), dtype=np.uint8)
    one[4 * 128 + 16, 2] = 7
    w = w3.fp6_from_sorted_codes(one).view("<u4").reshape(2, 4, 4, 4, 3)
    assert int(w[1, 2, 2, 0, 0]) == 7 and int(w.sum()) == 7
    with pytest.raises(ValueError):
        w3.fp6_from_sorted_codes(np.zeros((384, 4), dtype=np.uint8))
