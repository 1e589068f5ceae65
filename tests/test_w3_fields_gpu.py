"""GPU parity of the W3 field layout: the bind-time repack (fx_w3_planes_to_fields)
bit for bit against the oracle's restatement of the layout, and the field-layout
GEMV (fx_w3_gemv_fields) against the float64 oracle of the planar payload it was
repacked from.

GEMV bar: half an output ulp of the exact x @ (s*(q-z)).T plus 3e-5 * max|y| --
the field kernel runs the fp16 MFMA on fp16 subnormal codes, which rounds such
products at ~2e-7 relative per instruction (the same bar as the planar kernel's
fp16-activation path).
"""
import numpy as np
import pytest
import torch

from marlin_style_fluxbin_amd import _lib
from oracle import w3
from tests.payloads import (assert_half_ulp, assert_within_terms, config_codes, layout_from_codes, oracle_layout,
                            outlier_activations, silence_columns)

pytestmark = pytest.mark.gpu


def _repack(planes):
    lib = _lib.library()
    fields = torch.full_like(planes, 0xA5)
    g, _, o, _ = planes.shape
    _lib.check(lib.fx_w3_planes_to_fields(planes.data_ptr(), fields.data_ptr(), o, 128 * g,
                                          _lib.stream_handle(planes.device)), "planes_to_fields")
    return fields


@pytest.mark.parametrize("o,k", [(64, 512), (37, 1536), (300, 2048), (1, 128), (17, 384), (4096, 4096)])
def test_planes_to_fields_matches_oracle(gpu, o, k):
    codes, scales, zeros, perm = config_codes(o, k, seed=o * 7 + k, zeros=True, scale_dtype=torch.float16,
                                              permute=True)
    layout = layout_from_codes(codes, scales, zeros, perm)
    fields = _repack(layout["planes"].to(gpu)).cpu().numpy()
    assert np.array_equal(fields, w3.fields_from_planar(layout["planes"].numpy()))
    # the sorted codes survive the repack
    assert np.array_equal(w3.sorted_codes_from_fields(fields), w3.codes_from_planar(layout["planes"].numpy()))


@pytest.mark.parametrize("o,k", [(4096, 4096), (12288, 4096), (4096, 12288), (37, 1536), (96, 384), (1, 128)])
@pytest.mark.parametrize("xdtype,tag", [(torch.bfloat16, "bf16"), (torch.float16, "f16")])
@pytest.mark.parametrize("scale_dtype,zeros", [(torch.float16, True), (torch.bfloat16, False)])
def test_gemv_fields_matches_oracle(gpu, o, k, xdtype, tag, scale_dtype, zeros):
    codes, scales, zero, _ = config_codes(o, k, seed=o + 3 * k, zeros=zeros, scale_dtype=scale_dtype)
    layout = layout_from_codes(codes, scales, zero, None)
    dl = {n: t.to(gpu) for n, t in layout.items()}
    fields = _repack(dl["planes"])
    x = torch.randn(1, k, generator=torch.Generator().manual_seed(o)).to(xdtype)
    out = torch.full((1, o), float("nan"), dtype=xdtype, device=gpu)
    lib = _lib.library()
    _lib.check(lib.fx_w3_gemv_fields(x.to(gpu).data_ptr(), _lib.dtype_code(xdtype), fields.data_ptr(),
                                     dl["scales"].data_ptr(), _lib.dtype_code(scale_dtype), _lib.ptr(dl.get("zeros")),
                                     out.data_ptr(), o, k, _lib.stream_handle(gpu)), "gemv_fields")
    exact = w3.matvec_exact(x.float().numpy(), oracle_layout(layout))
    assert_half_ulp(out.float().cpu().numpy(), exact, tag, rel_slack=3e-5, what=f"fields {o}x{k}")


@pytest.mark.parametrize("scale", [1e-30, 1e-3, 1.0, 1e4, 1e30])
def test_gemv_fields_activation_range(gpu, scale):
    """The fp16 operands are exact over the activation's whole range: each group's
    power-of-two exponent puts its largest |x| near 2^14 whatever the scale."""
    o, k = 256, 1024
    codes, scales, zero, _ = config_codes(o, k, seed=9, zeros=True, scale_dtype=torch.float16)
    layout = layout_from_codes(codes, scales, zero, None)
    dl = {n: t.to(gpu) for n, t in layout.items()}
    fields = _repack(dl["planes"])
    x = (torch.randn(1, k, generator=torch.Generator().manual_seed(1)) * scale).to(torch.bfloat16)
    out = torch.empty(1, o, dtype=torch.bfloat16, device=gpu)
    lib = _lib.library()
    _lib.check(lib.fx_w3_gemv_fields(x.to(gpu).data_ptr(), _lib.dtype_code(torch.bfloat16), fields.data_ptr(),
                                     dl["scales"].data_ptr(), _lib.dtype_code(torch.float16), dl["zeros"].data_ptr(),
                                     out.data_ptr(), o, k, _lib.stream_handle(gpu)), "gemv_fields")
    exact = w3.matvec_exact(x.float().numpy(), oracle_layout(layout))
    assert_half_ulp(out.float().cpu().numpy(), exact, "bf16", rel_slack=3e-5, what=f"scale {scale}")


@pytest.mark.parametrize("xdtype,tag", [(torch.bfloat16, "bf16"), (torch.float16, "f16")])
@pytest.mark.parametrize("ratio", [10.0, 1e3, 1e4])
def test_gemv_fields_outlier_channels(gpu, xdtype, tag, ratio):
    """A few channels `ratio` times larger than the rest of their group (Qwen3's
    massive activations), with half of the rows' weights on those channels
    exactly zero.  The group's exponent follows the outlier; the fp16 operands
    x * 2^(E - p) keep the other elements' 8 (bf16) or 11 (fp16) significant bits
    while they lie within 2^24 (bf16) or 2^21 (fp16) of the group's largest |x|
    (the largest lands in [2^7, 2^14) after the 2^-p, and fp16 subnormals end at
    2^-24).  Every row lies within half an ulp plus 2^-18 of its terms' scale
    (11 max(s) sum|x|; the fp16 MFMA rounds products of subnormal codes at ~2e-7
    relative)."""
    o, k = 96, 1024
    codes, scales, zero, _ = config_codes(o, k, seed=12, zeros=True, scale_dtype=torch.float16)
    channels = [5, 300, 301, 777]
    silence_columns(codes, zero, None, channels, np.arange(0, o, 2))
    layout = layout_from_codes(codes, scales, zero, None)
    dl = {n: t.to(gpu) for n, t in layout.items()}
    fields = _repack(dl["planes"])
    x = outlier_activations(1, k, ratio=ratio, seed=3, channels=channels, dtype=xdtype)
    out = torch.full((1, o), float("nan"), dtype=xdtype, device=gpu)
    lib = _lib.library()
    _lib.check(lib.fx_w3_gemv_fields(x.to(gpu).data_ptr(), _lib.dtype_code(xdtype), fields.data_ptr(),
                                     dl["scales"].data_ptr(), _lib.dtype_code(torch.float16), dl["zeros"].data_ptr(),
                                     out.data_ptr(), o, k, _lib.stream_handle(gpu)), "gemv_fields")
    exact = w3.matvec_exact(x.float().numpy(), oracle_layout(layout))
    assert_within_terms(out.float().cpu().numpy(), exact, tag, x, scales, 2.0 ** -18, what=f"ratio {ratio}")


def test_field_layout_argument_checks(gpu):
    lib = _lib.library()
    t = torch.zeros(3 * 16 * 16, dtype=torch.uint8, device=gpu)
    perm = torch.arange(128, dtype=torch.int16, device=gpu)
    assert lib.fx_w3_planes_to_fields(t.data_ptr(), t.data_ptr(), 16, 128, None) == 1  # in place
    assert "in place" in lib.fx_last_error().decode()
    x = torch.zeros(1, 128, dtype=torch.bfloat16, device=gpu)
    sc = torch.ones(1, 16, dtype=torch.float16, device=gpu)
    out = torch.zeros(1, 16, dtype=torch.bfloat16, device=gpu)
    part = torch.zeros(1, device=gpu)
    rc = lib.fx_w3_gemv_residual(x.data_ptr(), 2, t.data_ptr(), sc.data_ptr(), 1, None, perm.data_ptr(),
                                 out.data_ptr(), out.data_ptr(), part.data_ptr(), perm.data_ptr(), None, 16, 128,
                                 _lib.PAYLOAD_FIELDS, None)
    assert rc == 1 and "together" in lib.fx_last_error().decode()
    rc = lib.fx_w3_gemv_residual(x.data_ptr(), 2, t.data_ptr(), sc.data_ptr(), 1, None, None, out.data_ptr(),
                                 out.data_ptr(), part.data_ptr(), None, None, 16, 128, 7, None)
    assert rc == 1 and "payload_format" in lib.fx_last_error().decode()


@pytest.mark.parametrize("fmt", ["planar", "fields"])
@pytest.mark.parametrize("o,k,batch", [(4096, 4096, 3), (1024, 4096, 5), (12288, 4096, 2), (4096, 12288, 2),
                                        (128, 256, 1)])
def test_strided_batch_equals_single_calls(gpu, fmt, o, k, batch):
    """fx_w3_gemv_strided_batched: payload p of one launch is bit-identical to the
    same payload's single call of the same format (fx_w3_gemv / fx_w3_gemv_fields)."""
    from marlin_style_fluxbin_amd.w3_lut_deployment import W3Gemv

    print(f"strided batch {fmt} {o}x{k} x{batch}", flush=True)
    lib = _lib.library()
    layouts = []
    for p in range(batch):
        codes, scales, zeros, _ = config_codes(o, k, seed=o + k + p, zeros=p % 2 == 0 or batch == 1,
                                               scale_dtype=torch.float16)
        if zeros is None:
            zeros = torch.full((k // 128, o), 4, dtype=torch.uint8)
        layouts.append({n: t.to(gpu) for n, t in layout_from_codes(codes, scales, zeros, None).items()})
    planes = torch.stack([l["planes"] for l in layouts]).contiguous()
    if fmt == "fields":
        fields = torch.empty_like(planes)
        for p in range(batch):
            _lib.check(lib.fx_w3_planes_to_fields(planes[p].data_ptr(), fields[p].data_ptr(), o, k,
                                                  _lib.stream_handle(gpu)), "planes_to_fields")
        weights = fields
    else:
        weights = planes
    scales = torch.stack([l["scales"] for l in layouts]).contiguous()
    zeros = torch.stack([l["zeros"] for l in layouts]).contiguous()
    x = torch.randn(batch, k, generator=torch.Generator().manual_seed(k)).to(torch.bfloat16).to(gpu)
    got = torch.full((batch, o), float("nan"), dtype=torch.bfloat16, device=gpu)
    _lib.check(lib.fx_w3_gemv_strided_batched(
        x.data_ptr(), _lib.FX_BF16, k, weights.data_ptr(), weights[0].numel(), scales.data_ptr(), _lib.FX_F16,
        scales[0].numel(), zeros.data_ptr(), zeros[0].numel(), got.data_ptr(), o, batch, o, k,
        _lib.PAYLOAD_PLANAR if fmt == "planar" else _lib.PAYLOAD_FIELDS, _lib.stream_handle(gpu)),
        "strided batch")
    for p in range(batch):
        want = torch.full((1, o), float("nan"), dtype=torch.bfloat16, device=gpu)
        if fmt == "planar":
            W3Gemv(layouts[p], perm_identity=True)(x[p:p + 1], want)
        else:
            _lib.check(lib.fx_w3_gemv_fields(x[p:p + 1].data_ptr(), _lib.FX_BF16, weights[p].data_ptr(),
                                             scales[p].data_ptr(), _lib.FX_F16, zeros[p].data_ptr(), want.data_ptr(),
                                             o, k, _lib.stream_handle(gpu)), "gemv_fields")
        torch.cuda.synchronize()
        assert torch.equal(got[p:p + 1], want), p
