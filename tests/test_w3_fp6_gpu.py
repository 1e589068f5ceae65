"""GPU parity of the fp6 layout (fx_w3_planes_to_fp6) and its GEMVs, which run
gfx950's scaled f8f6f4 matrix instruction with fp6 e2m3 weight fields (q / 8,
exact) against two fp8 e4m3 digits of each bf16 activation.

Bars: the repack bit for bit against the oracle's restatement; the GEMV against
the float64 oracle of the planar payload within half an output ulp plus 3e-5 *
max|y| (the digits are exact down to 2^-10 of each group's max|x|, the
instruction sums a group's 128 products in fp32); with outlier channels, within
the zero-point terms' scale (``assert_within_terms``); the decode forms (residual
epilogue, normalising prologue, SwiGLU) against the field layout's same forms."""
import numpy as np
import pytest
import torch

from marlin_style_fluxbin_amd import _lib
from oracle import w3
from tests.payloads import assert_half_ulp, assert_within_terms, config_codes, layout_from_codes, oracle_layout, \
    outlier_activations

pytestmark = pytest.mark.gpu


def _repack(planes, fn="fx_w3_planes_to_fp6"):
    lib = _lib.library()
    out = torch.full_like(planes, 0xA5)
    g, _, o, _ = planes.shape
    _lib.check(getattr(lib, fn)(planes.data_ptr(), out.data_ptr(), o, 128 * g, _lib.stream_handle(planes.device)), fn)
    return out


def _gemv_fp6(x, fp6, dl, scale_dtype, o, k, gpu):
    out = torch.full((1, o), float("nan"), dtype=torch.bfloat16, device=gpu)
    _lib.check(_lib.library().fx_w3_gemv_fp6(x.to(gpu).data_ptr(), _lib.dtype_code(torch.bfloat16), fp6.data_ptr(),
                                             dl["scales"].data_ptr(), _lib.dtype_code(scale_dtype),
                                             _lib.ptr(dl.get("zeros")), out.data_ptr(), o, k,
                                             _lib.stream_handle(gpu)), "gemv_fp6")
    return out


@pytest.mark.parametrize("o,k", [(64, 512), (48, 1536), (300, 2048), (4096, 4096)])
def test_planes_to_fp6_matches_oracle(gpu, o, k):
    codes, scales, zeros, perm = config_codes(o, k, seed=o * 5 + k, zeros=True, scale_dtype=torch.float16,
                                              permute=True)
    layout = layout_from_codes(codes, scales, zeros, perm)
    fp6 = _repack(layout["planes"].to(gpu)).cpu().numpy()
    assert np.array_equal(fp6, w3.fp6_from_planar(layout["planes"].numpy()))
    assert np.array_equal(w3.sorted_codes_from_fp6(fp6), w3.codes_from_planar(layout["planes"].numpy()))


@pytest.mark.parametrize("o,k", [(4096, 4096), (12288, 4096), (4096, 12288), (1024, 4096), (64, 512), (160, 1536)])
@pytest.mark.parametrize("scale_dtype,zeros", [(torch.float16, True), (torch.bfloat16, False)])
def test_gemv_fp6_matches_oracle(gpu, o, k, scale_dtype, zeros):
    codes, scales, zero, _ = config_codes(o, k, seed=o + 7 * k, zeros=zeros, scale_dtype=scale_dtype)
    layout = layout_from_codes(codes, scales, zero, None)
    dl = {n: t.to(gpu) for n, t in layout.items()}
    fp6 = _repack(dl["planes"])
    x = torch.randn(1, k, generator=torch.Generator().manual_seed(o)).to(torch.bfloat16)
    out = _gemv_fp6(x, fp6, dl, scale_dtype, o, k, gpu)
    exact = w3.matvec_exact(x.float().numpy(), oracle_layout(layout))
    assert_half_ulp(out.float().cpu().numpy(), exact, "bf16", rel_slack=3e-5, what=f"fp6 {o}x{k}")


@pytest.mark.parametrize("scale", [1e-30, 1e-3, 1.0, 1e4, 1e30])
def test_gemv_fp6_activation_range(gpu, scale):
    """Each group's digit scale follows its max|x| over the activation's range."""
    o, k = 256, 1024
    codes, scales, zero, _ = config_codes(o, k, seed=11, zeros=True, scale_dtype=torch.float16)
    layout = layout_from_codes(codes, scales, zero, None)
    dl = {n: t.to(gpu) for n, t in layout.items()}
    x = (torch.randn(1, k, generator=torch.Generator().manual_seed(2)) * scale).to(torch.bfloat16)
    out = _gemv_fp6(x, _repack(dl["planes"]), dl, torch.float16, o, k, gpu)
    exact = w3.matvec_exact(x.float().numpy(), oracle_layout(layout))
    assert_half_ulp(out.float().cpu().numpy(), exact, "bf16", rel_slack=3e-5, what=f"scale {scale}")


@pytest.mark.parametrize("ratio", [1e2, 1e4])
def test_gemv_fp6_outlier_channels(gpu, ratio):
    """Outlier channels coarsen only their own groups' small values (below 2^-10 of
    the group's max the digits keep 2^-17 of it); the error stays at the scale of
    the zero-point terms, as for the other kernels."""
    o, k = 512, 4096
    codes, scales, zero, _ = config_codes(o, k, seed=3, zeros=True, scale_dtype=torch.float16)
    layout = layout_from_codes(codes, scales, zero, None)
    dl = {n: t.to(gpu) for n, t in layout.items()}
    x = outlier_activations(1, k, ratio=ratio, seed=4, channels=[5, 700, 2049, 4000])
    out = _gemv_fp6(x, _repack(dl["planes"]), dl, torch.float16, o, k, gpu)
    exact = w3.matvec_exact(x.float().numpy(), oracle_layout(layout))
    assert_within_terms(out.float().cpu().numpy(), exact, "bf16", x, layout["scales"], 1e-4, what=f"ratio {ratio}")


def _decode_forms(gpu, o, k, fmt, payload, dl, x, residual, tile_sums, weight, swiglu):
    """residual, normalising and SwiGLU forms of one payload format."""
    lib, s = _lib.library(), _lib.stream_handle(gpu)
    bf = _lib.dtype_code(torch.bfloat16)
    sd = _lib.dtype_code(dl["scales"].dtype)
    res = residual.clone()
    part = torch.empty((o + 15) // 16, dtype=torch.float32, device=gpu)
    _lib.check(lib.fx_w3_gemv_residual(x.data_ptr(), bf, payload.data_ptr(), dl["scales"].data_ptr(), sd,
                                       _lib.ptr(dl.get("zeros")), None, res.data_ptr(), res.data_ptr(), part.data_ptr(),
                                       None, None, o, k, fmt, s), "residual")
    if k > 4096:  # the normalising prologue serves K <= 4096 (the decode's q|k|v and gate|up)
        torch.cuda.synchronize(gpu)
        return res, part, None
    normed = torch.empty(1, o // 2 if swiglu else o, dtype=torch.bfloat16, device=gpu)
    _lib.check(lib.fx_w3_gemv_rmsnormed(x.data_ptr(), bf, payload.data_ptr(), dl["scales"].data_ptr(), sd,
                                        _lib.ptr(dl.get("zeros")), tile_sums.data_ptr(), tile_sums.numel(),
                                        weight.data_ptr(), 1e-6, None, normed.data_ptr(), o, k, int(swiglu), fmt, s),
               "rmsnormed")
    torch.cuda.synchronize(gpu)
    return res, part, normed


@pytest.mark.parametrize("o,k,swiglu", [(4096, 4096, False), (24576, 4096, True), (6144, 4096, False),
                                        (4096, 12288, False)])
def test_decode_forms_match_the_field_layout(gpu, o, k, swiglu):
    codes, scales, zero, _ = config_codes(o, k, seed=o + k, zeros=True, scale_dtype=torch.float16)
    layout = layout_from_codes(codes, scales, zero, None)
    dl = {n: t.to(gpu) for n, t in layout.items()}
    fp6 = _repack(dl["planes"])
    fields = _repack(dl["planes"], "fx_w3_planes_to_fields")
    g = torch.Generator().manual_seed(9)
    x = torch.randn(1, k, generator=g).to(torch.bfloat16).to(gpu)
    residual = torch.randn(1, o, generator=g).to(torch.bfloat16).to(gpu)
    tile_sums = x.float().view(-1, 16).square().sum(-1).contiguous()
    weight = (1 + 0.02 * torch.randn(k, generator=g)).to(torch.bfloat16).to(gpu)
    got = _decode_forms(gpu, o, k, _lib.PAYLOAD_FP6, fp6, dl, x, residual, tile_sums, weight, swiglu)
    want = _decode_forms(gpu, o, k, _lib.PAYLOAD_FIELDS, fields, dl, x, residual, tile_sums, weight, swiglu)
    # both GEMVs are within half an ulp + 3e-5 max|y| of the exact y, so a few ulps
    # of the larger of y and the output apart at most (the residual form adds the
    # rounded y into the residual, where cancellation leaves y's ulp on a small sum)
    r_in = residual.float().cpu().numpy()
    for name, a, b in zip(("residual", "tile sums", "normalised"), got, want):
        if b is None:
            continue
        a, b = a.float().cpu().numpy(), b.float().cpu().numpy()
        if name == "tile sums":
            tol = 2.0 ** -5 * np.abs(b) + 1e-6
        else:
            mag = np.abs(b) + (np.abs(r_in) if name == "residual" else 0.0)
            tol = 2.0 ** (np.floor(np.log2(np.maximum(mag, 1e-30))) - 6) + 1e-4 * mag.max()
        assert np.all(np.abs(a - b) <= tol), (name, float(np.abs(a - b).max()))


def test_fp6_refuses_what_it_cannot_run(gpu):
    lib = _lib.library()
    codes, scales, zero, perm = config_codes(64, 384, seed=1, zeros=True, scale_dtype=torch.float16, permute=True)
    layout = layout_from_codes(codes, scales, zero, perm)
    dl = {n: t.to(gpu) for n, t in layout.items()}
    out = torch.empty(1, 64, dtype=torch.bfloat16, device=gpu)
    x = torch.zeros(1, 384, dtype=torch.bfloat16, device=gpu)
    s = _lib.stream_handle(gpu)
    assert lib.fx_w3_planes_to_fp6(dl["planes"].data_ptr(), out.data_ptr(), 64, 384, s) != 0  # K % 512
    assert lib.fx_w3_gemv_fp6(x.data_ptr(), _lib.dtype_code(torch.bfloat16), dl["planes"].data_ptr(),
                              dl["scales"].data_ptr(), _lib.dtype_code(torch.float16), dl["zeros"].data_ptr(),
                              out.data_ptr(), 64, 384, s) != 0
    xf = torch.zeros(1, 512, dtype=torch.float16, device=gpu)
    assert lib.fx_w3_gemv_fp6(xf.data_ptr(), _lib.dtype_code(torch.float16), dl["planes"].data_ptr(),
                              dl["scales"].data_ptr(), _lib.dtype_code(torch.float16), dl["zeros"].data_ptr(),
                              out.data_ptr(), 64, 512, s) != 0  # fp16 activations
    assert b"bf16" in lib.fx_last_error()


def test_native_decode_session_on_the_fp6_layout(gpu):
    """A whole decode run (NativeDecodeSession, w3_payload="fp6") against the same
    model's run on the field layout: the captured graph replays its own eager
    pass bit for bit, and the logits stay within the activation digits' rounding
    of the field layout's (each GEMV within a few output ulps of the other,
    compounded over three layers and eight steps)."""
    from marlin_style_fluxbin_amd.native_decode import NativeDecodeSession
    from marlin_style_fluxbin_amd.qwen3 import qwen3_config, random_qwen3_model, w3_quantize_qwen3_model

    # hidden and intermediate sizes whose K splits into whole four-group tiles
    config = qwen3_config(hidden_size=512, intermediate_size=1024, num_hidden_layers=3, num_attention_heads=8,
                          num_key_value_heads=2, head_dim=64, vocab_size=384, max_position_embeddings=128)
    model = random_qwen3_model(config, device=gpu, dtype=torch.bfloat16, seed=3)
    w3_quantize_qwen3_model(model)
    g = torch.Generator().manual_seed(6)
    ids = torch.randint(0, 384, (1, 20), generator=g).to(gpu)
    forced = torch.randint(0, 384, (1, 8), generator=g).to(gpu)
    with torch.inference_mode():
        sessions = {fmt: NativeDecodeSession(model, ids, forced, w3_payload=fmt) for fmt in ("fields", "fp6")}
        eager = sessions["fp6"].audit()
        graphs = {fmt: s.capture() for fmt, s in sessions.items()}
        assert torch.equal(graphs["fp6"]["logits"], eager["logits"])
        _, replay = sessions["fp6"].measure("sequence_graph")
        assert torch.equal(replay["logits"], graphs["fp6"]["logits"])
    a, b = graphs["fp6"]["logits"].float(), graphs["fields"]["logits"].float()
    nrmse = float(((a - b).square().mean() / b.square().mean()).sqrt())
    print(f"fp6 against fields: logits NRMSE {nrmse:.3g}", flush=True)
    # a wrong field, pairing or digit moves the logits by O(1) relative
    assert nrmse <= 0.03, nrmse
    with pytest.raises(ValueError, match="w3_payload"):
        NativeDecodeSession(model, ids, forced, w3_payload="fp4")
