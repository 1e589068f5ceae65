"""GPU parity of the MFMA W3 GEMV (the fast structural path) against the float64 oracle.

Every output element must lie within half an output ulp of the exact value
x @ (s*(q-z)).T plus 2e-6 * max|y| (fp32 accumulation before the final cast),
for every tiling variant, K split, activation-row count and dtype combination.
fp16 activations use 3e-5: the fp16 MFMA rounds products with subnormal fp16
operands at ~2e-7 relative per instruction (bf16 MFMA is exact).
"""
import numpy as np
import pytest
import torch

from marlin_style_fluxbin_amd import _lib
from oracle import w3
from tests.payloads import (assert_half_ulp, assert_within_terms, config_codes, layout_from_codes, oracle_layout,
                            outlier_activations, silence_columns)

pytestmark = pytest.mark.gpu

# (waves, batches in flight per wave, groups per K split, 16-row tiles per wave)
PLANS = [(4, 1, 4, 1), (4, 2, 8, 2), (4, 1, 16, 2), (8, 1, 32, 1), (8, 2, 16, 1), (8, 2, 12, 2),
         (8, 1, 64, 2), (4, 2, 32, 1)]


def _run_config(dl, x, out, waves, prefetch, gps, tiles, use_perm=True):
    lib = _lib.library()
    m, k = x.shape
    o = out.shape[1]
    nbytes = lib.fx_w3_gemv_config_workspace_bytes(m, o, k, waves, prefetch, gps, tiles)
    ws = torch.empty(nbytes + 256, dtype=torch.uint8, device=x.device)
    perm = dl["perm"].data_ptr() if use_perm else None
    _lib.check(lib.fx_w3_gemv_config(
        x.data_ptr(), _lib.dtype_code(x.dtype), dl["planes"].data_ptr(), dl["scales"].data_ptr(),
        _lib.dtype_code(dl["scales"].dtype), _lib.ptr(dl.get("zeros")), perm,
        ws.data_ptr(), nbytes, out.data_ptr(), m, o, k, waves, prefetch, gps, tiles,
        _lib.stream_handle(x.device)),
        "fx_w3_gemv_config")


@pytest.mark.parametrize("o,k", [(64, 512), (37, 1536), (300, 2048), (1, 128), (17, 384)])
@pytest.mark.parametrize("plan", PLANS)
@pytest.mark.parametrize("m", [1, 2, 3, 4, 8])
@pytest.mark.parametrize("permute", [True, False])
def test_mfma_plans(gpu, o, k, plan, m, permute):
    """Every tiling (waves, prefetch depth, K split, row tiles) at ragged O, K and
    M, with a random group-preserving permutation (gathered in the kernel) and
    with the identity passed as a null permutation."""
    codes, scales, zeros, perm = config_codes(o, k, seed=o + k + m, zeros=True, scale_dtype=torch.float16,
                                              permute=permute)
    layout = layout_from_codes(codes, scales, zeros, perm)
    dl = {n: t.to(gpu) for n, t in layout.items()}
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(m)).to(torch.bfloat16)
    out = torch.full((m, o), float("nan"), dtype=torch.bfloat16, device=gpu)
    _run_config(dl, x.to(gpu), out, *plan, use_perm=permute)
    exact = w3.matvec_exact(x.float().numpy(), oracle_layout(layout))
    assert_half_ulp(out.float().cpu().numpy(), exact, "bf16", what=f"plan {plan} m {m} perm {permute}")


@pytest.mark.parametrize("xdtype,tag", [(torch.bfloat16, "bf16"), (torch.float16, "f16")])
@pytest.mark.parametrize("scale_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("zeros", [False, True])
def test_mfma_dtypes_and_zero_modes(gpu, xdtype, tag, scale_dtype, zeros):
    codes, scales, z, perm = config_codes(256, 1024, seed=5, zeros=zeros, scale_dtype=scale_dtype)
    layout = layout_from_codes(codes, scales, z, perm)
    dl = {n: t.to(gpu) for n, t in layout.items()}
    x = torch.randn(1, 1024, generator=torch.Generator().manual_seed(3)).to(xdtype)
    out = torch.empty(1, 256, dtype=xdtype, device=gpu)
    _run_config(dl, x.to(gpu), out, 8, 2, 8, 2)
    exact = w3.matvec_exact(x.float().numpy(), oracle_layout(layout))
    # fp16 MFMA products with subnormal fp16 code operands round at ~2e-7 relative
    assert_half_ulp(out.float().cpu().numpy(), exact, tag, rel_slack=2e-6 if tag == "bf16" else 3e-5)


@pytest.mark.parametrize("scale", [1e-30, 1e-6, 1.0, 1e6, 1e30])
def test_mfma_activation_range(gpu, scale):
    """The per-row exponent offset keeps tiny and huge activations exact."""
    codes, scales, z, perm = config_codes(128, 512, seed=2, zeros=True, scale_dtype=torch.bfloat16)
    layout = layout_from_codes(codes, scales, z, perm)
    dl = {n: t.to(gpu) for n, t in layout.items()}
    x = (torch.randn(1, 512, generator=torch.Generator().manual_seed(4)) * scale).to(torch.bfloat16)
    out = torch.empty(1, 128, dtype=torch.bfloat16, device=gpu)
    _run_config(dl, x.to(gpu), out, 4, 1, 4, 1)
    exact = w3.matvec_exact(x.float().numpy(), oracle_layout(layout))
    assert np.all(np.isfinite(out.float().cpu().numpy()))
    assert_half_ulp(out.float().cpu().numpy(), exact, "bf16", what=f"scale {scale}")


@pytest.mark.parametrize("ratio", [10.0, 1e3, 1e4, 2.0 ** 20])
@pytest.mark.parametrize("plan,m,permute", [((8, 1, 32, 1), 1, False), ((4, 2, 8, 2), 3, True),
                                            ((8, 1, 4, 1), 8, True)])
def test_mfma_outlier_channels(gpu, ratio, plan, m, permute):
    """A few channels `ratio` times larger than the rest of their group (Qwen3's
    massive activations), with half of the rows' weights on those channels
    exactly zero.  Each (group, row) exponent follows the outlier and the bf16
    operands keep every other element exact, so every row, the small ones
    included, lies within half an ulp plus 2^-20 of its terms' scale
    (11 max(s) sum|x|, the scale of the unsigned dot and the zero-point term the
    kernel adds); a flush of the outlier groups' small elements misses that bar
    (pinned on the CPU in tests/test_oracle_w3.py)."""
    o, k = 96, 1024
    codes, scales, zeros, perm = config_codes(o, k, seed=11, zeros=True, scale_dtype=torch.float16,
                                              permute=permute)
    channels = [5, 300, 301, 777]
    silence_columns(codes, zeros, perm, channels, np.arange(0, o, 2))
    layout = layout_from_codes(codes, scales, zeros, perm)
    dl = {n: t.to(gpu) for n, t in layout.items()}
    x = outlier_activations(m, k, ratio=ratio, seed=m, channels=channels)
    out = torch.full((m, o), float("nan"), dtype=torch.bfloat16, device=gpu)
    _run_config(dl, x.to(gpu), out, *plan, use_perm=permute)
    exact = w3.matvec_exact(x.float().numpy(), oracle_layout(layout))
    assert_within_terms(out.float().cpu().numpy(), exact, "bf16", x, scales, 2.0 ** -20, what=f"ratio {ratio}")


def test_mfma_zero_activation(gpu):
    codes, scales, z, perm = config_codes(64, 256, seed=1)
    layout = layout_from_codes(codes, scales, z, perm)
    dl = {n: t.to(gpu) for n, t in layout.items()}
    out = torch.full((1, 64), float("nan"), dtype=torch.bfloat16, device=gpu)
    _run_config(dl, torch.zeros(1, 256, dtype=torch.bfloat16, device=gpu), out, 4, 1, 4, 2)
    assert torch.equal(out, torch.zeros_like(out))


@pytest.mark.parametrize("o,k", [(300, 2048), (96, 12288), (17, 640)])
@pytest.mark.parametrize("m", [1, 3])
def test_mfma_result_independent_of_waves_and_prefetch(gpu, o, k, m):
    """With one K split the K reduction always runs in the eight-wave order, so
    every (waves, prefetch, row tiles) tiling gives bitwise-equal outputs; a
    fused q|k|v or gate|up payload therefore reproduces the separate projections
    whatever plan each shape gets."""
    codes, scales, zeros, perm = config_codes(o, k, seed=o + m, zeros=True, scale_dtype=torch.float16,
                                              permute=True)
    dl = {n: t.to(gpu) for n, t in layout_from_codes(codes, scales, zeros, perm).items()}
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(k)).to(torch.bfloat16).to(gpu)
    padded = (k // 128 + 3) // 4 * 4
    outs = []
    for waves, prefetch, tiles in [(8, 1, 1), (4, 1, 1), (4, 2, 1), (8, 2, 2), (4, 1, 2)]:
        out = torch.full((m, o), float("nan"), dtype=torch.bfloat16, device=gpu)
        _run_config(dl, x, out, waves, prefetch, padded, tiles)
        outs.append(out)
    for out in outs[1:]:
        assert torch.equal(out, outs[0])


def _decoded(gpu, x, dl, o):
    """fx_w3_gemv with decoded_bf16 arithmetic (one row: the MFMA kernel with the
    +-3 correction chain)."""
    from marlin_style_fluxbin_amd.w3_lut_deployment import W3Gemv

    out = torch.full((x.shape[0], o), float("nan"), dtype=x.dtype, device=gpu)
    W3Gemv(dl, arithmetic="decoded_bf16")(x.to(gpu), out)
    return out


@pytest.mark.parametrize("o,k", [(4096, 4096), (1024, 4096), (12288, 4096), (4096, 12288), (37, 1536), (300, 2048)])
@pytest.mark.parametrize("permute", [False, True])
@pytest.mark.parametrize("zeros", [True, False])
def test_mfma_decoded_bf16_matches_the_decoded_oracle(gpu, o, k, permute, zeros):
    """decoded_bf16 on the matrix cores: each weight bf16(s (q - z)), zero-points 3 / 4
    (or the implicit 4), against the float64 dot with the oracle's restored weight
    (``oracle.w3.matvec_decoded``): half a bf16 ulp plus the fp32 accumulation.  The
    same payload's structural result differs from it (the correction is live)."""
    print(f"decoded_bf16 MFMA {o}x{k} perm {permute} zeros {zeros}", flush=True)
    codes, scales, zero, perm = config_codes(o, k, seed=o + k, zeros=zeros, scale_dtype=torch.bfloat16,
                                             permute=permute)
    layout = layout_from_codes(codes, scales, zero, perm)
    dl = {n: t.to(gpu) for n, t in layout.items()}
    x = torch.randn(1, k, generator=torch.Generator().manual_seed(k)).to(torch.bfloat16)
    got = _decoded(gpu, x, dl, o).float().cpu().numpy()
    truth = w3.matvec_decoded(x.float().numpy(), oracle_layout(layout), "bf16")
    assert_half_ulp(got, truth, "bf16", rel_slack=2e-6, what=f"decoded {o}x{k}")
    if o >= 1024:  # the correction is live: some outputs round differently from the structural kernel's
        from marlin_style_fluxbin_amd.w3_lut_deployment import W3Gemv

        structural = torch.empty(1, o, dtype=torch.bfloat16, device=gpu)
        W3Gemv(dl)(x.to(gpu), structural)
        assert (structural.float().cpu().numpy() != got).any()


@pytest.mark.parametrize("xdtype,tag,slack", [(torch.float16, "f16", 3e-5), (torch.bfloat16, "bf16", 2e-6)])
def test_mfma_decoded_bf16_activation_dtypes_and_outliers(gpu, xdtype, tag, slack):
    """fp16 activations (the fp16 MFMA rounds products of subnormal operands at
    ~2e-7 relative, hence 3e-5), and an outlier channel 2^10 times its group."""
    o, k = 512, 4096
    codes, scales, zero, _ = config_codes(o, k, seed=3, zeros=True, scale_dtype=torch.bfloat16)
    layout = layout_from_codes(codes, scales, zero, None)
    dl = {n: t.to(gpu) for n, t in layout.items()}
    for x in (torch.randn(1, k, generator=torch.Generator().manual_seed(1)).to(xdtype),
              outlier_activations(1, k, ratio=2.0 ** 10, seed=2, channels=[130, 2000], dtype=xdtype)):
        got = _decoded(gpu, x, dl, o).float().cpu().numpy()
        truth = w3.matvec_decoded(x.float().numpy(), oracle_layout(layout), "bf16")
        assert_half_ulp(got, truth, tag, rel_slack=slack, what=f"decoded {tag}")


def test_mfma_decoded_bf16_rejects_fp16_scales(gpu):
    lib = _lib.library()
    t = torch.zeros(3 * 16 * 16, dtype=torch.uint8, device=gpu)
    x = torch.zeros(1, 128, dtype=torch.bfloat16, device=gpu)
    sc = torch.ones(1, 16, dtype=torch.float16, device=gpu)
    out = torch.zeros(1, 16, dtype=torch.bfloat16, device=gpu)
    rc = lib.fx_w3_gemv(x.data_ptr(), 2, t.data_ptr(), sc.data_ptr(), 1, None, None, None, 0, out.data_ptr(), 1, 16,
                        128, _lib.ARITH_DECODED_BF16, None)
    assert rc == 1 and "bf16 scales" in lib.fx_last_error().decode()
