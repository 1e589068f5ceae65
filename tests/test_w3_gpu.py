"""GPU parity of the HIP W3 GEMV against the oracle (runs on the MI355X box).

Truths (oracle/w3.py, pinned in tests/test_oracle_w3.py):
* ``matvec_exact``   float64 x @ (s*(q-z)).T -- the structural route's target;
* ``matvec_decoded`` float64 x @ restore(W).T -- dequantize-then-matmul, the
  decoded_bf16 route's target and the reference's dense fallback value.
Tolerances (normwise max relative error, max|a-b|/max|b|):
* fp32 kernel results (single K split, no output cast) vs their own truth: 1e-5;
* fp16/bf16 outputs vs their own truth: 2^-8 (one output rounding) + 1e-5;
* any route vs dequantize-then-matmul: 1e-3 (fp32) / 1e-2 (bf16), the stated bar.
"""
import numpy as np
import pytest
import torch

from marlin_style_fluxbin_amd import (
    PackedW3Linear, W3Gemv, bf16_weight_semantics_w3_matvec, restore_planar_w3, structural_w3_matvec,
    w3_lut_m1_out, workspace_shape,
)
from oracle import w3
from tests.payloads import assert_half_ulp, assert_rel, config_codes, layout_from_codes, oracle_layout

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-5
HALF_TOL = 2.0 ** -8 + 1e-5


def _setup(o, k, *, seed=0, zeros=True, scale_dtype=torch.bfloat16, permute=False, device="cuda"):
    codes, scales, z, perm = config_codes(o, k, seed=seed, zeros=zeros, scale_dtype=scale_dtype, permute=permute)
    layout = layout_from_codes(codes, scales, z, perm)
    return layout, {name: t.to(device) for name, t in layout.items()}, oracle_layout(layout)


def _x(m, k, dtype, seed=1):
    return torch.randn(m, k, generator=torch.Generator().manual_seed(seed)).to(dtype)


SMALL = [(64, 256), (288, 384), (1, 128), (17, 256), (65, 384), (1025, 512), (300, 1280)]


@pytest.mark.parametrize("o,k", SMALL)
@pytest.mark.parametrize("m", [1, 2, 4, 8])
@pytest.mark.parametrize("zeros,permute", [(False, False), (True, True)])
def test_structural_fp32_matches_exact(gpu, o, k, m, zeros, permute):
    layout, dl, ol = _setup(o, k, seed=o + k, zeros=zeros, permute=permute)
    x = _x(m, k, torch.bfloat16, seed=m)
    got = structural_w3_matvec(x.to(gpu), dl).cpu().numpy()
    assert_rel(got, w3.matvec_exact(x.float().numpy(), ol), FP32_TOL)


@pytest.mark.parametrize("o,k", SMALL)
@pytest.mark.parametrize("zeros", [False, True])
def test_decoded_fp32_matches_dequantize_then_matmul(gpu, o, k, zeros):
    layout, dl, ol = _setup(o, k, seed=3 * o + k, zeros=zeros)
    x = _x(1, k, torch.bfloat16, seed=o)
    got = bf16_weight_semantics_w3_matvec(x.to(gpu), dl).cpu().numpy()
    assert_rel(got, w3.matvec_decoded(x.float().numpy(), ol, "bf16"), FP32_TOL)


@pytest.mark.parametrize("o,k", SMALL)
@pytest.mark.parametrize("m", [1, 3, 8])
@pytest.mark.parametrize("xdtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("scale_dtype", [torch.bfloat16, torch.float16])
def test_fused_fast_path(gpu, o, k, m, xdtype, scale_dtype):
    layout, dl, ol = _setup(o, k, seed=o * 7 + m, zeros=True, scale_dtype=scale_dtype, permute=True)
    x = _x(m, k, xdtype, seed=k + m)
    gemv = W3Gemv(dl)
    out = torch.full((m, o), float("nan"), dtype=xdtype, device=gpu)
    gemv(x.to(gpu), out)
    exact = w3.matvec_exact(x.float().numpy(), ol)
    got = out.float().cpu().numpy()
    assert_rel(got, exact, HALF_TOL)
    # fp16 activations run on the fp16 MFMA, whose products with subnormal fp16
    # code operands round at ~2e-7 relative (measured per instruction); bf16 is exact
    slack = 2e-6 if xdtype == torch.bfloat16 else 3e-5
    assert_half_ulp(got, exact, "bf16" if xdtype == torch.bfloat16 else "f16", rel_slack=slack)
    # a second call through the same workspace is bit-identical
    again = torch.empty_like(out)
    gemv(x.to(gpu), again)
    assert torch.equal(out, again)


@pytest.mark.parametrize("row_tile", [256, 512, 1024])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_reference_split_contract(gpu, row_tile, dtype):
    """Reference tests/test_w3_lut_correctness.py:51-135: NaN-poisoned workspace,
    repeat-exact after re-poisoning, graph replay bit-equality, both arithmetics."""
    for out_features, in_features in ((32, 128), (64, 256), (288, 384)):
        layout, dl, ol = _setup(out_features, in_features, seed=out_features, zeros=False)
        x = _x(1, in_features, dtype, seed=in_features).to(gpu)
        exact = w3.matvec_exact(x.float().cpu().numpy(), ol)
        for gps in sorted({1, in_features // 128}):
            out = torch.empty(1, out_features, device=gpu, dtype=dtype)
            workspace = torch.full(workspace_shape(out_features, in_features, gps), float("nan"), device=gpu)

            def run():
                return w3_lut_m1_out(x, dl, out, workspace, row_tile=row_tile, groups_per_split=gps)

            run()
            torch.cuda.synchronize()
            if workspace.shape[0] == 1:
                assert torch.isnan(workspace).all()
            else:
                assert torch.isfinite(workspace).all()
            assert_rel(out.float().cpu().numpy(), exact, HALF_TOL)
            saved = out.clone()
            workspace.fill_(float("nan"))
            run()
            assert torch.equal(out, saved)
            graph = torch.cuda.CUDAGraph()
            for _ in range(3):
                run()
            torch.cuda.synchronize()
            with torch.cuda.graph(graph):
                run()
            for _ in range(3):
                out.zero_()
                graph.replay()
                torch.cuda.synchronize()
                assert torch.equal(out, saved)
        if dtype == torch.bfloat16:
            decoded = w3.matvec_decoded(x.float().cpu().numpy(), ol, "bf16")
            for gps in (1, in_features // 128):
                corrected = torch.empty(1, out_features, device=gpu, dtype=dtype)
                ws = torch.full(workspace_shape(out_features, in_features, gps), float("nan"), device=gpu)
                w3_lut_m1_out(x, dl, corrected, ws, row_tile=256, groups_per_split=gps, arithmetic="decoded_bf16")
                assert_rel(corrected.float().cpu().numpy(), decoded, HALF_TOL)


def test_fused_path_graph_replays_track_input(gpu):
    """Graph-captured single-launch GEMV: every replay equals the eager result for
    the current input (the in-launch split counters must reset every time)."""
    layout, dl, ol = _setup(4096, 4096, seed=11, zeros=True, scale_dtype=torch.float16)
    gemv = W3Gemv(dl)
    x = _x(1, 4096, torch.bfloat16, seed=12).to(gpu)
    out = torch.empty(1, 4096, dtype=torch.bfloat16, device=gpu)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(3):
            gemv(x, out)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        gemv(x, out)
    for step in range(4):
        x.mul_(0.5 if step % 2 else -1.25)
        eager = torch.empty_like(out)
        gemv(x, eager)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), step


QWEN3_SHAPES = [(4096, 4096), (1024, 4096), (12288, 4096), (4096, 12288)]


@pytest.mark.parametrize("o,k", QWEN3_SHAPES)
@pytest.mark.parametrize("m", [1, 2, 4, 8])
def test_qwen3_shapes_config1(gpu, o, k, m):
    """Config 1: every Qwen3-8B Linear shape, W3 g128, fp16 scales, zeros U{3,4}."""
    layout, dl, ol = _setup(o, k, seed=0, zeros=True, scale_dtype=torch.float16)
    x = _x(m, k, torch.bfloat16, seed=0)
    exact = w3.matvec_exact(x.float().numpy(), ol)
    if m in (1, 2, 4, 8):
        got32 = structural_w3_matvec(x.to(gpu), dl).cpu().numpy()
        assert_rel(got32, exact, FP32_TOL)
    gemv = W3Gemv(dl)
    out = torch.empty(m, o, dtype=torch.bfloat16, device=gpu)
    gemv(x.to(gpu), out)
    got = out.float().cpu().numpy()
    assert_rel(got, exact, HALF_TOL)
    assert_half_ulp(got, exact, "bf16")
    # the stated bar against dequantize-then-matmul (bf16 weights from fp16 scales)
    decoded = w3.matvec_decoded(x.float().numpy(), ol, "bf16")
    assert_rel(got, decoded, 1e-2)


def test_config0_q_proj_seed0(gpu):
    """Config 0: q_proj 4096x4096, x N(0,1) bf16, fp16 scales U[0.005,0.02], zeros U{3,4}, seed 0."""
    layout, dl, ol = _setup(4096, 4096, seed=0, zeros=True, scale_dtype=torch.float16)
    x = _x(1, 4096, torch.bfloat16, seed=0)
    module = PackedW3Linear(dl, row_tile=256)
    with torch.inference_mode():
        y = module(x.to(gpu))
    assert module.route_counts == {"packed_m1": 1, "dense_fallback": 0}
    exact = w3.matvec_exact(x.float().numpy(), ol)
    assert_rel(y.float().cpu().numpy(), exact, HALF_TOL)
    got32 = structural_w3_matvec(x.to(gpu), dl).cpu().numpy()
    assert_rel(got32, exact, FP32_TOL)


@pytest.mark.parametrize("scale_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("weight_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("zeros", [False, True])
@pytest.mark.parametrize("o,k,order", [(96, 384, "random"), (37, 256, "identity"), (1041, 1024, "mixed")])
def test_restore_kernel_bitwise(gpu, scale_dtype, weight_dtype, zeros, o, k, order):
    """The dense weight bit for bit against the oracle's restore.  Orders: a
    scattered permutation (every value stored alone), the identity (16-byte row
    stores), and one that moves columns inside a few 8-column runs only (both
    store forms in one launch); row counts off the 16-row workgroup tile."""
    codes, scales, z, perm = config_codes(o, k, seed=o + k, zeros=zeros, scale_dtype=scale_dtype,
                                          permute=order == "random")
    if order == "mixed":
        perm = torch.arange(k, dtype=torch.int16)
        for start in (8, 136, 520, 1000):
            perm[start:start + 8] = perm[start:start + 8].flip(0)
        perm[300], perm[700] = 700, 300
    layout = layout_from_codes(codes, scales, z, perm)
    dl = {name: t.to(gpu) for name, t in layout.items()}
    got = restore_planar_w3(dl, dtype=weight_dtype).float().cpu().numpy()
    expected = w3.restore_weight(oracle_layout(layout), "bf16" if weight_dtype == torch.bfloat16 else "f16")
    assert np.array_equal(got, expected)


def test_restore_kernel_permutation_edge_entries(gpu):
    """The permuted form: an identity order passed as a permutation gives the
    NULL form's bits; an entry outside [0, K) is skipped, so the column that no
    entry names is zero."""
    from marlin_style_fluxbin_amd.w3_lut_deployment import restore_planar_w3_into

    layout, dl, ol = _setup(33, 768, seed=6, zeros=True)
    want = w3.restore_weight(ol, "bf16")
    as_perm = torch.empty(33, 768, dtype=torch.bfloat16, device=gpu)
    restore_planar_w3_into(dl, as_perm, perm_identity=False)
    assert np.array_equal(as_perm.float().cpu().numpy(), want)
    bad = dl["perm"].clone()
    bad[5], bad[600] = -3, 30000
    skipped = torch.full((33, 768), 7.0, dtype=torch.bfloat16, device=gpu)
    restore_planar_w3_into(dict(dl, perm=bad), skipped, perm_identity=False)
    want[:, [5, 600]] = 0
    assert np.array_equal(skipped.float().cpu().numpy(), want)


@pytest.mark.parametrize("order", ["identity", "random"])
def test_restore_kernel_unaligned_pointers(gpu, order):
    """A weight, then a permutation, 2 bytes off 16-byte alignment (element stores,
    element permutation loads): the same bits."""
    from marlin_style_fluxbin_amd.w3_lut_deployment import restore_planar_w3_into

    layout, dl, ol = _setup(40, 512, seed=2, zeros=True, permute=order == "random")
    want = w3.restore_weight(ol, "bf16")
    buf = torch.empty(40 * 512 + 1, dtype=torch.bfloat16, device=gpu)
    weight = buf[1:].view(40, 512)
    assert weight.data_ptr() % 16 == 2
    restore_planar_w3_into(dl, weight)
    assert np.array_equal(weight.float().cpu().numpy(), want)
    pbuf = torch.empty(513, dtype=torch.int16, device=gpu)
    pbuf[1:].copy_(dl["perm"])
    shifted = dict(dl, perm=pbuf[1:])
    assert shifted["perm"].data_ptr() % 16 == 2
    aligned = torch.empty(40, 512, dtype=torch.bfloat16, device=gpu)
    restore_planar_w3_into(shifted, aligned)
    assert np.array_equal(aligned.float().cpu().numpy(), want)


def test_dense_fallback_on_gpu_uses_device_restore(gpu):
    layout, dl, ol = _setup(64, 256, seed=4, zeros=False)
    module = PackedW3Linear(dl, fallback="dense", row_tile=256)
    x = _x(16, 256, torch.bfloat16, seed=4).to(gpu)
    with torch.inference_mode():
        y = module(x)
    assert module.route_counts["dense_fallback"] == 1
    decoded = w3.matvec_decoded(x.float().cpu().numpy(), ol, "bf16")
    assert_rel(y.float().cpu().numpy(), decoded, 1e-2)


def test_bias_is_added_in_place_as_the_reference_does(gpu):
    """PackedW3Linear adds its bias into the output in place (w3_lut_deployment.py:
    313-314, 357-358): a float32 bias leaves a bf16 output bf16, on the packed route
    and on the bound decode route, and the sum is rounded once."""
    layout, dl, ol = _setup(64, 256, seed=9, zeros=False)
    bias = torch.randn(64, generator=torch.Generator().manual_seed(3)).to(gpu)
    x = _x(1, 256, torch.bfloat16, seed=9).to(gpu)
    plain = PackedW3Linear(dl, row_tile=256)
    module = PackedW3Linear(dl, bias=bias, row_tile=256)
    with torch.inference_mode():
        y0 = plain(x)
        y = module(x)
        assert y.dtype == torch.bfloat16
        assert torch.equal(y, (y0.float() + bias).to(torch.bfloat16))
        module.bind_prepared_decode(torch.bfloat16)
        yb = module(x.view(1, 1, 256))
        assert yb.dtype == torch.bfloat16 and torch.equal(yb.view(1, 64), y)


@pytest.mark.parametrize("o,k", [(4096, 4096), (12288, 4096), (4096, 12288), (1024, 4096)])
@pytest.mark.parametrize("route", ["fast_corrected", "observed_exact", "structural"])
def test_module_routes_follow_the_reference_split_contract(gpu, o, k, route):
    """PackedW3Linear carries its route's groups_per_split and arithmetic onto the
    packed route (reference w3_lut_deployment.py:293-312): a decoded_bf16 or split
    route is bit-equal to w3_lut_m1_out with the same row tile and split, in eager
    and prepared form, and within the stated bars of its truth."""
    from marlin_style_fluxbin_amd import qwen3_w3_route

    layout, dl, ol = _setup(o, k, seed=5, zeros=True, scale_dtype=torch.bfloat16)
    policy = qwen3_w3_route(route, o, k)
    module = PackedW3Linear(dl, route=route, **policy)
    x = _x(1, k, torch.bfloat16, seed=6).to(gpu)
    with torch.inference_mode():
        y = module(x)
    assert module.route_counts == {"packed_m1": 1, "dense_fallback": 0}
    truth = (w3.matvec_decoded(x.float().cpu().numpy(), ol, "bf16") if policy["arithmetic"] == "decoded_bf16"
             else w3.matvec_exact(x.float().cpu().numpy(), ol))
    assert_half_ulp(y.float().cpu().numpy(), truth, "bf16", rel_slack=1e-5)
    if module.uses_table_route:
        ws = torch.full(workspace_shape(o, k, policy["groups_per_split"]), float("nan"), device=gpu)
        want = torch.empty(1, o, dtype=torch.bfloat16, device=gpu)
        w3_lut_m1_out(x, dl, want, ws, row_tile=policy["row_tile"], groups_per_split=policy["groups_per_split"],
                      arithmetic=policy["arithmetic"])
        assert torch.equal(y.view(torch.int16), want.view(torch.int16))
    module.bind_prepared_decode(torch.bfloat16)
    module._decode_audit = True
    with torch.inference_mode():
        prepared = module(x.view(1, 1, k))
    assert torch.equal(prepared.view(1, o).view(torch.int16), y.view(torch.int16))
    assert module.route_counts == {"packed_m1": 2, "dense_fallback": 0}


def test_module_small_m_opt_in(gpu):
    layout, dl, ol = _setup(1024, 4096, seed=7, zeros=True, scale_dtype=torch.float16)
    x = _x(4, 4096, torch.bfloat16, seed=7).to(gpu)
    default = PackedW3Linear(dl, fallback="dense", row_tile=512)
    opted = PackedW3Linear(dl, row_tile=512, max_packed_rows=8)
    with torch.inference_mode():
        dense = default(x)
        packed = opted(x)
    assert default.route_counts == {"packed_m1": 0, "dense_fallback": 1}
    assert opted.route_counts == {"packed_m1": 0, "dense_fallback": 0, "packed_small_m": 1}
    want = torch.empty(4, 1024, dtype=torch.bfloat16, device=gpu)
    W3Gemv(dl)(x, want)
    assert torch.equal(packed.view(torch.int16), want.view(torch.int16))
    assert_rel(dense.float().cpu().numpy(), w3.matvec_decoded(x.float().cpu().numpy(), ol, "bf16"), 1e-2)


def test_engine_w3_backend_apply_out(gpu):
    from marlin_style_fluxbin_amd.engine_interface import W3Backend

    layout, dl, ol = _setup(4096, 4096, seed=8, zeros=True, scale_dtype=torch.float16, permute=True)
    backend = W3Backend(allow_zeros=True, scale_dtype=torch.float16)
    workspace = torch.empty(backend.workspace_shape(4096, 4096), dtype=torch.uint8, device=gpu)
    for m in (1, 3):
        x = _x(m, 4096, torch.bfloat16, seed=m).to(gpu)
        out = torch.empty(m, 4096, dtype=torch.bfloat16, device=gpu)
        backend.apply_out(x, dl, out, workspace)
        want = torch.empty_like(out)
        W3Gemv(dl)(x, want)
        assert torch.equal(out.view(torch.int16), want.view(torch.int16))
    assert_half_ulp(out.float().cpu().numpy(), w3.matvec_exact(x.float().cpu().numpy(), ol), "bf16")
