"""GPU parity of the hybrid g128/s8 two-base GEMV (``fx_hybrid_gemv`` via ``m1_out``
and ``PackedHybridLinear``) against the float64 ``oracle.two_base.structural_reference``.

Bars: the reference's structural gate for bf16 outputs (``factored_reference.py``:
every |err| <= 0.02 (rms + |ref|), normalized RMSE <= 0.005), and the tighter
normwise max relative error 2^-8 for bf16 / fp16 outputs (output rounding plus the
kernel's 16-bit fixed-point activation operands).  Tails, K splits, both layout
families, refinement columns (basis vectors), streams, graphs and the prepared
decode binding are covered, after the reference's CUDA tests
(``tests/test_deployment.py:179-276``).
"""
import numpy as np
import pytest
import torch

from marlin_style_fluxbin_amd import deployment as d
from oracle import two_base as tb

pytestmark = pytest.mark.gpu

DT = {"bf16": torch.bfloat16, "f16": torch.float16}


def _payload(o, g, seed=19):
    return {k: torch.from_numpy(v) for k, v in tb.make_hybrid_payload(o, g, seed=seed).items()}


def _layout(p, kernel, device):
    return {k: v.to(device) for k, v in d.convert_artifact(p, kernel=kernel).items()}


def _reference(x, p):
    layout = tb.convert_artifact({k: v.numpy() for k, v in p.items()})
    return tb.structural_reference(x.float().cpu().numpy().astype(np.float64), layout)


def _check(y, ref):
    got = y.float().cpu().numpy().astype(np.float64)
    assert np.all(np.isfinite(got))
    rms = float(np.sqrt(np.mean(ref ** 2)))
    assert np.all(np.abs(got - ref) <= 0.02 * (rms + np.abs(ref)) + 1e-6)
    nrmse = float(np.sqrt(np.mean((got - ref) ** 2)) / max(rms, 1e-30))
    assert nrmse <= 0.005, nrmse
    assert float(np.max(np.abs(got - ref)) / max(np.max(np.abs(ref)), 1e-30)) <= 2 ** -8


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("o,g", [(1, 1), (7, 3), (17, 3), (65, 10), (1025, 2), (300, 32), (12288, 32), (4096, 96)])
def test_m1_out_matches_structural_reference(gpu, dtype, o, g):
    p = _payload(o, g, seed=o + g)
    layout = _layout(p, "v5_p1024", gpu)
    x = torch.randn(1, g * 128, generator=torch.Generator().manual_seed(o)).to(DT[dtype])
    ref = _reference(x, p)
    for gps in (1, 8, 1024):
        ws = torch.full(d.workspace_shape(o, g * 128, gps), float("nan"), device=gpu)
        y = torch.empty(1, o, dtype=DT[dtype], device=gpu)
        d.m1_out(x.to(gpu), layout, y, ws, groups_per_split=gps, kernel="v5_p1024")
        _check(y, ref)


@pytest.mark.parametrize("kernel", ["v1", "v4", "v5", "v5_p256"])
def test_interleaved_and_planar_kernels_agree(gpu, kernel):
    o, g = 65, 10
    p = _payload(o, g, seed=3)
    x = torch.randn(1, g * 128, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).to(gpu)
    planar = _layout(p, "v5_p1024", gpu)
    ws = torch.empty(d.workspace_shape(o, g * 128, 8, kernel=kernel), device=gpu)
    want = torch.empty(1, o, dtype=torch.bfloat16, device=gpu)
    d.m1_out(x, planar, want, torch.empty(d.workspace_shape(o, g * 128, 8), device=gpu), kernel="v5_p1024")
    y = torch.empty_like(want)
    d.m1_out(x, _layout(p, kernel, gpu), y, ws, kernel=kernel)
    assert torch.equal(y, want)


def test_basis_vectors_hit_main_and_refinement_columns(gpu):
    o, g = 48, 3
    p = _payload(o, g, seed=7)
    layout = _layout(p, "v5_p512", gpu)
    w = tb.materialize_hybrid({k: v.numpy() for k, v in p.items()}).astype(np.float64)
    cols = [0, 1, 7, 8, 100, 127, 128, 383] + [128 * gi + int(c) for gi in range(g) for c in p["refinement_indices"][gi][:2]]
    ws = torch.empty(d.workspace_shape(o, g * 128), device=gpu)
    for col in cols:
        x = torch.zeros(1, g * 128, dtype=torch.bfloat16, device=gpu)
        x[0, col] = 1.0
        y = torch.empty(1, o, dtype=torch.bfloat16, device=gpu)
        d.m1_out(x, layout, y, ws, kernel="v5_p512")
        got = y.float().cpu().numpy()[0]
        want = w[:, col]
        assert np.max(np.abs(got - want)) <= 2 ** -7 * np.max(np.abs(w)), col


def test_streams_graphs_and_repeated_calls(gpu):
    o, g = 1025, 4
    p = _payload(o, g, seed=5)
    layout = _layout(p, "v5_p1024", gpu)
    x = torch.randn(1, g * 128, device=gpu).to(torch.bfloat16)
    ws = torch.full(d.workspace_shape(o, g * 128, 1), float("nan"), device=gpu)
    y = torch.empty(1, o, dtype=torch.bfloat16, device=gpu)

    def run():
        d.m1_out(x, layout, y, ws, groups_per_split=1, kernel="v5_p1024")

    run()
    saved = y.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ws.fill_(float("nan"))
        run()
    torch.cuda.current_stream().wait_stream(side)
    assert torch.equal(saved, y)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    for _ in range(3):
        y.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(saved, y)
    with pytest.raises(RuntimeError):
        d.m1_out(x.expand(2, -1).contiguous(), layout, y, ws, kernel="v5_p1024")


@pytest.mark.parametrize("kernel", ["v1", "v5_p1024"])
def test_packed_hybrid_linear_routes_and_prepared_decode(gpu, kernel):
    o, g = 96, 4
    p = _payload(o, g, seed=11)
    bias = torch.randn(o).to(torch.bfloat16)
    module = d.PackedHybridLinear(p, bias=bias, kernel=kernel).to(gpu)
    x = torch.randn(1, 1, g * 128, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    ref = _reference(x.view(1, -1), p)[0] + bias.float().numpy()
    with torch.inference_mode():
        y = module(x.to(gpu))
        assert y.shape == (1, 1, o) and module.last_route == "packed_m1"
        got = y.float().cpu().numpy()[0, 0]
        assert np.max(np.abs(got - ref)) <= 2 ** -7 * np.max(np.abs(ref))
        module.bind_prepared_decode(torch.bfloat16)
        module._decode_audit = True
        first = module(x.to(gpu)).clone()
        second = module(x.to(gpu))
        assert torch.equal(first, second) and torch.equal(first, y)
        assert module.route_counts["packed_m1"] == 3
        with pytest.raises(ValueError):
            module(x.to(gpu).float())
        module.clear_prepared_decode()
        with pytest.raises(ValueError):
            module(torch.randn(1, 2, g * 128, device=gpu, dtype=torch.bfloat16))


@pytest.mark.parametrize("gps", [1, 8])
def test_outlier_activation_per_element_bound(gpu, gps):
    """An activation outlier (~1e3 in a group with tiny row scales, the rest ~1e-2):
    every output row within the per-group fixed-point bound 2^-7 B_o of the float64
    truth plus its bf16 rounding (the emulation in tests/test_hybrid_numerics.py
    shows a batch-wide exponent breaking this bound)."""
    from tests.test_hybrid_numerics import outlier_case, row_bound

    p, layout_np, x = outlier_case()
    o = layout_np["codes"].shape[1]
    layout = _layout({k: torch.from_numpy(v) for k, v in p.items()}, "v5_p1024", gpu)
    exact = tb.structural_reference(x, layout_np)[0]
    bound = row_bound(x, layout_np) + 2.0 ** -8 * np.abs(exact)
    xt = torch.from_numpy(x).to(torch.bfloat16).to(gpu)
    ws = torch.full(d.workspace_shape(o, x.shape[1], gps), float("nan"), device=gpu)
    y = torch.empty(1, o, dtype=torch.bfloat16, device=gpu)
    d.m1_out(xt, layout, y, ws, groups_per_split=gps, kernel="v5_p1024")
    got = y.float().cpu().numpy()[0].astype(np.float64)
    assert np.all(np.abs(got - exact) <= bound), float(np.max(np.abs(got - exact) / bound))


def test_out_of_range_refinement_index_gives_nan(gpu):
    p = _payload(24, 3, seed=8)
    layout = _layout(p, "v5_p1024", gpu)
    layout["indices"] = layout["indices"].clone()
    layout["indices"][1, 5] = 200
    x = torch.randn(1, 384, generator=torch.Generator().manual_seed(8)).to(torch.bfloat16).to(gpu)
    y = torch.zeros(1, 24, dtype=torch.bfloat16, device=gpu)
    ws = torch.empty(d.workspace_shape(24, 384, 8), device=gpu)
    d.m1_out(x, layout, y, ws, kernel="v5_p1024")
    assert torch.isnan(y.float()).all()
    layout["indices"][1, 5] = -3
    d.m1_out(x, layout, y, ws, kernel="v5_p1024")
    assert torch.isnan(y.float()).all()


@pytest.mark.parametrize("widths,g", [((64, 32, 32), 3), ((4096, 1024, 1024), 32), ((12288, 12288), 32),
                                      ((48,), 5), ((16, 48, 32, 64), 2)])
def test_segments_launch_equals_separate_calls(gpu, widths, g):
    """q|k|v / gate|up as one fx_hybrid_gemv_segments launch: every row has the bits
    of its own module's fx_hybrid_gemv call although the plans differ (q|k|v 6144
    rows: 2 tiles x 4 K parts per workgroup, q alone 1 x 8; gate|up 24576 rows:
    6 x 2, gate alone 3 x 4), since the kernel sums eight virtual K parts in a
    fixed order; segment starts off the tall-tile grid fall back to fewer tiles."""
    modules = [d.PackedHybridLinear(_payload(o, g, seed=31 + i), kernel="v5_p1024").to(gpu)
               for i, o in enumerate(widths)]
    x = torch.randn(1, g * 128, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).to(gpu)
    fused = d.HybridSegmentsGemv(modules)
    out = torch.full((1, sum(widths)), float("nan"), dtype=torch.bfloat16, device=gpu)
    fused(x, out)
    want = []
    with torch.inference_mode():
        for m in modules:
            y = torch.empty(1, m.out_features, dtype=torch.bfloat16, device=gpu)
            m._packed_kernel(1, gpu)(x, y)
            want.append(y)
    assert torch.equal(out, torch.cat(want, 1))
    # graph replay of the fused launch, twice, against the eager result
    graph = torch.cuda.CUDAGraph()
    replay = torch.empty_like(out)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        fused(x, replay)
    torch.cuda.current_stream().wait_stream(stream)
    with torch.cuda.graph(graph, stream=stream):
        fused(x, replay)
    for _ in range(2):
        replay.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(replay, out)


def test_segments_launch_with_other_split_count_agrees_to_the_last_bit(gpu):
    """Two 256-row modules at K = 16384: alone each splits K over 4 workgroups,
    the fused 512-row launch over one, so the fp32 partials meet in another order
    and the rows are not bit-identical; they agree within half a bf16 ulp of the
    row (plus the fp32 sums' reassociation) and both meet the oracle bar."""
    from marlin_style_fluxbin_amd import _lib

    lib = _lib.library()
    assert lib.fx_hybrid_gemv_workspace_bytes(256, 16384) > 0  # alone: split K
    assert lib.fx_hybrid_gemv_workspace_bytes(512, 16384) == 0  # fused: one split
    payloads = [_payload(256, 128, seed=41 + i) for i in range(2)]
    modules = [d.PackedHybridLinear(p, kernel="v5_p1024").to(gpu) for p in payloads]
    x = torch.randn(1, 128 * 128, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16).to(gpu)
    out = torch.full((1, 512), float("nan"), dtype=torch.bfloat16, device=gpu)
    d.HybridSegmentsGemv(modules)(x, out)
    with torch.inference_mode():
        want = torch.cat([m(x) for m in modules], 1)
    got, ref = out.float().cpu().numpy(), want.float().cpu().numpy()
    assert np.all(np.abs(got - ref) <= 2 ** -8 * np.abs(ref) + 1e-6 * np.abs(ref).max())
    for i, p in enumerate(payloads):
        _check(out[:, 256 * i:256 * (i + 1)], _reference(x, p))


def test_segments_argument_checks(gpu):
    from marlin_style_fluxbin_amd import _lib

    a = d.PackedHybridLinear(_payload(40, 2, seed=1), kernel="v5_p1024").to(gpu)
    b = d.PackedHybridLinear(_payload(32, 2, seed=2), kernel="v5_p1024").to(gpu)
    with pytest.raises(ValueError, match="multiples of 16"):
        d.HybridSegmentsGemv([a, b])
    c = d.PackedHybridLinear(_payload(32, 3, seed=3), kernel="v5_p1024").to(gpu)
    with pytest.raises(ValueError, match="in_features"):
        d.HybridSegmentsGemv([b, c])
    with pytest.raises(ValueError, match="1..4"):
        d.HybridSegmentsGemv([b] * 5)
    lib = _lib.library()
    rows = (__import__("ctypes").c_int * 1)(32)
    rc = lib.fx_hybrid_gemv_segments(None, 2, 0, rows, None, None, None, None, None, None, None, None, 0, None,
                                     256, None)
    assert rc == 1 and b"n_segments" in lib.fx_last_error()  # FX_EINVAL


def _single_split_gemv(module, x):
    """The module's GEMV with no workspace: one K split, the plan the residual
    epilogue runs."""
    from marlin_style_fluxbin_amd import _lib

    fused = d.HybridSegmentsGemv([module])
    y = torch.empty(1, module.out_features, dtype=x.dtype, device=x.device)
    _lib.check(fused.lib.fx_hybrid_gemv(
        x.data_ptr(), _lib.dtype_code(x.dtype), fused.codes.data_ptr(), fused.rows.data_ptr(),
        fused._columns[0].data_ptr(), fused._indices[0].data_ptr(), fused.sparse_codes.data_ptr(),
        fused.sparse_rows.data_ptr(), fused._sparse_columns[0].data_ptr(), None, 0, y.data_ptr(),
        module.out_features, module.in_features, _lib.stream_handle(x.device)), "fx_hybrid_gemv")
    return fused, y


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("o,g,swiglu", [(4096, 32, False), (4096, 96, True), (40, 32, False), (96, 3, True),
                                        (1040, 8, False), (1040, 8, True), (17, 1, False), (4112, 4, True)])
def test_residual_epilogue(gpu, dtype, o, g, swiglu):
    """fx_hybrid_gemv_residual: out = round(residual + round(y)) bit for bit (the
    single-split GEMV, then the dtype's own add), in place, and the sums of out^2
    over 16-row tiles against float64.  swiglu: x is gate | up and the GEMV's
    input equals fx_silu_mul's output bit for bit."""
    from marlin_style_fluxbin_amd import _lib

    module = d.PackedHybridLinear(_payload(o, g, seed=o + g), kernel="v5_p1024").to(gpu)
    k = g * 128
    gen = torch.Generator().manual_seed(o)
    x = (torch.randn(1, (2 if swiglu else 1) * k, generator=gen) * 3).to(DT[dtype]).to(gpu)
    res = (torch.randn(1, o, generator=gen) * 4).to(DT[dtype]).to(gpu)
    act = x
    if swiglu:
        act = torch.empty(1, k, dtype=x.dtype, device=gpu)
        lib = _lib.library()
        _lib.check(lib.fx_silu_mul(x.data_ptr(), x[:, k:].data_ptr(), act.data_ptr(), k, _lib.dtype_code(x.dtype),
                                   _lib.stream_handle(gpu)), "silu_mul")
    fused, y = _single_split_gemv(module, act)
    want = res + y
    tiles = (o + 15) // 16
    sums = torch.full((tiles,), float("nan"), device=gpu)
    got = res.clone()
    fused.residual(x, got, sums, swiglu=swiglu)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    h = want.double().cpu().numpy()[0]
    exact = np.array([np.sum(h[16 * t:16 * t + 16] ** 2) for t in range(tiles)])
    assert np.allclose(sums.cpu().numpy(), exact, rtol=2e-6, atol=0)
    with pytest.raises(ValueError):
        d.HybridSegmentsGemv([module, module]).residual(x, got, sums)


@pytest.mark.parametrize("widths,g,dtype", [((4096, 1024, 1024), 32, "bf16"), ((12288, 12288), 32, "bf16"),
                                            ((48,), 8, "f16"), ((16, 48, 32, 64), 2, "bf16"), ((37,), 1, "bf16"),
                                            ((4112, 4112), 4, "f16")])
def test_rmsnormed_prologue(gpu, widths, g, dtype):
    """fx_hybrid_gemv_segments_rmsnormed equals the RMSNorm kernel followed by the
    plain segments launch bit for bit.  h holds small integers, so every order of
    the fp32 sum of squares is exact and both paths form the same 1 / rms; the
    refinement columns read the normalised activations too."""
    from marlin_style_fluxbin_amd import _lib
    from marlin_style_fluxbin_amd.fused_modules import rms_norm

    k = g * 128
    modules = [d.PackedHybridLinear(_payload(o, g, seed=5 + i), kernel="v5_p1024").to(gpu)
               for i, o in enumerate(widths)]
    fused = d.HybridSegmentsGemv(modules)
    gen = torch.Generator().manual_seed(k)
    h = torch.randint(-6, 7, (1, k), generator=gen).to(DT[dtype]).to(gpu)
    weight = (1 + 0.1 * torch.randn(k, generator=gen)).to(DT[dtype]).to(gpu)
    hs = h.double().cpu().numpy()[0]
    sums = torch.tensor([np.sum(hs[16 * t:16 * t + 16] ** 2) for t in range((k + 15) // 16)],
                        dtype=torch.float32, device=gpu)
    normed = torch.empty_like(h)
    rms_norm(h, weight, 1e-6, out=normed)
    want = torch.empty(1, sum(widths), dtype=DT[dtype], device=gpu)
    fused(normed, want)
    got = torch.full_like(want, float("nan"))
    fused.rmsnormed(h, sums, weight, 1e-6, got)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    lib = fused.lib
    rc = lib.fx_hybrid_gemv_segments_rmsnormed(
        h.data_ptr(), _lib.dtype_code(h.dtype), fused._n, fused._segment_rows, fused.codes.data_ptr(),
        fused.rows.data_ptr(), fused._cols_ptrs, fused._idx_ptrs, fused.sparse_codes.data_ptr(),
        fused.sparse_rows.data_ptr(), fused._scols_ptrs, sums.data_ptr(), sums.numel() + 1, weight.data_ptr(), 1e-6,
        None, 0, got.data_ptr(), k, None)
    assert rc == 1 and "n_tiles" in lib.fx_last_error().decode()


@pytest.mark.parametrize("o,g", [(4096, 32), (12288, 32)])
def test_packed_linear_passes_the_product_structural_gate(gpu, o, g):
    """The reference trial's check: a packed hybrid Linear's bf16 output against
    factored_reference.structural_reference under structural_gate, both computed
    on the GPU from the module's own layout."""
    from marlin_style_fluxbin_amd.factored_reference import structural_gate, structural_reference

    p = _payload(o, g, seed=o)
    module = d.PackedHybridLinear(p, kernel="v5_p1024").to(gpu)
    x = torch.randn(1, g * 128, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16).to(gpu)
    with torch.inference_mode():
        y = module(x)
        expected = structural_reference(x, module.layout())
    gate = structural_gate(y, expected)
    assert gate["passed"], gate
    np.testing.assert_allclose(expected.cpu().numpy(), _reference(x, p), rtol=1e-12, atol=1e-12)


def test_bias_add_promotes_as_the_reference_does(gpu):
    """PackedHybridLinear's forward adds its bias out of place (deployment.py:
    295-296): a float32 bias gives a float32 output; the bound decode route adds
    it in place into its bf16 buffer (:262)."""
    o, g = 64, 2
    p = _payload(o, g, seed=11)
    bias = torch.randn(o, generator=torch.Generator().manual_seed(4)).to(gpu)
    x = torch.randn(1, g * 128, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16).to(gpu)
    plain = d.PackedHybridLinear(p, kernel="v5_p1024").to(gpu)
    module = d.PackedHybridLinear(p, bias=bias, kernel="v5_p1024").to(gpu)
    with torch.inference_mode():
        y0 = plain(x)
        y = module(x)
        assert y.dtype == torch.float32 and torch.equal(y, y0 + bias)
        module.bind_prepared_decode(torch.bfloat16)
        yb = module(x.view(1, 1, -1))
        assert yb.dtype == torch.bfloat16 and torch.equal(yb.view(1, o), (y0.float() + bias).to(torch.bfloat16))
