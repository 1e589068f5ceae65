"""Field-layout plans give the same bits.

Every field-layout entry point (plain, SwiGLU and residual epilogues, the
normalising prologue, permuted columns, output indices, the strided batch) runs
once per plan that can take the shape (``fx_w3_fields_plan``), once on the
one-tile kernel and once under the default plan; every output -- values,
reordered copies, tile sums of squares -- must be bitwise equal across all of
them.  The shapes include a partial last row block (65 tiles: a workgroup of 2,
3, 4 or 6 tiles holds tiles past O), a K with fewer batches than virtual waves
(4), 9 batches, K = 12288 (24 batches, three per virtual wave) and K = 16384.  The one-tile kernel itself is held to the float64 oracle by
tests/test_w3_fields_gpu.py; one wide plan is checked against it here too.
"""
from __future__ import annotations

import contextlib

import numpy as np
import pytest
import torch

from marlin_style_fluxbin_amd import _lib
from oracle import w3
from tests.payloads import assert_half_ulp, config_codes, layout_from_codes, oracle_layout

pytestmark = pytest.mark.gpu

PLANS = [(1, 8, 1, 1), (1, 8, 3, 3), (2, 4, 2, 1), (3, 4, 2, 1), (4, 2, 4, 1)]
ONE_TILE = (-1, 0, 0, 0)


@contextlib.contextmanager
def fields_plan(plan):
    lib = _lib.library()
    _lib.check(lib.fx_w3_fields_plan(*plan), f"fields plan {plan}")
    try:
        yield
    finally:
        _lib.check(lib.fx_w3_fields_plan(0, 0, 0, 0), "fields plan reset")


def fits(plan, o, k, perm=False):
    t, p, _, s = plan
    nb = k // 512
    return o % 16 == 0 and k % 512 == 0 and nb <= s * t * p and (not perm or k * 2 <= 48 * 1024)


def _payload(gpu, o, k, seed, scale_dtype=torch.float16, zeros=True):
    codes, scales, zero, _ = config_codes(o, k, seed=seed, zeros=zeros, scale_dtype=scale_dtype)
    layout = layout_from_codes(codes, scales, zero, None)
    dl = {n: t.to(gpu) for n, t in layout.items()}
    lib = _lib.library()
    fields = torch.empty_like(dl["planes"])
    _lib.check(lib.fx_w3_planes_to_fields(dl["planes"].data_ptr(), fields.data_ptr(), o, k, _lib.stream_handle(gpu)),
               "planes_to_fields")
    dl["fields"] = fields
    return layout, dl


def _perm(k, seed, gpu):
    g = torch.Generator().manual_seed(seed)
    groups = torch.randint(0, k // 128, (k,), generator=g)
    return torch.argsort(groups, stable=True).to(torch.int16).to(gpu)


def _index(n, seed, gpu):
    """A random output index (a permutation of n entries, int16)."""
    return torch.randperm(n, generator=torch.Generator().manual_seed(seed)).to(torch.int16).to(gpu)


DEFAULT = (0, 0, 0, 0)  # the entry points' own choice


def _across_plans(run, o, k, perm=False):
    """run() -> tuple of output tensors, under the one-tile kernel, the default
    and every plan that takes (o, k); asserts bitwise equality; returns the
    one-tile outputs."""
    with fields_plan(ONE_TILE):
        want = [t.clone() for t in run()]
    ran = 0
    for plan in [DEFAULT] + PLANS:
        if plan != DEFAULT and not fits(plan, o, k, perm):
            continue
        with fields_plan(plan):
            got = run()
        torch.cuda.synchronize()
        for i, (g, w) in enumerate(zip(got, want)):
            assert torch.equal(g, w), f"plan {plan} output {i}: max |diff| {(g.float() - w.float()).abs().max()}"
        ran += 1
    assert ran > 0
    return want


SHAPES = [(768, 4096), (1040, 2048), (256, 12288), (4096, 4096), (1040, 4608), (512, 8192), (256, 16384)]


@pytest.mark.parametrize("o,k", SHAPES)
@pytest.mark.parametrize("xdtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("scale_dtype,zeros", [(torch.float16, True), (torch.bfloat16, False)])
def test_plain_gemv_same_bits_every_plan(gpu, o, k, xdtype, scale_dtype, zeros):
    print(f"plain {o}x{k} {xdtype} {scale_dtype} zeros={zeros}", flush=True)
    _, dl = _payload(gpu, o, k, seed=o + k, scale_dtype=scale_dtype, zeros=zeros)
    x = torch.randn(1, k, generator=torch.Generator().manual_seed(o)).to(xdtype).to(gpu)
    lib = _lib.library()

    def run():
        out = torch.full((1, o), float("nan"), dtype=xdtype, device=gpu)
        _lib.check(lib.fx_w3_gemv_fields(x.data_ptr(), _lib.dtype_code(xdtype), dl["fields"].data_ptr(),
                                         dl["scales"].data_ptr(), _lib.dtype_code(scale_dtype),
                                         _lib.ptr(dl.get("zeros")), out.data_ptr(), o, k, _lib.stream_handle(gpu)),
                   "gemv_fields")
        return (out,)

    (out,) = _across_plans(run, o, k)
    assert torch.isfinite(out.float()).all()


@pytest.mark.parametrize("o,k", [(768, 4096), (1040, 2048), (256, 12288), (4096, 12288), (1040, 4608)])
@pytest.mark.parametrize("permuted", [False, True])
@pytest.mark.parametrize("indexed", [False, True])
def test_residual_epilogue_same_bits_every_plan(gpu, o, k, permuted, indexed):
    print(f"residual {o}x{k} perm={permuted} index={indexed}", flush=True)
    _, dl = _payload(gpu, o, k, seed=3 * o + k)
    g = torch.Generator().manual_seed(k)
    x = torch.randn(1, k, generator=g).bfloat16().to(gpu)
    res = torch.randn(1, o, generator=g).bfloat16().to(gpu)
    perm = _perm(k, o, gpu) if permuted else None
    index = _index(o, k, gpu) if indexed else None
    lib = _lib.library()

    def run():
        out = torch.full((1, o), float("nan"), dtype=torch.bfloat16, device=gpu)
        sums = torch.full(((o + 15) // 16,), float("nan"), dtype=torch.float32, device=gpu)
        sorted_out = torch.full((1, o), float("nan"), dtype=torch.bfloat16, device=gpu) if indexed else None
        _lib.check(lib.fx_w3_gemv_residual(x.data_ptr(), _lib.FX_BF16, dl["fields"].data_ptr(), dl["scales"].data_ptr(),
                                           _lib.FX_F16, dl["zeros"].data_ptr(), _lib.ptr(perm), res.data_ptr(),
                                           out.data_ptr(), sums.data_ptr(), _lib.ptr(index), _lib.ptr(sorted_out),
                                           o, k, _lib.PAYLOAD_FIELDS, _lib.stream_handle(gpu)), "gemv_residual")
        return (out, sums) + ((sorted_out,) if indexed else ())

    outs = _across_plans(run, o, k, perm=permuted)
    assert torch.isfinite(outs[1]).all()
    if indexed:  # the reordered copy is out[index^-1]
        assert torch.equal(outs[2][0, index.long()], outs[0][0])


@pytest.mark.parametrize("o,k", [(1536, 4096), (1056, 2048), (512, 12288)])
@pytest.mark.parametrize("permuted", [False, True])
@pytest.mark.parametrize("indexed", [False, True])
def test_swiglu_epilogue_same_bits_every_plan(gpu, o, k, permuted, indexed):
    print(f"swiglu {o}x{k} perm={permuted} index={indexed}", flush=True)
    _, dl = _payload(gpu, o, k, seed=o + 5 * k)
    x = torch.randn(1, k, generator=torch.Generator().manual_seed(o)).bfloat16().to(gpu)
    perm = _perm(k, o, gpu) if permuted else None
    index = _index(o // 2, k, gpu) if indexed else None
    lib = _lib.library()

    def run():
        out = torch.full((1, o // 2), float("nan"), dtype=torch.bfloat16, device=gpu)
        _lib.check(lib.fx_w3_gemv_swiglu(x.data_ptr(), _lib.FX_BF16, dl["fields"].data_ptr(), dl["scales"].data_ptr(),
                                         _lib.FX_F16, dl["zeros"].data_ptr(), _lib.ptr(perm), _lib.ptr(index),
                                         out.data_ptr(), o, k, _lib.PAYLOAD_FIELDS, _lib.stream_handle(gpu)),
                   "gemv_swiglu")
        return (out,)

    (out,) = _across_plans(run, o, k, perm=permuted)
    assert torch.isfinite(out.float()).all()


@pytest.mark.parametrize("o,k", [(768, 4096), (1040, 2048), (1536, 4096)])
@pytest.mark.parametrize("swiglu", [0, 1])
def test_normalising_prologue_same_bits_every_plan(gpu, o, k, swiglu):
    print(f"rmsnormed {o}x{k} swiglu={swiglu}", flush=True)
    _, dl = _payload(gpu, o, k, seed=o + 7 * k)
    g = torch.Generator().manual_seed(o + k)
    h = torch.randn(1, k, generator=g).bfloat16().to(gpu)
    sums = (h.float().view(-1, 16) ** 2).sum(1).contiguous()
    weight = (1 + 0.1 * torch.randn(k, generator=g)).bfloat16().to(gpu)
    index = _index(o // 2, k, gpu) if swiglu else None
    n_out = o // 2 if swiglu else o
    lib = _lib.library()

    def run():
        out = torch.full((1, n_out), float("nan"), dtype=torch.bfloat16, device=gpu)
        _lib.check(lib.fx_w3_gemv_rmsnormed(h.data_ptr(), _lib.FX_BF16, dl["fields"].data_ptr(), dl["scales"].data_ptr(),
                                            _lib.FX_F16, dl["zeros"].data_ptr(), sums.data_ptr(), k // 16,
                                            weight.data_ptr(), 1e-6, _lib.ptr(index), out.data_ptr(), o, k, swiglu,
                                            _lib.PAYLOAD_FIELDS, _lib.stream_handle(gpu)), "gemv_rmsnormed")
        return (out,)

    (out,) = _across_plans(run, o, k)
    assert torch.isfinite(out.float()).all()


@pytest.mark.parametrize("o,k,batch", [(1536, 4096, 3), (256, 12288, 2), (128, 16384, 3)])
def test_strided_batch_same_bits_every_plan(gpu, o, k, batch):
    print(f"strided {o}x{k} x{batch}", flush=True)
    lib = _lib.library()
    parts = [_payload(gpu, o, k, seed=o + k + p)[1] for p in range(batch)]
    fields = torch.stack([d["fields"] for d in parts]).contiguous()
    scales = torch.stack([d["scales"] for d in parts]).contiguous()
    zeros = torch.stack([d["zeros"] for d in parts]).contiguous()
    x = torch.randn(batch, k, generator=torch.Generator().manual_seed(k)).bfloat16().to(gpu)

    def run():
        out = torch.full((batch, o), float("nan"), dtype=torch.bfloat16, device=gpu)
        rc = lib.fx_w3_gemv_strided_batched(x.data_ptr(), _lib.FX_BF16, k, fields.data_ptr(), fields[0].numel(),
                                            scales.data_ptr(), _lib.FX_F16, scales[0].numel(), zeros.data_ptr(),
                                            zeros[0].numel(), out.data_ptr(), o, batch, o, k, _lib.PAYLOAD_FIELDS,
                                            _lib.stream_handle(gpu))
        _lib.check(rc, "strided batch")
        return (out,)

    # plans whose row blocks are not a multiple of 8 refuse a batch; run the rest
    with fields_plan(ONE_TILE):
        want = run()[0].clone()
    for plan in [DEFAULT] + PLANS:
        if plan != DEFAULT and (not fits(plan, o, k) or (o // 16 + plan[0] - 1) // plan[0] % 8):
            continue
        with fields_plan(plan):
            got = run()[0]
        torch.cuda.synchronize()
        assert torch.equal(got, want), plan


def test_wide_plan_matches_oracle_and_refuses_misfits(gpu):
    o, k = 1040, 2048
    layout, dl = _payload(gpu, o, k, seed=11)
    x = torch.randn(1, k, generator=torch.Generator().manual_seed(2)).bfloat16()
    lib = _lib.library()
    out = torch.full((1, o), float("nan"), dtype=torch.bfloat16, device=gpu)
    with fields_plan((3, 4, 2, 1)):
        _lib.check(lib.fx_w3_gemv_fields(x.to(gpu).data_ptr(), _lib.FX_BF16, dl["fields"].data_ptr(),
                                         dl["scales"].data_ptr(), _lib.FX_F16, dl["zeros"].data_ptr(), out.data_ptr(),
                                         o, k, _lib.stream_handle(gpu)), "gemv_fields")
        exact = w3.matvec_exact(x.float().numpy(), oracle_layout(layout))
        assert_half_ulp(out.float().cpu().numpy(), exact, "bf16", rel_slack=3e-5, what="wide plan")
        # a plan that cannot take the shape fails loudly (O % 16, then too many batches)
        rc = lib.fx_w3_gemv_fields(x.to(gpu).data_ptr(), _lib.FX_BF16, dl["fields"].data_ptr(), dl["scales"].data_ptr(),
                                   _lib.FX_F16, dl["zeros"].data_ptr(), out.data_ptr(), o - 8, k,
                                   _lib.stream_handle(gpu))
        assert rc == 1 and "O % 16 == 0" in lib.fx_last_error().decode()
    with fields_plan((1, 8, 1, 1)):
        big = _payload(gpu, 256, 12288, seed=3)[1]
        xb = torch.randn(1, 12288).bfloat16().to(gpu)
        ob = torch.empty(1, 256, dtype=torch.bfloat16, device=gpu)
        rc = lib.fx_w3_gemv_fields(xb.data_ptr(), _lib.FX_BF16, big["fields"].data_ptr(), big["scales"].data_ptr(),
                                   _lib.FX_F16, big["zeros"].data_ptr(), ob.data_ptr(), 256, 12288,
                                   _lib.stream_handle(gpu))
        assert rc == 1 and "more batches" in lib.fx_last_error().decode()
    with fields_plan((1, 16, 2, 2)):  # an M-row plan only: the one-row call refuses it
        rc = lib.fx_w3_gemv_fields(x.to(gpu).data_ptr(), _lib.FX_BF16, dl["fields"].data_ptr(), dl["scales"].data_ptr(),
                                   _lib.FX_F16, dl["zeros"].data_ptr(), out.data_ptr(), o, k, _lib.stream_handle(gpu))
        assert rc == 1 and "only the M-row form" in lib.fx_last_error().decode()


ROWS_PLANS = PLANS + [(1, 12, 2, 2), (1, 16, 2, 2)]


def rows_fit(plan, k, m):
    """Whether fx_w3_gemv_fields_rows takes (k, m) under `plan`: the waves stage
    every batch, and a plan of several tiles holds every batch of a launch's rows
    in LDS (8 of eight rows, 24 of four; eight rows run as chunks of four where
    they do not fit), where a solo plan (one tile) restages per batch."""
    t, p, _, st = plan
    nb, solo = k // 512, t == 1
    mb = 2 if m <= 2 else 4 if m <= 4 else 8
    if mb == 8 and not solo and nb > 8:
        mb = 4
    return nb <= st * t * p and (solo or nb <= (8 if mb == 8 else 24))


@pytest.mark.parametrize("o,k,m", [(768, 4096, 2), (768, 4096, 3), (768, 4096, 8), (1040, 2048, 5), (4096, 4096, 8),
                                   (256, 12288, 4), (256, 12288, 8), (12288, 4096, 8), (512, 1024, 6)])
@pytest.mark.parametrize("xdtype,scale_dtype,zeros", [(torch.bfloat16, torch.float16, True),
                                                       (torch.float16, torch.bfloat16, False)])
def test_rows_gemv_matches_oracle_and_plans(gpu, o, k, m, xdtype, scale_dtype, zeros):
    """fx_w3_gemv_fields_rows (M = 2..8 on the field layout): every row within the
    bar of the one-row field kernel (half an ulp of the float64 oracle plus 3e-5
    of the largest output), rows past M untouched, and every plan that takes the
    shape bit-identical to the default one (chunks of four rows where eight rows'
    staged operands do not fit, K = 12288)."""
    print(f"rows {o}x{k} M={m} {xdtype}", flush=True)
    layout, dl = _payload(gpu, o, k, seed=o + k + m, scale_dtype=scale_dtype, zeros=zeros)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(m + o)).to(xdtype)
    lib = _lib.library()

    def run():
        out = torch.full((m + 1, o), float("nan"), dtype=xdtype, device=gpu)
        _lib.check(lib.fx_w3_gemv_fields_rows(x.to(gpu).data_ptr(), _lib.dtype_code(xdtype), dl["fields"].data_ptr(),
                                              dl["scales"].data_ptr(), _lib.dtype_code(scale_dtype),
                                              _lib.ptr(dl.get("zeros")), out.data_ptr(), m, o, k,
                                              _lib.stream_handle(gpu)), "gemv_fields_rows")
        torch.cuda.synchronize()
        return out

    want = run()
    assert torch.isnan(want[m].float()).all()  # the row past M is not written
    exact = w3.matvec_exact(x.float().numpy(), oracle_layout(layout))
    tag = "bf16" if xdtype == torch.bfloat16 else "f16"
    assert_half_ulp(want[:m].float().cpu().numpy(), exact, tag, rel_slack=3e-5, what=f"rows {o}x{k} M={m}")
    ran = 0
    for plan in ROWS_PLANS:
        if not rows_fit(plan, k, m):
            continue
        with fields_plan(plan):
            got = run()
        assert torch.equal(got[:m], want[:m]), plan
        ran += 1
    assert ran > 0


def _rows_call(lib, gpu, x, dl, out, m, o, k, scale_dtype=torch.float16):
    _lib.check(lib.fx_w3_gemv_fields_rows(x.data_ptr(), _lib.dtype_code(x.dtype), dl["fields"].data_ptr(),
                                          dl["scales"].data_ptr(), _lib.dtype_code(scale_dtype),
                                          _lib.ptr(dl.get("zeros")), out.data_ptr(), m, o, k,
                                          _lib.stream_handle(gpu)), "gemv_fields_rows")


def test_rows_gemv_one_row_is_the_field_gemv(gpu):
    """M = 1 through fx_w3_gemv_fields_rows is fx_w3_gemv_fields, bit for bit."""
    o, k = 768, 4096
    _, dl = _payload(gpu, o, k, seed=21)
    x = torch.randn(1, k, generator=torch.Generator().manual_seed(4)).bfloat16().to(gpu)
    lib = _lib.library()
    a = torch.empty(1, o, dtype=torch.bfloat16, device=gpu)
    b = torch.empty_like(a)
    _rows_call(lib, gpu, x, dl, a, 1, o, k)
    _lib.check(lib.fx_w3_gemv_fields(x.data_ptr(), _lib.FX_BF16, dl["fields"].data_ptr(), dl["scales"].data_ptr(),
                                     _lib.FX_F16, dl["zeros"].data_ptr(), b.data_ptr(), o, k,
                                     _lib.stream_handle(gpu)), "gemv_fields")
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.parametrize("o,k,m", [(1040, 2048, 8), (256, 12288, 5)])
def test_rows_gemv_graph_replays_match_eager(gpu, o, k, m):
    """The M-row launch captured in a hipGraph: every replay, with eager work and
    synchronisations between replays, equals the eager result bit for bit."""
    _, dl = _payload(gpu, o, k, seed=o + m)
    lib = _lib.library()
    stream = torch.cuda.Stream(gpu)
    with torch.cuda.stream(stream):
        x = torch.randn(m, k, device=gpu, generator=torch.Generator(device=gpu).manual_seed(m)).bfloat16()
        eager = torch.empty(m, o, dtype=torch.bfloat16, device=gpu)
        out = torch.full_like(eager, float("nan"))
        _rows_call(lib, gpu, x, dl, eager, m, o, k)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        _rows_call(lib, gpu, x, dl, out, m, o, k)
    torch.cuda.synchronize()
    for i in range(4):
        out.fill_(float("nan"))
        scratch = torch.randn(4096, device=gpu).sum()  # eager work between the replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
        assert torch.isfinite(scratch)
