"""GPU parity of the rank-one two-base GEMV (config-4 format) against the float64 oracle.

Bars: bf16 / fp16 outputs within max relative error 2^-8 (normwise, max|err| /
max|y|) of the float64 dequantize-then-matmul ``oracle.two_base.rank_one_matvec``,
which covers the output rounding (2^-9) plus the kernel's 16-bit fixed-point
activation operands (~1e-4); the fp32 K-split partials summed on the host within
1e-3.  Basis-vector inputs read single weight columns and pin the column mapping
of the sign layout, the salient scatter and both bases bit-for-bit up to the
output rounding.
"""
import numpy as np
import pytest
import torch

from marlin_style_fluxbin_amd import _lib
from marlin_style_fluxbin_amd.two_base import (TwoBaseGemv, pack_rank_one_planes, two_base_gemv,
                                               unpack_rank_one_planes)
from oracle import two_base as tb

pytestmark = pytest.mark.gpu

DT = {"bf16": torch.bfloat16, "f16": torch.float16}
# (waves, batches of sign loads in flight, groups per K split, 16-row tiles per workgroup)
TILINGS = [(4, 1, 4, 1), (4, 2, 8, 1), (8, 1, 16, 1), (8, 2, 32, 1), (8, 2, 16, 2), (12, 2, 32, 3),
           (12, 1, 64, 3), (16, 2, 32, 4), (16, 2, 128, 2)]


def _layout(p, device):
    return {
        "planes": torch.from_numpy(p["planes"]).to(device),
        "coef": torch.from_numpy(p["coef"]).to(device),
        "srow": torch.from_numpy(p["srow"]).to(device),
        "tcol": torch.from_numpy(p["tcol"]).to(device),
        "salient": torch.from_numpy(p["sal"]).to(torch.bfloat16).to(device),
        "salient_idx": torch.from_numpy(p["sal_idx"]).to(device),
    }


def _x(k, dtype, seed):
    return torch.randn(1, k, generator=torch.Generator().manual_seed(seed)).to(DT[dtype])


def _max_rel(got, exact):
    return float(np.max(np.abs(got - exact)) / max(np.max(np.abs(exact)), 1e-30))


def test_pack_planes_matches_oracle(gpu):
    p = tb.make_rank_one_payload(40, 384, salient=3, seed=2)
    bases = torch.from_numpy(p["bases"])
    for device in ("cpu", gpu):
        planes = pack_rank_one_planes(bases.to(device)).cpu().numpy()
        assert np.array_equal(planes, p["planes"])
        assert torch.equal(unpack_rank_one_planes(torch.from_numpy(planes).to(device)).cpu(), bases)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("o,k,s", [(12288, 4096, 32), (1000, 384, 5), (17, 128, 0), (64, 12288, 32),
                                   (4096, 4096, 32), (33, 640, 32), (1024, 4096, 1)])
def test_rank_one_default_plan(gpu, dtype, o, k, s):
    p = tb.make_rank_one_payload(o, k, salient=s, seed=o + k + s)
    layout = _layout(p, gpu)
    x = _x(k, dtype, seed=o)
    exact = tb.rank_one_matvec(x.float().numpy(), p)
    out = torch.empty(1, o, dtype=DT[dtype], device=gpu)
    gemv = TwoBaseGemv(layout)
    gemv(x.to(gpu), out)
    got = out.float().cpu().numpy()
    assert np.all(np.isfinite(got))
    assert _max_rel(got, exact) <= 2 ** -8
    again = torch.empty_like(out)
    gemv(x.to(gpu), again)
    assert torch.equal(out, again)


@pytest.mark.parametrize("tiling", TILINGS)
@pytest.mark.parametrize("o,k", [(300, 2048), (17, 384), (64, 512)])
def test_rank_one_tilings_and_fp32_partials(gpu, tiling, o, k):
    p = tb.make_rank_one_payload(o, k, salient=7, seed=o * 3 + k)
    layout = _layout(p, gpu)
    x = _x(k, "bf16", seed=k).to(gpu)
    exact = tb.rank_one_matvec(x.float().cpu().numpy(), p)
    lib = _lib.library()
    nbytes = lib.fx_two_base_gemv_config_workspace_bytes(o, k, *tiling)
    ws = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=gpu)
    out = torch.empty(1, o, dtype=torch.bfloat16, device=gpu)
    two_base_gemv(x, layout, out, ws, tiling=tiling)
    assert _max_rel(out.float().cpu().numpy(), exact) <= 2 ** -8
    if nbytes:  # K split over workgroups: the fp32 partials sum to y
        splits = nbytes // (4 * o)
        partial = ws[:nbytes].view(torch.float32).view(splits, o).double().sum(0).cpu().numpy()
        assert _max_rel(partial, exact[0]) <= 1e-3


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_rank_one_basis_vectors_read_single_columns(gpu, dtype):
    o, k = 96, 768
    p = tb.make_rank_one_payload(o, k, salient=6, seed=11)
    layout = _layout(p, gpu)
    w = tb.rank_one_weight(p)
    gemv = TwoBaseGemv(layout)
    cols = sorted({0, 1, 15, 16, 17, 127, 128, 300, 511, 767} | set(int(c) for c in p["sal_idx"][:3]))
    for col in cols:
        x = torch.zeros(1, k, dtype=DT[dtype])
        x[0, col] = 1.0
        out = torch.empty(1, o, dtype=DT[dtype], device=gpu)
        gemv(x.to(gpu), out)
        want = torch.from_numpy(w[:, col]).float().to(DT[dtype]).float().numpy()
        got = out.float().cpu().numpy()[0]
        # one column times 1.0: only the fixed-point (2^-14 of the column max) and
        # the single output rounding separate the kernel from the exact column
        assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-3)) <= 2 ** -7, col


def test_rank_one_graph_replay_and_streams(gpu):
    o, k = 4096, 4096
    p = tb.make_rank_one_payload(o, k, seed=5)
    layout = _layout(p, gpu)
    x = _x(k, "bf16", seed=9).to(gpu)
    gemv = TwoBaseGemv(layout)
    out = torch.empty(1, o, dtype=torch.bfloat16, device=gpu)
    gemv(x, out)
    saved = out.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        out.zero_()
        gemv(x, out)
    torch.cuda.current_stream().wait_stream(side)
    assert torch.equal(out, saved)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gemv(x, out)
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, saved)


def test_rank_one_rejects_bad_arguments(gpu):
    lib = _lib.library()
    t = torch.zeros(1 << 16, dtype=torch.uint8, device=gpu)
    base = t.data_ptr()
    args = lambda **kw: dict(dict(x=base, xd=2, planes=base, coef=base, srow=base, tcol=base, sal=None, idx=None,
                                  s=0, ws=None, wsb=0, out=base, o=16, k=128), **kw)

    def call(a):
        return lib.fx_two_base_gemv(a["x"], a["xd"], a["planes"], a["coef"], a["srow"], a["tcol"], a["sal"],
                                    a["idx"], a["s"], a["ws"], a["wsb"], a["out"], a["o"], a["k"], None)

    assert call(args(k=200)) == 1 and "multiple of 128" in lib.fx_last_error().decode()
    assert call(args(planes=base + 8)) == 1 and "aligned" in lib.fx_last_error().decode()
    assert call(args(s=4)) == 1 and "salient" in lib.fx_last_error().decode()
    assert call(args(s=33, sal=base, idx=base)) == 1 and "n_salient" in lib.fx_last_error().decode()
    assert call(args(xd=0)) == 1 and "dtype" in lib.fx_last_error().decode()
    assert call(args(coef=None)) == 1 and "non-null" in lib.fx_last_error().decode()
    # narrow outputs split K: the workspace is required
    need = lib.fx_two_base_gemv_workspace_bytes(16, 8192)
    assert need > 0
    assert call(args(o=16, k=8192)) == 1 and "workspace" in lib.fx_last_error().decode()


@pytest.mark.parametrize("tiling", [None, (8, 2, 16, 1), (12, 1, 64, 3)])
def test_rank_one_outlier_activation(gpu, tiling):
    """One activation column ~1e3 among ~1e-2 (tests/test_two_base_numerics.py's
    case: in half the rows the outlier cancels and the small columns are the whole
    output).  The kernel equals the CPU emulation of its fixed point (one exponent
    per 512-column batch, two int8 digits) up to the bf16 output rounding and fp32
    sums, and so stays within the stated per-row bound of the float64 truth."""
    from tests.test_two_base_numerics import outlier_case, emulate

    p, x = outlier_case()
    layout = _layout(p, gpu)
    xt = torch.from_numpy(x).to(torch.bfloat16)
    o, k = p["planes"].shape[1], 128 * p["planes"].shape[0]
    out = torch.full((1, o), float("nan"), dtype=torch.bfloat16, device=gpu)
    if tiling is None:
        TwoBaseGemv(layout)(xt.to(gpu), out)
    else:
        nbytes = _lib.library().fx_two_base_gemv_config_workspace_bytes(o, k, *tiling)
        ws = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=gpu)
        two_base_gemv(xt.to(gpu), layout, out, ws, tiling=tiling)
    got = out.float().cpu().numpy()[0].astype(np.float64)
    exact = tb.rank_one_matvec(x, p)[0]
    emulated, bound = emulate(x, p)
    u_abs = np.abs(x[0].astype(np.float64) * p["tcol"].astype(np.float64)).sum()
    coef = np.abs(p["srow"].astype(np.float64)) * (np.abs(p["coef"][0]) + np.abs(p["coef"][1])).astype(np.float64)
    # half a bf16 ulp of the output (up to 2^-8 |y| just above a power of two) and
    # the fp32 sums of ~1e3-sized terms
    slack = 2.0 ** -8 * np.abs(got) + 2e-6 * coef * u_abs
    assert np.all(np.abs(got - emulated) <= slack), np.max(np.abs(got - emulated) / slack)
    assert np.all(np.abs(got - exact) <= bound + slack)
