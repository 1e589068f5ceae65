"""``fx_w3_gemv_noalloc`` (the allocation-free W3 GEMV) against ``fx_w3_gemv``.

Both are called through the C ABI (ctypes) on shapes whose plans use the K-split
scratch: a narrow output (MFMA kernel + finish), and the decoded-bf16 table route
with fp32 partials.  Two calls in a row, the second with a smaller input, each
bit-equal to ``fx_w3_gemv`` with a caller-owned workspace (same kernels, same
plan).  A shape whose split partials exceed the library's scratch must fail with
FX_EINVAL before any launch.
"""
from __future__ import annotations

import pytest
import torch

from marlin_style_fluxbin_amd import _lib
from tests.payloads import config_codes, layout_from_codes

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 4 << 20


def _payload(o, k, seed, device):
    codes, scales, zeros, perm = config_codes(o, k, seed=seed, zeros=True, scale_dtype=torch.bfloat16,
                                              permute=True)
    layout = {n: v.to(device) for n, v in layout_from_codes(codes, scales, zeros, perm).items()}
    return layout


def _args(layout, x):
    return (x.data_ptr(), _lib.dtype_code(x.dtype), layout["planes"].data_ptr(), layout["scales"].data_ptr(),
            _lib.dtype_code(layout["scales"].dtype), layout["zeros"].data_ptr(), layout["perm"].data_ptr())


def _both(lib, layout, x, m, o, k, arithmetic, device):
    stream = _lib.stream_handle(device)
    need = lib.fx_w3_gemv_workspace_bytes(m, o, k)
    assert 0 < need <= SCRATCH_BYTES, need
    ws = torch.full((need // 4 + 64,), float("nan"), dtype=torch.float32, device=device)
    want = torch.empty(m, o, dtype=x.dtype, device=device)
    got = torch.full((m, o), float("nan"), dtype=x.dtype, device=device)
    _lib.check(lib.fx_w3_gemv(*_args(layout, x), ws.data_ptr(), ws.numel() * 4, want.data_ptr(), m, o, k,
                              arithmetic, stream), "fx_w3_gemv")
    _lib.check(lib.fx_w3_gemv_noalloc(*_args(layout, x), got.data_ptr(), m, o, k, arithmetic, stream),
               "fx_w3_gemv_noalloc")
    torch.cuda.synchronize()
    return got, want


@pytest.mark.parametrize("arithmetic", [_lib.ARITH_STRUCTURAL, _lib.ARITH_DECODED_BF16])
def test_noalloc_matches_workspace_entry_twice(gpu, arithmetic):
    lib = _lib.library()
    # first call: the larger plan; second: a smaller input on the same scratch
    for (m, o, k, seed) in ((4, 256, 4096, 1), (1, 128, 1024, 2)):
        print(f"noalloc arithmetic {arithmetic} M={m} O={o} K={k}", flush=True)
        layout = _payload(o, k, seed, gpu)
        x = torch.randn(m, k, generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16).to(gpu)
        got, want = _both(lib, layout, x, m, o, k, arithmetic, gpu)
        assert torch.isfinite(got.float()).all()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_noalloc_decoded_route_with_many_splits(gpu):
    lib = _lib.library()
    m, o, k = 8, 1024, 4096
    layout = _payload(o, k, 3, gpu)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).to(gpu)
    got, want = _both(lib, layout, x, m, o, k, _lib.ARITH_DECODED_BF16, gpu)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_noalloc_rejects_scratch_overflow(gpu):
    lib = _lib.library()
    candidates = [(8, o, k) for o in (767, 511, 1023, 2047, 12288) for k in (32512, 16384, 4096)]
    big = next(((m, o, k) for m, o, k in candidates if lib.fx_w3_gemv_workspace_bytes(m, o, k) > SCRATCH_BYTES),
               None)
    assert big is not None, "no candidate shape needs more than the scratch"
    m, o, k = big
    x = torch.zeros(m, k, dtype=torch.bfloat16, device=gpu)
    planes = torch.zeros(k // 128, 3, o, 16, dtype=torch.uint8, device=gpu)
    scales = torch.zeros(k // 128, o, dtype=torch.bfloat16, device=gpu)
    out = torch.zeros(m, o, dtype=torch.bfloat16, device=gpu)
    rc = lib.fx_w3_gemv_noalloc(x.data_ptr(), _lib.FX_BF16, planes.data_ptr(), scales.data_ptr(), _lib.FX_BF16,
                                None, None, out.data_ptr(), m, o, k, _lib.ARITH_DECODED_BF16,
                                _lib.stream_handle(gpu))
    assert rc == 1
    assert b"scratch" in lib.fx_last_error()
    torch.cuda.synchronize()
    assert int(out.view(torch.int16).abs().sum()) == 0
