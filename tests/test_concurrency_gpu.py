"""Host threads calling the C ABI at once, each on its own stream.

The library keeps only per-thread error text and per-device caches (CU count,
guarded by a lock); every call's state lives in its arguments.  Four threads
launch W3 GEMVs (one with a K split through its own workspace) and RMSNorms on
four default-priority streams, fifty rounds each, released together by a
barrier; every output equals the one a single thread computed first, bit for
bit (the kernels are deterministic).
"""
import threading

import pytest
import torch

from marlin_style_fluxbin_amd import W3Gemv
from marlin_style_fluxbin_amd.fused_modules import rms_norm
from tests.payloads import config_codes, layout_from_codes

pytestmark = pytest.mark.gpu

SHAPES = [(1024, 2048), (64, 4096), (2048, 1024), (300, 1536)]  # (64, 4096): K split over workgroups


def _workloads(gpu):
    loads = []
    for i, (o, k) in enumerate(SHAPES):
        codes, scales, zeros, perm = config_codes(o, k, seed=40 + i, zeros=True, scale_dtype=torch.float16,
                                                  permute=i % 2 == 1)
        dl = {n: t.to(gpu) for n, t in layout_from_codes(codes, scales, zeros, perm).items()}
        x = torch.randn(1, k, generator=torch.Generator().manual_seed(i)).to(torch.bfloat16).to(gpu)
        h = torch.randn(2, 4096, generator=torch.Generator().manual_seed(100 + i)).to(torch.bfloat16).to(gpu)
        w = (1 + 0.02 * torch.randn(4096, generator=torch.Generator().manual_seed(200 + i))).to(torch.bfloat16).to(gpu)
        loads.append((dl, x, h, w))
    return loads


def test_threads_on_separate_streams_match_serial(gpu):
    loads = _workloads(gpu)
    serial = []
    for dl, x, h, w in loads:
        out = torch.empty(1, dl["planes"].shape[2], dtype=torch.bfloat16, device=gpu)
        W3Gemv(dl)(x, out)
        serial.append((out.clone(), rms_norm(h, w, 1e-6).clone()))
    torch.cuda.synchronize()

    rounds = 50
    barrier = threading.Barrier(len(loads), timeout=60)
    results = [None] * len(loads)
    errors = []

    def worker(i):
        try:
            dl, x, h, w = loads[i]
            stream = torch.cuda.Stream(gpu)
            gemv = W3Gemv(dl)  # its own workspace: a K-split GEMV's partials are per call site
            outs = torch.empty(rounds, 1, dl["planes"].shape[2], dtype=torch.bfloat16, device=gpu)
            norms = torch.empty(rounds, *h.shape, dtype=torch.bfloat16, device=gpu)
            torch.cuda.synchronize()
            barrier.wait()
            with torch.cuda.stream(stream):
                for r in range(rounds):
                    gemv(x, outs[r])
                    norms[r] = rms_norm(h, w, 1e-6)
            stream.synchronize()
            results[i] = (outs, norms)
        except Exception as exc:  # reported after the join; the others stop waiting
            errors.append(f"thread {i}: {exc!r}")
            barrier.abort()

    threads = [threading.Thread(target=worker, args=(i,), daemon=True) for i in range(len(loads))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    assert not errors, errors
    for i, (outs, norms) in enumerate(results):
        want_out, want_norm = serial[i]
        assert torch.equal(outs, want_out.expand_as(outs)), f"GEMV {SHAPES[i]} differs under concurrency"
        assert torch.equal(norms, want_norm.expand_as(norms)), f"RMSNorm {i} differs under concurrency"



def test_field_plans_are_thread_local(gpu):
    """fx_w3_fields_plan is per calling thread: four threads each hold another
    plan (the one-tile kernel, two shared-staging plans, an M-row-only plan) and
    launch the one-row field GEMV and the four-row field GEMV on their own
    streams; every output equals the serial default's bit for bit (every plan
    gives the same bits), no thread's plan reaches another (the M-row-only plan
    would refuse the one-row call), and the main thread keeps the default."""
    from marlin_style_fluxbin_amd import _lib

    lib = _lib.library()
    o, k, m = 768, 4096, 4
    codes, scales, zeros, _ = config_codes(o, k, seed=77, zeros=True, scale_dtype=torch.float16)
    dl = {n: t.to(gpu) for n, t in layout_from_codes(codes, scales, zeros, None).items()}
    fields = torch.empty_like(dl["planes"])
    _lib.check(lib.fx_w3_planes_to_fields(dl["planes"].data_ptr(), fields.data_ptr(), o, k,
                                          _lib.stream_handle(gpu)), "planes_to_fields")
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16).to(gpu)

    def run(out1, out4):
        handle = _lib.stream_handle(gpu)
        _lib.check(lib.fx_w3_gemv_fields(x.data_ptr(), _lib.FX_BF16, fields.data_ptr(), dl["scales"].data_ptr(),
                                         _lib.FX_F16, dl["zeros"].data_ptr(), out1.data_ptr(), o, k, handle),
                   "gemv_fields")
        _lib.check(lib.fx_w3_gemv_fields_rows(x.data_ptr(), _lib.FX_BF16, fields.data_ptr(), dl["scales"].data_ptr(),
                                              _lib.FX_F16, dl["zeros"].data_ptr(), out4.data_ptr(), m, o, k, handle),
                   "gemv_fields_rows")

    want1 = torch.empty(1, o, dtype=torch.bfloat16, device=gpu)
    want4 = torch.empty(m, o, dtype=torch.bfloat16, device=gpu)
    run(want1, want4)
    torch.cuda.synchronize()

    plans = [(-1, 0, 0, 0), (3, 4, 2, 1), (1, 8, 1, 1), (1, 16, 2, 2)]
    rounds = 20
    barrier = threading.Barrier(len(plans), timeout=60)
    results, errors = [None] * len(plans), []

    def worker(i):
        try:
            _lib.check(lib.fx_w3_fields_plan(*plans[i]), "fields plan")
            stream = torch.cuda.Stream(gpu)
            out1 = torch.empty(rounds, 1, o, dtype=torch.bfloat16, device=gpu)
            out4 = torch.empty(rounds, m, o, dtype=torch.bfloat16, device=gpu)
            torch.cuda.synchronize()
            barrier.wait()
            with torch.cuda.stream(stream):
                for r in range(rounds):
                    if plans[i] == (1, 16, 2, 2):  # M-row only: this thread's one-row call refuses it
                        rc = lib.fx_w3_gemv_fields(x.data_ptr(), _lib.FX_BF16, fields.data_ptr(),
                                                   dl["scales"].data_ptr(), _lib.FX_F16, dl["zeros"].data_ptr(),
                                                   out1[r].data_ptr(), o, k, _lib.stream_handle(gpu))
                        assert rc == 1 and "only the M-row form" in lib.fx_last_error().decode()
                        out1[r].copy_(want1)
                        _lib.check(lib.fx_w3_gemv_fields_rows(
                            x.data_ptr(), _lib.FX_BF16, fields.data_ptr(), dl["scales"].data_ptr(), _lib.FX_F16,
                            dl["zeros"].data_ptr(), out4[r].data_ptr(), m, o, k, _lib.stream_handle(gpu)), "rows")
                    else:
                        run(out1[r], out4[r])
            stream.synchronize()
            results[i] = (out1, out4)
        except Exception as exc:
            errors.append(f"thread {i} plan {plans[i]}: {exc!r}")
            barrier.abort()
        finally:
            lib.fx_w3_fields_plan(0, 0, 0, 0)

    threads = [threading.Thread(target=worker, args=(i,), daemon=True) for i in range(len(plans))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    assert not errors, errors
    for i, (out1, out4) in enumerate(results):
        assert torch.equal(out1, want1.expand_as(out1)), f"plan {plans[i]}: one-row output differs"
        assert torch.equal(out4, want4.expand_as(out4)), f"plan {plans[i]}: four-row output differs"
    again1, again4 = torch.empty_like(want1), torch.empty_like(want4)
    run(again1, again4)  # the main thread still runs its default
    torch.cuda.synchronize()
    assert torch.equal(again1, want1) and torch.equal(again4, want4)
