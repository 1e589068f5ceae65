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

