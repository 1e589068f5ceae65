"""Benchmark of the W3 packed-LUT decode path on one MI355X.

Metric: W3 GEMV HBM GB/s (% of peak) per Qwen3-8B shape; batch-1
decode tokens/sec.  Workload (config 1): the seven Qwen3-8B Linear shapes of a
decoder layer at M = 1, W3 g128, fp16 scales U[0.005,0.02], zero-points U{3,4},
random codes, synthetic bf16 activations.

A "step" is one replay of a HIP graph that runs the seven W3 GEMVs of a decoder
layer for ``LAYERS`` distinct layers' payloads (so a replay streams ~600 MB of
distinct weights; MI355X's 256 MB Infinity Cache cannot hold them).  ``value``
is algorithmic bytes of all GEMVs in the timed replays / their wall time on the
GPU (HIP events on the launch stream).

Per shape, a graph of >= 50 launches over rotating payload copies (>= 300 MB)
gives the average launch duration (one w3_mfma_kernel launch per call, plus a
finish launch only for split-K plans); the same-run bf16 arm runs torch.matmul
(hipBLASLt) on dequantized bf16 weights with the same rotation.  ``roofline``
is the gate/up shape's measurement: the dominant kernel of a decode step.
``config.field_layout`` (and each shape's ``fields_*``) times the same payloads
after the library's bind-time repack into its field layout (same bytes, half
the dequant instructions), the format the native decode reads; each shape's
``fp6_*`` times the opt-in fp6 layout (gfx950's scaled f8f6f4 instruction) on
the same payloads.
``roofline.traffic`` is the HBM bytes per launch measured with rocprofv3 PMC
counters (FETCH_SIZE + WRITE_SIZE, scaled by a plain read kernel of known size),
read from ``profiles/w3_mfma_traffic.json`` when present.

Also in the line: ``config.fused_ops`` (config 2: RMSNorm, residual add + RMSNorm,
q/k norm + RoPE per launch beside HF's eager ops), ``config.two_base`` (config 4),
``config.decode`` (config 3: W3 and bf16, HF module tree and native chain, plus
the hybrid two-base native arm) and ``cpu_baseline``: the reference's CPU route
(dequantize + ``F.linear`` per call, as the product's CPU torch code restates it)
on config 0, at the host's thread budget and at one thread.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBPS = 8000.0
DECODE_WARMUP_REPLAYS = 2  # untimed graph replays before the timed ones in the decode arms
SHAPES = {  # name: (O, K)
    "q_proj": (4096, 4096), "k_proj": (1024, 4096), "v_proj": (1024, 4096), "o_proj": (4096, 4096),
    "gate_proj": (12288, 4096), "up_proj": (12288, 4096), "down_proj": (4096, 12288),
}
UNIQUE = {"q/o": (4096, 4096), "k/v": (1024, 4096), "gate/up": (12288, 4096), "down": (4096, 12288)}


def algorithmic_bytes(o: int, k: int, m: int = 1, zeros: bool = True, perm: bool = False) -> int:
    """Planes 3OK/8 + fp16 scales 2GO (+ uint8 zeros GO) (+ perm 2K) + x 2MK + y 2MO."""
    g = k // 128
    total = 3 * o * k // 8 + 2 * g * o + 2 * m * k + 2 * m * o
    if zeros:
        total += g * o
    if perm:
        total += 2 * k
    return total


def make_payloads(o, k, device, generator, copies):
    """``copies`` payloads stored back to back (planes [copies, G, 3, O, 16], scales,
    zeros), returned as the stacked tensors and per-copy views: one strided-batch
    launch walks the stacked tensors, the per-launch arms take the views."""
    import torch

    g = k // 128
    stacked = {
        "planes": torch.randint(0, 256, (copies, g, 3, o, 16), dtype=torch.uint8, device=device, generator=generator),
        "scales": (torch.rand((copies, g, o), device=device, generator=generator) * 0.015 + 0.005).half(),
        "zeros": torch.randint(3, 5, (copies, g, o), dtype=torch.uint8, device=device, generator=generator),
    }
    perm = torch.arange(k, dtype=torch.int16, device=device)
    views = [{"planes": stacked["planes"][i], "scales": stacked["scales"][i], "perm": perm,
              "zeros": stacked["zeros"][i]} for i in range(copies)]
    return stacked, views


def batched_call(lib, x, weights, stacked, out, o, k, fmt, device):
    """One fx_w3_gemv_strided_batched launch over every stacked payload (x row p
    for payload p)."""
    from marlin_style_fluxbin_amd import _lib

    n = weights.shape[0]
    if x.numel() < n * k or out.numel() < n * o or not (x.is_contiguous() and out.is_contiguous()):
        raise ValueError(f"strided batch of {n}: x needs {n} x {k} and out {n} x {o} contiguous elements")
    _lib.check(lib.fx_w3_gemv_strided_batched(
        x.data_ptr(), _lib.dtype_code(x.dtype), k, weights.data_ptr(), weights[0].numel(),
        stacked["scales"].data_ptr(), _lib.dtype_code(stacked["scales"].dtype), stacked["scales"][0].numel(),
        stacked["zeros"].data_ptr(), stacked["zeros"][0].numel(), out.data_ptr(), o, n, o, k, fmt,
        _lib.stream_handle(device)), "fx_w3_gemv_strided_batched")


def make_payload(o, k, device, generator):
    import torch

    g = k // 128
    planes = torch.randint(0, 256, (g, 3, o, 16), dtype=torch.uint8, device=device, generator=generator)
    scales = (torch.rand((g, o), device=device, generator=generator) * 0.015 + 0.005).half()
    zeros = torch.randint(3, 5, (g, o), dtype=torch.uint8, device=device, generator=generator)
    perm = torch.arange(k, dtype=torch.int16, device=device)
    return {"planes": planes, "scales": scales, "perm": perm, "zeros": zeros}


def time_graph(graph, steps, warmup, stream):
    """ms per replay; replays and both events are issued on ``stream``."""
    import torch

    with torch.cuda.stream(stream):
        for _ in range(warmup):
            graph.replay()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(steps):
            graph.replay()
        end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


PAIRED_WARMUP, PAIRED_ROUNDS = 20, 7  # the reference's protocol (acceleration_checks.py:42-64)


def paired_graph_timing(graphs: dict, stream, repeats: int) -> dict:
    """µs per launch of each arm: ``graphs`` maps an arm name to (graph, launches
    per replay).  The product's ``paired_cuda_timing`` -- 20 untimed replays per
    arm, then 7 rounds of ``repeats`` replays per arm with the arm order reversed
    on every other round, HIP events on ``stream`` -- and the median round."""
    import torch

    from marlin_style_fluxbin_amd.acceleration_checks import paired_cuda_timing

    with torch.cuda.stream(stream):
        timing = paired_cuda_timing({name: graph.replay for name, (graph, _) in graphs.items()},
                                    warmup=PAIRED_WARMUP, repeats=repeats, rounds=PAIRED_ROUNDS)
    return {name: {"us": timing[name]["median_us"] / launches,
                   "relative_range": round(timing[name]["relative_range"], 4)}
            for name, (_, launches) in graphs.items()}


def capture(fn, stream):
    import torch

    with torch.cuda.stream(stream):
        for _ in range(2):
            fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        fn()
    torch.cuda.synchronize()
    return graph


def dominant_fields_us(shapes):
    return (shapes.get("gate/up") or next(iter(shapes.values()))).get("fields_us")


def dominant_fields_frac(shapes):
    return (shapes.get("gate/up") or next(iter(shapes.values()))).get("fields_frac_hbm")


def bench_shape(o, k, device, steps, warmup, stream, min_bytes=320e6, min_copies=50):
    """Average launch time of the W3 GEMV arms and of the bf16 arm over rotating
    copies, every arm timed by :func:`paired_graph_timing` (alternating rounds,
    median): the planar kernel (identity order, as config 1 draws it), the same
    payloads with a desc_act column permutation (the reference's real artifacts;
    the kernel gathers x[perm]), the field layout, M = 2 / 4 / 8, the bf16 arm,
    and the dense fallback's restore (identity and permuted)."""
    import torch

    from marlin_style_fluxbin_amd import W3Gemv, _lib
    from marlin_style_fluxbin_amd.gptq_deployment import restore_planar_w3
    from marlin_style_fluxbin_amd.qwen3 import desc_act_perm
    from marlin_style_fluxbin_amd.w3_lut_deployment import restore_planar_w3_into

    gen = torch.Generator(device=device).manual_seed(o * 7 + k)
    cpu_gen = torch.Generator().manual_seed(o + k)
    nbytes = algorithmic_bytes(o, k)
    perm_bytes = algorithmic_bytes(o, k, perm=True)
    copies = max(min_copies, int(min_bytes // nbytes) + 1)
    stacked, payloads = make_payloads(o, k, device, gen, copies)
    gemvs = [W3Gemv(p, perm_identity=True) for p in payloads]
    # desc_act: each copy its own group-preserving order (perm = argsort(g_idx))
    permuted = [W3Gemv(dict(p, perm=desc_act_perm(k, cpu_gen, device)), perm_identity=False) for p in payloads]
    x = torch.randn(1, k, device=device, generator=gen).to(torch.bfloat16)
    out = torch.empty(1, o, device=device, dtype=torch.bfloat16)
    graphs = {}

    def over(calls):
        def run():
            for call in calls:
                call()
        return run

    graphs["w3"] = (capture(over([lambda g=g: g(x, out) for g in gemvs]), stream), copies)
    pout = torch.empty_like(out)
    graphs["w3_perm"] = (capture(over([lambda g=g: g(x, pout) for g in permuted]), stream), copies)
    # decoded_bf16 (the fast_corrected route: bf16 scales, zero-points 3 / 4): the
    # MFMA kernel with the +-3 correction chain, and the reference's table kernel
    # (w3_lut_m1_out, one group per split) on the same payloads
    from marlin_style_fluxbin_amd.w3_lut_deployment import load_w3_lut_extension

    scales16 = stacked["scales"].to(torch.bfloat16)
    decoded_views = [dict(p, scales=scales16[i]) for i, p in enumerate(payloads)]
    decoded = [W3Gemv(p, arithmetic="decoded_bf16", perm_identity=True) for p in decoded_views]
    dout = torch.empty_like(out)
    graphs["w3_decoded"] = (capture(over([lambda g=g: g(x, dout) for g in decoded]), stream), copies)
    table = load_w3_lut_extension(1024)
    table_ws = torch.empty(k // 128, o, dtype=torch.float32, device=device)
    tout = torch.empty_like(out)
    graphs["table_decoded"] = (capture(over([lambda p=p: table.m1_out(
        x, p["planes"], p["scales"], None, table_ws, tout, 1, True, zeros=p["zeros"]) for p in decoded_views]), stream),
        copies)
    # config 1's small-M variants: M activation rows against the same payloads
    xm = {m: torch.randn(m, k, device=device, generator=gen).to(torch.bfloat16) for m in (2, 4, 8)}
    om = {m: torch.empty(m, o, device=device, dtype=torch.bfloat16) for m in (2, 4, 8)}
    for m in (2, 4, 8):
        graphs[f"M={m}"] = (capture(over([lambda g=g, m=m: g(xm[m], om[m]) for g in gemvs]), stream), copies)

    # the same payloads repacked once into the field layout (fx_w3_planes_to_fields)
    # and read by fx_w3_gemv_fields: the decode graph's weight format
    lib = _lib.library()
    fields = [torch.empty_like(p["planes"]) for p in payloads]
    for p, f in zip(payloads, fields):
        _lib.check(lib.fx_w3_planes_to_fields(p["planes"].data_ptr(), f.data_ptr(), o, k,
                                              _lib.stream_handle(device)), "fx_w3_planes_to_fields")
    fout = torch.empty_like(out)

    def field_call(p, f):
        _lib.check(lib.fx_w3_gemv_fields(x.data_ptr(), _lib.dtype_code(x.dtype), f.data_ptr(),
                                         p["scales"].data_ptr(), _lib.dtype_code(p["scales"].dtype),
                                         p["zeros"].data_ptr(), fout.data_ptr(), o, k,
                                         _lib.stream_handle(device)), "fx_w3_gemv_fields")

    graphs["fields"] = (capture(over([lambda p=p, f=f: field_call(p, f) for p, f in zip(payloads, fields)]),
                                stream), copies)
    # the opt-in fp6 layout (fx_w3_planes_to_fp6 / fx_w3_gemv_fp6) on the same payloads
    fp6 = [torch.empty_like(p["planes"]) for p in payloads]
    for p, f in zip(payloads, fp6):
        _lib.check(lib.fx_w3_planes_to_fp6(p["planes"].data_ptr(), f.data_ptr(), o, k,
                                           _lib.stream_handle(device)), "fx_w3_planes_to_fp6")
    f6out = torch.empty_like(out)

    def fp6_call(p, f):
        _lib.check(lib.fx_w3_gemv_fp6(x.data_ptr(), _lib.dtype_code(x.dtype), f.data_ptr(),
                                      p["scales"].data_ptr(), _lib.dtype_code(p["scales"].dtype),
                                      p["zeros"].data_ptr(), f6out.data_ptr(), o, k,
                                      _lib.stream_handle(device)), "fx_w3_gemv_fp6")

    graphs["fp6"] = (capture(over([lambda p=p, f=f: fp6_call(p, f) for p, f in zip(payloads, fp6)]), stream), copies)
    # config 1's small-M variants on the field layout (fx_w3_gemv_fields_rows)
    fom = {m: torch.empty(m, o, device=device, dtype=torch.bfloat16) for m in (2, 4, 8)}

    def rows_call(p, f, m):
        _lib.check(lib.fx_w3_gemv_fields_rows(xm[m].data_ptr(), _lib.dtype_code(xm[m].dtype), f.data_ptr(),
                                              p["scales"].data_ptr(), _lib.dtype_code(p["scales"].dtype),
                                              p["zeros"].data_ptr(), fom[m].data_ptr(), m, o, k,
                                              _lib.stream_handle(device)), "fx_w3_gemv_fields_rows")

    for m in (2, 4, 8):
        graphs[f"fields M={m}"] = (capture(over([lambda p=p, f=f, m=m: rows_call(p, f, m)
                                                 for p, f in zip(payloads, fields)]), stream), copies)
    # steady state: the same payloads walked by one launch (fx_w3_gemv_strided_batched),
    # planar and field layout -- the kernel without the per-launch cost
    fields_stacked = torch.stack(fields)
    # (default arguments bind the tensors now: the graphs hold their addresses, and
    # a later rebinding of a name must not free what a graph writes)
    xs = x.expand(copies, k).contiguous()
    batch_out = torch.empty(copies, o, device=device, dtype=torch.bfloat16)
    graphs["w3_batched"] = (capture(lambda xs=xs, w=stacked["planes"], y=batch_out: batched_call(
        lib, xs, w, stacked, y, o, k, _lib.PAYLOAD_PLANAR, device), stream), copies)
    graphs["fields_batched"] = (capture(lambda xs=xs, w=fields_stacked, y=batch_out: batched_call(
        lib, xs, w, stacked, y, o, k, _lib.PAYLOAD_FIELDS, device), stream), copies)

    # same-run bf16 arm: dense bf16 weights (5.3x the bytes), same rotation rule
    bf16_bytes = 2 * o * k + 2 * k + 2 * o
    bcopies = max(min_copies // 5, int(min_bytes // bf16_bytes) + 1)
    weights = [restore_planar_w3(payloads[i % copies], dtype=torch.bfloat16, perm_identity=True)
               for i in range(bcopies)]
    bout = torch.empty(1, o, device=device, dtype=torch.bfloat16)
    graphs["bf16"] = (capture(over([lambda w=w: torch.matmul(x, w.t(), out=bout) for w in weights]), stream),
                      bcopies)
    # the dense fallback's dequantize (fx_w3_restore) into the bf16 arm's buffers:
    # reads the payload, writes the 2OK-byte weight; identity order, then with a
    # scattered column permutation (the LDS-staged form)
    restore_bytes = algorithmic_bytes(o, k, m=0) + 2 * o * k
    graphs["restore"] = (capture(over([lambda i=i, w=w: restore_planar_w3_into(payloads[i % copies], w,
                                                                                 perm_identity=True)
                                       for i, w in enumerate(weights)]), stream), bcopies)
    shuffled = [dict(payloads[i % copies], perm=torch.randperm(k, generator=gen, device=device).to(torch.int16))
                for i in range(bcopies)]
    graphs["restore_permuted"] = (capture(over([lambda p=p, w=w: restore_planar_w3_into(p, w, perm_identity=False)
                                                for p, w in zip(shuffled, weights)]), stream), bcopies)

    t = paired_graph_timing(graphs, stream, repeats=max(steps, 10))
    # the arms compute the same GEMV of the last payload: the field layout within
    # two output ulps (fp32 sums in another order, fp16 MFMA); the permuted arm
    # bit-equal to the identity kernel on the gathered row
    gemvs[-1](x, out)
    field_call(payloads[-1], fields[-1])
    fp6_call(payloads[-1], fp6[-1])
    permuted[-1](x, pout)
    gathered = torch.empty_like(out)
    gemvs[-1](x[:, permuted[-1].layout["perm"].long()].contiguous(), gathered)
    torch.cuda.synchronize()
    if not torch.allclose(fout.float(), out.float(), rtol=2 ** -7, atol=1e-3 * float(out.float().abs().max())):
        raise RuntimeError("field-layout GEMV disagrees with the planar GEMV")
    if not torch.allclose(f6out.float(), out.float(), rtol=2 ** -7, atol=1e-3 * float(out.float().abs().max())):
        raise RuntimeError("fp6-layout GEMV disagrees with the planar GEMV")
    if not torch.equal(pout, gathered):
        raise RuntimeError("permuted GEMV differs from the identity GEMV on the gathered activations")
    decoded[-1](x, dout)
    table.m1_out(x, decoded_views[-1]["planes"], decoded_views[-1]["scales"], None, table_ws, tout, 1, True,
                 zeros=decoded_views[-1]["zeros"])
    torch.cuda.synchronize()
    if not torch.allclose(dout.float(), tout.float(), rtol=2 ** -7, atol=1e-3 * float(tout.float().abs().max())):
        raise RuntimeError("decoded_bf16 MFMA GEMV disagrees with the table kernel")
    batched_call(lib, xs, stacked["planes"], stacked, batch_out, o, k, _lib.PAYLOAD_PLANAR, device)
    torch.cuda.synchronize()
    if not torch.equal(batch_out[-1:], out):
        raise RuntimeError("strided-batch GEMV differs from the single launch")
    small_m = {}
    for m in (2, 4, 8):
        gemvs[-1](xm[m], om[m])
        rows_call(payloads[-1], fields[-1], m)
        torch.cuda.synchronize()
        if not torch.allclose(fom[m].float(), om[m].float(), rtol=2 ** -7,
                              atol=1e-3 * float(om[m].float().abs().max())):
            raise RuntimeError(f"field-layout M={m} GEMV disagrees with the planar GEMV")
        m_us, f_us = t[f"M={m}"]["us"], t[f"fields M={m}"]["us"]
        m_bytes = algorithmic_bytes(o, k, m)
        small_m[f"M={m}"] = {"us": round(m_us, 3), "GBps": round(m_bytes / m_us / 1e3, 1),
                             "frac_hbm": round(m_bytes / m_us / 1e3 / HBM_PEAK_GBPS, 4),
                             "algorithmic_bytes": m_bytes, "vs_M=1": round(m_us / t["w3"]["us"], 3),
                             "fields_us": round(f_us, 3), "fields_GBps": round(m_bytes / f_us / 1e3, 1),
                             "fields_vs_planar": round(f_us / m_us, 3)}
    w3_us, fields_us, bf16_us, perm_us = t["w3"]["us"], t["fields"]["us"], t["bf16"]["us"], t["w3_perm"]["us"]
    decoded_us, table_us = t["w3_decoded"]["us"], t["table_decoded"]["us"]
    restore_us, restore_perm_us = t["restore"]["us"], t["restore_permuted"]["us"]
    steady = {}
    for name, arm in (("planar", "w3_batched"), ("fields", "fields_batched")):
        us = t[arm]["us"]
        steady[name] = {"us_per_gemv": round(us, 3), "GBps": round(nbytes / us / 1e3, 1),
                        "frac_hbm": round(nbytes / us / 1e3 / HBM_PEAK_GBPS, 4)}
    steady["note"] = (f"one fx_w3_gemv_strided_batched launch over the {copies} payloads (bit-identical "
                      "outputs): the kernel's rate without the per-launch cost")
    fp6_us = t["fp6"]["us"]
    del graphs, shuffled, weights, payloads, gemvs, permuted, fields, fp6, fields_stacked, stacked, batch_out, decoded
    del decoded_views, scales16, table_ws
    torch.cuda.empty_cache()
    return {
        "O": o, "K": k, "copies": copies, "algorithmic_bytes": nbytes,
        "w3_us": round(w3_us, 3), "w3_GBps": round(nbytes / w3_us / 1e3, 1),
        "w3_frac_hbm": round(nbytes / w3_us / 1e3 / HBM_PEAK_GBPS, 4),
        "w3_perm_us": round(perm_us, 3), "w3_perm_GBps": round(perm_bytes / perm_us / 1e3, 1),
        "w3_perm_frac_hbm": round(perm_bytes / perm_us / 1e3 / HBM_PEAK_GBPS, 4),
        "decoded_bf16_us": round(decoded_us, 3), "decoded_bf16_vs_structural": round(decoded_us / w3_us, 3),
        "table_decoded_bf16_us": round(table_us, 3),
        "bf16_us": round(bf16_us, 3), "bf16_GBps": round(bf16_bytes / bf16_us / 1e3, 1),
        "w3_speedup_vs_bf16": round(bf16_us / w3_us, 3),
        "fields_us": round(fields_us, 3), "fields_GBps": round(nbytes / fields_us / 1e3, 1),
        "fields_frac_hbm": round(nbytes / fields_us / 1e3 / HBM_PEAK_GBPS, 4),
        "fp6_us": round(fp6_us, 3), "fp6_GBps": round(nbytes / fp6_us / 1e3, 1),
        "fp6_vs_fields": round(fp6_us / fields_us, 3),
        "small_m": small_m,
        "steady_state": steady,
        "restore_us": round(restore_us, 3), "restore_GBps": round(restore_bytes / restore_us / 1e3, 1),
        "restore_permuted_us": round(restore_perm_us, 3),
        "restore_permuted_GBps": round((restore_bytes + 2 * k) / restore_perm_us / 1e3, 1),
        "timing": {"protocol": f"alternating arm order, {PAIRED_WARMUP} warm-up replays per arm, median of "
                               f"{PAIRED_ROUNDS} rounds of {max(steps, 10)} replays",
                   "relative_range": {name: v["relative_range"] for name, v in t.items()}},
    }


FIELDS_PLANS = [(1, 8, 1, 1), (1, 8, 3, 3), (2, 4, 2, 1), (3, 4, 2, 1), (4, 2, 4, 1)]
SWEEP_SHAPES = {"q/o": (4096, 4096), "k/v": (1024, 4096), "gate/up": (12288, 4096), "down": (4096, 12288),
                "gate|up": (24576, 4096), "q|k|v": (6144, 4096), "gate|up normed swiglu": (24576, 4096),
                "q|k|v normed": (6144, 4096)}
NORMED_SWEEP = {"gate|up normed swiglu": 1, "q|k|v normed": 0}  # name -> swiglu


def fields_plan_sweep(device, stream, shapes=None, min_bytes=320e6, min_copies=50, steady_state=True):
    """µs per launch of the field-layout GEMV under every plan that can take each
    Qwen3-8B shape (fx_w3_fields_plan) and the one-tile kernel (plan "one-tile"),
    graph-timed over rotating payloads with the paired protocol; the outputs of
    every plan are checked bit-equal to the one-tile kernel's on the first copy."""
    import torch

    from marlin_style_fluxbin_amd import _lib

    lib = _lib.library()
    result = {}
    for name, (o, k) in (shapes or SWEEP_SHAPES).items():
        gen = torch.Generator(device=device).manual_seed(o + 3 * k)
        copies = max(min_copies, int(min_bytes // algorithmic_bytes(o, k)) + 1)
        with torch.cuda.stream(stream):  # every allocation, repack and call on the one stream
            stacked, payloads = make_payloads(o, k, device, gen, copies)
            fields = torch.empty_like(stacked["planes"])
            for p in range(copies):
                _lib.check(lib.fx_w3_planes_to_fields(stacked["planes"][p].data_ptr(), fields[p].data_ptr(), o, k,
                                                      _lib.stream_handle(device)), "planes_to_fields")
            x = torch.randn(1, k, device=device, generator=gen).to(torch.bfloat16)
            out = torch.empty(1, o, device=device, dtype=torch.bfloat16)
        torch.cuda.synchronize()

        def call(p, dst=out):
            _lib.check(lib.fx_w3_gemv_fields(x.data_ptr(), _lib.FX_BF16, fields[p].data_ptr(),
                                             payloads[p]["scales"].data_ptr(), _lib.FX_F16,
                                             payloads[p]["zeros"].data_ptr(), dst.data_ptr(), o, k,
                                             _lib.stream_handle(device)), "gemv_fields")

        normed = name in NORMED_SWEEP
        if normed:  # the decode chain's normalising form (and SwiGLU at gate|up)
            h = x
            sums = (h.float().view(-1, 16) ** 2).sum(1).contiguous()
            norm_w = (1 + 0.05 * torch.randn(k, device=device, generator=gen)).to(torch.bfloat16)
            swiglu = NORMED_SWEEP[name]
            out = torch.empty(1, o // 2 if swiglu else o, device=device, dtype=torch.bfloat16)
            torch.cuda.synchronize()

            def call(p, dst=out):
                _lib.check(lib.fx_w3_gemv_rmsnormed(h.data_ptr(), _lib.FX_BF16, fields[p].data_ptr(),
                                                    payloads[p]["scales"].data_ptr(), _lib.FX_F16,
                                                    payloads[p]["zeros"].data_ptr(), sums.data_ptr(), k // 16,
                                                    norm_w.data_ptr(), 1e-6, None, dst.data_ptr(), o, k, swiglu,
                                                    _lib.PAYLOAD_FIELDS, _lib.stream_handle(device)), "rmsnormed")

        def run():
            for p in range(copies):
                call(p)

        plans = [("one-tile", (-1, 0, 0, 0)), ("default", (0, 0, 0, 0))]
        plans += [(",".join(map(str, pl)), pl) for pl in FIELDS_PLANS
                  if o % 16 == 0 and k % 512 == 0 and k // 512 <= pl[3] * pl[0] * pl[1]]
        graphs, first = {}, {}
        for label, plan in plans:
            _lib.check(lib.fx_w3_fields_plan(*plan), "fields plan")
            try:
                with torch.cuda.stream(stream):
                    refs = [torch.full_like(out, float("nan")) for _ in range(2)]
                    for ref in refs:
                        call(0, ref)
                    torch.cuda.synchronize()
                    first[label] = refs
                    graphs[label] = (capture(run, stream), copies)
            finally:
                _lib.check(lib.fx_w3_fields_plan(0, 0, 0, 0), "fields plan reset")
        want = first["one-tile"][0]
        differing = {label: int((refs[0] != want).sum()) + int((refs[1] != want).sum()) for label, refs in first.items()}
        same = all(n == 0 for n in differing.values())
        timing = paired_graph_timing(graphs, stream, repeats=10)
        # steady state: one strided launch walks every payload (no per-launch cost)
        steady = {}
        if steady_state and not normed and (o // 16) % 8 == 0:
            xs = torch.randn(copies, k, device=device, generator=gen).to(torch.bfloat16)
            outs = torch.empty(copies, o, device=device, dtype=torch.bfloat16)
            torch.cuda.synchronize()
            sgraphs = {}
            for label, plan in plans:
                if plan[0] > 0 and (o // 16 + plan[0] - 1) // plan[0] % 8:
                    continue
                _lib.check(lib.fx_w3_fields_plan(*plan), "fields plan")
                try:
                    sgraphs[label] = (capture(lambda: batched_call(lib, xs, fields, stacked, outs, o, k,
                                                                   _lib.PAYLOAD_FIELDS, device), stream), copies)
                finally:
                    _lib.check(lib.fx_w3_fields_plan(0, 0, 0, 0), "fields plan reset")
            steady = {label: round(t["us"], 3) for label, t in paired_graph_timing(sgraphs, stream, repeats=5).items()}
            del sgraphs, xs, outs
        nbytes = algorithmic_bytes(o, k)
        result[name] = {"O": o, "K": k, "bit_equal": same, "differing": differing,
                        "us": {label: round(t["us"], 3) for label, t in timing.items()},
                        "steady_us": steady,
                        "frac_hbm": {label: round(nbytes / (t["us"] * 1e3) / HBM_PEAK_GBPS, 4) for label, t in timing.items()}}
        print(f"# sweep {name}: {result[name]}", file=sys.stderr, flush=True)
        del graphs, fields, stacked, payloads
        torch.cuda.empty_cache()
    return result


ROWS_ONLY_PLANS = [(1, 12, 2, 2), (1, 16, 2, 2)]
ROWS_SHAPES = {"q/o": (4096, 4096), "k/v": (1024, 4096), "gate/up": (12288, 4096), "down": (4096, 12288)}


def rows_sweep(device, stream, shapes=None, rows=(2, 4, 8), min_bytes=320e6, min_copies=50):
    """µs per launch of M activation rows (config 1's small-M case) on the field
    layout (fx_w3_gemv_fields_rows, every plan that takes the shape and the default
    one) next to the planar fx_w3_gemv on the same payloads, graph-timed over
    rotating payloads with the paired protocol; every plan's output is checked
    bit-equal to the default plan's."""
    import torch

    from marlin_style_fluxbin_amd import W3Gemv, _lib

    lib = _lib.library()
    result = {}
    for name, (o, k) in (shapes or ROWS_SHAPES).items():
        gen = torch.Generator(device=device).manual_seed(o + 5 * k)
        copies = max(min_copies, int(min_bytes // algorithmic_bytes(o, k)) + 1)
        with torch.cuda.stream(stream):
            stacked, payloads = make_payloads(o, k, device, gen, copies)
            fields = torch.empty_like(stacked["planes"])
            for p in range(copies):
                _lib.check(lib.fx_w3_planes_to_fields(stacked["planes"][p].data_ptr(), fields[p].data_ptr(), o, k,
                                                      _lib.stream_handle(device)), "planes_to_fields")
            gemvs = [W3Gemv(p, perm_identity=True) for p in payloads]
        torch.cuda.synchronize()
        shape = {"O": o, "K": k, "copies": copies}
        for m in rows:
            with torch.cuda.stream(stream):
                x = torch.randn(m, k, device=device, generator=gen).to(torch.bfloat16)
                out = torch.empty(m, o, device=device, dtype=torch.bfloat16)
            torch.cuda.synchronize()

            def call(p, dst=out, x=x, m=m):
                _lib.check(lib.fx_w3_gemv_fields_rows(x.data_ptr(), _lib.FX_BF16, fields[p].data_ptr(),
                                                      payloads[p]["scales"].data_ptr(), _lib.FX_F16,
                                                      payloads[p]["zeros"].data_ptr(), dst.data_ptr(), m, o, k,
                                                      _lib.stream_handle(device)), "gemv_fields_rows")

            graphs = {"planar": (capture(lambda x=x, out=out: [g(x, out) for g in gemvs], stream), copies)}
            refs = {}
            nb = k // 512
            # a solo plan (one tile) restages per batch; the others
            # hold every batch in LDS: 24 of four rows (eight rows past 8 batches
            # run as chunks of four)
            plans = [("default", (0, 0, 0, 0))] + [
                (",".join(map(str, pl)), pl) for pl in FIELDS_PLANS + ROWS_ONLY_PLANS
                if nb <= pl[3] * pl[0] * pl[1] and (pl[0] == 1 or nb <= 24)]
            for label, plan in plans:
                _lib.check(lib.fx_w3_fields_plan(*plan), "fields plan")
                try:
                    with torch.cuda.stream(stream):
                        refs[label] = torch.full_like(out, float("nan"))
                        call(0, refs[label])
                        torch.cuda.synchronize()
                        graphs[label] = (capture(lambda: [call(p) for p in range(copies)], stream), copies)
                finally:
                    _lib.check(lib.fx_w3_fields_plan(0, 0, 0, 0), "fields plan reset")
            with torch.cuda.stream(stream):
                planar = torch.empty_like(out)
                gemvs[0](x, planar)
            torch.cuda.synchronize()
            same = all(torch.equal(r, refs["default"]) for r in refs.values())
            # the two layouts sum in other orders: within the GEMV's output ulps
            close = torch.allclose(refs["default"].float(), planar.float(), rtol=2 ** -7,
                                   atol=1e-3 * float(planar.float().abs().max()))
            timing = paired_graph_timing(graphs, stream, repeats=10)
            shape[f"M={m}"] = {"bit_equal_plans": same, "close_to_planar": close,
                               "us": {label: round(t["us"], 3) for label, t in timing.items()}}
            print(f"# rows {name} M={m}: {shape[f'M={m}']}", file=sys.stderr, flush=True)
            del graphs
        result[name] = shape
        del fields, stacked, payloads, gemvs
        torch.cuda.empty_cache()
    return result


def fused_ops_bench(device, steps, warmup, stream, launches=64, seed=0):
    """Config 2: the fused non-Linear decode ops at Qwen3-8B shapes, batch 1, one
    token.  Per launch (a graph of ``launches`` calls over distinct inputs and
    positions): RMSNorm over hidden 4096; the residual add fused with RMSNorm;
    per-head q/k RMSNorm + RoPE (32 query and 8 KV heads of 128, theta 1e6,
    positions uniform in [0, 4095]) with the value copied into its cache slot,
    one launch.  Beside each: the HF eager ops they replace (Qwen3RMSNorm's
    arithmetic, q_norm / k_norm + apply_rotary_pos_emb), graph-captured the same
    way, and the largest ulp distance between the two outputs."""
    import torch
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RotaryEmbedding, apply_rotary_pos_emb

    from marlin_style_fluxbin_amd import _lib
    from marlin_style_fluxbin_amd.fused_modules import add_rms_norm, head_norm_rope, rms_norm, rms_norm_reference
    from marlin_style_fluxbin_amd.qwen3 import qwen3_config

    g = torch.Generator(device=device).manual_seed(seed)
    bf = torch.bfloat16
    eps = 1e-6

    def bf16_ulps(a, b):
        ia = a.contiguous().view(torch.int16).int()
        ib = b.contiguous().view(torch.int16).int()
        ia = torch.where(ia < 0, -32768 - ia, ia)  # sign-magnitude -> ordered integers
        ib = torch.where(ib < 0, -32768 - ib, ib)
        return int((ia - ib).abs().max())

    def paired(fused, eager):
        """Fused launch vs HF's eager ops, alternating rounds (paired_graph_timing)."""
        t = paired_graph_timing({"fused_us": (capture(fused, stream), launches),
                                 "hf_eager_us": (capture(eager, stream), launches)}, stream, repeats=steps)
        return {name: round(v["us"], 3) for name, v in t.items()}

    # RMSNorm and residual add + RMSNorm, hidden 4096
    xs = [torch.randn(1, 4096, device=device, generator=g).to(bf) for _ in range(launches)]
    res = [torch.randn(1, 4096, device=device, generator=g).to(bf) for _ in range(launches)]
    w = (1 + 0.02 * torch.randn(4096, device=device, generator=g)).to(bf)
    outs = [torch.empty_like(x) for x in xs]
    res_out = [torch.empty_like(x) for x in xs]
    ref_outs = [torch.empty_like(x) for x in xs]

    def norm_fused():
        for x, o in zip(xs, outs):
            rms_norm(x, w, eps, out=o)

    def norm_eager():
        for x, o in zip(xs, ref_outs):
            o.copy_(rms_norm_reference(x, w, eps))

    def add_norm_fused():
        for x, r, o, ro in zip(xs, res, outs, res_out):
            add_rms_norm(x, r, w, eps, out=o, residual_out=ro)

    def add_norm_eager():
        for x, r, o, ro in zip(xs, res, ref_outs, res_out):
            ro.copy_(x + r)
            o.copy_(rms_norm_reference(ro, w, eps))

    result = {"rmsnorm_4096": paired(norm_fused, norm_eager)}
    norm_fused()
    norm_eager()
    torch.cuda.synchronize()
    result["rmsnorm_4096"]["max_ulps_vs_hf"] = max(bf16_ulps(a, b) for a, b in zip(outs, ref_outs))
    result["add_rmsnorm_4096"] = paired(add_norm_fused, add_norm_eager)
    add_norm_fused()
    fused_add = [o.clone() for o in outs]
    add_norm_eager()
    torch.cuda.synchronize()
    result["add_rmsnorm_4096"]["max_ulps_vs_hf"] = max(bf16_ulps(a, b) for a, b in zip(fused_add, ref_outs))

    # per-head q/k RMSNorm + RoPE (+ v into its cache slot), HF's rotary rows
    config = qwen3_config()
    rotary = Qwen3RotaryEmbedding(config=config).to(device)
    positions = torch.randint(0, 4096, (launches,), device=device, generator=g)
    cos, sin = rotary(xs[0], positions[None])  # [1, launches, 128] in bf16
    cos, sin = cos[0].contiguous(), sin[0].contiguous()
    qs = [torch.randn(32, 128, device=device, generator=g).to(bf) for _ in range(launches)]
    ks = [torch.randn(8, 128, device=device, generator=g).to(bf) for _ in range(launches)]
    vs = [torch.randn(8, 128, device=device, generator=g).to(bf) for _ in range(launches)]
    qw = (1 + 0.02 * torch.randn(128, device=device, generator=g)).to(bf)
    kw = (1 + 0.02 * torch.randn(128, device=device, generator=g)).to(bf)
    q_out = [torch.empty_like(q) for q in qs]
    k_cache = torch.zeros(8, launches, 128, device=device, dtype=bf)
    v_cache = torch.zeros(8, launches, 128, device=device, dtype=bf)
    q_ref = [torch.empty_like(q) for q in qs]
    k_ref = torch.zeros_like(k_cache)
    v_ref = torch.zeros_like(v_cache)
    strides = dict(in_strides=(0, 128, 0))

    def rope_fused():
        for i in range(launches):
            head_norm_rope([
                dict(x=qs[i], out=q_out[i], weight=qw, heads=32, rope=True, out_strides=(0, 128, 0), **strides),
                dict(x=ks[i], out=k_cache[:, i], weight=kw, heads=8, rope=True,
                     out_strides=(0, launches * 128, 0), **strides),
                dict(x=vs[i], out=v_cache[:, i], weight=None, heads=8, rope=False,
                     out_strides=(0, launches * 128, 0), **strides),
            ], cos=cos[i], sin=sin[i], eps=eps, rope_mode=_lib.ROPE_STOCK)

    def rope_eager():
        for i in range(launches):
            qn = rms_norm_reference(qs[i], qw, eps)[None, :, None]  # [1, 32, 1, 128]
            kn = rms_norm_reference(ks[i], kw, eps)[None, :, None]
            qr, kr = apply_rotary_pos_emb(qn, kn, cos[i][None, None], sin[i][None, None])
            q_ref[i].copy_(qr[0, :, 0])
            k_ref[:, i].copy_(kr[0, :, 0])
            v_ref[:, i].copy_(vs[i])

    result["qk_norm_rope_32q_8kv"] = paired(rope_fused, rope_eager)
    rope_fused()
    rope_eager()
    torch.cuda.synchronize()
    result["qk_norm_rope_32q_8kv"]["max_ulps_vs_hf"] = max(
        max(bf16_ulps(a, b) for a, b in zip(q_out, q_ref)), bf16_ulps(k_cache, k_ref))
    result["qk_norm_rope_32q_8kv"]["v_slots_equal"] = bool(torch.equal(v_cache, v_ref))
    result["note"] = ("launch-bound: each call moves under 25 KB; the fused launch replaces the eager ops' "
                      "kernels (the norm in the decode graph is further folded into the GEMV staging); "
                      f"paired timing: {PAIRED_WARMUP} warm-up replays, median of {PAIRED_ROUNDS} alternating rounds")
    return result


def two_base_bench(device, steps, warmup, stream, o=12288, k=4096, salient=32, min_bytes=640e6):
    """Config 4: rank-one two-base GEMV with 32 salient columns at the gate shape,
    M=1, over rotating payload copies, beside the bf16 arm on the dense weight."""
    import torch

    from marlin_style_fluxbin_amd.two_base import TwoBaseGemv, pack_rank_one_planes, rank_one_reference_weight

    gen = torch.Generator(device=device).manual_seed(4)
    nbytes = (2 * o * k // 8 + 4 * o + 2 * o + 2 * k + 2 * salient * o + 4 * salient) + 2 * k + 2 * o
    copies = max(50, int(min_bytes // nbytes) + 1)

    def payload():
        bases = torch.randint(0, 2, (2, o, k), device=device, generator=gen, dtype=torch.int8) * 2 - 1
        return {
            "planes": pack_rank_one_planes(bases),
            "coef": (torch.rand(2, o, device=device, generator=gen) + 0.5).half(),
            "srow": (torch.rand(o, device=device, generator=gen) * 0.015 + 0.005).half(),
            "tcol": (torch.rand(k, device=device, generator=gen) * 0.4 + 0.8).half(),
            "salient": (torch.randn(o, salient, device=device, generator=gen) * 0.05).bfloat16(),
            "salient_idx": torch.randperm(k, device=device, generator=gen)[:salient].sort().values.int(),
        }

    layouts = [payload() for _ in range(copies)]
    gemvs = [TwoBaseGemv(layout) for layout in layouts]
    x = torch.randn(1, k, device=device, generator=gen).to(torch.bfloat16)
    outs = [torch.empty(1, o, dtype=torch.bfloat16, device=device) for _ in range(copies)]
    # parity spot check against the dequantize-then-matmul of the same payload (fp32)
    gemvs[0](x, outs[0])
    want = x.float() @ rank_one_reference_weight(layouts[0]).t()
    max_rel = float((outs[0].float() - want).abs().max() / want.abs().max())

    def run():
        for gemv, out in zip(gemvs, outs):
            gemv(x, out)

    dense_copies = max(4, int(min_bytes // (2 * o * k)) + 1)
    dense = [rank_one_reference_weight(layouts[i % copies], torch.bfloat16) for i in range(dense_copies)]

    def bf16_arm():
        for i, w in enumerate(dense):
            torch.matmul(x, w.t(), out=outs[i % copies])

    t = paired_graph_timing({"two_base": (capture(run, stream), copies),
                             "bf16": (capture(bf16_arm, stream), dense_copies)}, stream, repeats=max(steps, 10))
    ms, ms_bf16 = t["two_base"]["us"] / 1e3, t["bf16"]["us"] / 1e3
    gbps = nbytes / (ms / 1e3) / 1e9
    traffic = None
    traffic_file = ROOT / "profiles" / "w3_mfma_traffic.json"
    if traffic_file.exists():
        traffic = json.loads(traffic_file.read_text()).get("two_base", {}).get("rank_one_kernel", {}).get(
            "traffic_bytes")
    return {
        "workload": f"config 4: rank-one two-base GEMV {o}x{k}, M=1, {salient} salient bf16 columns",
        "traffic_bytes": traffic,
        "algorithmic_bytes": nbytes,
        "us": round(ms * 1e3, 3),
        "GBps": round(gbps, 1),
        "frac_hbm": round(gbps / HBM_PEAK_GBPS, 4),
        "bf16_arm_us": round(ms_bf16 * 1e3, 3),
        "speedup_vs_bf16": round(ms_bf16 / ms, 3),
        "copies": copies,
        "timing": {"protocol": f"paired, {PAIRED_WARMUP} warm-up replays, median of {PAIRED_ROUNDS} rounds",
                   "relative_range": {name: v["relative_range"] for name, v in t.items()}},
        "parity_max_rel_vs_fp32_dequant_matmul": round(max_rel, 6),
        "data": "synthetic: random +-1 bases, a1,a2 ~U[0.5,1.5], s_r ~U[0.005,0.02], t_c ~U[0.8,1.2] (fp16), "
                "salient bf16 ~N(0,0.05), x bf16 ~N(0,1)",
    }


def _cpu_model_name() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(warmup=3, repeats=10):
    """The reference's CPU route on config 0 (q_proj 4096 x 4096, M = 1, fp16 scales,
    zero-points U{3,4}), timed on this host's cores.

    The reference runs ``PackedW3Linear(fallback='dense')`` on CPU tensors as
    ``F.linear(x, restore_planar_w3(layout, x.dtype))`` (w3_lut_deployment.py:327-333,
    gptq_deployment.py:247-260): the weight is dequantized on every call.  Its
    restatement here is the product's CPU torch code for those two functions.
    Arms: (1) dequantize + F.linear in bf16 per call (the reference's route, the
    reported value); (2) ``structural_w3_matvec`` (the grouped fp32 form,
    gptq_deployment.py:263-277); (3) F.linear on a weight dequantized once.  Each
    arm at the host thread budget (``min(os.cpu_count(), OMP_NUM_THREADS)``) and at
    one thread; ``warmup`` untimed calls, then the median of ``repeats``."""
    import os
    import statistics

    import torch
    import torch.nn.functional as F

    from marlin_style_fluxbin_amd.gptq_deployment import planar_from_codes, restore_planar_w3, structural_w3_matvec

    o = k = 4096
    g = torch.Generator().manual_seed(0)
    codes = torch.randint(0, 8, (k, o), generator=g, dtype=torch.uint8)
    layout = {"planes": planar_from_codes(codes),
              "scales": (torch.rand((k // 128, o), generator=g) * 0.015 + 0.005).to(torch.float16),
              "perm": torch.arange(k, dtype=torch.int16),
              "zeros": torch.randint(3, 5, (k // 128, o), generator=g, dtype=torch.uint8)}
    x = torch.randn(1, k, generator=torch.Generator().manual_seed(0)).to(torch.bfloat16)
    dense = restore_planar_w3(layout, dtype=torch.bfloat16)
    arms = {
        "dequantize_per_call_linear_bf16": lambda: F.linear(x, restore_planar_w3(layout, dtype=torch.bfloat16)),
        "structural_fp32": lambda: structural_w3_matvec(x, layout),
        "linear_bf16_predequantized": lambda: F.linear(x, dense),
    }
    budget = min(os.cpu_count() or 1, int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1)))
    previous = torch.get_num_threads()
    results = {}
    try:
        for threads in sorted({budget, 1}, reverse=True):
            torch.set_num_threads(threads)
            for name, fn in arms.items():
                for _ in range(warmup):
                    fn()
                samples = []
                for _ in range(repeats):
                    t = time.perf_counter()
                    fn()
                    samples.append(time.perf_counter() - t)
                ms = statistics.median(samples) * 1e3
                results[f"{name}@{threads}t"] = {"median_ms": round(ms, 3),
                                                  "GBps": round(algorithmic_bytes(o, k) / (ms / 1e3) / 1e9, 4)}
    finally:
        torch.set_num_threads(previous)
    head = results[f"dequantize_per_call_linear_bf16@{budget}t"]
    return {"value": head["GBps"], "unit": "GB/s", "cores": budget, "kind": "port",
            "sample": f"config 0 q_proj 4096x4096 M=1: the reference's CPU route (restore_planar_w3 + F.linear "
                      f"bf16 per call, product CPU torch code), median of {repeats} after {warmup} warm-ups, "
                      f"{head['median_ms']} ms/call at {budget} threads",
            "host": {"os_cpu_count": os.cpu_count(), "threads_used": budget, "model_name": _cpu_model_name(),
                     "torch_threads_default": previous},
            "arms": results}


def decode_bench(layers=36, prefix=512, steps=32, replays=7, seed=0):
    """Config 3: random-init Qwen3-8B architecture, batch-1 greedy decode of
    ``steps`` tokens after a ``prefix``-token prefill, every step in one hipGraph.

    Four arms on one model: the bf16 model first (HF Linears = hipBLASLt), then
    the same model W3-quantized in place (RTN, fp16 scales, zeros).  For each,
    ``hf``: the reference protocol (StaticDecodeSession over the HF module tree
    with the fused RMSNorm / RoPE modules); ``native``: NativeDecodeSession (our
    kernel chain).  The W3 HF arm is gated against its own dynamic-KV trace
    (prefill via the dense fallback, packed M=1 steps), the W3 native arm against
    the W3 HF arm (same tokens).  Headline: W3 native vs bf16 native tokens/s.
    """
    import statistics

    import torch

    from marlin_style_fluxbin_amd.full_model_trial import compare_trace, decode_trace, validate_routes
    from marlin_style_fluxbin_amd.fused_modules import fused_qwen3_modules
    from marlin_style_fluxbin_amd.native_decode import NativeDecodeSession
    from marlin_style_fluxbin_amd.qwen3 import qwen3_config, random_qwen3_model, w3_quantize_qwen3_model
    from marlin_style_fluxbin_amd.static_decode import StaticDecodeSession, prepared_linears

    device = torch.device("cuda:0")
    config = qwen3_config(num_hidden_layers=layers)
    t0 = time.perf_counter()
    model = random_qwen3_model(config, device=device, dtype=torch.bfloat16, seed=seed)
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, config.vocab_size, (1, prefix), generator=g).to(device)
    print(f"# decode: model built in {time.perf_counter() - t0:.1f}s", file=sys.stderr, flush=True)

    def timed(session):
        for _ in range(DECODE_WARMUP_REPLAYS):  # untimed: clocks settle over the first replays
            session.measure("sequence_graph")
        samples = [session.measure("sequence_graph")[0]["device_ms"] for _ in range(replays)]
        ms = statistics.median(samples)
        return {"tokens_per_s": round(steps / (ms / 1e3), 2), "ms_per_token": round(ms / steps, 4),
                "graph_ms": [round(v, 3) for v in samples],
                "kernels_per_token": None if session.kernel_nodes is None else round(session.kernel_nodes / steps, 1)}

    def arms(name, packed):
        """Timed HF arm (reference protocol: fused modules, default attention),
        timed native arm, and the native arm's parity against an untimed HF run
        with the same arithmetic (stock modules, SDPA math backend; both
        prefills on that backend so the prefix KV match)."""
        from torch.nn.attention import SDPBackend, sdpa_kernel

        t = time.perf_counter()
        with fused_qwen3_modules():
            dynamic = decode_trace(model, ids, steps=steps)
            tokens = dynamic["fed_tokens"].to(device)
            hf = StaticDecodeSession(model, ids, tokens)
            if packed:
                with prepared_linears(model, torch.bfloat16):
                    hf_trace = hf.capture()
                    hf_result = timed(hf)
            else:
                hf_trace = hf.capture()
                hf_result = timed(hf)
        hf.graph = None
        del hf
        torch.cuda.empty_cache()
        with sdpa_kernel([SDPBackend.MATH]):
            ref = StaticDecodeSession(model, ids, tokens)
            if packed:
                with prepared_linears(model, torch.bfloat16):
                    ref_trace = ref.audit()
            else:
                ref_trace = ref.audit()
            del ref
            native = NativeDecodeSession(model, ids, tokens)
        native_trace = native.capture()
        native_result = timed(native)
        native.graph = None
        del native
        torch.cuda.empty_cache()
        vs_ref = compare_trace(native_trace, ref_trace, logprob_tolerance=0.1)
        same = int((native_trace["predictions"] == ref_trace["predictions"]).sum())
        native_result["parity_vs_hf_math_stock"] = {
            "greedy_tokens_equal": f"{same}/{native_trace['predictions'].numel()}",
            "max_abs_logprob_error": round(vs_ref["max_abs_logprob_error"], 5),
            "logits_normalized_rmse": vs_ref["logits"].get("normalized_rmse"),
            "first_step_normalized_rmse": vs_ref["stepwise_normalized_rmse"][1]}
        if packed:
            report = compare_trace(hf_trace, dynamic, logprob_tolerance=0.1)
            hf_result["parity_vs_dynamic_trace"] = {
                "passed": report["passed"], "greedy_tokens_equal": report["greedy_tokens_equal"],
                "max_abs_logprob_error": round(report["max_abs_logprob_error"], 5),
                "logits_normalized_rmse": report["logits"].get("normalized_rmse"),
                "routes_ok": validate_routes(dynamic, expected_linears=7 * layers, steps=steps)}
        print(f"# decode {name}: hf {hf_result} native {native_result} ({time.perf_counter() - t:.1f}s)",
              file=sys.stderr, flush=True)
        return {"hf": hf_result, "native": native_result}

    def noise_floor():
        """Two stock HF runs differing only in SDPA backend (math vs default):
        how far two valid bf16 implementations drift apart at this depth."""
        from torch.nn.attention import SDPBackend, sdpa_kernel

        tokens = torch.randint(0, config.vocab_size, (1, steps), generator=g).to(device)
        default = StaticDecodeSession(model, ids, tokens).audit()
        with sdpa_kernel([SDPBackend.MATH]):
            math = StaticDecodeSession(model, ids, tokens).audit()
        r = compare_trace(default, math, logprob_tolerance=0.1)
        same = int((default["predictions"] == math["predictions"]).sum())
        return {"greedy_tokens_equal": f"{same}/{default['predictions'].numel()}",
                "logits_normalized_rmse": round(r["logits"]["normalized_rmse"], 4),
                "max_abs_logprob_error": round(r["max_abs_logprob_error"], 3)}

    floor = noise_floor()
    print(f"# decode: HF default vs HF math attention (noise floor) {floor}", file=sys.stderr, flush=True)
    prefill = {"bf16": prefill_timing(model, ids)}
    bf16 = arms("bf16", packed=False)
    t = time.perf_counter()
    w3_quantize_qwen3_model(model)
    torch.cuda.empty_cache()
    print(f"# decode: W3 quantization {time.perf_counter() - t:.1f}s", file=sys.stderr, flush=True)
    prefill["w3_dense_fallback"] = prefill_timing(model, ids)
    print(f"# decode: prefill {prefill}", file=sys.stderr, flush=True)
    w3 = arms("w3", packed=True)
    return {"workload": f"config 3: Qwen3-8B arch random init, {layers} layers, prefill {prefix}, "
                        f"{steps} greedy steps in one hipGraph, batch 1",
            "w3": w3, "bf16": bf16, "noise_floor_hf_default_vs_hf_math": floor,
            "prefill": prefill,
            "w3_native_tokens_per_s": w3["native"]["tokens_per_s"],
            "w3_speedup_vs_bf16_native": round(w3["native"]["tokens_per_s"] / bf16["native"]["tokens_per_s"], 3),
            "w3_speedup_vs_bf16_hf": round(w3["hf"]["tokens_per_s"] / bf16["hf"]["tokens_per_s"], 3)}


def prefill_timing(model, ids, reps=3):
    """One prefill forward of the prompt through the HF module tree (packed W3
    Linears take their dense fallback at M > 8: the HIP restore of the weight,
    then a hipBLASLt GEMM): HIP events around the forward, median of ``reps``
    after one untimed run."""
    import statistics

    import torch
    from transformers import StaticCache

    samples = []
    with torch.inference_mode():
        for _ in range(reps + 1):
            cache = StaticCache(config=model.config, max_cache_len=ids.shape[1])
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            model(input_ids=ids, past_key_values=cache, use_cache=True, logits_to_keep=1)
            end.record()
            torch.cuda.synchronize()
            samples.append(start.elapsed_time(end))
            del cache
    ms = statistics.median(samples[1:])
    return {"ms": round(ms, 2), "tokens_per_s": round(ids.shape[1] / (ms / 1e3), 1)}


def decode_hybrid_native(layers=36, prefix=512, steps=32, replays=3, seed=0):
    """Config 3's architecture with the reference's hybrid two-base g128/s8 Linears
    (random payloads of the Qwen3-8B shapes; ``PackedHybridLinear`` everywhere,
    ``fx_hybrid_gemv``) through the native decode chain: tokens/s and kernels per
    token of the two-base full-model route."""
    import statistics

    import torch

    from marlin_style_fluxbin_amd.native_decode import NativeDecodeSession
    from marlin_style_fluxbin_amd.qwen3 import hybrid_qwen3_model, qwen3_config, random_qwen3_model

    device = torch.device("cuda:0")
    config = qwen3_config(num_hidden_layers=layers)
    model = random_qwen3_model(config, device=device, dtype=torch.bfloat16, seed=seed)
    linears = hybrid_qwen3_model(model, seed=seed)
    payload_bytes = sum(t.numel() * t.element_size() for m in model.model.layers
                        for name, t in m.named_buffers() if not name.endswith(("_planar", "_workspace", "lookup")))
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, config.vocab_size, (1, prefix), generator=g).to(device)
    tokens = torch.randint(0, config.vocab_size, (1, steps), generator=g).to(device)
    with torch.inference_mode():
        session = NativeDecodeSession(model, ids, tokens)
        session.capture()
        for _ in range(DECODE_WARMUP_REPLAYS):
            session.measure("sequence_graph")
        samples = [session.measure("sequence_graph")[0]["device_ms"] for _ in range(replays)]
    ms = statistics.median(samples)
    result = {"workload": f"config 3 architecture, hybrid two-base g128/s8 Linears (random payloads), {layers} "
                          f"layers, prefill {prefix}, {steps} steps, native chain",
              "linears": linears, "layer_payload_bytes_per_token": payload_bytes,
              "tokens_per_s": round(steps / (ms / 1e3), 2), "ms_per_token": round(ms / steps, 4),
              "graph_ms": [round(v, 3) for v in samples],
              "kernels_per_token": round(session.kernel_nodes / steps, 1)}
    del session, model
    torch.cuda.empty_cache()
    return result


def decode_desc_act_native(layers=36, prefix=512, steps=32, replays=7, seed=0, desc_act_seed=1):
    """Config 3 on the reference's real payload structure: every Linear's W3
    payload carries a desc_act column permutation (one per input group and layer:
    q|k|v share one, gate|up one, o and down their own; ``qwen3.desc_act_perm``).
    The native chain runs them fused -- each producer writes the next GEMV's
    sorted column order -- at the identity order's launch count; its tokens are
    checked against the HF module tree on the same payloads (stock modules, SDPA
    math, the packed Linears gathering x[perm] themselves)."""
    import statistics

    import torch
    from torch.nn.attention import SDPBackend, sdpa_kernel

    from marlin_style_fluxbin_amd.full_model_trial import compare_trace
    from marlin_style_fluxbin_amd.native_decode import NativeDecodeSession
    from marlin_style_fluxbin_amd.qwen3 import qwen3_config, random_qwen3_model, w3_quantize_qwen3_model
    from marlin_style_fluxbin_amd.static_decode import StaticDecodeSession, prepared_linears

    device = torch.device("cuda:0")
    config = qwen3_config(num_hidden_layers=layers)
    model = random_qwen3_model(config, device=device, dtype=torch.bfloat16, seed=seed)
    w3_quantize_qwen3_model(model, desc_act_seed=desc_act_seed)
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, config.vocab_size, (1, prefix), generator=g).to(device)
    tokens = torch.randint(0, config.vocab_size, (1, steps), generator=g).to(device)
    with sdpa_kernel([SDPBackend.MATH]):
        ref = StaticDecodeSession(model, ids, tokens)
        with prepared_linears(model, torch.bfloat16):
            ref_trace = ref.audit()
        del ref
        session = NativeDecodeSession(model, ids, tokens)
    fused = session.stream is not None
    with torch.inference_mode():
        trace = session.capture()
        for _ in range(DECODE_WARMUP_REPLAYS):
            session.measure("sequence_graph")
        samples = [session.measure("sequence_graph")[0]["device_ms"] for _ in range(replays)]
    ms = statistics.median(samples)
    vs_ref = compare_trace(trace, ref_trace, logprob_tolerance=0.1)
    same = int((trace["predictions"] == ref_trace["predictions"]).sum())
    result = {"workload": f"config 3 W3 native arm on desc_act payloads: {layers} layers, prefill {prefix}, "
                          f"{steps} steps (random fed tokens)",
              "fused_residual_stream": fused,
              "tokens_per_s": round(steps / (ms / 1e3), 2), "ms_per_token": round(ms / steps, 4),
              "graph_ms": [round(v, 3) for v in samples],
              "kernels_per_token": round(session.kernel_nodes / steps, 1),
              "parity_vs_hf_math_stock": {
                  "greedy_tokens_equal": f"{same}/{trace['predictions'].numel()}",
                  "max_abs_logprob_error": round(vs_ref["max_abs_logprob_error"], 5),
                  "logits_normalized_rmse": vs_ref["logits"].get("normalized_rmse"),
                  "first_step_normalized_rmse": vs_ref["stepwise_normalized_rmse"][1]}}
    session.graph = None
    del session, model
    torch.cuda.empty_cache()
    return result


def decode_native_only(layers=36, prefix=512, steps=32, replays=3, seed=0):
    """The config-3 W3 native decode arm alone (no HF arms, no parity audit):
    the workload for a kernel trace of the decode step.  Same model, prefix and
    token protocol as decode_bench; the fed tokens are random instead of a
    greedy trace (the kernels and their shapes are the same)."""
    import statistics

    import torch

    from marlin_style_fluxbin_amd.native_decode import NativeDecodeSession
    from marlin_style_fluxbin_amd.qwen3 import qwen3_config, random_qwen3_model, w3_quantize_qwen3_model

    device = torch.device("cuda:0")
    config = qwen3_config(num_hidden_layers=layers)
    model = random_qwen3_model(config, device=device, dtype=torch.bfloat16, seed=seed)
    w3_quantize_qwen3_model(model)
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, config.vocab_size, (1, prefix), generator=g).to(device)
    tokens = torch.randint(0, config.vocab_size, (1, steps), generator=g).to(device)
    with torch.inference_mode():
        session = NativeDecodeSession(model, ids, tokens)
        head = lm_head_timing(session)  # first, so a kernel trace ends on the graph replays
        session.capture()
        for _ in range(DECODE_WARMUP_REPLAYS):
            session.measure("sequence_graph")
        samples = [session.measure("sequence_graph")[0]["device_ms"] for _ in range(replays)]
    ms = statistics.median(samples)
    return {"workload": f"config 3 W3 native arm: {layers} layers, prefill {prefix}, {steps} steps",
            "tokens_per_s": round(steps / (ms / 1e3), 2), "ms_per_token": round(ms / steps, 4),
            "graph_ms": [round(v, 3) for v in samples],
            "kernels_per_token": round(session.kernel_nodes / steps, 1), "lm_head": head}


def lm_head_timing(session, calls=20, reps=3):
    """The decode step's last launch alone on the session's resident LM-head
    weight: fx_lm_head_argmax (final RMSNorm + head + argmax) against hipBLASLt
    torch.matmul + torch.argmax of the same normalised row; HIP events around
    ``calls`` back-to-back calls on the current stream, best of ``reps``."""
    import torch

    from marlin_style_fluxbin_amd import _lib
    from marlin_style_fluxbin_amd.fused_modules import rms_norm

    weight, lib = session.lm_head, session.lib
    vocab, hidden = weight.shape
    h = session.residual
    logits = torch.empty(vocab, dtype=weight.dtype, device=weight.device)
    pred = torch.empty(1, dtype=torch.int64, device=weight.device)
    ws = torch.zeros(lib.fx_lm_head_argmax_workspace_bytes(), dtype=torch.uint8, device=weight.device)
    normed = rms_norm(h, session.final_norm, session.eps)
    out = torch.empty(1, vocab, dtype=weight.dtype, device=weight.device)
    p2 = torch.empty(1, 1, dtype=torch.int64, device=weight.device)
    stream = _lib.stream_handle(weight.device)

    def fused():
        _lib.check(lib.fx_lm_head_argmax(h.data_ptr(), session.final_norm.data_ptr(), session.eps, weight.data_ptr(),
                                         logits.data_ptr(), pred.data_ptr(), ws.data_ptr(), ws.numel(), vocab,
                                         hidden, _lib.dtype_code(weight.dtype), stream), "fx_lm_head_argmax")

    def library():
        torch.matmul(normed, weight.t(), out=out)
        torch.argmax(out, dim=-1, keepdim=True, out=p2)

    result = {"shape": [vocab, hidden], "bytes": vocab * hidden * weight.element_size()}
    for name, fn in (("fused_us", fused), ("hipblaslt_argmax_us", library)):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        best = float("inf")
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(calls):
                fn()
            b.record()
            torch.cuda.synchronize()
            best = min(best, a.elapsed_time(b) * 1e3 / calls)
        result[name] = round(best, 1)
    result["fused_tb_per_s"] = round(result["bytes"] / (result["fused_us"] * 1e-6) / 1e12, 2)
    if int(pred.item()) != int(torch.argmax(logits).item()):
        raise RuntimeError("fx_lm_head_argmax prediction disagrees with its own logits")
    return result


def pmc_target():
    """Workload for ``rocprofv3 --pmc`` passes: the gate/up W3 GEMV (default plan)
    over 24 rotating payloads, twice; the LUT kernel (reference-style tables in
    LDS) at the same shape, 8 launches; the two-base GEMVs at the same shape (the
    rank-one kernel over 24 payloads twice, the hybrid kernel 8 launches); and
    torch's copy kernel over 16 distinct 20 MiB float32 buffers, whose FETCH_SIZE /
    WRITE_SIZE readings calibrate the counters to bytes."""
    import torch

    from marlin_style_fluxbin_amd import W3Gemv
    from marlin_style_fluxbin_amd.w3_lut_deployment import inline_main, workspace_shape

    device = torch.device("cuda:0")
    gen = torch.Generator(device=device).manual_seed(0)
    o, k = UNIQUE["gate/up"]
    payloads = [make_payload(o, k, device, gen) for _ in range(24)]
    gemvs = [W3Gemv(p, perm_identity=True) for p in payloads]
    x = torch.randn(1, k, device=device, generator=gen).to(torch.bfloat16)
    out = torch.empty(1, o, device=device, dtype=torch.bfloat16)
    for _ in range(2):
        for gemv in gemvs:
            gemv(x, out)
    # the same payloads in the field layout, 24 launches twice
    from marlin_style_fluxbin_amd import _lib

    lib = _lib.library()
    fields = [torch.empty_like(p["planes"]) for p in payloads]
    for p, f in zip(payloads, fields):
        _lib.check(lib.fx_w3_planes_to_fields(p["planes"].data_ptr(), f.data_ptr(), o, k,
                                              _lib.stream_handle(device)), "fx_w3_planes_to_fields")
    for _ in range(2):
        for p, f in zip(payloads, fields):
            _lib.check(lib.fx_w3_gemv_fields(x.data_ptr(), _lib.dtype_code(x.dtype), f.data_ptr(),
                                             p["scales"].data_ptr(), _lib.dtype_code(p["scales"].dtype),
                                             p["zeros"].data_ptr(), out.data_ptr(), o, k,
                                             _lib.stream_handle(device)), "fx_w3_gemv_fields")
    del fields
    partial = torch.empty(workspace_shape(o, k), dtype=torch.float32, device=device)
    for p in payloads[:8]:
        inline_main(x, p, partial, row_tile=256)
    del gemvs, payloads
    # the two-base GEMVs at the same shape: config 4's rank-one kernel, 24 rotating
    # payloads twice, and the hybrid (reference layout) kernel, 8 payloads
    from marlin_style_fluxbin_amd import deployment
    from marlin_style_fluxbin_amd.two_base import TwoBaseGemv, pack_rank_one_planes

    g = k // 128
    rank_one = []
    for _ in range(24):
        bases = torch.randint(0, 2, (2, o, k), device=device, generator=gen, dtype=torch.int8) * 2 - 1
        rank_one.append(TwoBaseGemv({
            "planes": pack_rank_one_planes(bases),
            "coef": (torch.rand(2, o, device=device, generator=gen) + 0.5).half(),
            "srow": (torch.rand(o, device=device, generator=gen) * 0.015 + 0.005).half(),
            "tcol": (torch.rand(k, device=device, generator=gen) * 0.4 + 0.8).half(),
            "salient": (torch.randn(o, 32, device=device, generator=gen) * 0.05).bfloat16(),
            "salient_idx": torch.randperm(k, device=device, generator=gen)[:32].sort().values.int()}))
    for _ in range(2):
        for gemv in rank_one:
            gemv(x, out)
    del rank_one
    ws = torch.empty(deployment.workspace_shape(o, k), device=device)
    for _ in range(8):
        layout = {"codes": torch.randint(0, 256, (g, o, 2, 16), dtype=torch.uint8, device=device, generator=gen),
                  "rows": torch.randn(g, o, 2, device=device, generator=gen) * 0.1,
                  "columns": torch.randn(g, 128, 2, device=device, generator=gen),
                  "indices": torch.arange(8, dtype=torch.int16, device=device).repeat(g, 1) * 16,
                  "sparse_codes": torch.randint(0, 256, (g, o, 2, 1), dtype=torch.uint8, device=device,
                                                generator=gen),
                  "sparse_rows": torch.randn(g, o, 2, device=device, generator=gen) * 0.07,
                  "sparse_columns": torch.randn(g, 8, 2, device=device, generator=gen)}
        deployment.m1_out(x, layout, out, ws, kernel="v5_p1024")
    src = [torch.empty(CALIBRATION_BYTES // 4, device=device) for _ in range(16)]
    dst = [torch.empty_like(t) for t in src]
    for a, b in zip(src, dst):
        b.copy_(a)
    torch.cuda.synchronize()
    print("pmc target done", flush=True)


CALIBRATION_BYTES = 20 * 1024 * 1024


def summarize_trace(csv_path, last):
    """Per-kernel duration summary of the last ``last`` dispatches (by start time)
    of a rocprofv3 kernel-trace CSV: the span they cover, the sum of their
    durations, and per (kernel, grid) count / total / mean / median in us."""
    import csv
    import statistics
    from collections import defaultdict

    rows = []
    with open(csv_path, newline="") as f:
        for r in csv.DictReader(f):
            # the full grid: a strided-batch launch shares a kernel and grid x with
            # its single-GEMV form and walks its payloads on grid y
            grid = r.get("Grid_Size_X", "")
            if r.get("Grid_Size_Y", "1") not in ("", "1") or r.get("Grid_Size_Z", "1") not in ("", "1"):
                grid = f"{grid} x {r.get('Grid_Size_Y', '1')} x {r.get('Grid_Size_Z', '1')}"
            rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"], grid))
    rows.sort()
    tail = rows[-last:]
    groups = defaultdict(list)
    for start, end, name, grid in tail:
        groups[(name.split("(")[0], grid)].append((end - start) / 1000.0)
    span = (tail[-1][1] - tail[0][0]) / 1000.0
    busy = sum(sum(v) for v in groups.values())
    print(f"last {len(tail)} dispatches: span {span:.1f} us, kernel time {busy:.1f} us ({100 * busy / span:.1f}%)")
    print("| kernel | grid (threads; x, or x x y x z) | dispatches | total us | mean us | median us |")
    print("|---|---:|---:|---:|---:|---:|")
    for (name, grid), v in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
        print(f"| `{name}` | {grid} | {len(v)} | {sum(v):.1f} | {statistics.mean(v):.2f} | {statistics.median(v):.2f} |")


def pmc_hybrid_target(copies=4, reps=8):
    """Workload for ``rocprofv3 --pmc`` passes over the hybrid decode launches:
    one Qwen3-8B layer's hybrid two-base Linears (random payloads, ``copies``
    rotating copies) run as the native decode chain runs them -- q|k|v and gate|up
    normalising the residual, o adding into it, down forming the SwiGLU and adding
    into it -- ``reps`` times each, with a progress line per round."""
    import torch

    from marlin_style_fluxbin_amd.deployment import HybridSegmentsGemv, PackedHybridLinear
    from marlin_style_fluxbin_amd.qwen3 import random_hybrid_payload

    device = torch.device("cuda:0")
    gen = torch.Generator(device=device).manual_seed(0)
    hidden, inter, kv = 4096, 12288, 1024

    def module(o, k):
        return PackedHybridLinear(random_hybrid_payload(o, k, device=device, generator=gen), kernel="v5_p1024",
                                  groups_per_split=8).to(device)

    layers = []
    for _ in range(copies):
        layers.append({"qkv": HybridSegmentsGemv([module(hidden, hidden), module(kv, hidden), module(kv, hidden)]),
                       "o": HybridSegmentsGemv([module(hidden, hidden)]),
                       "gate_up": HybridSegmentsGemv([module(inter, hidden), module(inter, hidden)]),
                       "down": HybridSegmentsGemv([module(hidden, inter)])})
    residual = torch.randn(1, hidden, device=device, generator=gen).to(torch.bfloat16)
    sums = torch.rand(hidden // 16, device=device, generator=gen) * 16
    weight = (1 + 0.02 * torch.randn(hidden, device=device, generator=gen)).to(torch.bfloat16)
    qkv_out = torch.empty(1, hidden + 2 * kv, dtype=torch.bfloat16, device=device)
    attn = torch.randn(1, hidden, device=device, generator=gen).to(torch.bfloat16)
    gate_up = torch.empty(1, 2 * inter, dtype=torch.bfloat16, device=device)
    for r in range(reps):
        for layer in layers:
            layer["qkv"].rmsnormed(residual, sums, weight, 1e-6, qkv_out)
            layer["o"].residual(attn, residual, sums)
            layer["gate_up"].rmsnormed(residual, sums, weight, 1e-6, gate_up)
            layer["down"].residual(gate_up, residual, sums, swiglu=True)
        torch.cuda.synchronize()
        print(f"# pmc-hybrid round {r + 1}/{reps}", flush=True)


def summarize_sq(csv_path, name_filter):
    """Per-kernel (and grid) SQ instruction mix from a rocprofv3 counter CSV:
    waves, cycles, VALU / MFMA / LDS / VMEM instructions per wave and LDS bank
    conflicts per active LDS cycle, for kernels whose name contains name_filter."""
    import csv
    from collections import defaultdict

    vals = defaultdict(lambda: defaultdict(list))
    with open(csv_path, newline="") as f:
        for row in csv.DictReader(f):
            name = row["Kernel_Name"].split("(")[0]
            if name_filter not in name:
                continue
            key = (name, row.get("Grid_Size") or row.get("Grid_Size_X", ""))
            vals[key][row["Counter_Name"]].append(float(row["Counter_Value"]))
    print("| kernel | grid | waves | cycles / wave | VALU / wave | MFMA / wave | LDS / wave | VMEM / wave | "
          "bank conflicts / active LDS |")
    print("|---|---:|---:|---:|---:|---:|---:|---:|---:|")
    for (name, grid), d in sorted(vals.items()):
        m = {c: sum(v) / len(v) for c, v in d.items()}
        w = max(m.get("SQ_WAVES", 1.0), 1.0)
        conflicts = m.get("SQ_LDS_BANK_CONFLICT", 0.0) / max(m.get("SQ_ACTIVE_INST_LDS", 1.0), 1.0)
        print(f"| `{name}` | {grid} | {w:.0f} | {m.get('SQ_WAVE_CYCLES', 0) / w:.0f} | "
              f"{m.get('SQ_INSTS_VALU', 0) / w:.1f} | {m.get('SQ_INSTS_MFMA', 0) / w:.1f} | "
              f"{m.get('SQ_INSTS_LDS', 0) / w:.1f} | {m.get('SQ_INSTS_VMEM', 0) / w:.1f} | {conflicts:.2f} |")


def summarize_counters(csv_paths, name_filter):
    """Every counter of one or more rocprofv3 counter CSVs, averaged per dispatch
    for each (kernel, grid) whose name contains name_filter; per wave too where
    the CSV holds SQ_WAVES.  FETCH_SIZE / WRITE_SIZE are KiB per dispatch, unscaled."""
    import csv
    from collections import defaultdict

    vals = defaultdict(lambda: defaultdict(list))
    for path in csv_paths:
        with open(path, newline="") as f:
            for row in csv.DictReader(f):
                name = row["Kernel_Name"].split("(")[0]
                if name_filter in name:
                    key = (name, row.get("Grid_Size") or row.get("Grid_Size_X", ""))
                    vals[key][row["Counter_Name"]].append(float(row["Counter_Value"]))
    for (name, grid), d in sorted(vals.items()):
        m = {c: sum(v) / len(v) for c, v in d.items()}
        waves = m.get("SQ_WAVES")
        print(f"`{name}` grid {grid}, {max(len(v) for v in d.values())} dispatches")
        print("| counter | mean per dispatch | per wave |")
        print("|---|---:|---:|")
        for c in sorted(m):
            per_wave = f"{m[c] / waves:.1f}" if waves and c.startswith("SQ_") and c != "SQ_WAVES" else ""
            print(f"| {c} | {m[c]:.1f} | {per_wave} |")


def pmc_small_m_target(shape, copies=24):
    """Workload for ``rocprofv3`` passes over the small-M GEMV (config 1): the
    planar ``fx_w3_gemv`` at one Qwen3-8B shape for M = 1, 2, 4, 8 (the default
    plans), then the field layout's ``fx_w3_gemv_fields_rows`` for M = 2, 4, 8 on
    the same payloads, ``copies`` rotating payloads each, a progress line per M."""
    import torch

    from marlin_style_fluxbin_amd import _lib

    lib = _lib.library()
    device = torch.device("cuda:0")
    o, k = UNIQUE[shape]
    gen = torch.Generator(device=device).manual_seed(o + k)
    stacked, payloads = make_payloads(o, k, device, gen, copies)
    ws = torch.zeros(lib.fx_w3_gemv_workspace_bytes(8, o, k) + 256, dtype=torch.uint8, device=device)
    for m in (1, 2, 4, 8):
        x = torch.randn(m, k, device=device, generator=gen).to(torch.bfloat16)
        out = torch.empty(m, o, device=device, dtype=torch.bfloat16)
        torch.cuda.synchronize()
        for p in range(copies):
            _lib.check(lib.fx_w3_gemv(x.data_ptr(), _lib.FX_BF16, payloads[p]["planes"].data_ptr(),
                                      payloads[p]["scales"].data_ptr(), _lib.FX_F16, payloads[p]["zeros"].data_ptr(),
                                      None, ws.data_ptr(), ws.numel(), out.data_ptr(), m, o, k, _lib.ARITH_STRUCTURAL,
                                      _lib.stream_handle(device)), "fx_w3_gemv")
        torch.cuda.synchronize()
        print(f"# pmc-small-m {shape} M = {m} done", flush=True)
    fields = torch.empty_like(stacked["planes"])
    for p in range(copies):
        _lib.check(lib.fx_w3_planes_to_fields(stacked["planes"][p].data_ptr(), fields[p].data_ptr(), o, k,
                                              _lib.stream_handle(device)), "fx_w3_planes_to_fields")
    for m in (2, 4, 8):
        x = torch.randn(m, k, device=device, generator=gen).to(torch.bfloat16)
        out = torch.empty(m, o, device=device, dtype=torch.bfloat16)
        torch.cuda.synchronize()
        for p in range(copies):
            _lib.check(lib.fx_w3_gemv_fields_rows(x.data_ptr(), _lib.FX_BF16, fields[p].data_ptr(),
                                                  payloads[p]["scales"].data_ptr(), _lib.FX_F16,
                                                  payloads[p]["zeros"].data_ptr(), out.data_ptr(), m, o, k,
                                                  _lib.stream_handle(device)), "fx_w3_gemv_fields_rows")
        torch.cuda.synchronize()
        print(f"# pmc-small-m {shape} field rows M = {m} done", flush=True)


def pmc_attention_target(layers=36, position=543, rounds=8):
    """Workload for ``rocprofv3 --pmc`` passes over the decode attention: Qwen3-8B
    heads (32 query / 8 KV heads of 128), the native decode's call
    (``fx_decode_attention_rope``: q/k norm, RoPE and the cache write folded in;
    its combine launch), over ``layers`` distinct 544-slot KV caches (as the decode
    graph walks them) at ``position``, ``rounds`` times, a progress line per round."""
    import math

    import torch

    from marlin_style_fluxbin_amd import _lib

    device = torch.device("cuda:0")
    gen = torch.Generator(device=device).manual_seed(0)
    hq, hk, d, lmax = 32, 8, 128, position + 1
    lib = _lib.library()
    bf = torch.bfloat16
    kc = [torch.randn(hk, lmax, d, device=device, generator=gen).to(bf) for _ in range(layers)]
    vc = [torch.randn(hk, lmax, d, device=device, generator=gen).to(bf) for _ in range(layers)]
    qkv = torch.randn(hq * d + 2 * hk * d, device=device, generator=gen).to(bf)
    q, k, v = qkv[:hq * d], qkv[hq * d:(hq + hk) * d], qkv[(hq + hk) * d:]
    w = (1 + 0.02 * torch.randn(2, d, device=device, generator=gen)).to(bf)
    cos = torch.randn(d, device=device, generator=gen).to(bf)
    sin = torch.randn(d, device=device, generator=gen).to(bf)
    nbytes = lib.fx_decode_attention_workspace_bytes(hq, lmax, d)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
    out = torch.empty(hq * d, dtype=bf, device=device)
    for r in range(rounds):
        for kl, vl in zip(kc, vc):
            _lib.check(lib.fx_decode_attention_rope(
                q.data_ptr(), k.data_ptr(), v.data_ptr(), w[0].data_ptr(), w[1].data_ptr(), cos.data_ptr(),
                sin.data_ptr(), 1e-6, _lib.ROPE_STOCK, kl.data_ptr(), vl.data_ptr(), ws.data_ptr(), nbytes, None,
                out.data_ptr(), hq, hk, lmax, d, position, 1 / math.sqrt(d), _lib.FX_BF16,
                _lib.stream_handle(device)), "fx_decode_attention_rope")
        torch.cuda.synchronize()
        print(f"# pmc-attention round {r + 1}/{rounds}", flush=True)


def attention_sweep(layers=36, positions=(512, 543), lmax=1024):
    """µs per call of the decode attention (``fx_decode_attention_rope``, Qwen3-8B
    heads, split + combine launches) under every (keys per thread, head groups)
    plan (``fx_decode_attention_plan``), graph-timed over ``layers`` distinct
    caches as the decode walks them, paired protocol; outputs checked bit-equal
    across head groups (the per-head arithmetic does not depend on the group)."""
    import math

    import torch

    from marlin_style_fluxbin_amd import _lib

    device = torch.device("cuda:0")
    stream = torch.cuda.Stream(device)
    gen = torch.Generator(device=device).manual_seed(0)
    hq, hk, d = 32, 8, 128
    lib = _lib.library()
    bf = torch.bfloat16
    with torch.cuda.stream(stream):
        kc = [torch.randn(hk, lmax, d, device=device, generator=gen).to(bf) for _ in range(layers)]
        vc = [torch.randn(hk, lmax, d, device=device, generator=gen).to(bf) for _ in range(layers)]
        qkv = torch.randn(hq * d + 2 * hk * d, device=device, generator=gen).to(bf)
        w = (1 + 0.02 * torch.randn(2, d, device=device, generator=gen)).to(bf)
        cos = torch.randn(d, device=device, generator=gen).to(bf)
        sin = torch.randn(d, device=device, generator=gen).to(bf)
        nbytes = lib.fx_decode_attention_workspace_bytes(hq, lmax, d)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
        outs = torch.empty(layers, hq * d, dtype=bf, device=device)
    torch.cuda.synchronize()
    q, k, v = qkv[:hq * d], qkv[hq * d:(hq + hk) * d], qkv[(hq + hk) * d:]
    result = {}
    for pos in positions:
        def run(pos=pos):
            for layer in range(layers):
                _lib.check(lib.fx_decode_attention_rope(
                    q.data_ptr(), k.data_ptr(), v.data_ptr(), w[0].data_ptr(), w[1].data_ptr(), cos.data_ptr(),
                    sin.data_ptr(), 1e-6, _lib.ROPE_STOCK, kc[layer].data_ptr(), vc[layer].data_ptr(),
                    ws.data_ptr(), nbytes, None, outs[layer].data_ptr(), hq, hk, lmax, d, pos, 1 / math.sqrt(d),
                    _lib.FX_BF16, _lib.stream_handle(device)), "fx_decode_attention_rope")

        graphs, first, equal = {}, {}, True
        for kpt in (1, 2, 4):
            for groups in (1, 2, 4):
                _lib.check(lib.fx_decode_attention_plan(kpt, groups), "attention plan")
                try:
                    with torch.cuda.stream(stream):
                        run()
                    torch.cuda.synchronize()
                    got = outs.clone()
                    graphs[f"kpt{kpt}/g{groups}"] = (capture(run, stream), layers)
                finally:
                    _lib.check(lib.fx_decode_attention_plan(0, 0), "attention plan reset")
                if kpt in first:
                    equal = equal and torch.equal(got, first[kpt])
                else:
                    first[kpt] = got
        timing = paired_graph_timing(graphs, stream, repeats=5)
        result[f"pos {pos}"] = {"us": {n: round(t["us"], 3) for n, t in timing.items()}, "groups_bit_equal": equal}
        print(f"# attention sweep pos {pos}: {result[f'pos {pos}']}", file=sys.stderr, flush=True)
        del graphs
    return result


def summarize_pmc(csv_paths, out_json):
    """Average rocprofv3 counter CSVs per kernel; scale FETCH_SIZE / WRITE_SIZE
    (KiB per dispatch) by what they read for the copy kernel of known size."""
    import csv
    from collections import defaultdict

    values = defaultdict(lambda: defaultdict(list))
    for path in csv_paths:
        with open(path, newline="") as f:
            for row in csv.DictReader(f):
                values[row["Kernel_Name"]][row["Counter_Name"]].append(float(row["Counter_Value"]))
    mean = {k: {c: sum(v) / len(v) for c, v in d.items()} for k, d in values.items()}
    # the 16 copies of 20 MiB run as the runtime's buffer-copy kernel; smaller copies
    # elsewhere in the workload share its name, so calibrate on the 16 largest
    for k, d in values.items():
        if "copyBuffer" in k:
            mean[k] = {c: sum(sorted(v)[-16:]) / len(sorted(v)[-16:]) for c, v in d.items()}
    copy = [k for k in mean if "copyBuffer" in k and "FETCH_SIZE" in mean[k]]
    # the planar kernel and the field-layout one: FIELDS is the tenth template
    # argument of w3_mfma_kernel
    def fields_arg(name):
        head = name.split("(")[0]
        args = head[head.index("<") + 1:head.rindex(">")].split(",")
        return len(args) > 9 and args[9].strip() == "true"

    w3 = [k for k in mean if "w3_mfma_kernel" in k and not fields_arg(k)]
    w3_fields = [k for k in mean if "w3_mfma_kernel" in k and fields_arg(k)]
    if not copy or not w3:
        raise SystemExit("counter CSVs lack the copy kernel or the W3 kernel")
    kib = CALIBRATION_BYTES / 1024
    fetch_scale = kib / mean[copy[0]]["FETCH_SIZE"]
    write_scale = kib / mean[copy[0]]["WRITE_SIZE"] if mean[copy[0]].get("WRITE_SIZE") else None
    kernel = w3[0]
    fetch = mean[kernel]["FETCH_SIZE"] * fetch_scale * 1024
    write = mean[kernel].get("WRITE_SIZE", 0.0) * (write_scale or 1.0) * 1024
    o, k = UNIQUE["gate/up"]
    summary = {
        "kernel": kernel.split("(")[0],
        "workload": "gate/up 12288x4096 M=1, fp16 scales, uint8 zeros, identity perm",
        "fetch_kib_raw": round(mean[kernel]["FETCH_SIZE"], 1),
        "write_kib_raw": round(mean[kernel].get("WRITE_SIZE", 0.0), 1),
        "fetch_scale": round(fetch_scale, 4),
        "write_scale": None if write_scale is None else round(write_scale, 4),
        "traffic_bytes": int(round(fetch + write)),
        "algorithmic_bytes": algorithmic_bytes(o, k),
        "counters": {k.split("(")[0]: {c: round(v, 1) for c, v in d.items()} for k, d in mean.items()
                     if "w3_" in k or "copyBuffer" in k or "rank_one" in k or "hybrid" in k},
    }
    if w3_fields and "FETCH_SIZE" in mean[w3_fields[0]]:
        m = mean[w3_fields[0]]
        summary["field_layout"] = {
            "kernel": w3_fields[0].split("(")[0],
            "fetch_kib_raw": round(m["FETCH_SIZE"], 1),
            "write_kib_raw": round(m.get("WRITE_SIZE", 0.0), 1),
            "traffic_bytes": int(round(m["FETCH_SIZE"] * fetch_scale * 1024
                                       + m.get("WRITE_SIZE", 0.0) * (write_scale or 1.0) * 1024)),
            "algorithmic_bytes": algorithmic_bytes(o, k)}
    g = k // 128
    two_base_bytes = {"rank_one_kernel": 2 * o * k // 8 + 6 * o + 2 * k + 64 * o + 128 + 2 * k + 2 * o,
                      "hybrid_kernel": 32 * g * o + 8 * g * o + 1024 * g + 16 * g + 2 * g * o + 8 * g * o
                                       + 64 * g + 2 * k + 2 * o}
    for name, nbytes in two_base_bytes.items():
        hit = [kk for kk in mean if name in kk and "FETCH_SIZE" in mean[kk]]
        if hit:
            m = mean[hit[0]]
            summary.setdefault("two_base", {})[name] = {
                "fetch_kib_raw": round(m["FETCH_SIZE"], 1),
                "write_kib_raw": round(m.get("WRITE_SIZE", 0.0), 1),
                "traffic_bytes": int(round(m["FETCH_SIZE"] * fetch_scale * 1024
                                           + m.get("WRITE_SIZE", 0.0) * (write_scale or 1.0) * 1024)),
                "algorithmic_bytes": nbytes}
    Path(out_json).write_text(json.dumps(summary, indent=1) + "\n")
    print(json.dumps(summary, indent=1))


def main():
    parser = argparse.ArgumentParser()
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--layers", type=int, default=8)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--shapes", default="all", help="comma list of q/o,k/v,gate/up,down or all")
    parser.add_argument("--pmc-target", action="store_true", help="run the counter-collection workload")
    parser.add_argument("--pmc-hybrid", action="store_true",
                        help="run the counter-collection workload of the hybrid decode launches")
    parser.add_argument("--summarize-sq", nargs=2, metavar=("CSV", "NAME"),
                        help="per-kernel SQ instruction mix of a counter CSV (kernels matching NAME)")
    parser.add_argument("--decode", action="store_true", help="run only the config-3 decode benchmark")
    parser.add_argument("--decode-native", action="store_true",
                        help="run only the config-3 W3 native decode arm (the kernel-trace workload)")
    parser.add_argument("--decode-hybrid", action="store_true",
                        help="run only the config-3 architecture with hybrid two-base Linears, native chain")
    parser.add_argument("--decode-desc-act", action="store_true",
                        help="run only the config-3 W3 native arm on desc_act (column-permuted) payloads")
    parser.add_argument("--decode-layers", type=int, default=36)
    parser.add_argument("--no-decode", action="store_true", help="skip the config-3 decode benchmark")
    parser.add_argument("--no-two-base", action="store_true", help="skip the config-4 two-base benchmark")
    parser.add_argument("--no-fused-ops", action="store_true", help="skip the config-2 fused-ops benchmark")
    parser.add_argument("--fused-ops", action="store_true", help="run only the config-2 fused-ops benchmark")
    parser.add_argument("--summarize-pmc", nargs="+", metavar="CSV",
                        help="rocprofv3 counter CSVs -> profiles/w3_mfma_traffic.json")
    parser.add_argument("--pmc-attention", action="store_true",
                        help="run the counter-collection workload of the decode attention")
    parser.add_argument("--summarize-counters", nargs="+", metavar="ARG",
                        help="NAME CSV [CSV ...]: every counter per dispatch of kernels matching NAME")
    parser.add_argument("--pmc-small-m", metavar="SHAPE",
                        help="run the small-M counter workload at one shape (q/o, k/v, gate/up or down)")
    parser.add_argument("--sweep-attention", action="store_true",
                        help="time every attention plan (keys per thread x head groups) at 513 and 544 keys")
    parser.add_argument("--sweep-fields", nargs="?", const="all", default=None, metavar="NAMES",
                        help="time every field-layout plan at the Qwen3-8B shapes (one JSON line); "
                             "optional comma list of shape names")
    parser.add_argument("--sweep-rows", nargs="?", const="all", default=None, metavar="NAMES",
                        help="time M = 2, 4, 8 rows on the field layout (every plan) against the planar "
                             "kernel at the Qwen3-8B shapes (one JSON line); optional comma list of shapes")
    parser.add_argument("--summarize-trace", nargs=2, metavar=("CSV", "LAST"),
                        help="per-kernel summary of the last LAST dispatches of a kernel-trace CSV")
    args = parser.parse_args()
    if args.summarize_pmc:
        summarize_pmc(args.summarize_pmc, ROOT / "profiles" / "w3_mfma_traffic.json")
        return
    if args.summarize_trace:
        summarize_trace(args.summarize_trace[0], int(args.summarize_trace[1]))
        return
    if args.pmc_target:
        pmc_target()
        return
    if args.pmc_hybrid:
        pmc_hybrid_target()
        return
    if args.pmc_attention:
        pmc_attention_target()
        return
    if args.pmc_small_m:
        pmc_small_m_target(args.pmc_small_m)
        return
    if args.summarize_counters:
        summarize_counters(args.summarize_counters[1:], args.summarize_counters[0])
        return
    if args.summarize_sq:
        summarize_sq(args.summarize_sq[0], args.summarize_sq[1])
        return
    if args.decode_native:
        print(json.dumps(decode_native_only(layers=args.decode_layers)), flush=True)
        return
    if args.decode_hybrid:
        print(json.dumps(decode_hybrid_native(layers=args.decode_layers)), flush=True)
        return
    if args.decode_desc_act:
        print(json.dumps(decode_desc_act_native(layers=args.decode_layers)), flush=True)
        return
    if args.decode:
        print(json.dumps(decode_bench(layers=args.decode_layers)), flush=True)
        return
    if args.sweep_attention:
        print(json.dumps(attention_sweep()), flush=True)
        return
    if args.sweep_fields:
        import torch

        device = torch.device("cuda:0")
        names = list(SWEEP_SHAPES) if args.sweep_fields == "all" else args.sweep_fields.split(",")
        print(json.dumps(fields_plan_sweep(device, torch.cuda.Stream(device),
                                           {n: SWEEP_SHAPES[n] for n in names})), flush=True)
        return
    if args.sweep_rows:
        import torch

        device = torch.device("cuda:0")
        names = list(ROWS_SHAPES) if args.sweep_rows == "all" else args.sweep_rows.split(",")
        print(json.dumps(rows_sweep(device, torch.cuda.Stream(device), {n: ROWS_SHAPES[n] for n in names})),
              flush=True)
        return
    if args.fused_ops:
        import torch

        device = torch.device("cuda:0")
        print(json.dumps(fused_ops_bench(device, args.steps, args.warmup, torch.cuda.Stream(device))), flush=True)
        return
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(each box has one MI355X); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    from marlin_style_fluxbin_amd import W3Gemv
    from marlin_style_fluxbin_amd._lib import library

    library()
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    stream = torch.cuda.Stream(device)

    # --- per-shape GEMV vs bf16 arm ---------------------------------------------------
    wanted = list(UNIQUE) if args.shapes == "all" else args.shapes.split(",")
    shapes = {}
    for name in wanted:
        o, k = UNIQUE[name]
        shapes[name] = bench_shape(o, k, device, max(args.steps, 10), args.warmup, stream)
        print(f"# {name}: {shapes[name]}", file=sys.stderr, flush=True)

    # --- the step: 7 GEMVs x LAYERS distinct layers, one graph ------------------------
    gen = torch.Generator(device=device).manual_seed(0)
    layers = []
    for _ in range(args.layers):
        layer = {}
        for name, (o, k) in SHAPES.items():
            layer[name] = W3Gemv(make_payload(o, k, device, gen), perm_identity=True)
        layers.append(layer)
    xs = {4096: torch.randn(1, 4096, device=device, generator=gen).to(torch.bfloat16),
          12288: torch.randn(1, 12288, device=device, generator=gen).to(torch.bfloat16)}
    outs = {name: torch.empty(1, o, device=device, dtype=torch.bfloat16) for name, (o, k) in SHAPES.items()}

    def step():
        for layer in layers:
            for name, (o, k) in SHAPES.items():
                layer[name](xs[k], outs[name])

    graph = capture(step, stream)
    torch.cuda.synchronize()
    ms = time_graph(graph, args.steps, args.warmup, stream)
    step_bytes = args.layers * sum(algorithmic_bytes(o, k) for o, k in SHAPES.values())
    value = step_bytes / (ms / 1e3) / 1e9

    # the same step on the field layout (the payloads repacked once, as the
    # native decode session does): fx_w3_gemv_fields per GEMV
    from marlin_style_fluxbin_amd import _lib

    lib = _lib.library()
    field_calls = []
    for layer in layers:
        for name, (o, k) in SHAPES.items():
            lay = layer[name].layout
            f = torch.empty_like(lay["planes"])
            _lib.check(lib.fx_w3_planes_to_fields(lay["planes"].data_ptr(), f.data_ptr(), o, k,
                                                  _lib.stream_handle(device)), "fx_w3_planes_to_fields")
            field_calls.append((xs[k], f, lay, outs[name], o, k))

    def field_step():
        for x, f, lay, out, o, k in field_calls:
            _lib.check(lib.fx_w3_gemv_fields(x.data_ptr(), _lib.dtype_code(x.dtype), f.data_ptr(),
                                             lay["scales"].data_ptr(), _lib.dtype_code(lay["scales"].dtype),
                                             lay["zeros"].data_ptr(), out.data_ptr(), o, k,
                                             _lib.stream_handle(device)), "fx_w3_gemv_fields")

    fgraph = capture(field_step, stream)
    fms = time_graph(fgraph, args.steps, args.warmup, stream)
    field_value = step_bytes / (fms / 1e3) / 1e9
    del fgraph, field_calls

    dominant = shapes.get("gate/up") or next(iter(shapes.values()))
    traffic = None
    traffic_file = ROOT / "profiles" / "w3_mfma_traffic.json"
    if traffic_file.exists() and "gate/up" in shapes:
        traffic = json.loads(traffic_file.read_text()).get("traffic_bytes")
    result = {
        "metric": "W3 GEMV HBM GB/s (% of peak) per Qwen3-8B shape; batch-1 decode tokens/sec",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random W3 codes, fp16 scales U[0.005,0.02], zeros U{3,4}, bf16 x ~ N(0,1))",
        "config": {
            "workload": f"config 1: 7 Qwen3-8B Linear shapes at M=1 x {args.layers} distinct layers per step",
            "frac_hbm_peak": round(value / HBM_PEAK_GBPS, 4),
            "shapes": shapes,
            "field_layout": {
                "note": "the same payloads repacked once by fx_w3_planes_to_fields (same bytes); "
                        "value and roofline above are the planar payload, the reference's layout",
                "step_GBps": round(field_value, 1), "ms_per_step": round(fms, 4),
                "frac_hbm_peak": round(field_value / HBM_PEAK_GBPS, 4),
                "gate_up_us": dominant_fields_us(shapes), "gate_up_frac_hbm": dominant_fields_frac(shapes),
            },
        },
        "roofline": {
            "bound": "hbm",
            "achieved": dominant["w3_GBps"],
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": dominant["w3_frac_hbm"],
            "traffic": traffic,
            "algorithmic_bytes": dominant["algorithmic_bytes"],
            "kernel": f"w3_mfma_kernel at gate/up {dominant['O']}x{dominant['K']}, M=1 "
                      f"(average launch over {dominant['copies']} rotating payloads)",
        },
    }
    field_traffic = None
    if traffic_file.exists() and "gate/up" in shapes:
        field_traffic = json.loads(traffic_file.read_text()).get("field_layout", {}).get("traffic_bytes")
    if dominant.get("fields_GBps") is not None:
        result["roofline_field_layout"] = {
            "bound": "hbm",
            "achieved": dominant["fields_GBps"],
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": dominant["fields_frac_hbm"],
            "traffic": field_traffic,
            "algorithmic_bytes": dominant["algorithmic_bytes"],
            "kernel": f"w3_mfma_kernel on the field layout (fx_w3_gemv_fields) at gate/up "
                      f"{dominant['O']}x{dominant['K']}, M=1, same payloads repacked once",
        }
    if dominant.get("steady_state"):
        st = dominant["steady_state"]
        result["roofline_steady_state"] = {
            "bound": "hbm", "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "planar": {"achieved": st["planar"]["GBps"], "frac": st["planar"]["frac_hbm"]},
            "field_layout": {"achieved": st["fields"]["GBps"], "frac": st["fields"]["frac_hbm"]},
            "algorithmic_bytes_per_gemv": dominant["algorithmic_bytes"],
            "kernel": f"w3_mfma_kernel at gate/up {dominant['O']}x{dominant['K']}, M=1, one strided-batch launch "
                      f"over {dominant['copies']} payloads (the same payloads as roofline): the kernel without the "
                      "per-launch cost",
            "per_shape_frac": {name: {"planar": sh["steady_state"]["planar"]["frac_hbm"],
                                      "fields": sh["steady_state"]["fields"]["frac_hbm"]}
                               for name, sh in shapes.items() if sh.get("steady_state")},
        }
    if not args.no_fused_ops:
        result["config"]["fused_ops"] = fused_ops_bench(device, max(args.steps, 10), args.warmup, stream)
        print(f"# fused ops (config 2): {result['config']['fused_ops']}", file=sys.stderr, flush=True)
    if not args.no_two_base:
        result["config"]["two_base"] = two_base_bench(device, max(args.steps, 10), args.warmup, stream)
        print(f"# two-base: {result['config']['two_base']}", file=sys.stderr, flush=True)
        torch.cuda.empty_cache()
    if not args.no_decode:
        del graph, layers
        torch.cuda.empty_cache()
        result["config"]["decode"] = decode_bench(layers=args.decode_layers)
        torch.cuda.empty_cache()
        result["config"]["decode"]["hybrid_two_base_native"] = decode_hybrid_native(layers=args.decode_layers)
        print(f"# decode hybrid: {result['config']['decode']['hybrid_two_base_native']}", file=sys.stderr, flush=True)
        torch.cuda.empty_cache()
        result["config"]["decode"]["w3_desc_act_native"] = decode_desc_act_native(layers=args.decode_layers)
        print(f"# decode desc_act: {result['config']['decode']['w3_desc_act_native']}", file=sys.stderr, flush=True)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
