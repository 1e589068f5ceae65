"""The reference's real payloads on the GPU path: desc_act column permutations.

The reference's artifact preparer requires ``desc_act=True``
(``scripts/prepare_qwen3_8b_w3_lut_artifacts.py:99``) and its converter stores
``perm = stable_argsort(g_idx)`` (``src/fluxbin_style/gptq_deployment.py:199-227``),
so every real artifact carries a column permutation that keeps each group's
columns in ascending order (``qwen3.desc_act_perm``).  Here:

* the gather is exactly a reordering of the activation: ``fx_w3_gemv(x, perm)``
  bit-equals ``fx_w3_gemv(x[:, perm], identity)`` at every Qwen3-8B Linear shape
  and activation-row count, and the field layout's gather form bit-equals the
  field kernel on the pre-gathered row (so either matches the float64 oracle to
  the same bar the identity order is held to, ``tests/test_w3_mfma_gpu.py``);
* the attention's output index writes the row-ordered output, reordered;
* the native decode chain runs permuted payloads fused (218 launches per token at
  the Qwen3-8B shapes, the same count as the identity order) and matches the HF
  module tree on them, layer by layer at the real shapes (tests/test_config3_gpu.py's
  bars) and over a whole small-model decode;
* the reference's table routes (``decoded_bf16``, ``groups_per_split > 1``) keep
  their own split contract inside the native decode: each Linear's output there is
  bit-identical to the module's own forward.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from marlin_style_fluxbin_amd import _lib
from marlin_style_fluxbin_amd.full_model_trial import compare_trace
from marlin_style_fluxbin_amd.native_decode import NativeDecodeSession, _Linear, inverse_index
from marlin_style_fluxbin_amd.qwen3 import desc_act_perm, qwen3_config, random_qwen3_model, w3_quantize_qwen3_model
from marlin_style_fluxbin_amd.static_decode import StaticDecodeSession, prepared_linears
from marlin_style_fluxbin_amd.w3_lut_deployment import PackedW3Linear, W3Gemv
from oracle import decode
from tests.payloads import config_codes, layout_from_codes

pytestmark = pytest.mark.gpu

QWEN3_SHAPES = [(4096, 4096), (1024, 4096), (12288, 4096), (4096, 12288)]


def _nrmse(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.double().flatten(), b.double().flatten()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


@pytest.mark.parametrize("o,k", QWEN3_SHAPES)
@pytest.mark.parametrize("m", [1, 8])
def test_gemv_gather_is_a_reordering_of_x(gpu, o, k, m):
    print(f"desc_act gather: {o}x{k}, M={m}", flush=True)
    codes, scales, zeros, _ = config_codes(o, k, seed=o + m, zeros=True, scale_dtype=torch.float16)
    perm = desc_act_perm(k, torch.Generator().manual_seed(k + m))
    dl = {n: t.to(gpu) for n, t in layout_from_codes(codes, scales, zeros, perm).items()}
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(o)).to(torch.bfloat16).to(gpu)
    gathered = torch.full((m, o), float("nan"), dtype=torch.bfloat16, device=gpu)
    W3Gemv(dl, perm_identity=False)(x, gathered)
    identity = dict(dl, perm=torch.arange(k, dtype=torch.int16, device=gpu))
    reordered = torch.full_like(gathered, float("nan"))
    W3Gemv(identity, perm_identity=True)(x[:, perm.long().to(gpu)].contiguous(), reordered)
    torch.cuda.synchronize()
    assert torch.equal(gathered, reordered)


def test_gemv_gather_matches_the_oracle_at_q_proj(gpu):
    """The permuted form against the float64 dequantize-then-matmul (a wrong gather
    direction, perm vs its inverse, fails this by O(1))."""
    from oracle import w3
    from tests.payloads import assert_half_ulp, oracle_layout

    o = k = 4096
    codes, scales, zeros, _ = config_codes(o, k, seed=0, zeros=True, scale_dtype=torch.float16)
    perm = desc_act_perm(k, torch.Generator().manual_seed(0))
    layout = layout_from_codes(codes, scales, zeros, perm)
    dl = {n: t.to(gpu) for n, t in layout.items()}
    x = torch.randn(1, k, generator=torch.Generator().manual_seed(0)).to(torch.bfloat16)
    out = torch.full((1, o), float("nan"), dtype=torch.bfloat16, device=gpu)
    W3Gemv(dl)(x.to(gpu), out)
    exact = w3.matvec_exact(x.float().numpy(), oracle_layout(layout))
    assert_half_ulp(out.float().cpu().numpy(), exact, "bf16", what="desc_act q_proj")


@pytest.mark.parametrize("pos", [40, 543])
def test_attention_output_index(gpu, pos):
    """fx_decode_attention with an output index writes value i to out[index[i]]:
    the row-ordered output reordered (one split at 41 keys, split + combine at 544)."""
    hq, hk, d, lmax = 32, 8, 128, 544
    g = torch.Generator().manual_seed(pos)
    q = torch.randn(hq, d, generator=g).to(torch.bfloat16).to(gpu)
    kc = torch.randn(hk, lmax, d, generator=g).to(torch.bfloat16).to(gpu)
    vc = torch.randn(hk, lmax, d, generator=g).to(torch.bfloat16).to(gpu)
    nxt = torch.randperm(hq * d, generator=g).to(torch.int16).to(gpu)
    index = inverse_index(nxt)
    lib = _lib.library()
    nbytes = lib.fx_decode_attention_workspace_bytes(hq, lmax, d)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=gpu)
    outs = []
    for idx in (None, index):
        out = torch.full((hq, d), float("nan"), dtype=torch.bfloat16, device=gpu)
        _lib.check(lib.fx_decode_attention(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), ws.data_ptr(), nbytes,
                                           _lib.ptr(idx), out.data_ptr(), hq, hk, lmax, d, pos, 1 / np.sqrt(d),
                                           _lib.FX_BF16, _lib.stream_handle(gpu)), "attention")
        outs.append(out)
    torch.cuda.synchronize()
    plain, indexed = outs
    assert torch.equal(indexed.flatten(), plain.flatten()[nxt.long()])
    exact = decode.gqa_attention(q.float().cpu().numpy(), kc.float().cpu().numpy(), vc.float().cpu().numpy(), pos,
                                 1 / np.sqrt(d))
    assert np.abs(plain.float().cpu().numpy() - exact).max() <= 2e-2 * np.abs(exact).max()


# ----------------------------------------------------------------- native decode
PREFIX, STEPS = 20, 8


def _small(gpu, **quant):
    config = qwen3_config(hidden_size=256, intermediate_size=512, num_hidden_layers=3, num_attention_heads=4,
                          num_key_value_heads=2, head_dim=64, vocab_size=384, max_position_embeddings=128)
    model = random_qwen3_model(config, device=gpu, dtype=torch.bfloat16, seed=2)
    w3_quantize_qwen3_model(model, **quant)
    g = torch.Generator().manual_seed(5)
    ids = torch.randint(0, 384, (1, PREFIX), generator=g).to(gpu)
    forced = torch.randint(0, 384, (1, STEPS), generator=g).to(gpu)
    return model, ids, forced


def _against_hf(model, ids, forced, payload):
    from torch.nn.attention import SDPBackend, sdpa_kernel

    with sdpa_kernel([SDPBackend.MATH]):
        hf = StaticDecodeSession(model, ids, forced)
        with prepared_linears(model, torch.bfloat16):
            want = hf.audit()
        native = NativeDecodeSession(model, ids, forced, w3_payload=payload)
    eager = native.audit()
    graph = native.capture()
    assert torch.equal(graph["logits"], eager["logits"])
    report = compare_trace(graph, want, logprob_tolerance=0.05)
    # the bars of tests/test_native_decode_gpu.py::test_native_session_matches_hf_static_session
    assert report["greedy_tokens_equal"] and report["fed_tokens_equal"], report
    assert report["max_abs_logprob_error"] <= 0.05, report
    assert report["logits"]["normalized_rmse"] <= 0.02, report
    assert report["stepwise_normalized_rmse"][1] <= 0.01, report
    return native


@pytest.mark.parametrize("payload", ["fields", "planar"])
def test_native_session_desc_act_matches_hf(gpu, payload):
    print(f"native decode, desc_act payloads, {payload}", flush=True)
    model, ids, forced = _small(gpu, desc_act_seed=7)
    perms = [model.model.layers[0].get_submodule(n).perm for n in ("self_attn.q_proj", "self_attn.o_proj",
                                                                    "mlp.gate_proj", "mlp.down_proj")]
    assert all(not torch.equal(p.long().cpu(), torch.arange(p.numel())) for p in perms)
    native = _against_hf(model, ids, forced, payload)
    # the fused residual-stream chain, not the per-Linear fallback
    assert native.stream is not None and native.stream.o_index[0] is not None
    assert native.kernel_nodes / STEPS <= 5 * 3 + 6


@pytest.mark.parametrize("route", ["fast_corrected", "observed_exact"])
def test_native_session_table_routes(gpu, route):
    """Table-route Linears (decoded_bf16 arithmetic; observed_exact also two groups
    per split) run their own split contract in the native decode: every Linear's
    decode call bit-equals the module's forward, and the session matches HF with
    the same modules.  desc_act payloads, so the table kernel's gather runs too."""
    print(f"native decode, table route {route}", flush=True)
    model, ids, forced = _small(gpu, desc_act_seed=3, scale_dtype=torch.bfloat16, zeros=False)
    gps = 2 if route == "observed_exact" else 1
    for block in model.model.layers:
        for name in ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
                     "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"):
            old = block.get_submodule(name)
            new = PackedW3Linear(old.layout(), fallback="dense", row_tile=256, groups_per_split=gps,
                                 arithmetic="decoded_bf16", route=route)
            parent, attr = name.rsplit(".", 1)
            setattr(block.get_submodule(parent), attr, new)
    g = torch.Generator().manual_seed(1)
    with torch.inference_mode():
        for name in ("self_attn.q_proj", "mlp.down_proj"):
            module = model.model.layers[1].get_submodule(name)
            x = torch.randn(1, module.in_features, generator=g).to(torch.bfloat16).to(gpu)
            out = torch.full((1, module.out_features), float("nan"), dtype=torch.bfloat16, device=gpu)
            _Linear(module)(x, out)
            assert torch.equal(out, module(x)), name
    native = _against_hf(model, ids, forced, "fields")
    assert native.stream is None  # table routes do not fuse


def test_config3_desc_act_first_step_layer_by_layer(gpu):
    """tests/test_config3_gpu.py's layer-by-layer check at the Qwen3-8B shapes (4
    layers, prefill 512) on desc_act payloads, field layout; and the exact launch
    count of the fused chain: 6 per layer + 2 per token + the last merge."""
    from torch.nn.attention import SDPBackend, sdpa_kernel

    print("config 3 desc_act: 4 layers, first decode step layer by layer", flush=True)
    config = qwen3_config(num_hidden_layers=4)
    model = random_qwen3_model(config, device=gpu, dtype=torch.bfloat16, seed=0)
    assert w3_quantize_qwen3_model(model, desc_act_seed=11) == 28
    g = torch.Generator().manual_seed(0)
    ids = torch.randint(0, config.vocab_size, (1, 512), generator=g).to(gpu)
    tokens = torch.randint(0, config.vocab_size, (1, 2), generator=g).to(gpu)
    hf_layers, native_layers = {}, {}

    def hook(index):
        def record(module, args, output):
            hidden = output[0] if isinstance(output, tuple) else output
            hf_layers.setdefault(index, hidden.detach().reshape(-1).clone())
        return record

    with sdpa_kernel([SDPBackend.MATH]):
        hf = StaticDecodeSession(model, ids, tokens)
        handles = [layer.register_forward_hook(hook(i)) for i, layer in enumerate(model.model.layers)]
        try:
            with prepared_linears(model, torch.bfloat16):
                want = hf.audit()
        finally:
            for h in handles:
                h.remove()
        native = NativeDecodeSession(model, ids, tokens)
    assert native.stream is not None and native.stream.qkv_index[0] is not None

    def observe(step, layer, residual):
        if step == 0:
            native_layers[layer] = residual.detach().reshape(-1).clone()

    native.layer_observer = observe
    got = native.audit()
    native.layer_observer = None
    errors = [_nrmse(native_layers[i], hf_layers[i]) for i in range(4)]
    print(f"desc_act per-layer NRMSE of the first decode step: {errors}", flush=True)
    bound = 0.0
    for err in errors:
        bound += 6e-3
        assert err <= bound, errors
    report = compare_trace(got, want, logprob_tolerance=0.1)
    assert report["stepwise_normalized_rmse"][1] <= 2e-2, report["stepwise_normalized_rmse"]
    assert torch.equal(got["predictions"][:, :2], want["predictions"][:, :2])
    graph = native.capture()
    assert torch.equal(graph["logits"], got["logits"])
    assert native.kernel_nodes == 2 * (6 * 4 + 2) + 1, native.kernel_nodes
