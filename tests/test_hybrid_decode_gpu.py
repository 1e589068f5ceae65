"""Full-model decode with the reference's hybrid two-base g128/s8 Linears
(``PackedHybridLinear`` on every Linear of every block, ``fx_hybrid_gemv``), after
the reference's prepared-decode trial (``scripts/run_qwen3_8b_prepared_m1_trial.py``,
``full_model_trial.py:10-12``): the HF module tree through ``prepared_linears``
against its own dynamic-KV trace (routes exact), and the native kernel chain
against the HF module tree run with the same arithmetic (SDPA math backend).
Bars as for the W3 native session: same greedy tokens on the same context,
log-probs within 0.05, logits NRMSE within 0.02, the first decode step within
0.01, graph replay bit-equal to the eager run.
"""
from __future__ import annotations

import pytest
import torch

from marlin_style_fluxbin_amd.deployment import PackedHybridLinear
from marlin_style_fluxbin_amd.full_model_trial import compare_trace, decode_trace, packed_modules, validate_routes
from marlin_style_fluxbin_amd.native_decode import NativeDecodeSession
from marlin_style_fluxbin_amd.qwen3 import hybrid_qwen3_model, qwen3_config, random_qwen3_model
from marlin_style_fluxbin_amd.static_decode import StaticDecodeSession, prepared_linears

pytestmark = pytest.mark.gpu

PREFIX, STEPS = 20, 8


def _model(gpu):
    config = qwen3_config(hidden_size=256, intermediate_size=512, num_hidden_layers=3, num_attention_heads=4,
                          num_key_value_heads=2, head_dim=64, vocab_size=384, max_position_embeddings=128)
    model = random_qwen3_model(config, device=gpu, dtype=torch.bfloat16, seed=3)
    assert hybrid_qwen3_model(model, seed=4) == 21
    g = torch.Generator().manual_seed(6)
    ids = torch.randint(0, 384, (1, PREFIX), generator=g).to(gpu)
    forced = torch.randint(0, 384, (1, STEPS), generator=g).to(gpu)
    return model, ids, forced


def test_hybrid_hf_static_session_matches_dynamic_trace(gpu):
    model, ids, _ = _model(gpu)
    modules = packed_modules(model)
    assert len(modules) == 21 and all(isinstance(m, PackedHybridLinear) for m in modules.values())
    dynamic = decode_trace(model, ids, steps=STEPS)
    assert validate_routes(dynamic, expected_linears=21, steps=STEPS)
    session = StaticDecodeSession(model, ids, dynamic["fed_tokens"].to(gpu))
    with prepared_linears(model, torch.bfloat16):
        audit = session.audit()
        assert all(r == {"dense_fallback": 0, "packed_m1": STEPS} for r in audit["routes"].values())
        graph = session.capture()
    assert torch.equal(graph["logits"], audit["logits"])
    assert compare_trace(audit, dynamic, logprob_tolerance=0.05)["greedy_tokens_equal"]


def test_hybrid_native_session_matches_hf(gpu):
    from torch.nn.attention import SDPBackend, sdpa_kernel

    model, ids, forced = _model(gpu)
    with sdpa_kernel([SDPBackend.MATH]):
        hf = StaticDecodeSession(model, ids, forced)
        with prepared_linears(model, torch.bfloat16):
            want = hf.audit()
        native = NativeDecodeSession(model, ids, forced)
    # hybrid Linears take the residual-stream chain: normalising q|k|v and gate|up
    # launches, o and down adding into the residual, the SwiGLU kernel
    assert native.stream is not None and native.stream.kind == "hybrid"
    eager = native.audit()
    graph = native.capture()
    assert torch.equal(graph["logits"], eager["logits"])
    report = compare_trace(graph, want, logprob_tolerance=0.05)
    assert report["greedy_tokens_equal"] and report["fed_tokens_equal"], report
    assert report["max_abs_logprob_error"] <= 0.05, report
    assert report["logits"]["normalized_rmse"] <= 0.02, report
    assert report["stepwise_normalized_rmse"][1] <= 0.01, report
    for _ in range(2):
        _, replay = native.measure("sequence_graph")
        assert torch.equal(replay["logits"], graph["logits"])
