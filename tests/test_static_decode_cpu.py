"""CPU contract of the static-KV decode session and the prepared-binding context.

Ports the reference's CPU tests (``tests/test_static_decode.py:14-72``): a tiny
random Qwen3 on the CPU, static decode equal to the dynamic-KV ``decode_trace``
and to a full-prefix recompute, reset between passes with the cache storage kept,
future slots ignored even when poisoned, no graph capture without a GPU; the
prepared-binding context clears every binding after a failure part-way through,
and a device move clears a binding.
"""
from __future__ import annotations

from unittest.mock import patch

import pytest
import torch

from marlin_style_fluxbin_amd.deployment import PackedHybridLinear
from marlin_style_fluxbin_amd.full_model_trial import compare_trace, decode_trace, validate_routes
from marlin_style_fluxbin_amd.static_decode import StaticDecodeSession, prepared_linears
from oracle import two_base as tb


def _model():
    from transformers import Qwen3Config, Qwen3ForCausalLM

    torch.manual_seed(17)
    cfg = Qwen3Config(vocab_size=64, hidden_size=32, intermediate_size=64, num_hidden_layers=2,
                      num_attention_heads=2, num_key_value_heads=1, head_dim=16)
    cfg._attn_implementation = "sdpa"
    return Qwen3ForCausalLM(cfg).eval()


def test_static_matches_dynamic_full_prefix_and_reset():
    model = _model()
    ids = torch.tensor([[1, 3, 7]])
    dynamic = decode_trace(model, ids, steps=3)
    assert dynamic["cache_length"] == 6 and dynamic["predictions"].shape == (1, 4)
    assert dynamic["prefill_device_ms"] is None and dynamic["step_device_ms"] == []
    session = StaticDecodeSession(model, ids, dynamic["fed_tokens"])
    storage = [(layer.keys.data_ptr(), layer.values.data_ptr()) for layer in session.cache.layers]
    first = session.audit()
    torch.testing.assert_close(first["logits"], dynamic["logits"], atol=1e-6, rtol=1e-5)
    for _ in range(2):
        timing, trace = session.measure("prepared_eager")
        assert timing["wall_ms"] > 0 and timing["device_ms"] is None
        assert torch.equal(trace["logits"], first["logits"]) and trace["cache_length"] == 6
    assert storage == [(layer.keys.data_ptr(), layer.values.data_ptr()) for layer in session.cache.layers]
    with torch.inference_mode():
        session.reset()
        for layer in session.cache.layers:  # stale values in future slots must stay masked
            layer.keys[:, :, 4:].fill_(100)
            layer.values[:, :, 4:].fill_(100)
        poisoned = session.trace(session.run())
        torch.testing.assert_close(poisoned["logits"], first["logits"], atol=0, rtol=0)
        for i in range(4):
            prefix = torch.cat((ids, dynamic["fed_tokens"][:, :i]), 1)
            expected = model(input_ids=prefix, use_cache=False).logits[:, -1, :]
            torch.testing.assert_close(first["logits"][:, i, :], expected, atol=1e-6, rtol=1e-5)
    assert compare_trace(first, dynamic, logprob_tolerance=0.0)["greedy_tokens_equal"]
    with pytest.raises(RuntimeError, match="CUDA"):
        session.capture()
    with pytest.raises(ValueError, match="capture first"):
        session.measure("sequence_graph")
    with pytest.raises(ValueError, match="unknown mode"):
        session.measure("other")


def test_session_rejects_bad_inputs():
    model = _model()
    with pytest.raises(ValueError, match="prefix"):
        StaticDecodeSession(model, torch.tensor([[1]]), torch.tensor([[2]]))
    with pytest.raises(ValueError, match="continuation"):
        StaticDecodeSession(model, torch.tensor([[1, 2]]), torch.zeros(1, 0, dtype=torch.long))
    model.train()
    with pytest.raises(ValueError, match="eval model"):
        StaticDecodeSession(model, torch.tensor([[1, 2]]), torch.tensor([[2]]))


def test_forced_decode_trace_and_routes():
    model = _model()
    ids = torch.tensor([[5, 9]])
    forced = torch.tensor([[1, 2, 3]])
    trace = decode_trace(model, ids, steps=3, forced_tokens=forced)
    assert torch.equal(trace["fed_tokens"], forced) and trace["routes"] == {}
    assert validate_routes(trace, expected_linears=0, steps=3)
    with pytest.raises(ValueError, match=r"\[1,steps\]"):
        decode_trace(model, ids, steps=2, forced_tokens=forced)
    with pytest.raises(ValueError, match="batch1"):
        decode_trace(model, ids, steps=0)


def _hybrid(o, g):
    return PackedHybridLinear({k: torch.from_numpy(v) for k, v in tb.make_hybrid_payload(o, g).items()})


def test_binding_rejects_cpu_and_cleans_up_after_partial_failure():
    modules = torch.nn.Sequential(_hybrid(32, 1), _hybrid(32, 1))
    with pytest.raises(ValueError, match="CUDA"):
        modules[0].bind_prepared_decode(torch.bfloat16)

    def partial(module, dtype):
        module._decode_binding = lambda x: x
        if module is modules[1]:
            raise RuntimeError("partial failure")

    with patch.object(PackedHybridLinear, "bind_prepared_decode", partial):
        with pytest.raises(RuntimeError, match="partial failure"):
            with prepared_linears(modules, torch.bfloat16):
                pass
    assert all(m._decode_binding is None for m in modules)
    modules[0]._decode_binding = lambda x: x
    modules[0].to("cpu")
    assert modules[0]._decode_binding is None
    modules[0]._decode_binding = lambda x: x
    with pytest.raises(ValueError, match="overlap"):
        with prepared_linears(modules, torch.bfloat16):
            pass
