"""GPU decode protocol on a small Qwen3 with W3 Linears (HF model, our kernels).

Mirrors the reference's static-decode checks (tests/test_static_decode.py,
tests/test_w3_lut_adapter.py:117-155 in maxiu188-afk/Marlin_Style_Fluxbin):
the dynamic-KV trace (prefill through the dense fallback, packed M=1 steps),
the prepared eager static run and the captured graph must agree; graph replays
must reproduce the captured run; poisoned future KV slots must be ignored.
"""
import pytest
import torch

from marlin_style_fluxbin_amd.acceleration_checks import numerical_gate
from marlin_style_fluxbin_amd.full_model_trial import compare_trace, decode_trace, packed_modules, validate_routes
from marlin_style_fluxbin_amd.fused_modules import fused_qwen3_modules
from marlin_style_fluxbin_amd.qwen3 import qwen3_config, random_qwen3_model, w3_quantize_qwen3_model
from marlin_style_fluxbin_amd.static_decode import StaticDecodeSession, prepared_linears

pytestmark = pytest.mark.gpu

PREFIX, STEPS = 12, 6


def _model(gpu, zeros=True):
    config = qwen3_config(hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
                          num_key_value_heads=2, head_dim=64, vocab_size=384, max_position_embeddings=128)
    model = random_qwen3_model(config, device=gpu, dtype=torch.bfloat16, seed=1)
    assert w3_quantize_qwen3_model(model, zeros=zeros) == 14
    return model


def _inputs(gpu):
    g = torch.Generator().manual_seed(3)
    ids = torch.randint(0, 384, (1, PREFIX), generator=g).to(gpu)
    forced = torch.randint(0, 384, (1, STEPS), generator=g).to(gpu)
    return ids, forced


@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("zeros", [True, False])
def test_dynamic_static_graph_agree(gpu, fused, zeros):
    model = _model(gpu, zeros)
    ids, forced = _inputs(gpu)
    ctx = fused_qwen3_modules() if fused else torch.no_grad()
    with ctx:
        dynamic = decode_trace(model, ids, steps=STEPS, forced_tokens=forced)
        assert validate_routes(dynamic, expected_linears=14, steps=STEPS)
        session = StaticDecodeSession(model, ids, forced)
        with prepared_linears(model, torch.bfloat16):
            eager = session.audit()
            graph = session.capture()
            routes = session.capture_routes
    assert all(r == {"dense_fallback": 0, "packed_m1": STEPS} for r in eager["routes"].values())
    assert all(r == {"dense_fallback": 0, "packed_m1": STEPS} for r in routes.values())
    # at least the 14 W3 GEMV launches per step are kernel nodes of the graph
    assert session.kernel_nodes is not None and session.kernel_nodes >= 14 * STEPS
    # the graph replays exactly the prepared eager computation
    assert torch.equal(graph["logits"], eager["logits"])
    # static KV + prepared binding vs dynamic KV: same arithmetic, different attention masking path
    report = compare_trace(graph, dynamic, logprob_tolerance=0.05)
    assert report["passed"], report
    assert all(m._decode_binding is None for m in packed_modules(model).values())


def test_graph_replays_track_eager_between(gpu):
    """Replays interleaved with the program's own eager work and synchronisations
    all reproduce the captured trace bit for bit."""
    model = _model(gpu)
    ids, forced = _inputs(gpu)
    session = StaticDecodeSession(model, ids, forced)
    with prepared_linears(model, torch.bfloat16):
        first = session.capture()
        for _ in range(3):
            eager = session.audit()
            torch.cuda.synchronize()
            timing, replay = session.measure("sequence_graph")
            assert torch.equal(replay["logits"], first["logits"])
            assert torch.equal(eager["logits"], first["logits"])
            assert timing["device_ms"] > 0


def test_poisoned_future_kv_slots_and_full_prefix_recompute(gpu):
    """Stale values in future cache slots are masked out (finite poison, as in the
    reference's test: NaN would leak through 0 * NaN in any P.V product), and each
    step's logits match a cache-free forward over the whole prefix."""
    model = _model(gpu)
    ids, forced = _inputs(gpu)
    session = StaticDecodeSession(model, ids, forced)
    with prepared_linears(model, torch.bfloat16):
        clean = session.audit()
        session.reset()
        with torch.inference_mode():
            for layer in session.cache.layers:
                layer.keys[:, :, PREFIX:].fill_(100)
                layer.values[:, :, PREFIX:].fill_(100)
        poisoned = session.trace(session.run())
    assert torch.equal(poisoned["logits"], clean["logits"])
    with torch.inference_mode():
        for i in range(STEPS):
            prefix = torch.cat((ids, forced[:, :i]), 1)
            full = model(input_ids=prefix, use_cache=False).logits[:, -1, :].float().cpu()
            gate = numerical_gate(clean["logits"][:, i, :].float(), full)
            assert gate["normalized_rmse"] < 0.02, (i, gate)


def test_w3_decode_close_to_bf16_model(gpu):
    """Quantization error only: the W3 model's prefill logits stay correlated with
    the bf16 model it was quantized from (a sanity bar, not a parity claim)."""
    config = qwen3_config(hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
                          num_key_value_heads=2, head_dim=64, vocab_size=384, max_position_embeddings=128)
    dense = random_qwen3_model(config, device=gpu, dtype=torch.bfloat16, seed=1)
    ids, _ = _inputs(gpu)
    with torch.inference_mode():
        want = dense(input_ids=ids).logits.float()
    w3_quantize_qwen3_model(dense)
    with torch.inference_mode():
        got = dense(input_ids=ids).logits.float()
    # 3-bit round-to-nearest on N(0, 0.02) weights through two layers measures
    # ~0.88 cosine similarity; a broken packing or scale would be near 0
    cos = torch.nn.functional.cosine_similarity(got.flatten(), want.flatten(), dim=0)
    assert cos > 0.75, cos


def test_decode_trace_short_prompt_on_small_m_modules(gpu):
    """Modules that opt into 2..8-row inputs (max_packed_rows=8) serve a 4-token
    prompt on the small-M packed route inside decode_trace, whose counter reset
    keeps that route's key.  Against the same trace with the prompt served densely:
    the dense fallback multiplies by the bf16-rounded restored weight, the packed
    route by the exact s (q - z), so the prompt's logits differ by more than the
    frozen gate's bf16 NRMSE; the bars are those of two implementations of the same
    model (same greedy tokens, log-probs within 0.05, logits NRMSE within 0.02)."""
    from marlin_style_fluxbin_amd.w3_lut_deployment import PackedW3Linear

    model = _model(gpu)
    ids, forced = _inputs(gpu)
    short = ids[:, :4]
    dense = decode_trace(model, short, steps=STEPS, forced_tokens=forced)
    for block in model.model.layers:
        for name, module in list(block.named_modules()):
            if isinstance(module, PackedW3Linear):
                parent, attr = name.rsplit(".", 1)
                setattr(block.get_submodule(parent), attr,
                        PackedW3Linear(module.layout(), fallback="dense", row_tile=256, max_packed_rows=8))
    small = decode_trace(model, short, steps=STEPS, forced_tokens=forced)
    assert all(r == {"packed_m1": STEPS, "dense_fallback": 0, "packed_small_m": 1} for r in small["routes"].values())
    assert validate_routes(small, expected_linears=14, steps=STEPS)
    report = compare_trace(small, dense, logprob_tolerance=0.05)
    assert report["greedy_tokens_equal"] and report["fed_tokens_equal"], report
    assert report["max_abs_logprob_error"] <= 0.05, report
    assert report["logits"]["normalized_rmse"] <= 0.02, report
