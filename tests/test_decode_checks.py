"""CPU tests of the decode gates and trace comparison (no GPU needed)."""
import pytest
import torch

from marlin_style_fluxbin_amd.acceleration_checks import numerical_gate, paired_cuda_timing, stepwise_nrmse
from marlin_style_fluxbin_amd.full_model_trial import compare_trace, validate_routes


def test_numerical_gate_thresholds():
    b = torch.linspace(-1, 1, 101, dtype=torch.float32)
    assert numerical_gate(b.clone(), b)["passed"]
    # fp32 reference: tol 0.002 elementwise on rms + |b| and nrmse <= 0.0005
    rms = float(b.square().mean().sqrt())
    bump = b.clone()
    bump[50] += 0.002 * (rms + abs(float(b[50]))) * 0.99
    assert numerical_gate(bump, b)["passed"]
    bump[50] += 0.002 * rms
    assert not numerical_gate(bump, b)["passed"]
    # bf16 references use the 10x looser factor
    assert numerical_gate(bump.bfloat16(), b.bfloat16())["elementwise_tolerance_factor"] == 0.02
    assert numerical_gate(b[:5], b)["reason"] == "shape mismatch"
    nan = b.clone()
    nan[0] = float("nan")
    assert numerical_gate(nan, b)["reason"] == "nonfinite output"
    # the reference's zero-reference cases (tests/test_acceleration_preparation.py:16-21)
    zero = torch.zeros(1, 7, dtype=torch.bfloat16)
    assert numerical_gate(zero, zero)["passed"]
    assert not numerical_gate(torch.ones_like(zero), zero)["passed"]
    assert not numerical_gate(zero + float("nan"), zero)["passed"]
    assert not numerical_gate(torch.zeros(2, 7), zero)["passed"]


def test_engine_backend_contract_known_answers():
    """M1Backend's contract (reference tests/test_acceleration_preparation.py:23-28)."""
    from marlin_style_fluxbin_amd.engine_interface import M1Backend

    backend = M1Backend()
    assert backend.contract.supported_m == (1,) and not backend.contract.tensor_parallel
    assert backend.workspace_shape(4096, 12288) == (12, 4096)
    with pytest.raises(ValueError):
        M1Backend(0)


def test_stepwise_nrmse():
    expected = torch.ones(1, 3, 8)
    actual = expected.clone()
    actual[0, 1] += 0.5
    values = stepwise_nrmse(actual, expected)
    assert values == pytest.approx([0.0, 0.5, 0.0])
    assert stepwise_nrmse(actual[0], expected[0]) is None


def _trace(logits, preds, fed):
    return {"logits": logits, "predictions": preds, "fed_tokens": fed}


def test_compare_trace_requires_tokens_contexts_and_logprobs():
    g = torch.Generator().manual_seed(0)
    logits = torch.randn(1, 4, 16, generator=g)
    preds = logits.argmax(-1)
    fed = torch.tensor([[1, 2, 3]])
    ref = _trace(logits, preds, fed)
    assert compare_trace(_trace(logits.clone(), preds, fed), ref, logprob_tolerance=0.0)["passed"]
    assert not compare_trace(_trace(logits, preds, fed + 1), ref, logprob_tolerance=1.0)["passed"]
    shifted = preds.clone()
    shifted[0, 0] += 1
    assert not compare_trace(_trace(logits, shifted, fed), ref, logprob_tolerance=1.0)["passed"]
    noisy = logits + 1e-3 * torch.randn(1, 4, 16, generator=g)
    report = compare_trace(_trace(noisy, preds, fed), ref, logprob_tolerance=1e-6)
    assert not report["passed"] and report["max_abs_logprob_error"] > 1e-6
    with pytest.raises(ValueError):
        compare_trace(ref, ref, logprob_tolerance=-1)


def test_validate_routes():
    trace = {"routes": {"a": {"dense_fallback": 1, "packed_m1": 4}, "b": {"dense_fallback": 1, "packed_m1": 4}}}
    assert validate_routes(trace, expected_linears=2, steps=4)
    assert not validate_routes(trace, expected_linears=3, steps=4)
    trace["routes"]["b"]["packed_m1"] = 3
    assert not validate_routes(trace, expected_linears=2, steps=4)


def test_paired_timing_argument_checks():
    with pytest.raises(ValueError):
        paired_cuda_timing({"a": lambda: None}, rounds=2)
    with pytest.raises(ValueError):
        paired_cuda_timing({"a": lambda: None}, warmup=0)
