"""The PPL harness's three arms on the GPU, packed arm included (reference
``scripts/run_qwen3_8b_w3_packed_m1_ppl.py``): a two-layer Qwen3 checkpoint and a
hash-bound W3 artifact of its 14 Linears.

Pins: the packed arm's route smoke (every Linear takes ``packed_m1`` once), its
per-transition NLLs against the decoded-W3 arm's (the same weights through
hipBLASLt ``F.linear``: the two differ only by bf16 rounding inside the
Linears, so each NLL agrees within 0.03 nats and the mean within 0.005; the whole
model in float32 instead of bf16 moves them by up to 0.014), and the
full command line over all three arms.
"""
from __future__ import annotations

import pytest
import torch
from safetensors.torch import save_file

from marlin_style_fluxbin_amd import ppl
from marlin_style_fluxbin_amd.qwen3 import random_qwen3_model
from marlin_style_fluxbin_amd.static_decode import prepared_linears
from tests.test_ppl import _artifact, _config, _tokens

pytestmark = pytest.mark.gpu


def test_packed_arm_matches_decoded_arm(gpu, tmp_path):
    config = _config(vocab=256)
    root, sha, _ = _artifact(tmp_path, config)
    blocks = ppl.token_blocks(_tokens(48, vocab=256, seed=9), 16)
    nll = {}
    for arm in ("decoded_w3_bf16", "packed_w3_inline"):
        model = random_qwen3_model(config, device=gpu, dtype=torch.bfloat16, seed=11).eval()
        coverage = ppl.prepare_arm(model, arm, artifact_root=root, expected_manifest_sha256=sha)
        packed = arm == "packed_w3_inline"
        assert (coverage["linear_count"] == 14) if packed else coverage is None
        record = ppl.score_m1_ppl(model, blocks, arm=arm, device=gpu, expected_packed_linears=14 if packed else 0)
        assert record["metrics_valid"] and record["scored_transition_count"] == 45
        if packed:
            assert record["packed_route_smoke"] == {"passed": True, "linear_count": 14, "calls_per_linear": 1}
        with torch.inference_mode(), (prepared_linears(model, torch.bfloat16) if packed else torch.no_grad()):
            nll[arm] = torch.cat([ppl._TransitionScorer(model, gpu).block(b) for b in blocks]).cpu()
        nll[arm + ":record"] = record
    diff = (nll["packed_w3_inline"] - nll["decoded_w3_bf16"]).abs()
    assert float(diff.max()) <= 0.03, float(diff.max())
    delta = nll["packed_w3_inline:record"]["mean_nll"] - nll["decoded_w3_bf16:record"]["mean_nll"]
    assert abs(delta) <= 0.005, delta


def test_command_line_three_arms(gpu, tmp_path):
    config = _config(vocab=256)
    root, sha, _ = _artifact(tmp_path, config)
    snapshot = tmp_path / "snapshot"
    random_qwen3_model(config, device="cpu", dtype=torch.bfloat16, seed=12).save_pretrained(snapshot)
    tokens = tmp_path / "tokens.safetensors"
    save_file({"tokens": torch.tensor(_tokens(64, vocab=256, seed=13), dtype=torch.int32)}, str(tokens))
    summary = ppl.main(["--snapshot-root", str(snapshot), "--token-artifact", str(tokens), "--sequence-length", "16",
                        "--w3-layout-root", str(root), "--w3-layout-manifest-sha256", sha,
                        "--output-dir", str(tmp_path / "run"), "--device", str(gpu)])
    assert summary["status"] == "completed_pending_effect_size_review", summary["validity_gates"]
    assert set(summary["comparisons"]) == {"decoded_w3_vs_original_bf16", "packed_w3_vs_decoded_w3",
                                           "packed_w3_vs_original_bf16"}
    packed = summary["arms"]["packed_w3_inline"]
    assert packed["packed_linear_count"] == 14 and packed["scored_transition_count"] == 60
    assert abs(summary["comparisons"]["packed_w3_vs_decoded_w3"]["mean_nll_delta"]) <= 0.005
