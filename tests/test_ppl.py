"""CPU tests of the teacher-forced M=1 PPL harness (reference
``scripts/run_qwen3_8b_w3_packed_m1_ppl.py:230-347``).

Pins: the cached one-token NLLs equal the NLLs of one full-sequence forward of a
float32 model (an off-by-one label or position, or a wrong log-softmax, breaks
the equality); the arm record's aggregates against the per-block values; the
decoded arm's weights against the artifact's restore; the hash framing and the
block cut by construction.  The packed arm needs the GPU (``test_ppl_gpu.py``).
"""
from __future__ import annotations

import json
import math

import pytest
import torch
from safetensors.torch import save_file

from marlin_style_fluxbin_amd import gptq_deployment as gd
from marlin_style_fluxbin_amd import ppl
from marlin_style_fluxbin_amd.qwen3 import (QWEN3_LINEAR_MODULES, expected_qwen3_linear_shape, qwen3_config,
                                            random_qwen3_model)
from marlin_style_fluxbin_amd.w3_lut_artifacts import sha256_file, write_w3_lut_artifacts
from tests.payloads import synthetic_raw

CPU = torch.device("cpu")


def _config(vocab=96):
    return qwen3_config(hidden_size=128, intermediate_size=256, num_hidden_layers=2, num_attention_heads=4,
                        num_key_value_heads=2, head_dim=32, vocab_size=vocab, max_position_embeddings=64)


def _tokens(n, vocab=96, seed=0):
    return torch.randint(0, vocab, (n,), generator=torch.Generator().manual_seed(seed)).tolist()


def test_cached_nll_equals_full_forward_nll():
    model = random_qwen3_model(_config(), device="cpu", dtype=torch.float32, seed=3).eval()
    block = _tokens(13, seed=1)
    with torch.inference_mode():
        cached = ppl._TransitionScorer(model, CPU).block(block)
        logits = model(input_ids=torch.tensor([block]), use_cache=False).logits[0].float()
        full = torch.nn.functional.cross_entropy(logits[:-1], torch.tensor(block[1:]), reduction="none")
        shifted = torch.nn.functional.cross_entropy(logits[1:], torch.tensor(block[1:]), reduction="none")
    assert cached.dtype == torch.float32 and cached.shape == (12,)
    torch.testing.assert_close(cached, full, rtol=1e-5, atol=1e-5)
    assert not torch.allclose(cached, shifted, atol=1e-3)  # a position off by one is visible


def test_arm_record_aggregates():
    model = random_qwen3_model(_config(), device="cpu", dtype=torch.bfloat16, seed=4).eval()
    blocks = ppl.token_blocks(_tokens(30, seed=2), 10)
    record = ppl.score_m1_ppl(model, blocks, arm="original_bf16", device=CPU, expected_packed_linears=0)
    assert record["status"] == "completed" and record["metrics_valid"]
    assert record["block_count"] == 3 and record["scored_transition_count"] == 27
    with torch.inference_mode():
        sums = [float(ppl._TransitionScorer(model, CPU).block(b).double().sum()) for b in blocks]
    assert record["total_nll"] == pytest.approx(math.fsum(sums), rel=1e-12)
    assert record["mean_nll"] == pytest.approx(record["total_nll"] / 27, rel=1e-12)
    assert record["perplexity"] == pytest.approx(math.exp(record["mean_nll"]), rel=1e-12)
    assert len(record["block_nll_sha256"]) == 3 and record["packed_route_smoke"] is None
    assert record["logits_dtype"] == "torch.bfloat16" and record["nll_logits_dtype"] == "torch.float32"


def test_nonfinite_block_stops_the_arm(monkeypatch):
    model = random_qwen3_model(_config(), device="cpu", dtype=torch.float32, seed=5).eval()
    blocks = ppl.token_blocks(_tokens(24, seed=3), 8)
    original = ppl._TransitionScorer.block
    calls = []

    def poisoned(self, block):
        calls.append(1)
        nll = original(self, block)
        if len(calls) == 2:
            nll[3] = float("nan")
        return nll

    monkeypatch.setattr(ppl._TransitionScorer, "block", poisoned)
    record = ppl.score_m1_ppl(model, blocks, arm="original_bf16", device=CPU, expected_packed_linears=0)
    assert record["status"] == "invalid" and not record["metrics_valid"]
    assert record["nonfinite_block_indices"] == [1] and record["block_count"] == 1 and len(calls) == 2
    assert record["total_nll"] is None and record["perplexity"] is None


def test_finite_perplexity():
    assert ppl.finite_perplexity(2.0) == pytest.approx(math.exp(2.0))
    for bad in (None, float("nan"), float("inf"), 1e6):
        assert ppl.finite_perplexity(bad) is None


def test_blocks_hashes_and_token_artifact(tmp_path):
    assert ppl.token_blocks(list(range(10)), 4) == [[0, 1, 2, 3], [4, 5, 6, 7]]
    assert ppl.token_blocks(list(range(10)), 2, used_token_count=4) == [[0, 1], [2, 3]]
    for bad in (dict(used_token_count=5), dict(used_token_count=12)):
        with pytest.raises(ValueError):
            ppl.token_blocks(list(range(10)), 4, **bad)
    with pytest.raises(ValueError):
        ppl.token_blocks(list(range(10)), 1)
    # the framing separates sequences: the same tokens cut differently hash differently
    h = ppl.sha256_token_sequences
    assert h([[1, 2], [3]]) != h([[1], [2, 3]]) != h([[1, 2, 3]])
    assert h([[-1]]) != h([[2 ** 64 - 1 - 2 ** 63]]) and h([]) != h([[]])
    path = tmp_path / "tokens.safetensors"
    save_file({"tokens": torch.arange(20, dtype=torch.int32)}, str(path))
    tokens = ppl.load_token_artifact(path, expected_file_sha256=sha256_file(path),
                                     expected_tokens_sha256=h([list(range(20))]))
    assert tokens == list(range(20))
    with pytest.raises(ValueError, match="token artifact hash"):
        ppl.load_token_artifact(path, expected_file_sha256="0" * 64)
    with pytest.raises(ValueError, match="token stream hash"):
        ppl.load_token_artifact(path, expected_tokens_sha256=h([list(range(19))]))
    extra = tmp_path / "extra.safetensors"
    save_file({"tokens": torch.arange(4, dtype=torch.int32), "mask": torch.ones(4)}, str(extra))
    with pytest.raises(ValueError, match="inventory"):
        ppl.load_token_artifact(extra)


def _artifact(tmp_path, config):
    layers = []
    for layer in range(config.num_hidden_layers):
        modules = {}
        for i, name in enumerate(QWEN3_LINEAR_MODULES):
            o, k = expected_qwen3_linear_shape(config.to_dict(), name)
            modules[name], _, _ = synthetic_raw(k=k, o=o, seed=50 * layer + i, zero=4)
        layers.append((layer, modules))
    root = tmp_path / "w3"
    write_w3_lut_artifacts(root, layers, num_layers=config.num_hidden_layers)
    return root, sha256_file(root / "manifest.json"), layers


def test_decoded_arm_installs_the_restored_weights(tmp_path):
    config = _config()
    root, sha, layers = _artifact(tmp_path, config)
    model = random_qwen3_model(config, device="cpu", dtype=torch.bfloat16, seed=6).eval()
    assert ppl.prepare_arm(model, "decoded_w3_bf16", artifact_root=root, expected_manifest_sha256=sha) is None
    for layer, modules in layers:
        for name, raw in modules.items():
            want = gd.restore_planar_w3(gd.convert_gptq_w3_to_planar(raw), dtype=torch.bfloat16)
            assert torch.equal(model.model.layers[layer].get_submodule(name).weight, want), (layer, name)
    with pytest.raises(ValueError, match="manifest drift"):
        ppl.prepare_arm(model, "decoded_w3_bf16", artifact_root=root, expected_manifest_sha256="0" * 64)


def test_command_line_dense_arms_and_resume(tmp_path):
    config = _config()
    root, sha, _ = _artifact(tmp_path, config)
    snapshot = tmp_path / "snapshot"
    random_qwen3_model(config, device="cpu", dtype=torch.bfloat16, seed=7).save_pretrained(snapshot)
    tokens = tmp_path / "tokens.safetensors"
    save_file({"tokens": torch.tensor(_tokens(40, seed=8), dtype=torch.int32)}, str(tokens))
    out = tmp_path / "run"

    def argv(output, arms=("original_bf16", "decoded_w3_bf16"), manifest=sha):
        return ["--snapshot-root", str(snapshot), "--token-artifact", str(tokens), "--sequence-length", "8",
                "--max-blocks", "3", "--w3-layout-root", str(root), "--w3-layout-manifest-sha256", manifest,
                "--output-dir", str(output), "--device", "cpu", "--arms", *arms]

    summary = ppl.main(argv(out))
    assert summary["status"] == "completed_pending_effect_size_review"
    assert set(summary["arms"]) == {"original_bf16", "decoded_w3_bf16"}
    assert all(a["scored_transition_count"] == 21 for a in summary["arms"].values())
    assert set(summary["comparisons"]) == {"decoded_w3_vs_original_bf16"}
    # the W3 weights change the model: the two arms' NLLs differ
    assert summary["arms"]["original_bf16"]["total_nll"] != summary["arms"]["decoded_w3_bf16"]["total_nll"]
    with pytest.raises(FileExistsError):
        ppl.main(argv(out))
    again = ppl.main(argv(out) + ["--resume"])
    assert again["arms"] == summary["arms"]
    record = json.loads((out / "arms" / "decoded_w3_bf16.json").read_text())
    # every arm records the kernel library's build contract key
    from marlin_style_fluxbin_amd.w3_lut_deployment import w3_lut_extension_build

    assert record["provenance"]["w3_kernel_build_cache_key"] == w3_lut_extension_build(256)[1]["cache_key"]
    kept = dict(record)
    record["provenance"] = dict(record["provenance"], w3_kernel_build_cache_key="0" * 64)
    (out / "arms" / "decoded_w3_bf16.json").write_text(json.dumps(record))
    with pytest.raises(ValueError, match="resumable"):
        ppl.main(argv(out) + ["--resume"])
    record = kept
    record["provenance"]["blocks_sha256"] = "0" * 64
    (out / "arms" / "decoded_w3_bf16.json").write_text(json.dumps(record))
    with pytest.raises(ValueError, match="resumable"):
        ppl.main(argv(out) + ["--resume"])
    with pytest.raises(ValueError, match="manifest drifted"):
        ppl.main(argv(tmp_path / "drift", manifest="0" * 64))
    # the packed arm needs a GPU: prepared decode refuses a CPU model loudly
    with pytest.raises(ValueError, match="CUDA"):
        ppl.main(argv(tmp_path / "packed", arms=("packed_w3_inline",)))
