"""CPU tests of the on-disk W3 artifact: converter, manifest, hash-bound loader and
the model installer (reference ``w3_lut_artifacts.py:14-118`` and
``scripts/prepare_qwen3_8b_w3_lut_artifacts.py:145-294``).

A two-layer Qwen3 with small shapes gets raw GPTQ int3 tensors per Linear (the
reference's ``synthetic_raw`` generator, desc_act permutations); the artifact is
written, loaded back bit for bit, refused after any drift (manifest bytes, a layer
file's bytes, the manifest's gate), and installed so that the model's dense
fallback equals ``F.linear`` on the restored weights.
"""
from __future__ import annotations

import json

import pytest
import torch
from safetensors.torch import save_file

from marlin_style_fluxbin_amd import gptq_deployment as gd
from marlin_style_fluxbin_amd.qwen3 import QWEN3_LINEAR_MODULES, expected_qwen3_linear_shape, qwen3_config
from marlin_style_fluxbin_amd.w3_lut_artifacts import (load_w3_lut_layer, main, replace_w3_model_linears,
                                                        sha256_file, write_w3_lut_artifacts)
from marlin_style_fluxbin_amd.w3_lut_deployment import PackedW3Linear
from tests.payloads import synthetic_raw


def _config():
    return qwen3_config(hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
                        num_key_value_heads=2, head_dim=64, vocab_size=96, max_position_embeddings=64)


def _source(config, zero=4):
    layers = []
    for layer in range(config.num_hidden_layers):
        modules = {}
        for i, name in enumerate(QWEN3_LINEAR_MODULES):
            o, k = expected_qwen3_linear_shape(config.to_dict(), name)
            raw, _, _ = synthetic_raw(k=k, o=o, seed=100 * layer + i, zero=zero)
            modules[name] = raw
        layers.append((layer, modules))
    return layers


def test_artifact_round_trip_and_drift_refusals(tmp_path):
    config = _config()
    source = _source(config)
    out = tmp_path / "artifact"
    manifest = write_w3_lut_artifacts(out, source, num_layers=2)
    assert manifest["format"] == gd.REFERENCE_FORMAT and manifest["layers"] == 2
    assert manifest["canonical_semantics_gate"]["inspected_linears"] == 14
    assert not (tmp_path / "artifact.incomplete").exists()
    sha = sha256_file(out / "manifest.json")
    for layer, modules in source:
        tensors, entry = load_w3_lut_layer(out, layer, expected_manifest_sha256=sha)
        assert entry["path"] == f"payloads/layer-{layer:03d}.safetensors"
        for name, raw in modules.items():
            want = gd.convert_gptq_w3_to_planar(raw, qzero_format=1)
            for field, value in want.items():
                assert torch.equal(tensors[f"{name}.{field}"], value), (layer, name, field)
    with pytest.raises(ValueError, match="manifest drift"):
        load_w3_lut_layer(out, 0, expected_manifest_sha256="0" * 64)
    with pytest.raises(ValueError, match="outside"):
        load_w3_lut_layer(out, 2, expected_manifest_sha256=sha)
    # one flipped payload byte: refused by hash
    layer_file = out / "payloads" / "layer-001.safetensors"
    blob = bytearray(layer_file.read_bytes())
    blob[-1] ^= 1
    layer_file.write_bytes(bytes(blob))
    with pytest.raises(ValueError, match="hash/size drift"):
        load_w3_lut_layer(out, 1, expected_manifest_sha256=sha)
    load_w3_lut_layer(out, 0, expected_manifest_sha256=sha)  # the other layer still loads
    # a manifest whose gate drifted is refused even when its hash is the expected one
    data = json.loads((out / "manifest.json").read_text())
    data["canonical_semantics_gate"]["inspected_linears"] = 13
    (out / "manifest.json").write_text(json.dumps(data))
    with pytest.raises(ValueError, match="gate"):
        load_w3_lut_layer(out, 0, expected_manifest_sha256=sha256_file(out / "manifest.json"))
    with pytest.raises(FileExistsError):
        write_w3_lut_artifacts(out, source, num_layers=2)


def test_inventory_drift_is_refused(tmp_path):
    config = _config()
    out = tmp_path / "artifact"
    write_w3_lut_artifacts(out, _source(config), num_layers=2)
    from safetensors.torch import load_file

    path = out / "payloads" / "layer-000.safetensors"
    tensors = load_file(str(path))
    del tensors["mlp.down_proj.perm"]
    save_file(tensors, str(path))
    data = json.loads((out / "manifest.json").read_text())
    for entry in data["files"]:
        if entry["layer"] == 0:
            entry["bytes"], entry["sha256"] = path.stat().st_size, sha256_file(path)
    (out / "manifest.json").write_text(json.dumps(data))
    with pytest.raises(ValueError, match="inventory drift"):
        load_w3_lut_layer(out, 0, expected_manifest_sha256=sha256_file(out / "manifest.json"))


def test_gate_runs_before_any_write(tmp_path):
    config = _config()
    source = _source(config, zero=3)
    with pytest.raises(ValueError, match="decoded zero=4"):
        write_w3_lut_artifacts(tmp_path / "a", source, num_layers=2)
    assert not (tmp_path / "a").exists() and not (tmp_path / "a.incomplete").exists()
    with pytest.raises(ValueError, match="every Linear"):
        write_w3_lut_artifacts(tmp_path / "b", source[:1], num_layers=2, allow_zeros=True)
    manifest = write_w3_lut_artifacts(tmp_path / "c", source, num_layers=2, allow_zeros=True,
                                      scale_dtype=torch.float16)
    assert manifest["format"] == gd.FORMAT and manifest["canonical_semantics_gate"]["decoded_zero_unique"] == [3]
    tensors, _ = load_w3_lut_layer(tmp_path / "c", 1, expected_manifest_sha256=sha256_file(tmp_path / "c/manifest.json"))
    assert tensors["self_attn.q_proj.zeros"].unique().tolist() == [3]
    assert tensors["self_attn.q_proj.scales"].dtype == torch.float16


def test_decoded_bf16_check_and_installer(tmp_path):
    from marlin_style_fluxbin_amd.qwen3 import random_qwen3_model

    config = _config()
    source = _source(config)
    decoded = {f"model.layers.{layer}.{name}": gd.restore_planar_w3(gd.convert_gptq_w3_to_planar(raw))
               for layer, modules in source for name, raw in modules.items()}
    out = tmp_path / "artifact"
    manifest = write_w3_lut_artifacts(out, source, num_layers=2, decoded_bf16=decoded)
    assert all(m["decoded_bf16_bitwise_exact"] for m in manifest["modules"])
    bad = dict(decoded)
    key = "model.layers.1.mlp.up_proj"
    bad[key] = bad[key].clone()
    bad[key][0, 0] += 1
    with pytest.raises(RuntimeError, match="bitwise round trip"):
        write_w3_lut_artifacts(tmp_path / "bad", source, num_layers=2, decoded_bf16=bad)
    assert (tmp_path / "bad.incomplete" / "failure.json").exists()

    model = random_qwen3_model(config, device="cpu", dtype=torch.bfloat16, seed=1)
    sha = sha256_file(out / "manifest.json")
    record = replace_w3_model_linears(model, out, expected_manifest_sha256=sha, allow_prefill_fallback=True)
    assert record["linear_count"] == 14 and record["status"] == "installed_not_validated"
    layer = model.model.layers[1]
    module = layer.get_submodule("mlp.up_proj")
    assert isinstance(module, PackedW3Linear)
    x = torch.randn(3, 256, generator=torch.Generator().manual_seed(0)).to(torch.bfloat16)
    with torch.inference_mode():
        assert torch.equal(module(x), torch.nn.functional.linear(x, decoded[key]))
    wrong = random_qwen3_model(qwen3_config(hidden_size=256, intermediate_size=384, num_hidden_layers=2,
                                            num_attention_heads=4, num_key_value_heads=2, head_dim=64,
                                            vocab_size=96), device="cpu", dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="drift|mismatch"):
        replace_w3_model_linears(wrong, out, expected_manifest_sha256=sha)
    assert isinstance(wrong.model.layers[0].mlp.up_proj, torch.nn.Linear)  # nothing installed


def test_command_line_converter(tmp_path):
    config = _config()
    root = tmp_path / "gptq"
    root.mkdir()
    tensors = {f"model.layers.{layer}.{name}.{field}": value
               for layer, modules in _source(config) for name, raw in modules.items() for field, value in raw.items()}
    save_file(tensors, str(root / "model.safetensors"))
    main(["prepare", "--gptq-root", str(root), "--output-dir", str(tmp_path / "out")])
    manifest = json.loads((tmp_path / "out" / "manifest.json").read_text())
    assert manifest["layers"] == 2 and len(manifest["files"]) == 2
