"""CPU contract of the W3 LUT Linear API (``w3_lut_deployment``).

Ports the reference's CPU-runnable known answers:
* workspace shapes (``tests/test_w3_lut_correctness.py:23-29``);
* the frozen Qwen3-8B row-tile and route policies (``tests/test_w3_lut_adapter.py:56-85``);
* the module's constructor contract, dense fallback and fail-closed prepared
  binding (``tests/test_w3_lut_adapter.py:38-54,87-115``), with the reference's
  two route keys;
* the extension loader refusing the timing-only wrong-result build and the
  missing-GPU case.
"""
from __future__ import annotations

import pytest
import torch
from torch import nn

from marlin_style_fluxbin_amd import gptq_deployment as gd
from marlin_style_fluxbin_amd import w3_lut_deployment as wl
from marlin_style_fluxbin_amd.full_model_trial import packed_modules
from marlin_style_fluxbin_amd.qwen3 import QWEN3_LINEAR_MODULES
from tests.payloads import synthetic_raw


def tiny_layout(out_features=32, in_features=128):
    raw, _, _ = synthetic_raw(k=in_features, o=out_features)
    return gd.convert_gptq_w3_to_planar(raw, qzero_format=1)


def tiny_block():
    block = nn.Module()
    block.self_attn = nn.Module()
    block.mlp = nn.Module()
    for name in QWEN3_LINEAR_MODULES:
        parent, attribute = name.rsplit(".", 1)
        setattr(block.get_submodule(parent), attribute, nn.Linear(128, 32, bias=False))
    return block


def test_workspace_shape_known_answers():
    assert wl.workspace_shape(1024, 4096) == (32, 1024)
    assert wl.workspace_shape(1024, 4096, 4) == (8, 1024)
    assert wl.workspace_shape(1024, 4096, 32) == (1, 1024)
    assert wl.workspace_shape(4096, 12288, 2) == (48, 4096)
    assert wl.workspace_shape(12288, 4096, 3) == (11, 12288)
    for bad in ((1024, 4097), (1024, 4096, 0), (1024, 4096, 33), (0, 128), (65537, 128), (32, 32768)):
        with pytest.raises(ValueError):
            wl.workspace_shape(*bad)
    with pytest.raises(ValueError):
        wl.workspace_shape(1024, 4096, 1.0)


def test_shape_policy_is_frozen():
    assert wl.qwen3_row_tile(4096, 4096) == 256
    assert wl.qwen3_row_tile(1024, 4096) == 512
    assert wl.qwen3_row_tile(12288, 4096) == 1024
    assert wl.qwen3_row_tile(4096, 12288) == 1024
    with pytest.raises(ValueError):
        wl.qwen3_row_tile(32, 128)


def test_corrected_full_model_routes_are_frozen():
    expected = {(4096, 4096): (256, 1), (1024, 4096): (512, 1), (12288, 4096): (1024, 4), (4096, 12288): (1024, 2)}
    for shape, (row_tile, exact_gps) in expected.items():
        assert wl.qwen3_w3_route("fast_corrected", *shape) == {
            "row_tile": row_tile, "groups_per_split": 1, "arithmetic": "decoded_bf16"}
        assert wl.qwen3_w3_route("observed_exact", *shape) == {
            "row_tile": row_tile, "groups_per_split": exact_gps, "arithmetic": "decoded_bf16"}
        assert wl.qwen3_w3_route("structural", *shape) == {
            "row_tile": row_tile, "groups_per_split": 1, "arithmetic": "structural"}
    with pytest.raises(ValueError):
        wl.qwen3_w3_route("missing", 4096, 4096)
    with pytest.raises(ValueError):
        wl.qwen3_w3_route("structural", 32, 128)
    # a returned policy is a copy: editing it does not move the frozen table
    policy = wl.qwen3_w3_route("observed_exact", 12288, 4096)
    policy["groups_per_split"] = 99
    assert wl.qwen3_w3_route("observed_exact", 12288, 4096)["groups_per_split"] == 4


def test_linear_carries_explicit_arithmetic_and_split_policy():
    module = wl.PackedW3Linear(tiny_layout(), row_tile=256, groups_per_split=1, arithmetic="decoded_bf16",
                               route="fast_corrected")
    assert (module.arithmetic, module.groups_per_split, module.route) == ("decoded_bf16", 1, "fast_corrected")
    assert not module.uses_table_route  # one group per split: the one-launch MFMA kernel
    assert not wl.PackedW3Linear(tiny_layout(), row_tile=256).uses_table_route
    two_groups = {"planes": gd.planar_from_codes(torch.zeros(256, 8, dtype=torch.uint8)),
                  "scales": torch.ones(2, 8, dtype=torch.bfloat16), "perm": torch.arange(256, dtype=torch.int16)}
    two = wl.PackedW3Linear(two_groups, row_tile=256, groups_per_split=2, arithmetic="decoded_bf16",
                            route="observed_exact")
    assert two.uses_table_route  # a K split: the reference's split contract on the table kernel
    assert wl.PackedW3Linear(tiny_layout(), row_tile=256, groups_per_split=1).route_counts == {
        "packed_m1": 0, "dense_fallback": 0}
    with pytest.raises(ValueError):
        wl.PackedW3Linear(tiny_layout(), row_tile=256, arithmetic="missing")
    with pytest.raises(ValueError):
        wl.PackedW3Linear(tiny_layout(), row_tile=128)
    with pytest.raises(ValueError):
        wl.PackedW3Linear(tiny_layout(), row_tile=256, groups_per_split=2)  # K = 128 has one group
    with pytest.raises(ValueError):
        wl.PackedW3Linear(tiny_layout(), row_tile=256, fallback="maybe")
    with pytest.raises(ValueError):
        wl.PackedW3Linear(tiny_layout(), row_tile=256, max_packed_rows=9)
    fp16 = tiny_layout()
    fp16["scales"] = fp16["scales"].half()
    with pytest.raises(ValueError, match="bf16 scales"):
        wl.PackedW3Linear(fp16, row_tile=256, arithmetic="decoded_bf16")


def test_dense_fallback_matches_restored_weight_with_reference_route_keys():
    layout = tiny_layout()
    module = wl.PackedW3Linear(layout, fallback="dense", row_tile=256)
    x = torch.randn(2, 128, dtype=torch.bfloat16)
    with torch.inference_mode():
        actual = module(x)
        expected = torch.nn.functional.linear(x, gd.restore_planar_w3(layout))
    assert torch.equal(actual, expected)
    assert module.route_counts == {"packed_m1": 0, "dense_fallback": 1}
    assert module.last_route == "dense_fallback"
    with torch.inference_mode():
        module(torch.randn(1, 3, 128, dtype=torch.bfloat16))   # a 3-token prompt: dense, as in the reference
    assert module.route_counts == {"packed_m1": 0, "dense_fallback": 2}


def test_strict_cpu_and_prepared_binding_fail_closed():
    module = wl.PackedW3Linear(tiny_layout(), row_tile=256)
    with torch.inference_mode(), pytest.raises(ValueError, match="unsupported input"):
        module(torch.randn(1, 128, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="prepared decode requires"):
        module.bind_prepared_decode(torch.bfloat16)
    with pytest.raises(ValueError, match="FP16/BF16"):
        module.bind_prepared_decode(torch.float32)
    with pytest.raises(RuntimeError, match="no_grad"):
        module(torch.randn(1, 128, dtype=torch.bfloat16))
    with torch.inference_mode(), pytest.raises(ValueError, match=r"\[\.\.\.,K\]"):
        module(torch.randn(1, 64, dtype=torch.bfloat16))


def test_module_buffers_and_layout_round_trip():
    layout = tiny_layout()
    layout["zeros"] = torch.full((1, 32), 4, dtype=torch.uint8)
    module = wl.PackedW3Linear(layout, row_tile=256)
    assert set(module.layout()) == {"planes", "scales", "perm", "zeros"}
    for name, value in layout.items():
        assert torch.equal(module.layout()[name], value)
        assert module.layout()[name].data_ptr() != value.data_ptr()  # the module owns copies
    state = module.state_dict()
    assert {"planes", "scales", "perm", "zeros"} <= set(state)


def test_complete_block_replacement_and_discovery():
    layout = tiny_layout()
    payload = {f"{name}.{field}": value.clone() for name in QWEN3_LINEAR_MODULES for field, value in layout.items()}
    block = tiny_block()
    names = wl.replace_w3_block_linears(block, payload, fallback="dense", row_tile_by_shape={(32, 128): 256})
    assert names == list(QWEN3_LINEAR_MODULES)
    assert len(packed_modules(block)) == 7
    assert all(isinstance(m, wl.PackedW3Linear) for m in packed_modules(block).values())


def test_block_replacement_validates_before_mutating():
    layout = tiny_layout()
    payload = {f"{name}.{field}": value.clone() for name in QWEN3_LINEAR_MODULES for field, value in layout.items()}
    payload["mlp.down_proj.perm"] = torch.zeros(128, dtype=torch.int16)  # not a bijection
    block = tiny_block()
    before = {name: block.get_submodule(name) for name in QWEN3_LINEAR_MODULES}
    with pytest.raises(ValueError):
        wl.replace_w3_block_linears(block, payload, fallback="dense", row_tile_by_shape={(32, 128): 256})
    assert all(block.get_submodule(name) is before[name] for name in QWEN3_LINEAR_MODULES)
    payload = {f"{name}.{field}": value.clone() for name in QWEN3_LINEAR_MODULES for field, value in layout.items()}
    del payload["mlp.up_proj.scales"]
    with pytest.raises(ValueError, match="seven complete"):
        wl.replace_w3_block_linears(block, payload, fallback="dense", row_tile_by_shape={(32, 128): 256})
    with pytest.raises(ValueError, match="row-tile policy"):
        payload = {f"{n}.{f}": v.clone() for n in QWEN3_LINEAR_MODULES for f, v in layout.items()}
        wl.replace_w3_block_linears(block, payload, fallback="dense")


def test_extension_loader_contract(monkeypatch):
    wl.load_w3_lut_extension.cache_clear()
    try:
        with pytest.raises(ValueError):
            wl.load_w3_lut_extension(128)
        with pytest.raises(ValueError, match="probe"):
            wl.load_w3_lut_extension(256, uniform_index_probe=True)
        monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
        with pytest.raises(RuntimeError, match="no CPU substitute"):
            wl.load_w3_lut_extension(256)
    finally:
        wl.load_w3_lut_extension.cache_clear()


def test_extension_build_contract(monkeypatch, tmp_path):
    """w3_lut_extension_build (reference w3_lut_deployment.py:49-68): one contract
    for every row tile, a key over the canonical fields that follows source bytes
    and flags but not documentation, and the reference's refusals."""
    import hashlib
    import json
    import shutil
    from pathlib import Path

    from marlin_style_fluxbin_amd import build

    with pytest.raises(ValueError, match="row_tile"):
        wl.w3_lut_extension_build(128)
    with pytest.raises(ValueError, match="probe"):
        wl.w3_lut_extension_build(256, uniform_index_probe=True)
    contracts = [wl.w3_lut_extension_build(r)[1] for r in wl.EXPERIMENTAL_ROW_TILES]
    assert all(c == contracts[0] for c in contracts)
    kwargs, contract = wl.w3_lut_extension_build(256)
    assert kwargs["row_tile"] == 256 and kwargs["library"].endswith("libfluxbin_amd.so")
    names = {s["name"] for s in contract["sources"]}
    assert {"capi.hip", "w3_mfma.hip", "common.h", "fluxbin_amd.h"} <= names
    assert set(contract["compile_sources"]) == {p.name for p in build.compile_units()}
    assert "w3_lut.hip" in contract["content_dependencies"]  # included by its instantiation units
    keyed = {k: v for k, v in contract.items()
             if k not in ("cache_key", "compile_sources", "content_dependencies", "library_sha256")}
    canonical = json.dumps(keyed, sort_keys=True, separators=(",", ":")).encode()
    assert contract["cache_key"] == hashlib.sha256(canonical).hexdigest()

    # a copy of the tree: one source byte or one flag moves the key, a note does not
    pkg = tmp_path / "pkg"
    shutil.copytree(build.CSRC, pkg / "csrc", ignore=shutil.ignore_patterns("*.o"))
    (tmp_path / "include").mkdir()
    shutil.copy(build.PACKAGE.parent / "include" / "fluxbin_amd.h", tmp_path / "include")
    monkeypatch.setattr(build, "CSRC", pkg / "csrc")
    monkeypatch.setattr(build, "PACKAGE", pkg)
    base = wl.w3_lut_extension_build(512)[1]["cache_key"]
    assert base == contract["cache_key"]
    (pkg / "NOTES.md").write_text("documentation only\n")
    assert wl.w3_lut_extension_build(512)[1]["cache_key"] == base
    src = pkg / "csrc" / "norms.hip"
    src.write_bytes(src.read_bytes() + b"\n")
    edited = wl.w3_lut_extension_build(512)[1]["cache_key"]
    assert edited != base
    # a header is a content dependency: it moves the key but is not a compile source
    header = pkg / "csrc" / "common.h"
    header.write_bytes(header.read_bytes() + b"\n")
    kwargs2, contract2 = wl.w3_lut_extension_build(512)
    assert contract2["cache_key"] not in (base, edited)
    assert {Path(s).name for s in kwargs2["sources"]} == set(contract2["compile_sources"])
    assert "common.h" in contract2["content_dependencies"]
    edited = contract2["cache_key"]
    assert "git" not in contract2
    monkeypatch.setattr(build, "HIPCC_FLAGS", build.HIPCC_FLAGS + ["-DFX_EXTRA=1"])
    assert wl.w3_lut_extension_build(512)[1]["cache_key"] not in (base, edited)


def test_engine_backends_for_w3_and_hybrid_formats():
    from marlin_style_fluxbin_amd import deployment as d
    from marlin_style_fluxbin_amd.engine_interface import M1Backend, W3Backend, backend_for_format

    raw, codes, _ = synthetic_raw()
    backend = backend_for_format(gd.REFERENCE_FORMAT)
    assert isinstance(backend, W3Backend) and backend.contract.target_arch == "gfx950"
    layout = backend.convert(raw)
    assert torch.equal(gd.decode_planar_w3_codes(layout), codes)
    assert gd.layout_storage(layout)["format"] == backend.contract.format
    zero3, _, _ = synthetic_raw(zero=3)
    with_zeros = W3Backend(allow_zeros=True, scale_dtype=torch.float16)
    converted = with_zeros.convert(zero3)
    assert converted["scales"].dtype == torch.float16 and "zeros" in converted
    assert gd.layout_storage(converted)["format"] == with_zeros.contract.format == gd.FORMAT
    assert isinstance(backend_for_format(d.PLANAR_FORMAT), M1Backend)
    assert backend_for_format(d.PLANAR_FORMAT).kernel == "v5_p1024"
    assert backend_for_format(d.FORMAT).kernel == "v1"
    with pytest.raises(ValueError):
        backend_for_format("unknown-format")


def test_route_counter_reset_keeps_the_small_m_key():
    """The trial and session resets zero every counter a module keeps: a module
    that opts into 2..8-row inputs keeps ``packed_small_m`` across a reset (a
    reset to the two reference keys made its next small-M call a KeyError), and
    the route check accepts a short prompt served on that route."""
    from marlin_style_fluxbin_amd.full_model_trial import _fallback_policy, validate_routes

    module = wl.PackedW3Linear(tiny_layout(), row_tile=256, max_packed_rows=8)
    module._count("packed_small_m")
    with _fallback_policy({"m": module}):
        assert module.route_counts == {"packed_m1": 0, "dense_fallback": 0, "packed_small_m": 0}
        module._count("packed_small_m")
        module._count("packed_m1")
    plain = wl.PackedW3Linear(tiny_layout(), row_tile=256)
    plain.reset_route_counts()
    assert plain.route_counts == {"packed_m1": 0, "dense_fallback": 0}
    plain._count("dense_fallback")
    plain._count("packed_m1")
    trace = {"routes": {"a": dict(module.route_counts), "b": dict(plain.route_counts)}}
    assert validate_routes(trace, expected_linears=2, steps=1)
    trace["routes"]["a"]["dense_fallback"] = 1  # the prompt served twice
    assert not validate_routes(trace, expected_linears=2, steps=1)
