"""CPU tests of the two-base hybrid drop-in API (``deployment``, ``packing``,
``evaluation``, ``engine_interface``), after the reference's own tests
(``tests/test_deployment.py``, ``test_planar_layout.py``, ``test_packing.py``):
conversions, fail-closed contracts, the dense fallback and the block adapter, all
checked against the numpy oracle (``oracle.two_base``)."""
import copy

import numpy as np
import pytest
import torch
from torch import nn

from marlin_style_fluxbin_amd import deployment as d
from marlin_style_fluxbin_amd.engine_interface import M1Backend
from marlin_style_fluxbin_amd.evaluation import materialize_hybrid_s8_weight
from marlin_style_fluxbin_amd.packing import pack_two_bases, unpack_two_bases
from oracle import bf16, two_base as tb


def payload(o=7, g=3, seed=19):
    return {k: torch.from_numpy(v) for k, v in tb.make_hybrid_payload(o, g, seed=seed).items()}


def np_payload(p):
    return {k: v.numpy() for k, v in p.items()}


def test_packing_kat_round_trip_and_oracle():
    bases = torch.tensor([[[-1, 1, -1, 1]], [[-1, -1, 1, 1]]], dtype=torch.int8)
    assert int(pack_two_bases(bases).item()) == 0b11100100
    g = torch.Generator().manual_seed(31)
    bases = torch.where(torch.rand(2, 7, 20, generator=g) < 0.5, -1, 1).to(torch.int8)
    codes = pack_two_bases(bases)
    assert codes.shape == (7, 5) and torch.equal(unpack_two_bases(codes), bases)
    assert np.array_equal(codes.numpy(), tb.pack_two_bases(bases.numpy()))
    with pytest.raises(ValueError):
        pack_two_bases(torch.zeros(2, 3, 8, dtype=torch.int8))


def test_planes_all_65536_words():
    word = torch.arange(65536, dtype=torch.int32)
    inter = torch.stack((word & 255, word >> 8), dim=-1).to(torch.uint8)
    planes = d._to_planes(inter)
    for basis in range(2):
        expected = torch.zeros_like(word)
        for k in range(8):
            expected |= ((word >> (2 * k + basis)) & 1) << k
        assert torch.equal(planes[:, basis, 0], expected.to(torch.uint8))
    assert torch.equal(d._from_planes(planes), inter)


@pytest.mark.parametrize("o,g", [(1, 1), (7, 3), (17, 10)])
def test_conversion_lossless_and_matches_oracle(o, g):
    p = payload(o, g)
    for kernel in ("v1", "v5_p1024"):
        q = d.convert_artifact(p, kernel=kernel)
        want = tb.convert_artifact(np_payload(p), planar=kernel in d.PLANAR_KERNELS)
        for key in d.LAYOUT_FIELDS:
            assert np.array_equal(q[key].numpy(), want[key]), key
        back = d.restore_artifact(q)
        for key in d.FIELDS:
            assert torch.equal(back[key], p[key]), key
        assert d.layout_format(q) == (d.PLANAR_FORMAT if kernel in d.PLANAR_KERNELS else d.FORMAT)
    saved = q["rows"].clone()
    p["global_row_scales"].zero_()  # conversion is independent of later source changes
    assert torch.equal(saved, q["rows"])


def test_decode_layout_matches_oracle_in_every_dtype():
    p = payload(9, 2, seed=4)
    w32 = tb.materialize_hybrid(np_payload(p))
    for kernel in ("v1", "v5_p256"):
        layout = d.convert_artifact(p, kernel=kernel)
        assert np.array_equal(d.decode_layout(layout, torch.float32).numpy(), w32)
        assert np.array_equal(d.decode_layout(layout, torch.bfloat16).float().numpy(), bf16.round_bf16(w32))
        assert np.array_equal(d.decode_layout(layout, torch.float16).float().numpy(), bf16.round_f16(w32))
    w = materialize_hybrid_s8_weight(**p, group_size=128, columns_per_group=8, device="cpu",
                                     output_dtype=torch.float32)
    assert np.array_equal(w.numpy(), w32)


def test_fail_closed_payload_contract():
    for field, mutate in (
        ("refinement_indices", lambda x: x.fill_(128)),
        ("refinement_indices", lambda x: x.zero_()),
        ("global_row_scales", lambda x: x.fill_(float("nan"))),
        ("global_column_scales", lambda x: x.half()),
        ("refinement_sign_codes", lambda x: x.long()),
    ):
        p = payload()
        p[field] = mutate(p[field])
        with pytest.raises(ValueError):
            d.convert_artifact(p)
    with pytest.raises(ValueError):
        d.convert_artifact({})
    with pytest.raises(ValueError):
        d.convert_artifact(payload(), kernel="v9")


def test_workspace_shapes_and_backend_contract():
    assert d.workspace_shape(17, 384, 4, kernel="v4") == (3 * 272 + 17,)
    assert d.workspace_shape(17, 384, 4) == (1, 17)
    assert d.workspace_shape(12288, 4096) == (4, 12288)
    for bad in ((17, 384, 0), (0, 384, 8), (17, 200, 8), (17, 384, 2000)):
        with pytest.raises(ValueError):
            d.workspace_shape(*bad)
    backend = M1Backend(kernel="v5_p512")
    assert backend.contract.format == d.PLANAR_FORMAT and backend.contract.arithmetic == "factored_fp32_v1"
    assert backend.convert(payload(17, 3))["codes"].shape == (3, 17, 2, 16)
    assert M1Backend(kernel="v4_late").workspace_shape(17, 384) == (3 * 272 + 17,)
    assert M1Backend().contract.format == d.FORMAT
    with pytest.raises(ValueError):
        M1Backend(groups_per_split=0)
    rec = d.conversion_record(payload(17, 3), d.convert_artifact(payload(17, 3), kernel="v5_p1024"))
    assert rec["format"] == d.PLANAR_FORMAT
    legacy = d.conversion_record(payload(17, 3), d.convert_artifact(payload(17, 3)))
    assert rec["layout_bytes"] == legacy["layout_bytes"]


def test_dense_fallback_routes_and_shape_preservation():
    p = payload()
    x = torch.randn(1, 2, 384)
    strict = d.PackedHybridLinear(p)
    with torch.inference_mode():
        with pytest.raises(ValueError):
            strict(x)
        layer = d.PackedHybridLinear(p, fallback="dense")
        y = layer(x)
        want = torch.from_numpy(x.numpy().astype(np.float64) @ tb.materialize_hybrid(np_payload(p)).astype(np.float64).T)
        assert y.shape == (1, 2, 7) and torch.allclose(y.double(), want, rtol=1e-5, atol=1e-5)
        assert layer.last_route == "dense_fallback" and layer.route_counts == {"packed_m1": 0, "dense_fallback": 1}
    with pytest.raises(RuntimeError):
        layer(x)  # grad enabled
    layer.half()
    with torch.inference_mode(), pytest.raises(ValueError):
        layer(x.half())
    planar = d.PackedHybridLinear(p, kernel="v5_p1024", fallback="dense")
    assert planar.codes.shape == (3, 7, 2, 16) and planar._codes_planar is None
    with torch.inference_mode():
        xb = torch.randn(2, 384, dtype=torch.bfloat16)
        assert torch.equal(planar(xb), xb @ d.decode_layout(d.convert_artifact(p)).T)


def test_block_adapter_validates_before_mutation():
    from marlin_style_fluxbin_amd.qwen3 import QWEN3_LINEAR_MODULES

    block = nn.Module()
    block.self_attn = nn.Module()
    block.mlp = nn.Module()
    layer_payload = {}
    for name in QWEN3_LINEAR_MODULES:
        parent, attr = name.split(".")
        setattr(block.get_submodule(parent), attr, nn.Linear(128, 7, bias=False))
        layer_payload.update({name + "." + k: v for k, v in payload(7, 1).items()})
    broken = dict(layer_payload)
    broken.pop(next(iter(broken)))
    with pytest.raises(ValueError):
        d.replace_block_linears(block, broken)
    assert all(isinstance(block.get_submodule(n), nn.Linear) for n in QWEN3_LINEAR_MODULES)
    assert len(d.replace_block_linears(block, layer_payload, fallback="dense")) == 7
    with torch.inference_mode():
        assert tuple(block.self_attn.q_proj(torch.zeros(1, 128)).shape) == (1, 7)


def test_real_qwen3_block_with_dense_fallback_is_bit_equal():
    from transformers import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3DecoderLayer, Qwen3RotaryEmbedding

    from marlin_style_fluxbin_amd.qwen3 import QWEN3_LINEAR_MODULES

    config = Qwen3Config(hidden_size=128, intermediate_size=256, num_hidden_layers=1, num_attention_heads=4,
                         num_key_value_heads=2, head_dim=32)
    config._attn_implementation = "sdpa"
    torch.manual_seed(0)
    block = Qwen3DecoderLayer(config, 0).to(torch.bfloat16).eval()
    layer_payload = {}
    with torch.no_grad():
        for i, name in enumerate(QWEN3_LINEAR_MODULES):
            linear = block.get_submodule(name)
            p = payload(linear.out_features, linear.in_features // 128, seed=i)
            w = bf16.round_bf16(tb.materialize_hybrid(np_payload(p)))
            linear.weight.copy_(torch.from_numpy(w).to(torch.bfloat16))
            layer_payload.update({name + "." + k: v for k, v in p.items()})
    candidate = copy.deepcopy(block)
    d.replace_block_linears(candidate, layer_payload, fallback="dense")
    rotary = Qwen3RotaryEmbedding(config)
    x = torch.randn(1, 1, 128, dtype=torch.bfloat16)
    pos = torch.zeros(1, 1, dtype=torch.long)
    with torch.inference_mode():
        kwargs = {"position_ids": pos, "position_embeddings": rotary(x, pos), "use_cache": False}
        out_ref = block(x, **kwargs)
        out_new = candidate(x, **kwargs)
        out_ref = out_ref[0] if isinstance(out_ref, tuple) else out_ref
        out_new = out_new[0] if isinstance(out_new, tuple) else out_new
        assert torch.equal(out_ref, out_new)
    assert all(m.rows.dtype == torch.float32 for m in candidate.modules() if isinstance(m, d.PackedHybridLinear))


@pytest.mark.parametrize("o,g", [(1, 1), (7, 3), (33, 4)])
@pytest.mark.parametrize("kernel", ["v1", "v5_p512"])
def test_structural_reference_matches_oracle(o, g, kernel):
    """factored_reference.structural_reference (reference factored_reference.py:8-42)
    on interleaved and planar layouts against the numpy oracle, which the oracle's
    own tests pin to an independent factored dot."""
    from marlin_style_fluxbin_amd.factored_reference import structural_reference

    p = payload(o, g, seed=o + g)
    layout = d.convert_artifact(p, kernel=kernel)
    x = torch.randn(1, 128 * g, generator=torch.Generator().manual_seed(g), dtype=torch.float64)
    got = structural_reference(x, layout)
    want = tb.structural_reference(x.numpy(), {k: v.numpy() for k, v in layout.items()})
    assert got.dtype == torch.float64 and got.shape == (1, o)
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-12, atol=1e-12)
    # its own bf16 rounding passes the gate; the bf16-weight dense product is a
    # different (rounded-weight) result (reference tests/test_factored_reference.py:21-24)
    from marlin_style_fluxbin_amd.factored_reference import structural_gate

    assert structural_gate(got.to(torch.bfloat16), got)["passed"]
    if o * g >= 21:
        legacy = x @ d.decode_layout(layout, torch.bfloat16).double().t()
        assert float((got - legacy).abs().max()) > 1e-5
    with pytest.raises(ValueError, match="G\\*128"):
        structural_reference(x[:, :64], layout)


def test_structural_reference_known_answer():
    """All signs +1, unit scales: every main weight is 2; the refinement (signs +1,
    row scales 1 and 2, column scale 1) adds 3 at its columns."""
    from marlin_style_fluxbin_amd.factored_reference import structural_reference

    o = 3
    layout = {
        "codes": torch.full((1, o, 32), 0xFF, dtype=torch.uint8),
        "rows": torch.ones(1, o, 2), "columns": torch.ones(1, 128, 2),
        "indices": torch.tensor([[0, 5, 9, 40, 64, 77, 100, 127]], dtype=torch.int16),
        "sparse_codes": torch.full((1, o, 2), 0xFF, dtype=torch.uint8),
        "sparse_rows": torch.tensor([[[1.0, 2.0]] * o]), "sparse_columns": torch.ones(1, 8, 2),
    }
    x = torch.zeros(1, 128, dtype=torch.float64)
    x[0, 5], x[0, 6] = 1.0, 10.0  # a refined and an unrefined column
    y = structural_reference(x, layout)
    assert torch.equal(y, torch.full((1, o), 2.0 * 1 + 3.0 * 1 + 2.0 * 10, dtype=torch.float64))


def test_structural_gate_thresholds():
    """structural_gate: bf16 outputs within 0.02 (rms + |e|) elementwise and NRMSE
    0.005 pass; fp32 outputs keep numerical_gate's 0.002 bars; the record names the
    reference."""
    from marlin_style_fluxbin_amd.factored_reference import REFERENCE, structural_gate

    e = torch.linspace(-1, 1, 64, dtype=torch.float64)[None]
    rms = float(e.square().mean().sqrt())
    ok = structural_gate((e * (1 + 2e-3)).to(torch.bfloat16), e)
    assert ok["passed"] and ok["reference"] == REFERENCE and ok["normalized_rmse_limit"] == 0.005
    bad = e.clone()
    bad[0, 3] += 0.05 * (rms + abs(float(e[0, 3])))
    assert not structural_gate(bad.to(torch.bfloat16), e)["passed"]
    spread = structural_gate((e * 1.008).to(torch.bfloat16), e)  # NRMSE 0.008 > 0.005
    assert not spread["passed"]
    f32 = structural_gate((e * (1 + 2e-3)).float(), e)
    assert not f32["passed"] and f32["elementwise_tolerance_factor"] == 0.002
    assert not structural_gate(torch.full_like(e, float("nan")).to(torch.bfloat16), e)["passed"]


def test_evaluation_hashes_and_atomic_json(tmp_path):
    """evaluation.sha256_file / sha256_token_sequences / atomic_json (reference
    evaluation.py:20-45,205-212): the token framing is a big-endian uint64 length
    then big-endian int64 tokens per sequence; the file hash is the plain digest."""
    import hashlib
    import json
    import struct

    from marlin_style_fluxbin_amd import evaluation as ev

    framed = struct.pack(">Q", 2) + struct.pack(">qq", 1, -2) + struct.pack(">Q", 0)
    assert ev.sha256_token_sequences([[1, -2], []]) == hashlib.sha256(framed).hexdigest()
    target = tmp_path / "sub" / "record.json"
    ev.atomic_json(target, {"b": [1, 2], "a": 0.5})
    assert json.loads(target.read_text()) == {"a": 0.5, "b": [1, 2]}
    assert target.read_text().startswith('{\n  "a"') and not list(target.parent.glob(".*tmp*"))
    assert ev.sha256_file(target) == hashlib.sha256(target.read_bytes()).hexdigest()
