"""CPU checks of host helpers the benchmarks and loaders lean on: the W3 RTN
quantizer (config 3's weights), the rank-one layout contract, the tensor hash,
the Qwen3-8B shape table and the GPU-only guards of the HIP entry points."""
import hashlib
import json

import numpy as np
import pytest
import torch

from marlin_style_fluxbin_amd import _lib
from marlin_style_fluxbin_amd.deployment import load_extension
from marlin_style_fluxbin_amd.evaluation import tensor_sha256
from marlin_style_fluxbin_amd.qwen3 import qwen3_8b_linear_shapes, quantize_w3_rtn
from marlin_style_fluxbin_amd.two_base import validate_rank_one
from oracle import w3
from tests.payloads import oracle_layout


def _dequant(layout):
    """Dense [O, K] float64 weight of a planar layout through the oracle."""
    k = layout["planes"].shape[0] * 128
    return w3.matvec_exact(np.eye(k), oracle_layout(layout)).T


@pytest.mark.parametrize("zeros", [True, False])
def test_rtn_quantizer_round_trip(zeros):
    """Codes in [0, 7]; every weight within half a step of its dequantized value
    (a step = the group's scale), plus what the scale's fp16 rounding moves the
    ends of the range (7 steps at 2^-11 relative: 0.0034 of a step) when the
    zero-point rounds the range toward one end; the symmetric form stores no
    zero-points (z = 4) and clamps the top of its range at 3 steps."""
    gen = torch.Generator().manual_seed(3)
    w = torch.randn(48, 384, generator=gen) * 0.02
    w[5, 130] = 0.3  # an outlier widens one group's range
    layout = quantize_w3_rtn(w, zeros=zeros)
    assert ("zeros" in layout) == zeros
    assert layout["scales"].dtype == torch.float16 and layout["scales"].shape == (3, 48)
    codes = w3.codes_from_planar(layout["planes"].numpy())
    assert codes.min() >= 0 and codes.max() <= 7
    deq = _dequant(layout)
    step = np.repeat(layout["scales"].float().numpy().T, 128, axis=1)  # [O, K]
    err = np.abs(deq - w.double().numpy())
    if zeros:
        assert np.all(err <= (0.5 + 7 * 2.0 ** -11) * step + 1e-7)
    else:  # z = 4: codes -4..3 cover [-4 s, 3 s]; the top of the range clamps at 3 s
        inside = w.double().numpy() <= 3 * step
        assert np.all(err[inside] <= (0.5 + 7 * 2.0 ** -11) * step[inside] + 1e-7)
    # the identity permutation
    assert torch.equal(layout["perm"].long(), torch.arange(384))


def test_rtn_quantizer_rejects_ragged_k():
    with pytest.raises(ValueError, match="multiple of 128"):
        quantize_w3_rtn(torch.zeros(4, 100))


def _rank_one_layout(o=32, k=256, s=4):
    return {
        "planes": torch.zeros(k // 128, o, 2, 16, dtype=torch.uint8),
        "coef": torch.ones(2, o, dtype=torch.float16),
        "srow": torch.ones(o, dtype=torch.float16),
        "tcol": torch.ones(k, dtype=torch.float16),
        "salient": torch.zeros(o, s, dtype=torch.bfloat16),
        "salient_idx": torch.arange(s, dtype=torch.int32),
    }


def test_validate_rank_one_contract():
    assert validate_rank_one(_rank_one_layout()) == (32, 256, 4)
    bare = _rank_one_layout()
    bare["salient"] = None
    bare["salient_idx"] = None
    assert validate_rank_one(bare) == (32, 256, 0)
    broken = [
        ("planes", torch.zeros(2, 32, 2, 8, dtype=torch.uint8), "planes must be"),
        ("coef", torch.ones(2, 32, dtype=torch.float32), "coef must be"),
        ("srow", torch.ones(31, dtype=torch.float16), "srow must be"),
        ("tcol", torch.ones(128, dtype=torch.float16), "tcol must be"),
        ("salient", torch.zeros(32, 4, dtype=torch.float16), "salient must be"),
        ("salient_idx", torch.arange(4, dtype=torch.int64), "salient_idx must be"),
        ("tcol", torch.ones(512, dtype=torch.float16)[::2], "contiguous"),
    ]
    for name, value, message in broken:
        layout = _rank_one_layout()
        layout[name] = value
        with pytest.raises(ValueError, match=message):
            validate_rank_one(layout)


def test_tensor_sha256_closed_form():
    t = torch.arange(12, dtype=torch.int16).reshape(3, 4)
    want = hashlib.sha256(b"torch.int16" + json.dumps([3, 4]).encode() + t.numpy().tobytes()).hexdigest()
    assert tensor_sha256(t) == want
    # the same bytes under another shape or dtype hash differently
    assert tensor_sha256(t.reshape(4, 3)) != want
    assert tensor_sha256(t.view(torch.uint8).reshape(3, 8)) != want
    # views hash their own elements, not the storage
    assert tensor_sha256(t[:, 1:3]) == tensor_sha256(t[:, 1:3].contiguous())


def test_qwen3_8b_linear_shapes():
    assert qwen3_8b_linear_shapes() == {
        "self_attn.q_proj": (4096, 4096), "self_attn.k_proj": (1024, 4096), "self_attn.v_proj": (1024, 4096),
        "self_attn.o_proj": (4096, 4096), "mlp.gate_proj": (12288, 4096), "mlp.up_proj": (12288, 4096),
        "mlp.down_proj": (4096, 12288),
    }


def test_gpu_only_guards():
    with pytest.raises(ValueError, match="GPU tensor"):
        _lib.require_gpu_tensor(torch.zeros(4), "x")
    with pytest.raises(ValueError, match="kernel must be one of"):
        load_extension("v9")
    if not torch.cuda.is_available():
        with pytest.raises(RuntimeError, match="no CPU substitute"):
            load_extension("v1")
