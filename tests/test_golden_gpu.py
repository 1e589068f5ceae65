"""GPU kernels against the committed golden fixtures (``tests/golden/``).

The fixtures are frozen outputs of the CPU oracle (``tests/golden/make_golden.py``;
``tests/test_golden.py`` checks the oracle still reproduces them).  Here the HIP
path runs on the payloads stored in them:

* W3 GEMV at the reference's own test shapes (64 x 256, 288 x 384; the reference's
  GPTQ generator, desc_act permutation): the MFMA fast path and the table kernel
  of the reference contract, bf16 and fp16 activations, within half an output ulp
  of the float64 structural truth; the decoded-bf16 arithmetic against the
  float64 dequantize-then-matmul; the restore kernel bit for bit (sha256);
* config 0 (q_proj 4096 x 4096, fp16 scales, zero-points U{3,4}): payload bytes
  rebuilt from the seed must hash to the recorded sha256, and 64 sampled outputs
  must lie within half a bf16 ulp of the recorded float64 values;
* config 2: RMSNorm, per-head q/k RMSNorm and stock / fused RoPE, bit-equal to the
  recorded bf16 patterns (RMSNorm within one ulp: its sum of squares runs in a
  different fixed order than numpy's);
* the two-base hybrid layout at 257 x 384 and the rank-one format at 64 x 256.
"""
from __future__ import annotations

import hashlib

import numpy as np
import pytest
import torch

from marlin_style_fluxbin_amd import W3Gemv, _lib
from marlin_style_fluxbin_amd import deployment as d
from marlin_style_fluxbin_amd.fused_modules import head_norm_rope, rms_norm
from marlin_style_fluxbin_amd.two_base import two_base_gemv, two_base_workspace_bytes
from marlin_style_fluxbin_amd.w3_lut_deployment import (
    gemv_fp32_device, restore_planar_w3_device, w3_lut_m1_out, workspace_shape)
from tests.golden_data import load_json, load_npz
from tests.payloads import assert_half_ulp

pytestmark = pytest.mark.gpu


def _bits_to(bits: np.ndarray, dtype: torch.dtype, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(dtype).to(device)


def _w3_layout(f, device):
    return {"planes": torch.from_numpy(f["planes"]).to(device),
            "scales": _bits_to(f["scales_bf16_bits"], torch.bfloat16, device),
            "perm": torch.from_numpy(f["perm"]).to(device)}


@pytest.mark.parametrize("name", ["w3_gptq_64x256.npz", "w3_gptq_288x384.npz"])
def test_w3_gemv_golden(gpu, name):
    f = load_npz(name)
    layout = _w3_layout(f, gpu)
    o, k = f["codes"].shape[1], f["codes"].shape[0]
    for bits_key, dtype, exact_key in (("x_bf16_bits", torch.bfloat16, "y_exact_bf16x"),
                                       ("x_f16_bits", torch.float16, "y_exact_f16x")):
        x = _bits_to(f[bits_key], dtype, gpu).reshape(1, k)
        label = "bf16" if dtype == torch.bfloat16 else "f16"
        out = torch.empty(1, o, dtype=dtype, device=gpu)
        W3Gemv(layout)(x, out)
        torch.cuda.synchronize()
        assert_half_ulp(out.float().cpu().numpy(), f[exact_key], label, rel_slack=3e-5,
                        what=f"{name} fast path {label}")
        for row_tile in (256, 1024):
            for gps in (1, 2):
                ws = torch.full(workspace_shape(o, k, gps), float("nan"), device=gpu)
                y = torch.empty(1, o, dtype=dtype, device=gpu)
                w3_lut_m1_out(x, layout, y, ws, row_tile=row_tile, groups_per_split=gps)
                assert_half_ulp(y.float().cpu().numpy(), f[exact_key], label, rel_slack=2e-6,
                                what=f"{name} table path {label} rt {row_tile} gps {gps}")
    xb = _bits_to(f["x_bf16_bits"], torch.bfloat16, gpu).reshape(1, k)
    fp32 = gemv_fp32_device(xb, layout, arithmetic="structural").cpu().numpy()
    exact = f["y_exact_bf16x"]
    assert np.abs(fp32 - exact).max() <= 1e-5 * np.abs(exact).max()
    decoded = gemv_fp32_device(xb, layout, arithmetic="decoded_bf16").cpu().numpy()
    assert np.abs(decoded - f["y_decoded_bf16x"]).max() <= 1e-5 * np.abs(f["y_decoded_bf16x"]).max()
    restored = restore_planar_w3_device(layout, dtype=torch.bfloat16).view(torch.int16).cpu().numpy()
    digest = hashlib.sha256(np.ascontiguousarray(restored.view(np.uint16)).tobytes()).hexdigest()
    assert digest == str(f["restored_bf16_sha256"])


def test_config0_q_proj_golden(gpu):
    record = load_json("w3_q_proj_config0.json")
    o, k = record["out_features"], record["in_features"]
    generator = torch.Generator().manual_seed(0)
    codes = torch.randint(0, 8, (k, o), generator=generator, dtype=torch.uint8)
    scales = (torch.rand((k // 128, o), generator=generator) * 0.015 + 0.005).to(torch.float16)
    zeros = torch.randint(3, 5, (k // 128, o), generator=generator, dtype=torch.uint8)
    x = torch.randn(1, k, generator=torch.Generator().manual_seed(0)).to(torch.bfloat16)
    from oracle import w3
    planes = w3.planar_from_codes(codes.numpy())
    sha = lambda a: hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()  # noqa: E731
    assert sha(planes) == record["planes_sha256"]
    assert sha(scales.view(torch.int16).numpy()) == record["scales_f16_sha256"]
    assert sha(zeros.numpy()) == record["zeros_sha256"]
    assert sha(x.view(torch.int16).numpy()) == record["x_bf16_sha256"]
    layout = {"planes": torch.from_numpy(planes).to(gpu), "scales": scales.to(gpu),
              "perm": torch.arange(k, dtype=torch.int16, device=gpu), "zeros": zeros.to(gpu)}
    out = torch.empty(1, o, dtype=torch.bfloat16, device=gpu)
    W3Gemv(layout)(x.to(gpu), out)
    rows = np.asarray(record["sample_rows"])
    got = out.float().cpu().numpy()[0, rows]
    assert_half_ulp(got, np.asarray(record["y_exact_sample"]), "bf16", what="config 0 samples")


def test_norms_config2_golden(gpu):
    f = load_npz("norms_config2.npz")
    bf = torch.bfloat16
    hidden = _bits_to(f["hidden"], bf, gpu)
    out = rms_norm(hidden, _bits_to(f["norm_weight"], bf, gpu), float(f["eps"]))
    got = out.view(torch.int16).cpu().numpy().view(np.uint16).astype(np.int32)
    assert np.abs(got - f["rms_out"].astype(np.int32)).max() <= 1
    q = _bits_to(f["q"], bf, gpu)
    k = _bits_to(f["k"], bf, gpu)
    qw, kw = _bits_to(f["q_norm_weight"], bf, gpu), _bits_to(f["k_norm_weight"], bf, gpu)
    cos_all, sin_all = _bits_to(f["cos"], bf, gpu), _bits_to(f["sin"], bf, gpu)
    for mode, qkey, kkey in ((_lib.ROPE_STOCK, "q_rope_stock", "k_rope_stock"),
                             (_lib.ROPE_FUSED, "q_rope_fused", "k_rope_fused")):
        for i in range(len(f["positions"])):
            q_out, k_out = torch.empty_like(q), torch.empty_like(k)
            tensors = [dict(x=q, out=q_out, weight=qw, heads=32, rope=True, in_strides=(0, 128, 0),
                            out_strides=(0, 128, 0)),
                       dict(x=k, out=k_out, weight=kw, heads=8, rope=True, in_strides=(0, 128, 0),
                            out_strides=(0, 128, 0))]
            head_norm_rope(tensors, cos=cos_all[i].contiguous(), sin=sin_all[i].contiguous(), eps=1e-6,
                           rope_mode=mode)
            torch.cuda.synchronize()
            for t, key in ((q_out, qkey), (k_out, kkey)):
                got = t.view(torch.int16).cpu().numpy().view(np.uint16)
                np.testing.assert_array_equal(got, f[key][i], err_msg=f"{key} position {f['positions'][i]}")


def test_hybrid_two_base_golden(gpu):
    f = load_npz("two_base_hybrid_257x384.npz")
    p = {k[len("payload_"):]: torch.from_numpy(v) for k, v in f.items() if k.startswith("payload_")}
    layout = {k: v.to(gpu) for k, v in d.convert_artifact(p, kernel="v5_p1024").items()}
    for k_name, v in f.items():  # the product's conversion reproduces the stored deployment layout
        if k_name.startswith("layout_"):
            np.testing.assert_array_equal(layout[k_name[len("layout_"):]].cpu().numpy(), v, err_msg=k_name)
    x = _bits_to(f["x_bf16_bits"], torch.bfloat16, gpu)
    y = torch.empty(1, 257, dtype=torch.bfloat16, device=gpu)
    for gps in (1, 8):
        ws = torch.full(d.workspace_shape(257, 384, gps), float("nan"), device=gpu)
        d.m1_out(x, layout, y, ws, groups_per_split=gps, kernel="v5_p1024")
        got = y.float().cpu().numpy().astype(np.float64)
        ref = f["y_structural"]
        assert np.abs(got - ref).max() <= 2 ** -8 * np.abs(ref).max()


def test_rank_one_two_base_golden(gpu):
    f = load_npz("two_base_rank_one_64x256.npz")
    layout = {"planes": torch.from_numpy(f["planes"]).to(gpu), "coef": torch.from_numpy(f["coef"]).to(gpu),
              "srow": torch.from_numpy(f["srow"]).to(gpu), "tcol": torch.from_numpy(f["tcol"]).to(gpu),
              "salient": _bits_to(f["sal_bf16_bits"], torch.bfloat16, gpu),
              "salient_idx": torch.from_numpy(f["sal_idx"]).to(gpu)}
    x = _bits_to(f["x_bf16_bits"], torch.bfloat16, gpu)
    y = torch.empty(1, 64, dtype=torch.bfloat16, device=gpu)
    ws = torch.zeros(max(two_base_workspace_bytes(64, 256), 256), dtype=torch.uint8, device=gpu)
    two_base_gemv(x, layout, y, ws)
    got = y.float().cpu().numpy().astype(np.float64)
    assert np.abs(got - f["y"]).max() <= 2 ** -8 * np.abs(f["y"]).max()
