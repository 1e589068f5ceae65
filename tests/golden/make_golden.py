"""Write the committed golden fixtures under tests/golden/ from the CPU oracle.

Run from the repository root:  python tests/golden/make_golden.py

Every fixture is data produced by this repository's oracle (``oracle/``) on
seeded inputs, frozen so later changes to the oracle, the product's CPU
functions or the HIP kernels are checked against fixed numbers:

* ``w3_gptq_64x256.npz`` / ``w3_gptq_288x384.npz`` -- raw GPTQ int3 tensors drawn
  with the generator of the reference's ``tests/test_gptq_w3_planar.py:21-39``
  (seed 20260916, desc_act permutation, zero 4), packed by the oracle's own
  bitstream packer; the planar payload; a bf16 and an fp16 activation row; the
  float64 structural output ``x @ (s (q - 4)).T`` and the float64
  dequantize-then-matmul output with the bf16-rounded weight.  The (64, 256) and
  (288, 384) shapes are the reference's own test shapes
  (``tests/test_w3_lut_correctness.py``).
* ``w3_q_proj_config0.json`` -- config 0 (q_proj 4096 x 4096, fp16 scales
  U[0.005, 0.02], zero-points U{3,4}, bf16 x ~N(0,1), seed 0): sha256 of the
  payload and activation bytes and 64 sampled float64 outputs.
* ``norms_config2.npz`` -- config 2: RMSNorm over hidden 4096 (eps 1e-6), per-head
  q/k RMSNorm of 32 / 8 heads x 128 and RoPE (theta 1e6) at positions drawn from
  U{0..4095}, stock and fused (addcmul) rounding; bf16 bit patterns.
* ``two_base_hybrid_257x384.npz`` -- the reference's two-base hybrid g128/s8 format
  at O = 257, K = 384 (``tests/test_deployment.py:12-22`` distributions), its
  deployment layout, and the float64 structural output for one activation row.
* ``two_base_rank_one_64x256.npz`` -- the config-4 rank-one format at 64 x 256.
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

from oracle import bf16, norms, two_base, w3  # noqa: E402

HERE = Path(__file__).resolve().parent


def sha256(array: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(array).tobytes()).hexdigest()


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def f16_bits(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.float16).view(torch.int16).numpy().view(np.uint16)


def reference_synthetic_raw(k: int, o: int, seed: int = 20260916, zero: int = 4):
    """The draws of the reference's ``synthetic_raw`` (same generator calls in the
    same order), packed with the oracle's bitstream packer."""
    generator = torch.Generator().manual_seed(seed)
    codes = torch.randint(0, 8, (k, o), generator=generator, dtype=torch.uint8)
    groups = k // 128
    zeros = np.full((groups, o), zero, dtype=np.uint8)
    scales = (torch.rand((groups, o), generator=generator) * 0.125 + 0.001).half()
    activation_order = torch.randperm(k, generator=generator)
    g_idx = torch.empty(k, dtype=torch.int32)
    g_idx[activation_order] = torch.arange(groups, dtype=torch.int32).repeat_interleave(128)
    codes_np = codes.numpy()
    raw = {
        "qweight": w3.pack_gptq_w3_codes(codes_np, packed_axis=0),
        "qzeros": w3.pack_gptq_w3_codes(((zeros.astype(np.int16) - 1) & 7).astype(np.uint8), packed_axis=1),
        "scales_f16_bits": f16_bits(scales),
        "g_idx": g_idx.numpy(),
    }
    return raw, codes_np, scales.float().numpy()


def w3_gptq_case(o: int, k: int, path: Path) -> None:
    raw, codes, scales_f16 = reference_synthetic_raw(k, o)
    layout = w3.convert_gptq_w3_to_planar(raw["qweight"], raw["qzeros"], scales_f16, raw["g_idx"],
                                          qzero_format=1, scale_dtype="bf16")
    x = torch.randn(1, k, generator=torch.Generator().manual_seed(9))
    x_bf16 = bf16_bits(x)
    x_f16 = f16_bits(x)
    xb = bf16.bf16_bits_to_f32(x_bf16).astype(np.float64)
    xh = x.to(torch.float16).float().numpy().astype(np.float64)
    np.savez_compressed(
        path,
        qweight=raw["qweight"], qzeros=raw["qzeros"], scales_f16_bits=raw["scales_f16_bits"],
        g_idx=raw["g_idx"], codes=codes, planes=layout["planes"], perm=layout["perm"],
        scales_bf16_bits=bf16.f32_to_bf16_bits(layout["scales"]),
        x_bf16_bits=x_bf16, x_f16_bits=x_f16,
        y_exact_bf16x=w3.matvec_exact(xb, layout), y_exact_f16x=w3.matvec_exact(xh, layout),
        y_decoded_bf16x=w3.matvec_decoded(xb, layout, "bf16"),
        restored_bf16_sha256=np.array(sha256(bf16.f32_to_bf16_bits(w3.restore_weight(layout, "bf16")))),
    )


def config0_case(path: Path) -> None:
    o = k = 4096
    generator = torch.Generator().manual_seed(0)
    groups = k // 128
    codes = torch.randint(0, 8, (k, o), generator=generator, dtype=torch.uint8).numpy()
    scales = (torch.rand((groups, o), generator=generator) * 0.015 + 0.005).to(torch.float16)
    zeros = torch.randint(3, 5, (groups, o), generator=generator, dtype=torch.uint8).numpy()
    x = torch.randn(1, k, generator=torch.Generator().manual_seed(0)).to(torch.bfloat16)
    layout = {"planes": w3.planar_from_codes(codes), "scales": scales.float().numpy(), "scale_dtype": "f16",
              "perm": None, "zeros": zeros}
    y = w3.matvec_exact(x.float().numpy(), layout)[0]
    sample = np.random.default_rng(0).choice(o, size=64, replace=False)
    sample.sort()
    record = {
        "config": "config 0: q_proj 4096x4096, codes U{0..7}, fp16 scales U[0.005,0.02], zero-points U{3,4}, "
                  "x bf16 N(0,1), seed 0 (torch.Generator draws: codes randint, scales rand, zeros randint; "
                  "x randn from its own seed-0 generator)",
        "out_features": o, "in_features": k,
        "planes_sha256": sha256(layout["planes"]),
        "scales_f16_sha256": sha256(f16_bits(scales)),
        "zeros_sha256": sha256(zeros),
        "x_bf16_sha256": sha256(bf16_bits(x)),
        "sample_rows": sample.tolist(),
        "y_exact_sample": [float(v) for v in y[sample]],
        "y_bf16_sample": [float(v) for v in bf16.round_bf16(y[sample].astype(np.float32))],
        "y_exact_sum": float(y.sum()),
        "y_exact_abs_max": float(np.abs(y).max()),
    }
    path.write_text(json.dumps(record, indent=1) + "\n")


def norms_case(path: Path) -> None:
    generator = torch.Generator().manual_seed(2)
    hidden = torch.randn(1, 4096, generator=generator).to(torch.bfloat16)
    norm_w = (1 + 0.02 * torch.randn(4096, generator=generator)).to(torch.bfloat16)
    q = torch.randn(32, 128, generator=generator).to(torch.bfloat16)
    k = torch.randn(8, 128, generator=generator).to(torch.bfloat16)
    qw = (1 + 0.02 * torch.randn(128, generator=generator)).to(torch.bfloat16)
    kw = (1 + 0.02 * torch.randn(128, generator=generator)).to(torch.bfloat16)
    positions = torch.randint(0, 4096, (4,), generator=generator).numpy()
    f = lambda t: t.float().numpy()  # noqa: E731
    rms = norms.rms_norm(f(hidden), f(norm_w), 1e-6, "bf16")
    cos, sin = norms.rope_cos_sin(positions, 128, 1e6, "bf16")
    q_stock, k_stock, q_fused, k_fused = [], [], [], []
    qn = norms.rms_norm(f(q), f(qw), 1e-6, "bf16")
    kn = norms.rms_norm(f(k), f(kw), 1e-6, "bf16")
    for i in range(len(positions)):
        q_stock.append(norms.apply_rope(qn, cos[i], sin[i], "bf16"))
        k_stock.append(norms.apply_rope(kn, cos[i], sin[i], "bf16"))
        q_fused.append(norms.apply_rope(qn, cos[i], sin[i], "bf16", fused=True))
        k_fused.append(norms.apply_rope(kn, cos[i], sin[i], "bf16", fused=True))
    b = bf16.f32_to_bf16_bits
    np.savez_compressed(
        path, hidden=bf16_bits(hidden), norm_weight=bf16_bits(norm_w), rms_out=b(rms), eps=np.float32(1e-6),
        q=bf16_bits(q), k=bf16_bits(k), q_norm_weight=bf16_bits(qw), k_norm_weight=bf16_bits(kw),
        positions=positions.astype(np.int64), theta=np.float64(1e6), cos=b(cos), sin=b(sin),
        q_norm=b(qn), k_norm=b(kn), q_rope_stock=b(np.stack(q_stock)), k_rope_stock=b(np.stack(k_stock)),
        q_rope_fused=b(np.stack(q_fused)), k_rope_fused=b(np.stack(k_fused)),
    )


def hybrid_case(path: Path) -> None:
    payload = two_base.make_hybrid_payload(257, 3, seed=19)
    layout = two_base.convert_artifact(payload, planar=True)
    x = torch.randn(1, 384, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    y = two_base.structural_reference(x.float().numpy(), layout)
    np.savez_compressed(path, **{f"payload_{k}": v for k, v in payload.items()},
                        **{f"layout_{k}": v for k, v in layout.items()},
                        x_bf16_bits=bf16_bits(x), y_structural=y,
                        materialized_f32_sha256=np.array(sha256(two_base.materialize_hybrid(payload))))


def rank_one_case(path: Path) -> None:
    p = two_base.make_rank_one_payload(64, 256, salient=32, seed=3)
    x = torch.randn(1, 256, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    y = two_base.rank_one_matvec(x.float().numpy(), p)
    np.savez_compressed(path, planes=p["planes"], coef=p["coef"], srow=p["srow"], tcol=p["tcol"],
                        sal_bf16_bits=bf16.f32_to_bf16_bits(p["sal"]), sal_idx=p["sal_idx"], bases=p["bases"],
                        x_bf16_bits=bf16_bits(x), y=y)


def main() -> None:
    w3_gptq_case(64, 256, HERE / "w3_gptq_64x256.npz")
    w3_gptq_case(288, 384, HERE / "w3_gptq_288x384.npz")
    config0_case(HERE / "w3_q_proj_config0.json")
    norms_case(HERE / "norms_config2.npz")
    hybrid_case(HERE / "two_base_hybrid_257x384.npz")
    rank_one_case(HERE / "two_base_rank_one_64x256.npz")
    for p in sorted(HERE.iterdir()):
        if p.suffix in (".npz", ".json"):
            print(f"{p.name}: {p.stat().st_size} bytes")


if __name__ == "__main__":
    main()
