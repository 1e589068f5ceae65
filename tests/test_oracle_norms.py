"""Pins for the RMSNorm / RoPE oracle (CPU).

The oracle (``oracle/norms.py``) restates stock HF Qwen3 arithmetic.  It is pinned
against transformers' own ``Qwen3RMSNorm``, ``Qwen3RotaryEmbedding`` and
``apply_rotary_pos_emb`` (a library present in this image, not the reference),
against ``torch.addcmul`` for the fused RoPE rounding, and against float64
closed forms.  A dropped eps, sum instead of mean, a missing weight, a rounding
point moved or removed, a swapped rotate_half sign or a wrong frequency
exponent each fails at least one test.
"""
import numpy as np
import pytest
import torch

from oracle import norms
from oracle.bf16 import round_to

modeling_qwen3 = pytest.importorskip("transformers.models.qwen3.modeling_qwen3")
from transformers import Qwen3Config  # noqa: E402

DTYPES = {"bf16": torch.bfloat16, "f32": torch.float32}


def _ulp_bf16(v):
    """Spacing of bf16 numbers at |v| (float32 array)."""
    a = np.abs(np.asarray(v, np.float32))
    e = np.floor(np.log2(np.maximum(a, np.float32(2.0 ** -126))))
    return np.float32(2.0) ** (e - 7)


def _hf_rms(x, w, eps):
    norm = modeling_qwen3.Qwen3RMSNorm(x.shape[-1], eps=eps).to(x.dtype)
    with torch.no_grad():
        norm.weight.copy_(w)
        return norm(x)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("hidden,rows", [(4096, 3), (128, 40)])
def test_rms_norm_matches_hf(dtype, hidden, rows):
    g = torch.Generator().manual_seed(hidden + rows)
    x = torch.randn(rows, hidden, generator=g).to(DTYPES[dtype])
    w = (1 + 0.02 * torch.randn(hidden, generator=g)).to(DTYPES[dtype])
    want = _hf_rms(x, w, 1e-6).float().numpy()
    got = norms.rms_norm(x.float().numpy(), w.float().numpy(), 1e-6, dtype)
    if dtype == "f32":
        np.testing.assert_allclose(got, want, rtol=2e-6, atol=0)
    else:
        diff = np.abs(got - want)
        # the fp32 mean may differ from torch's summation order in its last bit
        assert np.all(diff <= _ulp_bf16(want))
        assert np.mean(diff == 0) > 0.99


def test_rms_norm_closed_form_and_eps():
    g = torch.Generator().manual_seed(7)
    x = torch.randn(2, 4096, generator=g).float().numpy()
    w = (1 + 0.02 * torch.randn(4096, generator=g)).float().numpy()
    exact = norms.rms_norm_exact(x, w, 1e-6)
    got = norms.rms_norm(x, w, 1e-6, "f32")
    np.testing.assert_allclose(got, exact, rtol=1e-5)
    # eps matters for tiny inputs: x = 1e-4 everywhere -> x / sqrt(1e-8 + eps)
    tiny = np.full((1, 64), 1e-4, np.float32)
    got = norms.rms_norm(tiny, np.ones(64, np.float32), 1e-6, "f32")
    np.testing.assert_allclose(got, 1e-4 / np.sqrt(1e-8 + 1e-6), rtol=1e-5)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_stock_rope_matches_hf(dtype):
    g = torch.Generator().manual_seed(20260914)
    q = torch.randn(1, 32, 1, 128, generator=g).to(DTYPES[dtype])
    k = torch.randn(1, 8, 1, 128, generator=g).to(DTYPES[dtype])
    cos = torch.randn(1, 1, 128, generator=g).to(DTYPES[dtype])
    sin = torch.randn(1, 1, 128, generator=g).to(DTYPES[dtype])
    want_q, want_k = modeling_qwen3.apply_rotary_pos_emb(q, k, cos, sin)
    c, s = cos.float().numpy()[0], sin.float().numpy()[0]
    got_q = norms.apply_rope(q.float().numpy(), c, s, dtype)
    got_k = norms.apply_rope(k.float().numpy(), c, s, dtype)
    assert np.array_equal(got_q, want_q.float().numpy())
    assert np.array_equal(got_k, want_k.float().numpy())


def test_fused_rope_rounding_is_addcmul():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(40, 128, generator=g).to(torch.bfloat16)
    cos = torch.randn(128, generator=g).to(torch.bfloat16)
    sin = torch.randn(128, generator=g).to(torch.bfloat16)
    rotated = torch.cat((-x[..., 64:], x[..., :64]), dim=-1)
    want = torch.addcmul(x * cos, rotated, sin).float().numpy()
    got = norms.apply_rope(x.float().numpy(), cos.float().numpy(), sin.float().numpy(), "bf16", fused=True)
    assert np.array_equal(got, want)
    stock = norms.apply_rope(x.float().numpy(), cos.float().numpy(), sin.float().numpy(), "bf16")
    assert not np.array_equal(got, stock)  # the two rounding recipes really differ


def test_rotate_half_and_rope_closed_form():
    # rotating (x1, x2) pairs by angle a: x1 cos a - x2 sin a, x2 cos a + x1 sin a
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, 128)).astype(np.float32)
    angle = rng.uniform(0, 6.28, 64).astype(np.float32)
    c = np.concatenate([np.cos(angle), np.cos(angle)]).astype(np.float32)
    s = np.concatenate([np.sin(angle), np.sin(angle)]).astype(np.float32)
    got = norms.apply_rope(x, c, s, "f32")
    x1, x2 = x[:, :64].astype(np.float64), x[:, 64:].astype(np.float64)
    want = np.concatenate([x1 * np.cos(angle) - x2 * np.sin(angle), x2 * np.cos(angle) + x1 * np.sin(angle)], 1)
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-5)


def test_cos_sin_match_hf_rotary_embedding():
    config = Qwen3Config(head_dim=128, rope_parameters={"rope_type": "default", "rope_theta": 1e6},
                         max_position_embeddings=40960)
    rotary = modeling_qwen3.Qwen3RotaryEmbedding(config)
    positions = torch.arange(0, 4096)
    x = torch.zeros(1, dtype=torch.bfloat16)
    want_cos, want_sin = rotary(x, positions[None, :])
    # same fp32 frequencies as HF: the angle and cos/sin recipe must then agree
    got_cos, got_sin = norms.rope_cos_sin(positions.numpy(), 128, 1e6, "bf16",
                                          inv_freq=rotary.inv_freq.numpy())
    for got, want in ((got_cos, want_cos[0].float().numpy()), (got_sin, want_sin[0].float().numpy())):
        diff = np.abs(got - want)
        # torch's fp32 cos/sin may differ from the float64-then-rounded oracle by
        # an fp32 ulp of 1, which moves a bf16 rounding only rarely
        assert np.all(diff <= _ulp_bf16(want) + 2.0 ** -23)
        assert np.mean(diff == 0) > 0.995
    # the frequencies themselves: a pow and a division, each rounded to fp32, so
    # within two fp32 ulps of the closed form; HF's are too
    inv = norms.rope_inv_freq(128, 1e6)
    exact = 1e6 ** (-np.arange(0, 128, 2) / 128.0)
    np.testing.assert_allclose(inv, exact, rtol=2.4e-7)
    np.testing.assert_allclose(rotary.inv_freq.numpy(), exact, rtol=2.4e-7)
    assert inv[0] == 1.0 and abs(inv[-1] - 1e6 ** (-126 / 128)) < 1e-12


def test_qk_norm_rope_matches_hf_chain():
    g = torch.Generator().manual_seed(11)
    q = torch.randn(32, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(8, 128, generator=g).to(torch.bfloat16)
    qw = (1 + 0.02 * torch.randn(128, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.02 * torch.randn(128, generator=g)).to(torch.bfloat16)
    config = Qwen3Config(head_dim=128, rope_parameters={"rope_type": "default", "rope_theta": 1e6})
    cos, sin = modeling_qwen3.Qwen3RotaryEmbedding(config)(q, torch.tensor([[1234]]))
    qn, kn = _hf_rms(q, qw, 1e-6), _hf_rms(k, kw, 1e-6)
    want_q, want_k = modeling_qwen3.apply_rotary_pos_emb(qn[None, :, None], kn[None, :, None], cos, sin)
    got_q, got_k = norms.qk_norm_rope(q.float().numpy(), k.float().numpy(), qw.float().numpy(),
                                      kw.float().numpy(), cos[0, 0].float().numpy(),
                                      sin[0, 0].float().numpy(), 1e-6)
    for got, want in ((got_q, want_q[0, :, 0].float().numpy()), (got_k, want_k[0, :, 0].float().numpy())):
        diff = np.abs(got - want)
        assert np.all(diff <= 2 * _ulp_bf16(want) + 1e-30)
        assert np.mean(diff == 0) > 0.98


def test_round_to_f32_is_identity():
    v = np.float32([1.0, 1e-40, 3.3e38])
    assert np.array_equal(round_to(v, "f32"), v)
