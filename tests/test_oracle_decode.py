"""Pins for the decode-attention / SwiGLU oracle against torch library routines."""
import numpy as np
import pytest
import torch

from oracle import decode


@pytest.mark.parametrize("hq,hk,d,pos", [(32, 8, 128, 543), (4, 2, 64, 0), (8, 8, 64, 70)])
def test_attention_matches_torch_sdpa(hq, hk, d, pos):
    g = torch.Generator().manual_seed(hq + pos)
    q = torch.randn(hq, d, generator=g, dtype=torch.float64)
    k = torch.randn(hk, pos + 9, d, generator=g, dtype=torch.float64)
    v = torch.randn(hk, pos + 9, d, generator=g, dtype=torch.float64)
    mask = torch.arange(pos + 9) <= pos
    kk = k.repeat_interleave(hq // hk, 0)
    vv = v.repeat_interleave(hq // hk, 0)
    want = torch.nn.functional.scaled_dot_product_attention(q[:, None], kk, vv, attn_mask=mask[None, None])[:, 0]
    got = decode.gqa_attention(q.numpy(), k.numpy(), v.numpy(), pos, 1 / np.sqrt(d))
    np.testing.assert_allclose(got, want.numpy(), rtol=1e-12, atol=1e-12)


def test_attention_small_cases():
    # one key: output is that key's value; equal scores: mean of the values
    q = np.ones((2, 4))
    k = np.zeros((1, 3, 4))
    v = np.arange(12, dtype=np.float64).reshape(1, 3, 4)
    np.testing.assert_allclose(decode.gqa_attention(q, k, v, 0, 0.5), np.tile(v[0, 0], (2, 1)))
    np.testing.assert_allclose(decode.gqa_attention(q, k, v, 2, 0.5), np.tile(v[0].mean(0), (2, 1)))
    # later slots are never read: poison them
    k2 = k.copy()
    k2[:, 2] = np.nan
    assert np.all(np.isfinite(decode.gqa_attention(q, k2, v, 1, 0.5)))


def test_silu_mul_matches_torch():
    g = torch.Generator().manual_seed(0)
    gate = (torch.randn(4096, generator=g) * 4).to(torch.bfloat16)
    up = torch.randn(4096, generator=g).to(torch.bfloat16)
    want = (torch.nn.functional.silu(gate) * up).float().numpy()
    got = decode.silu_mul(gate.float().numpy(), up.float().numpy(), "bf16")
    diff = np.abs(got - want)
    # torch's fp32 exp may differ from float64 by an fp32 ulp: rare bf16 flips
    assert np.mean(diff == 0) > 0.995
    assert np.all(diff <= np.abs(want) * 2 ** -7 + 1e-30)

