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



def test_qwen3_layer_step_matches_hf_decoder_layer_float64():
    """The float64 layer step against transformers' Qwen3 model run in float64 on the
    CPU: the first decoder layer's output for the token after a 5-token prompt,
    with that layer's cached prefix keys / values and the model's own rotary rows."""
    from transformers import DynamicCache, Qwen3Config, Qwen3ForCausalLM

    torch.manual_seed(3)
    cfg = Qwen3Config(vocab_size=50, hidden_size=64, intermediate_size=96, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=16, rms_norm_eps=1e-6)
    cfg._attn_implementation = "eager"
    model = Qwen3ForCausalLM(cfg).double().eval()
    for norm in [m for n, m in model.named_modules() if n.endswith("norm")]:
        torch.nn.init.normal_(norm.weight, 1.0, 0.1)  # non-trivial norm weights
    prompt = torch.tensor([[3, 9, 1, 7, 4]])
    token = torch.tensor([[11]])
    captured = {}
    layer = model.model.layers[0]
    handle = layer.register_forward_hook(lambda m, a, o: captured.__setitem__("out", o[0] if isinstance(o, tuple) else o))
    with torch.no_grad():
        cache = DynamicCache(config=cfg)
        model(input_ids=prompt, past_key_values=cache, use_cache=True)
        k_prefix = cache.layers[0].keys[0].clone().numpy()
        v_prefix = cache.layers[0].values[0].clone().numpy()
        model(input_ids=token, past_key_values=cache, use_cache=True)
        cos, sin = model.model.rotary_emb(torch.zeros(1, dtype=torch.float64), torch.tensor([[5]]))
    handle.remove()
    a = layer.self_attn
    w = {"in_norm": layer.input_layernorm.weight, "post_norm": layer.post_attention_layernorm.weight,
         "q_norm": a.q_norm.weight, "k_norm": a.k_norm.weight, "q": a.q_proj.weight, "k": a.k_proj.weight,
         "v": a.v_proj.weight, "o": a.o_proj.weight, "gate": layer.mlp.gate_proj.weight,
         "up": layer.mlp.up_proj.weight, "down": layer.mlp.down_proj.weight}
    w = {n: t.detach().numpy() for n, t in w.items()}
    hidden = model.model.embed_tokens.weight[11].detach().numpy()
    got, k_new, v_new = decode.qwen3_layer_step(hidden, w, k_prefix, v_prefix, cos[0, 0].numpy(),
                                                sin[0, 0].numpy(), eps=1e-6, heads=4, kv_heads=2, head_dim=16)
    # HF keeps its RMSNorm and softmax in fp32 even in a float64 model: agreement
    # to ~1e-5 relative; the planted mistakes below move the output by more than 1e-4
    want = captured["out"][0, -1].numpy()
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-7)
    np.testing.assert_allclose(k_new, cache.layers[0].keys[0, :, -1].numpy(), rtol=1e-4, atol=1e-7)
    np.testing.assert_allclose(v_new, cache.layers[0].values[0, :, -1].numpy(), rtol=1e-4, atol=1e-7)
    # a rotation with the wrong sign is visible
    flipped, _, _ = decode.qwen3_layer_step(hidden, w, k_prefix, v_prefix, cos[0, 0].numpy(),
                                            -sin[0, 0].numpy(), eps=1e-6, heads=4, kv_heads=2, head_dim=16)
    assert np.abs(flipped - want).max() > 1e-4
    # a dropped term is visible: without the MLP residual the output moves
    w_no_mlp = dict(w, down=np.zeros_like(w["down"]))
    moved, _, _ = decode.qwen3_layer_step(hidden, w_no_mlp, k_prefix, v_prefix, cos[0, 0].numpy(),
                                          sin[0, 0].numpy(), eps=1e-6, heads=4, kv_heads=2, head_dim=16)
    assert np.abs(moved - got).max() > 1e-3
