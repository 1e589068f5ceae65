"""Known-answer tests of ``fused_modules`` as the reference's ``tests/test_fused_modules.py``
states them, and the GPU kernel counts the fused modules remove.

CPU (the reference's own arithmetic, which ``fused_modules`` runs for CPU tensors):
* op counts: stock HF ``apply_rotary_pos_emb`` issues 10 compute ops, the fused
  tensor algebra 5 (``tests/test_fused_modules.py:50-55`` in the reference); in a
  whole tiny-Qwen3 decode step the RoPE patch removes exactly 5 ops per layer
  (:143-148); stock Qwen3RMSNorm is 8 compute ops per call in bf16 (6 in fp32: the
  two casts vanish), called 4 times per layer plus the final norm, and is the
  majority of the step's non-Linear ops (:150-165);
* fused RoPE equals stock within two fp32 ulps in fp32 (the reference: exactly; see
  the test) and within 2^-7 in bf16 (:57-66);
  ``rms_norm_reference`` is bit-exact with stock Qwen3RMSNorm (:77-86);
* the patch is applied and restored, selectively, and restored when the body raises
  (:167-190).

GPU (``-m gpu``): each fused op is one HIP launch where the stock module issues one
kernel per compute op, so in a captured decode step of a tiny Qwen3 the two patches
remove exactly (8 - 1) kernels per RMSNorm call and (10 - 1) per RoPE call.
"""
from __future__ import annotations

import collections

import pytest
import torch
from torch.utils._python_dispatch import TorchDispatchMode

from marlin_style_fluxbin_amd.fused_modules import (fused_apply_rotary_pos_emb, fused_qwen3_modules,
                                                    fused_rms_norm_forward, rms_norm_reference)

# metadata-only ops issue no kernel
VIEW_OPS = {"view", "_unsafe_view", "slice", "narrow", "unsqueeze", "squeeze", "transpose", "permute", "expand",
            "reshape", "detach", "t", "select", "alias"}
LAYERS = 4


class _OpCounter(TorchDispatchMode):
    def __init__(self):
        super().__init__()
        self.ops = collections.Counter()

    def __torch_dispatch__(self, func, types, args=(), kwargs=None):
        self.ops[func.overloadpacket.__name__] += 1
        return func(*args, **(kwargs or {}))


def _compute_ops(call) -> int:
    with _OpCounter() as counter:
        call()
    return sum(n for op, n in counter.ops.items() if op not in VIEW_OPS)


def _rope_inputs(dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(20260914)
    return tuple(torch.randn(shape, generator=g).to(dtype)
                 for shape in ((1, 32, 1, 128), (1, 8, 1, 128), (1, 1, 128), (1, 1, 128)))


def _modeling():
    from transformers.models.qwen3 import modeling_qwen3

    return modeling_qwen3


def test_rope_op_counts():
    m = _modeling()
    q, k, cos, sin = _rope_inputs()
    assert _compute_ops(lambda: m.apply_rotary_pos_emb(q, k, cos, sin)) == 10
    assert _compute_ops(lambda: fused_apply_rotary_pos_emb(q, k, cos, sin)) == 5


def test_rope_matches_stock():
    """The reference holds fp32 to 0.0; torch's CPU addcmul on this host computes
    the multiply-add with one rounding (``addcmul(a, b, c) - (a + b * c)`` is an fp32
    ulp here), so fp32 is held to two ulps of the largest output."""
    m = _modeling()
    for dtype, limit in ((torch.float32, 2 ** -22), (torch.bfloat16, 2 ** -7)):
        q, k, cos, sin = _rope_inputs(dtype)
        for got, want in zip(fused_apply_rotary_pos_emb(q, k, cos, sin), m.apply_rotary_pos_emb(q, k, cos, sin)):
            assert got.shape == want.shape and got.dtype == want.dtype
            assert (got.float() - want.float()).abs().max() <= limit * want.float().abs().max()
    q, k, cos, sin = _rope_inputs()
    with pytest.raises(ValueError):
        fused_apply_rotary_pos_emb(q, k.float(), cos, sin)
    with pytest.raises(ValueError):
        fused_apply_rotary_pos_emb(q, k[..., :64], cos, sin)


def test_rms_norm_reference_is_bit_exact_with_stock():
    m = _modeling()
    for dtype in (torch.float32, torch.bfloat16):
        g = torch.Generator().manual_seed(20260914)
        norm = m.Qwen3RMSNorm(4096).to(dtype)
        with torch.no_grad():
            norm.weight.copy_(1 + 0.02 * torch.randn(4096, generator=g))
        hidden = torch.randn(1, 1, 4096, generator=g).to(dtype)
        assert torch.equal(rms_norm_reference(hidden, norm.weight, norm.variance_epsilon), norm(hidden))
        assert torch.equal(fused_rms_norm_forward(norm, hidden), norm(hidden))  # CPU: the same arithmetic
    # compute ops per call: pow, mean, add, rsqrt, mul, mul, and the two dtype
    # casts when the input is not fp32
    weight, hidden = torch.randn(4096), torch.randn(1, 1, 4096)
    assert _compute_ops(lambda: rms_norm_reference(hidden, weight, 1e-6)) == 6
    hidden16, weight16 = hidden.bfloat16(), weight.bfloat16()
    assert _compute_ops(lambda: rms_norm_reference(hidden16, weight16, 1e-6)) == 8


def _tiny_qwen3(device="cpu"):
    from transformers import Qwen3Config

    m = _modeling()
    config = Qwen3Config(hidden_size=128, intermediate_size=256, num_hidden_layers=LAYERS, num_attention_heads=8,
                         num_key_value_heads=2, head_dim=16, vocab_size=256, max_position_embeddings=64,
                         attn_implementation="sdpa")
    torch.manual_seed(20260914)
    return m.Qwen3ForCausalLM(config).eval().to(device)


def test_whole_decode_step_op_counts():
    m = _modeling()
    model = _tiny_qwen3()
    with torch.inference_mode():
        cache = model(input_ids=torch.tensor([[1, 2, 3, 4]]), use_cache=True).past_key_values

    def decode():
        with torch.inference_mode():
            model(input_ids=torch.tensor([[5]]), past_key_values=cache, use_cache=True)

    stock = _compute_ops(decode)
    with fused_qwen3_modules(rms_norm=False):
        rope_fused = _compute_ops(decode)
    assert stock - rope_fused == 5 * LAYERS
    calls = []
    original = m.Qwen3RMSNorm.forward
    try:
        m.Qwen3RMSNorm.forward = lambda self, x: calls.append(1) or original(self, x)
        total = _compute_ops(decode)
    finally:
        m.Qwen3RMSNorm.forward = original
    assert len(calls) == 4 * LAYERS + 1
    assert len(calls) * 8 / total > 0.5


def test_patch_lifecycle_and_restore_on_error():
    m = _modeling()
    original_forward, original_rope = m.Qwen3RMSNorm.forward, m.apply_rotary_pos_emb
    with fused_qwen3_modules() as applied:
        assert applied == {"rms_norm": True, "rope": True}
        assert m.Qwen3RMSNorm.forward is fused_rms_norm_forward
        assert m.apply_rotary_pos_emb is fused_apply_rotary_pos_emb
    assert m.Qwen3RMSNorm.forward is original_forward and m.apply_rotary_pos_emb is original_rope
    with fused_qwen3_modules(rms_norm=False) as applied:
        assert applied == {"rms_norm": False, "rope": True}
        assert m.Qwen3RMSNorm.forward is original_forward
        assert m.apply_rotary_pos_emb is fused_apply_rotary_pos_emb
    with fused_qwen3_modules(rope=False) as applied:
        assert applied == {"rms_norm": True, "rope": False}
        assert m.apply_rotary_pos_emb is original_rope
    with pytest.raises(RuntimeError, match="boom"):
        with fused_qwen3_modules():
            raise RuntimeError("boom")
    assert m.Qwen3RMSNorm.forward is original_forward and m.apply_rotary_pos_emb is original_rope


@pytest.mark.gpu
def test_decode_step_kernel_counts_on_gpu(gpu):
    """A captured decode step of the tiny Qwen3 (bf16, static cache): the RoPE
    patch removes 10 - 1 kernels per layer, the RMSNorm patch 8 - 1 per call
    (4 per layer + the final norm): each fused op is one HIP launch."""
    from marlin_style_fluxbin_amd.static_decode import StaticDecodeSession

    model = _tiny_qwen3(gpu).to(torch.bfloat16)
    ids = torch.tensor([[1, 2, 3, 4]], device=gpu)
    forced = torch.tensor([[5]], device=gpu)

    def kernels(**patch):
        if patch:
            with fused_qwen3_modules(**patch):
                session = StaticDecodeSession(model, ids, forced)
                session.capture()
        else:
            session = StaticDecodeSession(model, ids, forced)
            session.capture()
        return session.kernel_nodes

    stock = kernels()
    rope = kernels(rms_norm=False, rope=True)
    both = kernels(rms_norm=True, rope=True)
    print(f"kernels per decode step: stock {stock}, fused RoPE {rope}, fused RoPE + RMSNorm {both}", flush=True)
    assert stock - rope == (10 - 1) * LAYERS
    assert rope - both == (8 - 1) * (4 * LAYERS + 1)
