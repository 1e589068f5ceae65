"""numpy restatement of Qwen3 RMSNorm, per-head q/k RMSNorm and RoPE.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Reference arithmetic: ``rms_norm_reference`` (``fused_modules.py:30-41``) which is
stock HF ``Qwen3RMSNorm.forward``; ``fused_apply_rotary_pos_emb``
(``fused_modules.py:66-85``) and stock HF ``apply_rotary_pos_emb`` /
``rotate_half`` / ``Qwen3RotaryEmbedding`` (transformers ``modeling_qwen3.py``).
The rounding points are kept where the reference has them:

* RMSNorm: ``h = fp32(x)``; ``var = mean(h^2)`` in fp32; ``h * rsqrt(var + eps)``
  in fp32; cast to the input dtype; multiply by the weight in the weight dtype.
* RoPE cos/sin: ``inv_freq = 1 / theta ** (arange(0, d, 2) / d)`` in fp32,
  ``angle = fp32(pos * inv_freq)``, ``cos/sin`` in fp32 then cast to the model dtype.
* RoPE apply (stock): ``round(round(x*cos) + round(rotate_half(x)*sin))``;
  (fused) ``round(round(x*cos) + rotate_half(x)*sin)`` (``addcmul``).

Pinned in ``tests/test_oracle_norms.py`` against transformers' own
``Qwen3RMSNorm`` / ``Qwen3RotaryEmbedding`` / ``apply_rotary_pos_emb`` (a library
routine present in this image) and against float64 closed forms.
"""
from __future__ import annotations

import numpy as np

from .bf16 import round_to


def rms_norm(x: np.ndarray, weight: np.ndarray, eps: float, dtype: str = "bf16") -> np.ndarray:
    """Qwen3RMSNorm over the last axis; ``x``/``weight`` hold ``dtype`` values."""
    h = np.asarray(x, dtype=np.float32)
    variance = np.mean(h.astype(np.float64) ** 2, axis=-1, keepdims=True).astype(np.float32)
    inv = (1.0 / np.sqrt(variance.astype(np.float64) + np.float64(np.float32(eps)))).astype(np.float32)
    normed = round_to((h * inv).astype(np.float32), dtype)
    return round_to(np.asarray(weight, dtype=np.float32) * normed, dtype)


def rope_inv_freq(head_dim: int, theta: float) -> np.ndarray:
    exponent = (np.arange(0, head_dim, 2, dtype=np.float32) / np.float32(head_dim)).astype(np.float32)
    powered = np.power(np.float32(theta), exponent, dtype=np.float32)
    return (np.float32(1.0) / powered).astype(np.float32)


def rope_cos_sin(positions, head_dim: int, theta: float, dtype: str = "bf16", inv_freq=None):
    """``[L] -> ([L, head_dim], [L, head_dim])`` cos/sin as HF builds them.

    ``inv_freq`` (fp32 ``[head_dim/2]``) defaults to :func:`rope_inv_freq`; a
    caller may pass another fp32 rounding of the same frequencies (torch's ``pow``
    can differ from numpy's in the last bit, and positions up to 4096 amplify it).
    """
    inv = rope_inv_freq(head_dim, theta) if inv_freq is None else np.asarray(inv_freq, np.float32)
    pos = np.asarray(positions, dtype=np.float32).reshape(-1, 1)
    freqs = (pos * inv[None, :]).astype(np.float32)
    emb = np.concatenate([freqs, freqs], axis=-1)
    cos = np.cos(emb.astype(np.float64)).astype(np.float32)
    sin = np.sin(emb.astype(np.float64)).astype(np.float32)
    return round_to(cos, dtype), round_to(sin, dtype)


def rotate_half(x: np.ndarray) -> np.ndarray:
    half = x.shape[-1] // 2
    return np.concatenate([-x[..., half:], x[..., :half]], axis=-1)


def apply_rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, dtype: str = "bf16",
               fused: bool = False) -> np.ndarray:
    """RoPE on ``[..., head_dim]`` with cos/sin broadcastable to it."""
    x = np.asarray(x, dtype=np.float32)
    first = round_to(x * cos, dtype)
    second = rotate_half(x) * sin
    if not fused:
        second = round_to(second, dtype)
    return round_to(first + second, dtype)


def qk_norm_rope(q, k, q_weight, k_weight, cos, sin, eps: float, dtype: str = "bf16"):
    """Per-head RMSNorm of q ``[Hq, D]`` and k ``[Hk, D]`` followed by stock RoPE."""
    qn = rms_norm(q, q_weight, eps, dtype)
    kn = rms_norm(k, k_weight, eps, dtype)
    return apply_rope(qn, cos, sin, dtype), apply_rope(kn, cos, sin, dtype)


def rms_norm_exact(x, weight, eps):
    """float64 closed form ``w * x / sqrt(mean(x^2) + eps)`` with no rounding."""
    h = np.asarray(x, dtype=np.float64)
    return np.asarray(weight, dtype=np.float64) * h / np.sqrt(np.mean(h * h, axis=-1, keepdims=True) + eps)
