"""numpy restatement of the batch-1 decode attention and the Qwen3 SwiGLU.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Reference arithmetic: stock HF ``Qwen3Attention`` with a static KV cache and a
boolean mask (SDPA; the reference's ``static_decode.py:73-81`` runs it) and
``Qwen3MLP`` (``down(act(gate(x)) * up(x))``, act = SiLU).  Pinned in
``tests/test_oracle_decode.py`` against ``torch.nn.functional.
scaled_dot_product_attention`` and ``torch.nn.functional.silu`` (library
routines present in this image) and against hand-computed small cases.
"""
from __future__ import annotations

import numpy as np

from .bf16 import round_to


def gqa_attention(q, k_cache, v_cache, position: int, scale: float) -> np.ndarray:
    """float64 attention of one token.

    ``q [Hq, D]``, caches ``[Hk, L, D]``; query head ``h`` uses KV head
    ``h // (Hq // Hk)`` and slots ``0..position``.  Returns ``[Hq, D]`` float64.
    """
    q = np.asarray(q, np.float64)
    k = np.asarray(k_cache, np.float64)[:, :position + 1]
    v = np.asarray(v_cache, np.float64)[:, :position + 1]
    hq, hk = q.shape[0], k.shape[0]
    group = hq // hk
    out = np.empty_like(q)
    for h in range(hq):
        g = h // group
        s = k[g] @ q[h] * scale
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ v[g]
    return out


def silu_mul(gate, up, dtype: str = "bf16") -> np.ndarray:
    """``round(round(silu(gate)) * up)`` with silu evaluated in float64."""
    g = np.asarray(gate, np.float64)
    s = round_to((g / (1.0 + np.exp(-g))).astype(np.float32), dtype)
    return round_to((s * np.asarray(up, np.float32)).astype(np.float32), dtype)


def _rms(x, weight, eps):
    x = np.asarray(x, np.float64)
    return np.asarray(weight, np.float64) * x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)


def _rotate_half(x):
    half = x.shape[-1] // 2
    return np.concatenate([-x[..., half:], x[..., :half]], axis=-1)


def qwen3_layer_step(hidden, w, k_prefix, v_prefix, cos, sin, *, eps: float, heads: int, kv_heads: int,
                     head_dim: int):
    """float64 decoder layer of HF ``Qwen3DecoderLayer`` for one new token, no rounding.

    ``hidden [H]`` is the token's input hidden state; ``w`` holds float64 weights:
    ``in_norm``, ``post_norm`` ``[H]``, ``q_norm``, ``k_norm`` ``[D]``, ``q``, ``k``,
    ``v``, ``o``, ``gate``, ``up``, ``down`` ``[out, in]``; ``k_prefix`` /
    ``v_prefix`` ``[Hk, P, D]`` the cached keys / values of the earlier positions;
    ``cos`` / ``sin`` ``[D]`` the rotary rows of the token's position.  The layer:
    ``a = rms(h)``; q / k / v projections, per-head RMSNorm of q and k, RoPE
    ``x cos + rotate_half(x) sin``, GQA softmax attention over prefix + token with
    scale ``D^-1/2``, ``h += o(attn)``; ``b = rms(h)``, ``h += down(silu(gate(b)) * up(b))``.
    Returns ``(h_out [H], k_new [Hk, D], v_new [Hk, D])``.
    """
    h = np.asarray(hidden, np.float64)
    a = _rms(h, w["in_norm"], eps)
    q = (np.asarray(w["q"], np.float64) @ a).reshape(heads, head_dim)
    k = (np.asarray(w["k"], np.float64) @ a).reshape(kv_heads, head_dim)
    v = (np.asarray(w["v"], np.float64) @ a).reshape(kv_heads, head_dim)
    q = _rms(q, w["q_norm"], eps)
    k = _rms(k, w["k_norm"], eps)
    c, s = np.asarray(cos, np.float64), np.asarray(sin, np.float64)
    q = q * c + _rotate_half(q) * s
    k = k * c + _rotate_half(k) * s
    keys = np.concatenate([np.asarray(k_prefix, np.float64), k[:, None, :]], axis=1)
    values = np.concatenate([np.asarray(v_prefix, np.float64), v[:, None, :]], axis=1)
    attn = gqa_attention(q, keys, values, keys.shape[1] - 1, head_dim ** -0.5)
    h = h + np.asarray(w["o"], np.float64) @ attn.reshape(-1)
    b = _rms(h, w["post_norm"], eps)
    g = np.asarray(w["gate"], np.float64) @ b
    u = np.asarray(w["up"], np.float64) @ b
    h = h + np.asarray(w["down"], np.float64) @ (g / (1.0 + np.exp(-g)) * u)
    return h, k, v
