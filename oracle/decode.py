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
