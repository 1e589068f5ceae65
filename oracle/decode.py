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


def gqa_attention(q, k_cache, v_cache, position: int, scale: float, prob_dtype: str | None = None,
                  chunk: int = 64) -> np.ndarray:
    """float64 attention of one token.

    ``q [Hq, D]``, caches ``[Hk, L, D]``; query head ``h`` uses KV head
    ``h // (Hq // Hk)`` and slots ``0..position``.  Returns ``[Hq, D]`` float64.
    With ``prob_dtype``, the probabilities ``e^(s - m)`` (m = the maximum of each
    ``chunk`` of keys) are rounded to that dtype before the P.V product while
    their sum stays exact -- the fused SDPA kernels' rounding point.
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
        if prob_dtype is None:
            p = np.exp(s - s.max())
            out[h] = (p / p.sum()) @ v[g]
            continue
        m = s.max()
        num = np.zeros(q.shape[1])
        den = 0.0
        for c in range(0, s.shape[0], chunk):
            sc = s[c:c + chunk]
            mc = sc.max()
            pc = np.exp(sc - mc)
            pr = round_to(pc.astype(np.float32), prob_dtype).astype(np.float64)
            w = np.exp(mc - m)
            num += w * (pr @ v[g][c:c + chunk])
            den += w * pc.sum()
        out[h] = num / den
    return out


def silu_mul(gate, up, dtype: str = "bf16") -> np.ndarray:
    """``round(round(silu(gate)) * up)`` with silu evaluated in float64."""
    g = np.asarray(gate, np.float64)
    s = round_to((g / (1.0 + np.exp(-g))).astype(np.float32), dtype)
    return round_to((s * np.asarray(up, np.float32)).astype(np.float32), dtype)
