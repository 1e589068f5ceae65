"""Qwen3 Linear inventory and the Qwen3-8B architecture constants.

Reference: ``src/fluxbin_style/qwen3.py:16-69`` (module names, expected shapes)
and ``src/fluxbin_style/qwen3_8b.py:19-23`` (architecture).
"""
from __future__ import annotations

from typing import Any

QWEN3_LINEAR_MODULES = (
    "self_attn.q_proj",
    "self_attn.k_proj",
    "self_attn.v_proj",
    "self_attn.o_proj",
    "mlp.gate_proj",
    "mlp.up_proj",
    "mlp.down_proj",
)

ARCHITECTURE = {
    "model_type": "qwen3", "num_hidden_layers": 36, "hidden_size": 4096,
    "intermediate_size": 12288, "num_attention_heads": 32,
    "num_key_value_heads": 8, "head_dim": 128,
}
VOCAB_SIZE = 151936
RMS_NORM_EPS = 1e-6
ROPE_THETA = 1_000_000.0


def expected_qwen3_linear_shape(config: dict[str, Any], module: str) -> list[int]:
    """``[out_features, in_features]`` of one block Linear."""
    values = {}
    for key in ("hidden_size", "intermediate_size", "num_attention_heads", "num_key_value_heads", "head_dim"):
        value = config.get(key)
        if not isinstance(value, int) or value <= 0:
            raise ValueError(f"Qwen3 config requires positive integer {key}")
        values[key] = value
    hidden = values["hidden_size"]
    if module == "self_attn.q_proj":
        return [values["num_attention_heads"] * values["head_dim"], hidden]
    if module in ("self_attn.k_proj", "self_attn.v_proj"):
        return [values["num_key_value_heads"] * values["head_dim"], hidden]
    if module == "self_attn.o_proj":
        return [hidden, values["num_attention_heads"] * values["head_dim"]]
    if module in ("mlp.gate_proj", "mlp.up_proj"):
        return [values["intermediate_size"], hidden]
    if module == "mlp.down_proj":
        return [hidden, values["intermediate_size"]]
    raise ValueError(f"unsupported Qwen3 module: {module}")


def qwen3_8b_linear_shapes() -> dict[str, tuple[int, int]]:
    return {m: tuple(expected_qwen3_linear_shape(ARCHITECTURE, m)) for m in QWEN3_LINEAR_MODULES}
