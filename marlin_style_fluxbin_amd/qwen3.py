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


def qwen3_config(**overrides):
    """``transformers.Qwen3Config`` of the Qwen3-8B architecture (random-init decode
    benchmarks), full attention, untied bf16 LM head; keyword overrides shrink it."""
    from transformers import Qwen3Config

    values = dict(
        hidden_size=ARCHITECTURE["hidden_size"], intermediate_size=ARCHITECTURE["intermediate_size"],
        num_hidden_layers=ARCHITECTURE["num_hidden_layers"],
        num_attention_heads=ARCHITECTURE["num_attention_heads"],
        num_key_value_heads=ARCHITECTURE["num_key_value_heads"], head_dim=ARCHITECTURE["head_dim"],
        vocab_size=VOCAB_SIZE, rms_norm_eps=RMS_NORM_EPS, max_position_embeddings=40960,
        rope_parameters={"rope_type": "default", "rope_theta": ROPE_THETA}, tie_word_embeddings=False,
        attn_implementation="sdpa",
    )
    values.update(overrides)
    return Qwen3Config(**values)


def random_qwen3_model(config, *, device, dtype, seed: int = 0):
    """Random-init ``Qwen3ForCausalLM`` (HF init: weights ~ N(0, initializer_range=0.02))
    built directly on ``device`` in ``dtype``, in eval mode."""
    import torch
    from transformers.models.qwen3.modeling_qwen3 import Qwen3ForCausalLM

    torch.manual_seed(seed)
    previous = torch.get_default_dtype()
    torch.set_default_dtype(dtype)
    try:
        with torch.device(device):
            model = Qwen3ForCausalLM(config)
    finally:
        torch.set_default_dtype(previous)
    return model.eval()


def desc_act_perm(k: int, generator, device=None):
    """The column permutation a GPTQ ``desc_act=True`` checkpoint carries after the
    reference's conversion (``gptq_deployment.py:199-227``): columns are quantized
    in a random activation order, group ``g`` holds the columns ranked
    ``[128 g, 128 g + 128)`` in it (``g_idx``), and ``perm = stable_argsort(g_idx)``
    lists each group's columns in ascending index order.  int16 ``[k]``."""
    import torch

    order = torch.randperm(k, generator=generator)
    g_idx = torch.empty(k, dtype=torch.int64)
    g_idx[order] = torch.arange(k) // 128
    return torch.argsort(g_idx, stable=True).to(torch.int16).to(device)


def quantize_w3_rtn(weight, *, scale_dtype=None, zeros: bool = True, perm=None) -> dict:
    """Round-to-nearest W3 g128 planar payload of a dense ``[O, K]`` weight.

    Asymmetric per (row, 128-column group): ``s = (max - min) / 7`` rounded to
    ``scale_dtype`` (fp16 by default), ``z = clamp(round(-min / s), 0, 7)``,
    ``q = clamp(round(w / s) + z, 0, 7)``.  With ``zeros=False`` the
    GPTQ-symmetric convention ``s = 2 max|w| / 7``, ``z = 4`` is used and no
    ``zeros`` field is stored.  ``perm`` (int ``[K]``, default the identity): the
    groups are formed over the sorted columns ``weight[:, perm]``, as a desc_act
    checkpoint's are, and the payload stores it.  Runs on the weight's device.
    """
    import torch

    from .gptq_deployment import planar_from_codes

    scale_dtype = torch.float16 if scale_dtype is None else scale_dtype
    o, k = weight.shape
    if k % 128:
        raise ValueError("K must be a multiple of 128")
    w = weight.detach().float()
    if perm is not None:
        if perm.numel() != k:
            raise ValueError("perm must have K entries")
        w = w[:, perm.to(device=w.device, dtype=torch.int64)]
    w = w.reshape(o, k // 128, 128)
    if zeros:
        lo = w.amin(-1)
        hi = w.amax(-1)
        scale = ((hi - lo) / 7).to(scale_dtype).float()
        scale = torch.where(scale > 0, scale, torch.ones_like(scale))
        zero = torch.clamp(torch.round(-lo / scale), 0, 7)
    else:
        scale = (2 * w.abs().amax(-1) / 7).to(scale_dtype).float()
        scale = torch.where(scale > 0, scale, torch.ones_like(scale))
        zero = torch.full_like(scale, 4.0)
    q = torch.clamp(torch.round(w / scale[..., None]) + zero[..., None], 0, 7).to(torch.uint8)
    codes = q.reshape(o, k).t().contiguous()  # [K, O], sorted column order
    layout = {
        "planes": planar_from_codes(codes),
        "scales": scale.t().contiguous().to(scale_dtype),          # [G, O]
        "perm": (torch.arange(k, dtype=torch.int16, device=weight.device) if perm is None
                 else perm.to(device=weight.device, dtype=torch.int16).contiguous()),
    }
    if zeros:
        layout["zeros"] = zero.t().contiguous().to(torch.uint8)
    return layout


# Linears that read the same activation, and so share one desc_act column order
# (GPTQ orders columns by the Hessian of their common input).
QWEN3_INPUT_GROUPS = (("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj"), ("self_attn.o_proj",),
                      ("mlp.gate_proj", "mlp.up_proj"), ("mlp.down_proj",))


def quantize_qwen3_block(block, *, desc_act_generator=None, **kwargs) -> dict:
    """W3 payload ``{"<module>.<field>": tensor}`` for the seven Linears of a block.
    ``desc_act_generator`` (a CPU ``torch.Generator``): each input group of
    ``QWEN3_INPUT_GROUPS`` gets one random desc_act column order
    (:func:`desc_act_perm`), the structure of the reference's real artifacts."""
    perms = {}
    if desc_act_generator is not None:
        for group in QWEN3_INPUT_GROUPS:
            k = block.get_submodule(group[0]).weight.shape[1]
            perm = desc_act_perm(k, desc_act_generator)
            perms.update({name: perm for name in group})
    payload = {}
    for name in QWEN3_LINEAR_MODULES:
        layout = quantize_w3_rtn(block.get_submodule(name).weight, perm=perms.get(name), **kwargs)
        payload.update({f"{name}.{field}": value for field, value in layout.items()})
    return payload


def w3_quantize_qwen3_model(model, *, fallback: str = "dense", row_tile_by_shape=None, desc_act_seed=None,
                            **kwargs) -> int:
    """Replace every decoder block's seven Linears by ``PackedW3Linear`` (in place).
    ``desc_act_seed``: payloads with desc_act column orders drawn from that seed
    (one per input group and block).  Returns the number of replaced Linears."""
    import torch

    from .w3_lut_deployment import QWEN3_ROW_TILE_BY_SHAPE, replace_w3_block_linears

    generator = None if desc_act_seed is None else torch.Generator().manual_seed(desc_act_seed)
    count = 0
    for block in model.model.layers:
        payload = quantize_qwen3_block(block, desc_act_generator=generator, **kwargs)
        policy = row_tile_by_shape
        if policy is None:
            shapes = {tuple(block.get_submodule(n).weight.shape) for n in QWEN3_LINEAR_MODULES}
            policy = None if shapes <= set(QWEN3_ROW_TILE_BY_SHAPE) else {s: 256 for s in shapes}
        count += len(replace_w3_block_linears(block, payload, fallback=fallback, row_tile_by_shape=policy))
    return count


def random_hybrid_payload(out_features: int, in_features: int, *, device, generator, row_scale: float = 0.01) -> dict:
    """A random hybrid g128/s8 two-base payload of one Linear (the seven fields of
    ``deployment.FIELDS``): uniform random signs, row scales ~ N(0, row_scale),
    column scales ~ N(0, 1), sorted distinct refinement columns.  The reference
    builds these payloads offline from real weights (out of scope here); random
    ones exercise the same kernels at the same shapes and byte counts."""
    import torch

    from .packing import pack_two_bases

    g = in_features // 128
    kw = {"device": device, "generator": generator}

    def signs(k):
        return pack_two_bases(torch.randint(0, 2, (2, out_features, k), **kw) * 2 - 1)

    idx = torch.sort(torch.rand(g, 128, **kw).argsort(dim=1)[:, :8], dim=1).values.to(torch.int16)
    return {
        "global_sign_codes": signs(in_features),
        "global_row_scales": torch.randn(2, out_features, g, **kw) * row_scale,
        "global_column_scales": torch.randn(2, g, 128, **kw),
        "refinement_indices": idx,
        "refinement_sign_codes": signs(g * 8),
        "refinement_row_scales": torch.randn(2, out_features, g, **kw) * (0.7 * row_scale),
        "refinement_column_scales": torch.randn(2, g, 8, **kw),
    }


def hybrid_qwen3_model(model, *, seed: int = 0, kernel: str = "v5_p1024", groups_per_split: int = 8,
                       fallback: str = "dense") -> int:
    """Replace every decoder block's seven Linears by ``PackedHybridLinear`` with
    random hybrid payloads of the same shapes (in place); returns the count."""
    import torch

    from .deployment import replace_block_linears

    device = model.model.embed_tokens.weight.device
    generator = torch.Generator(device=device).manual_seed(seed)
    count = 0
    for block in model.model.layers:
        payload = {}
        for name in QWEN3_LINEAR_MODULES:
            o, k = block.get_submodule(name).weight.shape
            for field, value in random_hybrid_payload(o, k, device=device, generator=generator).items():
                payload[f"{name}.{field}"] = value
        count += len(replace_block_linears(block, payload, fallback=fallback, groups_per_split=groups_per_split,
                                           kernel=kernel))
    return count
