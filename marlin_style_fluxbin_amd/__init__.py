"""MI355X-native (gfx950) W3 packed-LUT batch-1 decode path.

Drop-in for the deployment API of maxiu188-afk/Marlin_Style_Fluxbin's
``fluxbin_style`` package: the planar W3 payload (``gptq_deployment``), the W3
LUT Linear (``w3_lut_deployment``), fused RMSNorm / RoPE (``fused_modules``) and
the static-KV decode session (``static_decode``), and the two-base binary-basis
formats (``packing``, ``evaluation``, ``deployment``, ``engine_interface``; the
benchmark's rank-one variant in ``two_base``).  GPU work runs in hand-written
HIP kernels behind the C ABI of ``libfluxbin_amd.so`` (``include/fluxbin_amd.h``).
"""
from .gptq_deployment import (  # noqa: F401
    FIELDS,
    FORMAT,
    GROUP_SIZE,
    OPTIONAL_FIELDS,
    ZERO,
    bf16_weight_semantics_w3_matvec,
    convert_gptq_w3_to_planar,
    decode_planar_w3_codes,
    inspect_gptq_checkpoint,
    layout_storage,
    pack_gptq_w3_codes,
    planar_from_codes,
    restore_planar_w3,
    structural_w3_matvec,
    unpack_gptq_w3_qweight,
    unpack_gptq_w3_qzeros,
    validate_planar_w3,
)
from .w3_lut_deployment import (  # noqa: F401
    PackedW3Linear,
    W3Gemv,
    finish,
    inline_main,
    load_w3_lut_extension,
    qwen3_row_tile,
    qwen3_w3_route,
    replace_w3_block_linears,
    w3_lut_m1_out,
    workspace_shape,
)

from .fused_modules import (  # noqa: F401
    add_rms_norm,
    fused_apply_rotary_pos_emb,
    fused_qwen3_modules,
    fused_rms_norm_forward,
    head_norm_rope,
    rms_norm,
    rms_norm_reference,
)

from .packing import pack_two_bases, unpack_two_bases  # noqa: F401
from .evaluation import materialize_global_two_base_weight, materialize_hybrid_s8_weight  # noqa: F401
from .deployment import PackedHybridLinear  # noqa: F401
from .w3_lut_artifacts import load_w3_lut_layer, replace_w3_model_linears, write_w3_lut_artifacts  # noqa: F401
from .two_base import TwoBaseGemv, pack_rank_one_planes, two_base_gemv, unpack_rank_one_planes  # noqa: F401

__version__ = "0.1.0"
