"""Every C-ABI entry point fails closed on a bad argument, on the host, before any
device call: FX_EINVAL with a message naming the problem.

CPU-only.  Device pointers are stand-in addresses that are never dereferenced on
the host (each call is rejected before it reaches the device); host-side arrays
(segment tables, head-norm descriptors) are real ctypes arrays.  Each case breaks
one argument of an otherwise valid call, so the message shows which check fired.
"""
import ctypes
import re
import threading
from pathlib import Path

import pytest

from marlin_style_fluxbin_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "fluxbin_amd.h"
D = 1 << 24  # a 256-byte-aligned stand-in device address


def _parameters():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    out = {}
    for m in re.finditer(r"\b(?:int|size_t)\s+(fx_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
        out[m.group(1)] = [p.strip().split()[-1].lstrip("*") for p in m.group(2).split(",")
                           if p.strip() and p.strip() != "void"]
    return out


PARAMS = _parameters()


def _ptrs(*values):
    return (ctypes.c_void_p * len(values))(*values)


def _ints(*values):
    return (ctypes.c_int * len(values))(*values)


W3 = dict(x=D, x_dtype=2, planes=D, scales=D, scale_dtype=2, zeros=None, perm=None, partial=D, workspace=None,
          workspace_bytes=0, out=D, M=1, O=64, K=256, groups_per_split=2, row_tile=256, arithmetic=0,
          residual=D, tile_sumsq=D, payload_format=0, out_index=None, sorted_out=None, stream=None)
HYBRID = dict(x=D, h=D, x_dtype=2, codes=D, rows=D, columns=D, indices=D, sparse_codes=D, sparse_rows=D,
              sparse_columns=D, workspace=None, workspace_bytes=0, out=D, O=64, K=256, residual=D, tile_sumsq=D,
              swiglu=0, n_segments=2, n_tiles=16, norm_weight=D, eps=1e-6, stream=None)

DEFAULTS = {
    "fx_w3_inline_main": W3,
    "fx_w3_finish": dict(partial=D, out=D, out_dtype=2, splits=2, M=1, O=64, stream=None),
    "fx_w3_m1_out": W3,
    "fx_w3_gemv": W3,
    "fx_w3_gemv_noalloc": W3,
    "fx_w3_gemv_swiglu": W3,
    "fx_w3_gemv_residual": W3,
    "fx_w3_gemv_rmsnormed": dict(W3, h=D, n_tiles=16, norm_weight=D, eps=1e-6, swiglu=0),
    "fx_w3_planes_to_fields": dict(planes=D, fields=D + 4096, O=64, K=256, stream=None),
    "fx_w3_gemv_strided_batched": dict(W3, O=128, x_stride=256, planes_stride=3 * 2 * 128 * 16, scales_stride=256,
                                       zeros_stride=256, out_stride=128, batch=4),
    "fx_w3_gemv_fields": dict(W3, fields=D),
    "fx_w3_planes_to_fp6": dict(planes=D, fp6=D + 4096, O=64, K=512, stream=None),
    "fx_w3_gemv_fp6": dict(W3, fp6=D, K=512),
    "fx_w3_fields_plan": dict(tiles=3, parts=4, prefetch=2, stage=1),
    "fx_w3_gemv_fields_rows": dict(W3, fields=D, M=8, O=128, K=1024),
    "fx_decode_attention_plan": dict(keys_per_thread=2, head_groups=2),
    "fx_w3_gemv_config": dict(W3, waves=8, prefetch=1, tiles=1),
    "fx_w3_restore": dict(planes=D, scales=D, scale_dtype=2, zeros=None, perm=None, weight=D, weight_dtype=2,
                          O=64, K=256, stream=None),
    "fx_rmsnorm": dict(x=D, residual=None, weight=D, out=D, residual_out=None, rows=1, hidden=4096, eps=1e-6,
                       dtype=2, stream=None),
    "fx_decode_attention": dict(q=D, k_cache=D, v_cache=D, workspace=D, workspace_bytes=1 << 24, out_index=None, out=D,
                                n_q_heads=32, n_kv_heads=8, max_len=1024, head_dim=128, position=100,
                                scale=0.088, dtype=2, stream=None),
    "fx_silu_mul": dict(gate=D, up=D, out=D, n=4096, dtype=2, stream=None),
    "fx_lm_head_argmax": dict(hidden=D, norm_weight=D, eps=1e-6, weight=D, logits=D, prediction=D, workspace=D,
                              workspace_bytes=1 << 20, vocab=1000, hidden_size=4096, dtype=2, stream=None),
    "fx_lm_head_merge": dict(workspace=D, workspace_bytes=1 << 20, vocab=1000, prediction=D, stream=None),
    "fx_decode_embed": dict(token=D, table=D, vocab=1000, hidden=4096, out=D, tile_sumsq=D, out_index=None,
                            sorted_out=None, lm_workspace=None,
                            lm_workspace_bytes=0, lm_vocab=0, prediction=None, dtype=2, stream=None),
    "fx_two_base_gemv": dict(x=D, x_dtype=2, planes=D, coef=D, srow=D, tcol=D, salient=None, salient_idx=None,
                             n_salient=0, workspace=None, workspace_bytes=0, out=D, O=64, K=256, stream=None),
    "fx_hybrid_gemv": HYBRID,
    "fx_hybrid_gemv_residual": HYBRID,
}
DEFAULTS["fx_lm_head_logits"] = DEFAULTS["fx_lm_head_argmax"]
DEFAULTS["fx_decode_attention_rope"] = dict(DEFAULTS["fx_decode_attention"], k=D, v=D, q_norm_weight=D,
                                            k_norm_weight=D, cos=D, sin=D, eps=1e-6, rope_mode=1)
DEFAULTS["fx_two_base_gemv_config"] = dict(DEFAULTS["fx_two_base_gemv"], waves=8, prefetch=1, groups_per_split=4,
                                           tiles=1)


def _segments(**over):
    """fx_hybrid_gemv_segments(_rmsnormed) arguments with real host tables."""
    rows = over.pop("segment_rows", (32, 32))
    cols = over.pop("columns", (D, D + 4096))
    args = dict(HYBRID, segment_rows=None if rows is None else _ints(*rows), columns=_ptrs(*cols),
                indices=_ptrs(D, D), sparse_columns=_ptrs(D, D))
    args.update(over)
    return args


def _head_norm_rope(**over):
    """fx_head_norm_rope arguments: one q-like tensor of 4 heads, normalised and rotated."""
    n = over.pop("ntensors", 1)
    args = dict(ntensors=n, inputs=_ptrs(over.pop("input", D)), outputs=_ptrs(D + 8192), weights=_ptrs(D + 16384),
                heads=_ints(over.pop("heads", 4)), rope=_ints(over.pop("rope", 1)),
                strides=(ctypes.c_longlong * 6)(512, 128, 512, 512, 128, 512), batch=1, seq=1, head_dim=128,
                cos=D + 32768, sin=D + 65536, cos_strides=(ctypes.c_longlong * 2)(0, 128), position=None, eps=1e-6,
                rope_mode=1, dtype=2, stream=None)
    args.update(over)
    return args


def _call(name, args):
    lib = _lib.library()
    values = [args[p] for p in PARAMS[name]]
    return getattr(lib, name)(*values), lib.fx_last_error().decode()


CASES = [
    # W3 payload checks shared by every W3 entry point
    ("fx_w3_gemv", dict(x_dtype=0), "x dtype must be fp16 or bf16"),
    ("fx_w3_gemv", dict(scale_dtype=5), "scale dtype must be fp16 or bf16"),
    ("fx_w3_gemv", dict(M=0), "M must be in [1,64]"),
    ("fx_w3_gemv", dict(M=65), "M must be in [1,64]"),
    ("fx_w3_gemv", dict(O=0), "O out of range"),
    ("fx_w3_gemv", dict(K=200), "multiple of 128"),
    ("fx_w3_gemv", dict(K=0), "multiple of 128"),
    ("fx_w3_gemv", dict(planes=D + 8), "planes must be 16-byte aligned"),
    ("fx_w3_gemv", dict(O=65536, K=131072), "exceeds 2 GiB"),
    ("fx_w3_gemv", dict(arithmetic=7), "unknown arithmetic"),
    ("fx_w3_gemv", dict(arithmetic=1, scale_dtype=1), "requires bf16 scales"),
    ("fx_w3_gemv", dict(out=None), "out must be non-null"),
    ("fx_w3_gemv", dict(scales=None), "non-null"),
    ("fx_w3_gemv_noalloc", dict(x=None), "non-null"),
    ("fx_w3_gemv_noalloc", dict(out=None), "out must be non-null"),
    ("fx_w3_gemv_noalloc", dict(K=200), "multiple of 128"),
    # the reference contract (inline_main / finish / m1_out)
    ("fx_w3_inline_main", dict(partial=None), "partial workspace must be non-null"),
    ("fx_w3_inline_main", dict(row_tile=300), "row_tile must be 256, 512 or 1024"),
    ("fx_w3_inline_main", dict(groups_per_split=0), "groups_per_split must be in [1, K/128]"),
    ("fx_w3_inline_main", dict(groups_per_split=3), "groups_per_split must be in [1, K/128]"),
    ("fx_w3_inline_main", dict(M=3), "inline_main supports M in {1,2,4,8}"),
    ("fx_w3_m1_out", dict(out=None), "out must be non-null"),
    ("fx_w3_m1_out", dict(row_tile=128), "row_tile must be 256, 512 or 1024"),
    ("fx_w3_m1_out", dict(M=5), "m1_out supports M in {1,2,4,8}"),
    ("fx_w3_m1_out", dict(groups_per_split=1, workspace=None), "workspace must be non-null when K is split"),
    ("fx_w3_finish", dict(partial=None), "partial and out must be non-null"),
    ("fx_w3_finish", dict(out_dtype=0), "out dtype must be fp16 or bf16"),
    ("fx_w3_finish", dict(splits=0), "splits, M and O must be positive"),
    # decode forms
    ("fx_w3_gemv_swiglu", dict(O=63), "even row count"),
    ("fx_w3_gemv_swiglu", dict(out=None), "out must be non-null"),
    ("fx_w3_gemv_residual", dict(residual=None), "residual, out and tile_sumsq must be non-null"),
    ("fx_w3_gemv_residual", dict(tile_sumsq=None), "residual, out and tile_sumsq must be non-null"),
    ("fx_w3_gemv_residual", dict(payload_format=7), "payload_format"),
    ("fx_w3_gemv_residual", dict(out_index=D), "given together"),
    ("fx_w3_gemv_residual", dict(sorted_out=D + 4096), "given together"),
    ("fx_w3_gemv_residual", dict(out_index=D + 1, sorted_out=D + 4096), "out_index must be 2-byte aligned"),
    ("fx_w3_gemv_residual", dict(out_index=D + 4096, sorted_out=D), "must not alias"),
    ("fx_w3_gemv_swiglu", dict(out_index=D + 1), "out_index must be 2-byte aligned"),
    ("fx_w3_gemv_rmsnormed", dict(out_index=D + 4096, swiglu=0), "out_index applies to the SwiGLU output"),
    ("fx_w3_gemv_rmsnormed", dict(n_tiles=15), "n_tiles must be ceil(K / 16)"),
    ("fx_w3_gemv_rmsnormed", dict(norm_weight=D + 2), "norm weight must be 16-byte aligned"),
    ("fx_w3_gemv_rmsnormed", dict(tile_sumsq=None), "must be non-null"),
    ("fx_w3_gemv_rmsnormed", dict(swiglu=1, O=63), "even row count"),
    ("fx_w3_gemv_rmsnormed", dict(K=131072, n_tiles=8192), "too large for the normalising prologue"),
    # strided batch
    ("fx_w3_gemv_strided_batched", dict(batch=0), "batch must be in [1, 65535]"),
    ("fx_w3_gemv_strided_batched", dict(planes_stride=1024), "strides must cover"),
    ("fx_w3_gemv_strided_batched", dict(out_stride=64), "strides must cover"),
    ("fx_w3_gemv_strided_batched", dict(planes_stride=3 * 2 * 128 * 16 + 8), "multiple of 16 bytes"),
    ("fx_w3_gemv_strided_batched", dict(O=64, scales_stride=128, zeros_stride=128, out_stride=64,
                                        planes_stride=3 * 2 * 64 * 16), "multiple of 8"),
    ("fx_w3_gemv_strided_batched", dict(payload_format=5), "payload_format"),
    ("fx_w3_gemv_strided_batched", dict(out=None), "out must be non-null"),
    # field layout
    ("fx_w3_planes_to_fields", dict(fields=D), "cannot run in place"),
    ("fx_w3_planes_to_fields", dict(O=0), "O must be positive and K a multiple of 128"),
    ("fx_w3_planes_to_fields", dict(K=100), "O must be positive and K a multiple of 128"),
    ("fx_w3_planes_to_fields", dict(planes=D + 4), "16-byte aligned"),
    ("fx_w3_planes_to_fields", dict(fields=None), "non-null"),
    ("fx_w3_gemv_fields", dict(out=None), "out must be non-null"),
    ("fx_w3_planes_to_fp6", dict(fp6=D), "cannot run in place"),
    ("fx_w3_planes_to_fp6", dict(K=384), "K a multiple of 512"),
    ("fx_w3_planes_to_fp6", dict(planes=D + 4), "16-byte aligned"),
    ("fx_w3_planes_to_fp6", dict(fp6=None), "non-null"),
    ("fx_w3_gemv_fp6", dict(out=None), "out must be non-null"),
    ("fx_w3_gemv_fp6", dict(x_dtype=1), "bf16 activations"),
    ("fx_w3_gemv_fp6", dict(O=40), "O % 16 == 0 and K % 512 == 0"),
    ("fx_w3_gemv_fp6", dict(K=256), "O % 16 == 0 and K % 512 == 0"),
    ("fx_w3_gemv_residual", dict(payload_format=2, perm=D, K=512), "no permutation"),
    ("fx_w3_gemv_residual", dict(payload_format=3), "FX_W3_FP6"),
    ("fx_w3_fields_plan", dict(tiles=5), "no shared-staging kernel for plan (5, 4, 2, 1)"),
    ("fx_w3_fields_plan", dict(prefetch=3), "no shared-staging kernel"),
    ("fx_w3_fields_plan", dict(tiles=1, parts=8, prefetch=2, stage=2), "no shared-staging kernel"),
    ("fx_decode_attention_plan", dict(keys_per_thread=3), "keys_per_thread must be 0 (default), 1, 2 or 4"),
    ("fx_w3_gemv_fields_rows", dict(M=9), "M must be in [1, 8]"),
    ("fx_w3_gemv_fields_rows", dict(out=None), "out must be non-null"),
    ("fx_w3_gemv_fields_rows", dict(O=120), "O % 16 == 0"),
    ("fx_w3_gemv_fields_rows", dict(K=640), "K % 512 == 0"),
    ("fx_decode_attention_plan", dict(head_groups=8), "head_groups must be 0 (default), 1, 2 or 4"),
    ("fx_w3_gemv_fields", dict(fields=D + 8), "16-byte aligned"),
    # explicit tilings
    ("fx_w3_gemv_config", dict(waves=3), "unsupported waves/prefetch/tiles"),
    ("fx_w3_gemv_config", dict(groups_per_split=0), "groups_per_split must be positive"),
    ("fx_w3_gemv_config", dict(out=None), "out must be non-null"),
    # dense restore
    ("fx_w3_restore", dict(scale_dtype=0), "scale and weight dtypes must be fp16 or bf16"),
    ("fx_w3_restore", dict(weight_dtype=0), "scale and weight dtypes must be fp16 or bf16"),
    ("fx_w3_restore", dict(O=0), "bad O/K"),
    ("fx_w3_restore", dict(K=200), "bad O/K"),
    ("fx_w3_restore", dict(K=65536, perm=D), "K <= 32768"),
    ("fx_w3_restore", dict(planes=D + 2), "planes must be 16-byte aligned"),
    ("fx_w3_restore", dict(weight=None), "non-null"),
    # norms
    ("fx_rmsnorm", dict(residual=D), "a residual needs residual_out"),
    ("fx_rmsnorm", dict(dtype=0), "dtype must be fp16 or bf16"),
    ("fx_rmsnorm", dict(hidden=12), "hidden a multiple of 8"),
    ("fx_rmsnorm", dict(rows=0), "rows must be positive"),
    ("fx_rmsnorm", dict(x=D + 8), "16-byte aligned"),
    ("fx_rmsnorm", dict(eps=-1.0), "eps must be non-negative"),
    ("fx_rmsnorm", dict(weight=None), "non-null"),
    # decode attention
    ("fx_decode_attention", dict(dtype=0), "dtype must be fp16 or bf16"),
    ("fx_decode_attention", dict(head_dim=96), "head_dim must be 64, 128 or 256"),
    ("fx_decode_attention", dict(n_q_heads=6, n_kv_heads=4), "positive multiple of KV heads"),
    ("fx_decode_attention", dict(position=1024), "outside the cache"),
    ("fx_decode_attention", dict(position=-1), "outside the cache"),
    ("fx_decode_attention", dict(q=D + 8), "q and caches must be 16-byte aligned"),
    ("fx_decode_attention", dict(workspace_bytes=16), "attention workspace needs"),
    ("fx_decode_attention", dict(k_cache=None), "non-null"),
    ("fx_decode_attention_rope", dict(rope_mode=9), "rope_mode must be FX_ROPE_STOCK or FX_ROPE_FUSED"),
    ("fx_decode_attention_rope", dict(k=D + 8), "16-byte aligned"),
    ("fx_decode_attention_rope", dict(cos=None), "non-null"),
    ("fx_decode_attention", dict(out_index=D + 1), "out_index must be 2-byte aligned"),
    ("fx_silu_mul", dict(n=0), "n must be positive"),
    ("fx_silu_mul", dict(dtype=0), "dtype must be fp16 or bf16"),
    ("fx_silu_mul", dict(up=None), "non-null"),
    # LM head and the step's first launch
    ("fx_lm_head_argmax", dict(dtype=0), "dtype must be fp16 or bf16"),
    ("fx_lm_head_argmax", dict(hidden_size=500), "multiple of 512"),
    ("fx_lm_head_argmax", dict(vocab=0), "vocab must be positive"),
    ("fx_lm_head_argmax", dict(prediction=D + 4), "prediction must be 8-byte aligned"),
    ("fx_lm_head_argmax", dict(workspace_bytes=16), "LM-head workspace needs"),
    ("fx_lm_head_argmax", dict(logits=D + 1), "logits must be 2-byte aligned"),
    ("fx_lm_head_argmax", dict(weight=D + 8), "16-byte aligned"),
    ("fx_lm_head_argmax", dict(prediction=None), "non-null"),
    ("fx_lm_head_logits", dict(hidden_size=1000), "multiple of 512"),
    ("fx_lm_head_logits", dict(workspace=None), "non-null"),
    ("fx_lm_head_merge", dict(prediction=None), "prediction must be non-null"),
    ("fx_lm_head_merge", dict(prediction=D + 4), "prediction must be 8-byte aligned"),
    ("fx_decode_embed", dict(vocab=0), "vocab must be positive"),
    ("fx_decode_embed", dict(hidden=20), "positive multiple of 16"),
    ("fx_decode_embed", dict(table=D + 8), "aligned"),
    ("fx_decode_embed", dict(dtype=0), "dtype must be fp16 or bf16"),
    ("fx_decode_embed", dict(out=None), "non-null"),
    ("fx_decode_embed", dict(out_index=D + 8192), "given together"),
    ("fx_decode_embed", dict(out_index=D + 8200, sorted_out=D + 16384), "out_index must be 16-byte aligned"),
    ("fx_decode_embed", dict(out_index=D + 8192, sorted_out=D), "must not alias"),
    # two-base GEMVs
    ("fx_two_base_gemv", dict(O=0), "O must be positive and K a positive multiple of 128"),
    ("fx_two_base_gemv", dict(K=200), "O must be positive and K a positive multiple of 128"),
    ("fx_two_base_gemv", dict(n_salient=33), "n_salient must be in [0, 32]"),
    ("fx_two_base_gemv", dict(n_salient=2), "salient values and indices must be non-null"),
    ("fx_two_base_gemv", dict(x_dtype=0), "x dtype must be fp16 or bf16"),
    ("fx_two_base_gemv", dict(planes=D + 4), "16-byte aligned"),
    ("fx_two_base_gemv", dict(coef=None), "non-null"),
    ("fx_two_base_gemv_config", dict(waves=5), "unsupported waves/prefetch/tiles"),
    ("fx_hybrid_gemv", dict(O=0), "O must be in [1, 65536]"),
    ("fx_hybrid_gemv", dict(O=70000), "O must be in [1, 65536]"),
    ("fx_hybrid_gemv", dict(K=200), "K must be a multiple of 128 in [128, 131072]"),
    ("fx_hybrid_gemv", dict(x_dtype=1, x=D + 8), "16-byte aligned"),
    ("fx_hybrid_gemv", dict(x_dtype=0), "x dtype must be fp16 or bf16"),
    ("fx_hybrid_gemv", dict(columns=D + 4), "16-byte aligned"),
    ("fx_hybrid_gemv", dict(sparse_rows=None), "non-null"),
    ("fx_hybrid_gemv_residual", dict(residual=None), "residual, out and tile_sumsq must be non-null"),
    ("fx_hybrid_gemv_residual", dict(O=16, K=131072), "the residual epilogue takes one"),
]


@pytest.mark.parametrize("name,over,message", CASES, ids=[f"{c[0]}-{i}" for i, c in enumerate(CASES)])
def test_entry_point_rejects(name, over, message):
    args = dict(DEFAULTS[name])
    args.update(over)
    rc, error = _call(name, args)
    assert rc == 1, f"{name} {over}: rc {rc} ({error})"
    assert message in error, f"{name} {over}: {error!r}"


SEGMENT_CASES = [
    (dict(n_segments=0), "n_segments must be in [1, 4]"),
    (dict(n_segments=5), "n_segments must be in [1, 4]"),
    (dict(segment_rows=(17, 16)), "concatenated segments must be multiples of 16"),
    (dict(segment_rows=(0, 16)), "segment 0 has 0 rows"),
    (dict(columns=(D, D + 4)), "segment 1: columns must be 16-byte aligned"),
    (dict(columns=(None, D)), "segment 0: columns, indices and sparse columns must be non-null"),
    (dict(segment_rows=None), "segment arrays must be non-null"),
    (dict(codes=None), "non-null"),
    (dict(K=100), "K must be a multiple of 128"),
]


@pytest.mark.parametrize("over,message", SEGMENT_CASES)
@pytest.mark.parametrize("name", ["fx_hybrid_gemv_segments", "fx_hybrid_gemv_segments_rmsnormed"])
def test_hybrid_segments_reject(name, over, message):
    if "n_tiles" not in over and "K" in over:
        over = dict(over, n_tiles=(over["K"] + 15) // 16)
    rc, error = _call(name, _segments(**over))
    assert rc == 1, f"{name} {over}: rc {rc} ({error})"
    assert message in error, f"{name} {over}: {error!r}"


@pytest.mark.parametrize("over,message", [
    (dict(n_tiles=15), "n_tiles must be ceil(K / 16)"),
    (dict(norm_weight=D + 2), "norm weight must be 16-byte aligned"),
    (dict(tile_sumsq=None), "tile_sumsq and norm weight must be non-null"),
])
def test_hybrid_rmsnormed_prologue_rejects(over, message):
    rc, error = _call("fx_hybrid_gemv_segments_rmsnormed", _segments(**over))
    assert rc == 1 and message in error, error


@pytest.mark.parametrize("over,message", [
    (dict(ntensors=0), "ntensors must be in [1,"),
    (dict(ntensors=5), "ntensors must be in [1,"),
    (dict(dtype=0), "dtype must be fp16 or bf16"),
    (dict(head_dim=0), "bad batch/seq/head_dim"),
    (dict(batch=0), "bad batch/seq/head_dim"),
    (dict(rope_mode=9), "unknown rope_mode"),
    (dict(eps=-1.0), "eps must be non-negative"),
    (dict(input=None), "tensor 0: null input or output"),
    (dict(heads=0), "tensor 0: heads must be positive"),
    (dict(cos=None), "RoPE needs cos, sin and their strides"),
    (dict(inputs=None), "tensor arrays must be non-null"),
])
def test_head_norm_rope_rejects(over, message):
    rc, error = _call("fx_head_norm_rope", _head_norm_rope(**over))
    assert rc == 1, f"{over}: rc {rc} ({error})"
    assert message in error, f"{over}: {error!r}"


def test_every_compute_entry_point_has_a_case():
    covered = {c[0] for c in CASES} | {"fx_hybrid_gemv_segments", "fx_hybrid_gemv_segments_rmsnormed",
                                        "fx_head_norm_rope"}
    queries = {n for n in PARAMS if n.endswith("_workspace_bytes")} | {"fx_abi_version"}
    assert set(PARAMS) - queries - covered == set()


def test_error_text_is_per_thread():
    """fx_last_error() is the calling thread's: two threads failing at once each
    read their own message, and the main thread's stays as it was."""
    lib = _lib.library()
    assert lib.fx_lm_head_merge(None, 0, 1, None, None) == 1
    mine = lib.fx_last_error().decode()
    seen = {}
    barrier = threading.Barrier(2)

    def fail(tag, call):
        barrier.wait()
        rc = call()
        seen[tag] = (rc, lib.fx_last_error().decode())

    threads = [
        threading.Thread(target=fail, args=("finish", lambda: lib.fx_w3_finish(None, None, 2, 1, 1, 1, None))),
        threading.Thread(target=fail, args=("silu", lambda: lib.fx_silu_mul(None, None, None, 0, 2, None))),
    ]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert seen["finish"][0] == 1 and "partial and out" in seen["finish"][1]
    assert seen["silu"][0] == 1 and "gate, up and out" in seen["silu"][1]
    assert lib.fx_last_error().decode() == mine and "prediction" in mine
