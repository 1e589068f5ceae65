"""ctypes binding of ``libfluxbin_amd.so`` (the C ABI in ``include/fluxbin_amd.h``).

There is no fallback: if the library is missing or does not load, every caller
gets a ``RuntimeError`` naming the build step.  Errors reported by the library
(``FX_EINVAL`` / ``FX_EHIP``) are raised as ``RuntimeError`` with the message
from ``fx_last_error()``, the way the reference's ``TORCH_CHECK`` failures
surface (``csrc/w3_lut.cu:191-226``).
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIBRARY_PATH = Path(__file__).resolve().parent / "libfluxbin_amd.so"
ABI_VERSION = 19
PAYLOAD_PLANAR, PAYLOAD_FIELDS, PAYLOAD_FP6 = 0, 1, 2  # FX_W3_PLANAR / FX_W3_FIELDS / FX_W3_FP6

FX_F32, FX_F16, FX_BF16 = 0, 1, 2
ARITH_STRUCTURAL, ARITH_DECODED_BF16 = 0, 1
ROPE_NONE, ROPE_STOCK, ROPE_FUSED = 0, 1, 2

_DTYPE_CODES = {torch.float32: FX_F32, torch.float16: FX_F16, torch.bfloat16: FX_BF16}

_p = ctypes.c_void_p
_i = ctypes.c_int
_sz = ctypes.c_size_t
_f = ctypes.c_float

# name -> (restype, argtypes); mirrors include/fluxbin_amd.h
SIGNATURES: dict[str, tuple] = {
    "fx_abi_version": (_i, []),
    "fx_last_error": (ctypes.c_char_p, []),
    "fx_w3_inline_main": (_i, [_p, _i, _p, _p, _i, _p, _p, _p, _i, _i, _i, _i, _i, _i, _p]),
    "fx_w3_finish": (_i, [_p, _p, _i, _i, _i, _i, _p]),
    "fx_w3_m1_out": (_i, [_p, _i, _p, _p, _i, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _p]),
    "fx_w3_gemv_workspace_bytes": (_sz, [_i, _i, _i]),
    "fx_w3_gemv": (_i, [_p, _i, _p, _p, _i, _p, _p, _p, _sz, _p, _i, _i, _i, _i, _p]),
    "fx_w3_gemv_noalloc": (_i, [_p, _i, _p, _p, _i, _p, _p, _p, _i, _i, _i, _i, _p]),
    "fx_w3_gemv_swiglu": (_i, [_p, _i, _p, _p, _i, _p, _p, _p, _p, _i, _i, _i, _p]),
    "fx_w3_gemv_residual": (_i, [_p, _i, _p, _p, _i, _p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _p]),
    "fx_w3_gemv_rmsnormed": (_i, [_p, _i, _p, _p, _i, _p, _p, _i, _p, ctypes.c_float, _p, _p, _i, _i, _i, _i, _p]),
    "fx_w3_gemv_strided_batched": (_i, [_p, _i, ctypes.c_longlong, _p, ctypes.c_longlong, _p, _i, ctypes.c_longlong,
                                        _p, ctypes.c_longlong, _p, ctypes.c_longlong, _i, _i, _i, _i, _p]),
    "fx_w3_planes_to_fields": (_i, [_p, _p, _i, _i, _p]),
    "fx_w3_gemv_fields": (_i, [_p, _i, _p, _p, _i, _p, _p, _i, _i, _p]),
    "fx_w3_planes_to_fp6": (_i, [_p, _p, _i, _i, _p]),
    "fx_w3_gemv_fp6": (_i, [_p, _i, _p, _p, _i, _p, _p, _i, _i, _p]),
    "fx_w3_fields_plan": (_i, [_i, _i, _i, _i]),
    "fx_w3_gemv_fields_rows": (_i, [_p, _i, _p, _p, _i, _p, _p, _i, _i, _i, _p]),
    "fx_w3_gemv_config_workspace_bytes": (_sz, [_i, _i, _i, _i, _i, _i, _i]),
    "fx_w3_gemv_config": (_i, [_p, _i, _p, _p, _i, _p, _p, _p, _sz, _p, _i, _i, _i, _i, _i, _i, _i, _p]),
    "fx_w3_restore": (_i, [_p, _p, _i, _p, _p, _p, _i, _i, _i, _p]),
    "fx_rmsnorm": (_i, [_p, _p, _p, _p, _p, _i, _i, _f, _i, _p]),
    "fx_head_norm_rope": (_i, [_i, _p, _p, _p, _p, _p, _p, _i, _i, _i, _p, _p, _p, _p, _f, _i, _i, _p]),
    "fx_decode_attention_workspace_bytes": (_sz, [_i, _i, _i]),
    "fx_decode_attention_plan": (_i, [_i, _i]),
    "fx_decode_attention": (_i, [_p, _p, _p, _p, _sz, _p, _p, _i, _i, _i, _i, _i, _f, _i, _p]),
    "fx_decode_attention_rope": (_i, [_p, _p, _p, _p, _p, _p, _p, ctypes.c_float, _i, _p, _p, _p, _sz, _p, _p, _i, _i, _i, _i, _i, ctypes.c_float, _i, _p]),
    "fx_silu_mul": (_i, [_p, _p, _p, _i, _i, _p]),
    "fx_lm_head_argmax_workspace_bytes": (_sz, []),
    "fx_lm_head_argmax": (_i, [_p, _p, _f, _p, _p, _p, _p, _sz, _i, _i, _i, _p]),
    "fx_lm_head_logits": (_i, [_p, _p, _f, _p, _p, _p, _sz, _i, _i, _i, _p]),
    "fx_lm_head_merge": (_i, [_p, _sz, _i, _p, _p]),
    "fx_decode_embed": (_i, [_p, _p, _i, _i, _p, _p, _p, _p, _p, _sz, _i, _p, _i, _p]),
    "fx_two_base_gemv_workspace_bytes": (_sz, [_i, _i]),
    "fx_two_base_gemv": (_i, [_p, _i, _p, _p, _p, _p, _p, _p, _i, _p, _sz, _p, _i, _i, _p]),
    "fx_two_base_gemv_config_workspace_bytes": (_sz, [_i, _i, _i, _i, _i, _i]),
    "fx_two_base_gemv_config": (_i, [_p, _i, _p, _p, _p, _p, _p, _p, _i, _p, _sz, _p, _i, _i,
                                     _i, _i, _i, _i, _p]),
    "fx_hybrid_gemv_workspace_bytes": (_sz, [_i, _i]),
    "fx_hybrid_gemv": (_i, [_p, _i, _p, _p, _p, _p, _p, _p, _p, _p, _sz, _p, _i, _i, _p]),
    "fx_hybrid_gemv_segments": (_i, [_p, _i, _i, _p, _p, _p, _p, _p, _p, _p, _p, _p, _sz, _p, _i, _p]),
    "fx_hybrid_gemv_residual": (_i, [_p, _i, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _p]),
    "fx_hybrid_gemv_segments_rmsnormed": (_i, [_p, _i, _i, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i, _p, _f, _p, _sz,
                                                _p, _i, _p]),
}

_lock = threading.Lock()
_library = None


def library():
    """Load and type the shared library once per process (raises if absent)."""
    global _library
    if _library is not None:
        return _library
    with _lock:
        if _library is not None:
            return _library
        if not LIBRARY_PATH.exists():
            raise RuntimeError(
                f"{LIBRARY_PATH.name} is not built; run `python -m marlin_style_fluxbin_amd.build` "
                "(or __graft_entry__.build()). There is no CPU substitute for the HIP kernels."
            )
        lib = ctypes.CDLL(str(LIBRARY_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        if lib.fx_abi_version() != ABI_VERSION:
            raise RuntimeError("libfluxbin_amd.so ABI version mismatch; rebuild it")
        _library = lib
    return _library


def check(rc: int, what: str) -> None:
    if rc != 0:
        message = library().fx_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed ({rc}): {message}")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError as exc:
        raise ValueError(f"unsupported dtype {dtype}") from exc


def ptr(tensor: torch.Tensor | None) -> int | None:
    return None if tensor is None else tensor.data_ptr()


def stream_handle(device: torch.device | None = None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def require_gpu_tensor(tensor: torch.Tensor, name: str) -> None:
    if not tensor.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor for the HIP path")
