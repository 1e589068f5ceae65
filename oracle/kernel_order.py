"""ctypes access to ``oracle/kernel_order.c`` and ``oracle/_ref`` (test infrastructure only)."""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
_KERNEL_ORDER = HERE / "_build" / "liboracle_kernel_order.so"
_REF = HERE / "_ref" / "libref_lut.so"

_f32p = ctypes.POINTER(ctypes.c_float)


def _ptr(array, ctype):
    return array.ctypes.data_as(ctypes.POINTER(ctype))


def load_kernel_order():
    if not _KERNEL_ORDER.exists():
        raise FileNotFoundError(f"{_KERNEL_ORDER} missing: run `make -C oracle`")
    lib = ctypes.CDLL(str(_KERNEL_ORDER))
    lib.oracle_lut_unsigned.argtypes = [_f32p, _f32p]
    lib.oracle_lut_signed.argtypes = [_f32p, _f32p]
    lib.oracle_w3_kernel_order.argtypes = [
        _f32p, ctypes.POINTER(ctypes.c_uint8), _f32p, ctypes.POINTER(ctypes.c_int16),
        ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p,
    ]
    return lib


def load_reference_lut():
    """The reference's own LUT header compiled by ``oracle/Makefile`` (may be absent)."""
    if not _REF.exists():
        return None
    lib = ctypes.CDLL(str(_REF))
    lib.ref_build_unsigned_table.argtypes = [_f32p, _f32p]
    lib.ref_build_signed_table.argtypes = [_f32p, _f32p]
    lib.ref_pattern.argtypes = [ctypes.c_uint]
    lib.ref_pattern.restype = ctypes.c_uint
    return lib


def lut_unsigned(lib, values) -> np.ndarray:
    v = np.ascontiguousarray(values, dtype=np.float32)
    table = np.full(256, np.nan, dtype=np.float32)
    lib.oracle_lut_unsigned(_ptr(v, ctypes.c_float), _ptr(table, ctypes.c_float))
    return table


def w3_kernel_order(x, layout, *, groups_per_split: int = 1, decoded: bool = False) -> np.ndarray:
    """fp32 result of the reference kernel's order for one activation row ``x [K]``."""
    lib = load_kernel_order()
    planes = np.ascontiguousarray(layout["planes"], dtype=np.uint8)
    g, _, o, _ = planes.shape
    scales = np.ascontiguousarray(layout["scales"], dtype=np.float32)
    perm = layout.get("perm")
    perm_arr = None if perm is None else np.ascontiguousarray(perm, dtype=np.int16)
    xv = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    out = np.zeros(o, dtype=np.float32)
    lib.oracle_w3_kernel_order(
        _ptr(xv, ctypes.c_float), _ptr(planes, ctypes.c_uint8), _ptr(scales, ctypes.c_float),
        None if perm_arr is None else _ptr(perm_arr, ctypes.c_int16),
        o, g, groups_per_split, int(decoded), _ptr(out, ctypes.c_float),
    )
    return out
