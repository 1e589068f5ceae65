"""numpy restatement of the W3 g128 planar payload and its GEMV semantics.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Reference: ``src/fluxbin_style/gptq_deployment.py`` in maxiu188-afk/Marlin_Style_Fluxbin.
Everything here is written from the format's definition, not from that code's
shift tables, so the two can disagree if either has a mistake:

* GPTQ int3 packing (``gptq_deployment.py:25-71,331-348``) is a little-endian
  96-bit bitstream per 32 codes: code ``i`` occupies bits ``3i..3i+2`` of
  ``word0 | word1 << 32 | word2 << 64``.  Pinned by the reference's boundary KAT
  (``tests/test_gptq_w3_planar.py:43-60``, re-run in ``tests/test_oracle_w3.py``).
* Planar layout (``gptq_deployment.py:199-244``): input columns sorted by
  ``g_idx`` (stable), ``planes[g, p, o, c]`` holds bit ``p`` of the 8 codes
  ``k = 128 g + 8 c + j`` (``j`` = bit position, LSB first) of output row ``o``;
  plane 2 is stored inverted.  Pinned by brute force over every byte value and
  every (code, position) pair.
* Dequantize (``restore_planar_w3``, ``gptq_deployment.py:247-260``):
  ``W[o, perm[s]] = round_scale_dtype(scale[g, o] * (q - zero))`` then cast to the
  output dtype.  The reference fixes ``zero = 4`` and bf16 scales; the benchmark
  configs add per-group integer zero-points (``zeros`` uint8 ``[G, O]``) and fp16
  scales, which follow the same formula.  Pinned bitwise against the direct
  formula of ``tests/test_gptq_w3_planar.py:83-90``.
* ``matvec_exact`` / ``matvec_decoded`` are float64 dequantize-then-matmul
  (exact scales, or per-weight rounded weights); pinned by basis-vector inputs,
  linearity and brute-force loops on tiny shapes.
"""
from __future__ import annotations

import numpy as np

from .bf16 import round_to

GROUP = 128
BITS = 3
ZERO = 4


# --------------------------------------------------------------------------- GPTQ int3
def pack_gptq_w3_codes(codes: np.ndarray, packed_axis: int = 0) -> np.ndarray:
    """Pack uint8 codes in [0,7] (packed dimension multiple of 32) into int32 words.

    Restates ``pack_gptq_w3_codes`` (``gptq_deployment.py:331-348``) as a bitstream.
    """
    codes = np.asarray(codes, dtype=np.uint8)
    logical = codes if packed_axis == 0 else codes.T
    if logical.shape[0] % 32 or (logical > 7).any():
        raise ValueError("packed dimension must be a multiple of 32 and codes must be W3")
    blocks = logical.astype(np.uint64).reshape(-1, 32, logical.shape[1])
    words = np.zeros((blocks.shape[0], 3, logical.shape[1]), dtype=np.uint64)
    for i in range(32):
        bit = 3 * i
        for b in range(3):
            position = bit + b
            value = (blocks[:, i] >> np.uint64(b)) & np.uint64(1)
            words[:, position // 32] |= value << np.uint64(position % 32)
    packed = words.reshape(-1, logical.shape[1]).astype(np.uint32).view(np.int32)
    return packed if packed_axis == 0 else np.ascontiguousarray(packed.T)


def unpack_gptq_w3(words: np.ndarray, packed_axis: int = 0) -> np.ndarray:
    """Inverse of :func:`pack_gptq_w3_codes` (``gptq_deployment.py:42-77``)."""
    words = np.asarray(words, dtype=np.int32)
    logical = words if packed_axis == 0 else words.T
    if logical.shape[0] % 3:
        raise ValueError("packed count must be divisible by three")
    u = logical.view(np.uint32).astype(np.uint64).reshape(-1, 3, logical.shape[1])
    out = np.zeros((u.shape[0], 32, logical.shape[1]), dtype=np.uint8)
    for i in range(32):
        value = np.zeros((u.shape[0], logical.shape[1]), dtype=np.uint64)
        for b in range(3):
            position = 3 * i + b
            value |= ((u[:, position // 32] >> np.uint64(position % 32)) & np.uint64(1)) << np.uint64(b)
        out[:, i] = value.astype(np.uint8)
    codes = out.reshape(-1, logical.shape[1])
    return codes if packed_axis == 0 else np.ascontiguousarray(codes.T)


def unpack_gptq_w3_qzeros(qzeros: np.ndarray, qzero_format: int) -> np.ndarray:
    """Logical zero points ``[G, O]``; format 1 stores ``zero - 1`` (``gptq_deployment.py:80-93``)."""
    if qzero_format not in (1, 2):
        raise ValueError("qzero_format must be 1 or 2")
    zeros = unpack_gptq_w3(qzeros, packed_axis=1)
    if qzero_format == 1:
        zeros = ((zeros.astype(np.int16) + 1) & 7).astype(np.uint8)
    return zeros


# --------------------------------------------------------------------------- planar layout
def pack_bytes_lsb(bits: np.ndarray) -> np.ndarray:
    """``[..., 128]`` 0/1 -> ``[..., 16]`` uint8, bit ``j`` of byte ``c`` = element ``8c+j``."""
    bits = np.asarray(bits, dtype=np.uint8)
    chunks = bits.reshape(*bits.shape[:-1], bits.shape[-1] // 8, 8).astype(np.uint16)
    weights = (1 << np.arange(8, dtype=np.uint16))
    return (chunks * weights).sum(-1).astype(np.uint8)


def unpack_bytes_lsb(values: np.ndarray) -> np.ndarray:
    values = np.asarray(values, dtype=np.uint8)
    bits = (values[..., None] >> np.arange(8, dtype=np.uint8)) & 1
    return bits.reshape(*values.shape[:-1], values.shape[-1] * 8).astype(np.uint8)


def planar_from_codes(codes: np.ndarray, perm: np.ndarray | None = None) -> np.ndarray:
    """Original-order codes ``[K, O]`` -> planes ``[G, 3, O, 16]``.

    ``perm[s]`` is the original input column at sorted position ``s``
    (``gptq_deployment.py:209-224``); ``None`` means identity.
    """
    codes = np.asarray(codes, dtype=np.uint8)
    k, o = codes.shape
    if k % GROUP:
        raise ValueError("K must be a multiple of 128")
    sorted_codes = codes if perm is None else codes[np.asarray(perm, dtype=np.int64)]
    grouped = sorted_codes.reshape(k // GROUP, GROUP, o).transpose(0, 2, 1)  # [G, O, 128]
    b0 = grouped & 1
    b1 = (grouped >> 1) & 1
    b2_inverted = 1 - ((grouped >> 2) & 1)
    return np.ascontiguousarray(
        np.stack([pack_bytes_lsb(b0), pack_bytes_lsb(b1), pack_bytes_lsb(b2_inverted)], axis=1)
    )


def codes_from_planar(planes: np.ndarray, perm: np.ndarray | None = None) -> np.ndarray:
    """planes ``[G,3,O,16]`` -> codes ``[K, O]`` (original order when ``perm`` is given)."""
    planes = np.asarray(planes, dtype=np.uint8)
    g, three, o, sixteen = planes.shape
    if three != 3 or sixteen != 16:
        raise ValueError("planes must be [G,3,O,16]")
    b0 = unpack_bytes_lsb(planes[:, 0])
    b1 = unpack_bytes_lsb(planes[:, 1])
    b2 = 1 - unpack_bytes_lsb(planes[:, 2])
    sorted_codes = (b0 | (b1 << 1) | (b2 << 2)).transpose(0, 2, 1).reshape(g * GROUP, o)
    if perm is None:
        return np.ascontiguousarray(sorted_codes)
    out = np.empty_like(sorted_codes)
    out[np.asarray(perm, dtype=np.int64)] = sorted_codes
    return out


def convert_gptq_w3_to_planar(qweight, qzeros, scales_f16, g_idx, *, qzero_format=1,
                              scale_dtype="bf16", allow_zeros=False):
    """Raw GPTQ tensors -> planar layout dict (numpy).

    Follows ``convert_gptq_w3_to_planar`` (``gptq_deployment.py:199-227``): stable
    argsort of ``g_idx`` gives ``perm``; scales are cast from fp16 to
    ``scale_dtype``.  With ``allow_zeros`` a non-constant zero-point becomes the
    ``zeros`` field; without it only zero == 4 is accepted, as in the reference.
    """
    codes = unpack_gptq_w3(qweight, 0)
    zeros = unpack_gptq_w3_qzeros(qzeros, qzero_format)
    g_idx = np.asarray(g_idx, dtype=np.int64)
    perm = np.argsort(g_idx, kind="stable")
    groups = codes.shape[0] // GROUP
    if not np.array_equal(g_idx[perm], np.repeat(np.arange(groups), GROUP)):
        raise ValueError("sorted g_idx is not canonical group128")
    uniform = np.unique(zeros).tolist() == [ZERO]
    if not uniform and not allow_zeros:
        raise ValueError("constant-zero layout requires decoded zero=4")
    scales = round_to(np.asarray(scales_f16, dtype=np.float16).astype(np.float32), scale_dtype)
    layout = {
        "planes": planar_from_codes(codes, perm),
        "scales": scales,
        "scale_dtype": scale_dtype,
        "perm": perm.astype(np.int16),
        "zeros": None if uniform else zeros,
    }
    return layout


# --------------------------------------------------------------------------- dequantize
def _zeros_or_default(layout):
    planes = layout["planes"]
    zeros = layout.get("zeros")
    if zeros is None:
        return np.full((planes.shape[0], planes.shape[2]), ZERO, dtype=np.int16)
    return np.asarray(zeros, dtype=np.int16)


def _expand_groups(per_group: np.ndarray) -> np.ndarray:
    """``[G, O]`` -> ``[O, K_sorted]`` by repeating each group 128 times along K."""
    return np.repeat(np.asarray(per_group).T, GROUP, axis=1)


def signed_codes_sorted(layout) -> np.ndarray:
    """``q - zero`` as int16 ``[O, K]`` in sorted-column order."""
    codes = codes_from_planar(layout["planes"]).T.astype(np.int16)  # [O, K_sorted]
    return codes - _expand_groups(_zeros_or_default(layout))


def _unsort_columns(sorted_weight: np.ndarray, perm) -> np.ndarray:
    if perm is None:
        return sorted_weight
    out = np.empty_like(sorted_weight)
    out[:, np.asarray(perm, dtype=np.int64)] = sorted_weight
    return out


def restore_weight(layout, out_dtype: str = "bf16") -> np.ndarray:
    """Dequantize ``[O, K]`` with the reference's per-weight rounding.

    ``round_scale_dtype(scale * (q - zero))`` then ``round_out_dtype`` -- the
    arithmetic of ``restore_planar_w3`` (``gptq_deployment.py:254-260``), where a
    bf16 (or fp16) scale tensor times an int16 tensor rounds once to the scale
    dtype.  Returned as float32 holding ``out_dtype`` values.
    """
    signed = signed_codes_sorted(layout).astype(np.float32)
    scales = _expand_groups(np.asarray(layout["scales"], dtype=np.float32))
    product = round_to(scales * signed, layout["scale_dtype"])
    return round_to(_unsort_columns(product, layout.get("perm")), out_dtype)


def dequant_exact(layout) -> np.ndarray:
    """``[O, K]`` float64 ``scale * (q - zero)`` with no rounding."""
    signed = signed_codes_sorted(layout).astype(np.float64)
    scales = _expand_groups(np.asarray(layout["scales"], dtype=np.float64))
    return _unsort_columns(scales * signed, layout.get("perm"))


def matvec_exact(x: np.ndarray, layout) -> np.ndarray:
    """``[M, K] -> [M, O]`` float64 ``x @ (scale*(q-zero)).T`` (the structural truth)."""
    return np.asarray(x, dtype=np.float64) @ dequant_exact(layout).T


def matvec_decoded(x: np.ndarray, layout, weight_dtype: str = "bf16") -> np.ndarray:
    """float64 dot of ``x`` with the restored (per-weight rounded) weight.

    This is dequantize-then-matmul with exact accumulation: the value
    ``bf16_weight_semantics_w3_matvec`` approximates in fp32
    (``gptq_deployment.py:280-315``) and ``F.linear(x, restore_planar_w3(...))``
    approximates in the matmul's own order.
    """
    weight = restore_weight(layout, weight_dtype).astype(np.float64)
    return np.asarray(x, dtype=np.float64) @ weight.T


def layout_storage_bytes(layout) -> int:
    """Stored bytes: planes + 2-byte scales + 2-byte perm (+ 1-byte zeros)."""
    planes = layout["planes"]
    g, _, o, _ = planes.shape
    total = planes.size + 2 * g * o + 2 * g * GROUP
    if layout.get("zeros") is not None:
        total += g * o
    return total


# --------------------------------------------------------------------------- field layout
# The library's bind-time repack of the planar payload (no reference counterpart;
# written from its definition here, the kernel from the same definition in HIP).
# Same array shape as the planes, [G, 3, O, 16] uint8 = per (group, row) three
# "member" rows of four little-endian 32-bit words; the 32 sorted columns
# 32 w + t (t < 32) of word w are spread over member word w of members 0..2:
#   i = t // 2, h = t % 2 (low / high 16-bit half);
#   i < 15: the whole code in bits [16 h + 3 f, +3) of member i // 5, f = i % 5;
#   i = 15: bit k of the code in bit 15 + 16 h of member k.
# Three bits per code, as the planes.
def field_slots() -> list[list[tuple[int, int]]]:
    """For t in 0..31: the (member, bit) of code bits 0, 1, 2 within word w."""
    slots = []
    for t in range(32):
        i, h = t // 2, t % 2
        if i < 15:
            m, f = i // 5, i % 5
            slots.append([(m, 16 * h + 3 * f + k) for k in range(3)])
        else:
            slots.append([(k, 15 + 16 * h) for k in range(3)])
    return slots


def fields_from_sorted_codes(sorted_codes: np.ndarray) -> np.ndarray:
    """Sorted-order codes ``[K, O]`` -> field layout ``[G, 3, O, 16]``."""
    codes = np.asarray(sorted_codes, dtype=np.uint32)
    k, o = codes.shape
    if k % GROUP:
        raise ValueError("K must be a multiple of 128")
    grouped = codes.reshape(k // GROUP, GROUP, o).transpose(0, 2, 1)  # [G, O, 128]
    words = np.zeros((k // GROUP, 3, o, 4), dtype=np.uint32)
    for c in range(GROUP):
        w, t = divmod(c, 32)
        for bit, (m, pos) in enumerate(field_slots()[t]):
            words[:, m, :, w] |= ((grouped[:, :, c] >> bit) & 1) << np.uint32(pos)
    return np.ascontiguousarray(words.astype("<u4").view(np.uint8).reshape(k // GROUP, 3, o, 16))


def sorted_codes_from_fields(fields: np.ndarray) -> np.ndarray:
    """Field layout ``[G, 3, O, 16]`` -> sorted-order codes ``[K, O]``."""
    fields = np.asarray(fields, dtype=np.uint8)
    g, three, o, sixteen = fields.shape
    if three != 3 or sixteen != 16:
        raise ValueError("fields must be [G,3,O,16]")
    words = np.ascontiguousarray(fields).view("<u4").reshape(g, 3, o, 4).astype(np.uint32)
    codes = np.zeros((g, o, GROUP), dtype=np.uint32)
    for c in range(GROUP):
        w, t = divmod(c, 32)
        for bit, (m, pos) in enumerate(field_slots()[t]):
            codes[:, :, c] |= ((words[:, m, :, w] >> np.uint32(pos)) & 1) << np.uint32(bit)
    return np.ascontiguousarray(codes.transpose(0, 2, 1).reshape(g * GROUP, o).astype(np.uint8))


def fields_from_planar(planes: np.ndarray) -> np.ndarray:
    """The bind-time repack: planes ``[G,3,O,16]`` -> fields ``[G,3,O,16]`` (same sorted order)."""
    return fields_from_sorted_codes(codes_from_planar(planes))


# --------------------------------------------------------------------------- fp6 layout
# A second bind-time repack (no reference counterpart), for gfx950's
# v_mfma_scale_f32_16x16x128_f8f6f4 with fp6 e2m3 A operands: a 6-bit field
# with zero sign and exponent bits and the code q in its three mantissa bits is
# exactly q / 8.  One instruction covers a 16-row tile and one group (128
# columns): A lane block kb (lanes 16 kb .. 16 kb + 15, row = lane % 16) holds 32
# fields, field e at bits [6 e, 6 e + 6) of six 32-bit registers, and meets the
# fp8 B element of group column FP6_COLUMN(kb, e) (measured pairing of the
# instruction: A block kb, element e <-> B block 2 (kb % 2) + e // 16, element
# 16 (kb // 2) + e % 16, B block k holding columns 32 k .. 32 k + 31).
# Storage: bytes of the planes' size, ordered [G / 4, O, kb (4), group slot (4),
# 3 words]: the 12 bytes a lane reads for one group of its 4-group batch.  The
# kernel expands the three words s0, s1, s2 into the six registers with
#   R0 = s0 & M0, R2 = (s0 >> 1) & M2, R3 = s1 & M0, R5 = (s1 >> 1) & M2,
#   R1 = s2 & M1, R4 = ((s2 >> 3) with bits 29, 30 from s2 bits 1, 2) & M1
# (M0 = 0xC71C71C7, M1 = 0x71C71C71, M2 = 0x1C71C71C: the mantissa bits of the
# fields in each register); FP6_STORED_BIT restates that map bit by bit.
FP6_M0, FP6_M1, FP6_M2 = 0xC71C71C7, 0x71C71C71, 0x1C71C71C


def fp6_column(kb: int, e: int) -> int:
    """The group column that field e of A lane block kb multiplies."""
    return 32 * (2 * (kb % 2) + e // 16) + 16 * (kb // 2) + e % 16


def fp6_register_bit(e: int, j: int) -> tuple[int, int]:
    """(register, bit) of mantissa bit j of field e."""
    p = 6 * e + j
    return p // 32, p % 32


def fp6_stored_bit(reg: int, bit: int) -> tuple[int, int]:
    """(stored word, bit) that register bit (reg, bit) is expanded from."""
    if reg in (0, 3):
        return reg // 3, bit
    if reg in (2, 5):
        return (0 if reg == 2 else 1), bit + 1
    if reg == 1:
        return 2, bit
    return 2, (bit - 28) if bit in (29, 30) else bit + 3


def _fp6_slots() -> np.ndarray:
    """[kb, e, j] -> stored bit index (word * 32 + bit) within a lane's 3 words."""
    slots = np.zeros((4, 32, 3), dtype=np.int64)
    for kb in range(4):
        for e in range(32):
            for j in range(3):
                w, b = fp6_stored_bit(*fp6_register_bit(e, j))
                slots[kb, e, j] = 32 * w + b
    return slots


def fp6_from_sorted_codes(sorted_codes: np.ndarray) -> np.ndarray:
    """Sorted-order codes ``[K, O]`` -> fp6 layout (uint8, the planes' shape ``[G, 3, O, 16]``)."""
    codes = np.asarray(sorted_codes, dtype=np.uint32)
    k, o = codes.shape
    if k % (4 * GROUP):
        raise ValueError("K must be a multiple of 512")
    g = k // GROUP
    grouped = codes.reshape(g // 4, 4, GROUP, o).transpose(0, 3, 1, 2)  # [G/4, O, slot, 128]
    words = np.zeros((g // 4, o, 4, 4, 3), dtype=np.uint32)          # [G/4, O, kb, slot, 3]
    slots = _fp6_slots()
    for kb in range(4):
        for e in range(32):
            q = grouped[:, :, :, fp6_column(kb, e)]                   # [G/4, O, slot]
            for j in range(3):
                w, b = divmod(int(slots[kb, e, j]), 32)
                words[:, :, kb, :, w] |= ((q >> j) & 1) << np.uint32(b)
    return np.ascontiguousarray(words.astype("<u4").view(np.uint8).reshape(g, 3, o, 16))


def sorted_codes_from_fp6(fp6: np.ndarray) -> np.ndarray:
    """fp6 layout -> sorted-order codes ``[K, O]``."""
    fp6 = np.asarray(fp6, dtype=np.uint8)
    g, three, o, sixteen = fp6.shape
    if three != 3 or sixteen != 16 or g % 4:
        raise ValueError("fp6 payload must be [G,3,O,16] bytes with G % 4 == 0")
    words = np.ascontiguousarray(fp6).view("<u4").reshape(g // 4, o, 4, 4, 3).astype(np.uint32)
    grouped = np.zeros((g // 4, o, 4, GROUP), dtype=np.uint32)
    slots = _fp6_slots()
    for kb in range(4):
        for e in range(32):
            for j in range(3):
                w, b = divmod(int(slots[kb, e, j]), 32)
                grouped[:, :, :, fp6_column(kb, e)] |= ((words[:, :, kb, :, w] >> np.uint32(b)) & 1) << np.uint32(j)
    return np.ascontiguousarray(grouped.transpose(0, 2, 3, 1).reshape(g * GROUP, o).astype(np.uint8))


def fp6_from_planar(planes: np.ndarray) -> np.ndarray:
    """The bind-time repack: planes -> fp6 layout (same sorted order)."""
    return fp6_from_sorted_codes(codes_from_planar(planes))


def fp6_expand(s0: int, s1: int, s2: int) -> list[int]:
    """The kernel's expansion of one lane's three words into six fp6 registers."""
    mid = ((s2 >> 3) & ~0x60000000 | (s2 << 28) & 0x60000000) & 0xFFFFFFFF
    return [s0 & FP6_M0, s2 & FP6_M1, (s0 >> 1) & FP6_M2, s1 & FP6_M0, mid & FP6_M1, (s1 >> 1) & FP6_M2]
