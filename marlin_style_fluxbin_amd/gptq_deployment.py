"""W3 g128 planar payload: GPTQ int3 conversion, validation and dequantize.

Mirrors the public surface of the reference's ``gptq_deployment.py``
(maxiu188-afk/Marlin_Style_Fluxbin ``src/fluxbin_style/gptq_deployment.py``) with
two extensions the benchmark configs need:

* an optional ``zeros`` field (uint8 ``[G, O]`` per-group zero-points); when it
  is absent every zero-point is 4, the reference's only supported value;
* fp16 scales next to the reference's bf16 scales.

Layout (``gptq_deployment.py:199-227``): ``planes`` uint8 ``[G, 3, O, 16]`` holds
bit ``p`` of the code of sorted column ``128 g + 8 c + j`` of row ``o`` at bit
``j`` of byte ``planes[g, p, o, c]``; plane 2 is stored inverted, so
``q - 4 = b0 + 2 b1 - 4 * stored_b2``.  ``perm`` int16 ``[K]`` maps a sorted
column to the original input column (the ``desc_act`` canonicalisation).

GPU tensors are dequantized by the HIP kernel behind ``fx_w3_restore``; the
torch code here handles CPU tensors (offline conversion, the CPU dense route the
reference also offers, and tests).
"""
from __future__ import annotations

from typing import Mapping

import torch

FORMAT = "gptq-w3-g128-planar-amd-v1"
REFERENCE_FORMAT = "gptq-w3-g128-sym-planar-m1-v1"
GROUP_SIZE = 128
BITS = 3
ZERO = 4
FIELDS = ("planes", "scales", "perm")
OPTIONAL_FIELDS = ("zeros",)
SCALE_DTYPES = (torch.bfloat16, torch.float16)

# Bit offset of every code inside one 96-bit block of the GPTQ int3 stream:
# code i of a block of 32 occupies bits 3i .. 3i+2 of word0 | word1<<32 | word2<<64.
_CODE_BITS = torch.arange(32, dtype=torch.int64) * 3


def _require_cpu_int32(name: str, value: torch.Tensor, ndim: int) -> None:
    if value.device.type != "cpu" or value.dtype != torch.int32 or value.ndim != ndim:
        raise ValueError(f"{name} must be CPU int32 rank {ndim}")
    if not value.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _bitstream_unpack(words: torch.Tensor) -> torch.Tensor:
    """``[blocks, 3, N]`` int32 -> ``[blocks, 32, N]`` codes (little-endian 96-bit stream)."""
    u = words.to(torch.int64) & 0xFFFFFFFF
    codes = torch.zeros(words.shape[0], 32, words.shape[2], dtype=torch.int64)
    for bit in range(3):
        position = _CODE_BITS + bit                       # [32]
        word = position // 32
        shift = position % 32
        selected = u[:, word, :]                          # [blocks, 32, N]
        codes |= ((selected >> shift.view(1, 32, 1)) & 1) << bit
    return codes.to(torch.uint8)


def _bitstream_pack(codes: torch.Tensor) -> torch.Tensor:
    """``[blocks, 32, N]`` codes -> ``[blocks, 3, N]`` int32."""
    c = codes.to(torch.int64)
    words = torch.zeros(c.shape[0], 3, c.shape[2], dtype=torch.int64)
    for bit in range(3):
        position = _CODE_BITS + bit
        for w in range(3):
            mask = (position // 32) == w
            if mask.any():
                bits = ((c[:, mask, :] >> bit) & 1) << (position[mask] % 32).view(1, -1, 1)
                words[:, w, :] |= bits.sum(dim=1)
    words = torch.where(words >= 2**31, words - 2**32, words)
    return words.to(torch.int32)


def unpack_gptq_w3_qweight(qweight: torch.Tensor) -> torch.Tensor:
    """Logical unsigned codes ``[K, O]`` from GPTQ int3 ``qweight [3K/32, O]``."""
    _require_cpu_int32("qweight", qweight, 2)
    if qweight.shape[0] % 3:
        raise ValueError("packed row count must be divisible by three")
    blocks = qweight.reshape(qweight.shape[0] // 3, 3, qweight.shape[1])
    return _bitstream_unpack(blocks).reshape(-1, qweight.shape[1])


def unpack_gptq_w3_qzeros(qzeros: torch.Tensor, *, qzero_format: int) -> torch.Tensor:
    """Logical zero points ``[G, O]``; qzero format 1 (raw GPTQ) stores zero - 1."""
    _require_cpu_int32("qzeros", qzeros, 2)
    if qzero_format not in (1, 2):
        raise ValueError("qzero_format must be 1 (raw GPTQ) or 2 (loaded GPTQ_V2)")
    if qzeros.shape[1] % 3:
        raise ValueError("packed column count must be divisible by three")
    t = qzeros.T.contiguous()
    blocks = t.reshape(t.shape[0] // 3, 3, t.shape[1])
    zeros = _bitstream_unpack(blocks).reshape(-1, t.shape[1]).T.contiguous()
    if qzero_format == 1:
        zeros = ((zeros.to(torch.int16) + 1) & 7).to(torch.uint8)
    return zeros


def pack_gptq_w3_codes(codes: torch.Tensor, *, packed_axis: int = 0) -> torch.Tensor:
    """Canonical GPTQ int3 packer (test/fixture helper)."""
    if codes.device.type != "cpu" or codes.dtype != torch.uint8 or codes.ndim != 2:
        raise ValueError("codes must be CPU uint8 rank two")
    logical = codes if packed_axis == 0 else codes.T
    if logical.shape[0] % 32 or bool((logical > 7).any()):
        raise ValueError("packed logical dimension must be divisible by 32 and codes must be W3")
    blocks = logical.contiguous().reshape(-1, 32, logical.shape[1])
    packed = _bitstream_pack(blocks).reshape(-1, logical.shape[1])
    return packed if packed_axis == 0 else packed.T.contiguous()


def _pack_bytes(bits: torch.Tensor) -> torch.Tensor:
    """``[..., 128]`` 0/1 uint8 -> ``[..., 16]`` uint8, LSB-first within each byte."""
    if bits.dtype != torch.uint8 or bits.shape[-1] != GROUP_SIZE:
        raise ValueError("bit tensor must be uint8 with a 128-element final dimension")
    weights = (2 ** torch.arange(8, dtype=torch.int32)).to(bits.device)
    chunks = bits.reshape(*bits.shape[:-1], 16, 8).to(torch.int32)
    return (chunks * weights).sum(-1).to(torch.uint8)


def _unpack_bytes(values: torch.Tensor) -> torch.Tensor:
    if values.dtype != torch.uint8 or values.shape[-1] != 16:
        raise ValueError("packed planes must be uint8 with a 16-byte final dimension")
    shifts = torch.arange(8, dtype=torch.int32, device=values.device)
    return ((values.to(torch.int32).unsqueeze(-1) >> shifts) & 1).to(torch.uint8).flatten(-2)


def inspect_gptq_checkpoint(tensors: Mapping[str, torch.Tensor], *, qzero_format: int = 1) -> dict:
    required = {"qweight", "qzeros", "scales", "g_idx"}
    if set(tensors) != required:
        raise ValueError(f"expected exactly {sorted(required)}")
    qweight, qzeros, scales, g_idx = (tensors[n] for n in ("qweight", "qzeros", "scales", "g_idx"))
    _require_cpu_int32("qweight", qweight, 2)
    _require_cpu_int32("qzeros", qzeros, 2)
    _require_cpu_int32("g_idx", g_idx, 1)
    if scales.device.type != "cpu" or scales.dtype != torch.float16 or scales.ndim != 2:
        raise ValueError("scales must be contiguous CPU float16 [G,O]")
    if not scales.is_contiguous() or not torch.isfinite(scales).all():
        raise ValueError("scales must be contiguous and finite")
    codes = unpack_gptq_w3_qweight(qweight)
    zeros = unpack_gptq_w3_qzeros(qzeros, qzero_format=qzero_format)
    k, o = codes.shape
    if k % GROUP_SIZE or k > 32767:
        raise ValueError("K must be divisible by 128 and representable by int16")
    groups = k // GROUP_SIZE
    if tuple(scales.shape) != (groups, o) or tuple(zeros.shape) != (groups, o):
        raise ValueError("qzero/scale shape does not match qweight")
    if tuple(g_idx.shape) != (k,) or int(g_idx.min()) != 0 or int(g_idx.max()) != groups - 1:
        raise ValueError("g_idx shape or range drifted")
    counts = torch.bincount(g_idx.to(torch.int64), minlength=groups)
    if not bool((counts == GROUP_SIZE).all()):
        raise ValueError("each g_idx group must contain exactly 128 input columns")
    perm = torch.argsort(g_idx, stable=True)
    canonical = torch.arange(groups, dtype=torch.int32).repeat_interleave(GROUP_SIZE)
    if not torch.equal(g_idx[perm], canonical):
        raise ValueError("sorted g_idx is not canonical group128")
    return {
        "bits": BITS, "group_size": GROUP_SIZE,
        "qweight_shape": list(qweight.shape), "qzeros_shape": list(qzeros.shape),
        "scales_shape": list(scales.shape), "g_idx_shape": list(g_idx.shape),
        "in_features": k, "out_features": o, "groups": groups, "qzero_format": qzero_format,
        "decoded_zero_unique": [int(v) for v in torch.unique(zeros).tolist()],
        "permutation_identity": bool(torch.equal(perm, torch.arange(k))),
    }


def validate_planar_w3(layout: Mapping[str, torch.Tensor], *, check_values: bool = True) -> tuple[int, int]:
    """Validate the payload ABI; returns ``(out_features, in_features)``.

    ``check_values=False`` is the allocation-free runtime form: shapes, dtypes,
    devices and contiguity only.  The full form adds finite scales, zero-points
    in [0, 7] and a bijective ``perm``.
    """
    keys = set(layout)
    if keys != set(FIELDS) and keys != set(FIELDS) | set(OPTIONAL_FIELDS):
        raise ValueError(f"expected exactly {FIELDS} (+ optional {OPTIONAL_FIELDS})")
    planes, scales, perm = (layout[name] for name in FIELDS)
    if planes.dtype != torch.uint8 or planes.ndim != 4 or planes.shape[1] != 3 or planes.shape[3] != 16:
        raise ValueError("planes must be uint8 [G,3,O,16]")
    groups, _, out_features, _ = planes.shape
    if scales.dtype not in SCALE_DTYPES or tuple(scales.shape) != (groups, out_features):
        raise ValueError("deployment scales must be bfloat16 or float16 [G,O]")
    in_features = groups * GROUP_SIZE
    if in_features > 32767:
        raise ValueError("perm indices must be representable by int16")
    if perm.dtype != torch.int16 or tuple(perm.shape) != (in_features,):
        raise ValueError("perm must be int16 [K]")
    zeros = layout.get("zeros")
    if zeros is not None and (zeros.dtype != torch.uint8 or tuple(zeros.shape) != (groups, out_features)):
        raise ValueError("zeros must be uint8 [G,O]")
    if any(value.device != planes.device or not value.is_contiguous() for value in layout.values()):
        raise ValueError("layout tensors must be contiguous on one device")
    if check_values:
        if not torch.isfinite(scales).all():
            raise ValueError("scales must be finite")
        if zeros is not None and bool((zeros > 7).any()):
            raise ValueError("zero-points must be in [0,7]")
        p64 = perm.to(torch.int64)
        if (int(p64.min()) != 0 or int(p64.max()) != in_features - 1
                or torch.unique(p64).numel() != in_features):
            raise ValueError("perm must be a bijection over K")
    return out_features, in_features


def planar_from_codes(codes: torch.Tensor, perm: torch.Tensor | None = None) -> torch.Tensor:
    """Original-order unsigned codes ``[K, O]`` -> planes ``[G, 3, O, 16]``."""
    k, o = codes.shape
    if k % GROUP_SIZE:
        raise ValueError("K must be divisible by 128")
    sorted_codes = codes if perm is None else codes[perm.to(torch.int64)]
    grouped = sorted_codes.reshape(k // GROUP_SIZE, GROUP_SIZE, o).permute(0, 2, 1)
    b0 = grouped & 1
    b1 = (grouped >> 1) & 1
    b2_inverted = 1 - ((grouped >> 2) & 1)
    return torch.stack((_pack_bytes(b0), _pack_bytes(b1), _pack_bytes(b2_inverted)), dim=1).contiguous()


def convert_gptq_w3_to_planar(tensors: Mapping[str, torch.Tensor], *, qzero_format: int = 1,
                              scale_dtype: torch.dtype = torch.bfloat16,
                              allow_zeros: bool = False) -> dict[str, torch.Tensor]:
    """Raw GPTQ W3 g128 checkpoint tensors -> planar payload.

    Without ``allow_zeros`` only a constant zero-point of 4 is accepted (the
    reference's fast-path contract); with it, other zero-points are stored in
    the ``zeros`` field.
    """
    facts = inspect_gptq_checkpoint(tensors, qzero_format=qzero_format)
    if scale_dtype not in SCALE_DTYPES:
        raise ValueError("scale_dtype must be bfloat16 or float16")
    uniform = facts["decoded_zero_unique"] == [ZERO]
    if not uniform and not allow_zeros:
        raise ValueError(
            f"constant-zero layout requires decoded zero=4, got {facts['decoded_zero_unique']}")
    codes = unpack_gptq_w3_qweight(tensors["qweight"])
    perm64 = torch.argsort(tensors["g_idx"], stable=True)
    layout = {
        "planes": planar_from_codes(codes, perm64),
        # GPTQModel reloads fp16 checkpoint scales as bf16 before dequantizing;
        # the bf16 deployment value is the same number it multiplies by.
        "scales": tensors["scales"].to(scale_dtype).contiguous(),
        "perm": perm64.to(torch.int16).contiguous(),
    }
    if not uniform:
        layout["zeros"] = unpack_gptq_w3_qzeros(tensors["qzeros"], qzero_format=qzero_format).contiguous()
    validate_planar_w3(layout)
    return layout


def decode_planar_w3_codes(layout: Mapping[str, torch.Tensor], *, original_order: bool = True) -> torch.Tensor:
    """Unsigned codes ``[K, O]`` (original column order unless ``original_order=False``)."""
    out_features, in_features = validate_planar_w3(layout, check_values=False)
    planes = layout["planes"]
    b0 = _unpack_bytes(planes[:, 0])
    b1 = _unpack_bytes(planes[:, 1])
    b2 = 1 - _unpack_bytes(planes[:, 2])
    sorted_codes = (b0 | (b1 << 1) | (b2 << 2)).permute(0, 2, 1).reshape(in_features, out_features)
    if not original_order:
        return sorted_codes.contiguous()
    restored = torch.empty_like(sorted_codes)
    restored[layout["perm"].to(torch.int64)] = sorted_codes
    return restored


def _signed_sorted(layout) -> torch.Tensor:
    """``q - zero`` int16 ``[G, O, 128]`` in sorted column order."""
    out_features, in_features = validate_planar_w3(layout, check_values=False)
    groups = in_features // GROUP_SIZE
    codes = decode_planar_w3_codes(layout, original_order=False).to(torch.int16)
    codes = codes.reshape(groups, GROUP_SIZE, out_features).permute(0, 2, 1)
    zeros = layout.get("zeros")
    zero = (zeros.to(torch.int16) if zeros is not None
            else torch.full((groups, out_features), ZERO, dtype=torch.int16, device=codes.device))
    return codes - zero.unsqueeze(-1)


def restore_planar_w3(layout: Mapping[str, torch.Tensor], *, dtype: torch.dtype = torch.bfloat16,
                      perm_identity: bool | None = None) -> torch.Tensor:
    """Dense ``[O, K]`` weight ``round_dtype(round_scale_dtype(s * (q - z)))``.

    GPU layouts are dequantized by the HIP kernel (``fx_w3_restore``);
    ``perm_identity`` (known to the caller, else compared on the device) picks
    its identity-order form.  CPU layouts ignore it.
    """
    out_features, in_features = validate_planar_w3(layout, check_values=False)
    if dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError("dtype must be float16, bfloat16 or float32")
    if layout["planes"].is_cuda and dtype != torch.float32:
        from .w3_lut_deployment import restore_planar_w3_device
        return restore_planar_w3_device(layout, dtype=dtype, perm_identity=perm_identity)
    signed = _signed_sorted(layout)
    # scale dtype x int16 rounds once to the scale dtype, as the bf16 GPTQ dequantizer does
    product = layout["scales"].unsqueeze(-1) * signed
    sorted_weight = product.permute(1, 0, 2).reshape(out_features, in_features)
    weight = torch.empty_like(sorted_weight)
    weight[:, layout["perm"].to(torch.int64)] = sorted_weight
    return weight.to(dtype=dtype).contiguous()


def structural_w3_matvec(x: torch.Tensor, layout: Mapping[str, torch.Tensor]) -> torch.Tensor:
    """fp32 ``x [M, K] -> [M, O]`` with ``s * (q - z)`` weights (no per-weight rounding).

    On GPU this is the HIP LUT kernel with a single K split, whose fp32 result
    is returned before any cast; on CPU a grouped torch evaluation.
    """
    out_features, in_features = validate_planar_w3(layout, check_values=False)
    if x.ndim != 2 or x.shape[1] != in_features:
        raise ValueError("x must have shape [M,K]")
    if x.device != layout["planes"].device:
        raise ValueError("x and layout must share a device")
    if x.is_cuda:
        from .w3_lut_deployment import gemv_fp32_device
        return gemv_fp32_device(x, layout, arithmetic="structural")
    signed = _signed_sorted(layout).float()                        # [G, O, 128]
    sorted_x = x[:, layout["perm"].long()].float().reshape(x.shape[0], -1, GROUP_SIZE)
    dots = torch.einsum("gok,mgk->mgo", signed, sorted_x)
    return (dots * layout["scales"].float().unsqueeze(0)).sum(1)


def bf16_weight_semantics_w3_matvec(x: torch.Tensor, layout: Mapping[str, torch.Tensor]) -> torch.Tensor:
    """fp32 grouped matvec plus the per-weight bf16 rounding of ``s * (q - z)``.

    For bf16 scales and zero-points 3 or 4 only signed codes +-3 round; the
    correction ``(bf16(3 s) - 3 s) * (sum_{q-z=3} x - sum_{q-z=-3} x)`` restores the
    dequantize-then-matmul value (reference ``gptq_deployment.py:280-315``).
    """
    out_features, in_features = validate_planar_w3(layout, check_values=False)
    if x.ndim != 2 or x.shape[1] != in_features:
        raise ValueError("x must have shape [M,K]")
    if layout["scales"].dtype != torch.bfloat16:
        raise ValueError("bf16 weight semantics require bf16 scales")
    zeros = layout.get("zeros")
    if zeros is not None and not bool(((zeros == 3) | (zeros == 4)).all()):
        raise ValueError("bf16 weight semantics support zero-points 3 and 4")
    if x.is_cuda:
        from .w3_lut_deployment import gemv_fp32_device
        return gemv_fp32_device(x, layout, arithmetic="decoded_bf16")
    signed = _signed_sorted(layout)
    sorted_x = x[:, layout["perm"].long()].float().reshape(x.shape[0], -1, GROUP_SIZE)
    scales = layout["scales"]
    delta = (scales * 3).to(torch.bfloat16).float() - 3.0 * scales.float()
    integer_dot = torch.einsum("gok,mgk->mgo", signed.float(), sorted_x)
    correction = torch.einsum("gok,mgk->mgo", ((signed == 3).float() - (signed == -3).float()), sorted_x)
    return (integer_dot * scales.float().unsqueeze(0) + correction * delta.unsqueeze(0)).sum(1)


def layout_storage(layout: Mapping[str, torch.Tensor]) -> dict:
    out_features, in_features = validate_planar_w3(layout)
    sizes = {name: value.numel() * value.element_size() for name, value in layout.items()}
    total = sum(sizes.values())
    return {
        "format": FORMAT if "zeros" in layout or layout["scales"].dtype != torch.bfloat16 else REFERENCE_FORMAT,
        "shape": [out_features, in_features],
        "tensor_bytes": sizes,
        "total_bytes": total,
        "bits_per_weight": total * 8 / (out_features * in_features),
    }
