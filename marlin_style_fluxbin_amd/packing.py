"""Compact, lossless storage of two {-1, +1} binary bases (artifact format).

Reference: ``packing.py:14-49``.  Four K positions per byte; column ``4q + i`` of
base ``b`` is bit ``2i + b`` of byte ``q``.
"""
from __future__ import annotations

import torch

TWO_BASE_PACKED_FORMAT = "fluxbin-two-base-interleaved-2bit-v1"


def pack_two_bases(bases: torch.Tensor) -> torch.Tensor:
    """``[2, O, K]`` signs in {-1, +1} -> uint8 ``[O, K/4]``."""
    if bases.ndim != 3 or bases.shape[0] != 2:
        raise ValueError("bases must have shape [2, out_features, in_features]")
    if bases.shape[-1] % 4:
        raise ValueError("in_features must be divisible by four")
    if not torch.all((bases == -1) | (bases == 1)):
        raise ValueError("bases must contain only -1 and +1")
    o, k = bases.shape[1:]
    bits = (bases > 0).to(torch.uint8).reshape(2, o, k // 4, 4)
    shift = torch.arange(4, device=bases.device, dtype=torch.uint8) * 2
    packed = torch.bitwise_left_shift(bits[0], shift) | torch.bitwise_left_shift(bits[1], shift + 1)
    return packed.sum(dim=-1, dtype=torch.uint8)  # disjoint bits: the sum is the OR


def unpack_two_bases(codes: torch.Tensor) -> torch.Tensor:
    """uint8 ``[O, K/4]`` -> int8 bases ``[2, O, K]``."""
    if codes.ndim != 2 or codes.dtype != torch.uint8:
        raise ValueError("codes must be a uint8 tensor shaped [out_features, K/4]")
    shift = torch.arange(4, device=codes.device, dtype=torch.uint8) * 2
    expanded = codes.unsqueeze(-1)
    b0 = torch.bitwise_and(torch.bitwise_right_shift(expanded, shift), 1)
    b1 = torch.bitwise_and(torch.bitwise_right_shift(expanded, shift + 1), 1)
    return torch.stack((b0, b1)).to(torch.int8).mul(2).sub(1).reshape(2, codes.shape[0], codes.shape[1] * 4)
