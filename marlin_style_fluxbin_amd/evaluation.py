"""Dense materialisation of the two-base formats and tensor hashing.

Reference: ``evaluation.py`` (``sha256_file`` :20-25, ``tensor_sha256`` :28-34,
``sha256_token_sequences`` :37-45, ``materialize_global_two_base_weight`` :59-95,
``materialize_hybrid_s8_weight`` :98-175, ``atomic_json`` :205-212).  The file and
token-sequence hashes are the ones the artifact loader and the PPL harness record
(``w3_lut_artifacts.sha256_file``, ``ppl.sha256_token_sequences``), so hashes
recorded by either side compare.  The materialisers are the dequantize step of the two-base
PackedHybridLinear's dense fallback; they run fp32 torch arithmetic in the
reference's order (per base ``(sign * row) * col`` added to a zero start, the
refinement formed the same way and scatter-added at its columns) and cast once.
"""
from __future__ import annotations

import hashlib
import json
import os
from pathlib import Path
from typing import Any, Iterable, Sequence

import torch

from .packing import unpack_two_bases


def sha256_file(path: Path | str) -> str:
    from .w3_lut_artifacts import sha256_file as digest

    return digest(Path(path))


def sha256_token_sequences(sequences: Iterable[Sequence[int]]) -> str:
    from .ppl import sha256_token_sequences as digest

    return digest(sequences)


def atomic_json(path: Path | str, value: dict[str, Any]) -> None:
    """Write ``value`` as sorted, indented JSON through a temporary file and one
    rename, so a reader sees the old file or the new one, never a partial one."""
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    tmp = path.with_name(f".{path.name}.tmp-{os.getpid()}")
    tmp.write_text(json.dumps(value, indent=2, sort_keys=True) + "\n", encoding="utf-8")
    os.replace(tmp, path)


def tensor_sha256(tensor: torch.Tensor) -> str:
    value = tensor.detach().cpu().contiguous()
    digest = hashlib.sha256()
    digest.update(str(value.dtype).encode("ascii"))
    digest.update(json.dumps(list(value.shape)).encode("ascii"))
    digest.update(value.view(torch.uint8).numpy().tobytes())
    return digest.hexdigest()


def _validate_packed_global(sign_codes, row_scales, column_scales, *, group_size, device):
    if sign_codes.ndim != 2 or sign_codes.dtype != torch.uint8:
        raise ValueError("sign codes must be uint8 [O, K/4]")
    out_features, width = sign_codes.shape
    in_features = width * 4
    if in_features % group_size:
        raise ValueError("in_features must be divisible by group_size")
    num_groups = in_features // group_size
    if tuple(row_scales.shape) != (2, out_features, num_groups):
        raise ValueError("row-scale shape drifted")
    if tuple(column_scales.shape) != (2, num_groups, group_size):
        raise ValueError("column-scale shape drifted")
    for name, t in (("row", row_scales), ("column", column_scales)):
        if not t.is_floating_point() or not torch.isfinite(t).all():
            raise ValueError(f"{name} scales must be finite floating point")
    bases = unpack_two_bases(sign_codes.to(device=device))
    return bases, out_features, num_groups


def materialize_global_two_base_weight(sign_codes, row_scales, column_scales, *, group_size, device,
                                       output_dtype):
    bases, out_features, num_groups = _validate_packed_global(
        sign_codes, row_scales, column_scales, group_size=group_size, device=device)
    recon = torch.zeros(out_features, num_groups, group_size, device=device, dtype=torch.float32)
    row = row_scales.to(device=device, dtype=torch.float32)
    col = column_scales.to(device=device, dtype=torch.float32)
    for b in range(2):
        term = bases[b].reshape(out_features, num_groups, group_size).to(torch.float32)
        term.mul_(row[b].unsqueeze(-1))
        term.mul_(col[b].unsqueeze(0))
        recon.add_(term)
    return recon.reshape(out_features, -1).to(dtype=output_dtype)


def materialize_hybrid_s8_weight(global_sign_codes, global_row_scales, global_column_scales,
                                 refinement_indices, refinement_sign_codes, refinement_row_scales,
                                 refinement_column_scales, *, group_size, columns_per_group, device,
                                 output_dtype):
    weight = materialize_global_two_base_weight(global_sign_codes, global_row_scales, global_column_scales,
                                                group_size=group_size, device=device,
                                                output_dtype=torch.float32)
    out_features, in_features = weight.shape
    num_groups = in_features // group_size
    if refinement_indices.dtype not in (torch.int16, torch.int32, torch.int64):
        raise TypeError("refinement indices must use an integer dtype")
    if tuple(refinement_indices.shape) != (num_groups, columns_per_group):
        raise ValueError("refinement indices have the wrong shape")
    indices = refinement_indices.to(device=device, dtype=torch.int64)
    if torch.any(indices < 0) or torch.any(indices >= group_size):
        raise ValueError("refinement indices are outside the group")
    if columns_per_group > 1 and torch.any(indices[:, 1:] <= indices[:, :-1]):
        raise ValueError("refinement indices must be sorted and unique")
    if tuple(refinement_sign_codes.shape) != (out_features, num_groups * columns_per_group // 4):
        raise ValueError("refinement sign-code shape drifted")
    if tuple(refinement_row_scales.shape) != (2, out_features, num_groups):
        raise ValueError("refinement row-scale shape drifted")
    if tuple(refinement_column_scales.shape) != (2, num_groups, columns_per_group):
        raise ValueError("refinement column-scale shape drifted")
    for t in (refinement_row_scales, refinement_column_scales):
        if not t.is_floating_point() or not torch.isfinite(t).all():
            raise ValueError("refinement scales must be finite floating point")
    bases = unpack_two_bases(refinement_sign_codes.to(device=device)).reshape(
        2, out_features, num_groups, columns_per_group)
    row = refinement_row_scales.to(device=device, dtype=torch.float32)
    col = refinement_column_scales.to(device=device, dtype=torch.float32)
    selected = torch.zeros(out_features, num_groups, columns_per_group, device=device, dtype=torch.float32)
    for b in range(2):
        term = bases[b].to(torch.float32)
        term.mul_(row[b].unsqueeze(-1))
        term.mul_(col[b].unsqueeze(0))
        selected.add_(term)
    grouped = weight.reshape(out_features, num_groups, group_size)
    grouped.scatter_add_(2, indices.unsqueeze(0).expand(out_features, -1, -1), selected)
    return grouped.reshape(out_features, in_features).to(dtype=output_dtype)
