"""Fused RMSNorm / RoPE drop-ins for the HF Qwen3 decode path, on gfx950 kernels.

Reference: ``fused_modules.py`` (``rms_norm_reference`` :30-41,
``fused_rms_norm_forward`` :61-63, ``fused_apply_rotary_pos_emb`` :66-85,
``fused_qwen3_modules`` :88-112).  The reference fuses RMSNorm with Inductor
and RoPE with tensor algebra (5 kernels).  Here each is one HIP launch
(``fx_rmsnorm``, ``fx_head_norm_rope``); the decode path also uses
:func:`add_rms_norm` (residual add + norm, one launch) and
:func:`head_norm_rope` (q/k per-head norm + RoPE + KV-cache write, one launch).

Routing: GPU tensors in bf16/fp16 run the HIP kernels and raise if the library
is missing.  Other dtypes (fp32 models, mixed weight/activation dtypes) and CPU
tensors run the reference's own torch arithmetic, as the reference does for
them.  Rounding points follow stock HF; RoPE is bit-exact to the torch algebra,
RMSNorm differs from torch only by fp32 summation order.
"""
from __future__ import annotations

import ctypes
from contextlib import contextmanager

import torch

from . import _lib

_HALF = (torch.float16, torch.bfloat16)


def rms_norm_reference(hidden_states: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """Stock Qwen3RMSNorm arithmetic as a free function (``fused_modules.py:30-41``)."""
    input_dtype = hidden_states.dtype
    hidden_states = hidden_states.to(torch.float32)
    variance = hidden_states.pow(2).mean(-1, keepdim=True)
    hidden_states = hidden_states * torch.rsqrt(variance + eps)
    return weight * hidden_states.to(input_dtype)


def _aligned(t: torch.Tensor) -> torch.Tensor:
    """Contiguous with a 16-byte aligned start (views at odd offsets are copied)."""
    t = t.contiguous()
    if t.data_ptr() % 16:
        t = t.clone()
    return t


def _hip_ok(*tensors: torch.Tensor) -> bool:
    first = tensors[0]
    return first.is_cuda and first.dtype in _HALF and all(t.dtype == first.dtype for t in tensors)


def rms_norm(hidden_states: torch.Tensor, weight: torch.Tensor, eps: float, *,
             out: torch.Tensor | None = None) -> torch.Tensor:
    """``weight * round(x * rsqrt(mean(x^2) + eps))`` over the last axis, one launch."""
    if not _hip_ok(hidden_states, weight):
        return rms_norm_reference(hidden_states, weight, eps)
    hidden = hidden_states.shape[-1]
    if weight.shape != (hidden,):
        raise ValueError("weight must have shape [hidden]")
    x = _aligned(hidden_states)
    w = _aligned(weight)
    result = out if out is not None else torch.empty_like(x)
    lib = _lib.library()
    _lib.check(lib.fx_rmsnorm(x.data_ptr(), None, w.data_ptr(), result.data_ptr(), None,
                              x.numel() // hidden, hidden, float(eps), _lib.dtype_code(x.dtype),
                              _lib.stream_handle(x.device)), "fx_rmsnorm")
    return result


def add_rms_norm(hidden_states: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                 eps: float, *, out: torch.Tensor, residual_out: torch.Tensor) -> None:
    """Decoder-layer residual add fused with the next RMSNorm (GPU, half dtypes):
    ``residual_out = round(x + residual)``; ``out = rms_norm(residual_out)``."""
    if not _hip_ok(hidden_states, residual, weight, out, residual_out):
        raise ValueError("add_rms_norm needs GPU tensors of one half dtype")
    hidden = hidden_states.shape[-1]
    lib = _lib.library()
    _lib.check(lib.fx_rmsnorm(hidden_states.data_ptr(), residual.data_ptr(), weight.data_ptr(),
                              out.data_ptr(), residual_out.data_ptr(), hidden_states.numel() // hidden,
                              hidden, float(eps), _lib.dtype_code(hidden_states.dtype),
                              _lib.stream_handle(hidden_states.device)), "fx_rmsnorm")


def fused_rms_norm_forward(self, hidden_states):
    """Drop-in for ``Qwen3RMSNorm.forward`` (``fused_modules.py:61-63``)."""
    return rms_norm(hidden_states, self.weight, self.variance_epsilon)


def _check_rope_inputs(q, k):
    if q.ndim != k.ndim or q.dtype != k.dtype or q.shape[-1] != k.shape[-1]:
        raise ValueError("fused RoPE requires q/k with matching rank, dtype and head_dim")


def _rope_torch(q, k, cos, sin, unsqueeze_dim):
    """The reference's tensor algebra (``fused_modules.py:74-85``)."""
    cos = cos.unsqueeze(unsqueeze_dim)
    sin = sin.unsqueeze(unsqueeze_dim)
    q_heads = q.shape[unsqueeze_dim]
    joined = torch.cat((q, k), dim=unsqueeze_dim)
    half = joined.shape[-1] // 2
    rotated = torch.cat((-joined[..., half:], joined[..., :half]), dim=-1)
    embedded = torch.addcmul(joined * cos, rotated, sin)
    return (embedded.narrow(unsqueeze_dim, 0, q_heads),
            embedded.narrow(unsqueeze_dim, q_heads, k.shape[unsqueeze_dim]))


class _HeadCall:
    """Marshals up to four [batch, heads, seq, head_dim] tensors for fx_head_norm_rope."""

    def __init__(self):
        self.inputs, self.outputs, self.weights, self.heads, self.rope, self.strides = [], [], [], [], [], []

    def add(self, x, out, weight, heads, in_strides, out_strides, rope):
        self.inputs.append(x.data_ptr())
        self.outputs.append(out.data_ptr())
        self.weights.append(None if weight is None else weight.data_ptr())
        self.heads.append(int(heads))
        self.rope.append(1 if rope else 0)
        self.strides.extend([int(s) for s in in_strides] + [int(s) for s in out_strides])

    def run(self, *, batch, seq, head_dim, cos, sin, cos_strides, position, eps, rope_mode, dtype, device):
        n = len(self.inputs)
        vp = ctypes.c_void_p
        lib = _lib.library()
        _lib.check(lib.fx_head_norm_rope(
            n, (vp * n)(*self.inputs), (vp * n)(*self.outputs), (vp * n)(*self.weights),
            (ctypes.c_int * n)(*self.heads), (ctypes.c_int * n)(*self.rope),
            (ctypes.c_longlong * (6 * n))(*self.strides), batch, seq, head_dim,
            None if cos is None else cos.data_ptr(), None if sin is None else sin.data_ptr(),
            (ctypes.c_longlong * 2)(*cos_strides), None if position is None else position.data_ptr(),
            float(eps), rope_mode, _lib.dtype_code(dtype), _lib.stream_handle(device)), "fx_head_norm_rope")


def _axes(unsqueeze_dim: int):
    if unsqueeze_dim == 1:   # [batch, heads, seq, head_dim]
        return 1, 2
    if unsqueeze_dim == 2:   # [batch, seq, heads, head_dim]
        return 2, 1
    raise ValueError("unsqueeze_dim must be 1 or 2")


def fused_apply_rotary_pos_emb(q, k, cos, sin, unsqueeze_dim=1):
    """Drop-in for ``apply_rotary_pos_emb`` with the reference's fused (addcmul)
    rounding (``fused_modules.py:66-85``): one HIP launch for q and k."""
    _check_rope_inputs(q, k)
    if not (q.ndim == 4 and _hip_ok(q, k, cos, sin) and cos.shape == sin.shape and cos.ndim == 3):
        return _rope_torch(q, k, cos, sin, unsqueeze_dim)
    head_axis, seq_axis = _axes(unsqueeze_dim)
    batch, seq, dim = q.shape[0], q.shape[seq_axis], q.shape[-1]
    if k.shape[0] != batch or k.shape[seq_axis] != seq or tuple(cos.shape) != (batch, seq, dim):
        return _rope_torch(q, k, cos, sin, unsqueeze_dim)
    q_in = q if q.stride(-1) == 1 else q.contiguous()
    k_in = k if k.stride(-1) == 1 else k.contiguous()
    cs = cos.contiguous()
    sn = sin.contiguous()
    q_out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    k_out = torch.empty(k.shape, dtype=k.dtype, device=k.device)
    call = _HeadCall()
    for src, dst in ((q_in, q_out), (k_in, k_out)):
        call.add(src, dst, None, src.shape[head_axis],
                 (src.stride(0), src.stride(head_axis), src.stride(seq_axis)),
                 (dst.stride(0), dst.stride(head_axis), dst.stride(seq_axis)), rope=True)
    call.run(batch=batch, seq=seq, head_dim=dim, cos=cs, sin=sn, cos_strides=(cs.stride(0), cs.stride(1)),
             position=None, eps=0.0, rope_mode=_lib.ROPE_FUSED, dtype=q.dtype, device=q.device)
    return q_out, k_out


def head_norm_rope(tensors, *, cos, sin, eps, seq=1, batch=1, position=None, rope_mode=_lib.ROPE_STOCK,
                   cos_strides=(0, 0)):
    """One launch over up to four head tensors (decode: q, k, v).

    ``tensors``: list of dicts with ``x`` (input) and ``out`` whose last
    dimension is head_dim (contiguous), ``weight`` (per-head RMSNorm weight or
    None), ``heads``, ``rope`` (bool) and element strides ``in_strides`` /
    ``out_strides`` as (batch, head, position).  ``position`` (device int32
    scalar) offsets the cos/sin rows by ``position * head_dim`` for
    graph-replayed decode.
    """
    head_dim = tensors[0]["x"].shape[-1]
    dtype = tensors[0]["x"].dtype
    for t in tensors:
        for key in ("x", "out"):
            if t[key].shape[-1] != head_dim or t[key].stride(-1) != 1 or t[key].dtype != dtype:
                raise ValueError(f"head_norm_rope: every {key} must end in a contiguous head_dim={head_dim} axis")
        if t.get("weight") is not None and t["weight"].shape != (head_dim,):
            raise ValueError("head_norm_rope: norm weights must have shape [head_dim]")
    call = _HeadCall()
    for t in tensors:
        call.add(t["x"], t["out"], t.get("weight"), t["heads"], t["in_strides"], t["out_strides"], t["rope"])
    call.run(batch=batch, seq=seq, head_dim=head_dim, cos=cos, sin=sin,
             cos_strides=cos_strides, position=position, eps=eps, rope_mode=rope_mode, dtype=dtype,
             device=tensors[0]["x"].device)


@contextmanager
def fused_qwen3_modules(*, rms_norm=True, rope=True):
    """Patch ``Qwen3RMSNorm.forward`` / ``apply_rotary_pos_emb`` at class/module
    scope and restore them on exit (``fused_modules.py:88-112``)."""
    from transformers.models.qwen3 import modeling_qwen3

    applied = {"rms_norm": bool(rms_norm), "rope": bool(rope)}
    originals = {}
    try:
        if rms_norm:
            originals["rms_norm"] = modeling_qwen3.Qwen3RMSNorm.forward
            modeling_qwen3.Qwen3RMSNorm.forward = fused_rms_norm_forward
        if rope:
            originals["rope"] = modeling_qwen3.apply_rotary_pos_emb
            modeling_qwen3.apply_rotary_pos_emb = fused_apply_rotary_pos_emb
        yield applied
    finally:
        if "rms_norm" in originals:
            modeling_qwen3.Qwen3RMSNorm.forward = originals["rms_norm"]
        if "rope" in originals:
            modeling_qwen3.apply_rotary_pos_emb = originals["rope"]
