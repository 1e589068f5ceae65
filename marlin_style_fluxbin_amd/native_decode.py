"""Native batch-1 Qwen3 decode: every step is a short, fixed chain of HIP kernels.

Same protocol and interface as :class:`static_decode.StaticDecodeSession`
(reference ``static_decode.py:26-138``): prefill the real prefix (through the HF
model and its dense fallback), keep the prefix KV, decode a fixed continuation,
capture all steps in one hipGraph, time a replay.  What differs is the step:
instead of the HF module tree (~27 kernels per layer) each decoder layer is,
with structural W3 Linears,

    q|k|v GEMV normalising the residual -> attention over key splits with q/k
    norm, RoPE and the KV-cache write folded in -> the splits' combine -> o
    GEMV adding into the residual -> gate|up GEMV normalising, with SwiGLU ->
    down GEMV adding into the residual

(6 launches; 5 while one split covers the context).  Each token starts with one
launch for the embedding row and its RMSNorm statistics (which also merges the
previous token's argmax partials) and ends with the final RMSNorm + bf16 LM head
launch; the last token's argmax merge is one more launch per sequence.  With
the hybrid two-base g128/s8 Linears of ``PackedHybridLinear`` the chain is the
same with the hybrid GEMV's normalising prologue and residual epilogue
(``fx_hybrid_gemv_segments_rmsnormed``, ``fx_hybrid_gemv_residual``), the
SwiGLU formed in the down GEMV's prologue (6 per layer).  Other Linears (dense bf16, the bf16
arm, ``torch.matmul``) run between add+RMSNorm kernels and the same attention
launches.  The arithmetic and rounding points are the stock HF Qwen3 modules'
(RMSNorm, RoPE, SDPA with fp32 softmax, SwiGLU).
"""
from __future__ import annotations

import math
import time

import torch

from . import _lib
from .fused_modules import add_rms_norm
from .static_decode import graph_kernel_count
from .deployment import HybridSegmentsGemv, PackedHybridLinear
from .w3_lut_deployment import PackedW3Linear, W3Gemv

_ATTN = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj")
_MLP = ("mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")


def _one_launch_w3(module) -> bool:
    """A W3 Linear whose packed route is the one-launch MFMA GEMV (one group per
    split, no bias): the form that fuses with its neighbours into one GEMV.
    Table-route modules (``groups_per_split > 1``) keep their own split contract
    and summation order."""
    return isinstance(module, PackedW3Linear) and not module.uses_table_route and module.bias is None


def _structural_w3(module) -> bool:
    """A one-launch W3 Linear with structural arithmetic: what the fused decode
    forms (SwiGLU epilogue, residual epilogue, normalising prologue) compute."""
    return _one_launch_w3(module) and module.arithmetic == "structural"


class _Linear:
    """One decode Linear writing ``out``: the W3 MFMA GEMV (either arithmetic), the
    module's own table route (``groups_per_split > 1``: ``fx_w3_m1_out`` with its
    row tile and split, as ``PackedW3Linear.forward`` runs it), the hybrid two-base
    GEMV (``fx_hybrid_gemv`` through the module's own packed kernel and
    workspace), or a dense matmul."""

    def __init__(self, module):
        self.gemv = None
        self.call = None
        if isinstance(module, PackedW3Linear) and module.uses_table_route:
            self.call = module._packed_kernel(1, module.planes.device)
        elif isinstance(module, PackedW3Linear):
            self.gemv = W3Gemv(module.layout(), arithmetic=module.arithmetic)
            self.call = self.gemv
        elif isinstance(module, PackedHybridLinear):
            self.call = module._packed_kernel(1, module.codes.device)
        elif isinstance(module, torch.nn.Linear):
            weight = module.weight
            self.call = lambda x, out: torch.matmul(x, weight.t(), out=out)
        else:
            raise TypeError(f"unsupported Linear type {type(module).__name__}")
        self.packed = not isinstance(module, torch.nn.Linear)
        self.bias = module.bias

    def __call__(self, x, out):
        self.call(x, out)
        if self.bias is not None:
            out.add_(self.bias)


class _FusedLinear:
    """Linears that read the same activation, run as one GEMV over their
    concatenated rows (q|k|v, gate|up): one launch instead of several.  W3 payloads
    concatenate along O when K, arithmetic, scale dtype, zero-point presence and
    the column permutation agree; hybrid two-base payloads run as one
    ``fx_hybrid_gemv_segments`` launch; dense weights concatenate along O.  Each output
    row is computed exactly as it would be alone, so the outputs are bit-identical
    to separate calls.  ``None`` from :meth:`build` when the modules do not fuse."""

    def __init__(self, call, widths):
        self.call = call
        self.widths = widths

    @staticmethod
    def build(modules):
        if any(isinstance(m, PackedW3Linear) and m.uses_table_route for m in modules):
            return None  # each keeps its own split contract
        if all(isinstance(m, PackedW3Linear) for m in modules):
            layouts = [m.layout() for m in modules]
            first = layouts[0]
            same = all(
                m.in_features == modules[0].in_features and m.arithmetic == modules[0].arithmetic
                and l["scales"].dtype == first["scales"].dtype and ("zeros" in l) == ("zeros" in first)
                and torch.equal(l["perm"], first["perm"]) for m, l in zip(modules, layouts))
            if not same or any(m.bias is not None for m in modules):
                return None
            fused = {"planes": torch.cat([l["planes"] for l in layouts], dim=2).contiguous(),
                     "scales": torch.cat([l["scales"] for l in layouts], dim=1).contiguous(),
                     "perm": first["perm"]}
            if "zeros" in first:
                fused["zeros"] = torch.cat([l["zeros"] for l in layouts], dim=1).contiguous()
            gemv = W3Gemv(fused, arithmetic=modules[0].arithmetic)
            return _FusedLinear(gemv, [m.out_features for m in modules])
        if all(isinstance(m, PackedHybridLinear) for m in modules):
            try:
                gemv = HybridSegmentsGemv(modules)
            except ValueError:
                return None
            return _FusedLinear(gemv, [m.out_features for m in modules])
        if all(type(m) is torch.nn.Linear for m in modules) and all(m.bias is None for m in modules):
            weight = torch.cat([m.weight for m in modules], dim=0).contiguous()
            return _FusedLinear(lambda x, out: torch.matmul(x, weight.t(), out=out),
                                [m.out_features for m in modules])
        return None

    def __call__(self, x, out):
        self.call(x, out)


def interleave_gate_up(gate: dict, up: dict) -> dict:
    """W3 payload whose rows alternate gate row r and up row r (planes, scales and
    zero-points alike), the layout ``fx_w3_gemv_swiglu`` reads."""
    def pair(a, b, dim):
        return torch.stack([a, b], dim=dim + 1).flatten(dim, dim + 1).contiguous()

    fused = {"planes": pair(gate["planes"], up["planes"], 2), "scales": pair(gate["scales"], up["scales"], 1),
             "perm": gate["perm"]}
    if "zeros" in gate:
        fused["zeros"] = pair(gate["zeros"], up["zeros"], 1)
    return fused


class _GateUpSwiGLU:
    """gate_proj, up_proj and SiLU(gate) * up of a Qwen3 MLP as one launch
    (``fx_w3_gemv_swiglu`` over the row-interleaved payload), bit-identical to the
    two GEMVs followed by the SwiGLU kernel.  ``None`` from :meth:`build` unless
    both Linears are structural W3 with matching K, scale dtype, zero-point
    presence and column permutation, equal widths and no bias."""

    def __init__(self, layout, width):
        self.layout = layout
        self.width = width
        self.lib = _lib.library()
        perm = layout["perm"]
        identity = torch.equal(perm.long(), torch.arange(perm.numel(), device=perm.device))
        self.perm_ptr = None if identity else perm.data_ptr()
        self.zeros_ptr = _lib.ptr(layout.get("zeros"))
        self.scale_code = _lib.dtype_code(layout["scales"].dtype)
        self.in_features = perm.numel()

    @staticmethod
    def build(gate, up):
        if not (_structural_w3(gate) and _structural_w3(up)):
            return None
        g, u = gate.layout(), up.layout()
        if (gate.in_features != up.in_features
                or gate.out_features != up.out_features or g["scales"].dtype != u["scales"].dtype
                or ("zeros" in g) != ("zeros" in u) or not torch.equal(g["perm"], u["perm"])):
            return None
        return _GateUpSwiGLU(interleave_gate_up(g, u), gate.out_features)

    def __call__(self, x, out):
        _lib.check(self.lib.fx_w3_gemv_swiglu(
            x.data_ptr(), _lib.dtype_code(x.dtype), self.layout["planes"].data_ptr(),
            self.layout["scales"].data_ptr(), self.scale_code, self.zeros_ptr, self.perm_ptr, None, out.data_ptr(),
            2 * self.width, self.in_features, _lib.PAYLOAD_PLANAR, _lib.stream_handle(x.device)),
            "fx_w3_gemv_swiglu")


def inverse_index(perm: torch.Tensor) -> torch.Tensor | None:
    """``inv`` with ``inv[perm[k]] = k`` (int16, on perm's device), or None for the
    identity: where a producer writes value i so that a GEMV whose sorted column
    k reads activation ``perm[k]`` finds it at position k."""
    k = perm.numel()
    order = torch.arange(k, device=perm.device)
    p = perm.long()
    if torch.equal(p, order):
        return None
    if not torch.equal(torch.sort(p).values, order):
        raise ValueError("column permutation is not a bijection of [0, K)")
    inv = torch.empty(k, dtype=torch.int16, device=perm.device)
    inv[p] = order.to(torch.int16)
    return inv


class _ResidualStream:
    """The decoder layers' residual adds and RMSNorms threaded through the GEMVs:
    the o and down GEMVs add their output into the residual in place and write
    per-16-row sums of its squares; the q|k|v and gate|up GEMVs read the residual
    and normalise it on the fly from those sums.  W3 (``kind`` "w3"):
    ``fx_w3_gemv_residual`` / ``fx_w3_gemv_rmsnormed``, gate|up with the SwiGLU
    epilogue, when every layer's o, down, q|k|v and gate|up are one-launch W3
    (q|k|v sharing one column permutation, gate|up another); with
    ``payload_format`` fields (the default) every layer's four payloads are
    repacked once into the field layout (``fx_w3_planes_to_fields``), whose
    dequantization costs half the instructions.  Hybrid two-base (``kind``
    "hybrid"): ``fx_hybrid_gemv_residual`` / ``fx_hybrid_gemv_segments_rmsnormed``
    with the SwiGLU formed in the down launch's prologue, when every layer's four
    are hybrid Linears without bias (q|k|v and gate|up fused).  ``None`` from
    :meth:`build` otherwise.

    Column-permuted W3 payloads (the reference's desc_act artifacts,
    ``perm = argsort(g_idx)``, ``gptq_deployment.py:199-227``): every producer
    writes its output in the next GEMV's sorted column order -- the step's first
    launch and the o / down residual epilogues a sorted copy of the residual
    (``sorted_residual``), the attention its output in o's order, the SwiGLU
    epilogue its output in down's order -- so every GEMV reads its activations
    contiguously with no gather; the normalising GEMVs read the RMSNorm weights
    reordered once here.  The results are bit-identical to the GEMVs gathering
    ``x[perm]`` themselves."""

    def __init__(self, lib, hidden, device, payload_format, kind="w3"):
        self.lib = lib
        self.kind = kind
        self.tiles = (hidden + 15) // 16
        self.partials = torch.zeros(self.tiles, dtype=torch.float32, device=device)
        self.format = payload_format
        self.o_out = self.down_out = None  # hybrid: per-layer single-module launches
        # planes data_ptr -> (the planes tensor, its field-layout copy); holding the
        # planes keeps their memory from being reused by another payload, and a
        # lookup must find the same tensor object
        self._fields = {}
        # per layer: where each producer writes (None = row order), and the norm
        # weights in the normalising GEMVs' sorted order
        self.qkv_index = self.o_index = self.gate_up_index = self.down_index = None
        self.in_norm = self.post_norm = None
        self.sorted_residual = None

    def payload(self, layout):
        """The weights the kernels read: the planes, or their field-layout copy."""
        planes = layout["planes"]
        if self.format == _lib.PAYLOAD_PLANAR:
            return planes
        entry = self._fields.get(planes.data_ptr())
        if entry is None or entry[0] is not planes:
            raise RuntimeError("no field-layout copy of this payload (repacked when the session is built)")
        return entry[1]

    def _repack(self, layout):
        planes = layout["planes"]
        if self.format == _lib.PAYLOAD_PLANAR:
            return
        entry = self._fields.get(planes.data_ptr())
        if entry is not None:
            if entry[0] is not planes:
                raise RuntimeError("two payload tensors share one address")
            return
        if not planes.is_contiguous():
            raise ValueError("W3 planes must be contiguous")
        fields = torch.empty_like(planes)
        g, _, o, _ = planes.shape
        name = "fx_w3_planes_to_fp6" if self.format == _lib.PAYLOAD_FP6 else "fx_w3_planes_to_fields"
        _lib.check(getattr(self.lib, name)(planes.data_ptr(), fields.data_ptr(), o, 128 * g,
                                           _lib.stream_handle(planes.device)), name)
        self._fields[planes.data_ptr()] = (planes, fields)

    @staticmethod
    def build(session, payload_format=None):
        if all(isinstance(l.self_attn.o_proj, PackedHybridLinear) for l in session.layers):
            return _ResidualStream._build_hybrid(session)
        return _ResidualStream._build_w3(session, payload_format)

    @staticmethod
    def _embed_ok(session):
        table = session.embed
        # the step's first launch reads the embedding rows as 16-byte vectors
        return (table.is_contiguous() and table.data_ptr() % 16 == 0 and table.dtype == session.dtype
                and session.hidden % 16 == 0)

    @staticmethod
    def _build_hybrid(session):
        def bare(m):
            return isinstance(m, PackedHybridLinear) and m.bias is None

        if session.hidden > 4096 or not _ResidualStream._embed_ok(session):
            return None  # the normalising prologue reads at most 256 tile sums
        for layer, qkv, gate_up in zip(session.layers, session.qkv, session.gate_up):
            if not (bare(layer.self_attn.o_proj) and bare(layer.mlp.down_proj)):
                return None
            if not all(f is not None and isinstance(f.call, HybridSegmentsGemv) for f in (qkv, gate_up)):
                return None
        stream = _ResidualStream(_lib.library(), session.hidden, session.device, None, kind="hybrid")
        stream.o_out = [HybridSegmentsGemv([l.self_attn.o_proj]) for l in session.layers]
        stream.down_out = [HybridSegmentsGemv([l.mlp.down_proj]) for l in session.layers]
        # the residual epilogue needs one K split: try each shape once on scratch
        for gemv, swiglu in ((stream.o_out[0], False), (stream.down_out[0], True)):
            x = torch.zeros(1, (2 if swiglu else 1) * gemv.in_features, dtype=session.dtype, device=session.device)
            res = torch.zeros(1, gemv.out_features, dtype=session.dtype, device=session.device)
            sums = torch.empty((gemv.out_features + 15) // 16, dtype=torch.float32, device=session.device)
            try:
                gemv.residual(x, res, sums, swiglu=swiglu)
            except RuntimeError:
                return None
        torch.cuda.synchronize(session.device)
        return stream

    @staticmethod
    def _build_w3(session, payload_format=None):
        for layer, qkv, swiglu in zip(session.layers, session.qkv, session.swiglu):
            o, down = layer.self_attn.o_proj, layer.mlp.down_proj
            if not (_structural_w3(o) and _structural_w3(down)) or qkv is None or swiglu is None:
                return None
            gemv = qkv.call
            if not (isinstance(gemv, W3Gemv) and gemv.arith == _lib.ARITH_STRUCTURAL):
                return None
        if not _ResidualStream._embed_ok(session):
            return None
        fmt = _lib.PAYLOAD_FIELDS if payload_format is None else payload_format
        stream = _ResidualStream(_lib.library(), session.hidden, session.device, fmt)
        for lin, qkv, swiglu in zip(session.lin, session.qkv, session.swiglu):
            for layout in (qkv.call.layout, swiglu.layout, lin["self_attn.o_proj"].gemv.layout,
                           lin["mlp.down_proj"].gemv.layout):
                stream._repack(layout)
        stream._orders(session)
        torch.cuda.synchronize(session.device)
        return stream

    def _orders(self, session):
        """Each producer's output order and the sorted norm weights (W3 chain)."""
        self.qkv_index = [inverse_index(q.call.layout["perm"]) for q in session.qkv]
        self.o_index = [inverse_index(lin["self_attn.o_proj"].gemv.layout["perm"]) for lin in session.lin]
        self.gate_up_index = [inverse_index(sw.layout["perm"]) for sw in session.swiglu]
        self.down_index = [inverse_index(lin["mlp.down_proj"].gemv.layout["perm"]) for lin in session.lin]

        def sort(weight, qkv_or_gu):
            return weight if qkv_or_gu is None else weight[qkv_or_gu.layout["perm"].long()].contiguous()

        self.in_norm = [w if i is None else sort(w, q.call)
                        for w, i, q in zip(session.in_norm, self.qkv_index, session.qkv)]
        self.post_norm = [w if i is None else sort(w, sw)
                          for w, i, sw in zip(session.post_norm, self.gate_up_index, session.swiglu)]
        if any(i is not None for i in self.qkv_index + self.gate_up_index):
            self.sorted_residual = torch.zeros_like(session.residual)

    def _residual_input(self, session, index):
        """What a normalising GEMV reads: the residual, or its sorted copy."""
        return session.residual if index is None else self.sorted_residual

    def residual(self, gemv: W3Gemv, x, residual, next_index=None, x_sorted=False):
        """residual <- round(residual + round(x @ W.T)); tile sums of its squares;
        with ``next_index`` also the residual in the next GEMV's sorted order.
        ``x_sorted``: x already comes in the payload's sorted column order."""
        lay = gemv.layout
        _lib.check(self.lib.fx_w3_gemv_residual(
            x.data_ptr(), _lib.dtype_code(x.dtype), self.payload(lay).data_ptr(), lay["scales"].data_ptr(),
            gemv.scale_code, gemv.zeros_ptr, None if x_sorted else gemv.perm_ptr, residual.data_ptr(),
            residual.data_ptr(), self.partials.data_ptr(), _lib.ptr(next_index),
            None if next_index is None else self.sorted_residual.data_ptr(), gemv.out_features, gemv.in_features,
            self.format, _lib.stream_handle(x.device)), "fx_w3_gemv_residual")

    def embed(self, token, table, out, lm_ws=None, lm_vocab=0, prediction=None):
        """out = table[*token], and the tile sums of its squares (the first layer's
        normalising GEMV reads them) and, for a permuted first q|k|v, the row in its
        sorted order; with ``prediction``, also the merge of the previous step's
        LM-head maxima in ``lm_ws`` into it (one launch)."""
        index = self.qkv_index[0] if self.qkv_index else None
        _lib.check(self.lib.fx_decode_embed(
            token.data_ptr(), table.data_ptr(), table.shape[0], table.shape[1], out.data_ptr(),
            self.partials.data_ptr(), _lib.ptr(index), None if index is None else self.sorted_residual.data_ptr(),
            _lib.ptr(lm_ws), 0 if lm_ws is None else lm_ws.numel(), lm_vocab,
            _lib.ptr(prediction), _lib.dtype_code(table.dtype), _lib.stream_handle(out.device)), "fx_decode_embed")

    def normed(self, layout, scale_code, zeros_ptr, rows, h, weight, eps, out, swiglu, out_index=None):
        """out = GEMV (or SwiGLU, written in ``out_index`` order) of RMSNorm(h) with
        the tile sums of h."""
        _lib.check(self.lib.fx_w3_gemv_rmsnormed(
            h.data_ptr(), _lib.dtype_code(h.dtype), self.payload(layout).data_ptr(), layout["scales"].data_ptr(),
            scale_code, zeros_ptr, self.partials.data_ptr(), self.tiles, weight.data_ptr(), eps, _lib.ptr(out_index),
            out.data_ptr(), rows, h.shape[-1], int(swiglu), self.format, _lib.stream_handle(h.device)),
            "fx_w3_gemv_rmsnormed")

    def attention_index(self, l):
        """Where the attention of layer l writes its output (o's sorted order)."""
        return self.o_index[l] if self.o_index else None

    # -- one decoder layer's four launches around the attention and the SwiGLU ------
    def qkv_in(self, session, l):
        """q|k|v of RMSNorm(residual) into session.qkv_out."""
        if self.kind == "hybrid":
            session.qkv[l].call.rmsnormed(session.residual, self.partials, session.in_norm[l], session.eps,
                                          session.qkv_out)
            return
        gemv = session.qkv[l].call
        self.normed(gemv.layout, gemv.scale_code, gemv.zeros_ptr, gemv.out_features,
                    self._residual_input(session, self.qkv_index[l]), self.in_norm[l], session.eps,
                    session.qkv_out, False)

    def attn_out(self, session, l):
        """residual += o_proj(attn), with its tile sums (and the sorted copy for a
        permuted gate|up)."""
        if self.kind == "hybrid":
            self.o_out[l].residual(session.attn, session.residual, self.partials)
            return
        self.residual(session.lin[l]["self_attn.o_proj"].gemv, session.attn, session.residual,
                      next_index=self.gate_up_index[l], x_sorted=True)

    def mlp_in(self, session, l):
        """SiLU(gate) * up of RMSNorm(residual) into session.act, in down's sorted
        order (hybrid: gate | up into session.gate_up_out; the down launch forms the
        SwiGLU)."""
        if self.kind == "hybrid":
            session.gate_up[l].call.rmsnormed(session.residual, self.partials, session.post_norm[l], session.eps,
                                              session.gate_up_out)
            return
        sw = session.swiglu[l]
        self.normed(sw.layout, sw.scale_code, sw.zeros_ptr, 2 * sw.width,
                    self._residual_input(session, self.gate_up_index[l]), self.post_norm[l], session.eps,
                    session.act, True, out_index=self.down_index[l])

    def mlp_out(self, session, l):
        """residual += down_proj(act), with its tile sums (and the sorted copy for
        the next layer's permuted q|k|v)."""
        if self.kind == "hybrid":
            self.down_out[l].residual(session.gate_up_out, session.residual, self.partials, swiglu=True)
            return
        nxt = self.qkv_index[l + 1] if l + 1 < len(self.qkv_index) else None
        self.residual(session.lin[l]["mlp.down_proj"].gemv, session.act, session.residual, next_index=nxt,
                      x_sorted=True)


class NativeDecodeSession:
    def __init__(self, model, input_ids: torch.Tensor, forced_tokens: torch.Tensor, w3_payload: str = "fields"):
        from transformers import StaticCache

        if input_ids.ndim != 2 or input_ids.shape[0] != 1 or input_ids.shape[1] < 2:
            raise ValueError("batch1 nonempty real prefix required")
        if forced_tokens.ndim != 2 or forced_tokens.shape[0] != 1 or forced_tokens.shape[1] < 1:
            raise ValueError("batch1 continuation required")
        if model.training:
            raise ValueError("eval model required")
        if not input_ids.is_cuda:
            raise ValueError("native decode runs on a GPU")
        cfg = model.config
        if set(cfg.layer_types) != {"full_attention"}:
            raise ValueError("this protocol supports full-attention Qwen3 only")
        dtype = model.model.embed_tokens.weight.dtype
        if dtype not in (torch.bfloat16, torch.float16):
            raise ValueError("native decode needs a bf16 or fp16 model")
        self.model, self.dtype, self.device = model, dtype, input_ids.device
        self.ids = input_ids
        self.tokens = forced_tokens.to(self.device).contiguous()
        self.steps = self.tokens.shape[1]
        self.prefix_length = input_ids.shape[1]
        self.maximum_length = self.prefix_length + self.steps
        self.hidden = cfg.hidden_size
        self.heads, self.kv_heads, self.head_dim = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        self.eps = cfg.rms_norm_eps
        self.scale = 1.0 / math.sqrt(self.head_dim)
        self.layers = model.model.layers
        n = len(self.layers)

        # prefill through the HF model (dense fallback for packed Linears)
        cache = StaticCache(config=cfg, max_cache_len=self.maximum_length)
        with torch.inference_mode():
            out = model(input_ids=input_ids, past_key_values=cache, use_cache=True, logits_to_keep=1)
            self.prefill_logits = out.logits[:, -1, :].detach().clone()
            shape = (n, self.kv_heads, self.maximum_length, self.head_dim)
            self.k_cache = torch.zeros(shape, dtype=dtype, device=self.device)
            self.v_cache = torch.zeros(shape, dtype=dtype, device=self.device)
            self.prefix_k = torch.stack([l.keys[0, :, :self.prefix_length] for l in cache.layers]).clone()
            self.prefix_v = torch.stack([l.values[0, :, :self.prefix_length] for l in cache.layers]).clone()
            # cos/sin rows for every position, built by the model's own rotary module
            positions = torch.arange(self.maximum_length, device=self.device)[None]
            cos, sin = model.model.rotary_emb(self.prefill_logits.to(dtype), positions)
            self.cos = cos[0].contiguous()
            self.sin = sin[0].contiguous()
        del cache

        # weights
        self.embed = model.model.embed_tokens.weight
        self.final_norm = model.model.norm.weight
        self.lm_head = model.lm_head.weight
        self.lin = [{name: _Linear(block.get_submodule(name)) for name in _ATTN + _MLP} for block in self.layers]
        # q|k|v and gate|up as one GEMV each where the payloads allow it
        self.qkv = [_FusedLinear.build([b.get_submodule(n) for n in _ATTN[:3]]) for b in self.layers]
        # gate|up + SwiGLU as one launch where both are structural W3; else gate|up
        # (fused where possible) and the SwiGLU kernel
        self.swiglu = [_GateUpSwiGLU.build(*(b.get_submodule(n) for n in _MLP[:2])) for b in self.layers]
        self.gate_up = [None if f is not None else _FusedLinear.build([b.get_submodule(n) for n in _MLP[:2]])
                        for f, b in zip(self.swiglu, self.layers)]
        if w3_payload not in ("fields", "planar", "fp6"):
            raise ValueError(f"w3_payload must be 'fields', 'planar' or 'fp6', got {w3_payload!r}")
        self.in_norm = [b.input_layernorm.weight for b in self.layers]
        self.post_norm = [b.post_attention_layernorm.weight for b in self.layers]
        self.q_norm = [b.self_attn.q_norm.weight for b in self.layers]
        self.k_norm = [b.self_attn.k_norm.weight for b in self.layers]

        # static activations (one token)
        def buf(width):
            return torch.empty((1, width), dtype=dtype, device=self.device)

        qd, kd = self.heads * self.head_dim, self.kv_heads * self.head_dim
        inter = cfg.intermediate_size
        self.residual, self.normed = buf(self.hidden), buf(self.hidden)
        # q|k|v and gate|up are views of one buffer each (what a fused GEMV writes)
        self.qkv_out = buf(qd + 2 * kd)
        self.q, self.k, self.v = self.qkv_out[:, :qd], self.qkv_out[:, qd:qd + kd], self.qkv_out[:, qd + kd:]
        self.gate_up_out = buf(2 * inter)
        self.gate, self.up = self.gate_up_out[:, :inter], self.gate_up_out[:, inter:]
        self.attn = buf(qd)
        self.o, self.act, self.down = buf(self.hidden), buf(inter), buf(self.hidden)
        self.logits = torch.empty((self.steps, cfg.vocab_size), dtype=dtype, device=self.device)
        self.predictions = torch.empty((self.steps, 1), dtype=torch.int64, device=self.device)
        self.stream = _ResidualStream.build(
            self, {"fields": _lib.PAYLOAD_FIELDS, "planar": _lib.PAYLOAD_PLANAR, "fp6": _lib.PAYLOAD_FP6}[w3_payload])
        lib = _lib.library()
        self.lib = lib
        # the final RMSNorm, LM head and argmax as one launch where the head allows it
        head = self.lm_head
        self.lm_ws = None
        if (head.dtype == dtype and head.is_contiguous() and head.data_ptr() % 16 == 0
                and self.hidden % 512 == 0 and self.hidden <= 8192):
            self.lm_ws = torch.empty(lib.fx_lm_head_argmax_workspace_bytes(), dtype=torch.uint8,
                                     device=self.device)  # per-workgroup argmax partials
        nbytes = lib.fx_decode_attention_workspace_bytes(self.heads, self.maximum_length, self.head_dim)
        self.attn_ws = torch.empty(nbytes // 4 + 64, dtype=torch.float32, device=self.device)  # split partials
        self.graph = None
        self.kernel_nodes = None
        self.launches_per_step = None
        # eager-only inspection: called as observer(step, layer, residual) after each
        # decoder layer of the residual-stream chain (a graph capture must leave it None)
        self.layer_observer = None

    # -- one token -------------------------------------------------------------------
    def _attention(self, layer, pos, out_index=None):
        """q/k RMSNorm + RoPE, the KV-cache write of position ``pos`` and the
        attention, from the raw q|k|v projections (one launch at decode lengths);
        ``out_index``: the output in the o projection's sorted column order."""
        lib = self.lib
        _lib.check(lib.fx_decode_attention_rope(
            self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(), self.q_norm[layer].data_ptr(),
            self.k_norm[layer].data_ptr(), self.cos[pos].data_ptr(), self.sin[pos].data_ptr(), self.eps,
            _lib.ROPE_STOCK, self.k_cache[layer].data_ptr(), self.v_cache[layer].data_ptr(),
            self.attn_ws.data_ptr(), self.attn_ws.numel() * 4, _lib.ptr(out_index), self.attn.data_ptr(),
            self.heads, self.kv_heads, self.maximum_length, self.head_dim, pos, self.scale,
            _lib.dtype_code(self.dtype), _lib.stream_handle(self.device)), "fx_decode_attention_rope")

    def _lm_head(self, i, hidden, norm_weight, merge=True):
        """Logits row ``i`` and its greedy token from the last hidden state
        (``norm_weight`` set: RMS-normalised first).  ``fx_lm_head_argmax`` where
        the head allows it (``merge`` False: ``fx_lm_head_logits`` only, the
        maxima merged by the next step's first launch or by :meth:`_merge_last`);
        else RMSNorm, the hipBLASLt matmul and torch.argmax."""
        if self.lm_ws is not None:
            if not merge:
                _lib.check(self.lib.fx_lm_head_logits(
                    hidden.data_ptr(), None if norm_weight is None else norm_weight.data_ptr(), self.eps,
                    self.lm_head.data_ptr(), self.logits[i].data_ptr(), self.lm_ws.data_ptr(), self.lm_ws.numel(),
                    self.logits.shape[1], self.hidden, _lib.dtype_code(self.dtype),
                    _lib.stream_handle(self.device)), "fx_lm_head_logits")
                return
            _lib.check(self.lib.fx_lm_head_argmax(
                hidden.data_ptr(), None if norm_weight is None else norm_weight.data_ptr(), self.eps,
                self.lm_head.data_ptr(), self.logits[i].data_ptr(), self.predictions[i].data_ptr(),
                self.lm_ws.data_ptr(), self.lm_ws.numel(), self.logits.shape[1], self.hidden,
                _lib.dtype_code(self.dtype), _lib.stream_handle(self.device)), "fx_lm_head_argmax")
            return
        from .fused_modules import rms_norm

        if norm_weight is not None:
            rms_norm(hidden, norm_weight, self.eps, out=self.normed)
            hidden = self.normed
        torch.matmul(hidden, self.lm_head.t(), out=self.logits[i:i + 1])
        torch.argmax(self.logits[i:i + 1], dim=-1, keepdim=True, out=self.predictions[i:i + 1])

    def _silu_mul(self):
        _lib.check(self.lib.fx_silu_mul(self.gate.data_ptr(), self.up.data_ptr(), self.act.data_ptr(),
                                        self.act.shape[1], _lib.dtype_code(self.dtype),
                                        _lib.stream_handle(self.device)), "fx_silu_mul")

    def _step_residual_stream(self, i):
        rs = self.stream
        # the step's first launch: embedding row, its tile sums, and the merge of
        # the previous step's LM-head maxima into that step's prediction
        split_head = self.lm_ws is not None
        merge_prev = split_head and i > 0
        rs.embed(self.tokens[0, i:i + 1], self.embed, self.residual,
                 self.lm_ws if merge_prev else None, self.logits.shape[1] if merge_prev else 0,
                 self.predictions[i - 1] if merge_prev else None)
        pos = self.prefix_length + i
        for l in range(len(self.lin)):
            rs.qkv_in(self, l)
            self._attention(l, pos, rs.attention_index(l))
            rs.attn_out(self, l)
            rs.mlp_in(self, l)
            rs.mlp_out(self, l)
            if self.layer_observer is not None:
                self.layer_observer(i, l, self.residual)
        self._lm_head(i, self.residual, self.final_norm, merge=not split_head)

    def _merge_last(self):
        """The last step's LM-head maxima into its prediction (the residual-stream
        chain merges every other step's in the next step's first launch)."""
        if self.stream is not None and self.lm_ws is not None:
            _lib.check(self.lib.fx_lm_head_merge(
                self.lm_ws.data_ptr(), self.lm_ws.numel(), self.logits.shape[1],
                self.predictions[self.steps - 1].data_ptr(), _lib.stream_handle(self.device)), "fx_lm_head_merge")

    def _step(self, i):
        if self.stream is not None:
            return self._step_residual_stream(i)
        pos = self.prefix_length + i
        torch.index_select(self.embed, 0, self.tokens[0, i:i + 1], out=self.residual)
        from .fused_modules import rms_norm

        rms_norm(self.residual, self.in_norm[0], self.eps, out=self.normed)
        for l, lin in enumerate(self.lin):
            if l > 0:
                add_rms_norm(self.down, self.residual, self.in_norm[l], self.eps, out=self.normed,
                             residual_out=self.residual)
            if self.qkv[l] is not None:
                self.qkv[l](self.normed, self.qkv_out)
            else:
                lin["self_attn.q_proj"](self.normed, self.q)
                lin["self_attn.k_proj"](self.normed, self.k)
                lin["self_attn.v_proj"](self.normed, self.v)
            self._attention(l, pos)
            lin["self_attn.o_proj"](self.attn, self.o)
            add_rms_norm(self.o, self.residual, self.post_norm[l], self.eps, out=self.normed,
                         residual_out=self.residual)
            if self.swiglu[l] is not None:
                self.swiglu[l](self.normed, self.act)
            else:
                if self.gate_up[l] is not None:
                    self.gate_up[l](self.normed, self.gate_up_out)
                else:
                    lin["mlp.gate_proj"](self.normed, self.gate)
                    lin["mlp.up_proj"](self.normed, self.up)
                self._silu_mul()
            lin["mlp.down_proj"](self.act, self.down)
        add_rms_norm(self.down, self.residual, self.final_norm, self.eps, out=self.normed,
                     residual_out=self.residual)
        self._lm_head(i, self.normed, None)

    # -- session protocol --------------------------------------------------------------
    @torch.inference_mode()
    def reset(self):
        self.k_cache.zero_()
        self.v_cache.zero_()
        self.k_cache[:, :, :self.prefix_length].copy_(self.prefix_k)
        self.v_cache[:, :, :self.prefix_length].copy_(self.prefix_v)

    @torch.inference_mode()
    def run(self):
        for i in range(self.steps):
            self._step(i)
        self._merge_last()
        return self.logits, self.predictions

    def trace(self, outputs=None) -> dict:
        logits = torch.cat([self.prefill_logits, self.logits], 0)[None].detach().cpu()
        predictions = torch.cat([self.prefill_logits.argmax(-1, keepdim=True), self.predictions], 0).t().cpu()
        if not bool(torch.isfinite(logits).all()):
            raise RuntimeError("nonfinite native decode logits")
        return {"logits": logits, "predictions": predictions, "fed_tokens": self.tokens.cpu(),
                "cache_length": self.maximum_length, "routes": {}}

    @torch.inference_mode()
    def audit(self) -> dict:
        self.reset()
        return self.trace(self.run())

    @torch.inference_mode()
    def capture(self) -> dict:
        if self.layer_observer is not None:
            raise RuntimeError("clear layer_observer before graph capture")
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            for _ in range(2):
                self.reset()
                self.run()
        torch.cuda.current_stream().wait_stream(stream)
        self.reset()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph(keep_graph=True)
        with torch.cuda.graph(graph, stream=stream):
            self.run()
        self.kernel_nodes = graph_kernel_count(graph)
        graph.instantiate()
        self.graph = graph
        self.reset()
        graph.replay()
        torch.cuda.synchronize()
        return self.trace()

    @torch.inference_mode()
    def measure(self, mode: str):
        if mode not in ("prepared_eager", "sequence_graph"):
            raise ValueError("unknown mode")
        if mode == "sequence_graph" and self.graph is None:
            raise ValueError("capture first")
        self.reset()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        wall = time.perf_counter()
        start.record()
        if mode == "sequence_graph":
            self.graph.replay()
        else:
            self.run()
        end.record()
        end.synchronize()
        wall_ms = (time.perf_counter() - wall) * 1000
        return {"wall_ms": wall_ms, "device_ms": start.elapsed_time(end)}, self.trace()
