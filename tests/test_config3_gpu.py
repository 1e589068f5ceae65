"""Config 3 at its real shapes: the Qwen3-8B architecture (hidden 4096, 32 / 8 heads of
128, SwiGLU 12288, vocab 151936), random init, W3 g128 Linears (RTN, fp16 scales,
zero-points), a 512-token prefill and greedy decode captured as one hipGraph.

* First decode step, layer by layer (4 layers, where bf16 depth chaos has not yet
  grown): the native kernel chain's residual stream after every decoder layer
  against the HF module tree run with the same arithmetic (stock modules, SDPA
  math backend, our W3 Linears through ``prepared_linears``), captured with
  forward hooks, for both weight formats of the native chain, and the first
  layer of both against the float64 oracle layer (``oracle.decode.qwen3_layer_step``,
  pinned to transformers in float64).  Bar: the NRMSE
  after layer l at most 6e-3 (l + 1) -- a few bf16 rounding flips per layer, where
  a layer bug moves the hidden state by O(1) -- and the first step's logits NRMSE
  <= 2e-2 with the same greedy token.
* The final RMSNorm + LM head + argmax launch at vocab 151936 against the oracle:
  float64 product of the weight with ``oracle.norms.rms_norm``'s activation;
  logits within two bf16 ulps plus 1e-3 of max|logit|, the prediction the first
  index of the kernel's own maximum and an index of the oracle's maximum within
  that slack.
* All 36 layers, prefill 512, 32 steps: the captured graph's replay is bit-equal
  to the eager run, on every replay, and each token is the argmax of its logits.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from marlin_style_fluxbin_amd import _lib
from marlin_style_fluxbin_amd.full_model_trial import compare_trace
from marlin_style_fluxbin_amd.native_decode import NativeDecodeSession
from marlin_style_fluxbin_amd.qwen3 import qwen3_config, random_qwen3_model, w3_quantize_qwen3_model
from marlin_style_fluxbin_amd.static_decode import StaticDecodeSession, prepared_linears

pytestmark = pytest.mark.gpu

PREFIX = 512


def _nrmse(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.double().flatten(), b.double().flatten()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def _model(gpu, layers, steps, seed=0):
    config = qwen3_config(num_hidden_layers=layers)
    model = random_qwen3_model(config, device=gpu, dtype=torch.bfloat16, seed=seed)
    assert w3_quantize_qwen3_model(model) == 7 * layers
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, config.vocab_size, (1, PREFIX), generator=g).to(gpu)
    tokens = torch.randint(0, config.vocab_size, (1, steps), generator=g).to(gpu)
    return model, ids, tokens


def _layer0_float64(model, native, tokens):
    """The first decoder layer for the first decode token in float64 (oracle
    ``decode.qwen3_layer_step``): exact W3 weights ``s (q - z)`` (oracle
    ``w3.dequant_exact``), the model's norm weights, the prefix keys / values the
    native session holds (the HF prefill's) and the bf16 rotary rows of the position."""
    from oracle import decode, w3
    from tests.payloads import oracle_layout

    layer = model.model.layers[0]
    names = {"q": "self_attn.q_proj", "k": "self_attn.k_proj", "v": "self_attn.v_proj", "o": "self_attn.o_proj",
             "gate": "mlp.gate_proj", "up": "mlp.up_proj", "down": "mlp.down_proj"}
    w = {key: w3.dequant_exact(oracle_layout({n: t.cpu() for n, t in layer.get_submodule(name).layout().items()}))
         for key, name in names.items()}
    f64 = lambda t: t.detach().double().cpu().numpy()  # noqa: E731
    w.update(in_norm=f64(layer.input_layernorm.weight), post_norm=f64(layer.post_attention_layernorm.weight),
             q_norm=f64(layer.self_attn.q_norm.weight), k_norm=f64(layer.self_attn.k_norm.weight))
    hidden = f64(model.model.embed_tokens.weight[int(tokens[0, 0])])
    pos = native.prefix_length
    out, _, _ = decode.qwen3_layer_step(hidden, w, f64(native.prefix_k[0]), f64(native.prefix_v[0]),
                                        f64(native.cos[pos]), f64(native.sin[pos]), eps=native.eps,
                                        heads=native.heads, kv_heads=native.kv_heads, head_dim=native.head_dim)
    return out


def test_config3_first_step_layer_by_layer(gpu):
    from torch.nn.attention import SDPBackend, sdpa_kernel

    print("config 3: 4 layers, first decode step layer by layer", flush=True)
    model, ids, tokens = _model(gpu, layers=4, steps=2)
    hf_layers = {}

    def hook(index):
        def record(module, args, output):
            hidden = output[0] if isinstance(output, tuple) else output
            hf_layers.setdefault(index, hidden.detach().reshape(-1).clone())
        return record

    with sdpa_kernel([SDPBackend.MATH]):
        hf = StaticDecodeSession(model, ids, tokens)
        handles = [layer.register_forward_hook(hook(i)) for i, layer in enumerate(model.model.layers)]
        try:
            with prepared_linears(model, torch.bfloat16):
                want = hf.audit()
        finally:
            for h in handles:
                h.remove()
        natives = {fmt: NativeDecodeSession(model, ids, tokens, w3_payload=fmt) for fmt in ("fields", "planar")}
    exact0 = _layer0_float64(model, natives["fields"], tokens)
    hf_err0 = _nrmse(hf_layers[0].cpu(), torch.from_numpy(exact0))
    print(f"layer 0 vs the float64 oracle: HF modules {hf_err0:.3g}", flush=True)
    assert hf_err0 <= 2e-2
    for fmt, native in natives.items():
        native_layers = {}

        def observe(step, layer, residual):
            if step == 0:
                native_layers[layer] = residual.detach().reshape(-1).clone()

        native.layer_observer = observe
        got = native.audit()
        native.layer_observer = None
        assert sorted(native_layers) == sorted(hf_layers) == [0, 1, 2, 3]
        errors = [_nrmse(native_layers[i], hf_layers[i]) for i in range(4)]
        native_err0 = _nrmse(native_layers[0].cpu(), torch.from_numpy(exact0))
        print(f"{fmt}: per-layer NRMSE of the first decode step: {errors}; layer 0 vs the float64 "
              f"oracle {native_err0:.3g}", flush=True)
        # both implementations sit within bf16 rounding of the exact layer (about
        # ten rounding points, each ~1e-3 RMS relative), where a dropped term or a
        # wrong index moves it by O(1)
        assert native_err0 <= 2e-2, (fmt, native_err0)
        # each layer adds at most a few bf16 rounding flips (fp32 sums in another
        # order before each of the layer's roundings): <= 6e-3 per layer; a wrong
        # index or a dropped term moves the hidden state by O(1)
        bound = 0.0
        for err in errors:
            bound += 6e-3
            assert err <= bound, (fmt, errors)
        report = compare_trace(got, want, logprob_tolerance=0.1)
        assert report["stepwise_normalized_rmse"][1] <= 2e-2, (fmt, report["stepwise_normalized_rmse"])
        assert torch.equal(got["predictions"][:, :2], want["predictions"][:, :2]), fmt


def test_lm_head_argmax_at_vocab_151936(gpu):
    from oracle import norms

    print("config 3: LM head + argmax, vocab 151936 x 4096", flush=True)
    vocab, k = 151936, 4096
    g = torch.Generator().manual_seed(11)
    weight = (torch.randn(vocab, k, generator=g) * 0.02).to(torch.bfloat16)
    hidden = (torch.randn(1, k, generator=g) * 3).to(torch.bfloat16)
    norm_w = (1 + 0.02 * torch.randn(k, generator=g)).to(torch.bfloat16)
    lib = _lib.library()
    ws = torch.zeros(lib.fx_lm_head_argmax_workspace_bytes(), dtype=torch.uint8, device=gpu)
    logits = torch.empty(vocab, dtype=torch.bfloat16, device=gpu)
    pred = torch.full((1,), -1, dtype=torch.int64, device=gpu)
    wg, hg, ng = weight.to(gpu), hidden.to(gpu), norm_w.to(gpu)
    for _ in range(2):  # a second call on the same workspace
        _lib.check(lib.fx_lm_head_argmax(hg.data_ptr(), ng.data_ptr(), 1e-6, wg.data_ptr(),
                                         logits.data_ptr(), pred.data_ptr(), ws.data_ptr(), ws.numel(), vocab, k,
                                         _lib.FX_BF16, _lib.stream_handle(gpu)), "fx_lm_head_argmax")
    torch.cuda.synchronize()
    x = norms.rms_norm(hidden.float().numpy(), norm_w.float().numpy(), 1e-6, "bf16").astype(np.float64)
    exact = np.empty(vocab, np.float64)
    w32 = weight.float().numpy()
    for start in range(0, vocab, 16384):  # float64 dot in row chunks (bounded host memory)
        exact[start:start + 16384] = w32[start:start + 16384].astype(np.float64) @ x[0]
    got = logits.float().cpu().numpy().astype(np.float64)
    scale = np.abs(exact).max()
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(exact), 2.0 ** -126))) - 7)
    assert np.all(np.abs(got - exact) <= 2 * ulp + 1e-3 * scale)
    p = int(pred.item())
    assert p == int(np.argmax(got)), "prediction is not the first maximum of the kernel's logits"
    assert exact[p] >= exact.max() - (2 * ulp.max() + 1e-3 * scale)


def test_config3_36_layers_graph_replay_equals_eager(gpu):
    print("config 3: 36 layers, prefill 512, 32 steps, eager vs graph", flush=True)
    model, ids, tokens = _model(gpu, layers=36, steps=32)
    with torch.inference_mode():
        native = NativeDecodeSession(model, ids, tokens)
        eager = native.audit()
        graph = native.capture()
    assert torch.equal(graph["logits"], eager["logits"])
    assert torch.equal(graph["predictions"], eager["predictions"])
    for _ in range(2):
        _, replay = native.measure("sequence_graph")
        assert torch.equal(replay["logits"], eager["logits"])
    logits = eager["logits"][0, 1:].float()
    assert torch.equal(eager["predictions"][0, 1:], torch.argmax(logits, dim=-1))
    per_token = native.kernel_nodes / 32
    print(f"kernels per token: {per_token}", flush=True)
    # 6 launches per layer (q|k|v normalising, attention splits + combine at 513-544
    # keys, o, gate|up + SwiGLU, down) and 2 per token (the embedding row with its
    # norm statistics and the previous argmax merge; the LM head), plus the last
    # token's argmax merge
    assert native.kernel_nodes == 32 * (6 * 36 + 2) + 1, native.kernel_nodes
