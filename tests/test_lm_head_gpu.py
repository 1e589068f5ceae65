"""GPU parity of the decode step's last launch: final RMSNorm + LM head + greedy
argmax (``fx_lm_head_argmax``).

Bars: logits within two output ulps plus 1e-3 of the largest |logit| of the
float64 product of the weight with the oracle's normalised activation
(``oracle.norms.rms_norm``, pinned to transformers); the normalising prologue
bit-identical to ``fx_rmsnorm`` (the logits from the raw hidden state equal the
logits from fx_rmsnorm's output bit for bit); the prediction exactly
``torch.argmax`` (CPU) of the kernel's own logits, including ties (first index)
and NaN (first NaN).
"""
import numpy as np
import pytest
import torch

from marlin_style_fluxbin_amd import _lib

pytestmark = pytest.mark.gpu

DT = {"bf16": torch.bfloat16, "f16": torch.float16}


def _ulp(v, dtype):
    a = np.abs(np.asarray(v, np.float32))
    bits, lo = (7, -126) if dtype == "bf16" else (10, -14)
    e = np.floor(np.log2(np.maximum(a, np.float32(2.0 ** lo))))
    return np.float32(2.0) ** (e - bits)


class _Head:
    def __init__(self, gpu):
        self.lib = _lib.library()
        self.gpu = gpu
        self.ws = torch.zeros(self.lib.fx_lm_head_argmax_workspace_bytes(), dtype=torch.uint8, device=gpu)

    def __call__(self, hidden, norm_weight, weight, eps=1e-6):
        vocab, k = weight.shape
        logits = torch.empty(vocab, dtype=weight.dtype, device=self.gpu)
        pred = torch.full((1,), -1, dtype=torch.int64, device=self.gpu)
        _lib.check(self.lib.fx_lm_head_argmax(
            hidden.data_ptr(), None if norm_weight is None else norm_weight.data_ptr(), eps, weight.data_ptr(),
            logits.data_ptr(), pred.data_ptr(), self.ws.data_ptr(), self.ws.numel(), vocab, k,
            _lib.dtype_code(weight.dtype), _lib.stream_handle(self.gpu)), "lm_head_argmax")
        return logits, pred


def _rmsnorm(lib, h, w, eps, gpu):
    out = torch.empty_like(h)
    _lib.check(lib.fx_rmsnorm(h.data_ptr(), None, w.data_ptr(), out.data_ptr(), None, 1, h.shape[-1], eps,
                              _lib.dtype_code(h.dtype), _lib.stream_handle(gpu)), "rmsnorm")
    return out


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("vocab,k", [(12289, 4096), (7, 512), (1, 1024), (3001, 8192), (4096, 2560)])
def test_lm_head_argmax_matches_oracle(gpu, dtype, vocab, k):
    from oracle import norms

    g = torch.Generator().manual_seed(vocab + k)
    h = (torch.randn(1, k, generator=g) * 3).to(DT[dtype])
    nw = (1 + 0.1 * torch.randn(k, generator=g)).to(DT[dtype])
    w = (torch.randn(vocab, k, generator=g) * 0.02).to(DT[dtype])
    hd, nwd, wd = h.to(gpu), nw.to(gpu), w.to(gpu)
    head = _Head(gpu)
    logits, pred = head(hd, nwd, wd)
    x = norms.rms_norm(h.float().numpy(), nw.float().numpy(), 1e-6, dtype)
    exact = w.double().numpy() @ x.astype(np.float64).reshape(-1)
    got = logits.float().cpu().numpy()
    assert np.all(np.isfinite(got))
    assert np.all(np.abs(got - exact) <= 2 * _ulp(exact, dtype) + 1e-3 * np.abs(exact).max())
    assert pred.item() == torch.argmax(logits.cpu()).item()
    # the normalising prologue is fx_rmsnorm bit for bit: the same logits from its output
    normed = _rmsnorm(head.lib, hd, nwd, 1e-6, gpu)
    logits2, pred2 = head(normed, None, wd)
    assert torch.equal(logits2.view(torch.int16), logits.view(torch.int16))
    assert pred2.item() == pred.item()


def test_lm_head_argmax_ties_and_nan(gpu):
    """Equal maxima resolve to the first index and a NaN logit wins, the first
    NaN over later ones, as torch.argmax on the same logits."""
    vocab, k = 9001, 4096
    g = torch.Generator().manual_seed(3)
    x = torch.randn(1, k, generator=g).to(torch.bfloat16)
    w = (torch.randn(vocab, k, generator=g) * 0.01).to(torch.bfloat16)
    top = (x.float() / x.float().norm()).to(torch.bfloat16)[0]
    w[4321] = top
    w[77] = top  # the same row: the same logit, the lower index wins
    w[8999] = top
    head = _Head(gpu)
    xd = x.to(gpu)
    logits, pred = head(xd, None, w.to(gpu))
    assert logits[77].item() == logits[4321].item() == logits[8999].item()
    assert pred.item() == 77 == torch.argmax(logits.cpu()).item()
    w[6000, 5] = float("nan")
    w[2500, 9] = float("nan")
    logits, pred = head(xd, None, w.to(gpu))
    assert torch.isnan(logits[2500]) and torch.isnan(logits[6000])
    assert pred.item() == 2500 == torch.argmax(logits.cpu()).item()


def test_lm_head_argmax_workspace_reuse(gpu):
    """One workspace, filled with junk first, across calls with different grids (1
    to 512 workgroups): every prediction is right (the merge reads only the
    partials the same call wrote; nothing needs clearing between calls)."""
    head = _Head(gpu)
    head.ws.fill_(0xA5)
    g = torch.Generator().manual_seed(5)
    for vocab in [151936, 3, 20000, 1, 4097]:
        x = torch.randn(1, 1024, generator=g).to(torch.bfloat16).to(gpu)
        w = torch.randn(vocab, 1024, generator=g).to(torch.bfloat16).to(gpu)
        logits, pred = head(x, None, w)
        assert pred.item() == torch.argmax(logits.cpu()).item(), vocab


def test_lm_head_argmax_rejects_bad_shapes(gpu):
    head = _Head(gpu)
    t = torch.zeros(4096, dtype=torch.bfloat16, device=gpu)
    p = torch.zeros(1, dtype=torch.int64, device=gpu)
    lib = head.lib
    for k, vocab in [(1000, 2), (16384 + 512, 1), (512, 0)]:
        rc = lib.fx_lm_head_argmax(t.data_ptr(), None, 1e-6, t.data_ptr(), t.data_ptr(), p.data_ptr(),
                                   head.ws.data_ptr(), head.ws.numel(), vocab, k, 2, None)
        assert rc == 1, (k, vocab)
    rc = lib.fx_lm_head_argmax(t.data_ptr(), None, 1e-6, t.data_ptr(), t.data_ptr(), p.data_ptr(),
                               head.ws.data_ptr(), 16, 2, 512, 2, None)
    assert rc == 1 and "workspace" in lib.fx_last_error().decode()


@pytest.mark.parametrize("vocab,k", [(12289, 4096), (7, 512), (151936, 4096)])
def test_split_launches_equal_the_fused_call(gpu, vocab, k):
    """fx_lm_head_logits then fx_lm_head_merge (or the merge inside fx_decode_embed,
    the decode chain's next-step launch) give fx_lm_head_argmax's logits and prediction."""
    lib = _lib.library()
    g = torch.Generator().manual_seed(vocab)
    h = torch.randn(1, k, generator=g).to(torch.bfloat16).to(gpu)
    w = (1 + 0.02 * torch.randn(k, generator=g)).to(torch.bfloat16).to(gpu)
    weight = (torch.randn(vocab, k, generator=g) * 0.05).to(torch.bfloat16).to(gpu)
    want_logits, want_pred = _Head(gpu)(h, w, weight)
    ws = torch.full((lib.fx_lm_head_argmax_workspace_bytes(),), 0xAB, dtype=torch.uint8, device=gpu)
    logits = torch.empty(vocab, dtype=torch.bfloat16, device=gpu)
    _lib.check(lib.fx_lm_head_logits(h.data_ptr(), w.data_ptr(), 1e-6, weight.data_ptr(), logits.data_ptr(),
                                     ws.data_ptr(), ws.numel(), vocab, k, _lib.FX_BF16, _lib.stream_handle(gpu)),
               "lm_head_logits")
    pred = torch.full((1,), -1, dtype=torch.int64, device=gpu)
    _lib.check(lib.fx_lm_head_merge(ws.data_ptr(), ws.numel(), vocab, pred.data_ptr(), _lib.stream_handle(gpu)),
               "lm_head_merge")
    assert torch.equal(logits, want_logits) and torch.equal(pred, want_pred)
    # the same merge inside the next step's embedding launch
    table = torch.randn(5, 256, generator=g).to(torch.bfloat16).to(gpu)
    token = torch.tensor([3], dtype=torch.int64, device=gpu)
    row = torch.empty(1, 256, dtype=torch.bfloat16, device=gpu)
    sums = torch.empty(16, dtype=torch.float32, device=gpu)
    pred2 = torch.full((1,), -1, dtype=torch.int64, device=gpu)
    _lib.check(lib.fx_decode_embed(token.data_ptr(), table.data_ptr(), 5, 256, row.data_ptr(), sums.data_ptr(),
                                   None, None, ws.data_ptr(), ws.numel(), vocab, pred2.data_ptr(), _lib.FX_BF16,
                                   _lib.stream_handle(gpu)), "decode_embed")
    assert torch.equal(pred2, want_pred)


def test_decode_embed_row_and_tile_sums(gpu):
    """fx_decode_embed: the token's row bit for bit, each 16-element tile's sum of
    squares against float64, NaNs for a token outside the table, no merge when
    prediction is NULL; with an output index, the row also in the first q|k|v's
    sorted column order (sorted[k] = row[P[k]] for out_index = P^-1)."""
    from marlin_style_fluxbin_amd.native_decode import inverse_index

    lib = _lib.library()
    g = torch.Generator().manual_seed(3)
    nxt = torch.randperm(4096, generator=g).to(torch.int16).to(gpu)
    index = inverse_index(nxt)
    for dtype, code in ((torch.bfloat16, _lib.FX_BF16), (torch.float16, _lib.FX_F16)):
        table = (torch.randn(40, 4096, generator=g) * 2).to(dtype).to(gpu)
        out = torch.empty(1, 4096, dtype=dtype, device=gpu)
        sorted_out = torch.empty(1, 4096, dtype=dtype, device=gpu)
        sums = torch.empty(256, dtype=torch.float32, device=gpu)
        for tok in (0, 17, 39):
            token = torch.tensor([tok], dtype=torch.int64, device=gpu)
            for idx, so in ((None, None), (index, sorted_out)):
                sorted_out.fill_(float("nan"))
                _lib.check(lib.fx_decode_embed(token.data_ptr(), table.data_ptr(), 40, 4096, out.data_ptr(),
                                               sums.data_ptr(), _lib.ptr(idx), _lib.ptr(so), None, 0, 0, None, code,
                                               _lib.stream_handle(gpu)), "decode_embed")
                assert torch.equal(out[0], table[tok])
                if idx is not None:
                    assert torch.equal(sorted_out[0], table[tok][nxt.long()])
                want = (table[tok].double().cpu().view(256, 16) ** 2).sum(1)
                np.testing.assert_allclose(sums.double().cpu().numpy(), want.numpy(), rtol=1e-5, atol=0)
        for bad in (-1, 40):
            token = torch.tensor([bad], dtype=torch.int64, device=gpu)
            _lib.check(lib.fx_decode_embed(token.data_ptr(), table.data_ptr(), 40, 4096, out.data_ptr(),
                                           sums.data_ptr(), index.data_ptr(), sorted_out.data_ptr(), None, 0, 0, None,
                                           code, _lib.stream_handle(gpu)), "decode_embed")
            assert torch.isnan(out.float()).all() and torch.isnan(sums).all()
            assert torch.isnan(sorted_out.float()).all()
    rc = lib.fx_decode_embed(token.data_ptr(), table.data_ptr(), 40, 4004, out.data_ptr(), sums.data_ptr(), None,
                             None, None, 0, 0, None, _lib.FX_BF16, _lib.stream_handle(gpu))
    assert rc == 1 and b"multiple of 16" in lib.fx_last_error()
