"""CPU emulation of the fp6 layout's activation digits (``stage_fp6_8`` in
``marlin_style_fluxbin_amd/csrc/w3_mfma.hip``): each 8-element block of bf16
activations gets S = 2^(e - 8) from frexp of its max|x| (e clamped at -118), and
each element two fp8 e4m3 digits hi = fp8(x / S), lo = fp8(x / S - hi), both
rounded to nearest even.

What is pinned: the e4m3 rounding restated here from the format (4 significant
bits, exponent floor -6, subnormal step 2^-9) against torch's float8_e4m3fn cast;
then the two error claims the GPU tolerances rest on: every element with |x| >=
2^(e - 10) is exact in hi + lo, and every element is within 2^(e - 18) (2^-17 of
the block's max, since max|x| >= 2^(e - 1)) of S (hi + lo)."""
import numpy as np
import torch


def _e4m3(v: np.ndarray) -> np.ndarray:
    """Round to the nearest e4m3 value, ties to even (no overflow in this use)."""
    v = np.asarray(v, dtype=np.float64)
    a = np.abs(v)
    exp = np.floor(np.log2(np.where(a > 0, a, 1.0)))
    q = np.exp2(np.maximum(exp, -6.0) - 3.0)
    return np.sign(v) * np.round(a / q) * q


def _digits(x: np.ndarray):
    """hi, lo and S per element for a [..., 8]-block view of x (float64 values of bf16)."""
    blocks = x.reshape(-1, 8)
    mx = np.abs(blocks).max(axis=1)
    _, e = np.frexp(mx)
    e = np.where(mx > 0, e, 0)
    e = np.maximum(e, -118)
    s = np.exp2(e - 8.0)[:, None]
    v = blocks / s
    hi = _e4m3(v)
    lo = _e4m3(v - hi)
    return hi, lo, s, e[:, None]


def _bf16_values(n, scale, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(n, generator=g, dtype=torch.float64) * scale).to(torch.bfloat16).double().numpy()


def test_e4m3_rounding_matches_torch_cast():
    g = torch.Generator().manual_seed(0)
    v = torch.cat([torch.randn(20000, generator=g, dtype=torch.float64) * 40,
                   torch.randn(20000, generator=g, dtype=torch.float64) * 2.0 ** -7,
                   torch.tensor([0.0, 2.0 ** -9, 2.0 ** -10, 3 * 2.0 ** -11, 1.0625, 1.1875, 17.0, 240.0, 448.0],
                                dtype=torch.float64)])
    v = v[v.abs() <= 448]
    # through float32, as the kernel's operands are
    want = v.float().to(torch.float8_e4m3fn).double().numpy()
    np.testing.assert_array_equal(_e4m3(v.float().double().numpy()), want)


def test_digits_are_exact_above_and_bounded_below():
    for scale, seed in ((1.0, 1), (1e-3, 2), (1e4, 3), (1e-30, 4), (1e30, 5)):
        x = _bf16_values(8 * 4096, scale, seed)
        # outlier elements inside some blocks coarsen only those blocks' small values
        x[::64] *= 1000.0
        x = torch.from_numpy(x).to(torch.bfloat16).double().numpy()
        hi, lo, s, e = _digits(x)
        blocks = x.reshape(-1, 8)
        # the digits never overflow e4m3 (|x / S| < 256 <= 448)
        assert np.all(np.abs(hi) <= 256) and np.all(np.abs(lo) <= 16)
        got = s * (hi + lo)
        err = np.abs(got - blocks)
        big = np.abs(blocks) >= np.exp2(e - 10.0)
        assert np.all(err[big] == 0), (scale, float(err[big].max()))
        assert np.all(err <= np.exp2(e - 18.0)), (scale, float((err / np.exp2(e - 18.0)).max()))
        # the bound is reached: some small elements do lose bits (a test of the
        # emulation itself, so that a split that kept everything would be noticed)
        if scale == 1.0:
            assert np.any(err > 0)


def test_digit_split_of_a_hand_case():
    # block max 3.0 -> frexp e = 2, S = 2^-6; x = 1.1171875 (bf16 0x3F8F) -> v = 71.5:
    # hi = 72 (4 significant bits), lo = -0.5 exactly
    x = np.array([3.0, 1.1171875, 0, 0, 0, 0, 0, 0])
    hi, lo, s, e = _digits(x)
    assert e[0, 0] == 2 and s[0, 0] == 2.0 ** -6
    assert hi[0, 0] == 192 and lo[0, 0] == 0
    assert hi[0, 1] == 72 and lo[0, 1] == -0.5
