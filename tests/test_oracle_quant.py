"""Pins the oracle's absmax + fp8 quantisers (txo_quant_mx, txo_quant_row).

MX (the reference's _compute_scale_and_quantize, mxfp8_utils.py:17-38): the
e8m0 scale of every block with a normal fp32 quotient amax / fmax is the
smallest power of two at or above it (checked as a closed-form property, not
by repeating the bit trick; a subnormal quotient gives 2^-126), and the
codes equal PyTorch's own fp8 cast of the clamped, scaled values (an
independent conversion).  Row-wise: the scale is amax / fmax and
the codes PyTorch's cast of clamp(x * fmax / amax).  Special blocks: zeros,
NaN (ignored by the scale, kept as NaN), Inf, denormals; bf16 input."""
import numpy as np
import pytest
import torch

FMAX = {1: 448.0, 2: 57344.0}
TD = {1: torch.float8_e4m3fn, 2: torch.float8_e5m2}


def _torch_codes(v, fmt):
    """PyTorch fp8 cast of fp32 values already clamped (NaN kept)."""
    return torch.from_numpy(np.ascontiguousarray(v, np.float32)).to(TD[fmt]).view(torch.uint8).numpy()


def _mx_input(g, rows, K):
    x = (g.standard_normal((rows, K)) * np.exp2(g.integers(-20, 20, (rows, 1)))).astype(np.float32)
    return x


@pytest.mark.parametrize("fmt", [1, 2])
def test_mx_scale_is_smallest_power_of_two_at_or_above(oracle, fmt):
    g = np.random.default_rng(fmt)
    rows, K = 64, 256
    x = _mx_input(g, rows, K)
    q, s = oracle.quant_mx(x, fmt)
    amax = np.abs(x.reshape(rows, K // 32, 32)).max(axis=2)
    descale = (amax.astype(np.float32) / np.float32(FMAX[fmt])).astype(np.float64)
    S = np.exp2(s.astype(np.float64) - 127)
    assert np.all(S >= descale) and np.all(S / 2 < descale)
    # codes: PyTorch's cast of clamp(x / S)
    xs = (x.reshape(rows, K // 32, 32) * (1.0 / S)[:, :, None].astype(np.float32)).astype(np.float32)
    want = _torch_codes(np.clip(xs, -FMAX[fmt], FMAX[fmt]).reshape(rows, K), fmt)
    assert np.array_equal(q, want)


@pytest.mark.parametrize("fmt", [1, 2])
def test_mx_special_blocks(oracle, fmt):
    K = 32 * 6
    x = np.ones((1, K), np.float32)
    x[0, 0:32] = 0.0                                  # all zero: scale code 0, codes 0
    x[0, 32:64] = np.linspace(-3, 3, 32)
    x[0, 40] = np.nan                                 # NaN ignored by the scale, kept as NaN
    x[0, 64:96] = 1.0
    x[0, 70] = np.inf                                 # Inf: scale 255, zeros, NaN for the Inf
    x[0, 96:128] = np.float32(1e-40)                  # denormal amax
    x[0, 128:160] = np.float32(2.0 ** 100)
    x[0, 160:192] = -np.float32(FMAX[fmt])            # amax exactly fmax: scale 2^0
    q, s = oracle.quant_mx(x, fmt)
    assert s[0, 0] == 0 and np.all(q[0, 0:32] == 0)
    ref_nan = oracle.quant_mx(np.where(np.isnan(x), 0, x)[:, 32:64].copy(), fmt)
    assert s[0, 1] == ref_nan[1][0, 0]
    assert (q[0, 40] & 0x7F) == 0x7F
    assert np.array_equal(np.delete(q[0, 32:64], 8), np.delete(ref_nan[0][0], 8))
    assert s[0, 2] == 255 and (q[0, 70] & 0x7F) == 0x7F and np.all(np.delete(q[0, 64:96], 6) == 0)
    # a subnormal quotient has exponent field 0: adding 0x007FFFFF carries into
    # field 1, so the reference's rounding gives 2^-126, not a smaller power
    assert s[0, 3] == 1
    assert s[0, 5] == 127 and np.all(q[0, 160:192] == _torch_codes(x[0, 160:192], fmt))


@pytest.mark.parametrize("fmt", [1, 2])
def test_rowwise_scale_and_codes(oracle, fmt):
    g = np.random.default_rng(10 + fmt)
    rows, K = 20, 300
    x = _mx_input(g, rows, K)
    x[3] = 0.0
    x[5, 7] = np.nan
    q, s = oracle.quant_rowwise(x, fmt)
    amax = np.abs(np.nan_to_num(x, nan=0.0)).max(axis=1).astype(np.float32)
    amax[amax == 0] = 1.0
    assert np.array_equal(s, (amax / np.float32(FMAX[fmt])).astype(np.float32))
    mult = (np.float32(FMAX[fmt]) / amax).astype(np.float32)
    want = _torch_codes(np.clip((x * mult[:, None]).astype(np.float32), -FMAX[fmt], FMAX[fmt]), fmt)
    nan = np.isnan(x)
    assert np.array_equal(q[~nan], want[~nan]) and np.all((q[nan] & 0x7F) == 0x7F)
    assert np.all(q[3] == 0)


def test_bf16_input_is_widened_exactly(oracle):
    g = np.random.default_rng(4)
    x = g.standard_normal((8, 64)).astype(np.float32)
    xb = torch.from_numpy(x).to(torch.bfloat16)
    bits = xb.view(torch.int16).numpy().view(np.uint16)
    q1, s1 = oracle.quant_mx(bits, 1)
    q2, s2 = oracle.quant_mx(xb.float().numpy(), 1)
    assert np.array_equal(q1, q2) and np.array_equal(s1, s2)


def test_workload_generator_agrees(oracle):
    """The benchmark's numpy MX quantiser (workloads.quant_mx) gives the
    oracle's bytes."""
    import workloads
    g = np.random.default_rng(9)
    x = g.standard_normal((16, 512)).astype(np.float32)
    for name, fmt in (("e4m3fn", 1), ("e5m2", 2)):
        q1, s1 = workloads.quant_mx(x, name)
        q2, s2 = oracle.quant_mx(x, fmt)
        assert np.array_equal(q1, q2) and np.array_equal(s1, s2)
