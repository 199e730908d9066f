"""Pins for the oracle's fp16 / bf16 conversions and its stochastic rounding (CPU only).

Round to nearest even is checked against numpy's float16 and torch's
bfloat16 conversions (their saturating forms after clamp(+-max), the
reference's idiom), round toward zero against a search of the sorted
representable values, the format-generic method against the fp8 encoders
pinned in test_oracle_fp8.py, and stochastic rounding against its definition
(round toward zero, one step up iff r + floor(frac * 2^32) >= 2^32) computed
in exact rational arithmetic, on both sides of every threshold.
"""
from fractions import Fraction

import numpy as np
import pytest
import torch

E4, E5, BF16, F16 = 1, 2, 3, 6
FORMATS = [E4, E5, BF16, F16]
MAXC = {E4: 0x7E, E5: 0x7B, BF16: 0x7F7F, F16: 0x7BFF}
SIGN = {E4: 0x80, E5: 0x80, BF16: 0x8000, F16: 0x8000}
NANC = {E4: 0x7F, E5: 0x7F, BF16: 0x7FC0, F16: 0x7E00}


def values(oracle, fmt):
    """Exact magnitudes (float64) of codes 0 .. max, from a source other than
    the oracle's own table where one exists."""
    codes = np.arange(MAXC[fmt] + 1)
    if fmt == F16:
        return codes.astype(np.uint16).view(np.float16).astype(np.float64)
    if fmt == BF16:
        return (codes.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    return oracle.decode(codes.astype(np.uint8), fmt).astype(np.float64)  # pinned vs torch


def samples(seed, n=200_000):
    """Random fp32 bit patterns (all classes) plus specials, subnormals and
    values at and around the formats' largest finite values and ties."""
    g = np.random.default_rng(seed)
    raw = g.integers(0, 2 ** 32, size=n, dtype=np.uint64).astype(np.uint32).view(np.float32)
    scaled = (g.standard_normal(n) * np.exp2(g.integers(-30, 20, size=n))).astype(np.float32)
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 65504.0, 65519.99, 65520.0, 65536.0,
                        448.0, 464.0, 480.0, 57344.0, 61440.0, 3.3895313892515355e38, 3.4e38,
                        5.96e-8, 2.98e-8, 6.1e-5, 1e-45, -1e-40, 1.00048828125, 1.00146484375],
                       np.float32)
    return np.concatenate([raw, scaled, special, -special])


@pytest.mark.parametrize("sat", [False, True])
def test_f16_rne_vs_numpy(oracle, sat):
    x = samples(1)
    got = oracle.encode_fmt(x, F16, rtz=False, sat=sat)
    with np.errstate(over="ignore", invalid="ignore"):
        want = (np.clip(x, -65504, 65504) if sat else x).astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.array_equal(got[nan], NANC[F16] | ((x[nan].view(np.uint32) >> 16) & 0x8000).astype(np.uint16))


@pytest.mark.parametrize("sat", [False, True])
def test_bf16_rne_vs_torch(oracle, sat):
    x = samples(2)
    got = oracle.encode_fmt(x, BF16, rtz=False, sat=sat)
    t = torch.from_numpy(x.copy())
    if sat:
        m = float(np.float32(3.3895313892515355e38))
        t = torch.clamp(t, -m, m)
    want = t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all((got[nan] & 0x7FFF) == NANC[BF16])


@pytest.mark.parametrize("fmt", [F16, BF16])
@pytest.mark.parametrize("sat", [False, True])
def test_rtz_is_largest_value_not_above(oracle, fmt, sat):
    x = samples(3 + fmt)
    got = oracle.encode_fmt(x, fmt, rtz=True, sat=sat)
    v = values(oracle, fmt)
    a = np.abs(x.astype(np.float64))
    fin = np.isfinite(x)
    want = np.minimum(np.searchsorted(v, a[fin], side="right") - 1, MAXC[fmt]).astype(np.uint32)
    want |= np.where(np.signbit(x[fin]), SIGN[fmt], 0).astype(np.uint32)
    assert np.array_equal(got[fin].astype(np.uint32), want)
    inf = np.isinf(x)
    ovf = MAXC[fmt] if sat else {F16: 0x7C00, BF16: 0x7F80}[fmt]
    assert np.all((got[inf] & 0x7FFF) == ovf)


@pytest.mark.parametrize("fmt", [E4, E5])
@pytest.mark.parametrize("rtz", [False, True])
@pytest.mark.parametrize("sat", [False, True])
def test_generic_method_matches_fp8_encoders(oracle, fmt, rtz, sat):
    x = samples(7)
    got = oracle.encode_fmt(x, fmt, rtz=rtz, sat=sat)
    want = (oracle.encode_rtz if rtz else oracle.encode)(x, fmt, sat)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("fmt", FORMATS)
def test_rs_with_zero_bits_is_saturating_rtz(oracle, fmt):
    x = samples(11)
    got = oracle.round_rs(x, np.zeros(x.size, np.uint32), fmt)
    assert np.array_equal(got, oracle.encode_fmt(x, fmt, rtz=True, sat=True))


@pytest.mark.parametrize("fmt", FORMATS)
def test_rs_threshold_in_exact_arithmetic(oracle, fmt):
    """floor(frac * 2^32) from Fractions; r one below the threshold keeps the
    truncated code, r at it moves one step up."""
    v = values(oracle, fmt)
    g = np.random.default_rng(20 + fmt)
    # finite values strictly below max, spread over the whole range incl. subnormals
    lo_i = g.integers(0, MAXC[fmt], size=3000)
    t = g.random(3000)
    x = (v[lo_i] + t * (v[lo_i + 1] - v[lo_i])).astype(np.float32)
    x = np.concatenate([x, v[lo_i].astype(np.float32)])  # exactly representable values too
    x = x * np.where(g.random(x.size) < 0.5, -1, 1).astype(np.float32)
    a = np.abs(x.astype(np.float64))
    ok = a < v[-1]
    x, a = x[ok], a[ok]
    lo = np.searchsorted(v, a, side="right") - 1
    thr = np.array([int(((Fraction(float(ai)) - Fraction(float(v[l]))) / (Fraction(float(v[l + 1])) - Fraction(float(v[l])))) * 2 ** 32)
                    for ai, l in zip(a, lo)], dtype=np.uint64)
    sign = np.where(np.signbit(x), SIGN[fmt], 0).astype(np.uint32)
    # below the threshold (or any r when thr == 0): the truncated code
    r_below = np.where(thr > 0, (2 ** 32 - thr - 1), 2 ** 32 - 1).astype(np.uint32)
    assert np.array_equal(oracle.round_rs(x, r_below, fmt).astype(np.uint32), lo.astype(np.uint32) | sign)
    up = thr > 0
    r_at = (2 ** 32 - thr[up]).astype(np.uint32)
    assert np.array_equal(oracle.round_rs(x[up], r_at, fmt).astype(np.uint32),
                          (lo[up] + 1).astype(np.uint32) | sign[up])
    assert up.sum() > 1000


@pytest.mark.parametrize("fmt", FORMATS)
def test_rs_is_unbiased(oracle, fmt):
    """Mean of the rounded values over uniform random bits equals x (within
    5 standard errors), and every result is one of the two neighbours."""
    v = values(oracle, fmt)
    g = np.random.default_rng(40 + fmt)
    n = 200_000
    for i in (3, 100, len(v) // 2, len(v) - 3):
        xv = np.float32(v[i] + 0.3 * (v[i + 1] - v[i]))
        x = np.full(n, xv, np.float32)
        r = g.integers(0, 2 ** 32, size=n, dtype=np.uint64).astype(np.uint32)
        codes = oracle.round_rs(x, r, fmt).astype(np.int64)
        assert set(np.unique(codes)) <= {i, i + 1}
        frac = (float(xv) - v[i]) / (v[i + 1] - v[i])
        mean = v[codes].mean()
        se = (v[i + 1] - v[i]) * np.sqrt(frac * (1 - frac) / n)
        assert abs(mean - float(xv)) < 5 * se, (fmt, i, mean, float(xv), se)
