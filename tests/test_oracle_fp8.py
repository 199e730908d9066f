"""Pins for the fp8 codec of the oracle (CPU only).

Each check compares the oracle with something independent of it: the OCP
spec's defining values, PyTorch's float8 dtypes (committed fixture and live),
and a brute-force search over the decoded code table for round-toward-zero.
"""
import json
import os

import numpy as np
import pytest
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
E4, E5 = 1, 2
NAMES = {E4: "e4m3fn", E5: "e5m2"}
TD = {E4: torch.float8_e4m3fn, E5: torch.float8_e5m2}
FMAX = {E4: 448.0, E5: 57344.0}


@pytest.fixture(scope="module")
def golden():
    with open(os.path.join(HERE, "golden", "fp8_golden.json")) as f:
        return json.load(f)


def bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


# --- decode -----------------------------------------------------------------
@pytest.mark.parametrize("fmt", [E4, E5])
def test_decode_all_codes_match_fixture(oracle, golden, fmt):
    got = bits(oracle.decode(np.arange(256, dtype=np.uint8), fmt))
    ref = np.array(golden["decode"][NAMES[fmt]], dtype=np.uint32)
    ref_nan = (ref & 0x7FFFFFFF) > 0x7F800000
    assert np.array_equal(got[~ref_nan], ref[~ref_nan])
    # NaN codes: canonical quiet NaN carrying the code's sign
    codes = np.arange(256)[ref_nan]
    assert np.array_equal(got[ref_nan], 0x7FC00000 | ((codes >> 7) << 31).astype(np.uint32))


def test_decode_spec_values(oracle):
    # OCP FP8 spec, table of E4M3/E5M2 limits
    d4 = lambda c: oracle.decode1(c, E4)
    d5 = lambda c: oracle.decode1(c, E5)
    assert d4(0x7E) == 448.0 and d4(0xFE) == -448.0
    assert d4(0x08) == 2.0 ** -6 and d4(0x01) == 2.0 ** -9 and d4(0x07) == 7 * 2.0 ** -9
    assert d4(0x38) == 1.0 and d4(0x00) == 0.0 and np.signbit(d4(0x80))
    assert np.isnan(d4(0x7F)) and np.isnan(d4(0xFF))
    assert d5(0x7B) == 57344.0 and d5(0x04) == 2.0 ** -14 and d5(0x01) == 2.0 ** -16
    assert d5(0x3C) == 1.0 and d5(0x7C) == np.inf and d5(0xFC) == -np.inf
    assert all(np.isnan(d5(c)) for c in (0x7D, 0x7E, 0x7F, 0xFD, 0xFE, 0xFF))


# --- encode -----------------------------------------------------------------
@pytest.mark.parametrize("fmt", [E4, E5])
@pytest.mark.parametrize("sat", [False, True])
def test_encode_matches_fixture(oracle, golden, fmt, sat):
    x = np.array(golden["encode_inputs"], dtype=np.uint32).view(np.float32)
    key = "encode_sat" if sat else "encode"
    ref = np.array(golden[key][NAMES[fmt]], dtype=np.uint8)
    got = oracle.encode(x, fmt, sat)
    bad = np.nonzero(got != ref)[0]
    assert bad.size == 0, [(hex(int(bits(x[i]))), int(got[i]), int(ref[i])) for i in bad[:10]]


@pytest.mark.parametrize("fmt", [E4, E5])
def test_encode_ties_go_to_even(oracle, fmt):
    # midpoint of neighbouring codes c, c+1 rounds to the one with a 0 last bit
    codes = np.arange(0, 0x7E if fmt == E4 else 0x7B, dtype=np.uint8)
    lo = oracle.decode(codes, fmt).astype(np.float64)
    hi = oracle.decode(codes + 1, fmt).astype(np.float64)
    mid = ((lo + hi) / 2).astype(np.float32)
    assert np.array_equal(mid.astype(np.float64), (lo + hi) / 2)  # exact in fp32
    even = np.where(codes % 2 == 0, codes, codes + 1).astype(np.uint8)
    assert np.array_equal(oracle.encode(mid, fmt, False), even)
    assert np.array_equal(oracle.encode(-mid, fmt, False), even | 0x80)


def test_encode_overflow_rules(oracle):
    enc = oracle.encode1
    # e4m3fn: 464 is the tie between 448 and the (NaN) slot above it -> 448
    assert enc(464.0, E4, False) == 0x7E
    assert enc(np.nextafter(np.float32(464), np.float32(1e9)), E4, False) == 0x7F
    assert enc(480.0, E4, False) == 0x7F and enc(-1e30, E4, False) == 0xFF
    assert enc(np.inf, E4, False) == 0x7F and enc(np.inf, E4, True) == 0x7E
    assert enc(-np.inf, E4, True) == 0xFE and enc(1e30, E4, True) == 0x7E
    # e5m2: 61440 ties between 57344 (odd code) and Inf (even) -> Inf
    assert enc(61440.0, E5, False) == 0x7C and enc(61439.99, E5, False) == 0x7B
    assert enc(np.inf, E5, False) == 0x7C and enc(np.inf, E5, True) == 0x7B
    assert enc(-65536.0, E5, True) == 0xFB
    for fmt in (E4, E5):
        for sat in (False, True):
            assert enc(np.float32("nan"), fmt, sat) == 0x7F
            assert enc(-np.float32("nan"), fmt, sat) == 0xFF
            assert enc(-0.0, fmt, sat) == 0x80
            assert enc(np.float32(1e-45), fmt, sat) == 0x00


@pytest.mark.parametrize("fmt", [E4, E5])
def test_encode_random_vs_torch(oracle, fmt):
    g = np.random.default_rng(7)
    x = g.integers(0, 1 << 32, size=2_000_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    t = torch.from_numpy(x.copy())
    ref = t.to(TD[fmt]).view(torch.uint8).numpy()
    assert np.array_equal(oracle.encode(x, fmt, False), ref)
    tc = torch.where(torch.isnan(t), t, t.clamp(-FMAX[fmt], FMAX[fmt]))
    assert np.array_equal(oracle.encode(x, fmt, True), tc.to(TD[fmt]).view(torch.uint8).numpy())


@pytest.mark.parametrize("fmt", [E4, E5])
def test_encode_strided_sweep_vs_torch(oracle, fmt):
    # every 251st fp32 bit pattern (17.1 M patterns covering all exponents)
    x = (np.arange(0, 1 << 32, 251, dtype=np.uint64)).astype(np.uint32).view(np.float32)
    t = torch.from_numpy(x)
    assert np.array_equal(oracle.encode(x, fmt, False), t.to(TD[fmt]).view(torch.uint8).numpy())


@pytest.mark.parametrize("fmt", [E4, E5])
def test_rtz_brute_force(oracle, fmt):
    """Round toward zero = the largest-magnitude code not above |x|, clamped
    to max for finite x; found here by searching PyTorch's decode table."""
    table = torch.arange(128, dtype=torch.uint8).view(TD[fmt]).float().numpy().astype(np.float64)
    maxc = 0x7E if fmt == E4 else 0x7B
    mags = table[: maxc + 1]  # increasing
    g = np.random.default_rng(11)
    x = np.concatenate([
        (g.standard_normal(200_000) * np.exp2(g.uniform(-20, 18, 200_000))).astype(np.float32),
        oracle.decode(np.arange(256, dtype=np.uint8), fmt)])
    x = x[np.isfinite(x)]
    a = np.abs(x.astype(np.float64))
    lo = np.searchsorted(mags, a, side="right") - 1
    lo = np.minimum(lo, maxc)
    expect = (lo | np.where(np.signbit(x), 0x80, 0)).astype(np.uint8)
    got = oracle.encode_rtz(x, fmt, False)
    assert np.array_equal(got, expect)
    # saturation flag does not change finite round-toward-zero results
    assert np.array_equal(oracle.encode_rtz(x, fmt, True), expect)
    for sat in (False, True):
        inf_code = oracle.encode_rtz(np.array([np.inf], np.float32), fmt, sat)[0]
        assert inf_code == (maxc if sat else (0x7F if fmt == E4 else 0x7C))


@pytest.mark.slow
@pytest.mark.parametrize("fmt", [E4, E5])
@pytest.mark.parametrize("sat", [False, True])
def test_encode_exhaustive_vs_torch(oracle, fmt, sat):
    """All 2^32 fp32 bit patterns (opt-in: TX_SLOW=1, about a minute each)."""
    step = 1 << 26
    for start in range(0, 1 << 32, step):
        x = np.arange(start, start + step, dtype=np.uint64).astype(np.uint32).view(np.float32)
        t = torch.from_numpy(x)
        if sat:
            t = torch.where(torch.isnan(t), t, t.clamp(-FMAX[fmt], FMAX[fmt]))
        ref = t.to(TD[fmt]).view(torch.uint8).numpy()
        got = oracle.encode(x, fmt, sat)
        assert np.array_equal(got, ref), f"mismatch in [{start:#x}, {start + step:#x})"


def test_roundtrip_identity_on_codes(oracle):
    for fmt in (E4, E5):
        codes = np.arange(256, dtype=np.uint8)
        vals = oracle.decode(codes, fmt)
        fin = np.isfinite(vals)
        assert np.array_equal(oracle.encode(vals[fin], fmt, False), codes[fin])
