"""The oracle's conversions with a bf16, fp16 or fp8 source (oracle.convert:
the source widened exactly to fp32, then rounded once), pinned independently
of the oracle's own encoder:

* round to nearest even, non-saturating: PyTorch's casts, over every bf16
  and fp16 bit pattern and every fp8 code, to every other format;
* saturating: PyTorch's cast of the value clamped to +-max in fp32 (the
  reference's clamp-then-convert idiom, mxfp8_utils.py:36-38), NaN kept;
* round toward zero: the largest-magnitude destination value not above the
  source's magnitude, found by searching the sorted table of every
  destination value.
"""
import numpy as np
import pytest
import torch

import oracle as O

TD = {O.BF16: torch.bfloat16, O.F16: torch.float16, O.E4M3FN: torch.float8_e4m3fn, O.E5M2: torch.float8_e5m2}
BITS = {O.BF16: torch.int16, O.F16: torch.int16, O.E4M3FN: torch.uint8, O.E5M2: torch.uint8}
NP_BITS = {O.BF16: np.uint16, O.F16: np.uint16, O.E4M3FN: np.uint8, O.E5M2: np.uint8}
FMAX = {O.BF16: 3.3895313892515355e38, O.F16: 65504.0, O.E4M3FN: 448.0, O.E5M2: 57344.0}
PAIRS = [(O.BF16, d) for d in (O.E4M3FN, O.E5M2, O.F16)] + \
        [(O.F16, d) for d in (O.E4M3FN, O.E5M2, O.BF16)] + \
        [(O.E4M3FN, O.E5M2), (O.E5M2, O.E4M3FN)]


def all_codes(fmt):
    n = 1 << (8 * np.dtype(NP_BITS[fmt]).itemsize)
    return np.arange(n, dtype=np.uint32).astype(NP_BITS[fmt])


def torch_cast(codes, src, dst, values=None):
    """torch's cast of the source codes (or of fp32 `values`) to dst, as bits."""
    t = torch.from_numpy(values) if values is not None else \
        torch.from_numpy(codes.view(np.int16) if NP_BITS[src] == np.uint16 else codes).view(TD[src])
    out = t.to(TD[dst]).view(BITS[dst]).numpy()
    return out.view(NP_BITS[dst])


@pytest.mark.parametrize("src,dst", PAIRS)
def test_rtne_matches_torch(src, dst):
    c = all_codes(src)
    got = O.convert(c, src, dst)
    want = torch_cast(c, src, dst)
    x = O.widen(c, src)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan]), np.flatnonzero(got[~nan] != want[~nan])[:8]
    # NaN: the destination's canonical NaN code, the source's sign
    canon = {O.BF16: 0x7FC0, O.F16: 0x7E00, O.E4M3FN: 0x7F, O.E5M2: 0x7F}[dst]
    sbit = np.signbit(x[nan]).astype(np.uint32) << (8 * np.dtype(NP_BITS[dst]).itemsize - 1)
    assert np.array_equal(got[nan].astype(np.uint32), canon | sbit)


@pytest.mark.parametrize("src,dst", PAIRS)
def test_saturating_matches_clamp_then_torch(src, dst):
    c = all_codes(src)
    x = O.widen(c, src)
    got = O.convert(c, src, dst, sat=True)
    m = np.float32(FMAX[dst])
    want = torch_cast(c, src, dst, values=np.clip(x, -m, m).astype(np.float32))
    ok = ~np.isnan(x)
    assert np.array_equal(got[ok], want[ok])


@pytest.mark.parametrize("src,dst", PAIRS)
def test_rtz_is_the_largest_value_not_above(src, dst):
    c = all_codes(src)
    x = O.widen(c, src).astype(np.float64)
    got = O.convert(c, src, dst, rtz=True, sat=True)
    with np.errstate(invalid="ignore"):
        table = O.widen(all_codes(dst), dst).astype(np.float64)
    fin = np.sort(np.unique(np.abs(table[np.isfinite(table)])))
    ok = np.isfinite(x)
    ax = np.abs(x[ok])
    idx = np.searchsorted(fin, ax, side="right") - 1
    want_mag = fin[idx]
    got_val = O.widen(got[ok], dst).astype(np.float64)
    assert np.array_equal(np.abs(got_val), want_mag)
    # the sign follows the source's (zeros included)
    assert np.array_equal(np.signbit(got_val), np.signbit(x[ok]))


@pytest.mark.parametrize("src", [O.BF16, O.F16, O.E4M3FN, O.E5M2])
def test_widen_is_exact(src):
    c = all_codes(src)
    x = O.widen(c, src)
    t = torch.from_numpy(c.view(np.int16) if NP_BITS[src] == np.uint16 else c).view(TD[src]).float().numpy()
    both = np.isnan(x) & np.isnan(t)
    assert np.array_equal(x[~both].view(np.uint32), t[~both].view(np.uint32))
    assert np.array_equal(np.isnan(x), np.isnan(t))
