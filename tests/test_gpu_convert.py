"""GPU: tt.fp_to_fp with a bf16, fp16 or fp8 source, bit for bit against the
oracle (the source widened exactly to fp32, then rounded once; pinned to
PyTorch's casts in tests/test_oracle_convert.py).

Every bf16 / fp16 bit pattern and every fp8 code, to every other format,
in all four rounding / saturation variants; large arrays (the 16-byte
streaming kernels) with ragged lengths and misaligned starts (the element
tail and the scalar kernels); the table op.
"""
import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu

TD = {O.F32: torch.float32, O.BF16: torch.bfloat16, O.F16: torch.float16,
      O.E4M3FN: torch.float8_e4m3fn, O.E5M2: torch.float8_e5m2}
NP = {O.F32: np.float32, O.BF16: np.uint16, O.F16: np.uint16, O.E4M3FN: np.uint8, O.E5M2: np.uint8}
SRCS = [O.BF16, O.F16, O.E4M3FN, O.E5M2]
PAIRS = [(s, d) for s in SRCS for d in (O.F32, O.BF16, O.F16, O.E4M3FN, O.E5M2) if s != d and
         not (s in (O.E4M3FN, O.E5M2) and d == O.F32)]   # fp8 -> fp32: the decode path, tested elsewhere


def all_codes(fmt):
    n = 1 << (8 * np.dtype(NP[fmt]).itemsize)
    return np.arange(n, dtype=np.uint32).astype(NP[fmt])


def to_dev(codes, fmt, dev):
    a = codes if NP[fmt] != np.uint16 else codes.view(np.int16)
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev).view(TD[fmt])


def bits(t, fmt):
    if fmt == O.F32:
        return t.cpu().numpy().view(np.uint32)
    v = t.view(torch.int16 if NP[fmt] == np.uint16 else torch.uint8).cpu().numpy()
    return v.view(NP[fmt])


def want_bits(codes, src, dst, rtz, sat):
    r = O.convert(codes, src, dst, rtz=rtz, sat=sat)
    return r.view(np.uint32) if dst == O.F32 else r


@pytest.mark.parametrize("src,dst", PAIRS)
@pytest.mark.parametrize("rounding,sat", [("rtne", False), ("rtne", True), ("rtz", False), ("rtz", True)])
def test_every_source_code(tx, dev, src, dst, rounding, sat):
    c = all_codes(src)
    c = np.concatenate([c] * (8192 // c.size + 1))   # fp8: past one vector chunk
    out = tx.fp_to_fp(to_dev(c, src, dev), TD[dst], rounding=rounding, saturate=sat)
    got, want = bits(out, dst), want_bits(c, src, dst, rounding == "rtz", sat)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, (bad[:5], got[bad[:5]], want[bad[:5]], c[bad[:5]])


@pytest.mark.parametrize("src,dst", [(O.BF16, O.E4M3FN), (O.F16, O.E5M2), (O.E4M3FN, O.BF16),
                                     (O.E5M2, O.F16), (O.BF16, O.F32), (O.F16, O.BF16), (O.E5M2, O.E4M3FN)])
@pytest.mark.parametrize("n,offset", [(1_000_003, 0), (4096 * 37, 0), (130, 0), (65, 1), (17, 3), (50_001, 1)])
def test_large_ragged_misaligned(tx, dev, src, dst, n, offset):
    """Random codes: the streaming kernels on whole chunks, the element kernel
    on the rest, and only the element kernel when the buffers start off
    their access alignment (an offset of whole elements)."""
    g = np.random.default_rng(n + 7 * offset + src)
    c = g.integers(0, 1 << (8 * np.dtype(NP[src]).itemsize), size=n + offset, dtype=np.uint64).astype(NP[src])
    x = to_dev(c, src, dev)[offset:]
    out_full = torch.empty(n + offset, dtype=TD[dst], device=dev)
    out = out_full[offset:]
    for rounding, sat in (("rtne", False), ("rtz", True)):
        tx.fp_to_fp(x, TD[dst], rounding=rounding, saturate=sat, out=out)
        got, want = bits(out, dst), want_bits(c[offset:], src, dst, rounding == "rtz", sat)
        assert np.array_equal(got, want)


def test_table_op_and_errors(tx, dev):
    c = all_codes(O.BF16)
    x = to_dev(c, O.BF16, dev)
    out = torch.empty(c.size, dtype=torch.float8_e4m3fn, device=dev)
    tx.invoke("tt.fp_to_fp", [out, x, c.size, tx._lib.BF16, tx._lib.FP8E4M3FN, tx.RTNE, 1])
    assert np.array_equal(bits(out, O.E4M3FN), O.convert(c, O.BF16, O.E4M3FN, sat=True))
    with pytest.raises(tx.TxError, match="float32 source"):
        tx.fp_to_fp(x, torch.float8_e4m3fn, rounding="rs", saturate=True,
                    rbits=torch.zeros(c.size, dtype=torch.int32, device=dev))
    with pytest.raises(tx.TxError, match="not served"):
        tx.fp_to_fp(x, torch.int32)
