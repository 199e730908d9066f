"""GPU parity: tt.fp_to_fp (fp32 <-> e4m3fn / e5m2) vs the oracle, bit-exact."""
import json
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
FMTS = {1: torch.float8_e4m3fn, 2: torch.float8_e5m2}


def _golden_inputs():
    with open(os.path.join(HERE, "golden", "fp8_golden.json")) as f:
        return np.array(json.load(f)["encode_inputs"], dtype=np.uint32).view(np.float32)


def _enc(tx, x_np, fmt, sat, rounding="rtne", dev="cuda:0"):
    x = torch.from_numpy(x_np).to(dev)
    return tx.fp_to_fp(x, FMTS[fmt], rounding=rounding, saturate=sat).view(torch.uint8).cpu().numpy()


def _dec(tx, codes_np, fmt, dev="cuda:0"):
    c = torch.from_numpy(codes_np).to(dev).view(FMTS[fmt])
    return tx.fp_to_fp(c, torch.float32).cpu().numpy()


@pytest.mark.parametrize("fmt", [1, 2])
def test_decode_every_code(tx, oracle, dev, fmt):
    # 256 codes tiled past one vector chunk, plus a tail
    codes = np.tile(np.arange(256, dtype=np.uint8), 33)
    got = _dec(tx, codes, fmt).view(np.uint32)
    ref = oracle.decode(codes, fmt).view(np.uint32)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("fmt", [1, 2])
@pytest.mark.parametrize("sat", [False, True])
@pytest.mark.parametrize("rounding", ["rtne", "rtz"])
def test_encode_golden_inputs(tx, oracle, dev, fmt, sat, rounding):
    x = np.tile(_golden_inputs(), 3)
    got = _enc(tx, x, fmt, sat, rounding)
    ref = oracle.encode(x, fmt, sat) if rounding == "rtne" else oracle.encode_rtz(x, fmt, sat)
    bad = np.nonzero(got != ref)[0]
    assert bad.size == 0, [(hex(int(x[i:i + 1].view(np.uint32)[0])), int(got[i]), int(ref[i]))
                           for i in bad[:8]]


@pytest.mark.parametrize("fmt", [1, 2])
@pytest.mark.parametrize("sat", [False, True])
def test_roundtrip_config_full_size(tx, oracle, dev, fmt, sat):
    """16,777,216 values of the fp8 round-trip workload, encode then decode."""
    import workloads
    x_np = workloads.fp8_input()
    x = torch.from_numpy(x_np).to(dev)
    q = tx.fp_to_fp(x, FMTS[fmt], saturate=sat)
    back = tx.fp_to_fp(q, torch.float32)
    ref_q = oracle.encode(x_np, fmt, sat)
    got_q = q.view(torch.uint8).cpu().numpy()
    assert np.array_equal(got_q, ref_q), f"{np.count_nonzero(got_q != ref_q)} encode mismatches"
    ref_b = oracle.decode(ref_q, fmt).view(np.uint32)
    assert np.array_equal(back.cpu().numpy().view(np.uint32), ref_b)


@pytest.mark.parametrize("n", [0, 1, 3, 4095, 4097, 70001])
def test_sizes_and_tails(tx, oracle, dev, n):
    g = np.random.default_rng(n)
    x = g.integers(0, 1 << 32, size=n, dtype=np.uint64).astype(np.uint32).view(np.float32)
    for fmt in (1, 2):
        got = _enc(tx, x, fmt, False)
        assert np.array_equal(got, oracle.encode(x, fmt, False))
        codes = g.integers(0, 256, size=n, dtype=np.uint8)
        assert np.array_equal(_dec(tx, codes, fmt).view(np.uint32),
                              oracle.decode(codes, fmt).view(np.uint32))


def test_unaligned_buffers_take_scalar_path(tx, oracle, dev):
    g = np.random.default_rng(3)
    x_np = g.standard_normal(20000).astype(np.float32) * 300
    x = torch.from_numpy(x_np).to(dev)
    xv = x[1:]  # 4-byte aligned, not 16
    out = torch.empty(xv.numel() + 1, dtype=torch.uint8, device=dev)[1:]
    tx.fp_to_fp(xv, torch.float8_e4m3fn, out=out.view(torch.float8_e4m3fn))
    assert np.array_equal(out.cpu().numpy(), oracle.encode(x_np[1:], 1, False))


def test_invalid_requests_raise(tx, dev):
    x = torch.zeros(16, device=dev)
    with pytest.raises(tx.TxError, match="UNSUPPORTED"):
        tx.fp_to_fp(x, torch.float8_e4m3fn, rounding="rs")
    with pytest.raises(tx.TxError, match="UNSUPPORTED"):
        tx.fp_to_fp(x.to(torch.bfloat16), torch.float8_e4m3fn, rounding="rs")
