"""GPU parity of 16-bit dots whose operands the fast path reads in place
although their rows are not whole 16-byte chunks apart or long (rows 4-byte
aligned, any K of at least two 64-element steps): the persistent tile
(tx_gemm_*_persist_kt) for products of at least one 256 x 256 tile per CU,
the 256 x 128 tile with K split otherwise, and the few columns past the last
256-column block of a wide product by the VALU strip kernel.

The last chunk of each row is fetched as the row's last 16 bytes and its
repeated bytes are cleared in registers, so the cases put that chunk at
every kind of place in the last K step: its first chunk (the lane offsets
then need the shifted scalar offset to stay non-negative), a middle one,
the last one, and none (whole chunks past the row end only).  Integer-valued
operands make every fp32 sum exact, so the outputs must equal the oracle's
rounding bit for bit: a repeated or dropped K position changes a sum.
"""
import numpy as np
import pytest
import torch

from test_gpu_gemm import BF16_TOL, _np_bits, check_close

pytestmark = pytest.mark.gpu

BF16, F16 = 3, 6
_TD = {BF16: torch.bfloat16, F16: torch.float16}


def _int_codes(g, shape, fmt):
    """Integers in [-3, 3] as bf16 / fp16 bits (exact in both formats)."""
    x = g.integers(-3, 4, size=shape).astype(np.float32)
    if fmt == F16:
        return x.astype(np.float16).view(np.uint16)
    return (x.view(np.uint32) >> 16).astype(np.uint16)


def _dev(bits, fmt, dev, pad=0):
    """bits (rows x K) on the device, rows `pad` elements longer than K."""
    rows, k = bits.shape
    buf = np.zeros((rows, k + pad), np.uint16)
    buf[:, :k] = bits
    t = torch.from_numpy(buf.view(np.int16)).to(dev).view(_TD[fmt])
    return t[:, :k]


def _exact(tx, oracle, dev, M, N, K, fmt=BF16, out_fmt=BF16, pad_a=0, pad_b=0, seed=0):
    g = np.random.default_rng(seed)
    A = _int_codes(g, (M, K), fmt)
    B = _int_codes(g, (N, K), fmt)
    C = _np_bits(tx.dot(_dev(A, fmt, dev, pad_a), _dev(B, fmt, dev, pad_b), out_dtype=_TD[out_fmt]))
    _, r16 = oracle.gemm16_rows(A, B, 0, M, fmt, out_fmt=out_fmt)
    bad = np.argwhere(C != r16)
    assert bad.size == 0, (len(bad), bad[:5].tolist())


# K bytes 260 (partial chunk = chunk 0 of the last step), 500 (chunk 7),
# 400 (chunks past the row end, none partial), 2060 (chunk 0), 2200 (chunk 1)
@pytest.mark.parametrize("K", [130, 250, 200, 1030, 1100])
def test_ragged_persistent_exact(tx, oracle, dev, K):
    # 272 tiles: 16 workgroups walk two (the operand stream crosses tiles)
    _exact(tx, oracle, dev, 4352, 4096, K, seed=K)


@pytest.mark.parametrize("fmt,out_fmt", [(F16, F16), (F16, BF16), (BF16, F16)])
def test_ragged_persistent_formats(tx, oracle, dev, fmt, out_fmt):
    _exact(tx, oracle, dev, 4196, 4168, 266, fmt, out_fmt, seed=fmt + out_fmt)


def test_ragged_rows_whole_chunks(tx, oracle, dev):
    """K a whole number of steps but rows 4-byte aligned (pitch K + 2): the
    persistent tile and the 256 x 128 one read them in place."""
    _exact(tx, oracle, dev, 4352, 4096, 512, pad_a=2, pad_b=6, seed=5)
    _exact(tx, oracle, dev, 600, 1000, 512, pad_a=2, pad_b=2, seed=6)


@pytest.mark.parametrize("M,N,K", [(300, 500, 4100),   # 13 K splits, the last one ragged
                                   (600, 1000, 1030),
                                   (257, 501, 2050),
                                   (255, 257, 130)])   # two K steps
def test_ragged_narrow_tile_split_k(tx, oracle, dev, M, N, K):
    _exact(tx, oracle, dev, M, N, K, seed=M + K)


@pytest.mark.parametrize("M,N,K,fmt,out_fmt", [(4095, 4097, 4100, BF16, BF16),
                                               (4096, 4099, 1030, F16, F16),
                                               (4096, 4104, 520, BF16, F16),
                                               (4096, 4102, 263, F16, BF16)])  # 2-byte rows: padded copies
def test_column_strip_exact(tx, oracle, dev, M, N, K, fmt, out_fmt):
    """N 1 to 8 columns past a multiple of 256 (a 17th tile column would cost
    a second round): the columns past the last 256-column block take the
    16-bit strip kernel."""
    _exact(tx, oracle, dev, M, N, K, fmt, out_fmt, seed=N)


@pytest.mark.parametrize("N", [4096, 4099])
def test_ragged_strided_unaligned_out(tx, oracle, dev, N):
    """C a view 3 elements into a buffer with row pitch N + 1 (rows 2-byte
    aligned): every output lands in its row and the rest keeps its contents
    (N = 4099: the last 3 columns from the strip kernel)."""
    M, K = 4096 if N % 256 else 4352, 1100
    g = np.random.default_rng(9)
    A = _int_codes(g, (M, K), BF16)
    B = _int_codes(g, (N, K), BF16)
    flat = torch.full((M * (N + 1) + 8,), 0x7777, dtype=torch.int16, device=dev)
    out = flat[3:3 + M * (N + 1)].view(M, N + 1)[:, :N].view(torch.bfloat16)
    tx.dot(_dev(A, BF16, dev), _dev(B, BF16, dev), out=out)
    allb = flat.cpu().numpy().view(np.uint16)
    grid = allb[3:3 + M * (N + 1)].reshape(M, N + 1)
    assert np.all(allb[:3] == 0x7777) and np.all(allb[3 + M * (N + 1):] == 0x7777)
    assert np.all(grid[:, N] == 0x7777)
    _, r16 = oracle.gemm16_rows(A, B, 0, M, BF16)
    assert np.array_equal(grid[:, :N], r16)


def test_ragged_normal_values(tx, oracle, dev):
    """Normal-distributed operands at the ragged config shape's K, full
    output against the oracle's fp64 sums (the tolerances of the GEMM tests)."""
    import workloads
    M, N, K = 4352, 4104, 4100
    A, B = workloads.bf16_gemm_input(M, N, K, seed_stream=12)
    C = _np_bits(tx.dot(_dev(A, BF16, dev), _dev(B, BF16, dev)))
    r32, r16 = oracle.gemm16_rows(A, B, 0, M, BF16)
    check_close(C, r32, r16, BF16_TOL)


@pytest.mark.parametrize("M,N,K", [(4352, 4096, 1031),   # >= 2^30 multiply-adds: padded copies
                                   (600, 1000, 1031),    # below: the generic kernel
                                   (4096, 4100, 1031),   # with a column tail of 4
                                   (4096, 4132, 263)])   # a 36-column tail
def test_odd_k_even_pitch_exact(tx, oracle, dev, M, N, K):
    """An odd K read through [:, :K] views of rows K + 1 long: the row
    pitches are 4-byte multiples but the rows are not whole 4-byte words, so
    the fast path's in-place read (the last chunk fetched as the row's last
    16 bytes) does not apply; the products take the zero-padded copies or
    the generic kernel, bit-exact."""
    _exact(tx, oracle, dev, M, N, K, pad_a=1, pad_b=1, seed=K + N)


def test_tall_column_tail_ragged_k(tx, oracle, dev):
    """M = 65536 rows (a 256 x 256 tile per CU with one column block), N a
    20-column tail past 256 (N % 8 != 0) and a ragged K: the main 256 columns
    on the persistent tile, the tail on the 256 x 128 tile (decided before
    the main part is launched).  Sampled rows, bit-exact."""
    M, N, K = 65536, 276, 1030
    g = np.random.default_rng(65)
    A = _int_codes(g, (M, K), BF16)
    B = _int_codes(g, (N, K), BF16)
    C = _np_bits(tx.dot(_dev(A, BF16, dev), _dev(B, BF16, dev)))
    for r in sorted({0, 1, M - 1} | set(g.integers(0, M, 40).tolist())):
        _, r16 = oracle.gemm16_rows(A, B, r, r + 1, BF16)
        assert np.array_equal(C[r:r + 1], r16), r
