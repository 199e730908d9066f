"""GPU parity: tt.dot on 16-bit operands (bf16 / fp16, both B layouts, bf16 /
fp16 output) and the reference's matmul(a, b) caller, vs the oracle.

The reference's only AMD GEMM caller is matmul(a, b) with fp16 a (M x K) and
row-major fp16 b (K x N), fp16 output (test_amd_gemm_pipelined.py:303-331);
test_op runs it at 8192 x 8192 (:338-348) and the benchmark at square sizes
256 ... 4096 (:355-399).  Tolerance: rel err <= 1e-2 against the oracle's fp64
accumulation (max |gpu - ref| / max |ref| and the Frobenius ratio), plus an
ulp-distance bound to the oracle's own rounding of the output type.
"""
import numpy as np
import pytest
import torch

from test_gpu_gemm import block_rows, sample_rows

pytestmark = pytest.mark.gpu

TOL = 1e-2
BF16, F16 = 3, 6


def widen(bits, fmt):
    bits = np.asarray(bits, np.uint16)
    if fmt == F16:
        return bits.view(np.float16).astype(np.float64)
    return (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def check16(got_bits, ref32, ref_bits, fmt, tol=TOL):
    got = widen(got_bits, fmt)
    ref = ref32.astype(np.float64)
    scale = np.abs(ref).max() if ref.size else 0.0
    if scale == 0:
        assert np.all(got == 0)
        return
    rel_max = np.abs(got - ref).max() / scale
    rel_fro = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-300)
    assert rel_max <= tol and rel_fro <= tol, (rel_max, rel_fro)

    def ordinal(b):
        b = b.astype(np.int32)
        return np.where(b & 0x8000, -(b & 0x7FFF), b & 0x7FFF)
    # fp32 accumulation order moves a result across a rounding boundary of
    # the output type only rarely (fp16's grid is 8x finer than bf16's, so
    # the share of 1-ulp moves is larger); by more than 2 ulps only for
    # near-cancelling sums, hence the bound on outputs >= 1% of the scale
    d = np.abs(ordinal(got_bits) - ordinal(ref_bits))
    big = np.abs(ref) >= 1e-2 * scale
    assert np.mean(d > 0) <= 0.2 and np.mean(d[big] > 2) <= 0.002, \
        (np.mean(d > 0), np.mean(d[big] > 2), d.max())


def _t(bits, fmt, dev):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(dev).view(
        torch.float16 if fmt == F16 else torch.bfloat16)


def _bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def _inputs(M, N, K, fmt, seed):
    import workloads
    return workloads.matmul16_input(M, N, K, fp16=fmt == F16, seed_stream=seed)


CASES = [(1, 1, 1), (17, 33, 65), (96, 80, 64), (257, 130, 96), (300, 200, 1000),
         (513, 129, 72), (64, 4097, 520)]


@pytest.mark.parametrize("fmt", [F16, BF16])
@pytest.mark.parametrize("out_fmt", [F16, BF16])
@pytest.mark.parametrize("kn", [True, False])
@pytest.mark.parametrize("M,N,K", CASES)
def test_small_shapes_all_variants(tx, oracle, dev, fmt, out_fmt, kn, M, N, K):
    A, Bkn = _inputs(M, N, K, fmt, seed=M + 3 * N + 7 * K)
    a = _t(A, fmt, dev)
    odt = torch.float16 if out_fmt == F16 else torch.bfloat16
    if kn:
        C = tx.dot_kn(a, _t(Bkn, fmt, dev), out_dtype=odt)
    else:
        C = tx.dot(a, _t(Bkn.T, fmt, dev), out_dtype=odt)
    r32, r16 = oracle.gemm16_rows(A, Bkn, 0, M, fmt=fmt, b_kn=True, out_fmt=out_fmt)
    check16(_bits(C), r32, r16, out_fmt)


@pytest.mark.parametrize("kn", [True, False])
def test_strided_and_misaligned_operands(tx, oracle, dev, kn):
    """Row pitches wider than the rows and base addresses off 16 bytes: the
    padded A copy, the element-wise transpose and the generic kernels."""
    M, N, K = 130, 150, 260
    A, Bkn = _inputs(M, N, K, F16, seed=91)
    abig = torch.zeros((M, K + 9), dtype=torch.float16, device=dev)
    a = abig[:, 1:K + 1]
    a.copy_(_t(A, F16, dev))
    if kn:
        bbig = torch.zeros((K, N + 5), dtype=torch.float16, device=dev)
        b = bbig[:, 3:N + 3]
        b.copy_(_t(Bkn, F16, dev))
        C = tx.dot_kn(a, b)
    else:
        bbig = torch.zeros((N, K + 3), dtype=torch.float16, device=dev)
        b = bbig[:, 1:K + 1]
        b.copy_(_t(Bkn.T, F16, dev))
        C = tx.dot(a, b)
    r32, r16 = oracle.gemm16_rows(A, Bkn, 0, M, fmt=F16, b_kn=True)
    check16(_bits(C), r32, r16, F16)


def test_reference_test_op_8192(tx, oracle, dev):
    """test_op's problem: matmul(a, b) on fp16 8192 x 8192 (row-major b).  One
    sampled row per 128-row block and 24 more against the oracle; the whole
    output by exact doubling (matmul(2a, b) == 2 matmul(a, b) wherever the
    result is an fp16 normal) and against torch.matmul within the tolerance."""
    M = N = K = 8192
    A, Bkn = _inputs(M, N, K, F16, seed=0)
    a, b = _t(A, F16, dev), _t(Bkn, F16, dev)
    C = tx.matmul(a, b)
    assert C.dtype == torch.float16 and tuple(C.shape) == (M, N)
    rows = sorted(set(block_rows(M, seed=5)) | set(sample_rows(M, seed=5)))
    got = _bits(C)[rows]
    r32, r16 = oracle.gemm16_rows(A[rows], Bkn, 0, len(rows), fmt=F16, b_kn=True)
    check16(got, r32, r16, F16)
    C2 = tx.matmul(a * 2, b)
    normal = C.abs() >= 2.0 ** -13
    assert torch.equal((C * 2)[normal], C2[normal])
    T = torch.matmul(a, b).float()
    rel = (C.float() - T).norm() / T.norm()
    assert rel.item() <= TOL, rel.item()


@pytest.mark.parametrize("fmt,out_fmt", [(F16, F16), (F16, BF16), (BF16, BF16), (BF16, F16)])
@pytest.mark.parametrize("shape", [(4100, 4104, 192),    # 256 x 256 tiles
                                   (2100, 2056, 256),    # 128 x 128 tiles
                                   (4096, 2048, 128),    # 128 x 128, two tiles per workgroup
                                   (1030, 1032, 192),    # 64 x 64 tiles
                                   (2048, 1024, 128),    # 64 x 64, two tiles per workgroup
                                   (512, 512, 512)])     # 64 x 64, fewer tiles than CUs
def test_row_major_b_read_in_tile(tx, oracle, dev, fmt, out_fmt, shape):
    """Products the persistent tile takes (at least one 256 x 256 tile per CU,
    or else one 128 x 128 or 64 x 64 tile per CU; K a whole number of 64-element steps,
    N a multiple of 8) read the row-major b in place through transposing LDS
    reads.  Partial last row and column tiles; every output element against
    the oracle, then tile by tile so that a misplaced block cannot hide
    behind the others."""
    M, N, K = shape
    A, Bkn = _inputs(M, N, K, fmt, seed=M + N + K + fmt)
    odt = torch.float16 if out_fmt == F16 else torch.bfloat16
    C = tx.dot_kn(_t(A, fmt, dev), _t(Bkn, fmt, dev), out_dtype=odt)
    r32, r16 = oracle.gemm16_rows(A, Bkn, 0, M, fmt=fmt, b_kn=True, out_fmt=out_fmt)
    got = _bits(C)
    check16(got, r32, r16, out_fmt)
    tb = 64 if M * N <= 1 << 22 else 128
    for m0 in range(0, M, tb):
        for n0 in range(0, N, tb):
            t = (slice(m0, m0 + tb), slice(n0, n0 + tb))
            check16(got[t], r32[t], r16[t], out_fmt)


def test_row_major_b_read_in_tile_strided(tx, oracle, dev):
    """b a view of wider K rows (pitch N + 72) whose padding holds NaN codes:
    the last column tile reads the padding into columns past N, whose
    products are dropped; no NaN may reach a stored column."""
    M, N, K = 4096, 4032, 256
    A, Bkn = _inputs(M, N, K, F16, seed=77)
    bbig = torch.full((K, N + 72), float("nan"), dtype=torch.float16, device=dev)
    b = bbig[:, :N]
    b.copy_(_t(Bkn, F16, dev))
    C = tx.dot_kn(_t(A, F16, dev), b)
    assert not torch.isnan(C).any()
    r32, r16 = oracle.gemm16_rows(A, Bkn, 0, M, fmt=F16, b_kn=True)
    check16(_bits(C), r32, r16, F16)


@pytest.mark.parametrize("M,N,K", [(4096, 4096, 128), (2048, 2048, 256), (1024, 1032, 192)])
def test_row_major_b_in_tile_all_strided(tx, oracle, dev, M, N, K):
    """The in-place row-major-b tiles (256, 128 and 64 square) on views: A
    rows of K + 64 elements, b K rows of N + 72 with NaN codes in the
    padding, and the output a view of rows N + 40 wide whose padding must
    keep its contents."""
    A, Bkn = _inputs(M, N, K, F16, seed=M + K)
    abig = torch.zeros((M, K + 64), dtype=torch.float16, device=dev)
    a = abig[:, :K]
    a.copy_(_t(A, F16, dev))
    bbig = torch.full((K, N + 72), float("nan"), dtype=torch.float16, device=dev)
    b = bbig[:, :N]
    b.copy_(_t(Bkn, F16, dev))
    cbig = torch.full((M, N + 40), 0x7777, dtype=torch.int16, device=dev)
    out = cbig.view(torch.float16)[:, :N]
    tx.dot_kn(a, b, out=out)
    allb = cbig.cpu().numpy().view(np.uint16)
    assert np.all(allb[:, N:] == 0x7777)
    r32, r16 = oracle.gemm16_rows(A, Bkn, 0, M, fmt=F16, b_kn=True)
    check16(allb[:, :N], r32, r16, F16)


@pytest.mark.parametrize("kn", [True, False])
@pytest.mark.parametrize("fmt", [F16, BF16])
@pytest.mark.parametrize("M,N,K", [(1, 8, 128), (3, 24, 192), (65, 72, 128), (17, 136, 256),
                                   (200, 8, 2048), (130, 264, 640)])
def test_tiny_products_on_the_persistent_tile(tx, oracle, dev, kn, fmt, M, N, K):
    """Products far below one tile per CU that still meet the persistent
    tile's conditions (K a whole number of 64-element steps, at least two and
    at most 32 128-byte steps; N a multiple of 8; rows 16-byte aligned) run on
    the 64 x 64 tile, with a row-major b read in place: from one partial tile
    (M = 1, N = 8) to a few, every row, column and K position past the
    product outside the buffer ranges (zeros in, stores dropped)."""
    A, Bkn = _inputs(M, N, K, fmt, seed=5 * M + N + K)
    a = _t(A, fmt, dev)
    C = tx.dot_kn(a, _t(Bkn, fmt, dev)) if kn else tx.dot(a, _t(Bkn.T, fmt, dev))
    r32, r16 = oracle.gemm16_rows(A, Bkn, 0, M, fmt=fmt, b_kn=True)
    check16(_bits(C), r32, r16, fmt)


@pytest.mark.parametrize("kn", [False, True])
@pytest.mark.parametrize("fmt", [F16, BF16])
@pytest.mark.parametrize("M,N,K", [(4096, 4096, 128),   # 256 x 256 persistent tile
                                   (2048, 2048, 128),   # 128 x 128
                                   (1024, 1024, 128),   # 64 x 64, one tile per CU
                                   (512, 512, 128)])    # 64 x 64, fewer tiles than CUs
def test_persistent_tiles_round_exactly_and_keep_nonfinite(tx, oracle, dev, kn, fmt, M, N, K):
    """One nonzero per row of A, so every output is a single 16-bit product,
    exact in fp32: each persistent tile size, with b as N x K and read in place
    as row-major K x N, must round it as the oracle does, bit for bit, on every
    output.  Row 0 of A holds +Inf and row 1 a NaN; column 5 of b is zero, so
    row 0 is Inf with b's sign except NaN (Inf x 0) in column 5, and row 1 is
    NaN throughout."""
    g = np.random.default_rng(M + 7 * fmt + int(kn))
    codes = (lambda x: x.astype(np.float16).view(np.uint16)) if fmt == F16 else (
        lambda x: __import__("workloads").to_bf16_bits(x))
    a = np.zeros((M, K), np.float32)
    a[np.arange(M), np.arange(M) % K] = g.uniform(0.5, 2.0, M) * g.choice([-1.0, 1.0], M)
    b = (g.uniform(0.5, 2.0, (K, N)) * g.choice([-1.0, 1.0], (K, N))).astype(np.float32)
    b[:, 5] = 0.0
    A, Bkn = codes(a), codes(b)
    A[0, 0] = 0x7C00 if fmt == F16 else 0x7F80
    A[1, 1] = 0x7E00 if fmt == F16 else 0x7FC0
    at, bt = _t(A, fmt, dev), _t(Bkn, fmt, dev)
    C = _bits(tx.dot_kn(at, bt) if kn else tx.dot(at, bt.t().contiguous()))
    Cf = widen(C, fmt)
    cols = np.arange(N) != 5
    assert np.all(np.isinf(Cf[0, cols])) and np.array_equal(np.signbit(Cf[0, cols]), np.signbit(b[0, cols]))
    assert np.isnan(Cf[0, 5]) and np.all(np.isnan(Cf[1]))
    _, r16 = oracle.gemm16_rows(A, Bkn, 2, M, fmt=fmt, b_kn=True)
    got = C[2:]
    nz = widen(r16, fmt) != 0
    assert np.array_equal(got[nz], r16[nz]), np.argwhere(got != r16)[:5]
    assert np.all(widen(got[~nz], fmt) == 0)


@pytest.mark.parametrize("S", [256, 512, 1024, 2048, 4096])
def test_reference_benchmark_shapes(tx, oracle, dev, S):
    A, Bkn = _inputs(S, S, S, F16, seed=S)
    C = tx.matmul(_t(A, F16, dev), _t(Bkn, F16, dev))
    rows = sorted(set(block_rows(S, seed=S)) | set(sample_rows(S, seed=S)))
    got = _bits(C)[rows]
    r32, r16 = oracle.gemm16_rows(A[rows], Bkn, 0, len(rows), fmt=F16, b_kn=True)
    check16(got, r32, r16, F16)


def test_matmul_b_layouts_agree(tx, dev):
    """matmul takes b row-major (the reference's), column-major (a transposed
    view) or any strides, with the same result."""
    M, N, K = 200, 190, 320
    A, Bkn = _inputs(M, N, K, F16, seed=4)
    a, b = _t(A, F16, dev), _t(Bkn, F16, dev)
    C1 = tx.matmul(a, b)
    C2 = tx.matmul(a, b.t().contiguous().t())
    C3 = tx.matmul(a, torch.empty((K, 2 * N), dtype=torch.float16, device=dev)[:, ::2].copy_(b))
    assert torch.equal(C1, C2) and torch.equal(C1, C3)
    with pytest.raises(AssertionError, match="Incompatible dimensions"):
        tx.matmul(a, b[:K - 1])
    with pytest.raises(AssertionError, match="contiguous"):
        tx.matmul(torch.empty((K, M), dtype=torch.float16, device=dev).t(), b)


def test_k_zero_and_table_forms(tx, oracle, dev):
    z = tx.dot_kn(torch.ones((5, 0), dtype=torch.float16, device=dev),
                  torch.ones((0, 7), dtype=torch.float16, device=dev))
    assert tuple(z.shape) == (5, 7) and torch.all(z == 0)
    M, N, K = 96, 80, 128
    A, Bkn = _inputs(M, N, K, F16, seed=12)
    a, b = _t(A, F16, dev), _t(Bkn, F16, dev)
    C1 = tx.dot_kn(a, b, out_dtype=torch.bfloat16)
    C2 = torch.empty_like(C1)
    tx.invoke("tt.dot", [C2, a, b, M, N, K, K, N, N, F16, BF16, 1])
    assert torch.equal(C1, C2)
    with pytest.raises(tx.TxError, match="INVALID_ARGUMENT"):
        tx.invoke("tt.dot", [C2, a, b, M, N, K, K, N, N, 0, BF16, 1])  # fp32 operands
    with pytest.raises(tx.TxError, match="INVALID_ARGUMENT"):
        tx.invoke("tt.dot", [C2, a, b, M, N, K, K, N - 1, N, F16, BF16, 1])  # ldb < N
    with pytest.raises(ValueError):
        tx.dot_kn(a, b.to(torch.bfloat16))
