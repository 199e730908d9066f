"""GPU parity: tt.dot bf16, fp8 scaled dot and the fp8 dequant GEMV vs the oracle.

Tolerances (stated per op): bf16 GEMM rel err <= 1e-2, fp8 scaled GEMM and
GEMV rel err <= 2e-2, each measured as max|gpu - ref| / max|ref| and as the
Frobenius ratio ||gpu - ref|| / ||ref||, against the oracle's fp64
accumulation.  On top of that, outputs must be within 1 bf16 ulp of the
oracle's own bf16 rounding for all but a tiny fraction of elements, which a
wrong index, dropped term or transposed operand would break at any size.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

BF16_TOL = 1e-2
FP8_TOL = 2e-2


def bf16_f32(h):
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def _t_bf16(bits_np, dev):
    return torch.from_numpy(bits_np.view(np.int16)).to(dev).view(torch.bfloat16)


def _np_bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def check_close(got_bits, ref32, ref_bits, tol):
    got = bf16_f32(got_bits).astype(np.float64)
    ref = ref32.astype(np.float64)
    scale = np.abs(ref).max() if ref.size else 0.0
    if scale == 0:
        assert np.all(got == 0)
        return
    rel_max = np.abs(got - ref).max() / scale
    rel_fro = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-300)
    assert rel_max <= tol and rel_fro <= tol, (rel_max, rel_fro)
    # ulp distance to the oracle's bf16 rounding (sign-magnitude -> ordinal)
    def ordinal(b):
        b = b.astype(np.int32)
        return np.where(b & 0x8000, -(b & 0x7FFF), b & 0x7FFF)
    # fp32 accumulation order only moves results across a bf16 rounding
    # boundary rarely, and by more than 2 ulps only for near-cancelling sums:
    # the 2-ulp bound is checked on outputs at least 1% of the output scale
    d = np.abs(ordinal(got_bits) - ordinal(ref_bits))
    big = np.abs(ref) >= 1e-2 * scale
    assert np.mean(d > 0) <= 0.05 and np.mean(d[big] > 2) <= 0.002, \
        (np.mean(d > 0), np.mean(d[big] > 2), d.max())


def sample_rows(M, k=24, seed=0):
    g = np.random.default_rng(seed)
    rows = set([0, 1, M - 1, M - 2] + list(g.integers(0, M, size=k)))
    return sorted(r for r in rows if 0 <= r < M)


def block_rows(M, seed=0):
    """One random row in every 128-row block (so in each half of every
    256-row tile, i.e. in every wavefront's share of it), plus the first and
    last rows: a misplaced, duplicated or skipped tile or wave block shows up
    in at least one of them."""
    g = np.random.default_rng(seed)
    rows = {0, M - 1}
    for b0 in range(0, M, 128):
        rows.add(int(g.integers(b0, min(b0 + 128, M))))
    return sorted(rows)


# --------------------------------------------------------------------- bf16
@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (17, 19, 23), (64, 64, 64), (128, 128, 128),
                                   (255, 257, 130), (300, 64, 1000), (513, 129, 72),
                                   (1024, 1024, 256), (33, 4097, 520)])
def test_bf16_small_shapes(tx, oracle, dev, M, N, K):
    import workloads
    A, B = workloads.bf16_gemm_input(M, N, K, seed_stream=M * 7 + N)
    C = tx.dot(_t_bf16(A, dev), _t_bf16(B, dev))
    r32, r16 = oracle.gemm_bf16_rows(A, B, 0, M)
    check_close(_np_bits(C), r32, r16, BF16_TOL)


@pytest.mark.parametrize("M,N,K", [(600, 1000, 256), (300, 500, 4096), (257, 501, 2048)])
def test_bf16_narrow_tile_and_split_k(tx, oracle, dev, M, N, K):
    """Fewer 256x256 tiles than CUs: 256x128 tiles, and K split into fp32
    partial planes (8 and 4 splits here, N not a multiple of 4 in the last)."""
    import workloads
    A, B = workloads.bf16_gemm_input(M, N, K, seed_stream=M + N)
    C = tx.dot(_t_bf16(A, dev), _t_bf16(B, dev))
    r32, r16 = oracle.gemm_bf16_rows(A, B, 0, M)
    check_close(_np_bits(C), r32, r16, BF16_TOL)


@pytest.mark.parametrize("K", [1003, 1001, 1002, 1004])
def test_bf16_padded_fast_path(tx, oracle, dev, K):
    """Rows not 16-byte aligned in a product of >= 2^30 multiply-adds.  Row
    lengths of 2006 and 2002 bytes (2-byte aligned rows): the operands are
    copied into zero-padded rows and take the fast path (source loads of 2
    bytes); 2004 and 2008 bytes (4-byte aligned): the fast path reads them
    in place, the last chunk of each row fetched as its last 16 bytes."""
    import workloads
    M, N = 1100, 1040
    A, B = workloads.bf16_gemm_input(M, N, K, seed_stream=77)
    C = _np_bits(tx.dot(_t_bf16(A, dev), _t_bf16(B, dev)))
    for r in sample_rows(M, k=40):
        r32, r16 = oracle.gemm_bf16_rows(A, B, r, r + 1)
        check_close(C[r:r + 1], r32, r16, BF16_TOL)


@pytest.mark.parametrize("M,N,K", [(4096, 4096, 4096), (4095, 4097, 4100)])
def test_bf16_config_shapes(tx, oracle, dev, M, N, K):
    import workloads
    A, B = workloads.bf16_gemm_input(M, N, K)
    C = _np_bits(tx.dot(_t_bf16(A, dev), _t_bf16(B, dev)))
    rows = sorted(set(block_rows(M, seed=M)) | set(sample_rows(M)))
    for r in rows:
        r32, r16 = oracle.gemm_bf16_rows(A, B, r, r + 1)
        check_close(C[r:r + 1], r32, r16, BF16_TOL)
    # full-size property: scaling A by 2 (exact in bf16) doubles every output bit-exactly
    A2 = _t_bf16(A, dev) * 2
    C2 = _np_bits(tx.dot(A2, _t_bf16(B, dev)))
    assert np.array_equal(bf16_f32(C2), 2 * bf16_f32(C))


@pytest.mark.parametrize("M,N,K", [(4096, 4096, 64), (512, 384, 64), (600, 1000, 8), (300, 500, 4096),
                                   (100, 200, 7)])
def test_bf16_output_rounding_exact(tx, oracle, dev, M, N, K):
    """One nonzero per row of A, so every output is a single bf16 x bf16
    product, exact in fp32: the kernel's rounding to bf16 must equal the
    oracle's round-to-nearest-even bit for bit (about one product in 256 is a
    tie).  Row 0 of A holds +Inf, row 1 a NaN: Inf * b keeps b's sign, Inf * 0
    and NaN * b are NaN.  Shapes cover the 256x256 and 256x128 tiles, split K
    and the generic kernel."""
    import workloads
    g = np.random.default_rng(M + K)
    a = np.zeros((M, K), np.float32)
    a[np.arange(M), np.arange(M) % K] = g.uniform(0.5, 2.0, M) * g.choice([-1.0, 1.0], M)
    b = (g.uniform(0.5, 2.0, (N, K)) * g.choice([-1.0, 1.0], (N, K))).astype(np.float32)
    b[5, :] = 0.0
    A, B = workloads.to_bf16_bits(a), workloads.to_bf16_bits(b)
    A[0, 0] = 0x7F80
    A[1, 1] = 0x7FC0
    C = _np_bits(tx.dot(_t_bf16(A, dev), _t_bf16(B, dev)))
    Cf = bf16_f32(C)
    bsign = np.signbit(bf16_f32(B[:, 0]))
    inf_cols = np.arange(N) != 5
    assert np.all(np.isinf(Cf[0, inf_cols])) and np.array_equal(np.signbit(Cf[0, inf_cols]), bsign[inf_cols])
    assert np.isnan(Cf[0, 5]) and np.all(np.isnan(Cf[1]))
    rows = [r for r in sample_rows(M, k=40) if r >= 2]
    for r in rows:
        _, r16 = oracle.gemm_bf16_rows(A, B, r, r + 1)
        got, want = C[r], r16[0]
        nz = bf16_f32(want) != 0
        assert np.array_equal(got[nz], want[nz]), (r, np.flatnonzero(got[nz] != want[nz])[:5])
        assert np.all(bf16_f32(got[~nz]) == 0)


def test_scratch_reuse_across_streams(tx, oracle, dev):
    """Split-K partial planes and padded operand copies live in scratch the
    library keeps per stream: shapes that grow and shrink it, interleaved on
    two streams with no synchronisation between the calls, all come out
    right."""
    import workloads
    shapes = [(300, 500, 4096), (1100, 1040, 1003), (257, 501, 2048), (600, 1000, 2050),
              (130, 260, 8192), (1024, 1100, 1001)]
    inputs = [workloads.bf16_gemm_input(M, N, K, seed_stream=40 + i) for i, (M, N, K) in enumerate(shapes)]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    dev_in = [(_t_bf16(A, dev), _t_bf16(B, dev)) for A, B in inputs]
    outs = [torch.empty((M, N), dtype=torch.bfloat16, device=dev) for (M, N, K) in shapes]
    torch.cuda.synchronize()
    for rep in range(2):
        for i in range(len(shapes)):
            with torch.cuda.stream(streams[(i + rep) % 2]):
                tx.dot(dev_in[i][0], dev_in[i][1], out=outs[i])
    torch.cuda.synchronize()
    for (M, N, K), (A, B), C in zip(shapes, inputs, outs):
        Cb = _np_bits(C)
        for r in sample_rows(M, k=6):
            r32, r16 = oracle.gemm_bf16_rows(A, B, r, r + 1)
            check_close(Cb[r:r + 1], r32, r16, BF16_TOL)


def test_bf16_strided_and_unaligned(tx, oracle, dev):
    import workloads
    M, N, K = 200, 150, 333
    A, B = workloads.bf16_gemm_input(M, N, K, seed_stream=99)
    # odd row strides force the narrow-load kernel variants
    Ap = np.zeros((M, K + 3), np.uint16); Ap[:, :K] = A
    Bp = np.zeros((N, K + 5), np.uint16); Bp[:, :K] = B
    At = _t_bf16(Ap, dev)[:, :K]
    Bt = _t_bf16(Bp, dev)[:, :K]
    out = torch.zeros((M, N + 7), dtype=torch.bfloat16, device=dev)[:, :N]
    tx.dot(At, Bt, out=out)
    r32, r16 = oracle.gemm_bf16_rows(A, B, 0, M)
    check_close(_np_bits(out), r32, r16, BF16_TOL)


def test_bf16_degenerate(tx, dev):
    a = torch.ones((5, 0), dtype=torch.bfloat16, device=dev)
    b = torch.ones((3, 0), dtype=torch.bfloat16, device=dev)
    c = tx.dot(a, b)
    assert torch.all(c == 0)
    e = tx.dot(torch.ones((0, 4), dtype=torch.bfloat16, device=dev),
               torch.ones((3, 4), dtype=torch.bfloat16, device=dev))
    assert e.shape == (0, 3)


def test_bf16_matmul_wrapper_and_table(tx, oracle, dev):
    import workloads
    M, N, K = 96, 80, 64
    A, B = workloads.bf16_gemm_input(M, N, K, seed_stream=5)
    b_kn = _t_bf16(B, dev).t()  # column-major K x N view
    C1 = tx.dot(_t_bf16(A, dev), _t_bf16(B, dev))
    C2 = torch.empty_like(C1)
    tx.invoke("tt.dot", [C2, _t_bf16(A, dev), _t_bf16(B, dev), M, N, K, K, K, N])
    r32, r16 = oracle.gemm_bf16_rows(A, B, 0, M)
    check_close(_np_bits(C1), r32, r16, BF16_TOL)
    assert torch.equal(C1, C2)
    # matmul's output is fp16, as the reference's (c = torch.empty(..., float16))
    C3 = tx.matmul(_t_bf16(A, dev), b_kn)
    assert C3.dtype == torch.float16
    C4 = tx.dot(_t_bf16(A, dev), _t_bf16(B, dev), out_dtype=torch.float16)
    assert torch.equal(C3, C4)
    ref16 = oracle.encode_fmt(r32, oracle.F16).reshape(r32.shape)
    got = C3.view(torch.int16).cpu().numpy().view(np.uint16)
    d = np.abs(got.view(np.float16).astype(np.float64) - ref16.view(np.float16).astype(np.float64))
    assert d.max() <= BF16_TOL * np.abs(r32).max()


# ---------------------------------------------------------------------- fp8
def _fp8_run(tx, dev, aq, sa, bq, sb, fa=torch.float8_e4m3fn, fb=torch.float8_e4m3fn):
    A = torch.from_numpy(aq).to(dev).view(fa)
    B = torch.from_numpy(bq).to(dev).view(fb)
    return _np_bits(tx.dot_scaled_rowcol(A, torch.from_numpy(sa).to(dev), B,
                                         torch.from_numpy(sb).to(dev)))


@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (16, 48, 128), (100, 200, 300), (256, 256, 512),
                                   (16, 1000, 4096), (600, 300, 260)])
def test_fp8_small_shapes(tx, oracle, dev, M, N, K):
    import workloads
    aq, sa, bq, sb = workloads.fp8_gemm_input(M, N, K, seed_stream=M + 3 * N)
    C = _fp8_run(tx, dev, aq, sa, bq, sb)
    r32, r16 = oracle.gemm_fp8_scaled_rows(aq, bq, sa, sb, 0, M)
    check_close(C, r32, r16, FP8_TOL)


@pytest.mark.parametrize("fa,fb", [(2, 2), (1, 2), (2, 1)])
def test_fp8_format_mixes(tx, oracle, dev, fa, fb):
    g = np.random.default_rng(fa * 10 + fb)
    M, N, K = 130, 190, 384
    aq = g.integers(0, 256, size=(M, K), dtype=np.uint8)
    bq = g.integers(0, 256, size=(N, K), dtype=np.uint8)
    # keep codes finite: clear NaN / Inf encodings
    for q, f in ((aq, fa), (bq, fb)):
        mag = q & 0x7F
        if f == 1:
            q[mag == 0x7F] &= 0xFE
        else:
            q[mag >= 0x7C] = 0x3C
    sa = g.uniform(0.5, 2, M).astype(np.float32) * 1e-3
    sb = g.uniform(0.5, 2, N).astype(np.float32) * 1e-3
    td = {1: torch.float8_e4m3fn, 2: torch.float8_e5m2}
    C = _fp8_run(tx, dev, aq, sa, bq, sb, td[fa], td[fb])
    r32, r16 = oracle.gemm_fp8_scaled_rows(aq, bq, sa, sb, 0, M, fa, fb)
    check_close(C, r32, r16, FP8_TOL)


@pytest.mark.parametrize("M,N,K,fa,fb", [(300, 500, 8192, 1, 1), (130, 777, 2048, 2, 1)])
def test_fp8_narrow_tile_and_split_k(tx, oracle, dev, M, N, K, fa, fb):
    """256x128 tiles with K split into fp32 partial planes; the scales are
    applied by the reduction."""
    import workloads
    aq, sa, bq, sb = workloads.fp8_gemm_input(M, N, K, seed_stream=M * 3 + N)
    td = {1: torch.float8_e4m3fn, 2: torch.float8_e5m2}
    if fa == 2:  # reinterpret the e4m3 codes as e5m2: finite, wider range
        aq = np.where((aq & 0x7F) >= 0x7C, aq & 0x80, aq).astype(np.uint8)
    C = _fp8_run(tx, dev, aq, sa, bq, sb, td[fa], td[fb])
    r32, r16 = oracle.gemm_fp8_scaled_rows(aq, bq, sa, sb, 0, M, fa, fb)
    check_close(C, r32, r16, FP8_TOL)


def test_column_tail_strip(tx, oracle, dev):
    """N just past a multiple of 256 where the last tile column would cost a
    whole round: the full columns take 256x256 tiles, the tail a second
    product (fp8: split-K 256x128 tiles; 16-bit, at most 8 columns: the VALU
    strip kernel)."""
    import workloads
    M, N, K = 4096, 4112, 1024
    aq, sa, bq, sb = workloads.fp8_gemm_input(M, N, K, seed_stream=21)
    C = _fp8_run(tx, dev, aq, sa, bq, sb)
    for r in sample_rows(M, k=12):
        r32, r16 = oracle.gemm_fp8_scaled_rows(aq, bq, sa, sb, r, r + 1)
        check_close(C[r:r + 1], r32, r16, FP8_TOL)
    M, N, K = 4096, 4100, 512
    A, B = workloads.bf16_gemm_input(M, N, K, seed_stream=22)
    Cb = _np_bits(tx.dot(_t_bf16(A, dev), _t_bf16(B, dev)))
    for r in sample_rows(M, k=12):
        r32, r16 = oracle.gemm_bf16_rows(A, B, r, r + 1)
        check_close(Cb[r:r + 1], r32, r16, BF16_TOL)


def test_tall_narrow_fast_path(tx, oracle, dev):
    """N below one 256-column block with enough row tiles to fill every CU:
    no column strip is split off (it would leave nothing for the main tiles)."""
    import workloads
    # rows are few columns wide: check the sampled rows as one set
    M, N, K = 65536 + 40, 40, 256
    A, B = workloads.bf16_gemm_input(M, N, K, seed_stream=23)
    Cb = _np_bits(tx.dot(_t_bf16(A, dev), _t_bf16(B, dev)))
    rows = sample_rows(M, k=32)
    refs = [oracle.gemm_bf16_rows(A, B, r, r + 1) for r in rows]
    check_close(Cb[rows], np.concatenate([x[0] for x in refs]), np.concatenate([x[1] for x in refs]),
                BF16_TOL)
    M, N, K = 65536 + 8, 16, 128
    aq, sa, bq, sb = workloads.fp8_gemm_input(M, N, K, seed_stream=24)
    C = _fp8_run(tx, dev, aq, sa, bq, sb)
    rows = sample_rows(M, k=32)
    refs = [oracle.gemm_fp8_scaled_rows(aq, bq, sa, sb, r, r + 1) for r in rows]
    check_close(C[rows], np.concatenate([x[0] for x in refs]), np.concatenate([x[1] for x in refs]),
                FP8_TOL)


def test_fp8_padded_fast_path(tx, oracle, dev):
    """Odd K (rows not 16-byte aligned) in a product of >= 2^30 multiply-adds:
    zero-padded copies of the operands take the fast path."""
    import workloads
    M, N, K = 1000, 1100, 1001
    aq, sa, bq, sb = workloads.fp8_gemm_input(M, N, K, seed_stream=13)
    C = _fp8_run(tx, dev, aq, sa, bq, sb)
    for r in sample_rows(M, k=40):
        r32, r16 = oracle.gemm_fp8_scaled_rows(aq, bq, sa, sb, r, r + 1)
        check_close(C[r:r + 1], r32, r16, FP8_TOL)


@pytest.mark.parametrize("M,N,K,fa,fb", [(1, 17, 128, 1, 1), (5, 33, 256, 2, 2), (16, 16, 1024, 1, 2),
                                         (17, 100, 384, 2, 1), (33, 250, 128, 1, 1),
                                         (64, 130, 2048, 1, 1), (40, 3000, 640, 2, 2),
                                         (8, 8200, 4608, 1, 1), (20, 300, 8192, 2, 1)])
def test_fp8_skinny_shapes(tx, oracle, dev, M, N, K, fa, fb):
    """M <= 64 and K % 128 == 0 take the skinny kernel (B streamed once):
    one or two LDS stages per wave, 8 or 16 wavefronts, 1, 2 or 4 blocks of M."""
    g = np.random.default_rng(M * 1000 + N)
    aq = g.integers(0, 256, size=(M, K), dtype=np.uint8)
    bq = g.integers(0, 256, size=(N, K), dtype=np.uint8)
    for q, f in ((aq, fa), (bq, fb)):
        mag = q & 0x7F
        if f == 1:
            q[mag == 0x7F] &= 0xFE
        else:
            q[mag >= 0x7C] = 0x3C
    sa = g.uniform(0.5, 2, M).astype(np.float32) * 1e-3
    sb = g.uniform(0.5, 2, N).astype(np.float32) * 1e-3
    td = {1: torch.float8_e4m3fn, 2: torch.float8_e5m2}
    C = _fp8_run(tx, dev, aq, sa, bq, sb, td[fa], td[fb])
    r32, r16 = oracle.gemm_fp8_scaled_rows(aq, bq, sa, sb, 0, M, fa, fb)
    check_close(C, r32, r16, FP8_TOL)


@pytest.mark.parametrize("M,N,K", [(16, 8200, 1024), (5, 100, 640), (33, 300, 384), (40, 3000, 256)])
def test_fp8_skinny_strided(tx, oracle, dev, M, N, K):
    """The skinny kernel's buffer ranges follow the row pitch: A and B as
    K-column views of wider rows (lda = K + 128, ldb = K + 256), with ragged
    last 16-row blocks of M and N; the bytes past K in each row are NaN codes
    that must never be read."""
    g = np.random.default_rng(M * 7 + N)
    aq = g.integers(0, 256, size=(M, K), dtype=np.uint8)
    bq = g.integers(0, 256, size=(N, K), dtype=np.uint8)
    for q in (aq, bq):
        q[(q & 0x7F) == 0x7F] &= 0xFE
    a_wide = np.full((M, K + 128), 0x7F, dtype=np.uint8)
    b_wide = np.full((N, K + 256), 0x7F, dtype=np.uint8)
    a_wide[:, :K] = aq
    b_wide[:, :K] = bq
    sa = g.uniform(0.5, 2, M).astype(np.float32) * 1e-3
    sb = g.uniform(0.5, 2, N).astype(np.float32) * 1e-3
    A = torch.from_numpy(a_wide).to(dev).view(torch.float8_e4m3fn)[:, :K]
    B = torch.from_numpy(b_wide).to(dev).view(torch.float8_e4m3fn)[:, :K]
    C = _np_bits(tx.dot_scaled_rowcol(A, torch.from_numpy(sa).to(dev), B, torch.from_numpy(sb).to(dev)))
    r32, r16 = oracle.gemm_fp8_scaled_rows(aq, bq, sa, sb, 0, M)
    check_close(C, r32, r16, FP8_TOL)


@pytest.mark.parametrize("M,N,K", [(16, 14336, 4096), (512, 14336, 4096), (8192, 14336, 4096),
                                   (16, 4096, 14336), (512, 4096, 14336), (8192, 4096, 14336),
                                   (8192, 8192, 8192)])
def test_fp8_config_shapes(tx, oracle, dev, M, N, K):
    """Every fp8 config shape: the oracle checks one row in every 128-row
    block of C (each half of every 256-row tile) plus random rows, each row
    over all N columns (every column tile); then full-size scale linearity."""
    import workloads
    aq, sa, bq, sb = workloads.fp8_gemm_input(M, N, K)
    C = _fp8_run(tx, dev, aq, sa, bq, sb)
    rows = sorted(set(block_rows(M, seed=M + N)) | set(sample_rows(M, k=8)))
    r32 = np.empty((len(rows), N), np.float32)
    r16 = np.empty((len(rows), N), np.uint16)
    for i, r in enumerate(rows):
        a32, a16 = oracle.gemm_fp8_scaled_rows(aq, bq, sa, sb, r, r + 1)
        r32[i], r16[i] = a32[0], a16[0]
    check_close(C[rows], r32, r16, FP8_TOL)
    for i, r in enumerate(rows):  # and row by row: no row may hide behind the others
        check_close(C[r:r + 1], r32[i:i + 1], r16[i:i + 1], FP8_TOL)
    # full-size property: scale linearity, C(2 * sa) == 2 * C bit-exactly
    C2 = _fp8_run(tx, dev, aq, (2 * sa).astype(np.float32), bq, sb)
    assert np.array_equal(bf16_f32(C2), 2 * bf16_f32(C))


# --------------------------------------------------------------------- gemv
@pytest.mark.parametrize("M", [1, 4, 16])
def test_gemv_config_full(tx, oracle, dev, M):
    import workloads
    x, wq, s = workloads.gemv_input(M)
    y = tx.gemv_fp8_dequant(_t_bf16(x, dev), torch.from_numpy(wq).to(dev).view(torch.float8_e5m2),
                            torch.from_numpy(s).to(dev))
    r32, r16 = oracle.gemv_fp8_dequant(x, wq, s)
    check_close(_np_bits(y), r32, r16, FP8_TOL)


@pytest.mark.parametrize("M,N,K,group,fmt", [(8, 8200, 384, 128, 2), (20, 8200, 512, 128, 2),
                                             (40, 8208, 256, 256, 1),
                                             (3, 100, 256, 128, 2), (33, 77, 1024, 256, 2),
                                             (64, 50, 384, 384, 1), (5, 1, 128, 128, 1),
                                             (1, 8200, 384, 128, 2), (2, 8208, 256, 256, 1),
                                             (1, 100, 1152, 384, 1), (2, 77, 3072, 128, 2),
                                             (1, 1, 128, 128, 2), (2, 3, 5120, 640, 1), (1, 3, 5120, 640, 1),
                                             (1, 14336, 4096, 128, 1),
                                             (3, 8200, 1152, 384, 2), (4, 100, 5120, 640, 1)])
def test_gemv_shapes(tx, oracle, dev, M, N, K, group, fmt):
    """Small and ragged shapes; N >= 8192 takes the wide variants (two W
    blocks per wave when M > 4, with an odd number of 16-row blocks); M = 1
    the streaming kernel (1 KiB slices: K not a multiple of 1024, odd N,
    groups of 384), M = 2, 3 and 4 beside it on the MFMA kernel (a streaming
    kernel for M = 4 ran 22.5 against 16.5 us at 14336 x 4096)."""
    g = np.random.default_rng(M * N)
    x = oracle.f32_to_bf16(g.standard_normal((M, K)).astype(np.float32))
    wq = g.integers(0, 256, size=(N, K), dtype=np.uint8)
    mag = wq & 0x7F
    if fmt == 1:
        wq[mag == 0x7F] = 0x38
    else:
        wq[mag >= 0x7C] = 0x3C
    s = g.uniform(0.1, 1.0, size=(N, K // group)).astype(np.float32) * 1e-3
    td = {1: torch.float8_e4m3fn, 2: torch.float8_e5m2}
    y = tx.gemv_fp8_dequant(_t_bf16(x, dev), torch.from_numpy(wq).to(dev).view(td[fmt]),
                            torch.from_numpy(s).to(dev), group=group)
    r32, r16 = oracle.gemv_fp8_dequant(x, wq, s, group=group, fmt_w=fmt)
    check_close(_np_bits(y), r32, r16, FP8_TOL)
