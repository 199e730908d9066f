"""GPU parity: tt.dot_scaled with MX block scales (tx_dot_scaled_mx) vs the
oracle's fp64 accumulation.

Tolerances: fp8 class, max|gpu - ref| / max|ref| <= 2e-2 (and Frobenius);
on top of that, element by element,
  |gpu - ref| <= 32 * 2^-13 * sum_b max_{k in b} |term_k|
                 + (K/64 + 2) * 2^-24 * sum|terms| + half an ulp of the output
(bf16 2^-8, fp16 2^-11 relative; fp16 subnormal spacing 2^-24).  The first
part is the scaled fp8 MFMA's own arithmetic: it sums the 32 products of a
block in fixed point aligned to the block's largest product and drops what
lies more than 13 bits below it (measured on the device: 1 + 2^-14 inside one
block gives 1, while blocks are combined exactly in fp32).  A wrong scale
block, lane, byte select or transposed scale is off by a factor of 2 or more
on whole blocks, far above the bound.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

FP8_TOL = 2e-2
TD = {1: torch.float8_e4m3fn, 2: torch.float8_e5m2}
OUT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def _codes(g, shape, fmt):
    top = 0x7F if fmt == 1 else 0x7C
    return g.integers(0, top, shape, dtype=np.uint8) | (g.integers(0, 2, shape, dtype=np.uint8) << 7)


def _run(tx, dev, aq, sa, bq, sb, fa=1, fb=1, out="bf16", lda=None, ld_s=None):
    """Operands and scales to the GPU (optionally as views into wider rows)."""
    M, K = aq.shape
    N = bq.shape[0]

    def put(x, ld, dtype=None):
        if ld is None or ld == x.shape[1]:
            t = torch.from_numpy(np.ascontiguousarray(x)).to(dev)
        else:
            w = np.zeros((x.shape[0], ld), np.uint8)
            w[:, :x.shape[1]] = x
            t = torch.from_numpy(w).to(dev)[:, :x.shape[1]]
        return t if dtype is None else t.view(dtype)

    A = put(aq, lda, TD[fa])
    B = put(bq, lda, TD[fb])
    SA = put(sa, ld_s)
    SB = put(sb, ld_s)
    C = tx.dot_scaled(A, SA, B, SB, out_dtype=OUT[out])
    torch.cuda.synchronize()
    return C.float().cpu().numpy()


def check_mx(got, ref, mag, bmax, K, out):
    got = got.astype(np.float64)
    ref = ref.astype(np.float64)
    mag = mag.astype(np.float64)
    bmax = bmax.astype(np.float64)
    scale = np.abs(ref).max()
    if scale > 0:
        assert np.abs(got - ref).max() / scale <= FP8_TOL
        assert np.linalg.norm(got - ref) / np.linalg.norm(ref) <= FP8_TOL
    ulp = {"f32": 2.0 ** -24, "bf16": 2.0 ** -8, "f16": 2.0 ** -11}[out]
    floor = {"f32": 0.0, "bf16": 0.0, "f16": 2.0 ** -25}[out]
    bound = 32 * 2.0 ** -13 * bmax + (K / 64 + 2) * 2.0 ** -24 * mag + ulp * np.abs(ref) * (1 + 1e-6) + floor
    bad = np.abs(got - ref) > bound
    assert not bad.any(), (int(bad.sum()), np.argwhere(bad)[:5], got[bad][:5], ref[bad][:5])


@pytest.mark.parametrize("M,N,K,fa,fb,out", [
    (256, 256, 256, 1, 1, "f32"), (256, 256, 256, 1, 1, "bf16"), (256, 256, 256, 1, 1, "f16"),
    (300, 500, 4096, 1, 1, "bf16"), (257, 501, 2048, 2, 1, "f32"), (64, 96, 96, 1, 2, "f32"),
    (130, 260, 1000, 2, 2, "bf16"), (77, 33, 33, 1, 1, "f32"), (1, 1, 32, 1, 1, "f32"),
    (600, 1000, 640, 1, 1, "f16"), (512, 2048, 4096, 1, 1, "f32"), (300, 1000, 2048, 2, 1, "bf16"),
    (256, 512, 8192, 1, 1, "f16")])
def test_mx_shapes(tx, oracle, dev, M, N, K, fa, fb, out):
    """256x256 tiles, 256x128 tiles with and without K split into fp32
    planes (the last three shapes split 4, 2 and 8 ways); K a multiple of
    128, of 32, or ragged (operands zero-padded)."""
    g = np.random.default_rng(M * 7 + N * 3 + K)
    aq, bq = _codes(g, (M, K), fa), _codes(g, (N, K), fb)
    nb = (K + 31) // 32
    lo, hi = (108, 118) if out == "f16" else (118, 134)   # keep fp16 outputs finite
    sa = g.integers(lo, hi, (M, nb), dtype=np.uint8)
    sb = g.integers(lo, hi, (N, nb), dtype=np.uint8)
    got = _run(tx, dev, aq, sa, bq, sb, fa, fb, out)
    ref, mag, bmax = oracle.gemm_mx_rows(aq, sa, bq, sb, 0, M, fa, fb, block_max=True)
    check_mx(got, ref, mag, bmax, K, out)


def test_mx_strided_operands_and_scales(tx, oracle, dev):
    """Operand rows wider than K (lda 16-aligned, then not) and scale rows
    wider than ceil(K/32) (4-aligned, then not)."""
    g = np.random.default_rng(11)
    M, N, K = 200, 300, 512
    aq, bq = _codes(g, (M, K), 1), _codes(g, (N, K), 1)
    sa = g.integers(120, 132, (M, K // 32), dtype=np.uint8)
    sb = g.integers(120, 132, (N, K // 32), dtype=np.uint8)
    ref, mag, bmax = oracle.gemm_mx_rows(aq, sa, bq, sb, 0, M, block_max=True)
    for lda, ld_s in ((K + 64, K // 32 + 4), (K + 3, K // 32 + 5)):
        got = _run(tx, dev, aq, sa, bq, sb, lda=lda, ld_s=ld_s, out="f32")
        check_mx(got, ref, mag, bmax, K, "f32")


def test_mx_special_scales(tx, oracle, dev):
    """e8m0 255 is NaN for every output it scales; code 0 is 2^-127 (0 on A
    against 254 on B gives the same bits as 127 against 127); exponents far
    from 127 (2^103 and 2^-87 on whole rows) stay within the fp32 bound."""
    g = np.random.default_rng(12)
    M, N, K = 256, 256, 256
    aq, bq = _codes(g, (M, K), 1), _codes(g, (N, K), 1)
    ones_a = np.full((M, K // 32), 127, np.uint8)
    ones_b = np.full((N, K // 32), 127, np.uint8)
    c11 = _run(tx, dev, aq, ones_a, bq, ones_b, out="f32")
    c0 = _run(tx, dev, aq, np.zeros_like(ones_a), bq, np.full_like(ones_b, 254), out="f32")
    assert np.array_equal(c0.view(np.uint32), c11.view(np.uint32))

    sa = g.integers(120, 134, (M, K // 32), dtype=np.uint8)
    sb = g.integers(100, 110, (N, K // 32), dtype=np.uint8)
    sa[5, 3] = 255
    sb[7, 0] = 255
    sa[10, :] = 230
    sa[11, :] = 40
    got = _run(tx, dev, aq, sa, bq, sb, out="f32")
    ref, mag, bmax = oracle.gemm_mx_rows(aq, sa, bq, sb, 0, M, block_max=True)
    assert np.all(np.isnan(got[5])) and np.all(np.isnan(got[:, 7]))
    keep = np.ones((M, N), bool)
    keep[5] = False
    keep[:, 7] = False
    assert np.all(np.isfinite(got[keep])) and np.all(np.isfinite(ref[keep]))
    d = np.abs(got.astype(np.float64) - ref)[keep]
    bound = 32 * 2.0 ** -13 * bmax.astype(np.float64) + (K / 64 + 2) * 2.0 ** -24 * mag.astype(np.float64)
    assert np.all(d <= bound[keep])
    assert np.abs(np.delete(got[10], 7)).max() > 2.0 ** 80
    assert 0 < np.abs(np.delete(got[11], 7)).max() < 2.0 ** -60


def test_mx_reference_check_form(tx, dev):
    """The reference's own check (test_tlx.py:2271-2292): operands are the
    values 20..39 cast to fp8, scales 124..129, fp16 output compared with a
    float32 matmul of the scale-expanded operands, atol 1e-2 * sqrt(K / 32),
    at its shape M = N = 256, K = 128."""
    M, N, K = 256, 256, 128
    torch.manual_seed(0)
    for fa, fb in ((1, 1), (2, 2), (1, 2), (2, 1)):
        a = torch.randint(20, 40, (M, K), dtype=torch.uint8).to(TD[fa])
        b = torch.randint(20, 40, (K, N), dtype=torch.uint8).to(TD[fb])
        sa = torch.randint(124, 130, (M, K // 32), dtype=torch.uint8)
        sb = torch.randint(124, 130, (N, K // 32), dtype=torch.uint8)
        c = tx.dot_scaled(a.to(dev), sa.to(dev), b.t().contiguous().to(dev), sb.to(dev),
                          out_dtype=torch.float16)
        sa_f = (sa.to(torch.int32) << 23).view(torch.float32).repeat_interleave(32, dim=1)[:M, :K]
        sb_f = (sb.to(torch.int32) << 23).view(torch.float32).repeat_interleave(32, dim=1).T.contiguous()[:K, :N]
        ref = torch.matmul(a.to(torch.float32) * sa_f, b.to(torch.float32) * sb_f).to(torch.float16)
        torch.testing.assert_close(ref, c.cpu(), atol=1e-2 * (K / 32) ** 0.5, rtol=0)


@pytest.mark.parametrize("M,N,K", [(8192, 8192, 8192), (512, 14336, 4096)])
def test_mx_quantised_config(tx, oracle, dev, M, N, K):
    """MX-quantised N(0,1) operands (the reference's quantiser idiom) at full
    size: sampled rows against the oracle, and the full-size scale property
    C(sa + 1) == 2 C bit-exactly."""
    import workloads
    aq, sa, bq, sb = workloads.mx_gemm_input(M, N, K)
    got = _run(tx, dev, aq, sa, bq, sb, out="bf16")
    g = np.random.default_rng(1)
    rows = sorted(set([0, M - 1] + list(g.integers(0, M, 6))))
    for r in rows:
        ref, mag, bmax = oracle.gemm_mx_rows(aq, sa, bq, sb, r, r + 1, block_max=True)
        check_mx(got[r:r + 1], ref, mag, bmax, K, "bf16")
    got2 = _run(tx, dev, aq, sa + 1, bq, sb, out="bf16")
    assert np.array_equal(got2, 2 * got)


def _tile_rows(M):
    """Two rows of every 256-row tile (its first and a seeded one), the last row."""
    g = np.random.default_rng(M)
    rows = {M - 1}
    for m0 in range(0, M, 256):
        rows |= {m0, int(g.integers(m0, min(M, m0 + 256)))}
    return sorted(rows)


@pytest.mark.parametrize("M,N,K,fa,fb,out", [
    (4096, 4096, 256, 1, 1, "bf16"),    # one tile per CU, two K steps
    (4196, 4168, 384, 2, 1, "f16"),     # partial last row and column tiles
    (4352, 4096, 256, 1, 2, "bf16"),    # 272 tiles: some workgroups walk two
    (4096, 4352, 512, 2, 2, "bf16")])
def test_mx_large_tiles(tx, oracle, dev, M, N, K, fa, fb, out):
    """Products of at least one 256 x 256 tile per CU (several rounds of
    workgroups, partial edge tiles), bf16 / fp16 out: two rows of every
    256-row tile (all columns) against the oracle, and for bf16 the whole
    output's exact doubling when every scale of A goes up by one."""
    g = np.random.default_rng(M + N + K + fa)
    aq, bq = _codes(g, (M, K), fa), _codes(g, (N, K), fb)
    nb = K // 32
    lo, hi = (108, 118) if out == "f16" else (118, 134)
    sa = g.integers(lo, hi, (M, nb), dtype=np.uint8)
    sb = g.integers(lo, hi, (N, nb), dtype=np.uint8)
    got = _run(tx, dev, aq, sa, bq, sb, fa, fb, out)
    for r in _tile_rows(M):
        ref, mag, bmax = oracle.gemm_mx_rows(aq, sa, bq, sb, r, r + 1, fa, fb, block_max=True)
        check_mx(got[r:r + 1], ref, mag, bmax, K, out)
    if out == "bf16":
        assert np.array_equal(_run(tx, dev, aq, sa + 1, bq, sb, fa, fb, out), 2 * got)


@pytest.mark.parametrize("M,N,K,out", [(4096, 4096, 512, "bf16"), (4196, 4168, 768, "f16"),
                                       (4352, 4096, 512, "bf16")])
def test_mx_fp4_large_tiles(tx, oracle, dev, M, N, K, out):
    """fp4 x fp4 products of at least one 256 x 256 tile per CU (two scale
    dwords per row and step): two rows of every 256-row tile against the
    oracle, and for bf16 the exact doubling under sa + 1."""
    g = np.random.default_rng(M * 5 + N + K)
    pa = g.integers(0, 256, (M, K // 2), dtype=np.uint8)
    pb = g.integers(0, 256, (N, K // 2), dtype=np.uint8)
    nb = K // 32
    lo, hi = (112, 122) if out == "f16" else (118, 136)
    sa = g.integers(lo, hi, (M, nb), dtype=np.uint8)
    sb = g.integers(lo, hi, (N, nb), dtype=np.uint8)
    got = _run_fp4(tx, dev, pa, sa, pb, sb, out)
    for r in _tile_rows(M):
        ref, mag, bmax = oracle.gemm_mx_rows(pa, sa, pb, sb, r, r + 1, fmt_a=4, fmt_b=4, block_max=True)
        check_mx(got[r:r + 1], ref, mag, bmax, K, out)
    if out == "bf16":
        assert np.array_equal(_run_fp4(tx, dev, pa, sa + 1, pb, sb, out), 2 * got)


def test_mx_table_op_and_errors(tx, oracle, dev):
    from tx import _lib
    g = np.random.default_rng(3)
    M, N, K = 64, 64, 128
    aq, bq = _codes(g, (M, K), 1), _codes(g, (N, K), 1)
    sa = g.integers(124, 130, (M, K // 32), dtype=np.uint8)
    sb = g.integers(124, 130, (N, K // 32), dtype=np.uint8)
    A = torch.from_numpy(aq).to(dev)
    B = torch.from_numpy(bq).to(dev)
    SA = torch.from_numpy(sa).to(dev)
    SB = torch.from_numpy(sb).to(dev)
    C = torch.empty((M, N), dtype=torch.float32, device=dev)
    tx.invoke("tt.dot_scaled", [C, A, B, SA, SB, M, N, K, K, K, N, K // 32, K // 32,
                                _lib.FP8E4M3FN, _lib.FP8E4M3FN, _lib.F32])
    torch.cuda.synchronize()
    ref, mag, bmax = oracle.gemm_mx_rows(aq, sa, bq, sb, 0, M, block_max=True)
    check_mx(C.cpu().numpy(), ref, mag, bmax, K, "f32")
    with pytest.raises(ValueError):
        tx.dot_scaled(A.view(torch.float8_e4m3fn), SA[:, :3], B.view(torch.float8_e4m3fn), SB)
    with pytest.raises(tx.TxError):
        tx.invoke("tt.dot_scaled", [C, A, B, SA, SB, M, N, K, K, K, N, 2, K // 32,
                                    _lib.FP8E4M3FN, _lib.FP8E4M3FN, _lib.F32])
    with pytest.raises(tx.TxError):
        tx.invoke("tt.dot_scaled", [C, A, B, SA, SB, M, N, K, K, K, N, K // 32, K // 32,
                                    _lib.FP8E4M3FN, _lib.BF16, _lib.F32])


# ---------------------------------------------------------------- fp4 (e2m1)
def _run_fp4(tx, dev, pa, sa, pb, sb, out="bf16", lda=None, dtype_form=False):
    """Packed fp4 operands (M x K/2 bytes) to the GPU as uint8 with format
    'e2m1' (or as float4_e2m1fn_x2), optionally as views into wider rows."""
    def put(x, ld):
        if ld is None or ld == x.shape[1]:
            return torch.from_numpy(np.ascontiguousarray(x)).to(dev)
        w = np.zeros((x.shape[0], ld), np.uint8)
        w[:, :x.shape[1]] = x
        return torch.from_numpy(w).to(dev)[:, :x.shape[1]]

    A, B = put(pa, lda), put(pb, lda)
    SA, SB = put(sa, None), put(sb, None)
    if dtype_form:
        C = tx.dot_scaled(A.view(torch.float4_e2m1fn_x2), SA, B.view(torch.float4_e2m1fn_x2), SB,
                          out_dtype=OUT[out])
    else:
        C = tx.dot_scaled(A, SA, B, SB, out_dtype=OUT[out], a_format="e2m1", b_format="e2m1")
    torch.cuda.synchronize()
    return C.float().cpu().numpy()


@pytest.mark.parametrize("M,N,K,out", [
    (256, 256, 256, "f32"), (256, 256, 512, "bf16"), (1024, 1280, 2048, "bf16"),
    (300, 500, 4096, "f32"), (77, 33, 64, "f32"), (130, 260, 1000, "f16"), (1, 1, 2, "f32"),
    (512, 2048, 8192, "f32"), (256, 512, 16384, "bf16")])
def test_mx_fp4_shapes(tx, oracle, dev, M, N, K, out):
    """fp4 x fp4 (two values a byte, the even K index in the low nibble):
    256x256 tiles, 256x128 tiles unsplit and split over K, K a multiple of
    256 (whole 128-byte steps), of 32, and ragged (rows zero-padded)."""
    g = np.random.default_rng(M * 5 + N + K)
    pa = g.integers(0, 256, (M, K // 2), dtype=np.uint8)
    pb = g.integers(0, 256, (N, K // 2), dtype=np.uint8)
    nb = (K + 31) // 32
    lo, hi = (112, 122) if out == "f16" else (118, 136)
    sa = g.integers(lo, hi, (M, nb), dtype=np.uint8)
    sb = g.integers(lo, hi, (N, nb), dtype=np.uint8)
    got = _run_fp4(tx, dev, pa, sa, pb, sb, out)
    ref, mag, bmax = oracle.gemm_mx_rows(pa, sa, pb, sb, 0, M, fmt_a=4, fmt_b=4, block_max=True)
    check_mx(got, ref, mag, bmax, K, out)


def test_mx_fp4_strided_and_dtype_form(tx, oracle, dev):
    """Operand rows wider than K/2 bytes (16-aligned, then not) and the
    float4_e2m1fn_x2 dtype in place of uint8 + format."""
    g = np.random.default_rng(31)
    M, N, K = 200, 300, 1024
    pa = g.integers(0, 256, (M, K // 2), dtype=np.uint8)
    pb = g.integers(0, 256, (N, K // 2), dtype=np.uint8)
    sa = g.integers(120, 132, (M, K // 32), dtype=np.uint8)
    sb = g.integers(120, 132, (N, K // 32), dtype=np.uint8)
    ref, mag, bmax = oracle.gemm_mx_rows(pa, sa, pb, sb, 0, M, fmt_a=4, fmt_b=4, block_max=True)
    for lda in (K // 2 + 64, K // 2 + 3):
        check_mx(_run_fp4(tx, dev, pa, sa, pb, sb, "f32", lda=lda), ref, mag, bmax, K, "f32")
    check_mx(_run_fp4(tx, dev, pa, sa, pb, sb, "f32", dtype_form=True), ref, mag, bmax, K, "f32")


def test_mx_fp4_reference_check_form(tx, dev):
    """The reference's mxfp4 check (test_tlx.py:4774-4856): M = N = K = 128,
    operands of 2.0 packed by triton's MXFP4Tensor, scales 127, fp16 output
    against a float32 matmul of the scale-expanded values, atol
    1e-2 * sqrt(K / 32); then the same with random values and scales
    124..129."""
    mxfp = pytest.importorskip("triton.tools.mxfp")
    M = N = K = 128
    torch.manual_seed(0)
    for rand in (False, True):
        if rand:
            a = torch.randint(0, 16, (M, K), dtype=torch.uint8)
            b = torch.randint(0, 16, (N, K), dtype=torch.uint8)
            ta, tb = mxfp.MXFP4Tensor(size=(M, K), device="cpu"), mxfp.MXFP4Tensor(size=(N, K), device="cpu")
            ta.data, tb.data = a, b
            sa = torch.randint(124, 130, (M, K // 32), dtype=torch.uint8)
            sb = torch.randint(124, 130, (N, K // 32), dtype=torch.uint8)
        else:
            ta = mxfp.MXFP4Tensor(data=torch.full((M, K), 2.0), device="cpu")
            tb = mxfp.MXFP4Tensor(data=torch.full((N, K), 2.0), device="cpu")
            sa = torch.full((M, K // 32), 127, dtype=torch.uint8)
            sb = torch.full((N, K // 32), 127, dtype=torch.uint8)
        c = tx.dot_scaled(ta.to_packed_tensor(dim=1).to(dev), sa.to(dev), tb.to_packed_tensor(dim=1).to(dev),
                          sb.to(dev), out_dtype=torch.float16, a_format="e2m1", b_format="e2m1")
        sa_f = (sa.to(torch.int32) << 23).view(torch.float32).repeat_interleave(32, dim=1)[:M, :K]
        sb_f = (sb.to(torch.int32) << 23).view(torch.float32).repeat_interleave(32, dim=1).T.contiguous()[:K, :N]
        ref = torch.matmul(ta.to(torch.float32) * sa_f, tb.to(torch.float32).T * sb_f).to(torch.float16)
        torch.testing.assert_close(ref, c.cpu(), atol=1e-2 * (K / 32) ** 0.5, rtol=0)


@pytest.mark.parametrize("M,N,K,a4,f8,out", [
    (256, 256, 256, True, 1, "f32"), (256, 256, 256, False, 1, "bf16"), (1024, 1280, 2048, True, 2, "bf16"),
    (300, 500, 4096, False, 2, "f32"), (77, 33, 64, True, 1, "f32"), (130, 260, 1000, False, 1, "f16"),
    (64, 96, 200, True, 2, "f32"), (512, 2048, 8192, False, 1, "f32")])
def test_mx_mixed_fp4_fp8(tx, oracle, dev, M, N, K, a4, f8, out):
    """fp4 x fp8 and fp8 x fp4 (the reference's mixed mxfp8 / mxfp4 pairs):
    the fp4 operand is expanded to e4m3fn, exactly, then meets the fp8 one in
    the fp8 tile; K a multiple of 128, ragged with the fp8 rows read in
    place (K % 16 == 0), and ragged with them padded (1000, 200)."""
    g = np.random.default_rng(M * 3 + N * 7 + K + a4)
    nb = (K + 31) // 32
    p4 = g.integers(0, 256, ((M if a4 else N), K // 2), dtype=np.uint8)
    c8 = _codes(g, ((N if a4 else M), K), f8)
    lo, hi = (112, 120) if out == "f16" else (118, 134)
    sa = g.integers(lo, hi, (M, nb), dtype=np.uint8)
    sb = g.integers(lo, hi, (N, nb), dtype=np.uint8)
    aq, bq = (p4, c8) if a4 else (c8, p4)
    fa, fb = (4, f8) if a4 else (f8, 4)
    A = torch.from_numpy(aq).to(dev)
    B = torch.from_numpy(bq).to(dev)
    if not a4:
        A = A.view(TD[f8])
    else:
        B = B.view(TD[f8])
    C = tx.dot_scaled(A, torch.from_numpy(sa).to(dev), B, torch.from_numpy(sb).to(dev), out_dtype=OUT[out],
                      a_format="e2m1" if a4 else None, b_format=None if a4 else "e2m1")
    torch.cuda.synchronize()
    ref, mag, bmax = oracle.gemm_mx_rows(aq, sa, bq, sb, 0, M, fmt_a=fa, fmt_b=fb, block_max=True)
    check_mx(C.float().cpu().numpy(), ref, mag, bmax, K, out)


@pytest.mark.parametrize("a_fmt,b_fmt", [("e4m3", "e2m1"), ("e2m1", "e4m3")])
def test_mx_mixed_reference_check_form(tx, dev, a_fmt, b_fmt):
    """The reference's mixed check (test_tlx.py:4866-5080): M = N = K = 128,
    the fp4 operand 2.0 packed by triton's MXFP4Tensor, the fp8 one the
    values 20..39 cast to e4m3fn, scales 127, fp16 output against a float32
    matmul, atol 1e-2 * sqrt(K / 32)."""
    mxfp = pytest.importorskip("triton.tools.mxfp")
    M = N = K = 128
    torch.manual_seed(0)
    if a_fmt == "e2m1":
        t = mxfp.MXFP4Tensor(data=torch.full((M, K), 2.0), device="cpu")
        a, a_ref = t.to_packed_tensor(dim=1), t.to(torch.float32)
    else:
        a = torch.randint(20, 40, (M, K), dtype=torch.uint8).to(torch.float8_e4m3fn)
        a_ref = a.to(torch.float32)
    if b_fmt == "e2m1":
        t = mxfp.MXFP4Tensor(data=torch.full((N, K), 2.0), device="cpu")
        b_nk, b_ref = t.to_packed_tensor(dim=1), t.to(torch.float32).T
    else:
        b = torch.randint(20, 40, (K, N), dtype=torch.uint8).to(torch.float8_e4m3fn)
        b_nk, b_ref = b.t().contiguous(), b.to(torch.float32)
    sa = torch.full((M, K // 32), 127, dtype=torch.uint8)
    sb = torch.full((N, K // 32), 127, dtype=torch.uint8)
    c = tx.dot_scaled(a.to(dev), sa.to(dev), b_nk.to(dev), sb.to(dev), out_dtype=torch.float16,
                      a_format=a_fmt, b_format=b_fmt)
    ref = torch.matmul(a_ref, b_ref).to(torch.float16)
    torch.testing.assert_close(ref, c.cpu(), atol=1e-2 * (K / 32) ** 0.5, rtol=0)


def test_mx_fp4_errors(tx, dev):
    from tx import _lib
    M, N, K = 64, 64, 128
    A = torch.zeros((M, K // 2), dtype=torch.uint8, device=dev)
    A8 = torch.zeros((M, K), dtype=torch.uint8, device=dev)
    S = torch.full((M, K // 32), 127, dtype=torch.uint8, device=dev)
    C = torch.empty((M, N), dtype=torch.float32, device=dev)
    with pytest.raises(tx.TxError):   # fp8 B rows shorter than K bytes
        tx.invoke("tt.dot_scaled", [C, A, A8, S, S, M, N, K, K // 2, K // 2, N, K // 32, K // 32,
                                    _lib.FP4E2M1, _lib.FP8E4M3FN, _lib.F32])
    with pytest.raises(tx.TxError):   # odd K
        tx.invoke("tt.dot_scaled", [C, A, A, S, S, M, N, K - 1, K // 2, K // 2, N, K // 32, K // 32,
                                    _lib.FP4E2M1, _lib.FP4E2M1, _lib.F32])
    with pytest.raises(ValueError):   # uint8 without a format
        tx.dot_scaled(A, S, A, S)
    with pytest.raises(ValueError):   # K of A (128) and B (64) disagree
        tx.dot_scaled(A, S, A8[:, :64].view(torch.float8_e4m3fn), S[:, :2], a_format="e2m1")
    # same K, fp4 x fp8: served (zeros in, zeros out)
    z = tx.dot_scaled(A, S, A8.view(torch.float8_e4m3fn), S, a_format="e2m1")
    assert torch.count_nonzero(z).item() == 0


def test_mx_fp4_special_scales(tx, oracle, dev):
    """fp4 operands under e8m0 special codes: 255 is NaN for every output it
    scales, code 0 (2^-127) against 254 gives the same bits as 127 against
    127, and far exponents (2^103, 2^-87 on whole rows) stay within the
    fp32 bound."""
    g = np.random.default_rng(13)
    M, N, K = 256, 256, 512
    pa = g.integers(0, 256, (M, K // 2), dtype=np.uint8)
    pb = g.integers(0, 256, (N, K // 2), dtype=np.uint8)
    ones_a = np.full((M, K // 32), 127, np.uint8)
    ones_b = np.full((N, K // 32), 127, np.uint8)
    c11 = _run_fp4(tx, dev, pa, ones_a, pb, ones_b, "f32")
    c0 = _run_fp4(tx, dev, pa, np.zeros_like(ones_a), pb, np.full_like(ones_b, 254), "f32")
    assert np.array_equal(c0.view(np.uint32), c11.view(np.uint32))
    sa = g.integers(120, 134, (M, K // 32), dtype=np.uint8)
    sb = g.integers(100, 110, (N, K // 32), dtype=np.uint8)
    sa[5, 3] = 255
    sb[7, 0] = 255
    sa[10, :] = 230
    sa[11, :] = 40
    got = _run_fp4(tx, dev, pa, sa, pb, sb, "f32")
    ref, mag, bmax = oracle.gemm_mx_rows(pa, sa, pb, sb, 0, M, fmt_a=4, fmt_b=4, block_max=True)
    assert np.all(np.isnan(got[5])) and np.all(np.isnan(got[:, 7]))
    keep = np.ones((M, N), bool)
    keep[5] = False
    keep[:, 7] = False
    assert np.all(np.isfinite(got[keep])) and np.all(np.isfinite(ref[keep]))
    d = np.abs(got.astype(np.float64) - ref)[keep]
    bound = 32 * 2.0 ** -13 * bmax.astype(np.float64) + (K / 64 + 2) * 2.0 ** -24 * mag.astype(np.float64)
    assert np.all(d <= bound[keep])
    assert np.abs(np.delete(got[10], 7)).max() > 2.0 ** 80
    assert 0 < np.abs(np.delete(got[11], 7)).max() < 2.0 ** -60
