"""Pins the oracle's MX-scaled dot (txo_gemm_mx_rows) against independent
computations: the closed form of the reference's scaled-dot check
(test_tlx.py:2271-2292: decoded operands times each e8m0 scale repeated over
its 32 K values, then a dense matmul) done in numpy float64; pure-Python
loops on a tiny case; exact doubling under a scale exponent shift; the e8m0
special codes 0 (2^-127) and 255 (NaN); K not a multiple of 32."""
import math

import numpy as np
import pytest


def _e8m0(codes):
    c = np.asarray(codes, np.float64)
    return np.where(c == 255, np.nan, np.exp2(c - 127.0))


def _closed_form(oracle, A, sa, B, sb, fa, fb):
    K = A.shape[1]
    a = oracle.decode(A.reshape(-1), fa).astype(np.float64).reshape(A.shape)
    b = oracle.decode(B.reshape(-1), fb).astype(np.float64).reshape(B.shape)
    SA = np.repeat(_e8m0(sa), 32, axis=1)[:, :K]
    SB = np.repeat(_e8m0(sb), 32, axis=1)[:, :K]
    return (a * SA) @ (b * SB).T


def _codes(g, shape, fmt):
    """Random finite codes of fmt (1 = e4m3fn, max 0x7E; 2 = e5m2, max 0x7B), both signs."""
    top = 0x7F if fmt == 1 else 0x7C
    return g.integers(0, top, shape, dtype=np.uint8) | (g.integers(0, 2, shape, dtype=np.uint8) << 7)


def _inputs(g, M, N, K, fa=1, fb=1, lo=120, hi=135):
    A = _codes(g, (M, K), fa)
    B = _codes(g, (N, K), fb)
    nb = (K + 31) // 32
    sa = g.integers(lo, hi, (M, nb), dtype=np.uint8)
    sb = g.integers(lo, hi, (N, nb), dtype=np.uint8)
    return A, sa, B, sb


@pytest.mark.parametrize("M,N,K,fa,fb", [(7, 9, 64, 1, 1), (5, 6, 96, 1, 2), (4, 8, 70, 2, 1),
                                         (3, 5, 33, 2, 2), (6, 4, 256, 1, 1)])
def test_mx_matches_repeated_scale_closed_form(oracle, M, N, K, fa, fb):
    g = np.random.default_rng(100 + K)
    A, sa, B, sb = _inputs(g, M, N, K, fa, fb)
    got, mag = oracle.gemm_mx_rows(A, sa, B, sb, 0, M, fa, fb)
    ref = _closed_form(oracle, A, sa, B, sb, fa, fb)
    assert np.all(np.abs(got - ref) <= 1e-6 * mag + 1e-37)
    # a transposed use of the scales or a k % 32 block index would not pass
    wrong = _closed_form(oracle, A, np.repeat(sa[:, :1], sa.shape[1], 1), B, sb, fa, fb)
    assert not np.allclose(got, wrong, rtol=1e-3, atol=0)


def test_mx_pure_python_loops(oracle):
    g = np.random.default_rng(5)
    M, N, K = 3, 4, 40
    A, sa, B, sb = _inputs(g, M, N, K, 1, 2)
    got, _ = oracle.gemm_mx_rows(A, sa, B, sb, 0, M, 1, 2)
    for m in range(M):
        for n in range(N):
            acc = 0.0
            for k in range(K):
                a = oracle.decode1(int(A[m, k]), 1) * 2.0 ** (int(sa[m, k // 32]) - 127)
                b = oracle.decode1(int(B[n, k]), 2) * 2.0 ** (int(sb[n, k // 32]) - 127)
                acc += a * b
            assert math.isclose(got[m, n], acc, rel_tol=1e-6, abs_tol=1e-30)


def test_mx_scale_shift_doubles_exactly(oracle):
    g = np.random.default_rng(6)
    M, N, K = 6, 5, 128
    A, sa, B, sb = _inputs(g, M, N, K)
    base, _ = oracle.gemm_mx_rows(A, sa, B, sb, 0, M)
    sa2 = sa.copy()
    sa2[2] += 1                       # row 2: every block twice as large
    sb2 = sb.copy()
    sb2[3] -= 2                       # column 3: a quarter
    got, _ = oracle.gemm_mx_rows(A, sa2, B, sb2, 0, M)
    want = base.copy()
    want[2] *= 2
    want[:, 3] /= 4
    assert np.array_equal(got, want)


def test_mx_special_scale_codes(oracle):
    g = np.random.default_rng(7)
    M, N, K = 4, 3, 64
    A, sa, B, sb = _inputs(g, M, N, K)
    # code 0 on A with 254 on B is 2^-127 * 2^127 = 1, the same as 127 and 127
    sa1, sb1 = sa.copy(), sb.copy()
    sa1[:, 1], sb1[:, 1] = 127, 127
    sa0, sb0 = sa.copy(), sb.copy()
    sa0[:, 1], sb0[:, 1] = 0, 254
    r1, _ = oracle.gemm_mx_rows(A, sa1, B, sb1, 0, M)
    r0, _ = oracle.gemm_mx_rows(A, sa0, B, sb0, 0, M)
    assert np.array_equal(r0, r1)
    # 255 is NaN: the whole row of C it scales
    sa_nan = sa.copy()
    sa_nan[1, 0] = 255
    rn, _ = oracle.gemm_mx_rows(A, sa_nan, B, sb, 0, M)
    assert np.all(np.isnan(rn[1])) and not np.any(np.isnan(np.delete(rn, 1, axis=0)))


def test_mx_block_max_output(oracle):
    g = np.random.default_rng(8)
    M, N, K = 3, 5, 100
    A, sa, B, sb = _inputs(g, M, N, K)
    _, mag, bmax = oracle.gemm_mx_rows(A, sa, B, sb, 0, M, block_max=True)
    a = oracle.decode(A.reshape(-1), 1).astype(np.float64).reshape(A.shape)
    b = oracle.decode(B.reshape(-1), 1).astype(np.float64).reshape(B.shape)
    want = np.zeros((M, N))
    for blk in range((K + 31) // 32):
        k = slice(32 * blk, min(32 * blk + 32, K))
        t = np.abs(a[:, None, k] * b[None, :, k]).max(axis=2)
        want += t * _e8m0(sa[:, blk])[:, None] * _e8m0(sb[:, blk])[None, :]
    assert np.allclose(bmax, want, rtol=1e-6, atol=0) and np.all(bmax <= mag * (1 + 1e-6))
