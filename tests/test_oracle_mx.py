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


# ---------------------------------------------------------------- fp4 (e2m1)
E2M1_TABLE = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]


def _fp4_unpack(P, K):
    """Packed rows (two nibbles a byte, even K low) -> nibble codes."""
    lo, hi = P & 15, P >> 4
    return np.stack([lo, hi], axis=2).reshape(P.shape[0], -1)[:, :K]


def _fp4_values(codes):
    mag = np.array(E2M1_TABLE)[codes & 7]
    return np.where(codes & 8, -mag, mag)


def test_e2m1_nibbles_are_the_ocp_table(oracle):
    got = [oracle.e2m1_value(n) for n in range(16)]
    assert got[:8] == E2M1_TABLE
    assert got[8:] == [-v for v in E2M1_TABLE] and math.copysign(1.0, got[8]) < 0


def test_e2m1_decode_and_packing_match_triton_mxfp4(oracle):
    """triton's MXFP4Tensor (the packer the reference's mxfp4 test uses,
    test_tlx.py:4783-4786) decodes the 16 nibbles to the oracle's values and
    packs the even K index into the low nibble, which the oracle's product
    of the packed rows must then reproduce."""
    torch = pytest.importorskip("torch")
    mxfp = pytest.importorskip("triton.tools.mxfp")
    t = mxfp.MXFP4Tensor(size=(1, 16), device="cpu")
    t.data = torch.arange(16, dtype=torch.uint8).reshape(1, 16)
    dec = t.to(torch.float32).numpy().reshape(-1)
    assert np.array_equal(dec, np.array([oracle.e2m1_value(n) for n in range(16)], np.float32))
    g = np.random.default_rng(21)
    M, N, K = 5, 7, 128
    va = g.choice(E2M1_TABLE, (M, K)) * g.choice([-1, 1], (M, K))
    vb = g.choice(E2M1_TABLE, (N, K)) * g.choice([-1, 1], (N, K))
    PA = mxfp.MXFP4Tensor(data=torch.from_numpy(va).float(), device="cpu").to_packed_tensor(dim=1).numpy()
    PB = mxfp.MXFP4Tensor(data=torch.from_numpy(vb).float(), device="cpu").to_packed_tensor(dim=1).numpy()
    assert PA.shape == (M, K // 2)
    sa = g.integers(124, 130, (M, K // 32), dtype=np.uint8)
    sb = g.integers(124, 130, (N, K // 32), dtype=np.uint8)
    o, _ = oracle.gemm_mx_rows(PA, sa, PB, sb, 0, M, fmt_a=4, fmt_b=4)
    want = (va * np.repeat(_e8m0(sa), 32, axis=1)) @ (vb * np.repeat(_e8m0(sb), 32, axis=1)).T
    assert np.array_equal(o, want.astype(np.float32))


@pytest.mark.parametrize("K", [64, 96, 130])
def test_fp4_dot_closed_form(oracle, K):
    """Random nibbles (ragged K too): the float64 matmul of the unpacked,
    scaled values, and a pure-Python loop on a corner."""
    g = np.random.default_rng(K)
    M, N = 9, 11
    PA = g.integers(0, 256, (M, (K + 1) // 2), dtype=np.uint8)
    PB = g.integers(0, 256, (N, (K + 1) // 2), dtype=np.uint8)
    if K % 2:  # the pad nibble of an odd K is zero, as the packer writes it
        PA[:, -1] &= 15
        PB[:, -1] &= 15
    nb = (K + 31) // 32
    sa = g.integers(118, 136, (M, nb), dtype=np.uint8)
    sb = g.integers(118, 136, (N, nb), dtype=np.uint8)
    o, mag = oracle.gemm_mx_rows(PA, sa, PB, sb, 0, M, fmt_a=4, fmt_b=4)
    a = _fp4_values(_fp4_unpack(PA, K)) * np.repeat(_e8m0(sa), 32, axis=1)[:, :K]
    b = _fp4_values(_fp4_unpack(PB, K)) * np.repeat(_e8m0(sb), 32, axis=1)[:, :K]
    want = a @ b.T
    np.testing.assert_allclose(o, want, rtol=1e-6, atol=1e-6 * np.abs(a).max() * np.abs(b).max())
    np.testing.assert_allclose(mag, np.abs(a) @ np.abs(b).T, rtol=1e-6)
    m, n = 3, 4
    s = 0.0
    for k in range(K):
        na = (PA[m, k // 2] >> (4 * (k % 2))) & 15
        nb_ = (PB[n, k // 2] >> (4 * (k % 2))) & 15
        s += oracle.e2m1_value(na) * oracle.e2m1_value(nb_) * \
            2.0 ** (int(sa[m, k // 32]) - 127) * 2.0 ** (int(sb[n, k // 32]) - 127)
    assert math.isclose(o[m, n], s, rel_tol=1e-6, abs_tol=1e-30)


def test_fp4_workload_quantiser_matches_triton_mxfp4(oracle):
    """The benchmark's fp4 quantiser (workloads.quant_mx_fp4): scales by
    the OCP rule floor(log2 absmax) - 2, codes equal to triton's MXFP4Tensor
    rounding of x / scale (packed by its to_packed_tensor), and every
    dequantised value within half an e2m1 step of x (or saturated at 6)."""
    torch = pytest.importorskip("torch")
    mxfp = pytest.importorskip("triton.tools.mxfp")
    import workloads
    g = np.random.default_rng(0)
    x = (g.standard_normal((64, 256)) * np.exp2(g.integers(-10, 10, (64, 1)))).astype(np.float32)
    x[0, :32] = 0.0
    x[2, 40:72] = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 6.0] * 4, np.float32)  # ties
    P, S = workloads.quant_mx_fp4(x)
    amax = np.abs(x.reshape(64, 8, 32)).max(axis=2)
    want_s = np.where(amax > 0, np.floor(np.log2(np.where(amax > 0, amax, 1))) - 2 + 127, 127)
    assert np.array_equal(S, want_s.astype(np.uint8))
    v = (x.reshape(64, 8, 32) * np.exp2(127.0 - S)[:, :, None]).reshape(64, 256).astype(np.float32)
    tp = mxfp.MXFP4Tensor(data=torch.from_numpy(v), device="cpu").to_packed_tensor(dim=1).numpy()
    assert np.array_equal(P, tp)
    codes = np.stack([P & 15, P >> 4], axis=2).reshape(64, 256)
    dq = np.array([oracle.e2m1_value(c) for c in range(16)])[codes]
    step = np.where(np.abs(v) < 2, 0.5, np.where(np.abs(v) < 4, 1.0, 2.0))
    assert np.all((np.abs(dq - v) <= step / 2) | (np.abs(dq) == 6.0))
