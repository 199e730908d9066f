"""Pins for the oracle's scatter, GEMM and GEMV functions (CPU only).

Each is compared with an independent computation: plain Python / numpy loops
on tiny inputs, numpy float64 matmul, math.fsum, and algebraic properties that
a dropped term, a wrong index or a transposed operand would break.
"""
import math

import numpy as np
import pytest
import torch


def bf16_bits(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16) \
        .view(torch.int16).numpy().view(np.uint16)


def bf16_val(h):
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------- scatter
def test_scatter_i32_brute_force_and_wrap(oracle):
    g = np.random.default_rng(0)
    n, nb = 5000, 37
    idx = g.integers(-2, nb + 2, size=n, dtype=np.int32)
    val = g.integers(-2 ** 31, 2 ** 31, size=n, dtype=np.int64).astype(np.int32)
    mask = (g.random(n) < 0.7).astype(np.uint8)
    init = g.integers(-100, 100, size=nb, dtype=np.int32)
    ref = [int(v) for v in init]
    for i in range(n):
        if 0 <= idx[i] < nb and mask[i]:
            ref[idx[i]] = (ref[idx[i]] + int(val[i]) + 2 ** 31) % 2 ** 32 - 2 ** 31
    assert np.array_equal(oracle.scatter_add_i32(init, idx, val, mask), np.array(ref, np.int32))


def test_scatter_i32_mt_matches_sequential(oracle):
    g = np.random.default_rng(1)
    idx = g.integers(0, 1000, size=200_000, dtype=np.int32)
    val = g.integers(0, 1 << 30, size=200_000, dtype=np.int32)
    seq = oracle.scatter_add_i32(np.zeros(1000, np.int32), idx, val)
    assert np.array_equal(oracle.scatter_add_i32_mt(1000, idx, val, nthreads=4), seq)


def test_scatter_f32_reference_sums(oracle):
    g = np.random.default_rng(2)
    n, nb = 3000, 11
    idx = g.integers(0, nb, size=n, dtype=np.int32)
    val = g.standard_normal(n).astype(np.float32)
    s, a = oracle.scatter_add_f32_ref(nb, idx, val)
    for b in range(nb):
        sel = val[idx == b].astype(np.float64)
        assert abs(s[b] - math.fsum(sel)) <= 1e-12 * max(1.0, np.abs(sel).sum())
        assert abs(a[b] - np.abs(sel).sum()) <= 1e-9
    # conservation of the total
    assert abs(s.sum() - math.fsum(val.astype(np.float64))) < 1e-9
    seq = oracle.scatter_add_f32_seq(np.zeros(nb, np.float32), idx, val)
    assert np.max(np.abs(seq - s) / np.maximum(a, 1e-30)) < 1e-5


# --------------------------------------------------------------------- bf16
def test_bf16_rounding_matches_torch(oracle):
    g = np.random.default_rng(3)
    x = g.integers(0, 1 << 32, size=200_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    fin = np.isfinite(x)
    assert np.array_equal(oracle.f32_to_bf16(x[fin]), bf16_bits(x[fin]))
    for v in x[:2000]:
        if np.isfinite(v):
            assert oracle.lib().txo_f32_to_bf16(float(v)) == bf16_bits(np.array([v]))[0]


@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (3, 5, 7), (17, 19, 23), (8, 64, 130)])
def test_gemm_bf16_vs_numpy(oracle, M, N, K):
    g = np.random.default_rng(M * N * K)
    A = bf16_bits(g.uniform(-1, 1, (M, K)))
    B = bf16_bits(g.uniform(-1, 1, (N, K)))
    r32, r16 = oracle.gemm_bf16_rows(A, B, 0, M)
    ref = bf16_val(A).astype(np.float64) @ bf16_val(B).astype(np.float64).T
    assert np.allclose(r32, ref, rtol=1e-6, atol=1e-6)
    assert np.array_equal(r16, bf16_bits(ref.astype(np.float32)))
    # row slices agree with the full product (no index mix-up between rows)
    r32b, _ = oracle.gemm_bf16_rows(A, B, M // 2, M)
    assert np.array_equal(r32b, r32[M // 2:])


def test_gemm_bf16_brute_force_loops(oracle):
    g = np.random.default_rng(4)
    M, N, K = 3, 4, 5
    A = bf16_bits(g.uniform(-1, 1, (M, K)))
    B = bf16_bits(g.uniform(-1, 1, (N, K)))
    r32, _ = oracle.gemm_bf16_rows(A, B, 0, M)
    a, b = bf16_val(A), bf16_val(B)
    for m in range(M):
        for n in range(N):
            assert abs(r32[m, n] - math.fsum(float(a[m, k]) * float(b[n, k]) for k in range(K))) < 1e-6


@pytest.mark.parametrize("fa,fb", [(1, 1), (2, 2), (1, 2)])
def test_gemm_fp8_scaled_vs_numpy(oracle, fa, fb):
    g = np.random.default_rng(fa + 3 * fb)
    M, N, K = 9, 13, 70
    aq = g.integers(0, 256, size=(M, K), dtype=np.uint8)
    bq = g.integers(0, 256, size=(N, K), dtype=np.uint8)
    td = {1: torch.float8_e4m3fn, 2: torch.float8_e5m2}
    af = torch.from_numpy(aq).view(td[fa]).float().numpy().astype(np.float64)
    bf = torch.from_numpy(bq).view(td[fb]).float().numpy().astype(np.float64)
    ok_a = np.isfinite(af).all(axis=1)
    ok_b = np.isfinite(bf).all(axis=1)
    sa = g.uniform(0.5, 2, M).astype(np.float32)
    sb = g.uniform(0.5, 2, N).astype(np.float32)
    r32, _ = oracle.gemm_fp8_scaled_rows(aq, bq, sa, sb, 0, M, fa, fb)
    with np.errstate(invalid="ignore"):  # rows holding NaN/Inf codes are excluded below
        ref = (af @ bf.T) * sa[:, None].astype(np.float64) * sb[None, :].astype(np.float64)
    sel = np.ix_(ok_a, ok_b)
    assert np.allclose(r32[sel], ref[sel], rtol=1e-6, atol=1e-3)
    # scale linearity
    r2, _ = oracle.gemm_fp8_scaled_rows(aq, bq, 2 * sa, sb, 0, M, fa, fb)
    assert np.array_equal(r2[sel], 2 * r32[sel])


def test_gemv_vs_numpy_and_group_split(oracle):
    g = np.random.default_rng(5)
    M, N, K, group = 3, 7, 512, 128
    x = bf16_bits(g.standard_normal((M, K)))
    wq = g.integers(0, 0x7C, size=(N, K), dtype=np.uint8)  # finite e5m2 codes
    wq |= (g.integers(0, 2, size=(N, K), dtype=np.uint8) << 7)
    s = g.uniform(0.1, 1, size=(N, K // group)).astype(np.float32)
    r32, r16 = oracle.gemv_fp8_dequant(x, wq, s, group=group)
    w = torch.from_numpy(wq).view(torch.float8_e5m2).float().numpy().astype(np.float64)
    wdq = w * np.repeat(s.astype(np.float64), group, axis=1)
    ref = bf16_val(x).astype(np.float64) @ wdq.T
    assert np.allclose(r32, ref, rtol=1e-6, atol=1e-6)
    assert np.array_equal(r16, bf16_bits(r32))
    # a group scale multiplies only its own 128 columns of K
    s2 = s.copy()
    s2[:, 1] *= 4
    r32b, _ = oracle.gemv_fp8_dequant(x, wq, s2, group=group)
    wdq2 = w * np.repeat(s2.astype(np.float64), group, axis=1)
    assert np.allclose(r32b, bf16_val(x).astype(np.float64) @ wdq2.T, rtol=1e-6, atol=1e-6)
