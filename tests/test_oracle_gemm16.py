"""CPU pins of the oracle's 16-bit tt.dot (oracle.gemm16_rows).

Checked against numpy's float64 matmul of the operands widened by numpy
(fp16) or torch (bf16), for both B layouts (N x K storage, and the row-major
K x N of the reference's matmul caller) with N != K so that reading B in the
wrong layout fails; the RNE output against numpy's / torch's own casts of
the fp32 result; exact fp16 subnormal and Inf / NaN propagation."""
import numpy as np
import torch

import oracle


def _widen(bits, fp16):
    if fp16:
        return bits.view(np.float16).astype(np.float64)
    return torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).double().numpy()


def _case(M, N, K, fp16, b_kn, seed):
    g = np.random.default_rng(seed)
    a = g.standard_normal((M, K)).astype(np.float32)
    b = g.standard_normal((N, K)).astype(np.float32)
    if fp16:
        A, B = a.astype(np.float16).view(np.uint16), b.astype(np.float16).view(np.uint16)
    else:
        A = torch.from_numpy(a).bfloat16().view(torch.int16).numpy().view(np.uint16)
        B = torch.from_numpy(b).bfloat16().view(torch.int16).numpy().view(np.uint16)
    ref = _widen(A, fp16) @ _widen(B, fp16).T
    Bs = np.ascontiguousarray(B.T) if b_kn else B
    return A, Bs, ref


def test_both_formats_and_layouts_against_numpy():
    for fp16 in (True, False):
        for b_kn in (False, True):
            A, B, ref = _case(37, 23, 61, fp16, b_kn, seed=3 + fp16 + 2 * b_kn)
            fmt = oracle.F16 if fp16 else oracle.BF16
            o32, o16 = oracle.gemm16_rows(A, B, 0, 37, fmt=fmt, b_kn=b_kn)
            assert np.allclose(o32, ref, rtol=1e-6, atol=1e-5)
            # rows subset
            p32, _ = oracle.gemm16_rows(A, B, 5, 9, fmt=fmt, b_kn=b_kn)
            assert np.array_equal(p32, o32[5:9])


def test_wrong_layout_would_fail():
    A, B, ref = _case(8, 12, 20, True, True, seed=11)
    # B is K x N; read as N x K it is another product (and another shape)
    o32, _ = oracle.gemm16_rows(A, B, 0, 8, fmt=oracle.F16, b_kn=True)
    assert np.allclose(o32, ref, rtol=1e-6, atol=1e-5)
    Bt = np.ascontiguousarray(B.T)  # N x K storage of the same matrix
    o32b, _ = oracle.gemm16_rows(A, Bt, 0, 8, fmt=oracle.F16, b_kn=False)
    assert np.array_equal(o32, o32b)


def test_output_rounding_is_the_casts():
    A, B, _ = _case(16, 9, 33, True, False, seed=5)
    o32, o16 = oracle.gemm16_rows(A, B, 0, 16, fmt=oracle.F16)
    assert np.array_equal(o16, o32.astype(np.float16).view(np.uint16))
    _, ob = oracle.gemm16_rows(A, B, 0, 16, fmt=oracle.F16, out_fmt=oracle.BF16)
    assert np.array_equal(ob, torch.from_numpy(o32).bfloat16().view(torch.int16).numpy().view(np.uint16))


def test_fp16_subnormals_and_specials():
    # 1 x K times K x 1: single products of exact fp16 values
    sub = np.array([0x0001, 0x03FF, 0x8200, 0x0400, 0x7BFF], np.uint16)  # 2^-24, max sub, -sub, min norm, max
    one = np.full(5, 0x3C00, np.uint16)
    for i in range(5):
        A = sub[i:i + 1].reshape(1, 1)
        B = one[i:i + 1].reshape(1, 1)
        o32, _ = oracle.gemm16_rows(A, B, 0, 1, fmt=oracle.F16, b_kn=True)
        assert o32[0, 0] == np.float32(sub[i:i + 1].view(np.float16)[0])
    A = np.array([[0x7C00, 0x3C00]], np.uint16)  # +Inf, 1
    B = np.array([[0x3C00], [0x3C00]], np.uint16)
    o32, o16 = oracle.gemm16_rows(A, B, 0, 1, fmt=oracle.F16, b_kn=True)
    assert np.isinf(o32[0, 0]) and o16[0, 0] == 0x7C00
    A = np.array([[0x7C00, 0xFC00]], np.uint16)  # Inf - Inf = NaN
    o32, o16 = oracle.gemm16_rows(A, B, 0, 1, fmt=oracle.F16, b_kn=True)
    assert np.isnan(o32[0, 0]) and (o16[0, 0] & 0x7FFF) > 0x7C00
