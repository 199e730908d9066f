"""GPU parity of tt.dot with its accumulator operand (tx_dot_acc):
D = round(s * A.B + C) in fp32, s = scale_a[m] * scale_b[n] for fp8
operands and 1 for 16-bit ones.

The reference keeps c as a real operand of tt.dot (TritonDotPattern,
uTLXConversionPatterns.cpp:273, 290-291) and its AMD kernel chains it
through the K loop (accumulator = tl.dot(a, b, accumulator),
test_amd_gemm_pipelined.py:274, 292).  Integer-valued operands and
accumulators make every fp32 sum exact, so those cases must equal the exact
result bit for bit (fp32 out) or its round-to-nearest-even (bf16 / fp16 out,
the oracle's encoder); N(0,1) cases are held to the GEMM tolerances against
the oracle's fp64 sums.
"""
import ctypes

import numpy as np
import pytest
import torch

from test_gpu_gemm import BF16_TOL, FP8_TOL

pytestmark = pytest.mark.gpu

BF16, F16, F32 = 3, 6, 0
_TD = {BF16: torch.bfloat16, F16: torch.float16}
_OUT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
_OUT_FMT = {"bf16": BF16, "f16": F16}


def _int16(g, shape, fmt):
    x = g.integers(-3, 4, size=shape).astype(np.float32)
    if fmt == F16:
        return x, torch.from_numpy(x.astype(np.float16))
    return x, torch.from_numpy(x).to(torch.bfloat16)


# e4m3fn / e5m2 codes of the integers -3 .. 3
_FP8_INT = {1: {0: 0x00, 1: 0x38, 2: 0x40, 3: 0x44}, 2: {0: 0x00, 1: 0x3C, 2: 0x40, 3: 0x42}}


def _int8(g, shape, fmt):
    x = g.integers(-3, 4, size=shape)
    lut = _FP8_INT[fmt]
    codes = np.vectorize(lambda v: lut[abs(int(v))] | (0x80 if v < 0 else 0))(x).astype(np.uint8)
    return x.astype(np.float32), codes


def _exact_ref(x, out, oracle):
    """x float64 (exact) -> the expected output bits / values."""
    if out == "f32":
        return x.astype(np.float32)
    return oracle.encode_fmt(x.astype(np.float32), _OUT_FMT[out]).reshape(x.shape)


def _got(t, out):
    if out == "f32":
        return t.cpu().numpy()
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (17, 19, 23), (64, 64, 64), (300, 500, 4100), (1024, 1100, 256),
                                   (4096, 4096, 512), (255, 257, 1031)])
@pytest.mark.parametrize("fmt", [BF16, F16])
@pytest.mark.parametrize("out", ["f32", "bf16"])
def test_dot_acc_16bit_exact(tx, oracle, dev, M, N, K, fmt, out):
    """Shapes over one and many K splits, ragged and odd K (padded copies),
    and a full 16 x 16 grid of 256 x 128 tiles."""
    g = np.random.default_rng(M * 7 + N + K + fmt)
    a, at = _int16(g, (M, K), fmt)
    b, bt = _int16(g, (N, K), fmt)
    c = g.integers(-50, 51, size=(M, N)).astype(np.float32)
    D = tx.dot_acc(at.to(dev), bt.to(dev), torch.from_numpy(c).to(dev), out_dtype=_OUT[out])
    want = _exact_ref(a.astype(np.float64) @ b.astype(np.float64).T + c, out, oracle)
    got = _got(D, out)
    assert np.array_equal(got, want), np.argwhere(got != want)[:5]


@pytest.mark.parametrize("fa,fb", [(1, 1), (2, 2), (1, 2)])
@pytest.mark.parametrize("M,N,K", [(16, 48, 128), (300, 500, 4096), (1000, 1100, 1001), (4096, 4096, 256)])
def test_dot_acc_fp8_exact(tx, oracle, dev, fa, fb, M, N, K):
    """fp8 codes of -3 .. 3 with power-of-two scales: exact sums, fp32 out."""
    g = np.random.default_rng(M + N + K + 10 * fa + fb)
    a, aq = _int8(g, (M, K), fa)
    b, bq = _int8(g, (N, K), fb)
    sa = (2.0 ** g.integers(-2, 3, M)).astype(np.float32)
    sb = (2.0 ** g.integers(-2, 3, N)).astype(np.float32)
    c = g.integers(-50, 51, size=(M, N)).astype(np.float32)
    td = {1: torch.float8_e4m3fn, 2: torch.float8_e5m2}
    D = tx.dot_acc(torch.from_numpy(aq).to(dev).view(td[fa]), torch.from_numpy(bq).to(dev).view(td[fb]),
                   torch.from_numpy(c).to(dev), scale_a=torch.from_numpy(sa).to(dev),
                   scale_b=torch.from_numpy(sb).to(dev))
    want = (sa[:, None].astype(np.float64) * sb[None, :]) * (a.astype(np.float64) @ b.astype(np.float64).T) + c
    assert np.array_equal(D.cpu().numpy(), want.astype(np.float32))


@pytest.mark.parametrize("out", ["f32", "bf16", "f16"])
def test_dot_acc_fp8_normal(tx, oracle, dev, out):
    """The fp8 config operands (absmax-quantised N(0,1)) with an N(0,1)
    accumulator: the fp8 GEMM tolerance against the oracle's fp64 sum plus C."""
    import workloads
    M, N, K = 512, 4096, 2048
    aq, sa, bq, sb = workloads.fp8_gemm_input(M, N, K, seed_stream=91)
    c = np.random.default_rng(3).standard_normal((M, N)).astype(np.float32) * 30
    D = tx.dot_acc(torch.from_numpy(aq).to(dev).view(torch.float8_e4m3fn),
                   torch.from_numpy(bq).to(dev).view(torch.float8_e4m3fn), torch.from_numpy(c).to(dev),
                   scale_a=torch.from_numpy(sa).to(dev), scale_b=torch.from_numpy(sb).to(dev),
                   out_dtype=_OUT[out])
    got = D.float().cpu().numpy().astype(np.float64)
    r32, _ = oracle.gemm_fp8_scaled_rows(aq, bq, sa, sb, 0, M)
    ref = r32.astype(np.float64) + c
    scale = np.abs(ref).max()
    assert np.abs(got - ref).max() <= FP8_TOL * scale
    assert np.linalg.norm(got - ref) <= FP8_TOL * np.linalg.norm(ref)


def test_dot_acc_chained_k_loop_in_place(tx, oracle, dev):
    """The reference's loop: the accumulator carried through K chunks,
    D = dot(A[:, k0:k1], B[:, k0:k1], D) in place; the chained result equals
    the whole product (exact integer sums)."""
    g = np.random.default_rng(5)
    M, N, K = 512, 384, 1024
    a, at = _int16(g, (M, K), F16)
    b, bt = _int16(g, (N, K), F16)
    at, bt = at.to(dev), bt.to(dev)
    acc = torch.zeros((M, N), dtype=torch.float32, device=dev)
    for k0 in range(0, K, 256):
        tx.dot_acc(at[:, k0:k0 + 256], bt[:, k0:k0 + 256], acc, out=acc)
    want = (a.astype(np.float64) @ b.astype(np.float64).T).astype(np.float32)
    assert np.array_equal(acc.cpu().numpy(), want)


@pytest.mark.parametrize("fmt", [BF16, F16])
def test_dot_acc_kn_layout_and_no_acc(tx, oracle, dev, fmt):
    """b row-major K x N (the reference's matmul operand) with and without
    an accumulator, against the oracle's 16-bit GEMM (both layouts)."""
    g = np.random.default_rng(fmt)
    M, N, K = 700, 900, 600
    a, at = _int16(g, (M, K), fmt)
    b, bt = _int16(g, (K, N), fmt)
    c = g.integers(-50, 51, size=(M, N)).astype(np.float32)
    exact = a.astype(np.float64) @ b.astype(np.float64)
    D = tx.dot_acc(at.to(dev), bt.to(dev), torch.from_numpy(c).to(dev), b_layout="kn")
    assert np.array_equal(D.cpu().numpy(), (exact + c).astype(np.float32))
    E = tx.dot_acc(at.to(dev), bt.to(dev), b_layout="kn", out_dtype=_TD[fmt])
    bits = at.view(torch.int16).numpy().view(np.uint16), bt.view(torch.int16).numpy().view(np.uint16)
    _, r16 = oracle.gemm16_rows(bits[0], bits[1], 0, M, fmt, b_kn=True)
    assert np.array_equal(E.view(torch.int16).cpu().numpy().view(np.uint16), r16)


def test_dot_acc_normal_values_and_k_zero(tx, oracle, dev):
    """N(0,1) bf16 operands (the bf16 GEMM tolerance), and K = 0, where
    D = round(C)."""
    import workloads
    M, N, K = 600, 1000, 777
    A, B = workloads.bf16_gemm_input(M, N, K, seed_stream=8)
    c = np.random.default_rng(9).standard_normal((M, N)).astype(np.float32) * 10
    at = torch.from_numpy(A.view(np.int16)).to(dev).view(torch.bfloat16)
    bt = torch.from_numpy(B.view(np.int16)).to(dev).view(torch.bfloat16)
    D = tx.dot_acc(at, bt, torch.from_numpy(c).to(dev))
    r32, _ = oracle.gemm_bf16_rows(A, B, 0, M)
    ref = r32.astype(np.float64) + c
    got = D.cpu().numpy().astype(np.float64)
    assert np.abs(got - ref).max() <= BF16_TOL * np.abs(ref).max()
    Z = tx.dot_acc(at[:, :0], bt[:, :0], torch.from_numpy(c).to(dev), out_dtype=torch.bfloat16)
    want = oracle.encode_fmt(c, BF16).reshape(c.shape)
    assert np.array_equal(Z.view(torch.int16).cpu().numpy().view(np.uint16), want)


def test_dot_acc_table_op_and_errors(tx, oracle, dev):
    """The 17-operand tt.dot table form equals the typed entry point; a
    bf16 D on top of C, fp8 with a K x N B, and missing scales are errors."""
    g = np.random.default_rng(4)
    M, N, K = 96, 80, 64
    _, at = _int16(g, (M, K), BF16)
    _, bt = _int16(g, (N, K), BF16)
    at, bt = at.to(dev), bt.to(dev)
    c = torch.from_numpy(g.integers(-9, 10, size=(M, N)).astype(np.float32)).to(dev)
    D1 = tx.dot_acc(at, bt, c, out_dtype=torch.bfloat16)
    D2 = torch.empty_like(D1)
    V = tx._lib.TxValue
    ops = [V.ptr(D2.data_ptr()), V.ptr(at.data_ptr()), V.ptr(bt.data_ptr()), V.int(M), V.int(N), V.int(K),
           V.int(K), V.int(K), V.int(N), V.int(tx._lib.BF16), V.int(tx._lib.BF16), V.int(tx._lib.B_NK),
           V.ptr(c.data_ptr()), V.int(N), V.ptr(None), V.ptr(None), V.int(tx._lib.BF16)]
    arr = (V * len(ops))(*ops)
    assert tx.lib.txInvokeOp(b"tt.dot", arr, len(ops), None) == 0, tx._lib.last_error()
    torch.cuda.synchronize()
    assert torch.equal(D1.view(torch.int16), D2.view(torch.int16))
    L, lib = tx.lib, tx._lib
    st = L.tx_dot_acc(ctypes.c_void_p(at.data_ptr()), lib.BF16, K, None, ctypes.c_void_p(bt.data_ptr()),
                      lib.BF16, lib.B_NK, K, None, ctypes.c_void_p(c.data_ptr()), N,
                      ctypes.c_void_p(c.data_ptr()), lib.BF16, N, M, N, K, None)
    assert st == lib.INVALID_ARGUMENT and "only for an fp32 / int32 D" in lib.last_error()
    q = torch.zeros((M, K), dtype=torch.uint8, device=dev)
    s1 = torch.ones(M, dtype=torch.float32, device=dev)
    st = L.tx_dot_acc(ctypes.c_void_p(q.data_ptr()), lib.FP8E4M3FN, K, ctypes.c_void_p(s1.data_ptr()),
                      ctypes.c_void_p(q.data_ptr()), lib.FP8E4M3FN, lib.B_KN, M, ctypes.c_void_p(s1.data_ptr()),
                      None, 0, ctypes.c_void_p(D1.data_ptr()), lib.F32, N, M, M, K, None)
    assert st == lib.UNSUPPORTED
    st = L.tx_dot_acc(ctypes.c_void_p(q.data_ptr()), lib.FP8E4M3FN, K, None, ctypes.c_void_p(q.data_ptr()),
                      lib.FP8E4M3FN, lib.B_NK, K, None, None, 0, ctypes.c_void_p(D1.data_ptr()), lib.BF16, N,
                      M, N, K, None)
    assert st == lib.INVALID_ARGUMENT and "scale" in lib.last_error()


@pytest.mark.parametrize("M,N,K,pad", [(1, 1, 1, 0), (17, 19, 23, 0), (128, 128, 128, 0), (300, 500, 4100, 0),
                                       (1024, 1100, 256, 0), (255, 257, 1031, 1), (600, 700, 999, 3)])
def test_dot_int8_exact(tx, dev, M, N, K, pad):
    """tt.dot on int8 operands: exact int32 sums (v_mfma_i32_16x16x64_i8),
    plus an int32 accumulator; rows padded by `pad` bytes take the narrower
    loads (1 byte: any alignment)."""
    g = np.random.default_rng(M + N + K + pad)
    a = g.integers(-128, 128, (M, K), dtype=np.int64)
    b = g.integers(-128, 128, (N, K), dtype=np.int64)
    c = g.integers(-2**20, 2**20, (M, N)).astype(np.int32)

    def put(x):
        w = np.zeros((x.shape[0], x.shape[1] + pad), np.int8)
        w[:, :x.shape[1]] = x
        return torch.from_numpy(w).to(dev)[:, :x.shape[1]]

    D = tx.dot_acc(put(a), put(b), torch.from_numpy(c).to(dev))
    assert D.dtype == torch.int32
    want = (a @ b.T + c).astype(np.int64)
    assert np.array_equal(D.cpu().numpy().astype(np.int64), want)


def test_dot_int8_wraps_modulo_2_32(tx, dev):
    """int32 accumulation wraps: an accumulator near 2^31 plus positive sums."""
    M, N, K = 64, 64, 1024
    a = np.full((M, K), 127, np.int8)
    b = np.full((N, K), 127, np.int8)
    c = np.full((M, N), 2**31 - 1000, np.int32)
    D = tx.dot_acc(torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev), torch.from_numpy(c).to(dev))
    want = ((127 * 127 * K + (2**31 - 1000)) & 0xFFFFFFFF)
    want = want - 2**32 if want >= 2**31 else want
    assert np.all(D.cpu().numpy() == want)


@pytest.mark.parametrize("M,N,K", [(17, 19, 23), (300, 500, 1000), (1024, 1024, 1024), (513, 129, 77)])
def test_dot_fp32(tx, dev, M, N, K):
    """tt.dot on fp32 operands (input precision ieee): integer values give
    exact sums, bit for bit; N(0,1) values stay within K * 2^-23 of the
    float64 product relative to the sum of |products|."""
    g = np.random.default_rng(M + K)
    ai = g.integers(-8, 9, (M, K)).astype(np.float32)
    bi = g.integers(-8, 9, (N, K)).astype(np.float32)
    c = g.integers(-100, 101, (M, N)).astype(np.float32)
    D = tx.dot_acc(torch.from_numpy(ai).to(dev), torch.from_numpy(bi).to(dev), torch.from_numpy(c).to(dev))
    assert np.array_equal(D.cpu().numpy(), (ai.astype(np.float64) @ bi.astype(np.float64).T + c).astype(np.float32))
    an = g.standard_normal((M, K)).astype(np.float32)
    bn = g.standard_normal((N, K)).astype(np.float32)
    E = tx.dot_acc(torch.from_numpy(an).to(dev), torch.from_numpy(bn).to(dev)).cpu().numpy().astype(np.float64)
    ref = an.astype(np.float64) @ bn.astype(np.float64).T
    mag = np.abs(an.astype(np.float64)) @ np.abs(bn.astype(np.float64)).T
    assert np.all(np.abs(E - ref) <= K * 2.0 ** -23 * mag)
