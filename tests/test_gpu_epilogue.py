"""GPU parity: the fp8 GEMM's fused epilogue (tx_dot_fp8_scaled_ex) --
bias, relu / gelu (tanh) / silu and bf16 / fp16 / fp32 / fp8 outputs -- on
every path of the fp8 GEMM (256x256 and 256x128 tiles, split K, the column
tail strip, zero-padded operands, the skinny kernel, the generic kernel),
against the oracle's fp64 sums passed through the epilogue in float64.

Tolerance: the fp8 GEMM bar (max and Frobenius relative error <= 2e-2)
plus, per element, |gpu - ref| <= 5e-3 * max|ref| + r * |ref| with r the
output's rounding (2^-23 fp32, 2^-8 bf16, 2^-11 fp16, 2^-3 fp8 including
one code step), which a misplaced bias, a wrong activation or a wrong
column breaks.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

ACTS = {"none": 0, "relu": 1, "gelu_tanh": 2, "silu": 3}
OUT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32,
       "e4m3fn": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}
REL = {"f32": 2.0 ** -23, "bf16": 2.0 ** -8, "f16": 2.0 ** -11, "e4m3fn": 2.0 ** -3, "e5m2": 2.0 ** -2}


def _inputs(M, N, K, seed):
    import workloads
    aq, sa, bq, sb = workloads.fp8_gemm_input(M, N, K, seed_stream=seed)
    bias = np.random.default_rng(seed).standard_normal(N).astype(np.float32) * 3
    return aq, sa, bq, sb, bias


def _run(tx, dev, aq, sa, bq, sb, bias, act, out, out_scale):
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    C = tx.dot_scaled_rowcol(t(aq).view(torch.float8_e4m3fn), t(sa), t(bq).view(torch.float8_e4m3fn), t(sb),
                             bias=None if bias is None else t(bias), activation=act,
                             out_dtype=OUT[out], out_scale=out_scale)
    torch.cuda.synchronize()
    if out in ("e4m3fn", "e5m2"):
        return C.float().cpu().numpy().astype(np.float64) * out_scale
    return C.float().cpu().numpy().astype(np.float64)


def _check(got, ref, out, out_scale=1.0):
    fmax = {"e4m3fn": 448.0, "e5m2": 57344.0}.get(out)
    if fmax is not None:   # saturation: values past the range come back as +-max
        ref = np.clip(ref, -fmax * out_scale, fmax * out_scale)
    scale = np.abs(ref).max()
    assert np.abs(got - ref).max() <= 2e-2 * scale + REL[out] * scale
    assert np.linalg.norm(got - ref) <= (2e-2 + REL[out]) * np.linalg.norm(ref)
    bad = np.abs(got - ref) > 5e-3 * scale + REL[out] * np.abs(ref)
    assert not bad.any(), (int(bad.sum()), np.argwhere(bad)[:4], got[bad][:4], ref[bad][:4])


CASES = [
    # (M, N, K, act, out, bias, path)
    (1024, 1024, 512, "relu", "bf16", True, "256x256"),
    (1024, 1024, 512, "gelu_tanh", "f32", True, "256x256"),
    (1024, 1024, 512, "silu", "f16", False, "256x256"),
    (1024, 1024, 512, "none", "e4m3fn", True, "256x256"),
    (512, 2048, 4096, "gelu_tanh", "bf16", True, "256x128 split K"),
    (512, 2048, 4096, "relu", "e5m2", False, "256x128 split K"),
    (300, 500, 256, "silu", "f32", True, "256x128"),
    (8192, 2088, 256, "relu", "e4m3fn", True, "column strip"),
    (4352, 4096, 512, "silu", "bf16", True, "256x256, more tiles than CUs"),
    (4352, 4096, 512, "gelu_tanh", "bf16", False, "256x256, more tiles than CUs"),
    (4196, 4168, 384, "relu", "bf16", True, "256x256, partial tiles"),
    (8192, 2088, 256, "none", "bf16", True, "column strip, bf16 out"),
    (16, 1000, 512, "gelu_tanh", "bf16", True, "skinny"),
    (40, 3000, 640, "none", "e4m3fn", True, "skinny"),
    (1000, 1100, 1001, "silu", "bf16", True, "padded"),
    (100, 130, 1000, "relu", "f16", True, "generic"),
    (33, 65, 47, "gelu_tanh", "e4m3fn", False, "generic"),
]


@pytest.mark.parametrize("M,N,K,act,out,with_bias,path", CASES)
def test_epilogue(tx, oracle, dev, M, N, K, act, out, with_bias, path):
    aq, sa, bq, sb, bias = _inputs(M, N, K, M + N + K)
    bias = bias if with_bias else None
    out_scale = 0.25 if out in ("e4m3fn", "e5m2") else 1.0
    got = _run(tx, dev, aq, sa, bq, sb, bias, act, out, out_scale)
    rows = np.arange(M) if M * N * K <= 2 ** 31 else np.unique(np.r_[0, 1, M - 1, np.random.default_rng(0).integers(0, M, 12)])
    for r0 in rows if len(rows) < M else [None]:
        r = slice(0, M) if r0 is None else slice(r0, r0 + 1)
        acc, _ = oracle.gemm_fp8_scaled_rows(aq, bq, sa, sb, r.start, r.stop)
        ref = oracle.gemm_fp8_epilogue(acc, bias, ACTS[act])
        _check(got[r], ref, out, out_scale)


@pytest.mark.parametrize("act,with_bias", [("silu", True), ("gelu_tanh", False), ("relu", True)])
def test_bf16_output_equals_rounded_f32(tx, oracle, dev, act, with_bias):
    """Every bf16 output of the fused epilogue is the round-to-nearest-even
    of the fp32 output of the same product (the same tiles and sums, only
    the output cast differs): the whole output checked bit for bit."""
    M, N, K = 4352, 4096, 768
    aq, sa, bq, sb, bias = _inputs(M, N, K, 7 + ACTS[act])
    bias = bias if with_bias else None
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    args = (t(aq).view(torch.float8_e4m3fn), t(sa), t(bq).view(torch.float8_e4m3fn), t(sb))
    kw = dict(bias=None if bias is None else t(bias), activation=act)
    y16 = tx.dot_scaled_rowcol(*args, out_dtype=torch.bfloat16, **kw)
    y32 = tx.dot_scaled_rowcol(*args, out_dtype=torch.float32, **kw)
    a = y16.view(torch.int16).cpu().numpy()
    b = y32.to(torch.bfloat16).view(torch.int16).cpu().numpy()
    bad = np.argwhere(a != b)
    assert bad.size == 0, (len(bad), bad[:5].tolist())


def test_fp8_output_saturates(tx, oracle, dev):
    """A small out_scale drives y / out_scale past the fp8 range: the codes
    saturate at +-max, never NaN."""
    aq, sa, bq, sb, bias = _inputs(256, 256, 256, 5)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    C = tx.dot_scaled_rowcol(t(aq).view(torch.float8_e4m3fn), t(sa), t(bq).view(torch.float8_e4m3fn), t(sb),
                             bias=t(bias), out_dtype=torch.float8_e4m3fn, out_scale=1e-3)
    codes = C.view(torch.uint8).cpu().numpy()
    acc, _ = oracle.gemm_fp8_scaled_rows(aq, bq, sa, sb, 0, 256)
    y = (acc + bias[None, :]) / 1e-3
    big = np.abs(y) > 500
    assert big.any() and np.all((codes[big] & 0x7F) == 0x7E)
    assert not np.any((codes & 0x7F) == 0x7F)


def test_epilogue_table_op_and_errors(tx, oracle, dev):
    import struct
    from tx import _lib
    aq, sa, bq, sb, bias = _inputs(128, 256, 256, 9)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    A, B, SA, SB, BI = t(aq), t(bq), t(sa), t(sb), t(bias)
    C = torch.empty((128, 256), dtype=torch.float32, device=dev)
    bits = struct.unpack("<I", struct.pack("<f", 1.0))[0]
    tx.invoke("tx.dot_fp8_scaled_ex", [C, A, B, SA, SB, BI, 128, 256, 256, 256, 256, 256,
                                       _lib.FP8E4M3FN, _lib.FP8E4M3FN, _lib.F32, _lib.ACT_SILU, bits])
    torch.cuda.synchronize()
    acc, _ = oracle.gemm_fp8_scaled_rows(aq, bq, sa, sb, 0, 128)
    _check(C.cpu().numpy().astype(np.float64), oracle.gemm_fp8_epilogue(acc, bias, 3), "f32")
    with pytest.raises(tx.TxError):   # unknown activation
        tx.invoke("tx.dot_fp8_scaled_ex", [C, A, B, SA, SB, BI, 128, 256, 256, 256, 256, 256,
                                           _lib.FP8E4M3FN, _lib.FP8E4M3FN, _lib.F32, 9, bits])
    Cq = torch.empty((128, 256), dtype=torch.uint8, device=dev)
    with pytest.raises(tx.TxError):   # fp8 output without a positive scale
        tx.invoke("tx.dot_fp8_scaled_ex", [Cq, A, B, SA, SB, BI, 128, 256, 256, 256, 256, 256,
                                           _lib.FP8E4M3FN, _lib.FP8E4M3FN, _lib.FP8E4M3FN, 0, 0])
    with pytest.raises(ValueError):
        tx.dot_scaled_rowcol(A.view(torch.float8_e4m3fn), SA, B.view(torch.float8_e4m3fn), SB,
                             activation="tanh")
