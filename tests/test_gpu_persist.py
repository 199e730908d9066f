"""GPU parity of the persistent 4-wavefront GEMM tile (gemm_persist.h).

The library takes it for 256 x 256-tiled products with at least one tile per
CU (16-bit operands with fewer: 128 x 128, else 64 x 64 tiles, at least one
per CU), K a
whole number (>= 2) of 128-byte steps, N a multiple of 8 and a 16-byte
aligned C.  These shapes exercise what that tile adds over the
one-workgroup-per-tile kernel: workgroups that walk several tiles (tile
counts that are and are not a multiple of the CU count), the operand stream
crossing tile boundaries (the first steps of the next tile loaded during the
last ones of the current), partial row and column tiles read through
per-tile buffer ranges, the shortest K (two steps), stores dropped past M and
N, a strided C whose padding must stay untouched, every fp8 format pair and
every 16-bit operand / output pairing.  Every output element is checked
against the oracle (fp64 accumulation) with the tolerances of the GEMM tests
(fp8 2e-2, 16-bit 1e-2, plus the bf16 / fp16 ulp-distance bound).
"""
import numpy as np
import pytest
import torch

from test_gpu_gemm import BF16_TOL, FP8_TOL, _fp8_run, _np_bits, check_close

pytestmark = pytest.mark.gpu

_FP8 = {1: torch.float8_e4m3fn, 2: torch.float8_e5m2}


@pytest.mark.parametrize("M,N,K", [(4352, 4096, 256),    # 272 tiles: 16 workgroups take two
                                   (4196, 4168, 384),    # partial last row and column tiles
                                   (4096, 4096, 256),    # one tile per CU, two K steps
                                   (8192, 4608, 512)])   # 576 tiles: two or three per workgroup
def test_persist_fp8_full_output(tx, oracle, dev, M, N, K):
    import workloads
    aq, sa, bq, sb = workloads.fp8_gemm_input(M, N, K, seed_stream=M + N + K)
    C = _fp8_run(tx, dev, aq, sa, bq, sb)
    r32, r16 = oracle.gemm_fp8_scaled_rows(aq, bq, sa, sb, 0, M)
    check_close(C, r32, r16, FP8_TOL)
    # tile by tile: a misplaced or skipped tile cannot hide behind the others
    for m0 in range(0, M, 256):
        for n0 in range(0, N, 256):
            check_close(C[m0:m0 + 256, n0:n0 + 256], r32[m0:m0 + 256, n0:n0 + 256],
                        r16[m0:m0 + 256, n0:n0 + 256], FP8_TOL)


@pytest.mark.parametrize("fa,fb", [(2, 2), (1, 2), (2, 1)])
def test_persist_fp8_formats(tx, oracle, dev, fa, fb):
    import workloads
    M, N, K = 4352, 4096, 256
    aq, sa, bq, sb = workloads.fp8_gemm_input(M, N, K, seed_stream=31 + fa + 3 * fb)
    # e5m2 codes of the same values (the generator quantises to e4m3fn)
    if fa == 2:
        aq = oracle.encode(oracle.decode(aq, 1), 2, True)
    if fb == 2:
        bq = oracle.encode(oracle.decode(bq, 1), 2, True)
    C = _fp8_run(tx, dev, aq, sa, bq, sb, _FP8[fa], _FP8[fb])
    r32, r16 = oracle.gemm_fp8_scaled_rows(aq, bq, sa, sb, 0, M, fa, fb)
    check_close(C, r32, r16, FP8_TOL)


def test_persist_fp8_strided_out(tx, oracle, dev):
    """C a view with row pitch N + 64: every output lands in its row and the
    64 padding columns keep their contents."""
    import workloads
    M, N, K = 4352, 4096, 512
    aq, sa, bq, sb = workloads.fp8_gemm_input(M, N, K, seed_stream=41)
    buf = torch.full((M, N + 64), 0x7777, dtype=torch.int16, device=dev)
    out = buf.view(torch.bfloat16)[:, :N]
    tx.dot_scaled_rowcol(torch.from_numpy(aq).to(dev).view(torch.float8_e4m3fn), torch.from_numpy(sa).to(dev),
                         torch.from_numpy(bq).to(dev).view(torch.float8_e4m3fn), torch.from_numpy(sb).to(dev),
                         out=out)
    allb = buf.cpu().numpy().view(np.uint16)
    assert np.all(allb[:, N:] == 0x7777)
    r32, r16 = oracle.gemm_fp8_scaled_rows(aq, bq, sa, sb, 0, M)
    check_close(allb[:, :N], r32, r16, FP8_TOL)


@pytest.mark.parametrize("fmt,out_fmt", [(3, 3), (3, 6), (6, 6), (6, 3)])
@pytest.mark.parametrize("M,N,K", [(4352, 4096, 128), (4196, 4168, 192),
                                   # fewer 256 x 256 tiles than CUs: 128 x 128 tiles
                                   (2048, 2048, 256),    # one tile per CU
                                   (2100, 2056, 192),    # partial last row and column tiles
                                   (4096, 2048, 128),    # two tiles per workgroup, two K steps
                                   # fewer 128 x 128 tiles than CUs: 64 x 64 tiles
                                   (1024, 1024, 256),    # one tile per CU
                                   (1030, 1032, 192),    # partial last row and column tiles
                                   (2048, 1024, 128),    # two tiles per workgroup
                                   # fewer 64 x 64 tiles than CUs, at most 32 K steps
                                   (512, 512, 512), (200, 136, 1024)])
def test_persist_16bit_full_output(tx, oracle, dev, fmt, out_fmt, M, N, K):
    import workloads
    g = np.random.default_rng(fmt * 7 + out_fmt + M)
    codes = (lambda x: x.astype(np.float16).view(np.uint16)) if fmt == 6 else workloads.to_bf16_bits
    A = codes(g.standard_normal((M, K), dtype=np.float32))
    Bnk = codes(g.standard_normal((N, K), dtype=np.float32))
    td = torch.float16 if fmt == 6 else torch.bfloat16
    od = torch.float16 if out_fmt == 6 else torch.bfloat16
    a = torch.from_numpy(A.view(np.int16)).to(dev).view(td)
    b = torch.from_numpy(np.ascontiguousarray(Bnk).view(np.int16)).to(dev).view(td)
    C = _np_bits(tx.dot(a, b, out_dtype=od))
    r32, r16 = oracle.gemm16_rows(A, Bnk, 0, M, fmt, out_fmt=out_fmt)
    if out_fmt == 3:
        check_close(C, r32, r16, BF16_TOL)
    else:
        got = C.view(np.float16).astype(np.float64)
        ref = r32.astype(np.float64)
        scale = np.abs(ref).max()
        assert np.abs(got - ref).max() / scale <= BF16_TOL
        assert np.mean(C != r16) <= 0.05
    # tile by tile (blocks of 128 x 128, 64 x 64 for the small products:
    # within one tile of every size taken): a misplaced or skipped tile
    # cannot hide behind the others
    tb = 64 if M * N <= 1 << 22 else 128
    for m0 in range(0, M, tb):
        for n0 in range(0, N, tb):
            t = (slice(m0, m0 + tb), slice(n0, n0 + tb))
            if out_fmt == 3:
                check_close(C[t], r32[t], r16[t], BF16_TOL)
            else:
                ref = r32[t].astype(np.float64)
                got = C[t].view(np.float16).astype(np.float64)
                assert np.abs(got - ref).max() / np.abs(r32).max() <= BF16_TOL
