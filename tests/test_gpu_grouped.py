"""GPU parity: the grouped (mixture-of-experts) and batched fp8 scaled dots
(tx_dot_fp8_scaled_grouped / _batched) against the oracle, group by group,
at the fp8 GEMM bar (2e-2 max and Frobenius, plus the bf16 ulp check).
Uneven and empty groups, groups not a multiple of the 256-row tile, rows
outside every group left untouched, strided batches, and a single group
that must reproduce the plain product bit for bit (same tile, same K
order)."""
import numpy as np
import pytest
import torch

from test_gpu_gemm import FP8_TOL, check_close, sample_rows

pytestmark = pytest.mark.gpu

TD = {1: torch.float8_e4m3fn, 2: torch.float8_e5m2}
ONE = 0x3F800000   # 1.0f as an fp32 bit pattern (the table ops' c_scale operand)


def _codes(g, shape, fmt):
    top = 0x7F if fmt == 1 else 0x7C
    return g.integers(0, top, shape, dtype=np.uint8) | (g.integers(0, 2, shape, dtype=np.uint8) << 7)


def _bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def _grouped_case(g, sizes, N, K, fa, fb, lead=0, tail=0):
    M = lead + sum(sizes) + tail
    off = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32) + lead
    aq = _codes(g, (M, K), fa)
    bq = _codes(g, (len(sizes), N, K), fb)
    sa = g.uniform(0.5, 2.0, M).astype(np.float32)
    sb = g.uniform(0.5, 2.0, (len(sizes), N)).astype(np.float32)
    return M, off, aq, bq, sa, sb


def _run_grouped(tx, dev, aq, bq, sa, sb, off, fa, fb, out=None):
    return tx.dot_scaled_rowcol_grouped(
        torch.from_numpy(aq).to(dev).view(TD[fa]), torch.from_numpy(sa).to(dev),
        torch.from_numpy(bq).to(dev).view(TD[fb]), torch.from_numpy(sb).to(dev),
        torch.from_numpy(off).to(dev), out=out)


@pytest.mark.parametrize("sizes,N,K,fa,fb", [
    ([300, 0, 17, 1024, 255], 384, 512, 1, 1), ([300, 0, 17, 1024, 255], 384, 512, 2, 1),
    ([1, 2, 3, 257], 96, 128, 1, 2), ([0, 0, 0, 512], 256, 1040, 2, 2), ([640] * 6, 1000, 256, 1, 1)])
def test_grouped_uneven_groups(tx, oracle, dev, sizes, N, K, fa, fb):
    g = np.random.default_rng(sum(sizes) + N + K + fa)
    M, off, aq, bq, sa, sb = _grouped_case(g, sizes, N, K, fa, fb)
    C = _run_grouped(tx, dev, aq, bq, sa, sb, off, fa, fb)
    torch.cuda.synchronize()
    got = _bits(C)
    for p in range(len(sizes)):
        r0, r1 = int(off[p]), int(off[p + 1])
        if r1 == r0:
            continue
        r32, r16 = oracle.gemm_fp8_scaled_rows(aq[r0:r1], bq[p], sa[r0:r1], sb[p], 0, r1 - r0, fa, fb)
        check_close(got[r0:r1], r32, r16, FP8_TOL)


def test_grouped_rows_outside_groups_untouched(tx, oracle, dev):
    """Offsets starting past row 0 and ending before M: those rows keep
    what the caller had in C."""
    g = np.random.default_rng(4)
    M, off, aq, bq, sa, sb = _grouped_case(g, [36, 200], 130, 256, 1, 1, lead=64, tail=100)
    C = torch.full((M, 130), 7.0, dtype=torch.bfloat16, device=dev)
    _run_grouped(tx, dev, aq, bq, sa, sb, off, 1, 1, out=C)
    got = _bits(C)
    seven = np.uint16(0x40E0)
    assert np.all(got[:64] == seven) and np.all(got[300:] == seven)
    for p in range(2):
        r0, r1 = int(off[p]), int(off[p + 1])
        r32, r16 = oracle.gemm_fp8_scaled_rows(aq[r0:r1], bq[p], sa[r0:r1], sb[p], 0, r1 - r0)
        check_close(got[r0:r1], r32, r16, FP8_TOL)


@pytest.mark.parametrize("N,K,fa,fb", [(1000, 256, 1, 1), (2048, 512, 2, 1)])
def test_grouped_many_small_experts(tx, oracle, dev, N, K, fa, fb):
    """64 experts of 0..200 rows (under 192 on average): the transposed tile
    (a group's rows along the tile's 128-wide side, C stored transposed),
    including empty groups and a ragged N."""
    g = np.random.default_rng(N + K)
    sizes = list(g.integers(0, 200, 64))
    sizes[5] = sizes[40] = 0
    M, off, aq, bq, sa, sb = _grouped_case(g, sizes, N, K, fa, fb)
    got = _bits(_run_grouped(tx, dev, aq, bq, sa, sb, off, fa, fb))
    for p in range(64):
        r0, r1 = int(off[p]), int(off[p + 1])
        if r1 > r0:
            r32, r16 = oracle.gemm_fp8_scaled_rows(aq[r0:r1], bq[p], sa[r0:r1], sb[p], 0, r1 - r0, fa, fb)
            check_close(got[r0:r1], r32, r16, FP8_TOL)


def test_grouped_small_rows_outside_groups_untouched(tx, oracle, dev):
    """The transposed tile writes only the groups' rows."""
    g = np.random.default_rng(5)
    M, off, aq, bq, sa, sb = _grouped_case(g, [36, 20], 130, 256, 1, 1, lead=64, tail=100)
    C = torch.full((M, 130), 7.0, dtype=torch.bfloat16, device=dev)
    _run_grouped(tx, dev, aq, bq, sa, sb, off, 1, 1, out=C)
    got = _bits(C)
    seven = np.uint16(0x40E0)
    assert np.all(got[:64] == seven) and np.all(got[120:] == seven)
    for p in range(2):
        r0, r1 = int(off[p]), int(off[p + 1])
        r32, r16 = oracle.gemm_fp8_scaled_rows(aq[r0:r1], bq[p], sa[r0:r1], sb[p], 0, r1 - r0)
        check_close(got[r0:r1], r32, r16, FP8_TOL)


def test_grouped_large_big_tiles(tx, oracle, dev):
    """8 experts x 1024 rows, N = 4096, K = 1024: 256 x 256 tiles; sampled
    rows of every group against the oracle."""
    g = np.random.default_rng(8)
    M, off, aq, bq, sa, sb = _grouped_case(g, [1024] * 8, 4096, 1024, 1, 1)
    got = _bits(_run_grouped(tx, dev, aq, bq, sa, sb, off, 1, 1))
    for p in range(8):
        r0 = int(off[p])
        rows = [r0 + r for r in sample_rows(1024, k=6, seed=p)]
        for r in rows:
            r32, r16 = oracle.gemm_fp8_scaled_rows(aq[r:r + 1], bq[p], sa[r:r + 1], sb[p], 0, 1)
            check_close(got[r:r + 1], r32, r16, FP8_TOL)


@pytest.mark.parametrize("fa,fb", [(1, 1), (2, 1)])
def test_grouped_persistent_uneven(tx, oracle, dev, fa, fb):
    """Groups of uneven, empty and non-multiple-of-256 sizes with enough
    256 x 256 tiles for the persistent kernel (each workgroup walks the real
    tiles of every group): every row of every group against the oracle, the
    rows before and after the groups untouched."""
    g = np.random.default_rng(30 + fa)
    sizes = [300, 0, 17, 1500, 255, 900]
    M, off, aq, bq, sa, sb = _grouped_case(g, sizes, 8192, 512, fa, fb, lead=40, tail=70)
    C = torch.full((M, 8192), 7.0, dtype=torch.bfloat16, device=dev)
    _run_grouped(tx, dev, aq, bq, sa, sb, off, fa, fb, out=C)
    got = _bits(C)
    seven = np.uint16(0x40E0)
    assert np.all(got[:40] == seven) and np.all(got[M - 70:] == seven)
    for p in range(len(sizes)):
        r0, r1 = int(off[p]), int(off[p + 1])
        if r1 > r0:
            r32, r16 = oracle.gemm_fp8_scaled_rows(aq[r0:r1], bq[p], sa[r0:r1], sb[p], 0, r1 - r0, fa, fb)
            check_close(got[r0:r1], r32, r16, FP8_TOL)


def test_single_group_equals_plain_product(tx, dev):
    """One group over all rows runs the plain product's 256 x 256 tile with
    the same K order: bit-identical output."""
    g = np.random.default_rng(12)
    M, off, aq, bq, sa, sb = _grouped_case(g, [4096], 4096, 1024, 1, 1)
    C1 = _run_grouped(tx, dev, aq, bq, sa, sb, off, 1, 1)
    C2 = tx.dot_scaled_rowcol(torch.from_numpy(aq).to(dev).view(TD[1]), torch.from_numpy(sa).to(dev),
                              torch.from_numpy(bq[0]).to(dev).view(TD[1]), torch.from_numpy(sb[0]).to(dev))
    assert torch.equal(C1.view(torch.int16), C2.view(torch.int16))


@pytest.mark.parametrize("Bt,M,N,K,rows_alloc", [(3, 300, 500, 256, 320), (4, 1024, 1024, 2048, 1024),
                                                 (2, 1, 64, 16, 8)])
def test_batched(tx, oracle, dev, Bt, M, N, K, rows_alloc):
    """Batches as slices of wider allocations (batch stride != M * K)."""
    g = np.random.default_rng(Bt * M + K)
    aq = _codes(g, (Bt, rows_alloc, K), 1)
    bq = _codes(g, (Bt, N, K), 2)
    sa = g.uniform(0.5, 2.0, (Bt, rows_alloc)).astype(np.float32)
    sb = g.uniform(0.5, 2.0, (Bt, N)).astype(np.float32)
    A = torch.from_numpy(aq).to(dev).view(TD[1])[:, :M]
    SA = torch.from_numpy(sa).to(dev)[:, :M]
    C = tx.dot_scaled_rowcol_batched(A, SA, torch.from_numpy(bq).to(dev).view(TD[2]), torch.from_numpy(sb).to(dev))
    torch.cuda.synchronize()
    got = _bits(C)
    for p in range(Bt):
        rows = sample_rows(M, k=40, seed=p) if M > 256 else list(range(M))
        r32, r16 = oracle.gemm_fp8_scaled_rows(aq[p, :M][rows], bq[p], sa[p, :M][rows], sb[p], 0, len(rows), 1, 2)
        check_close(got[p][rows], r32, r16, FP8_TOL)


def test_grouped_table_ops_and_errors(tx, oracle, dev):
    from tx import _lib
    g = np.random.default_rng(3)
    M, off, aq, bq, sa, sb = _grouped_case(g, [40, 88], 64, 128, 1, 1)
    A = torch.from_numpy(aq).to(dev)
    B = torch.from_numpy(bq).to(dev)
    SA, SB = torch.from_numpy(sa).to(dev), torch.from_numpy(sb).to(dev)
    O = torch.from_numpy(off).to(dev)
    C = torch.empty((M, 64), dtype=torch.bfloat16, device=dev)
    tx.invoke("tx.dot_fp8_scaled_grouped", [C, A, B, SA, SB, O, None, 2, M, 64, 128, 128, 128, 64, 64 * 128, 64,
                                            0, _lib.FP8E4M3FN, _lib.FP8E4M3FN, _lib.BF16, 0, ONE])
    C2 = torch.empty((2, 64, 64), dtype=torch.bfloat16, device=dev)
    tx.invoke("tx.dot_fp8_scaled_batched", [C2, A, B, SA, SB, 2, 64, 64, 128, 128, 128, 64, 64 * 128, 64,
                                            64 * 128, 64, 64 * 64, _lib.FP8E4M3FN, _lib.FP8E4M3FN])
    torch.cuda.synchronize()
    got = _bits(C)
    for p in range(2):
        r0, r1 = int(off[p]), int(off[p + 1])
        r32, r16 = oracle.gemm_fp8_scaled_rows(aq[r0:r1], bq[p], sa[r0:r1], sb[p], 0, r1 - r0)
        check_close(got[r0:r1], r32, r16, FP8_TOL)
        r32, r16 = oracle.gemm_fp8_scaled_rows(aq[64 * p:64 * p + 64], bq[p], sa[64 * p:64 * p + 64], sb[p], 0, 64)
        check_close(_bits(C2[p]), r32, r16, FP8_TOL)
    with pytest.raises(tx.TxError):   # K not a multiple of 16 bytes
        tx.invoke("tx.dot_fp8_scaled_grouped", [C, A, B, SA, SB, O, None, 2, M, 64, 120, 128, 128, 64, 64 * 128,
                                                64, 0, _lib.FP8E4M3FN, _lib.FP8E4M3FN, _lib.BF16, 0, ONE])
    with pytest.raises(tx.TxError):   # NULL offsets
        tx.invoke("tx.dot_fp8_scaled_grouped", [C, A, B, SA, SB, None, None, 2, M, 64, 128, 128, 128, 64,
                                                64 * 128, 64, 0, _lib.FP8E4M3FN, _lib.FP8E4M3FN, _lib.BF16, 0, ONE])
    with pytest.raises(tx.TxError):   # unknown activation
        tx.invoke("tx.dot_fp8_scaled_grouped", [C, A, B, SA, SB, O, None, 2, M, 64, 128, 128, 128, 64, 64 * 128,
                                                64, 0, _lib.FP8E4M3FN, _lib.FP8E4M3FN, _lib.BF16, 9, ONE])
    with pytest.raises(ValueError):   # offsets of the wrong length
        tx.dot_scaled_rowcol_grouped(A.view(TD[1]), SA, B.view(TD[1]), SB, O[:2])


EPI_OUT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32, "e4m3fn": torch.float8_e4m3fn,
           "e5m2": torch.float8_e5m2}
EPI_REL = {"f32": 2.0 ** -23, "bf16": 2.0 ** -8, "f16": 2.0 ** -11, "e4m3fn": 2.0 ** -3, "e5m2": 2.0 ** -2}
EPI_ACT = {"none": 0, "relu": 1, "gelu_tanh": 2, "silu": 3}


@pytest.mark.parametrize("sizes,N,K,act,out,with_bias", [
    ([300, 0, 17, 1024, 255], 384, 512, "silu", "bf16", True),
    ([300, 0, 17, 1024, 255], 384, 512, "gelu_tanh", "e4m3fn", True),
    ([1024] * 8, 2048, 512, "relu", "f32", True),
    ([640, 5, 700], 1000, 256, "none", "e5m2", False),
    ([129, 64], 96, 128, "gelu_tanh", "f16", True)])
def test_grouped_fused_epilogue(tx, oracle, dev, sizes, N, K, act, out, with_bias):
    """Per-expert bias, activation and output cast fused into the grouped
    product (256x256 and 256x128 tiles), against the oracle's fp64 sums of
    each group through the epilogue in float64: the fp8 GEMM bar plus, per
    element, 5e-3 of the output scale and the output type's rounding.
    Operands are absmax-quantised N(0,1) values (the fp8 GEMM workload), so
    outputs are O(1) and fp32 accumulation error stays far below the bound;
    raw random codes make near-cancelling sums of 1e5-sized terms whose fp32
    error the bound, relative to the saturated output scale, cannot hold."""
    import workloads
    g = np.random.default_rng(sum(sizes) + N + EPI_ACT[act])
    M = sum(sizes)
    off = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)
    aq, sa, bq, sb = workloads.fp8_gemm_input(M, len(sizes) * N, K, seed_stream=M + N)
    bq = bq.reshape(len(sizes), N, K)
    sb = sb.reshape(len(sizes), N)
    bias = (g.standard_normal((len(sizes), N)) * 3).astype(np.float32) if with_bias else None
    out_scale = 0.25 if out in ("e4m3fn", "e5m2") else 1.0
    C = tx.dot_scaled_rowcol_grouped(
        torch.from_numpy(aq).to(dev).view(TD[1]), torch.from_numpy(sa).to(dev),
        torch.from_numpy(bq).to(dev).view(TD[1]), torch.from_numpy(sb).to(dev), torch.from_numpy(off).to(dev),
        bias=None if bias is None else torch.from_numpy(bias).to(dev), activation=act, out_dtype=EPI_OUT[out],
        out_scale=out_scale)
    torch.cuda.synchronize()
    got = C.float().cpu().numpy().astype(np.float64) * (out_scale if out in ("e4m3fn", "e5m2") else 1.0)
    fmax = {"e4m3fn": 448.0, "e5m2": 57344.0}.get(out)
    for p in range(len(sizes)):
        r0, r1 = int(off[p]), int(off[p + 1])
        if r1 == r0:
            continue
        acc, _ = oracle.gemm_fp8_scaled_rows(aq[r0:r1], bq[p], sa[r0:r1], sb[p], 0, r1 - r0)
        ref = oracle.gemm_fp8_epilogue(acc, None if bias is None else bias[p], EPI_ACT[act])
        if fmax is not None:
            ref = np.clip(ref, -fmax * out_scale, fmax * out_scale)
        gg = got[r0:r1]
        scale = np.abs(ref).max()
        assert np.abs(gg - ref).max() <= (2e-2 + EPI_REL[out]) * scale
        bad = np.abs(gg - ref) > 5e-3 * scale + EPI_REL[out] * np.abs(ref)
        assert not bad.any(), (p, int(bad.sum()), gg[bad][:4], ref[bad][:4])
