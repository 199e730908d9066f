"""GPU parity with non-finite fp8 operand codes, on every fp8 GEMM path and
the GEMV.

The decode of `tt.fp_to_fp` fixes what an fp8 code means: e4m3fn 0x7F / 0xFF
are NaN, e5m2 0x7C / 0xFC are +-Inf and 0x7D..0x7F (with either sign) NaN
(uTLXConversionPatterns.cpp:577 passes the op through; the fp8 `tt.dot`,
:227-296, computes on the decoded values).  So a product reading such a code
gives what fp32 arithmetic on the decoded values gives: NaN where a NaN is
read or an Inf meets a zero or an Inf of the other sign, +-Inf with the sign
of the product otherwise.  A few codes are planted in A rows, B columns and
W rows; every output of the checked rows must have the oracle's class (NaN,
+Inf, -Inf or finite), and the finite outputs must meet the fp8 GEMM bar.
"""
import numpy as np
import pytest
import torch

from test_gpu_gemm import FP8_TOL, bf16_f32, check_close, sample_rows, _np_bits, _t_bf16

pytestmark = pytest.mark.gpu

TD = {1: torch.float8_e4m3fn, 2: torch.float8_e5m2}
# non-finite codes per format: e4m3fn NaN (both signs); e5m2 +-Inf and NaNs
SPECIAL = {1: [0x7F, 0xFF], 2: [0x7C, 0xFC, 0x7D, 0xFE]}


def _codes(g, shape, fmt):
    top = 0x7F if fmt == 1 else 0x7C
    return g.integers(0, top, shape, dtype=np.uint8) | (g.integers(0, 2, shape, dtype=np.uint8) << 7)


def _plant(g, q, fmt, rows):
    """One non-finite code in each listed row of q (rows x K codes), at a random K."""
    for i, r in enumerate(rows):
        q[r, g.integers(0, q.shape[1])] = SPECIAL[fmt][i % len(SPECIAL[fmt])]


def check_classes(got_f32, ref, tol=FP8_TOL, got_bits=None, ref_bits=None):
    """Same NaN / +-Inf pattern as the oracle, finite outputs within tol."""
    got = np.asarray(got_f32, np.float64)
    ref = np.asarray(ref, np.float64)
    nan_g, nan_r = np.isnan(got), np.isnan(ref)
    assert np.array_equal(nan_g, nan_r), (np.argwhere(nan_g != nan_r)[:5], nan_r.sum(), nan_g.sum())
    inf_g, inf_r = np.isinf(got), np.isinf(ref)
    assert np.array_equal(inf_g, inf_r), (np.argwhere(inf_g != inf_r)[:5], inf_r.sum(), inf_g.sum())
    assert np.array_equal(np.signbit(got[inf_r]), np.signbit(ref[inf_r]))
    fin = np.isfinite(ref)
    assert nan_r.sum() + inf_r.sum() > 0, "nothing non-finite planted in the checked rows"
    if not fin.any():
        return
    if got_bits is not None:
        check_close(got_bits[fin][None], ref[fin][None].astype(np.float32), ref_bits[fin][None], tol)
    else:
        scale = np.abs(ref[fin]).max()
        assert np.abs(got[fin] - ref[fin]).max() <= tol * scale


def _case(seed, M, N, K, fa, fb):
    g = np.random.default_rng(seed)
    aq = _codes(g, (M, K), fa)
    bq = _codes(g, (N, K), fb)
    a_rows = sorted({0, M // 2, M - 1})
    b_rows = sorted({1 % N, N // 3, N - 1})
    _plant(g, aq, fa, a_rows)
    _plant(g, bq, fb, b_rows)
    sa = g.uniform(0.5, 2.0, M).astype(np.float32) * 1e-2
    sb = g.uniform(0.5, 2.0, N).astype(np.float32) * 1e-2
    rows = sorted(set(a_rows) | set(sample_rows(M, k=6, seed=seed)))
    return g, aq, bq, sa, sb, rows


def _dev(x, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    return t if dtype is None else t.view(dtype)


# Shapes and the path each takes on 256 CUs: skinny (M <= 64, K % 128 == 0),
# the persistent 256 x 256 tile (at least one tile per CU, two K steps), the
# 256 x 128 tile unsplit (few K steps) and with K split into fp32 partials
# summed by the reduce kernel, the zero-padded copies (odd K, >= 2^30
# multiply-adds) and the generic kernel (odd K, small).
PATHS = {"skinny": (16, 1000, 512), "persistent": (4096, 4096, 256), "n128": (512, 512, 256),
         "splitk": (300, 500, 8192), "padded": (1000, 1100, 1001), "generic": (100, 200, 300)}


@pytest.mark.parametrize("path", list(PATHS))
@pytest.mark.parametrize("fa,fb", [(1, 1), (2, 2), (2, 1)])
def test_fp8_dot_nonfinite(tx, oracle, dev, path, fa, fb):
    M, N, K = PATHS[path]
    g, aq, bq, sa, sb, rows = _case(list(PATHS).index(path) * 100 + fa * 10 + fb, M, N, K, fa, fb)
    C = _np_bits(tx.dot_scaled_rowcol(_dev(aq, dev, TD[fa]), _dev(sa, dev), _dev(bq, dev, TD[fb]),
                                      _dev(sb, dev)))
    for r in rows:
        r32, r16 = oracle.gemm_fp8_scaled_rows(aq, bq, sa, sb, r, r + 1, fa, fb)
        if np.all(np.isfinite(r32)):
            check_close(C[r:r + 1], r32, r16, FP8_TOL)
        else:
            check_classes(bf16_f32(C[r]), r32[0], got_bits=C[r], ref_bits=r16[0])


@pytest.mark.parametrize("path", ["skinny", "persistent", "generic"])
def test_fp8_dot_epilogue_nonfinite(tx, oracle, dev, path):
    """The fused epilogue (bias + relu -> bf16) on the 256 x 256 tile, and
    after the skinny / generic kernels' scaled sums: relu keeps NaN and
    +Inf, and sends -Inf to 0."""
    M, N, K = PATHS[path]
    fa = fb = 2
    g, aq, bq, sa, sb, rows = _case(77 + M, M, N, K, fa, fb)
    bias = g.standard_normal(N).astype(np.float32)
    C = tx.dot_scaled_rowcol(_dev(aq, dev, TD[fa]), _dev(sa, dev), _dev(bq, dev, TD[fb]), _dev(sb, dev),
                             bias=_dev(bias, dev), activation="relu")
    got = C.float().cpu().numpy()
    for r in rows:
        r32, _ = oracle.gemm_fp8_scaled_rows(aq, bq, sa, sb, r, r + 1, fa, fb)
        y = oracle.gemm_fp8_epilogue(r32.astype(np.float64), bias, oracle.ACT_RELU)[0]
        if np.all(np.isfinite(y)):
            assert np.abs(got[r] - y).max() <= FP8_TOL * max(np.abs(y).max(), 1e-30)
        else:
            check_classes(got[r], y)


@pytest.mark.parametrize("persistent", [False, True])
def test_fp8_grouped_nonfinite(tx, oracle, dev, persistent):
    """Grouped (mixture-of-experts) dot: the per-group tile, and the
    persistent kernel that walks every group's 256 x 256 tiles."""
    fa, fb = 2, 1
    g = np.random.default_rng(5 + persistent)
    sizes, N, K = ([300, 0, 17, 1500, 255, 900], 8192, 512) if persistent else ([300, 17, 1024], 384, 512)
    M = sum(sizes)
    off = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)
    aq = _codes(g, (M, K), fa)
    bq = _codes(g, (len(sizes), N, K), fb)
    a_rows = [int(off[p]) + sizes[p] // 2 for p in range(len(sizes)) if sizes[p]]
    _plant(g, aq, fa, a_rows)
    for p in range(len(sizes)):
        _plant(g, bq[p], fb, [p % N, N - 1 - p])
    sa = g.uniform(0.5, 2.0, M).astype(np.float32) * 1e-2
    sb = g.uniform(0.5, 2.0, (len(sizes), N)).astype(np.float32) * 1e-2
    C = _np_bits(tx.dot_scaled_rowcol_grouped(_dev(aq, dev, TD[fa]), _dev(sa, dev), _dev(bq, dev, TD[fb]),
                                              _dev(sb, dev), _dev(off, dev)))
    for p in range(len(sizes)):
        r0, r1 = int(off[p]), int(off[p + 1])
        if r1 == r0:
            continue
        rows = sorted({r0, r1 - 1, r0 + sizes[p] // 2})
        for r in rows:
            r32, r16 = oracle.gemm_fp8_scaled_rows(aq[r:r + 1], bq[p], sa[r:r + 1], sb[p], 0, 1, fa, fb)
            check_classes(bf16_f32(C[r]), r32[0], got_bits=C[r], ref_bits=r16[0])


def test_fp8_batched_nonfinite(tx, oracle, dev):
    fa, fb = 1, 2
    g = np.random.default_rng(11)
    Bt, M, N, K = 3, 200, 300, 256
    aq = _codes(g, (Bt, M, K), fa)
    bq = _codes(g, (Bt, N, K), fb)
    for p in range(Bt):
        _plant(g, aq[p], fa, [p, M - 1])
        _plant(g, bq[p], fb, [2 * p, N - 2])
    sa = g.uniform(0.5, 2.0, (Bt, M)).astype(np.float32) * 1e-2
    sb = g.uniform(0.5, 2.0, (Bt, N)).astype(np.float32) * 1e-2
    C = _np_bits(tx.dot_scaled_rowcol_batched(_dev(aq, dev, TD[fa]), _dev(sa, dev), _dev(bq, dev, TD[fb]),
                                              _dev(sb, dev)))
    for p in range(Bt):
        for r in (p, M - 1, 17):
            r32, r16 = oracle.gemm_fp8_scaled_rows(aq[p], bq[p], sa[p], sb[p], r, r + 1, fa, fb)
            check_classes(bf16_f32(C[p, r]), r32[0], got_bits=C[p, r], ref_bits=r16[0])


@pytest.mark.parametrize("M,N,K", [(256, 256, 512), (300, 700, 1024)])
def test_mx_dot_nonfinite(tx, oracle, dev, M, N, K):
    """tt.dot_scaled (e8m0 block scales) with fp8 operands holding NaN / Inf
    codes; scales near 2^0 so every finite product stays in range."""
    fa, fb = 2, 1
    g = np.random.default_rng(M + K)
    aq = _codes(g, (M, K), fa)
    bq = _codes(g, (N, K), fb)
    _plant(g, aq, fa, [0, M // 2, M - 1])
    _plant(g, bq, fb, [3, N - 1])
    sa = g.integers(120, 128, (M, K // 32), dtype=np.uint8)
    sb = g.integers(120, 128, (N, K // 32), dtype=np.uint8)
    C = tx.dot_scaled(_dev(aq, dev, TD[fa]), _dev(sa, dev), _dev(bq, dev, TD[fb]), _dev(sb, dev),
                      out_dtype=torch.float32)
    got = C.cpu().numpy()
    for r in sorted({0, 1, M // 2, M - 1}):
        r32, _ = oracle.gemm_mx_rows(aq, sa, bq, sb, r, r + 1, fa, fb)
        check_classes(got[r], r32[0])


@pytest.mark.parametrize("M", [1, 4, 16])
@pytest.mark.parametrize("fmt", [2, 1])
def test_gemv_nonfinite(tx, oracle, dev, M, fmt):
    """The dequant GEMV at the decode shape (N = 14336, K = 4096): NaN / Inf
    weight codes in some W rows, and a bf16 Inf and NaN in x, give the
    oracle's classes for every M (M = 1 on the streaming kernel, 4 and 16 on
    the MFMA kernel whose bit-placement decode needs the non-finite path)."""
    N, K, group = 14336, 4096, 128
    g = np.random.default_rng(M * 10 + fmt)
    x = oracle.f32_to_bf16(g.standard_normal((M, K)).astype(np.float32))
    wq = _codes(g, (N, K), fmt)
    w_rows = [0, 5, 4097, 8000, N - 1]
    _plant(g, wq, fmt, w_rows)
    if M > 1:
        x[1, 17] = 0x7F80      # +Inf
    x[M - 1, 300] = 0x7FC0     # NaN: row M-1 all NaN
    s = g.uniform(0.1, 1.0, size=(N, K // group)).astype(np.float32) * 1e-3
    y = _np_bits(tx.gemv_fp8_dequant(_t_bf16(x, dev), _dev(wq, dev, TD[fmt]), _dev(s, dev), group=group))
    r32, r16 = oracle.gemv_fp8_dequant(x, wq, s, group=group, fmt_w=fmt)
    check_classes(bf16_f32(y), r32, got_bits=y, ref_bits=r16)
    assert np.all(np.isnan(bf16_f32(y[M - 1])))
