"""GPU parity: the absmax + fp8 quantisers (tx_quantize_mx, tx_quantize_rowwise)
against the oracle, bit for bit (codes and scales), on the vector and the
scalar paths, fp32 and bf16 inputs, both fp8 formats, special values, and
the full 8192 x 8192 size; then quantise -> GEMM round trips: the fp8 GEMM
bar (2e-2) against the float64 product of the dequantised operands, and the
quantisation-noise bound against the unquantised product."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

TD = {1: torch.float8_e4m3fn, 2: torch.float8_e5m2}
FMAX = {1: 448.0, 2: 57344.0}


def _x(g, rows, K, specials=False):
    x = (g.standard_normal((rows, K)) * np.exp2(g.integers(-30, 30, (rows, 1)))).astype(np.float32)
    if specials and x.size >= 64:
        flat = x.reshape(-1)
        pos = g.choice(flat.size, size=min(40, flat.size // 8), replace=False)
        vals = np.array([np.nan, -np.nan, np.inf, -np.inf, 0.0, -0.0, 1e-40, -3e-39,
                         2.0 ** 120, FMAX[1], -FMAX[2], 5e-45], np.float32)
        flat[pos] = vals[np.arange(pos.size) % vals.size]
    return x


def _dev(x, xt, dev, ldx=None):
    t = torch.from_numpy(x)
    if xt == "bf16":
        t = t.to(torch.bfloat16)
    if ldx is not None and ldx != x.shape[1]:
        w = torch.zeros((x.shape[0], ldx), dtype=t.dtype)
        w[:, :x.shape[1]] = t
        return w.to(dev)[:, :x.shape[1]], t
    return t.to(dev), t


def _host_x(t):
    """What the oracle takes: fp32 values or bf16 bits."""
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


@pytest.mark.parametrize("rows,K", [(1, 32), (7, 96), (64, 4096), (300, 1024), (2, 8192 + 32)])
@pytest.mark.parametrize("xt", ["f32", "bf16"])
@pytest.mark.parametrize("fmt", [1, 2])
def test_quantize_mx_exact(tx, oracle, dev, rows, K, xt, fmt):
    g = np.random.default_rng(rows * 31 + K + fmt)
    xd, xh = _dev(_x(g, rows, K, specials=True), xt, dev)
    q, s = tx.quantize_mx(xd, TD[fmt])
    torch.cuda.synchronize()
    rq, rs = oracle.quant_mx(_host_x(xh), fmt)
    assert np.array_equal(s.cpu().numpy(), rs)
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), rq)


@pytest.mark.parametrize("rows,K", [(1, 1), (5, 300), (64, 4096), (3, 100003), (1000, 64)])
@pytest.mark.parametrize("xt", ["f32", "bf16"])
@pytest.mark.parametrize("fmt", [1, 2])
def test_quantize_rowwise_exact(tx, oracle, dev, rows, K, xt, fmt):
    g = np.random.default_rng(rows * 17 + K + fmt)
    xd, xh = _dev(_x(g, rows, K, specials=True), xt, dev)
    q, s = tx.quantize_rowwise(xd, TD[fmt])
    torch.cuda.synchronize()
    rq, rs = oracle.quant_rowwise(_host_x(xh), fmt)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), rs.view(np.uint32))
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), rq)


@pytest.mark.parametrize("xt", ["f32", "bf16"])
def test_quantize_strided_rows_take_the_scalar_path(tx, oracle, dev, xt):
    """Row pitches that break the vector path's alignment (ldx odd) give the
    same bytes as the oracle."""
    g = np.random.default_rng(5)
    rows, K = 33, 320
    x = _x(g, rows, K, specials=True)
    for ldx in (K + 8, K + 1):
        xd, xh = _dev(x, xt, dev, ldx=ldx)
        q, s = tx.quantize_mx(xd, TD[1])
        rq, rs = oracle.quant_mx(_host_x(xh), 1)
        assert np.array_equal(q.view(torch.uint8).cpu().numpy(), rq) and np.array_equal(s.cpu().numpy(), rs)
        q2, s2 = tx.quantize_rowwise(xd, TD[2])
        rq2, rs2 = oracle.quant_rowwise(_host_x(xh), 2)
        assert np.array_equal(q2.view(torch.uint8).cpu().numpy(), rq2)
        assert np.array_equal(s2.cpu().numpy().view(np.uint32), rs2.view(np.uint32))


def test_quantize_full_size(tx, oracle, dev):
    """8192 x 8192 bf16: MX and row-wise, every byte."""
    g = np.random.default_rng(8)
    x = g.standard_normal((8192, 8192), dtype=np.float32)
    xd, xh = _dev(x, "bf16", dev)
    del x
    q, s = tx.quantize_mx(xd, TD[1])
    rq, rs = oracle.quant_mx(_host_x(xh), 1)
    assert np.array_equal(s.cpu().numpy(), rs) and np.array_equal(q.view(torch.uint8).cpu().numpy(), rq)
    q, s = tx.quantize_rowwise(xd, TD[1])
    rq, rs = oracle.quant_rowwise(_host_x(xh), 1)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), rs.view(np.uint32))
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), rq)


@pytest.mark.parametrize("M,N,K", [(256, 384, 1024), (1000, 700, 2048)])
def test_quantise_then_gemm(tx, oracle, dev, M, N, K):
    """fp32 operands -> quantisers -> the scaled GEMMs.  Against the float64
    product of the dequantised operands the fp8 GEMM bar holds (2e-2, max and
    Frobenius); against the unquantised product the error is e4m3's
    quantisation noise (3 mantissa bits: about 2^-4 / sqrt(3) per factor,
    ~5% Frobenius for products of two quantised values), bounded at 8%."""
    g = np.random.default_rng(M + N)
    a = g.standard_normal((M, K)).astype(np.float32)
    b = g.standard_normal((N, K)).astype(np.float32)
    exact = a.astype(np.float64) @ b.astype(np.float64).T
    A = torch.from_numpy(a).to(dev)
    B = torch.from_numpy(b).to(dev)

    def deq(q, fmt=1):
        return oracle.decode(q.view(torch.uint8).cpu().numpy().reshape(-1), fmt).astype(np.float64).reshape(q.shape)

    qa, sa = tx.quantize_rowwise(A)
    qb, sb = tx.quantize_rowwise(B)
    c1 = tx.dot_scaled_rowcol(qa, sa, qb, sb).float().cpu().numpy()
    ref1 = (deq(qa) * sa.cpu().numpy()[:, None]) @ (deq(qb) * sb.cpu().numpy()[:, None]).T
    ma, ea = tx.quantize_mx(A)
    mb, eb = tx.quantize_mx(B)
    c2 = tx.dot_scaled(ma, ea, mb, eb, out_dtype=torch.float32).cpu().numpy()
    sx = lambda e: np.repeat(np.exp2(e.cpu().numpy().astype(np.float64) - 127), 32, axis=1)
    ref2 = (deq(ma) * sx(ea)) @ (deq(mb) * sx(eb)).T
    for c, ref in ((c1, ref1), (c2, ref2)):
        rel = np.abs(c - ref).max() / np.abs(ref).max()
        fro = np.linalg.norm(c - ref) / np.linalg.norm(ref)
        assert rel <= 2e-2 and fro <= 2e-2, (rel, fro)
        assert np.linalg.norm(c - exact) / np.linalg.norm(exact) <= 0.08


def test_quantise_table_ops_and_errors(tx, oracle, dev):
    from tx import _lib
    g = np.random.default_rng(2)
    rows, K = 16, 256
    x = _x(g, rows, K)
    X = torch.from_numpy(x).to(dev)
    q = torch.empty((rows, K), dtype=torch.uint8, device=dev)
    s = torch.empty((rows, K // 32), dtype=torch.uint8, device=dev)
    tx.invoke("tx.quantize_mx", [q, s, X, rows, K, K, K, K // 32, _lib.F32, _lib.FP8E4M3FN])
    torch.cuda.synchronize()
    rq, rs = oracle.quant_mx(x, 1)
    assert np.array_equal(q.cpu().numpy(), rq) and np.array_equal(s.cpu().numpy(), rs)
    sf = torch.empty((rows,), dtype=torch.float32, device=dev)
    tx.invoke("tx.quantize_rowwise", [q, sf, X, rows, K, K, K, _lib.F32, _lib.FP8E5M2])
    torch.cuda.synchronize()
    rq, rs = oracle.quant_rowwise(x, 2)
    assert np.array_equal(q.cpu().numpy(), rq) and np.array_equal(sf.cpu().numpy(), rs)
    with pytest.raises(tx.TxError):   # K not a multiple of 32
        tx.quantize_mx(X[:, :100].contiguous())
    with pytest.raises(tx.TxError):   # fp16 input
        tx.invoke("tx.quantize_rowwise", [q, sf, X, rows, K, K, K, _lib.F16, _lib.FP8E5M2])
    with pytest.raises(ValueError):
        tx.quantize_rowwise(X.cpu())


@pytest.mark.parametrize("fmt", [1, 2])
def test_hardware_conversion_matches_the_software_encoder(tx, dev, fmt):
    """The quantisers convert with gfx950's packed fp8 instructions after the
    clamp; the codec's tt.fp_to_fp encoder (saturating RNE, integer method,
    pinned to the oracle elsewhere) is the reference.  Rows whose absmax is
    exactly fmax quantise with multiplier 1, so the codes must equal the
    saturating conversion of x itself: 2^28 fp32 patterns spread over all
    2^32 (every exponent, sign and low-bit mix, NaNs and infinities)."""
    K, rows = 1 << 20, 256
    i = torch.arange(rows * K, dtype=torch.int64, device=dev)
    bits = (i * 16 + (i % 13)).to(torch.int64) & 0xFFFFFFFF
    x = bits.to(torch.int32).view(torch.float32).reshape(rows, K).clone()
    del i, bits
    # amax must be exactly fmax: values beyond it (and infinities) would set
    # the row's scale, so they become +-fmax-sized NaN-free entries here, and
    # two entries pin amax
    big = ~torch.isnan(x) & (x.abs() > FMAX[fmt])
    x[big] = torch.where(x[big] > 0, FMAX[fmt], -FMAX[fmt])
    x[:, 0] = FMAX[fmt]
    x[:, 1] = -FMAX[fmt]
    q, s = tx.quantize_rowwise(x, TD[fmt])
    assert torch.all(s == 1.0)
    ref = tx.fp_to_fp(x.reshape(-1), TD[fmt], saturate=True).reshape(rows, K)
    assert torch.equal(q.view(torch.uint8), ref.view(torch.uint8))
