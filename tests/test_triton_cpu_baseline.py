"""The plain-Triton kernels that bench.py times under Triton's interpreter
compute the benchmarked ops: each one, on a small input, agrees with the
oracle wherever the interpreter's own numerics (its fp8 rounding defects and
its truncating fp32 -> bf16 cast) cannot show.  CPU only; skipped where
Triton is not importable."""
import os

import numpy as np
import pytest

os.environ["TRITON_INTERPRET"] = "1"   # before triton's first import, or its tl.* helpers compile
pytest.importorskip("triton")


@pytest.fixture(scope="module")
def tc():
    import triton_cpu
    assert triton_cpu.IMPORT_ERROR is None, triton_cpu.IMPORT_ERROR
    return triton_cpu


def _bf16_bits_to_f32(b):
    return (np.asarray(b, np.uint32) << 16).view(np.float32)


@pytest.mark.parametrize("fmt,code_fmt,maxv", [("e4m3fn", 1, 448.0), ("e5m2", 2, 57344.0)])
def test_convert_exact_values_and_saturation(tc, oracle, fmt, code_fmt, maxv):
    # every finite normal code decodes to a value the interpreter must return unchanged
    codes = np.arange(256, dtype=np.uint8)
    vals = oracle.decode(codes, code_fmt)
    keep = np.isfinite(vals) & (np.abs(vals) >= (2.0 ** -6 if fmt == "e4m3fn" else 2.0 ** -14))
    x = vals[keep].astype(np.float32)
    got = tc.convert(x, fmt, sat=False, block=64)
    assert np.array_equal(got, oracle.encode(x, code_fmt, False))
    # with tl.clamp first, overflow saturates to the largest finite code
    big = np.array([maxv * 4, -maxv * 4, maxv, -maxv], np.float32)
    got = tc.convert(big, fmt, sat=True, block=64)
    assert np.array_equal(got, oracle.encode(big, code_fmt, True))


@pytest.mark.parametrize("kind", ["i32", "f32"])
def test_scatter_matches_oracle(tc, oracle, kind):
    rng = np.random.default_rng(5)
    n, nbins = 50_000, 97
    idx = (rng.zipf(1.5, n) % nbins).astype(np.int32)
    if kind == "i32":
        val = rng.integers(-2**31, 2**31 - 1, n, dtype=np.int64).astype(np.int32)
        got = tc.scatter_add(nbins, idx, val, block=4096)
        assert np.array_equal(got, oracle.scatter_add_i32(np.zeros(nbins, np.int32), idx, val))
    else:
        val = rng.standard_normal(n).astype(np.float32)
        got = tc.scatter_add(nbins, idx, val, block=4096)
        ref, mag = oracle.scatter_add_f32_ref(nbins, idx, val)
        assert np.all(np.abs(got - ref) <= 1e-5 * np.maximum(mag, 1e-30))


def test_gemm_fp8_matches_oracle(tc, oracle):
    import workloads
    M, N, K = 40, 72, 200          # ragged against the 64 x 256 x 128 tile
    aq, sa, bq, sb = workloads.fp8_gemm_input(M, N, K)
    got = _bf16_bits_to_f32(tc.gemm_fp8(aq, bq, sa, sb)).reshape(M, N)
    ref = oracle.gemm_fp8_scaled_rows(aq, bq, sa, sb, 0, M)[0].reshape(M, N)
    # the interpreter truncates fp32 -> bf16: at most 2^-7 relative
    assert np.all(np.abs(got - ref) <= 2.0 ** -7 * np.abs(ref) + 1e-30)


def test_gemm_bf16_matches_oracle(tc, oracle):
    import workloads
    M, N, K = 33, 65, 130
    a, b = workloads.bf16_gemm_input(M, N, K)
    got = _bf16_bits_to_f32(tc.gemm_bf16(a, b, tile=(32, 64, 64))).reshape(M, N)
    ref = oracle.gemm_bf16_rows(a, b, 0, M)[0].reshape(M, N)
    assert np.all(np.abs(got - ref) <= 2.0 ** -7 * np.abs(ref) + 1e-30)


def test_gemv_matches_oracle(tc, oracle):
    import workloads
    x, wq, s = workloads.gemv_input(3, 300, 512, 128)
    got = _bf16_bits_to_f32(tc.gemv(x, wq, s, 128, block_n=128)).reshape(3, 300)
    ref = _bf16_bits_to_f32(oracle.gemv_fp8_dequant(x, wq, s, 128)[1]).reshape(3, 300)
    assert np.max(np.abs(got - ref)) <= 2e-2 * np.max(np.abs(ref))


@pytest.mark.parametrize("fmt,code_fmt", [("e4m3fn", 1), ("e5m2", 2)])
def test_decode_matches_oracle(tc, oracle, fmt, code_fmt):
    codes = np.arange(256, dtype=np.uint8)
    ref = oracle.decode(codes, code_fmt)
    got = tc.decode(codes, fmt, block=64)
    # finite codes only: the interpreter's cast does not return NaN for the
    # NaN codes (one of its fp8 defects), which the timing does not depend on
    fin = np.isfinite(ref)
    assert np.array_equal(got[fin], ref[fin])


def test_gemm_f16_kn_matches_oracle(tc, oracle):
    import workloads
    M, N, K = 40, 72, 200
    a, b = workloads.matmul16_input(M, N, K)
    got = tc.gemm_f16_kn(a, b, tile=(32, 64, 64)).view(np.float16).astype(np.float64).reshape(M, N)
    ref32, _ = oracle.gemm16_rows(a, b, 0, M, fmt=oracle.F16, b_kn=True)
    assert np.max(np.abs(got - ref32)) <= 1e-2 * np.max(np.abs(ref32))


def test_gemv_row_sample(tc, oracle):
    import workloads
    x, wq, s = workloads.gemv_input(4, 300, 512, 128)
    full = tc.gemv(x, wq, s, 128, block_n=128)
    part = tc.gemv(x, wq, s, 128, block_n=128, rows=2)
    assert np.array_equal(part, full[:2])
