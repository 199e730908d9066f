"""Plain-Triton kernels of the hot path run on the CPU by Triton's interpreter.

TEST AND BASELINE INFRASTRUCTURE ONLY: bench.py's cpu_baseline leg and the
tests import this module; the product never does.

The reference runs its kernels on the CPU through Triton's interpreter
(``TRITON_INTERPRET=1``: installed ``triton/runtime/interpreter.py``, which
executes ``@triton.jit`` bodies with NumPy, one program at a time on one Python
thread).  The reference's own TLX kernels cannot run there (the interpreter
has no ``utlx_*`` builders), so these are minimal plain-Triton kernels of the
same operations, written for this timing:

* ``convert_kernel``  ``x.to(tl.float8e4nv / tl.float8e5)``, ``tl.clamp`` first
  when saturating (the cast the reference lowers as ``tt.fp_to_fp``,
  installed ``language/semantic.py:803-827``);
* ``scatter_kernel``  ``tl.atomic_add(bins + idx, v)`` (``tt.atomic_rmw``,
  reference test_tlx.py:7627-7629);
* ``gemm_fp8_kernel`` tiled ``tl.dot`` of e4m3fn tiles with per-row and
  per-column fp32 scales in the epilogue, bf16 output;
* ``gemm_bf16_kernel`` tiled ``tl.dot`` of bf16 tiles upcast to fp32 first:
  the interpreter keeps bf16 as raw uint16 (interpreter.py:186-187) and its
  ``create_dot`` (:630-637) does not convert them;
* ``gemm_f16_kn_kernel`` the reference's matmul operands: fp16 a (M x K) and
  row-major fp16 b (K x N), upcast to fp32 for tl.dot, fp16 output;
* ``decode_kernel``   fp8 codes back to fp32 (the round trip's decode leg);
* ``gemv_kernel``     e5m2 weights dequantised by per-group fp32 scales,
  multiplied by one bf16 activation row per program.

The interpreter's own numerics differ from the fp8/bf16 semantics in places
(its fp8 rounding and its truncating fp32->bf16 cast); the results here are
timed, and the tests check them only where those differences cannot show.
"""
from __future__ import annotations

import os
import sys
import time

# Triton picks the interpreter when a function is decorated, its own library
# functions (tl.zeros, tl.sum, ...) included: the variable must be set before
# triton is first imported in the process.
_LATE = "triton" in sys.modules and os.environ.get("TRITON_INTERPRET") != "1"
os.environ["TRITON_INTERPRET"] = "1"

import numpy as np  # noqa: E402

try:  # noqa: SIM105
    import torch  # noqa: E402
    import triton  # noqa: E402
    import triton.language as tl  # noqa: E402
    IMPORT_ERROR = None
    if _LATE:
        IMPORT_ERROR = ("triton was imported before TRITON_INTERPRET=1 was set; "
                        "import triton_cpu first")
except Exception as e:  # pragma: no cover - reported, not raised
    IMPORT_ERROR = f"{type(e).__name__}: {e}"


if IMPORT_ERROR is None:
    @triton.jit
    def convert_kernel(x_ptr, y_ptr, n, DST: tl.constexpr, SAT: tl.constexpr,
                       MAXV: tl.constexpr, BLOCK: tl.constexpr):
        offs = tl.program_id(0) * BLOCK + tl.arange(0, BLOCK)
        m = offs < n
        x = tl.load(x_ptr + offs, mask=m, other=0.0)
        if SAT:
            x = tl.clamp(x, -MAXV, MAXV)
        tl.store(y_ptr + offs, x.to(DST), mask=m)

    @triton.jit
    def decode_kernel(x_ptr, y_ptr, n, BLOCK: tl.constexpr):
        offs = tl.program_id(0) * BLOCK + tl.arange(0, BLOCK)
        m = offs < n
        x = tl.load(x_ptr + offs, mask=m, other=0.0)
        tl.store(y_ptr + offs, x.to(tl.float32), mask=m)

    @triton.jit
    def scatter_kernel(bins_ptr, idx_ptr, v_ptr, n, BLOCK: tl.constexpr):
        offs = tl.program_id(0) * BLOCK + tl.arange(0, BLOCK)
        m = offs < n
        i = tl.load(idx_ptr + offs, mask=m, other=0)
        v = tl.load(v_ptr + offs, mask=m, other=0)
        tl.atomic_add(bins_ptr + i, v, mask=m)

    @triton.jit
    def gemm_fp8_kernel(a_ptr, b_ptr, sa_ptr, sb_ptr, c_ptr, M, N, K,
                        BM: tl.constexpr, BN: tl.constexpr, BK: tl.constexpr):
        rm = tl.program_id(0) * BM + tl.arange(0, BM)
        rn = tl.program_id(1) * BN + tl.arange(0, BN)
        rk = tl.arange(0, BK)
        mm = rm < M
        mn = rn < N
        acc = tl.zeros((BM, BN), dtype=tl.float32)
        for k in range(0, K, BK):
            kk = k + rk
            mk = kk < K
            a = tl.load(a_ptr + rm[:, None] * K + kk[None, :], mask=mm[:, None] & mk[None, :], other=0.0)
            b = tl.load(b_ptr + rn[None, :] * K + kk[:, None], mask=mk[:, None] & mn[None, :], other=0.0)
            acc += tl.dot(a, b)
        sa = tl.load(sa_ptr + rm, mask=mm, other=0.0)
        sb = tl.load(sb_ptr + rn, mask=mn, other=0.0)
        acc = acc * sa[:, None] * sb[None, :]
        tl.store(c_ptr + rm[:, None] * N + rn[None, :], acc.to(tl.bfloat16),
                 mask=mm[:, None] & mn[None, :])

    @triton.jit
    def gemm_bf16_kernel(a_ptr, b_ptr, c_ptr, M, N, K,
                         BM: tl.constexpr, BN: tl.constexpr, BK: tl.constexpr):
        rm = tl.program_id(0) * BM + tl.arange(0, BM)
        rn = tl.program_id(1) * BN + tl.arange(0, BN)
        rk = tl.arange(0, BK)
        mm = rm < M
        mn = rn < N
        acc = tl.zeros((BM, BN), dtype=tl.float32)
        for k in range(0, K, BK):
            kk = k + rk
            mk = kk < K
            a = tl.load(a_ptr + rm[:, None] * K + kk[None, :], mask=mm[:, None] & mk[None, :], other=0.0)
            b = tl.load(b_ptr + rn[None, :] * K + kk[:, None], mask=mk[:, None] & mn[None, :], other=0.0)
            acc += tl.dot(a.to(tl.float32), b.to(tl.float32))
        tl.store(c_ptr + rm[:, None] * N + rn[None, :], acc.to(tl.bfloat16),
                 mask=mm[:, None] & mn[None, :])

    @triton.jit
    def gemm_f16_kn_kernel(a_ptr, b_ptr, c_ptr, M, N, K,
                           BM: tl.constexpr, BN: tl.constexpr, BK: tl.constexpr):
        # the reference's matmul operands: a M x K, b K x N row-major, fp16 out
        rm = tl.program_id(0) * BM + tl.arange(0, BM)
        rn = tl.program_id(1) * BN + tl.arange(0, BN)
        rk = tl.arange(0, BK)
        mm = rm < M
        mn = rn < N
        acc = tl.zeros((BM, BN), dtype=tl.float32)
        for k in range(0, K, BK):
            kk = k + rk
            mk = kk < K
            a = tl.load(a_ptr + rm[:, None] * K + kk[None, :], mask=mm[:, None] & mk[None, :], other=0.0)
            b = tl.load(b_ptr + kk[:, None] * N + rn[None, :], mask=mk[:, None] & mn[None, :], other=0.0)
            acc += tl.dot(a.to(tl.float32), b.to(tl.float32))
        tl.store(c_ptr + rm[:, None] * N + rn[None, :], acc.to(tl.float16),
                 mask=mm[:, None] & mn[None, :])

    @triton.jit
    def gemv_kernel(x_ptr, w_ptr, s_ptr, y_ptr, N, K,
                    BN: tl.constexpr, G: tl.constexpr):
        rn = tl.program_id(0) * BN + tl.arange(0, BN)
        row = tl.program_id(1)
        mn = rn < N
        rg = tl.arange(0, G)
        ng = K // G
        acc = tl.zeros((BN,), dtype=tl.float32)
        for g in range(0, ng):
            kk = g * G + rg
            x = tl.load(x_ptr + row * K + kk).to(tl.float32)
            w = tl.load(w_ptr + rn[:, None] * K + kk[None, :], mask=mn[:, None], other=0.0)
            s = tl.load(s_ptr + rn * ng + g, mask=mn, other=0.0)
            acc += tl.sum(w.to(tl.float32) * x[None, :], axis=1) * s
        tl.store(y_ptr + row * N + rn, acc.to(tl.bfloat16), mask=mn)


def _need():
    if IMPORT_ERROR is not None:
        raise RuntimeError(f"Triton is not importable: {IMPORT_ERROR}")


def _t(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    return t if dtype is None else t.view(dtype)


# ------------------------------------------------------------ op wrappers
def convert(x: np.ndarray, fmt: str = "e4m3fn", sat: bool = False, block: int = 65536) -> np.ndarray:
    """fp32 -> fp8 codes (uint8) through the interpreter's cast."""
    _need()
    dst, maxv = {"e4m3fn": (tl.float8e4nv, 448.0), "e5m2": (tl.float8e5, 57344.0)}[fmt]
    xt = _t(x.astype(np.float32, copy=False))
    y = torch.empty(x.size, dtype=torch.uint8)
    yv = y.view(torch.float8_e4m3fn if fmt == "e4m3fn" else torch.float8_e5m2)
    convert_kernel[(triton.cdiv(x.size, block),)](xt, yv, x.size, DST=dst, SAT=sat, MAXV=maxv,
                                                 BLOCK=block)
    return y.numpy()


def decode(codes: np.ndarray, fmt: str = "e4m3fn", block: int = 65536) -> np.ndarray:
    """fp8 codes -> fp32 through the interpreter's cast."""
    _need()
    ct = _t(codes.astype(np.uint8, copy=False), torch.float8_e4m3fn if fmt == "e4m3fn" else torch.float8_e5m2)
    y = torch.empty(codes.size, dtype=torch.float32)
    decode_kernel[(triton.cdiv(codes.size, block),)](ct, y, codes.size, BLOCK=block)
    return y.numpy()


def scatter_add(nbins: int, idx: np.ndarray, val: np.ndarray, block: int = 65536) -> np.ndarray:
    """bins[idx[i]] += val[i] with tl.atomic_add (int32 wraps, fp32 adds in lane order)."""
    _need()
    bins = torch.zeros(nbins, dtype=torch.int32 if val.dtype == np.int32 else torch.float32)
    scatter_kernel[(triton.cdiv(idx.size, block),)](bins, _t(idx), _t(val), idx.size, BLOCK=block)
    return bins.numpy()


GEMM_TILE = (64, 256, 128)


def gemm_fp8(aq, bq, sa, sb, rows=None, tile=GEMM_TILE) -> np.ndarray:
    """C[:rows] (bf16 bits) of diag(sa) (Aq Bq^T) diag(sb); Aq M x K and Bq N x K e4m3fn codes."""
    _need()
    M, K = aq.shape
    N = bq.shape[0]
    rows = M if rows is None else rows
    BM, BN, BK = tile
    c = torch.empty(rows, N, dtype=torch.bfloat16)
    gemm_fp8_kernel[(triton.cdiv(rows, BM), triton.cdiv(N, BN))](
        _t(aq[:rows], torch.float8_e4m3fn), _t(bq, torch.float8_e4m3fn), _t(sa[:rows]), _t(sb), c,
        rows, N, K, BM=BM, BN=BN, BK=BK)
    return c.view(torch.uint16).numpy()


def gemm_bf16(a_bits, b_bits, rows=None, tile=GEMM_TILE) -> np.ndarray:
    """C[:rows] (bf16 bits) = A B^T with A M x K and B N x K given as bf16 bits."""
    _need()
    M, K = a_bits.shape
    N = b_bits.shape[0]
    rows = M if rows is None else rows
    BM, BN, BK = tile
    c = torch.empty(rows, N, dtype=torch.bfloat16)
    gemm_bf16_kernel[(triton.cdiv(rows, BM), triton.cdiv(N, BN))](
        _t(a_bits[:rows], torch.bfloat16), _t(b_bits, torch.bfloat16), c, rows, N, K,
        BM=BM, BN=BN, BK=BK)
    return c.view(torch.uint16).numpy()


def gemm_f16_kn(a_bits, b_bits, rows=None, tile=GEMM_TILE) -> np.ndarray:
    """C[:rows] (fp16 bits) = A B with A M x K and B K x N (row-major) fp16 bits."""
    _need()
    M, K = a_bits.shape
    N = b_bits.shape[1]
    rows = M if rows is None else rows
    BM, BN, BK = tile
    c = torch.empty(rows, N, dtype=torch.float16)
    gemm_f16_kn_kernel[(triton.cdiv(rows, BM), triton.cdiv(N, BN))](
        _t(a_bits[:rows], torch.float16), _t(b_bits, torch.float16), c, rows, N, K,
        BM=BM, BN=BN, BK=BK)
    return c.view(torch.uint16).numpy()


def gemv(x_bits, wq, s, group: int = 128, block_n: int = 256, rows=None) -> np.ndarray:
    """y (bf16 bits, rows x N) = x (M x K bf16 bits) times dequant(Wq e5m2 N x K,
    s N x K/group)^T, for the first `rows` rows of x (default all)."""
    _need()
    M, K = x_bits.shape
    rows = M if rows is None else rows
    N = wq.shape[0]
    y = torch.empty(rows, N, dtype=torch.bfloat16)
    gemv_kernel[(triton.cdiv(N, block_n), rows)](
        _t(x_bits[:rows], torch.bfloat16), _t(wq, torch.float8_e5m2), _t(s), y, N, K,
        BN=block_n, G=group)
    return y.view(torch.uint16).numpy()


# ------------------------------------------------------------ host facts
def host_facts() -> dict:
    """CPU model, cores visible to this process and the thread counts in force."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    blas = None
    try:
        import threadpoolctl
        info = [i for i in threadpoolctl.threadpool_info() if i.get("user_api") == "blas"]
        blas = info[0]["num_threads"] if info else None
    except Exception:
        pass
    return {"cpu_model": model, "nproc": cores, "python_threads": 1,
            "blas_threads": blas,
            "OMP_NUM_THREADS": os.environ.get("OMP_NUM_THREADS"),
            "OPENBLAS_NUM_THREADS": os.environ.get("OPENBLAS_NUM_THREADS")}


def _clock(fn):
    t0 = time.perf_counter()
    out = fn()
    return out, time.perf_counter() - t0


def baseline(gemm_rows: int = 64, bf16_rows: int = 64, progress=None) -> dict:
    """Time every kernel on the benchmark workloads (the GEMMs on their first rows).

    Conversions, the scatter and the GEMV run at full size.  The 8192^3 fp8
    GEMM and the 4096^3 bf16 GEMM run the programs of their first
    ``gemm_rows`` / ``bf16_rows`` rows of C (every column, the whole K loop),
    and the whole-problem time is that time scaled by M / rows: every program
    does the same work, and the interpreter runs programs one after another.
    """
    if IMPORT_ERROR is not None:
        return {"unavailable": IMPORT_ERROR}
    import workloads
    step = progress or (lambda name: None)
    out = {"engine": f"triton {triton.__version__} interpreter (TRITON_INTERPRET=1)",
           "host": host_facts()}

    x = workloads.fp8_input()
    for fmt, sat in (("e4m3fn", False), ("e4m3fn", True), ("e5m2", False), ("e5m2", True)):
        codes, dt = _clock(lambda: convert(x, fmt, sat))
        out[f"convert_{fmt}_{'sat' if sat else 'nonsat'}"] = {
            "value": 5.0 * x.size / dt / 1e9, "unit": "GB/s", "seconds": dt,
            "sample": f"full: {x.size:,} fp32 values, BLOCK=65536"}
        if not sat:
            _, dt = _clock(lambda: decode(codes, fmt))
            out[f"decode_{fmt}"] = {
                "value": 5.0 * x.size / dt / 1e9, "unit": "GB/s", "seconds": dt,
                "sample": f"full: {x.size:,} codes back to fp32 (the round trip's decode leg)"}
    del x, codes
    step("interpreter convert")

    for kind in ("i32", "f32"):
        idx, val = workloads.scatter_input(kind=kind)
        _, dt = _clock(lambda: scatter_add(65536, idx, val))
        out[f"scatter_{kind}"] = {
            "value": (8.0 * idx.size + 8.0 * 65536) / dt / 1e9, "unit": "GB/s", "seconds": dt,
            "gupdates_per_s": idx.size / dt / 1e9,
            "sample": f"full: {idx.size:,} Zipf(1.1) updates into 65,536 bins, BLOCK=65536"}
        step(f"interpreter scatter {kind}")
        del idx, val

    M = N = K = 8192
    aq, sa, bq, sb = workloads.fp8_gemm_input(gemm_rows, N, K)
    _, dt = _clock(lambda: gemm_fp8(aq, bq, sa, sb))
    out["fp8_gemm_8192"] = {
        "value": 2.0 * gemm_rows * N * K / dt / 1e12, "unit": "TFLOP/s",
        "seconds_sample": dt, "seconds_extrapolated": dt * M / gemm_rows,
        "sample": f"extrapolated: programs of the first {gemm_rows} of {M} rows of C "
                  f"(tiles {GEMM_TILE[0]}x{GEMM_TILE[1]}x{GEMM_TILE[2]}), time scaled by {M // gemm_rows}"}
    del aq, bq
    step("interpreter fp8 GEMM sample")

    a, b = workloads.bf16_gemm_input(bf16_rows, 4096, 4096)
    _, dt = _clock(lambda: gemm_bf16(a, b))
    out["bf16_gemm_4096"] = {
        "value": 2.0 * bf16_rows * 4096 * 4096 / dt / 1e12, "unit": "TFLOP/s",
        "seconds_sample": dt, "seconds_extrapolated": dt * 4096 / bf16_rows,
        "sample": f"extrapolated: programs of the first {bf16_rows} of 4096 rows of C, "
                  f"time scaled by {4096 // bf16_rows}"}
    step("interpreter bf16 GEMM sample")

    a, b = workloads.matmul16_input(bf16_rows, 4096, 4096)
    _, dt = _clock(lambda: gemm_f16_kn(a, b))
    out["matmul_f16_kn_4096"] = {
        "value": 2.0 * bf16_rows * 4096 * 4096 / dt / 1e12, "unit": "TFLOP/s",
        "seconds_sample": dt, "seconds_extrapolated": dt * 4096 / bf16_rows,
        "sample": f"extrapolated: the reference's matmul operands (fp16 a, row-major fp16 b), "
                  f"programs of the first {bf16_rows} of 4096 rows of C, time scaled by "
                  f"{4096 // bf16_rows}"}
    step("interpreter fp16 matmul sample")

    for m in (1, 4, 16):
        xg, wq, s = workloads.gemv_input(m)
        rows = 1  # every row's programs stream all of W: time is linear in the rows
        _, dt = _clock(lambda: gemv(xg, wq, s, rows=rows))
        dt_all = dt * m / rows
        nb = wq.size + 4 * s.size + 2 * xg.size + 2 * m * wq.shape[0]
        out[f"gemv_e5m2_m{m}"] = {
            "value": nb / dt_all / 1e9, "unit": "GB/s", "seconds": dt_all,
            "sample": (f"full: M=1, N=14336, K=4096, group 128" if m == 1 else
                       f"extrapolated: the programs of the first of {m} rows (each row's "
                       f"stream all of W), time scaled by {m}")}
    step("interpreter GEMV")
    return out
