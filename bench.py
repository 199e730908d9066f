"""Benchmark of the tx op library on one MI355X.

Prints ONE JSON line.  The headline metric pairs two numbers:
  * value: fp8 e4m3fn scaled GEMM at M = N = K = 8192 (per-row / per-column
    fp32 scales, bf16 output), TFLOP/s, with its MFMA roofline fraction;
  * fp8_convert: tt.fp_to_fp fp32 -> e4m3fn (RNE, non-saturating) over
    16,777,216 values, GB/s of algorithmic traffic (5 B per value), with its
    HBM roofline fraction.
The other configurations are reported under "secondary".

A step is one launch of the op over one batch of synthetic input already
resident in HBM.  Each measurement first runs the same step, untimed, for
PREROLL_S seconds: the GPU's power manager raises the clocks only after some
milliseconds of sustained load, and an op timed straight after the idle host
work that builds its inputs would be timed on the clock ramp.  Then come W
untimed launches, then exactly K launches between two HIP events on the
stream the op is launched on (torch's current stream, which tx passes to the
library), with torch.cuda.synchronize() before and after.  Inputs rotate
over enough buffer sets that the working set exceeds twice the 256 MB
Infinity Cache for the memory-bound ops.

cpu_baseline: the reference's own CPU path, plain-Triton kernels of each op
run by Triton's interpreter (TRITON_INTERPRET=1, one Python thread plus
NumPy's BLAS threads) at full size, the GEMMs on their first 64 rows of C
with the time scaled to the whole problem (oracle/triton_cpu.py); its value
is the 8192^3 fp8 GEMM.  Under "oracle" it also carries the CPU oracle
(oracle/, a C port of the path's semantics, OpenMP over all host cores)
timed on bounded samples of the same workloads: rows of the 8192^3 GEMM for
CPU_GEMM_S seconds and whole 16 Mi-value encodes for CPU_CONVERT_S seconds.

Every timed op rotates over buffer sets whose total footprint is at least
twice the 256 MB Infinity Cache (ring_count), so no operand is re-read from
it across launches.  The JSON line ends with the fp8_convert object, the
second half of the headline metric.

Progress lines ("bench: ... done") go to stderr; stdout holds the JSON line.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "triton-ext_amd"))
sys.path.insert(0, os.path.join(REPO, "tests"))  # workloads: the seeded input generators

METRIC = "fp8 GEMM TFLOP/s + % MFMA peak @8192^3; fp8 convert GB/s + % HBM peak"
HBM_PEAK_GBS = 8000.0
FP8_PEAK_TFLOPS = 5000.0     # dense fp8 MFMA
FP4_PEAK_TFLOPS = 10100.0    # dense fp4 MFMA
BF16_PEAK_TFLOPS = 2500.0    # dense bf16 MFMA
F16_PEAK_TFLOPS = 2500.0     # dense fp16 MFMA
MALL_BYTES = 256 << 20


def progress(step, algo_bytes=None):
    """Report a finished workload; the launch windows timed() recorded since
    the last call are labelled with it (for --windows)."""
    for w in _PENDING_WINDOWS:
        WINDOWS.append(dict(w, workload=step, algo_bytes=algo_bytes))
    _PENDING_WINDOWS.clear()
    print(f"bench: {step} done ({time.perf_counter() - T_START:.1f} s)", file=sys.stderr, flush=True)


# Host-clock intervals around each workload's launches, in the two clocks a
# profiler may stamp dispatches with, so counter records can be assigned to
# workloads afterwards (--windows, --pmc-summary).
WINDOWS = []
_PENDING_WINDOWS = []


def _clocks():
    return {"boot": time.clock_gettime_ns(time.CLOCK_BOOTTIME), "mono": time.monotonic_ns()}


def build_digest():
    """Digest of everything the device code and the library are built from:
    the sources under triton-ext_amd/csrc and the build script.  Counter
    tables carry the digest of the build they were measured on."""
    import hashlib
    h = hashlib.sha256()
    root = os.path.join(REPO, "triton-ext_amd")
    files = [os.path.join(root, "build.py")]
    for d, _, names in os.walk(os.path.join(root, "csrc")):
        files += [os.path.join(d, n) for n in names if n.endswith((".hip", ".h", ".cpp", ".c"))]
    for f in sorted(files):
        h.update(os.path.relpath(f, REPO).encode() + b"\0")
        with open(f, "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()[:16]


T_START = time.perf_counter()


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--quick", action="store_true", help="headline ops only")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--calibrate-copy", action="store_true",
                   help="run only a 256 MiB device copy (known-size kernel for scaling the "
                        "FETCH_SIZE / WRITE_SIZE counters)")
    p.add_argument("--windows", metavar="JSON",
                   help="write each workload's launch windows (host clocks) and the build digest")
    p.add_argument("--pmc-summary", nargs=6, metavar=("FETCH_WINDOWS", "FETCH_CSV", "WRITE_WINDOWS",
                                                     "WRITE_CSV", "CAL_FETCH_CSV", "CAL_WRITE_CSV"),
                   help="print the HBM traffic table from the rocprofv3 counter_collection.csv "
                        "files of two --windows runs (FETCH_SIZE, WRITE_SIZE) and of two "
                        "--calibrate-copy runs")
    p.add_argument("--trace-summary", nargs=2, metavar=("WINDOWS_JSON", "TRACE_CSV"),
                   help="print the per-workload kernel duration table of a kernel-trace run")
    p.add_argument("--mfma-summary", nargs=2, metavar=("WINDOWS_JSON", "MFMA_CSV"),
                   help="print MFMA busy and clock per GEMM workload from a --windows run "
                        "counted with SQ_VALU_MFMA_BUSY_CYCLES, GRBM_GUI_ACTIVE, SQ_BUSY_CYCLES")
    p.add_argument("--lds-summary", nargs=2, metavar=("WINDOWS_JSON", "LDS_CSV"),
                   help="print the LDS counter table of a --pmc run of the bench made with --windows")
    return p.parse_args()


PREROLL_S = 0.25


def timed(fn, steps, warmup):
    """Average ms per launch of fn(i) over exactly `steps` launches, after the
    clock pre-roll and `warmup` untimed launches."""
    import torch
    torch.cuda.synchronize()
    window = {"t0": _clocks()}
    t0 = time.perf_counter()
    i = 0
    while time.perf_counter() - t0 < PREROLL_S:
        for _ in range(4):
            fn(i)
            i += 1
        torch.cuda.synchronize()
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        fn(warmup + i)
    end.record()
    end.synchronize()
    torch.cuda.synchronize()
    window["t1"] = _clocks()
    _PENDING_WINDOWS.append(window)
    return start.elapsed_time(end) / steps


def ring_count(set_bytes):
    return max(1, -(-2 * MALL_BYTES // set_bytes))


# ------------------------------------------------------------------ ops
def gemm_sets(M, N, K, ea, ec):
    """Buffer sets for a GEMM of ea-byte operands and ec-byte output whose
    whole ring exceeds twice the Infinity Cache."""
    return ring_count((M + N) * K * ea + M * N * ec)


def bench_fp8_gemm(tx, torch, M, N, K, steps, warmup, sets=None):
    import workloads
    dev = torch.device("cuda:0")
    sets = sets or gemm_sets(M, N, K, 1, 2)
    aq, sa, bq, sb = workloads.fp8_gemm_input(M, N, K)
    bufs = []
    for s in range(sets):
        A = torch.from_numpy(aq).to(dev).view(torch.float8_e4m3fn)
        B = torch.from_numpy(bq).to(dev).view(torch.float8_e4m3fn)
        bufs.append((A, torch.from_numpy(sa).to(dev), B, torch.from_numpy(sb).to(dev),
                     torch.empty((M, N), dtype=torch.bfloat16, device=dev)))
    del aq, bq

    def step(i):
        A, a_s, B, b_s, C = bufs[i % sets]
        tx.dot_scaled_rowcol(A, a_s, B, b_s, out=C)

    ms = timed(step, steps, warmup)
    flops = 2.0 * M * N * K
    tflops = flops / (ms * 1e-3) / 1e12
    return {"ms": ms, "tflops": tflops, "flops": flops,
            "bytes": M * K + N * K + 4 * (M + N) + 2 * M * N}


def bench_fp8_gemm_epilogue(tx, torch, M, N, K, steps, warmup, act, out_dtype, sets=None):
    """fp8 scaled GEMM with the fused epilogue (bias, activation, output cast)."""
    import workloads
    import numpy as np
    dev = torch.device("cuda:0")
    sets = sets or gemm_sets(M, N, K, 1, out_dtype.itemsize)
    aq, sa, bq, sb = workloads.fp8_gemm_input(M, N, K)
    bias = torch.from_numpy(np.random.default_rng(2).standard_normal(N).astype(np.float32)).to(dev)
    bufs = []
    for s in range(sets):
        A = torch.from_numpy(aq).to(dev).view(torch.float8_e4m3fn)
        B = torch.from_numpy(bq).to(dev).view(torch.float8_e4m3fn)
        bufs.append((A, torch.from_numpy(sa).to(dev), B, torch.from_numpy(sb).to(dev),
                     torch.empty((M, N), dtype=out_dtype, device=dev)))
    del aq, bq

    def step(i):
        A, a_s, B, b_s, C = bufs[i % sets]
        tx.dot_scaled_rowcol(A, a_s, B, b_s, out=C, bias=bias, activation=act, out_dtype=out_dtype,
                             out_scale=0.5)

    ms = timed(step, steps, warmup)
    return {"ms": ms, "tflops": 2.0 * M * N * K / (ms * 1e-3) / 1e12}


def bench_fp8_grouped(tx, torch, G, total, N, K, steps, warmup):
    """Grouped fp8 scaled GEMM (mixture-of-experts layer): `total` routed
    rows split unevenly over G experts (workloads.moe_group_sizes), each
    expert's N x K weights; one grouped launch, and the same products as a
    loop of G plain calls for comparison.  Random finite e4m3fn codes."""
    import numpy as np
    import workloads
    dev = torch.device("cuda:0")
    sizes = workloads.moe_group_sizes(total, G)
    off_np = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)

    def codes(*shape):
        c = torch.randint(0, 127, shape, dtype=torch.uint8, device=dev, generator=gen)
        return (c | (torch.randint(0, 2, shape, dtype=torch.uint8, device=dev, generator=gen) << 7)).view(
            torch.float8_e4m3fn)

    A, B = codes(total, K), codes(G, N, K)
    sa = torch.rand(total, device=dev, generator=gen) + 0.5
    sb = torch.rand(G, N, device=dev, generator=gen) + 0.5
    off = torch.from_numpy(off_np).to(dev)
    C = torch.empty((total, N), dtype=torch.bfloat16, device=dev)
    ms = timed(lambda i: tx.dot_scaled_rowcol_grouped(A, sa, B, sb, off, out=C), steps, warmup)

    def loop(i):
        for p in range(G):
            r0, r1 = int(off_np[p]), int(off_np[p + 1])
            if r1 > r0:
                tx.dot_scaled_rowcol(A[r0:r1], sa[r0:r1], B[p], sb[p], out=C[r0:r1])

    ms_loop = timed(loop, steps, warmup)
    flops = 2.0 * total * N * K
    return {"ms": ms, "tflops": flops / (ms * 1e-3) / 1e12, "ms_loop": ms_loop,
            "tflops_loop": flops / (ms_loop * 1e-3) / 1e12, "sizes": sizes.tolist()}


def bench_mx_gemm(tx, torch, M, N, K, steps, warmup, sets=None, fp4=False):
    """tt.dot_scaled with MX block scales (e8m0 per 32 K), bf16 out; e4m3fn
    operands, or fp4 (e2m1, two per byte) with ``fp4``."""
    import workloads
    dev = torch.device("cuda:0")
    sets = sets or ring_count((M + N) * (K // 2 if fp4 else K) + (M + N) * K // 32 + 2 * M * N)
    if fp4:
        aq, sa, bq, sb = workloads.mx_fp4_gemm_input(M, N, K)
        dt, fmt = torch.uint8, "e2m1"
    else:
        aq, sa, bq, sb = workloads.mx_gemm_input(M, N, K)
        dt, fmt = torch.float8_e4m3fn, None
    bufs = []
    for s in range(sets):
        A = torch.from_numpy(aq).to(dev).view(dt)
        B = torch.from_numpy(bq).to(dev).view(dt)
        bufs.append((A, torch.from_numpy(sa).to(dev), B, torch.from_numpy(sb).to(dev),
                     torch.empty((M, N), dtype=torch.bfloat16, device=dev)))
    del aq, bq

    def step(i):
        A, a_s, B, b_s, C = bufs[i % sets]
        tx.dot_scaled(A, a_s, B, b_s, out_dtype=torch.bfloat16, out=C, a_format=fmt, b_format=fmt)

    ms = timed(step, steps, warmup)
    flops = 2.0 * M * N * K
    ob = K // 2 if fp4 else K
    return {"ms": ms, "tflops": flops / (ms * 1e-3) / 1e12, "flops": flops,
            "bytes": M * ob + N * ob + (M + N) * K // 32 + 2 * M * N}


def bench_quant(tx, torch, kind, xdt, steps, warmup, rows=8192, K=8192):
    """absmax + fp8 quantiser over a rows x K fp32 / bf16 matrix (MX or row-wise)."""
    import numpy as np
    dev = torch.device("cuda:0")
    g = np.random.default_rng(6)
    x0 = torch.from_numpy(g.standard_normal((rows, K), dtype=np.float32)).to(dev)
    if xdt == "bf16":
        x0 = x0.to(torch.bfloat16)
    es = x0.element_size()
    per_set = rows * K * (es + 1)
    sets = ring_count(per_set)
    xs = [x0] + [x0.clone() for _ in range(sets - 1)]
    fn = tx.quantize_mx if kind == "mx" else tx.quantize_rowwise

    def step(i):
        fn(xs[i % sets])

    ms = timed(step, steps, warmup)
    nbytes = rows * K * (es + 1) + (rows * K // 32 if kind == "mx" else 4 * rows)
    return {"ms": ms, "gbs": nbytes / (ms * 1e-3) / 1e9, "bytes": nbytes, "sets": sets}


def bench_bf16_gemm(tx, torch, M, N, K, steps, warmup):
    import workloads
    import numpy as np
    dev = torch.device("cuda:0")
    A, B = workloads.bf16_gemm_input(M, N, K)
    sets = gemm_sets(M, N, K, 2, 2)
    At = torch.from_numpy(A.view(np.int16)).to(dev).view(torch.bfloat16)
    Bt = torch.from_numpy(B.view(np.int16)).to(dev).view(torch.bfloat16)
    bufs = [(At, Bt) if i == 0 else (At.clone(), Bt.clone()) for i in range(sets)]
    Cs = [torch.empty((M, N), dtype=torch.bfloat16, device=dev) for _ in range(sets)]
    ms = timed(lambda i: tx.dot(bufs[i % sets][0], bufs[i % sets][1], out=Cs[i % sets]), steps, warmup)
    flops = 2.0 * M * N * K
    return {"ms": ms, "tflops": flops / (ms * 1e-3) / 1e12, "flops": flops, "sets": sets}


def bench_matmul16(tx, torch, S, steps, warmup):
    """The reference's matmul benchmark (test_amd_gemm_pipelined.py:355-399):
    matmul(a, b) on fp16 S x S operands, b row-major, fp16 output allocated
    per call, against torch.matmul on the same tensors (its rocBLAS line)."""
    import workloads
    import numpy as np
    dev = torch.device("cuda:0")
    A, B = workloads.matmul16_input(S, S, S)
    a = torch.from_numpy(A.view(np.int16)).to(dev).view(torch.float16)
    b = torch.from_numpy(B.view(np.int16)).to(dev).view(torch.float16)
    sets = gemm_sets(S, S, S, 2, 2)
    ops = [(a, b) if i == 0 else (a.clone(), b.clone()) for i in range(sets)]
    ms = timed(lambda i: tx.matmul(*ops[i % sets]), steps, warmup)
    ms_torch = timed(lambda i: torch.matmul(*ops[i % sets]), steps, warmup)
    flops = 2.0 * S ** 3
    return {"ms": ms, "tflops": flops / (ms * 1e-3) / 1e12, "torch_ms": ms_torch,
            "torch_tflops": flops / (ms_torch * 1e-3) / 1e12, "bytes": 6.0 * S * S}


def bench_fp8_convert(tx, torch, steps, warmup, n=16_777_216):
    import workloads
    dev = torch.device("cuda:0")
    x_np = workloads.fp8_input(n)
    sets = ring_count(5 * n)
    xs = [torch.from_numpy(x_np).to(dev) for _ in range(sets)]
    qs = [torch.empty(n, dtype=torch.float8_e4m3fn, device=dev) for _ in range(sets)]
    ms = timed(lambda i: tx.fp_to_fp(xs[i % sets], torch.float8_e4m3fn, out=qs[i % sets]),
               steps, warmup)
    enc_gbs = 5.0 * n / (ms * 1e-3) / 1e9
    fs = [torch.empty(n, dtype=torch.float32, device=dev) for _ in range(sets)]
    ms_dec = timed(lambda i: tx.fp_to_fp(qs[i % sets], torch.float32, out=fs[i % sets]),
                   steps, warmup)
    dec_gbs = 5.0 * n / (ms_dec * 1e-3) / 1e9
    # the memory system's ceiling for the encode's launch shape and bytes:
    # the same kernel shape with the conversion taken out (4:1 byte copy)
    # and a read-only stream of the same fp32 input
    import ctypes
    cur = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def ceiling(kind):
        def go(i):
            st = tx.lib.txStreamCeiling(kind, ctypes.c_void_p(xs[i % sets].data_ptr()),
                                        ctypes.c_void_p(qs[i % sets].data_ptr()), n, cur())
            if st != 0:
                raise RuntimeError(tx._lib.last_error())
        return timed(go, steps, warmup)

    ms_copy, ms_read = ceiling(0), ceiling(1)
    return {"ms": ms, "gbs": enc_gbs, "bytes": 5.0 * n, "sets": sets,
            "decode_ms": ms_dec, "decode_gbs": dec_gbs,
            "ceiling": {"copy_4to1_ms": round(ms_copy, 5),
                        "copy_4to1_gbs": round(5.0 * n / (ms_copy * 1e-3) / 1e9, 1),
                        "read_ms": round(ms_read, 5),
                        "read_gbs": round(4.0 * n / (ms_read * 1e-3) / 1e9, 1),
                        "encode_over_copy": round(ms_copy / ms, 4),
                        "what": "the encode's launch shape with the conversion taken out (4 B read, "
                                "1 B written per value) and reading only (4 B per value), same buffers"}}


def bench_convert_pair(tx, torch, src, dst, steps, warmup, n=16_777_216):
    """tt.fp_to_fp between two of bf16 / fp16 / e4m3fn / e5m2 (RNE, not
    saturating); the source is the fp32 workload cast (RNE) to `src`."""
    import workloads
    dev = torch.device("cuda:0")
    x = torch.from_numpy(workloads.fp8_input(n)).to(dev)
    if src.itemsize == 1:
        x = tx.fp_to_fp(x, src)
    else:
        x = x.to(src)
    per = src.itemsize + dst.itemsize
    sets = ring_count(per * n)
    xs = [x.clone() for _ in range(sets)]
    ys = [torch.empty(n, dtype=dst, device=dev) for _ in range(sets)]
    ms = timed(lambda i: tx.fp_to_fp(xs[i % sets], dst, out=ys[i % sets]), steps, warmup)
    return {"ms": ms, "gbs": per * n / (ms * 1e-3) / 1e9, "bytes": per * n, "sets": sets}


def bench_encode_sizes(tx, torch, steps, warmup, sizes=(67_108_864, 268_435_456)):
    """The headline encode at larger sizes: per-launch fixed cost (wave launch,
    the first bytes' latency, the drain) weighs less as the size grows."""
    import workloads
    dev = torch.device("cuda:0")
    base = torch.from_numpy(workloads.fp8_input(16_777_216)).to(dev)
    out = {}
    for n in sizes:
        sets = ring_count(5 * n)
        xs = [base.repeat(n // base.numel()) for _ in range(sets)]
        qs = [torch.empty(n, dtype=torch.float8_e4m3fn, device=dev) for _ in range(sets)]
        ms = timed(lambda i: tx.fp_to_fp(xs[i % sets], torch.float8_e4m3fn, out=qs[i % sets]), steps, warmup)
        out[n] = (ms, 5.0 * n)
        del xs, qs
    return out


def bench_torch_streams(torch, steps, warmup, n=16_777_216):
    """torch's own kernels over the convert's 16 Mi fp32 values, for reference:
    a cast to uint8 (the encode's 4 B -> 1 B traffic shape), a device copy
    (the runtime's copy kernel) and a sum (read only)."""
    dev = torch.device("cuda:0")
    out = {}
    sets = ring_count(5 * n)
    xs = [torch.randn(n, device=dev) for _ in range(sets)]
    ys = [torch.empty(n, dtype=torch.uint8, device=dev) for _ in range(sets)]
    ms = timed(lambda i: ys[i % sets].copy_(xs[i % sets]), steps, warmup)
    out["cast fp32->uint8 (4 B read, 1 B written per value)"] = (ms, 5.0 * n)
    zs = [torch.empty(n, device=dev) for _ in range(sets)]
    ms = timed(lambda i: zs[i % sets].copy_(xs[i % sets]), steps, warmup)
    out["copy fp32 (4 B read, 4 B written per value)"] = (ms, 8.0 * n)
    acc = torch.empty((), device=dev)
    ms = timed(lambda i: torch.sum(xs[i % sets], dim=0, out=acc), steps, warmup)
    out["sum fp32 (4 B read per value)"] = (ms, 4.0 * n)
    return out


def bench_scatter(tx, torch, kind, steps, warmup, n=67_108_864, nbins=65536):
    import workloads
    dev = torch.device("cuda:0")
    idx_np, val_np = workloads.scatter_input(n=n, nbins=nbins, kind=kind)
    sets = 2  # 2 x 512 MB of updates > 2 x MALL
    idx = [torch.from_numpy(idx_np).to(dev) for _ in range(sets)]
    val = [torch.from_numpy(val_np).to(dev) for _ in range(sets)]
    bins = torch.zeros(nbins, dtype=torch.int32 if kind == "i32" else torch.float32, device=dev)
    op = "add" if kind == "i32" else "fadd"
    ms = timed(lambda i: tx.atomic_rmw(op, bins, idx[i % sets], val[i % sets]), steps, warmup)
    algo = 8.0 * n + 8.0 * nbins
    return {"ms": ms, "gbs": algo / (ms * 1e-3) / 1e9, "bytes": algo,
            "updates_per_s": n / (ms * 1e-3)}


def bench_gemv(tx, torch, M, steps, warmup, N=14336, K=4096, group=128):
    import workloads
    import numpy as np
    dev = torch.device("cuda:0")
    x, wq, s = workloads.gemv_input(M, N, K, group)
    xt = torch.from_numpy(x.view(np.int16)).to(dev).view(torch.bfloat16)
    wbytes = N * K + 4 * s.size
    sets = ring_count(wbytes)
    ws = [torch.from_numpy(wq).to(dev).view(torch.float8_e5m2) for _ in range(sets)]
    ss = [torch.from_numpy(s).to(dev) for _ in range(sets)]
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    ms = timed(lambda i: tx.gemv_fp8_dequant(xt, ws[i % sets], ss[i % sets], group, out=y),
               steps, warmup)
    algo = N * K + 4.0 * N * (K // group) + 2.0 * M * K + 2.0 * M * N
    return {"ms": ms, "gbs": algo / (ms * 1e-3) / 1e9, "bytes": algo, "sets": sets}


# ------------------------------------------------------------ CPU baseline
CPU_GEMM_S = 8.0
CPU_CONVERT_S = 5.0


def cpu_baseline():
    """The reference's CPU path (plain-Triton kernels under Triton's
    interpreter) on the headline workloads, as `value`; the oracle (C,
    OpenMP) on bounded samples of the same workloads under `oracle`."""
    import numpy as np
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle
    import workloads
    oracle.build()
    cores = os.cpu_count() or 1
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        pass
    # fp8 GEMM: batches of R rows of C for the 8192^3 problem (2 * R * N * K
    # flops each), repeated until CPU_GEMM_S seconds have passed
    M = N = K = 8192
    R = 64
    g = np.random.default_rng(1)
    aq = g.integers(0, 0x7F, size=(R, K), dtype=np.uint8)
    bq = np.ascontiguousarray(workloads.fp8_gemm_input(16, N, K)[2])
    sa = np.ones(R, np.float32)
    sb = np.ones(N, np.float32)
    rows, t0 = 0, time.perf_counter()
    while rows == 0 or (time.perf_counter() - t0 < CPU_GEMM_S and rows < M):
        oracle.gemm_fp8_scaled_rows(aq, bq, sa, sb, 0, R, nthreads=cores)
        rows += R
    dt = time.perf_counter() - t0
    gemm_tflops = 2.0 * rows * N * K / dt / 1e12
    # fp8 convert: the full 16 Mi-value encode, repeated for CPU_CONVERT_S seconds
    x = workloads.fp8_input()
    reps, t0 = 0, time.perf_counter()
    while reps < 3 or time.perf_counter() - t0 < CPU_CONVERT_S:
        oracle.encode(x, 1, False, nthreads=cores)
        reps += 1
    dt_conv = (time.perf_counter() - t0) / reps
    from triton_cpu import baseline as interpreter_baseline
    progress("cpu baseline: oracle")
    interp = interpreter_baseline(progress=progress)
    progress("cpu baseline: triton interpreter")
    oracle_leg = {
        "value": gemm_tflops, "unit": "TFLOP/s", "cores": cores, "kind": "port",
        "what": "the oracle: this repository's C restatement of the path (OpenMP, fp64 accumulation)",
        "sample": f"fp8 scaled GEMM, {rows} of 8192 rows of M=N=K=8192 "
                  f"({2.0 * rows * N * K / 1e9:.0f} GFLOP in {dt:.1f} s)",
        "fp8_convert": {"value": 5.0 * x.size / dt_conv / 1e9, "unit": "GB/s",
                        "sample": f"encode e4m3fn RNE of 16,777,216 values x {reps}"},
    }
    if "unavailable" in interp:
        return {"value": None, "unit": "TFLOP/s", "cores": cores, "kind": "port",
                "what": "the reference's CPU path (Triton's interpreter) is unavailable on this host: "
                        + str(interp["unavailable"]), "oracle": oracle_leg}
    g = interp["fp8_gemm_8192"]
    facts = interp.get("host", {})
    conv = interp["convert_e4m3fn_nonsat"]
    return {
        "value": g["value"], "unit": "TFLOP/s",
        # one Python thread walks the grid; np.matmul inside tl.dot uses the BLAS threads
        "cores": max(1, int(facts.get("blas_threads") or 1)), "kind": "port",
        "what": "the reference's CPU path: plain-Triton kernels of each op under Triton's interpreter "
                "(TRITON_INTERPRET=1, one Python thread plus NumPy's BLAS threads for tl.dot); the "
                "oracle (C, OpenMP) is under 'oracle'",
        "sample": g["sample"],
        "fp8_convert": {"value": conv["value"], "unit": "GB/s", "sample": conv["sample"]},
        "oracle": oracle_leg,
        "triton_interpreter": interp,
    }


COPY_BYTES = 256 << 20
TRAFFIC_TABLE = os.path.join(REPO, "profiles", "hbm_traffic_bench_workloads.md")


def calibrate_copy():
    """A device-to-device copy of COPY_BYTES, 5 launches (the known-size kernel)."""
    import torch
    src = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device="cuda:0").uniform_()
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "copy", "bytes": COPY_BYTES, "launches": 5}))


def _dispatches(path, counters):
    """Per-dispatch records of a rocprofv3 counter_collection.csv: kernel,
    grid, start / end timestamps and each counter in `counters` (the rows of
    one dispatch and counter are summed)."""
    import csv
    out = {}
    with open(path) as f:
        for row in csv.DictReader(f):
            if row["Counter_Name"] not in counters:
                continue
            d = out.setdefault(row["Dispatch_Id"], {
                "kernel": row["Kernel_Name"], "grid": int(row["Grid_Size"]),
                "t0": int(row["Start_Timestamp"]), "t1": int(row["End_Timestamp"]), "c": {}})
            d["c"][row["Counter_Name"]] = d["c"].get(row["Counter_Name"], 0.0) + float(row["Counter_Value"])
    return list(out.values())


def _assign(windows, disp):
    """Label dispatches with the workload whose launch window holds their
    start, in whichever host clock the profiler's timestamps follow."""
    best = None
    for clock in ("boot", "mono"):
        spans = sorted((w["t0"][clock], w["t1"][clock], w) for w in windows)
        hits = []
        for d in disp:
            for lo, hi, w in spans:
                if lo <= d["t0"] <= hi:
                    hits.append((d, w))
                    break
        if best is None or len(hits) > len(best):
            best = hits
    return best


def _short(name):
    return name.split("(")[0][:72] if not name.startswith("void ") else name[5:].split("<")[0][:72]


def pmc_summary(fetch_windows, fetch_csv, write_windows, write_csv, cal_fetch_csv, cal_write_csv):
    with open(fetch_windows) as f:
        meta = json.load(f)
    with open(write_windows) as f:
        meta_w = json.load(f)
    if meta_w["digest"] != meta["digest"]:
        sys.exit("the FETCH_SIZE and WRITE_SIZE runs were made on different builds")
    # the copy's dispatches are the ones that move the most data
    cal_f = sorted(d["c"]["FETCH_SIZE"] for d in _dispatches(cal_fetch_csv, {"FETCH_SIZE"}))[-5:]
    cal_w = sorted(d["c"]["WRITE_SIZE"] for d in _dispatches(cal_write_csv, {"WRITE_SIZE"}))[-5:]
    kib = COPY_BYTES / 1024
    f_scale = kib / (sum(cal_f) / len(cal_f))
    w_scale = kib / (sum(cal_w) / len(cal_w))
    print(f"build digest: {meta['digest']}")
    print()
    print(f"copy calibration: {COPY_BYTES} B copied; FETCH_SIZE reads "
          f"{sum(cal_f) / len(cal_f):.0f} KiB, WRITE_SIZE {sum(cal_w) / len(cal_w):.0f} KiB per "
          f"launch; scale factors fetch {f_scale:.4f}, write {w_scale:.4f}")
    print()
    rows = {}
    for counter, path, m in (("FETCH_SIZE", fetch_csv, meta), ("WRITE_SIZE", write_csv, meta_w)):
        for d, w in _assign(m["windows"], _dispatches(path, {counter})):
            key = (w["workload"], _short(d["kernel"]), d["grid"])
            r = rows.setdefault(key, {"algo": w.get("algo_bytes"), "FETCH_SIZE": [], "WRITE_SIZE": []})
            r[counter].append(d["c"][counter])
    order = {w["workload"]: i for i, w in enumerate(meta["windows"])}
    print("| workload | kernel | grid | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB "
          "| traffic bytes per launch | algorithmic bytes per step | traffic / algorithmic |")
    print("|---|---|---|---|---|---|---|---|---|")
    for key in sorted(rows, key=lambda k: (order.get(k[0], 1 << 30), k[1], k[2])):
        r = rows[key]
        fv, wv = r["FETCH_SIZE"] or [0.0], r["WRITE_SIZE"] or [0.0]
        fk, wk = sum(fv) / len(fv), sum(wv) / len(wv)
        traffic = (fk * f_scale + wk * w_scale) * 1024
        algo = r["algo"]
        ratio = f"{traffic / algo:.3f}" if algo else ""
        print(f"| {key[0]} | {key[1]} | {key[2]} | {max(len(r['FETCH_SIZE']), len(r['WRITE_SIZE']))} "
              f"| {fk:.0f} | {wk:.0f} | {traffic:.0f} | {int(algo) if algo else ''} | {ratio} |")


def mfma_summary(windows_json, mfma_csv):
    with open(windows_json) as f:
        meta = json.load(f)
    names = {"SQ_VALU_MFMA_BUSY_CYCLES", "GRBM_GUI_ACTIVE", "SQ_BUSY_CYCLES"}
    rows = {}
    for d, w in _assign(meta["windows"], _dispatches(mfma_csv, names)):
        if d["c"].get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) <= 0.0:
            continue
        key = (w["workload"], _short(d["kernel"]), d["grid"])
        rows.setdefault(key, []).append(d)
    order = {w["workload"]: i for i, w in enumerate(meta["windows"])}
    print(f"build digest: {meta['digest']}")
    print()
    print("| workload | kernel | grid | dispatches | SQ_VALU_MFMA_BUSY_CYCLES | GRBM_GUI_ACTIVE per XCD "
          "| duration us | clock GHz | MFMA busy |")
    print("|---|---|---|---|---|---|---|---|---|")
    for key in sorted(rows, key=lambda k: (order.get(k[0], 1 << 30), k[1], k[2])):
        ds = rows[key]
        busy = sum(d["c"]["SQ_VALU_MFMA_BUSY_CYCLES"] for d in ds) / len(ds)
        gui = sum(d["c"]["GRBM_GUI_ACTIVE"] for d in ds) / len(ds) / XCDS
        dur = sum(d["t1"] - d["t0"] for d in ds) / len(ds)
        print(f"| {key[0]} | {key[1]} | {key[2]} | {len(ds)} | {busy:.4g} | {gui:.0f} | {dur / 1e3:.1f} "
              f"| {gui / dur:.2f} | {busy / (gui * SIMDS):.1%} |")


XCDS = 8
SIMDS = 1024  # 256 CUs x 4 SIMDs
LDS_COUNTERS = ("SQ_INSTS_LDS", "SQ_LDS_IDX_ACTIVE", "SQ_LDS_ADDR_CONFLICT", "SQ_LDS_BANK_CONFLICT",
                "GRBM_GUI_ACTIVE")


def lds_summary(windows_json, lds_csv):
    """LDS counters per workload and kernel: how much of the cycles the LDS
    spends on indexed operations goes to same-address conflicts (atomics
    from many lanes on one bin) and to bank conflicts."""
    with open(windows_json) as f:
        meta = json.load(f)
    rows = {}
    for d, w in _assign(meta["windows"], _dispatches(lds_csv, set(LDS_COUNTERS))):
        if d["c"].get("SQ_INSTS_LDS", 0.0) <= 0.0:
            continue
        rows.setdefault((w["workload"], _short(d["kernel"]), d["grid"]), []).append(d)
    order = {w["workload"]: i for i, w in enumerate(meta["windows"])}
    print(f"build digest: {meta['digest']}")
    print()
    print("| workload | kernel | grid | dispatches | duration us | SQ_INSTS_LDS | SQ_LDS_IDX_ACTIVE "
          "| SQ_LDS_ADDR_CONFLICT | SQ_LDS_BANK_CONFLICT | address conflict / LDS active "
          "| bank conflict / LDS active | LDS active / (GRBM_GUI_ACTIVE per XCD x 256 CUs) |")
    print("|---|---|---|---|---|---|---|---|---|---|---|---|")
    for key in sorted(rows, key=lambda k: (order.get(k[0], 1 << 30), k[1], k[2])):
        ds = rows[key]
        m = {c: sum(d["c"].get(c, 0.0) for d in ds) / len(ds) for c in LDS_COUNTERS}
        dur = sum(d["t1"] - d["t0"] for d in ds) / len(ds)
        act = m["SQ_LDS_IDX_ACTIVE"]
        cyc = m["GRBM_GUI_ACTIVE"] / XCDS * 256
        print(f"| {key[0]} | {key[1]} | {key[2]} | {len(ds)} | {dur / 1e3:.1f} | {m['SQ_INSTS_LDS']:.4g} "
              f"| {act:.4g} | {m['SQ_LDS_ADDR_CONFLICT']:.4g} | {m['SQ_LDS_BANK_CONFLICT']:.4g} "
              f"| {m['SQ_LDS_ADDR_CONFLICT'] / act if act else 0:.1%} "
              f"| {m['SQ_LDS_BANK_CONFLICT'] / act if act else 0:.1%} | {act / cyc if cyc else 0:.1%} |")


def trace_summary(windows_json, trace_csv):
    """Per-workload kernel durations of a `rocprofv3 --kernel-trace` run of the
    bench (made with --windows): every dispatch labelled with the workload
    whose launch window holds its start; the last 20 of a group are the timed
    launches of the GEMM and scatter lines."""
    import csv
    with open(windows_json) as f:
        meta = json.load(f)
    disp = []
    with open(trace_csv) as f:
        for row in csv.DictReader(f):
            disp.append({"kernel": row["Kernel_Name"], "t0": int(row["Start_Timestamp"]),
                         "t1": int(row["End_Timestamp"]),
                         "grid": f"{int(row['Grid_Size_X']) // max(1, int(row['Workgroup_Size_X']))} x "
                                 f"{row['Workgroup_Size_X']}"})
    rows = {}
    for d, w in _assign(meta["windows"], disp):
        key = (w["workload"], _short(d["kernel"]), d["grid"])
        rows.setdefault(key, []).append(d["t1"] - d["t0"])
    order = {w["workload"]: i for i, w in enumerate(meta["windows"])}
    print(f"build digest: {meta['digest']}")
    print()
    print("| workload | kernel | grid (workgroups x threads) | dispatches | avg us (all) | avg us (last 20) |")
    print("|---|---|---|---|---|---|")
    for key in sorted(rows, key=lambda k: (order.get(k[0], 1 << 30), k[1], k[2])):
        ds = rows[key]
        last = ds[-20:]
        print(f"| {key[0]} | `{key[1]}` | {key[2]} | {len(ds)} | {sum(ds) / len(ds) / 1e3:.2f} "
              f"| {sum(last) / len(last) / 1e3:.2f} |")


def traffic_from_table(workload, kernel_prefix):
    """HBM bytes per launch of a kernel on a workload, from the committed
    counter table, and whether the table was made on another build."""
    if not os.path.exists(TRAFFIC_TABLE):
        return None, None
    digest, value = None, None
    with open(TRAFFIC_TABLE) as f:
        for line in f:
            if line.startswith("build digest:"):
                digest = line.split(":", 1)[1].strip()
            cells = [c.strip() for c in line.strip().strip("|").split("|")]
            if len(cells) == 9 and cells[0] == workload and cells[1].startswith(kernel_prefix):
                try:
                    value = int(float(cells[6]))
                except ValueError:
                    pass
    if value is None:
        return None, None
    return value, {"table": os.path.relpath(TRAFFIC_TABLE, REPO), "table_build": digest,
                   "this_build": build_digest(), "stale": digest != build_digest()}


def main():
    args = parse()
    if args.pmc_summary:
        pmc_summary(*args.pmc_summary)
        return
    if args.mfma_summary:
        mfma_summary(*args.mfma_summary)
        return
    if args.lds_summary:
        lds_summary(*args.lds_summary)
        return
    if args.trace_summary:
        trace_summary(*args.trace_summary)
        return
    if args.calibrate_copy:
        calibrate_copy()
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "bench.py measures one GPU only: every op runs on one "
                                   "MI355X; multi-GPU sharding is not implemented"}))
        sys.exit(2)
    import torch
    import tx
    tx.init()
    K, W = args.steps, args.warmup

    gemm = bench_fp8_gemm(tx, torch, 8192, 8192, 8192, K, W)
    progress("fp8 GEMM 8192^3", gemm["bytes"])
    conv = bench_fp8_convert(tx, torch, max(K, 50), W)
    progress("fp8 convert 16Mi", conv["bytes"])
    secondary = []
    if not args.quick:
        for (m, n, k) in [(16, 14336, 4096), (512, 14336, 4096), (8192, 14336, 4096),
                          (16, 4096, 14336), (512, 4096, 14336), (8192, 4096, 14336)]:
            # small M streams B from HBM: rotate buffer sets past the Infinity Cache
            r = bench_fp8_gemm(tx, torch, m, n, k, K, W)
            secondary.append({"op": "fp8 scaled GEMM", "shape": [m, n, k], "ms": r["ms"],
                              "tflops": r["tflops"],
                              "frac_mfma": r["tflops"] / FP8_PEAK_TFLOPS,
                              "gbs": r["bytes"] / (r["ms"] * 1e-3) / 1e9})
            progress(secondary[-1]["op"] + " " + str(secondary[-1].get("shape", "")), r.get("bytes"))
        for act, odt, oname in (("gelu_tanh", torch.float8_e4m3fn, "e4m3fn"), ("silu", torch.bfloat16, "bf16")):
            r = bench_fp8_gemm_epilogue(tx, torch, 8192, 8192, 8192, K, W, act, odt)
            secondary.append({"op": f"fp8 scaled GEMM + bias + {act} -> {oname} (fused)",
                              "shape": [8192, 8192, 8192], "ms": r["ms"], "tflops": r["tflops"],
                              "frac_mfma": r["tflops"] / FP8_PEAK_TFLOPS})
            progress(secondary[-1]["op"], r.get("bytes"))
        for (m, n, k) in [(8192, 8192, 8192), (512, 14336, 4096)]:
            r = bench_mx_gemm(tx, torch, m, n, k, K, W)
            secondary.append({"op": "MX-scaled fp8 GEMM (e8m0 per 32 K)", "shape": [m, n, k],
                              "ms": r["ms"], "tflops": r["tflops"],
                              "frac_mfma": r["tflops"] / FP8_PEAK_TFLOPS})
            progress(secondary[-1]["op"] + " " + str(secondary[-1].get("shape", "")), r.get("bytes"))
        for (G, total, n, k) in [(8, 16384, 14336, 4096), (64, 8192, 2048, 4096)]:
            r = bench_fp8_grouped(tx, torch, G, total, n, k, K, W)
            secondary.append({"op": f"grouped fp8 scaled GEMM, {G} experts (one launch)",
                              "shape": [total, n, k], "ms": r["ms"], "tflops": r["tflops"],
                              "frac_mfma": r["tflops"] / FP8_PEAK_TFLOPS,
                              "loop_of_plain_ms": r["ms_loop"], "group_rows": r["sizes"]})
            progress(secondary[-1]["op"], r.get("bytes"))
        r = bench_mx_gemm(tx, torch, 8192, 8192, 8192, K, W, fp4=True)
        secondary.append({"op": "MX-scaled fp4 GEMM (e2m1, e8m0 per 32 K)", "shape": [8192, 8192, 8192],
                          "ms": r["ms"], "tflops": r["tflops"], "frac_mfma": r["tflops"] / FP4_PEAK_TFLOPS})
        progress(secondary[-1]["op"], r.get("bytes"))
        for kind, xdt in (("mx", "f32"), ("mx", "bf16"), ("rowwise", "f32"), ("rowwise", "bf16")):
            r = bench_quant(tx, torch, kind, xdt, max(K, 50), W)
            secondary.append({"op": f"absmax+fp8 quantise ({kind}) {xdt} 8192x8192 -> e4m3fn",
                              "ms": r["ms"], "gbs": r["gbs"], "frac_hbm": r["gbs"] / HBM_PEAK_GBS})
            progress(secondary[-1]["op"], r.get("bytes"))
        for (m, n, k) in [(4096, 4096, 4096), (4095, 4097, 4100)]:
            r = bench_bf16_gemm(tx, torch, m, n, k, K, W)
            secondary.append({"op": "bf16 GEMM", "shape": [m, n, k], "ms": r["ms"],
                              "tflops": r["tflops"], "frac_mfma": r["tflops"] / BF16_PEAK_TFLOPS})
            progress(secondary[-1]["op"] + " " + str(secondary[-1].get("shape", "")), r.get("bytes"))
        for S in (256, 512, 1024, 2048, 4096, 8192):
            r = bench_matmul16(tx, torch, S, K if S >= 4096 else max(K, 50), W)
            secondary.append({"op": "matmul fp16, b row-major K x N, fp16 out (the reference's "
                                    "matmul caller)", "shape": [S, S, S], "ms": r["ms"],
                              "tflops": r["tflops"], "frac_mfma": r["tflops"] / F16_PEAK_TFLOPS,
                              "torch_matmul_ms": r["torch_ms"], "torch_matmul_tflops": r["torch_tflops"]})
            progress(f"matmul fp16 {S}^3", r["bytes"])
        for kind in ("i32", "f32"):
            r = bench_scatter(tx, torch, kind, K, W)
            secondary.append({"op": f"scatter-reduce {kind} 64Mi->65536 Zipf(1.1)", "ms": r["ms"],
                              "gbs": r["gbs"], "frac_hbm": r["gbs"] / HBM_PEAK_GBS,
                              "gupdates_per_s": r["updates_per_s"] / 1e9})
            progress(secondary[-1]["op"] + " " + str(secondary[-1].get("shape", "")), r.get("bytes"))
        for m in (1, 4, 16):
            r = bench_gemv(tx, torch, m, max(K, 50), W)
            secondary.append({"op": "fp8 e5m2 dequant GEMV", "shape": [m, 14336, 4096],
                              "ms": r["ms"], "gbs": r["gbs"], "frac_hbm": r["gbs"] / HBM_PEAK_GBS})
            progress(f"fp8 e5m2 dequant GEMV M={m}", r["bytes"])
        secondary.append({"op": "fp8 decode e4m3fn->fp32 16Mi", "ms": conv["decode_ms"],
                          "gbs": conv["decode_gbs"], "frac_hbm": conv["decode_gbs"] / HBM_PEAK_GBS})
        for size in (67_108_864, 268_435_456):
            for n, (ms, nbytes) in bench_encode_sizes(tx, torch, max(K, 50), W, (size,)).items():
                secondary.append({"op": f"fp8 encode fp32->e4m3fn (RNE) {n >> 20}Mi", "ms": ms,
                                  "gbs": nbytes / (ms * 1e-3) / 1e9,
                                  "frac_hbm": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS})
                progress(secondary[-1]["op"], nbytes)
        for name, (ms, nbytes) in bench_torch_streams(torch, max(K, 50), W).items():
            secondary.append({"op": f"reference: torch {name} 16Mi", "ms": ms,
                              "gbs": nbytes / (ms * 1e-3) / 1e9,
                              "frac_hbm": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS})
        progress("reference: torch cast, copy, sum 16Mi")
        for sname, sdt, dname, ddt in (("bf16", torch.bfloat16, "e4m3fn", torch.float8_e4m3fn),
                                       ("e4m3fn", torch.float8_e4m3fn, "bf16", torch.bfloat16),
                                       ("fp16", torch.float16, "e5m2", torch.float8_e5m2)):
            r = bench_convert_pair(tx, torch, sdt, ddt, max(K, 50), W)
            secondary.append({"op": f"tt.fp_to_fp {sname}->{dname} (RNE) 16Mi", "ms": r["ms"],
                              "gbs": r["gbs"], "frac_hbm": r["gbs"] / HBM_PEAK_GBS})
            progress(secondary[-1]["op"], r.get("bytes"))

    if args.windows:
        with open(args.windows, "w") as f:
            json.dump({"digest": build_digest(), "windows": WINDOWS}, f)
    cpu = None if args.no_cpu else cpu_baseline()
    gemm_traffic = traffic_from_table("fp8 GEMM 8192^3", "tx_gemm_fp8_e4m3fn_e4m3fn_fast")
    conv_traffic = traffic_from_table("fp8 convert 16Mi", "tx_fp8_encode_e4m3fn_rtne_vec")
    line = {
        "metric": METRIC,
        "value": round(gemm["tflops"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(gemm["ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8e4m3fn",
        "data": "synthetic (seeded N(0,1), absmax-quantised; see tests/workloads.py)",
        "config": {"workload": "fp8 e4m3fn scaled GEMM M=N=K=8192, per-row/per-column fp32 "
                               "scales, bf16 output; plus fp32->e4m3fn RNE convert of 16Mi values",
                   "M": 8192, "N": 8192, "K": 8192, "preroll_s": PREROLL_S},
        "roofline": {"bound": "mfma", "achieved": round(gemm["tflops"], 2),
                     "peak": FP8_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(gemm["tflops"] / FP8_PEAK_TFLOPS, 4),
                     "traffic": gemm_traffic[0], "traffic_source": gemm_traffic[1]},
        "secondary": secondary,
        "cpu_baseline": cpu,
        # the headline's second half, last so that a tail of the output keeps it
        "fp8_convert": {"value": round(conv["gbs"], 1), "unit": "GB/s", "ms": round(conv["ms"], 5),
                        "workload": "tt.fp_to_fp fp32 -> e4m3fn, RNE, non-saturating, 16,777,216 values",
                        "roofline": {"bound": "hbm", "achieved": round(conv["gbs"], 1),
                                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                     "frac": round(conv["gbs"] / HBM_PEAK_GBS, 4),
                                     "traffic": conv_traffic[0], "traffic_source": conv_traffic[1]},
                        "buffer_sets": conv["sets"], "ceiling": conv["ceiling"]},
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
