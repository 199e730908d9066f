"""ctypes wrapper around oracle/libtxoracle.so -- TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg may
import this module, and only as the parity reference (or, for the baseline, as the timed
CPU port).  The product path never routes through it.

Each wrapper mirrors one C function of ``tx_oracle.c``; the C file states which
reference call site fixes each op's semantics.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libtxoracle.so")

E4M3FN = 1
E5M2 = 2
E2M1 = 4    # OCP MX fp4, two per byte (MX dot operands only)
BF16 = 3
F16 = 6
MAX_FINITE = {E4M3FN: 448.0, E5M2: 57344.0}
CODE_DTYPE = {E4M3FN: np.uint8, E5M2: np.uint8, BF16: np.uint16, F16: np.uint16}

_lib = None


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc + OpenMP); make rebuilds it
    when the source is newer than the library."""
    subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "all"], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        I = ctypes.c_int
        L.txo_init.argtypes = []
        L.txo_encode1.argtypes = [I, ctypes.c_float, I]
        L.txo_encode1.restype = ctypes.c_uint8
        L.txo_decode1.argtypes = [I, ctypes.c_uint8]
        L.txo_decode1.restype = ctypes.c_float
        L.txo_encode.argtypes = [P, P, I64, I, I, I]
        L.txo_decode.argtypes = [P, P, I64, I, I]
        L.txo_encode_rtz.argtypes = [P, P, I64, I, I, I]
        L.txo_scatter_add_i32.argtypes = [P, I64, P, P, P, I64]
        L.txo_scatter_add_f32_ref.argtypes = [P, P, I64, P, P, P, I64]
        L.txo_scatter_add_f32_seq.argtypes = [P, I64, P, P, P, I64]
        L.txo_scatter_add_i32_mt.argtypes = [P, I64, P, P, I64, I]
        L.txo_f32_to_bf16.argtypes = [ctypes.c_float]
        L.txo_f32_to_bf16.restype = ctypes.c_uint16
        L.txo_gemm_bf16_rows.argtypes = [P, I64, P, I64, I64, I64, I64, I64,
                                         P, P, I]
        L.txo_gemm16_rows.argtypes = [P, I64, P, I64, I, I, I64, I64, I64, I64, P, I]
        L.txo_gemm16_rows.restype = I
        L.txo_gemm_fp8_scaled_rows.argtypes = [P, I64, P, I64, P, P, I64, I64,
                                               I, I, I64, I64, P, P, I]
        L.txo_gemv_fp8_dequant.argtypes = [P, I64, P, I64, P, I64, I64, I64,
                                           I64, I64, I, P, P, I]
        L.txo_gemm_mx_rows.argtypes = [P, I64, P, I64, P, I64, P, I64, I64, I64, I, I, I64, I64,
                                       P, P, P, I]
        L.txo_e2m1_value.argtypes = [I]
        L.txo_e2m1_value.restype = ctypes.c_double
        L.txo_quant_mx.argtypes = [P, I64, I64, I64, I, P, P, I]
        L.txo_quant_row.argtypes = [P, I64, I64, I64, I, P, P, I]
        L.txo_encode_fmt.argtypes = [P, P, I64, I, I, I, I]
        L.txo_encode_fmt.restype = I
        L.txo_round_rs.argtypes = [P, P, P, I64, I, I]
        L.txo_round_rs.restype = I
        L.txo_init()
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# --------------------------------------------------------------------- fp8
def encode(x, fmt: int, sat: bool, nthreads: int = 0) -> np.ndarray:
    """fp32 -> fp8 codes (uint8), RNE; sat selects the clamp-then-convert form."""
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint8)
    lib().txo_encode(_p(x), _p(out), x.size, fmt, int(bool(sat)), nthreads)
    return out


def encode_rtz(x, fmt: int, sat: bool, nthreads: int = 0) -> np.ndarray:
    """fp32 -> fp8 codes, round toward zero (finite values clamp to max)."""
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint8)
    lib().txo_encode_rtz(_p(x), _p(out), x.size, fmt, int(bool(sat)), nthreads)
    return out


def decode(codes, fmt: int, nthreads: int = 0) -> np.ndarray:
    """fp8 codes -> fp32 (exact; NaN -> 0x7FC00000 with the code's sign)."""
    c = _c(codes, np.uint8)
    out = np.empty(c.shape, np.float32)
    lib().txo_decode(_p(c), _p(out), c.size, fmt, nthreads)
    return out


def encode1(x: float, fmt: int, sat: bool) -> int:
    return int(lib().txo_encode1(fmt, ctypes.c_float(x), int(bool(sat))))


def decode1(code: int, fmt: int) -> float:
    return float(lib().txo_decode1(fmt, code))


# ------------------------------------------------- any format, rs rounding
def encode_fmt(x, fmt: int, rtz: bool = False, sat: bool = False, nthreads: int = 0) -> np.ndarray:
    """fp32 -> codes of format fmt (E4M3FN, E5M2: uint8; BF16, F16: uint16),
    round to nearest even or toward zero, optionally saturating."""
    x = _c(x, np.float32)
    out = np.empty(x.shape, CODE_DTYPE[fmt])
    if lib().txo_encode_fmt(_p(x), _p(out), x.size, fmt, int(bool(rtz)), int(bool(sat)), nthreads):
        raise ValueError(f"format {fmt}")
    return out


F32 = 0


def widen(codes, fmt: int) -> np.ndarray:
    """Codes of format fmt (F32 values, BF16 / F16 uint16 bits, fp8 uint8) ->
    their fp32 values, exactly (every bf16, fp16 and fp8 value is an fp32
    value; NaN stays NaN)."""
    if fmt == F32:
        return np.ascontiguousarray(codes, np.float32)
    if fmt == BF16:
        return (np.asarray(codes, np.uint16).astype(np.uint32) << 16).view(np.float32)
    if fmt == F16:
        return np.asarray(codes, np.uint16).view(np.float16).astype(np.float32)
    return decode(codes, fmt)


def convert(codes, src: int, dst: int, rtz: bool = False, sat: bool = False) -> np.ndarray:
    """tt.fp_to_fp between any two of fp32, bf16, fp16, e4m3fn, e5m2
    (semantic.py:807-827 casts through tt.fp_to_fp, default rounding RTNE at
    :809): the source widened exactly to fp32, then encoded once as an fp32
    source is (encode_fmt: RNE or RTZ, the saturating clamp idiom of
    mxfp8_utils.py:36-38).  An fp32 destination is the widened value
    (saturation does not apply to it, as for the fp8 -> fp32 decode)."""
    x = widen(codes, src)
    if dst == F32:
        return x
    return encode_fmt(x, dst, rtz=rtz, sat=sat)


def round_rs(x, rbits, fmt: int, nthreads: int = 0) -> np.ndarray:
    """fp32 -> codes of format fmt with stochastic rounding (one uint32 of
    random bits per element; definition in tx_oracle.c)."""
    x = _c(x, np.float32)
    r = _c(rbits, np.uint32)
    if r.shape != x.shape:
        raise ValueError("rbits must match x")
    out = np.empty(x.shape, CODE_DTYPE[fmt])
    if lib().txo_round_rs(_p(x), _p(r), _p(out), x.size, fmt, nthreads):
        raise ValueError(f"format {fmt}")
    return out


# ----------------------------------------------------------------- scatter
def scatter_add_i32(bins, idx, val, mask=None) -> np.ndarray:
    """bins (copied) += val at idx; int32 wraps modulo 2^32."""
    b = np.array(bins, dtype=np.int32, copy=True)
    idx = _c(idx, np.int32)
    val = _c(val, np.int32)
    m = None if mask is None else _c(mask, np.uint8)
    lib().txo_scatter_add_i32(_p(b), b.size, _p(idx), _p(val), _p(m), idx.size)
    return b


def scatter_add_i32_mt(nbins, idx, val, nthreads: int = 0) -> np.ndarray:
    b = np.zeros(nbins, np.int32)
    idx = _c(idx, np.int32)
    val = _c(val, np.int32)
    lib().txo_scatter_add_i32_mt(_p(b), nbins, _p(idx), _p(val), idx.size,
                                 nthreads)
    return b


def scatter_add_f32_ref(nbins, idx, val, mask=None):
    """Return (fp64 per-bin sums, fp64 per-bin sums of |v|)."""
    s = np.empty(nbins, np.float64)
    a = np.empty(nbins, np.float64)
    idx = _c(idx, np.int32)
    val = _c(val, np.float32)
    m = None if mask is None else _c(mask, np.uint8)
    lib().txo_scatter_add_f32_ref(_p(s), _p(a), nbins, _p(idx), _p(val), _p(m),
                                  idx.size)
    return s, a


def scatter_add_f32_seq(bins, idx, val, mask=None) -> np.ndarray:
    b = np.array(bins, dtype=np.float32, copy=True)
    idx = _c(idx, np.int32)
    val = _c(val, np.float32)
    m = None if mask is None else _c(mask, np.uint8)
    lib().txo_scatter_add_f32_seq(_p(b), b.size, _p(idx), _p(val), _p(m),
                                  idx.size)
    return b


# -------------------------------------------------------------------- bf16
def f32_to_bf16(x) -> np.ndarray:
    """Vectorised RNE fp32 -> bf16 bits (numpy restatement of the C helper)."""
    u = _c(x, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    r = np.where(nan, (u >> 16) | 0x40, r)
    return r.astype(np.uint16)


def bf16_to_f32(h) -> np.ndarray:
    return (_c(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


# -------------------------------------------------------------------- gemm
def atomic_xchg_seq(bins, idx, val, mask=None):
    """tt.atomic_rmw xchg applied one update at a time in element order, one
    of the orders a device may pick: returns (bins after, old per update; 0
    for dropped updates).  32-bit patterns.  Where indices repeat, results
    from another order differ; atomic_xchg_consistent checks those."""
    b = np.array(bins, copy=True).view(np.uint32)
    v = np.asarray(val).view(np.uint32)
    idx = np.asarray(idx, np.int64)
    old = np.zeros(idx.size, np.uint32)
    live = (idx >= 0) & (idx < b.size)
    if mask is not None:
        live &= np.asarray(mask) != 0
    for i in np.flatnonzero(live):
        k = idx[i]
        old[i] = b[k]
        b[k] = v[i]
    return b.view(np.asarray(bins).dtype), old.view(np.asarray(val).dtype)


def atomic_cas_seq(bins, idx, cmp, val, mask=None):
    """tt.atomic_cas applied one update at a time in element order (one of the
    orders a device may pick): old = bins[k]; if old == cmp (bit for bit):
    bins[k] = val.  Returns (bins after, old per update; 0 for dropped
    updates)."""
    b = np.array(bins, copy=True).view(np.uint32)
    c = np.asarray(cmp).view(np.uint32)
    v = np.asarray(val).view(np.uint32)
    idx = np.asarray(idx, np.int64)
    old = np.zeros(idx.size, np.uint32)
    live = (idx >= 0) & (idx < b.size)
    if mask is not None:
        live &= np.asarray(mask) != 0
    for i in np.flatnonzero(live):
        k = idx[i]
        old[i] = b[k]
        if b[k] == c[i]:
            b[k] = v[i]
    return b.view(np.asarray(bins).dtype), old.view(np.asarray(val).dtype)


def _live(idx, nbins, mask):
    idx = np.asarray(idx, np.int64)
    live = (idx >= 0) & (idx < nbins)
    if mask is not None:
        live &= np.asarray(mask) != 0
    return idx, live


def atomic_xchg_consistent(init, final, idx, val, old, mask=None) -> bool:
    """Whether (final, old) is the outcome of the exchanges applied one at a
    time in SOME order: per bin, the old values of its updates together with
    its final value are its initial value together with its updates' values
    (as multisets), untouched bins keep their value and dropped updates
    return 0.  (In an order, each exchange hands back the value the previous
    one wrote, so the values written form one chain from the initial value.)"""
    init = np.asarray(init).view(np.uint32)
    final = np.asarray(final).view(np.uint32)
    v = np.asarray(val).view(np.uint32)
    o = np.asarray(old).view(np.uint32)
    idx, live = _live(idx, init.size, mask)
    if np.any(o[~live] != 0):
        return False
    touched = np.zeros(init.size, bool)
    touched[idx[live]] = True
    if np.any(final[~touched] != init[~touched]):
        return False
    bins = np.flatnonzero(touched)
    lhs = (np.concatenate([idx[live], bins]), np.concatenate([o[live], final[bins]]))
    rhs = (np.concatenate([idx[live], bins]), np.concatenate([v[live], init[bins]]))
    lo = np.lexsort((lhs[1], lhs[0]))
    ro = np.lexsort((rhs[1], rhs[0]))
    return bool(np.array_equal(lhs[0][lo], rhs[0][ro]) and np.array_equal(lhs[1][lo], rhs[1][ro]))


def atomic_cas_first_wins_consistent(init_value, final, idx, val, old, nbins) -> bool:
    """The first-writer-wins pattern (every bin starts at init_value, every
    update compares against init_value, values distinct and != init_value):
    in any order exactly one update per touched bin sees init_value and
    stores its value, and every other update of that bin sees that value."""
    final = np.asarray(final).view(np.uint32)
    v = np.asarray(val).view(np.uint32)
    o = np.asarray(old).view(np.uint32)
    idx = np.asarray(idx, np.int64)
    e = np.uint32(init_value)
    win = o == e
    touched = np.bincount(idx, minlength=nbins) > 0
    wins = np.bincount(idx[win], minlength=nbins)
    if not np.array_equal(wins, touched.astype(np.int64)):
        return False
    if np.any(final[idx[win]] != v[win]) or np.any(o[~win] != final[idx[~win]]):
        return False
    return bool(np.all(final[~touched] == e))


def atomic_cas_ticket_consistent(final, idx, cmp, old, nbins) -> bool:
    """The ticket pattern (bins start at 0; the updates of a bin with k
    updates compare against 0 .. k-1 once each and store cmp + 1): in any
    order the successful updates (old == cmp) of a bin are exactly those with
    cmp < final, and every other update saw a value in [0, final] other than
    its cmp."""
    final = np.asarray(final, np.int64)
    c = np.asarray(cmp, np.int64)
    o = np.asarray(old, np.int64)
    idx = np.asarray(idx, np.int64)
    ok = o == c
    f = final[idx]
    if not np.array_equal(ok, c < f):
        return False
    if not np.array_equal(np.bincount(idx[ok], minlength=nbins), np.asarray(final, np.int64)):
        return False
    return bool(np.all((o[~ok] >= 0) & (o[~ok] <= f[~ok])))


def gemm_bf16_rows(A, B, r0: int, r1: int, nthreads: int = 0):
    """Rows [r0, r1) of A @ B^T-stored-B (B given as N x K, K contiguous).

    A: uint16 (bf16 bits) M x K, B: uint16 N x K.  Returns (fp32 of the fp64
    accumulation, bf16 RNE bits)."""
    A = _c(A, np.uint16)
    B = _c(B, np.uint16)
    K = A.shape[1]
    N = B.shape[0]
    o32 = np.empty((r1 - r0, N), np.float32)
    o16 = np.empty((r1 - r0, N), np.uint16)
    lib().txo_gemm_bf16_rows(_p(A), K, _p(B), K, N, K, r0, r1, _p(o32),
                             _p(o16), nthreads)
    return o32, o16


def gemm16_rows(A, B, r0: int, r1: int, fmt: int = BF16, b_kn: bool = False,
                out_fmt: int | None = None, nthreads: int = 0):
    """Rows [r0, r1) of A @ B for 16-bit operands (fmt BF16 or F16, both).

    A: uint16 M x K; B: uint16 N x K (b_kn False) or K x N (b_kn True, the
    row-major b of the reference's matmul).  Returns (fp32 of the fp64
    accumulation, its RNE rounding to out_fmt (default fmt) as uint16)."""
    A = _c(A, np.uint16)
    B = _c(B, np.uint16)
    K = A.shape[1]
    N = B.shape[1] if b_kn else B.shape[0]
    o32 = np.empty((r1 - r0, N), np.float32)
    rc = lib().txo_gemm16_rows(_p(A), K, _p(B), B.shape[1], int(bool(b_kn)), fmt, N, K, r0, r1,
                               _p(o32), nthreads)
    if rc:
        raise ValueError(f"txo_gemm16_rows: {rc}")
    o16 = encode_fmt(o32, fmt if out_fmt is None else out_fmt).reshape(o32.shape)
    return o32, o16


def gemm_fp8_scaled_rows(A, B, sa, sb, r0: int, r1: int, fmt_a=E4M3FN,
                         fmt_b=E4M3FN, nthreads: int = 0):
    """Rows [r0, r1) of diag(sa) (Aq . Bq^T) diag(sb); Aq M x K, Bq N x K codes."""
    A = _c(A, np.uint8)
    B = _c(B, np.uint8)
    sa = _c(sa, np.float32)
    sb = _c(sb, np.float32)
    K = A.shape[1]
    N = B.shape[0]
    o32 = np.empty((r1 - r0, N), np.float32)
    o16 = np.empty((r1 - r0, N), np.uint16)
    lib().txo_gemm_fp8_scaled_rows(_p(A), K, _p(B), K, _p(sa), _p(sb), N, K,
                                   fmt_a, fmt_b, r0, r1, _p(o32), _p(o16),
                                   nthreads)
    return o32, o16


def gemm_mx_rows(A, sa, B, sb, r0: int, r1: int, fmt_a=E4M3FN, fmt_b=E4M3FN, nthreads: int = 0,
                 block_max: bool = False):
    """Rows [r0, r1) of the MX-scaled dot: Aq M x K and Bq N x K fp8 codes,
    sa M x ceil(K/32) and sb N x ceil(K/32) e8m0 codes.  Returns (fp32 of
    the fp64 sum, fp32 of the sum of |terms|), and with block_max also the
    sum over K blocks of the block's largest |term|."""
    A = _c(A, np.uint8)
    B = _c(B, np.uint8)
    sa = _c(sa, np.uint8)
    sb = _c(sb, np.uint8)
    # fp4 (format 4) rows hold two K values per byte
    K = A.shape[1] * (2 if fmt_a == E2M1 else 1)
    if K != B.shape[1] * (2 if fmt_b == E2M1 else 1):
        raise ValueError("A and B disagree on K")
    N = B.shape[0]
    o32 = np.empty((r1 - r0, N), np.float32)
    oab = np.empty((r1 - r0, N), np.float32)
    obm = np.empty((r1 - r0, N), np.float32) if block_max else None
    lib().txo_gemm_mx_rows(_p(A), A.shape[1], _p(sa), sa.shape[1], _p(B), B.shape[1], _p(sb), sb.shape[1],
                           N, K, fmt_a, fmt_b, r0, r1, _p(o32), _p(oab), _p(obm), nthreads)
    return (o32, oab, obm) if block_max else (o32, oab)


def e2m1_value(nib: int) -> float:
    """The oracle's decode of one fp4 (e2m1) nibble."""
    return lib().txo_e2m1_value(nib)


ACT_NONE, ACT_RELU, ACT_GELU_TANH, ACT_SILU = 0, 1, 2, 3


def activation(y, act: int):
    """The fp8 GEMM epilogue's activations in float64: relu (NaN kept), the
    tanh form of gelu (Hendrycks & Gimpel), silu."""
    y = np.asarray(y, np.float64)
    if act == ACT_RELU:
        return np.where(y < 0, 0.0, y)
    if act == ACT_GELU_TANH:
        return 0.5 * y * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (y + 0.044715 * y ** 3)))
    if act == ACT_SILU:
        return y / (1.0 + np.exp(-y))
    return y


def gemm_fp8_epilogue(acc, bias, act: int):
    """y = act(acc + bias) in float64 for acc = the scaled fp8 GEMM sums (rows x N)."""
    y = np.asarray(acc, np.float64)
    if bias is not None:
        y = y + np.asarray(bias, np.float64)[None, :]
    return activation(y, act)


def _widen(x):
    """fp32 values of x (fp32, or bf16 given as uint16 bits)."""
    x = np.asarray(x)
    if x.dtype == np.uint16:
        return (x.astype(np.uint32) << 16).view(np.float32)
    return np.ascontiguousarray(x, np.float32)


def quant_mx(x, fmt: int = E4M3FN, nthreads: int = 0):
    """MX quantisation of the rows of x (fp32, or bf16 bits as uint16), K a
    multiple of 32.  Returns (codes uint8 rows x K, e8m0 uint8 rows x K/32)."""
    xf = np.ascontiguousarray(_widen(x))
    rows, K = xf.shape
    q = np.empty((rows, K), np.uint8)
    s = np.empty((rows, K // 32), np.uint8)
    lib().txo_quant_mx(_p(xf), K, rows, K, fmt, _p(q), _p(s), nthreads)
    return q, s


def quant_rowwise(x, fmt: int = E4M3FN, nthreads: int = 0):
    """Row-wise absmax quantisation.  Returns (codes uint8 rows x K, fp32 scales[rows])."""
    xf = np.ascontiguousarray(_widen(x))
    rows, K = xf.shape
    q = np.empty((rows, K), np.uint8)
    s = np.empty((rows,), np.float32)
    lib().txo_quant_row(_p(xf), K, rows, K, fmt, _p(q), _p(s), nthreads)
    return q, s


def gemv_fp8_dequant(x, W, s, group: int = 128, fmt_w=E5M2, nthreads: int = 0):
    """y = x (M x K bf16 bits) times dequant(W (N x K codes), s (N x K/group))^T."""
    x = _c(x, np.uint16)
    W = _c(W, np.uint8)
    s = _c(s, np.float32)
    M, K = x.shape
    N = W.shape[0]
    o32 = np.empty((M, N), np.float32)
    o16 = np.empty((M, N), np.uint16)
    lib().txo_gemv_fp8_dequant(_p(x), K, _p(W), K, _p(s), s.shape[1], M, N, K,
                               group, fmt_w, _p(o32), _p(o16), nthreads)
    return o32, o16
