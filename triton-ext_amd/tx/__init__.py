"""tx: MI355X (gfx950) kernels for the data-parallel ops of the reference's
Triton-extension path, behind the C ABI of libtxamd.so.

Python host mirror of that path.  Each function takes torch tensors that
already live on the GPU (torch provides device memory and the current stream
only) and calls one C entry point; nothing here computes on the CPU and there
is no fallback: a missing library raises at import, a failing call raises
``TxError``.

Op names follow the Triton ops they replace:
  fp_to_fp          tt.fp_to_fp        (semantic.py:807-827; NewOps.cpp:249-303)
  atomic_rmw        tt.atomic_rmw      (uTLXConversionPatterns.cpp:611)
  dot / matmul      tt.dot, bf16       (test_amd_gemm_pipelined.py:184-331)
  dot_scaled_rowcol tt.dot, fp8 + row/column scale epilogue
  gemv_fp8_dequant  fp8 weight-only dequant GEMV
plus the registration surface (plugin_info, invoke) mirroring
tritonGetPluginInfo (support/Export.cpp:58-97).
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import TxError, check, lib

__all__ = [
    "TxError", "fp_to_fp", "stoch_round", "atomic_rmw", "dot", "matmul", "dot_scaled_rowcol",
    "dot_scaled_rowcol_grouped", "dot_scaled_rowcol_batched", "dot_scaled", "quantize_mx", "quantize_rowwise",
    "gemv_fp8_dequant", "plugin_info", "invoke", "get_fp8_format_name",
    "version", "init", "RTNE", "RTZ", "RS",
]

RTNE, RTZ, RS = _lib.RTNE, _lib.RTZ, _lib.RS
_ROUNDING = {"rtne": RTNE, "rtz": RTZ, "rs": RS, RTNE: RTNE, RTZ: RTZ, RS: RS}

_TX_DTYPE = {
    torch.float32: _lib.F32,
    torch.float8_e4m3fn: _lib.FP8E4M3FN,
    torch.float8_e5m2: _lib.FP8E5M2,
    torch.bfloat16: _lib.BF16,
    torch.float16: _lib.F16,
    torch.int32: _lib.I32,
    torch.uint32: _lib.U32,
    torch.int64: _lib.I64,
    torch.uint64: _lib.U64,
    torch.float64: _lib.F64,
    torch.int8: _lib.I8,
}
_FP8 = (torch.float8_e4m3fn, torch.float8_e5m2)


def version() -> str:
    return lib.txVersion().decode()


def init() -> None:
    """Load the gfx950 code objects on the current device (else lazily)."""
    check(lib.txInit())


def get_fp8_format_name(dtype) -> str:
    """Name of an fp8 dtype, as utility.py:92-105 names tl.float8e5/float8e4nv."""
    if dtype == torch.float8_e5m2:
        return "e5m2"
    if dtype == torch.float8_e4m3fn:
        return "e4m3"
    raise AssertionError(
        f"get_fp8_format_name only supports float8_e5m2 (e5m2) and float8_e4m3fn (e4m3), got {dtype}")


def _stream(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _on_gpu(*ts):
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("tx ops take GPU tensors only (no CPU path)")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError("all tensors must be on the same device")
    return dev


# --------------------------------------------------------------------------
def fp_to_fp(x: torch.Tensor, dtype, rounding="rtne", saturate: bool = False,
             out: torch.Tensor | None = None, rbits: torch.Tensor | None = None) -> torch.Tensor:
    """tt.fp_to_fp, elementwise: fp32 -> fp8 (e4m3fn / e5m2), fp16 or bf16;
    fp8 -> fp32; and bf16 / fp16 / fp8 -> any other of those formats (the
    source widened exactly to fp32, then rounded once as an fp32 source is).

    rounding: "rtne" (Triton's default downcast, semantic.py:809), "rtz", or
    "rs" (stochastic, fp32 source only, needs rbits: one int32/uint32 of random
    bits per element, as utlx_fp_to_fp_with_rbits, ops/NewOps.cpp:249-303;
    always saturating).
    saturate: the reference's clamp(x, -max, max)-then-convert idiom
    (mxfp8_utils.py:36-38); without it overflow gives NaN (e4m3fn) / Inf.
    """
    _on_gpu(x, out, rbits)
    if not x.is_contiguous():
        raise ValueError("fp_to_fp needs a contiguous input")
    if x.dtype not in _TX_DTYPE or dtype not in _TX_DTYPE:
        raise ValueError(f"unsupported conversion {x.dtype} -> {dtype}")
    if out is None:
        out = torch.empty(x.shape, dtype=dtype, device=x.device)
    elif out.dtype != dtype or out.numel() != x.numel() or not out.is_contiguous():
        raise ValueError("out must be a contiguous tensor of the target dtype and size")
    if rbits is None:
        check(lib.tx_fp_to_fp(_ptr(x), _TX_DTYPE[x.dtype], _ptr(out), _TX_DTYPE[dtype],
                              x.numel(), _ROUNDING[rounding], int(bool(saturate)), _stream(x)))
        return out
    if rbits.dtype not in (torch.int32, torch.uint32) or rbits.numel() != x.numel() \
            or not rbits.is_contiguous():
        raise ValueError("rbits must be a contiguous int32/uint32 tensor, one word per element")
    check(lib.tx_fp_to_fp_with_rbits(_ptr(x), _TX_DTYPE[x.dtype], _ptr(out), _TX_DTYPE[dtype],
                                     _ptr(rbits), x.numel(), _ROUNDING[rounding],
                                     int(bool(saturate)), _stream(x)))
    return out


def stoch_round(x: torch.Tensor, dtype, rbits: torch.Tensor,
                out: torch.Tensor | None = None) -> torch.Tensor:
    """Stochastic rounding of fp32 x to dtype (float16, bfloat16, float8_e5m2,
    float8_e4m3fn) with one 32-bit random word per element, as the
    reference's tlx.stoch_round(x, dtype, rbits) (test_tlx.py:5138-5153)."""
    return fp_to_fp(x, dtype, rounding="rs", saturate=True, out=out, rbits=rbits)


def atomic_rmw(op: str, bins: torch.Tensor, idx: torch.Tensor, val: torch.Tensor,
               mask: torch.Tensor | None = None, return_old: bool = False):
    """tt.atomic_rmw, scatter form: bins[idx[i]] (op)= val[i] for all i, in place.

    op: add | fadd | max | min | umax | umin | and | or | xor | xchg (as
    tl.atomic_*).  Integer ops take int32, uint32, int64 or uint64 bins;
    fadd takes fp32, fp64, fp16 or bf16 bins (fp16 / bf16 bins are rounded
    once per workgroup partial, summed in fp32); xchg takes any 32- or
    64-bit bins.
    Updates with idx outside [0, len(bins)) or mask[i] == 0 are dropped.
    return_old=True returns, per update, the bin's value before it (the
    tt.atomic_rmw result); that form does no pre-aggregation.
    """
    _on_gpu(bins, idx, val, mask)
    if op not in _lib.RMW:
        raise ValueError(f"unknown rmw op {op!r}")
    if idx.dtype != torch.int32:
        raise ValueError("idx must be int32")
    for t in (bins, idx, val) + ((mask,) if mask is not None else ()):
        if not t.is_contiguous():
            raise ValueError("atomic_rmw needs contiguous tensors")
    if val.numel() != idx.numel() or (mask is not None and mask.numel() != idx.numel()):
        raise ValueError("idx, val (and mask) must have the same number of elements")
    if mask is not None and mask.dtype not in (torch.uint8, torch.bool):
        raise ValueError("mask must be uint8 or bool")
    if val.dtype != bins.dtype:
        raise ValueError("val and bins must have the same dtype")
    old = torch.empty_like(val) if return_old else None
    check(lib.tx_atomic_rmw_scatter(_ptr(bins), _TX_DTYPE[bins.dtype], bins.numel(), _ptr(idx),
                                    _ptr(val), _ptr(mask), idx.numel(), _lib.RMW[op], _ptr(old),
                                    _stream(bins)))
    return old if return_old else bins


def histogram(x: torch.Tensor, num_bins: int, mask: torch.Tensor | None = None) -> torch.Tensor:
    """tt.histogram (tl.histogram(x, num_bins, mask)): int32 counts of the
    values 0 .. num_bins - 1 among x (int32) where mask (if given) is nonzero;
    values outside the range are not counted."""
    _on_gpu(x, mask)
    if x.dtype != torch.int32 or not x.is_contiguous():
        raise ValueError("x must be a contiguous int32 tensor")
    if mask is not None and (mask.numel() != x.numel() or mask.dtype not in (torch.uint8, torch.bool)
                             or not mask.is_contiguous()):
        raise ValueError("mask must be a contiguous uint8 / bool tensor of x's size")
    counts = torch.empty(int(num_bins), dtype=torch.int32, device=x.device)
    check(lib.tx_histogram(_ptr(x), _ptr(mask), x.numel(), _ptr(counts), int(num_bins), _stream(x)))
    return counts


def atomic_cas(bins: torch.Tensor, idx: torch.Tensor, cmp: torch.Tensor, val: torch.Tensor,
               mask: torch.Tensor | None = None, return_old: bool = True):
    """tt.atomic_cas, scatter form: for every i (not masked off, idx in range),
    atomically old[i] = bins[idx[i]]; if old[i] == cmp[i]: bins[idx[i]] = val[i]
    (bit patterns compared bit for bit; int32, uint32, fp32, int64, uint64 or
    fp64 bins).
    Returns old (the tt.atomic_cas result; 0 for dropped updates), or bins
    when return_old is False."""
    _on_gpu(bins, idx, cmp, val, mask)
    if idx.dtype != torch.int32:
        raise ValueError("idx must be int32")
    if bins.dtype not in (torch.int32, torch.uint32, torch.float32, torch.int64, torch.uint64, torch.float64):
        raise ValueError("atomic_cas takes int32, uint32, fp32, int64, uint64 or fp64 bins")
    if cmp.dtype != bins.dtype or val.dtype != bins.dtype:
        raise ValueError("cmp, val and bins must have the same dtype")
    for t in (bins, idx, cmp, val) + ((mask,) if mask is not None else ()):
        if not t.is_contiguous():
            raise ValueError("atomic_cas needs contiguous tensors")
    n = idx.numel()
    if cmp.numel() != n or val.numel() != n or (mask is not None and mask.numel() != n):
        raise ValueError("idx, cmp, val (and mask) must have the same number of elements")
    if mask is not None and mask.dtype not in (torch.uint8, torch.bool):
        raise ValueError("mask must be uint8 or bool")
    old = torch.empty_like(val) if return_old else None
    check(lib.tx_atomic_cas_scatter(_ptr(bins), _TX_DTYPE[bins.dtype], bins.numel(), _ptr(idx),
                                    _ptr(cmp), _ptr(val), _ptr(mask), n, _ptr(old), _stream(bins)))
    return old if return_old else bins


_DOT16 = (torch.bfloat16, torch.float16)


def _dot16(a, b, b_layout, out, out_dtype):
    _on_gpu(a, b, out)
    if a.dtype not in _DOT16 or b.dtype != a.dtype:
        raise ValueError(f"dot takes two bf16 or two fp16 operands (got {a.dtype}, {b.dtype})")
    if a.dim() != 2 or b.dim() != 2:
        raise ValueError("dot takes 2-D operands")
    M, K = a.shape
    if b_layout == _lib.B_NK:
        N = b.shape[0]
        if b.shape[1] != K:
            raise ValueError(f"incompatible shapes {tuple(a.shape)} and {tuple(b.shape)} (N x K)")
    else:
        N = b.shape[1]
        if b.shape[0] != K:
            raise ValueError(f"incompatible shapes {tuple(a.shape)} and {tuple(b.shape)} (K x N)")
    if a.stride(1) != 1 or b.stride(1) != 1:
        raise ValueError("operand rows must be contiguous")
    out_dtype = a.dtype if out_dtype is None else out_dtype
    if out_dtype not in _DOT16:
        raise ValueError("out_dtype must be bf16 or fp16")
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=a.device)
    if out.dtype != out_dtype or tuple(out.shape) != (M, N) or out.stride(1) != 1:
        raise ValueError(f"out must be a row-major {out_dtype} M x N tensor")
    check(lib.tx_dot(_ptr(a), _TX_DTYPE[a.dtype], a.stride(0), _ptr(b), b_layout, b.stride(0),
                     _ptr(out), _TX_DTYPE[out_dtype], out.stride(0), M, N, K, _stream(a)))
    return out


def dot(a: torch.Tensor, b_nk: torch.Tensor, out: torch.Tensor | None = None, *,
        out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """tt.dot on 16-bit operands: out[M,N] = a[M,K] @ b where b is column-major
    K x N, passed as its N x K (K-contiguous) storage ``b_nk``.  Both operands
    bf16 or both fp16; fp32 accumulate; output bf16 or fp16 (default: the
    operands' type), rounded to nearest even."""
    return _dot16(a, b_nk, _lib.B_NK, out, out_dtype)


def dot_kn(a: torch.Tensor, b_kn: torch.Tensor, out: torch.Tensor | None = None, *,
           out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """dot with b stored row-major K x N (rows of N contiguous), the layout of
    the reference's matmul caller; read in place by the persistent tiles,
    otherwise transposed into the library's stream scratch first."""
    return _dot16(a, b_kn, _lib.B_KN, out, out_dtype)


def matmul(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """The reference's matmul(a, b) (test_amd_gemm_pipelined.py:303-331): a
    (M x K, contiguous) times b (K x N), fp16 output allocated here, as its
    `c = torch.empty((M, N), dtype=torch.float16)`.  Operands fp16 (the
    reference's test_op and benchmark) or bf16.  b may be row-major (the
    reference's case), column-major, or any other strides (copied to
    row-major first)."""
    assert a.shape[1] == b.shape[0], "Incompatible dimensions"
    assert a.is_contiguous(), "Matrix A must be contiguous"
    if b.dim() == 2 and b.shape[1] > 0 and b.stride(1) == 1:
        return _dot16(a, b, _lib.B_KN, None, torch.float16)
    if b.dim() == 2 and b.shape[0] > 0 and b.stride(0) == 1:
        return _dot16(a, b.t(), _lib.B_NK, None, torch.float16)
    return _dot16(a, b.contiguous(), _lib.B_KN, None, torch.float16)


def dot_acc(a: torch.Tensor, b: torch.Tensor, acc: torch.Tensor | None = None, *,
            b_layout: str = "nk", scale_a: torch.Tensor | None = None,
            scale_b: torch.Tensor | None = None, out: torch.Tensor | None = None,
            out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """tt.dot with its accumulator operand: out = round(a @ b + acc) in fp32
    (the reference's ``accumulator = tl.dot(a, b, accumulator)``,
    test_amd_gemm_pipelined.py:274).  a: M x K; b: N x K storage of the
    column-major operand (``b_layout="nk"``) or row-major K x N (``"kn"``,
    16-bit operands only).  Operands both bf16 or both fp16, or fp8 (any
    pairing) with fp32 ``scale_a[M]`` and ``scale_b[N]`` multiplying the
    product.  Two fp32 operands give fp32 (ieee products and sums) and two
    int8 operands int32 (exact, wrapping), both with b as N x K.  acc: fp32
    (int32 for int8) M x N or None; out: fp32 (default), bf16 or fp16, and
    may be acc itself when 32-bit (accumulate in place)."""
    _on_gpu(a, b, acc, scale_a, scale_b, out)
    if a.dim() != 2 or b.dim() != 2:
        raise ValueError("dot_acc takes 2-D operands")
    if b_layout not in ("nk", "kn"):
        raise ValueError(f"b_layout must be 'nk' or 'kn' (got {b_layout!r})")
    fp8 = a.dtype in _FP8 and b.dtype in _FP8
    wide = a.dtype in (torch.float32, torch.int8) and b.dtype == a.dtype
    if not fp8 and not wide and not (a.dtype in _DOT16 and b.dtype == a.dtype):
        raise ValueError("dot_acc takes two bf16, fp16, fp32 or int8 operands, or two fp8 "
                         f"(got {a.dtype}, {b.dtype})")
    if (fp8 or wide) and b_layout != "nk":
        raise ValueError("fp8, fp32 and int8 operands take b as its N x K storage")
    if wide:  # fp32 -> fp32, int8 -> int32 (exact, wrapping)
        out_dtype = torch.float32 if a.dtype == torch.float32 else torch.int32
    if fp8 != (scale_a is not None and scale_b is not None) or (not fp8 and (scale_a is not None or
                                                                             scale_b is not None)):
        raise ValueError("scale_a and scale_b go with fp8 operands, and only with them")
    M, K = a.shape
    N = b.shape[0] if b_layout == "nk" else b.shape[1]
    if (b.shape[1] if b_layout == "nk" else b.shape[0]) != K:
        raise ValueError(f"incompatible shapes {tuple(a.shape)} and {tuple(b.shape)} ({b_layout})")
    if a.stride(1) != 1 or b.stride(1) != 1:
        raise ValueError("operand rows must be contiguous")
    if fp8 and (scale_a.dtype != torch.float32 or scale_b.dtype != torch.float32 or scale_a.numel() != M
                or scale_b.numel() != N or not scale_a.is_contiguous() or not scale_b.is_contiguous()):
        raise ValueError("scales must be contiguous fp32 vectors of length M and N")
    acc_dtype = torch.int32 if a.dtype == torch.int8 else torch.float32
    if acc is not None and (acc.dtype != acc_dtype or tuple(acc.shape) != (M, N) or acc.stride(1) != 1):
        raise ValueError(f"acc must be a row-major {acc_dtype} M x N tensor")
    if out_dtype not in (torch.float32, torch.bfloat16, torch.float16, torch.int32):
        raise ValueError("out_dtype must be fp32, bf16 or fp16 (int32 for int8 operands)")
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=a.device)
    if out.dtype != out_dtype or tuple(out.shape) != (M, N) or out.stride(1) != 1:
        raise ValueError(f"out must be a row-major {out_dtype} M x N tensor")
    layout = _lib.B_NK if b_layout == "nk" else _lib.B_KN
    check(lib.tx_dot_acc(_ptr(a), _TX_DTYPE[a.dtype], a.stride(0), _ptr(scale_a), _ptr(b), _TX_DTYPE[b.dtype],
                         layout, b.stride(0), _ptr(scale_b), _ptr(acc), 0 if acc is None else acc.stride(0),
                         _ptr(out), _TX_DTYPE[out_dtype], out.stride(0), M, N, K, _stream(a)))
    return out


_ACT = {None: _lib.ACT_NONE, "none": _lib.ACT_NONE, "relu": _lib.ACT_RELU,
        "gelu_tanh": _lib.ACT_GELU_TANH, "silu": _lib.ACT_SILU}


def dot_scaled_rowcol(a_q: torch.Tensor, scale_a: torch.Tensor, b_q_nk: torch.Tensor,
                      scale_b: torch.Tensor, out: torch.Tensor | None = None,
                      bias: torch.Tensor | None = None, activation: str | None = None,
                      out_dtype: torch.dtype = torch.bfloat16, out_scale: float = 1.0) -> torch.Tensor:
    """fp8 tt.dot with fp32 per-row (scale_a[M]) and per-column (scale_b[N])
    scales: out = bf16(scale_a[:,None] * scale_b[None,:] * (a_q @ b_q)).
    With bias (fp32[N]), activation ("relu", "gelu_tanh", "silu") or another
    out_dtype (fp16, fp32, or fp8 holding y / out_scale with saturation) the
    fused epilogue is applied: out = cast(act(that + bias))."""
    if bias is not None or activation not in (None, "none") or out_dtype != torch.bfloat16:
        return _dot_fp8_ex(a_q, scale_a, b_q_nk, scale_b, out, bias, activation, out_dtype, out_scale)
    _on_gpu(a_q, scale_a, b_q_nk, scale_b, out)
    if a_q.dtype not in _FP8 or b_q_nk.dtype not in _FP8:
        raise ValueError("dot_scaled_rowcol takes fp8 operands")
    if a_q.dim() != 2 or b_q_nk.dim() != 2 or a_q.shape[1] != b_q_nk.shape[1]:
        raise ValueError("incompatible shapes")
    if a_q.stride(1) != 1 or b_q_nk.stride(1) != 1:
        raise ValueError("operands must be K-contiguous")
    M, K = a_q.shape
    N = b_q_nk.shape[0]
    if scale_a.dtype != torch.float32 or scale_b.dtype != torch.float32 or \
            scale_a.numel() != M or scale_b.numel() != N or \
            not scale_a.is_contiguous() or not scale_b.is_contiguous():
        raise ValueError("scales must be contiguous fp32 vectors of length M and N")
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=a_q.device)
    if out.dtype != torch.bfloat16 or tuple(out.shape) != (M, N) or out.stride(1) != 1:
        raise ValueError("out must be a row-major bf16 M x N tensor")
    check(lib.tx_dot_fp8_scaled(_ptr(a_q), _TX_DTYPE[a_q.dtype], a_q.stride(0), _ptr(scale_a),
                                _ptr(b_q_nk), _TX_DTYPE[b_q_nk.dtype], b_q_nk.stride(0),
                                _ptr(scale_b), _ptr(out), out.stride(0), M, N, K, _stream(a_q)))
    return out


def _fp8_checks(*ts):
    for t in ts:
        if t.dtype not in _FP8:
            raise ValueError("fp8 operands expected")
        if t.stride(-1) != 1:
            raise ValueError("operands must be K-contiguous")


def dot_scaled_rowcol_grouped(a_q: torch.Tensor, scale_a: torch.Tensor, b_q_gnk: torch.Tensor,
                              scale_b: torch.Tensor, group_offsets: torch.Tensor,
                              out: torch.Tensor | None = None, bias: torch.Tensor | None = None,
                              activation: str | None = None, out_dtype: torch.dtype = torch.bfloat16,
                              out_scale: float = 1.0) -> torch.Tensor:
    """Grouped fp8 dot with row/column scales (mixture-of-experts layers):
    rows group_offsets[p] .. group_offsets[p+1] of a_q (M x K) against
    expert p's b_q_gnk[p] (N x K, the column-major K x N operand), scaled by
    scale_a[r] and scale_b[p, n], then the fused epilogue of
    dot_scaled_rowcol (bias[p] of a G x N bias, activation, out_dtype, fp8
    outputs holding y / out_scale); bf16 M x N by default.  group_offsets:
    int32 on the device, G + 1 nondecreasing row offsets within 0 .. M; the
    group sizes are never read back to the host."""
    _on_gpu(a_q, scale_a, b_q_gnk, scale_b, group_offsets, out, bias)
    _fp8_checks(a_q, b_q_gnk)
    if a_q.dim() != 2 or b_q_gnk.dim() != 3 or a_q.shape[1] != b_q_gnk.shape[2]:
        raise ValueError("a_q must be M x K and b_q_gnk G x N x K")
    if activation not in _ACT:
        raise ValueError(f"unknown activation {activation!r}")
    if out_dtype not in (torch.bfloat16, torch.float16, torch.float32) + _FP8:
        raise ValueError("out_dtype must be bf16, fp16, fp32 or fp8")
    M, K = a_q.shape
    G, N = b_q_gnk.shape[0], b_q_gnk.shape[1]
    if group_offsets.dtype != torch.int32 or group_offsets.numel() != G + 1 or not group_offsets.is_contiguous():
        raise ValueError("group_offsets must be G + 1 contiguous int32 values")
    if scale_a.dtype != torch.float32 or scale_a.numel() != M or not scale_a.is_contiguous() or \
            scale_b.dtype != torch.float32 or tuple(scale_b.shape) != (G, N) or scale_b.stride(1) != 1:
        raise ValueError("scale_a must be fp32[M] and scale_b fp32[G, N]")
    if bias is not None and (bias.dtype != torch.float32 or tuple(bias.shape) != (G, N) or bias.stride(1) != 1):
        raise ValueError("bias must be fp32[G, N]")
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=a_q.device)
    if out.dtype != out_dtype or tuple(out.shape) != (M, N) or out.stride(1) != 1:
        raise ValueError("out must be a row-major M x N tensor of out_dtype")
    check(lib.tx_dot_fp8_scaled_grouped(_ptr(a_q), _TX_DTYPE[a_q.dtype], a_q.stride(0), _ptr(scale_a),
                                        _ptr(b_q_gnk), _TX_DTYPE[b_q_gnk.dtype], b_q_gnk.stride(1),
                                        b_q_gnk.stride(0), _ptr(scale_b), scale_b.stride(0), _ptr(bias),
                                        0 if bias is None else bias.stride(0), _ACT[activation], _ptr(out),
                                        _TX_DTYPE[out_dtype], float(out_scale), out.stride(0),
                                        _ptr(group_offsets), G, M, N, K, _stream(a_q)))
    return out


def dot_scaled_rowcol_batched(a_q: torch.Tensor, scale_a: torch.Tensor, b_q_bnk: torch.Tensor,
                              scale_b: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """Batched fp8 dot with row/column scales: out[p] = bf16(scale_a[p][:,None]
    * scale_b[p][None,:] * (a_q[p] @ b_q_bnk[p].T)) for a_q B x M x K,
    b_q_bnk B x N x K, scale_a B x M, scale_b B x N (any batch strides)."""
    _on_gpu(a_q, scale_a, b_q_bnk, scale_b, out)
    _fp8_checks(a_q, b_q_bnk)
    if a_q.dim() != 3 or b_q_bnk.dim() != 3 or a_q.shape[0] != b_q_bnk.shape[0] or a_q.shape[2] != b_q_bnk.shape[2]:
        raise ValueError("a_q must be B x M x K and b_q_bnk B x N x K")
    Bt, M, K = a_q.shape
    N = b_q_bnk.shape[1]
    if scale_a.dtype != torch.float32 or tuple(scale_a.shape) != (Bt, M) or scale_a.stride(1) != 1 or \
            scale_b.dtype != torch.float32 or tuple(scale_b.shape) != (Bt, N) or scale_b.stride(1) != 1:
        raise ValueError("scales must be fp32 B x M and B x N")
    if out is None:
        out = torch.empty((Bt, M, N), dtype=torch.bfloat16, device=a_q.device)
    if out.dtype != torch.bfloat16 or tuple(out.shape) != (Bt, M, N) or out.stride(2) != 1:
        raise ValueError("out must be a bf16 B x M x N tensor with unit column stride")
    check(lib.tx_dot_fp8_scaled_batched(_ptr(a_q), _TX_DTYPE[a_q.dtype], a_q.stride(1), a_q.stride(0),
                                        _ptr(scale_a), scale_a.stride(0), _ptr(b_q_bnk),
                                        _TX_DTYPE[b_q_bnk.dtype], b_q_bnk.stride(1), b_q_bnk.stride(0),
                                        _ptr(scale_b), scale_b.stride(0), _ptr(out), out.stride(1),
                                        out.stride(0), Bt, M, N, K, _stream(a_q)))
    return out


def _dot_fp8_ex(a_q, scale_a, b_q_nk, scale_b, out, bias, activation, out_dtype, out_scale):
    _on_gpu(a_q, scale_a, b_q_nk, scale_b, out, bias)
    if a_q.dtype not in _FP8 or b_q_nk.dtype not in _FP8:
        raise ValueError("dot_scaled_rowcol takes fp8 operands")
    if a_q.dim() != 2 or b_q_nk.dim() != 2 or a_q.shape[1] != b_q_nk.shape[1]:
        raise ValueError("incompatible shapes")
    if a_q.stride(1) != 1 or b_q_nk.stride(1) != 1:
        raise ValueError("operands must be K-contiguous")
    if activation not in _ACT:
        raise ValueError(f"unknown activation {activation!r}")
    M, K = a_q.shape
    N = b_q_nk.shape[0]
    if bias is not None and (bias.dtype != torch.float32 or bias.numel() != N or not bias.is_contiguous()):
        raise ValueError("bias must be a contiguous fp32 vector of length N")
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=a_q.device)
    if out.dtype != out_dtype or tuple(out.shape) != (M, N) or out.stride(1) != 1:
        raise ValueError("out must be a row-major M x N tensor of out_dtype")
    check(lib.tx_dot_fp8_scaled_ex(_ptr(a_q), _TX_DTYPE[a_q.dtype], a_q.stride(0), _ptr(scale_a),
                                   _ptr(b_q_nk), _TX_DTYPE[b_q_nk.dtype], b_q_nk.stride(0),
                                   _ptr(scale_b), _ptr(bias), _ACT[activation], _ptr(out),
                                   _TX_DTYPE[out_dtype], float(out_scale), out.stride(0), M, N, K,
                                   _stream(a_q)))
    return out


def _e8m0_bytes(t: torch.Tensor) -> torch.Tensor:
    if t.dtype == torch.uint8:
        return t
    if t.dtype == getattr(torch, "float8_e8m0fnu", None):
        return t.view(torch.uint8)
    raise ValueError("MX scales must be uint8 (e8m0 codes) or float8_e8m0fnu")


_FP4 = getattr(torch, "float4_e2m1fn_x2", None)


def _mx_operand(t, fmt):
    """(tx dtype, logical K) of an MX operand: fp8 by dtype, or fp4 (e2m1)
    packed two per byte (even K in the low nibble) as float4_e2m1fn_x2 or as
    uint8 with format "e2m1"."""
    if fmt not in (None, "e4m3", "e5m2", "e2m1"):
        raise ValueError(f"unknown MX format {fmt!r}")
    if t.dtype in _FP8:
        if fmt is not None and fmt != {torch.float8_e4m3fn: "e4m3", torch.float8_e5m2: "e5m2"}[t.dtype]:
            raise ValueError(f"format {fmt!r} does not match dtype {t.dtype}")
        return _TX_DTYPE[t.dtype], t.shape[1]
    if (_FP4 is not None and t.dtype == _FP4 and fmt in (None, "e2m1")) or \
            (t.dtype == torch.uint8 and fmt == "e2m1"):
        return _lib.FP4E2M1, 2 * t.shape[1]
    raise ValueError("MX operands are fp8 tensors, or fp4 packed as float4_e2m1fn_x2 / uint8 with format 'e2m1'")


def dot_scaled(a_q: torch.Tensor, scale_a: torch.Tensor, b_q_nk: torch.Tensor,
               scale_b: torch.Tensor, out_dtype: torch.dtype = torch.float32,
               out: torch.Tensor | None = None, a_format: str | None = None,
               b_format: str | None = None) -> torch.Tensor:
    """tt.dot_scaled with MX block scales: one e8m0 scale per 32 K elements,
    out[m,n] = sum_k a_q[m,k] 2^(scale_a[m,k//32]-127) * b[k,n] 2^(scale_b[n,k//32]-127),
    fp32 accumulation, rounded to ``out_dtype`` (fp32, bf16 or fp16).
    a_q: M x K fp8, or fp4 (e2m1) M x K/2 bytes; b_q_nk: N x K likewise (the
    column-major K x N operand).  fp4 is packed two per byte with the even K
    index in the low nibble (triton's MXFP4Tensor.to_packed_tensor), given
    as float4_e2m1fn_x2 or as uint8 with ``a_format`` / ``b_format`` "e2m1";
    any pairing of fp4 and fp8 operands.  scale_a: M x ceil(K/32), scale_b:
    N x ceil(K/32), uint8 codes or float8_e8m0fnu."""
    _on_gpu(a_q, scale_a, b_q_nk, scale_b, out)
    if a_q.dim() != 2 or b_q_nk.dim() != 2:
        raise ValueError("incompatible shapes")
    ta, K = _mx_operand(a_q, a_format)
    tb, Kb = _mx_operand(b_q_nk, b_format)
    if K != Kb:
        raise ValueError("incompatible shapes")
    if a_q.stride(1) != 1 or b_q_nk.stride(1) != 1:
        raise ValueError("operands must be K-contiguous")
    M = a_q.shape[0]
    N = b_q_nk.shape[0]
    sa, sb = _e8m0_bytes(scale_a), _e8m0_bytes(scale_b)
    nblk = (K + 31) // 32
    if sa.dim() != 2 or sb.dim() != 2 or tuple(sa.shape) != (M, nblk) or \
            tuple(sb.shape) != (N, nblk) or sa.stride(1) != 1 or sb.stride(1) != 1:
        raise ValueError(f"scales must be row-major {M} x {nblk} and {N} x {nblk}")
    if out_dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise ValueError("out_dtype must be fp32, bf16 or fp16")
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=a_q.device)
    if out.dtype != out_dtype or tuple(out.shape) != (M, N) or out.stride(1) != 1:
        raise ValueError("out must be a row-major M x N tensor of out_dtype")
    check(lib.tx_dot_scaled_mx(_ptr(a_q), ta, a_q.stride(0), _ptr(sa), sa.stride(0),
                               _ptr(b_q_nk), tb, b_q_nk.stride(0), _ptr(sb),
                               sb.stride(0), _ptr(out), _TX_DTYPE[out_dtype], out.stride(0), M, N, K,
                               _stream(a_q)))
    return out


def _quant_checks(x, dtype):
    _on_gpu(x)
    if x.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("x must be fp32 or bf16")
    if dtype not in _FP8:
        raise ValueError("dtype must be torch.float8_e4m3fn or torch.float8_e5m2")
    if x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("x must be a 2-D tensor with contiguous rows")


def quantize_mx(x: torch.Tensor, dtype: torch.dtype = torch.float8_e4m3fn):
    """MX quantisation of x's rows (the reference's _compute_scale_and_quantize,
    mxfp8_utils.py:17-38): returns (q fp8 rows x K, e8m0 scales uint8 rows x K/32)."""
    _quant_checks(x, dtype)
    rows, K = x.shape
    q = torch.empty((rows, K), dtype=dtype, device=x.device)
    s = torch.empty((rows, K // 32), dtype=torch.uint8, device=x.device)
    check(lib.tx_quantize_mx(_ptr(x), _TX_DTYPE[x.dtype], x.stride(0), _ptr(q), _TX_DTYPE[dtype],
                             q.stride(0), _ptr(s), s.stride(0) if s.numel() else max(1, K // 32),
                             rows, K, _stream(x)))
    return q, s


def quantize_rowwise(x: torch.Tensor, dtype: torch.dtype = torch.float8_e4m3fn):
    """Per-row absmax quantisation: returns (q fp8 rows x K, fp32 scales[rows]) with
    x ~= q * scales[:, None] -- the operands of dot_scaled_rowcol (pass B as N x K)."""
    _quant_checks(x, dtype)
    rows, K = x.shape
    q = torch.empty((rows, K), dtype=dtype, device=x.device)
    s = torch.empty((rows,), dtype=torch.float32, device=x.device)
    check(lib.tx_quantize_rowwise(_ptr(x), _TX_DTYPE[x.dtype], x.stride(0), _ptr(q),
                                  _TX_DTYPE[dtype], q.stride(0), _ptr(s), rows, K, _stream(x)))
    return q, s


def gemv_fp8_dequant(x: torch.Tensor, w_q: torch.Tensor, scales: torch.Tensor, group: int = 128,
                     out: torch.Tensor | None = None) -> torch.Tensor:
    """Weight-only fp8 GEMV: out[M,N] = bf16(x[M,K] @ (w_q[N,K] * scales[N, k//group]).T).

    x: bf16 M x K, w_q: fp8 N x K, scales: fp32 N x ceil(K / group), all with
    contiguous rows; out (optional): a row-major bf16 M x N tensor.  Shapes
    and types are checked before the device (on CPU tensors too)."""
    if x.dtype != torch.bfloat16 or w_q.dtype not in _FP8 or scales.dtype != torch.float32:
        raise ValueError("x bf16, w_q fp8, scales fp32")
    if x.dim() != 2 or w_q.dim() != 2 or scales.dim() != 2:
        raise ValueError("x, w_q and scales must be 2-D")
    if group <= 0:
        raise ValueError("group must be positive")
    M, K = x.shape
    N = w_q.shape[0]
    if w_q.shape[1] != K or tuple(scales.shape) != (N, -(-K // group)):
        raise ValueError(f"incompatible shapes: x {tuple(x.shape)}, w_q {tuple(w_q.shape)}, "
                         f"scales {tuple(scales.shape)} (want {N} x {-(-K // group)})")
    if x.stride(1) != 1 or w_q.stride(1) != 1 or scales.stride(1) != 1:
        raise ValueError("rows must be contiguous")
    if out is not None and (out.dtype != torch.bfloat16 or tuple(out.shape) != (M, N) or out.stride(1) != 1):
        raise ValueError("out must be a row-major bf16 M x N tensor")
    _on_gpu(x, w_q, scales, out)
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    check(lib.tx_gemv_fp8_dequant(_ptr(x), x.stride(0), _ptr(w_q), _TX_DTYPE[w_q.dtype],
                                  w_q.stride(0), _ptr(scales), scales.stride(0), group,
                                  _ptr(out), out.stride(0), M, N, K, _stream(x)))
    return out


# --------------------------------------------------------------------------
def plugin_info():
    """The op table, as tritonGetPluginInfo exposes the reference's ops:
    returns (name, version, target, [(op name, signature), ...])."""
    info = lib.txGetPluginInfo()
    if not info:
        raise TxError(_lib.GENERIC_FAILURE, _lib.last_error())
    try:
        p = info.contents
        ops = [(p.ops[i].name.decode(), p.ops[i].signature.decode()) for i in range(p.num_ops)]
        return p.name.decode(), p.version.decode(), p.target.decode(), ops
    finally:
        lib.txReleasePluginInfo(info)


def invoke(name: str, operands, stream=None) -> None:
    """Call a registered op through the table.  operands: tensors (passed as
    device pointers), None (NULL pointer) or ints (integer constants);
    operands[0] is the result slot."""
    vals = (_lib.TxValue * max(1, len(operands)))()
    for i, o in enumerate(operands):
        if o is None:
            vals[i] = _lib.TxValue.ptr(None)
        elif isinstance(o, torch.Tensor):
            vals[i] = _lib.TxValue.ptr(o.data_ptr())
        else:
            vals[i] = _lib.TxValue.int(o)
    if stream is None and torch.cuda.is_available():
        stream = torch.cuda.current_stream().cuda_stream
    check(lib.txInvokeOp(name.encode(), vals, len(operands), ctypes.c_void_p(stream)))
