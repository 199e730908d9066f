"""ctypes binding of libtxamd.so (the C ABI declared in include/tx_plugin.h).

The library is required: importing this module raises if it is missing, and
there is no CPU or PyTorch fallback for any op.
"""
from __future__ import annotations

import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libtxamd.so")

# tx_status
SUCCESS = 0
GENERIC_FAILURE = 1
INVALID_ARGUMENT = 2
UNSUPPORTED = 3
NO_DEVICE = 4
CODE_OBJECT_ERROR = 5
LAUNCH_ERROR = 6
UNKNOWN_OP = 7
STATUS_NAMES = {
    0: "TX_SUCCESS", 1: "TX_GENERIC_FAILURE", 2: "TX_INVALID_ARGUMENT",
    3: "TX_UNSUPPORTED", 4: "TX_NO_DEVICE", 5: "TX_CODE_OBJECT_ERROR",
    6: "TX_LAUNCH_ERROR", 7: "TX_UNKNOWN_OP",
}

# tx_dtype
F32, FP8E4M3FN, FP8E5M2, BF16, I32, U32, F16, FP4E2M1, I64, U64, F64, I8 = 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11
ACT_NONE, ACT_RELU, ACT_GELU_TANH, ACT_SILU = 0, 1, 2, 3
# tx_rounding (ops/NewOps.cpp:270-286 numbering)
RTNE, RTZ, RS = 0, 1, 2
# tx_rmw_op
RMW = {"add": 0, "fadd": 1, "max": 2, "min": 3, "umax": 4, "umin": 5,
       "and": 6, "or": 7, "xor": 8, "xchg": 9}
# tx_value_kind
VALUE_PTR, VALUE_INT = 0, 1
# tx_b_layout
B_NK, B_KN = 0, 1

# Every symbol include/tx_plugin.h declares.
EXPORTED = [
    "txGetPluginInfo", "txReleasePluginInfo", "txFindOp", "txInvokeOp",
    "txGetLastError", "txInit", "txShutdown", "txVersion", "txScratchAllocations", "txStreamCeiling",
    "tx_fp_to_fp", "tx_fp_to_fp_with_rbits", "tx_atomic_rmw_scatter", "tx_atomic_cas_scatter", "tx_histogram",
    "tx_dot_bf16", "tx_dot", "tx_dot_acc",
    "tx_dot_fp8_scaled", "tx_dot_fp8_scaled_ex", "tx_dot_fp8_scaled_grouped",
    "tx_dot_fp8_scaled_grouped_noalloc", "tx_dot_fp8_scaled_batched",
    "tx_dot_scaled_mx", "tx_quantize_mx", "tx_quantize_rowwise",
    "tx_gemv_fp8_dequant",
]


class TxError(RuntimeError):
    """A tx_status other than TX_SUCCESS, with the library's message."""

    def __init__(self, status: int, message: str):
        self.status = status
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")


class TxValue(ctypes.Structure):
    class _U(ctypes.Union):
        _fields_ = [("ptr", ctypes.c_void_p), ("i", ctypes.c_int64)]

    _fields_ = [("kind", ctypes.c_int32), ("reserved", ctypes.c_int32), ("u", _U)]

    @classmethod
    def ptr(cls, p):
        v = cls()
        v.kind = VALUE_PTR
        v.u.ptr = p
        return v

    @classmethod
    def int(cls, i):
        v = cls()
        v.kind = VALUE_INT
        v.u.i = int(i)
        return v


OpFn = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.POINTER(TxValue), ctypes.c_size_t, ctypes.c_void_p)


class TxOpInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("fn", OpFn), ("signature", ctypes.c_char_p)]


class TxPluginInfo(ctypes.Structure):
    _fields_ = [("api_version", ctypes.c_uint32), ("name", ctypes.c_char_p),
                ("version", ctypes.c_char_p), ("ops", ctypes.POINTER(TxOpInfo)),
                ("num_ops", ctypes.c_size_t), ("target", ctypes.c_char_p)]


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python triton-ext_amd/build.py` "
            "(the tx ops have no fallback)")
    L = ctypes.CDLL(LIB_PATH)
    P, I64, I, VP = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p
    L.txGetPluginInfo.restype = ctypes.POINTER(TxPluginInfo)
    L.txGetPluginInfo.argtypes = []
    L.txReleasePluginInfo.argtypes = [ctypes.POINTER(TxPluginInfo)]
    L.txReleasePluginInfo.restype = None
    L.txFindOp.argtypes = [ctypes.c_char_p]
    L.txFindOp.restype = ctypes.POINTER(TxOpInfo)
    L.txInvokeOp.argtypes = [ctypes.c_char_p, ctypes.POINTER(TxValue), ctypes.c_size_t, VP]
    L.txInvokeOp.restype = I
    L.txGetLastError.restype = ctypes.c_char_p
    L.txGetLastError.argtypes = []
    L.txInit.restype = I
    L.txInit.argtypes = []
    L.txShutdown.restype = None
    L.txShutdown.argtypes = []
    L.txVersion.restype = ctypes.c_char_p
    L.txVersion.argtypes = []
    L.txScratchAllocations.restype = ctypes.c_uint64
    L.txScratchAllocations.argtypes = []
    L.txStreamCeiling.restype = I
    L.txStreamCeiling.argtypes = [I, P, P, I64, VP]
    L.tx_fp_to_fp.argtypes = [P, I, P, I, I64, I, I, VP]
    L.tx_fp_to_fp.restype = I
    L.tx_fp_to_fp_with_rbits.argtypes = [P, I, P, I, P, I64, I, I, VP]
    L.tx_fp_to_fp_with_rbits.restype = I
    L.tx_atomic_rmw_scatter.argtypes = [P, I, I64, P, P, P, I64, I, P, VP]
    L.tx_atomic_rmw_scatter.restype = I
    L.tx_histogram.argtypes = [P, P, I64, P, I64, VP]
    L.tx_histogram.restype = I
    L.tx_atomic_cas_scatter.argtypes = [P, I, I64, P, P, P, P, I64, P, VP]
    L.tx_atomic_cas_scatter.restype = I
    L.tx_dot_bf16.argtypes = [P, I64, P, I64, P, I64, I64, I64, I64, VP]
    L.tx_dot_bf16.restype = I
    L.tx_dot.argtypes = [P, I, I64, P, I, I64, P, I, I64, I64, I64, I64, VP]
    L.tx_dot.restype = I
    L.tx_dot_acc.argtypes = [P, I, I64, P, P, I, I, I64, P, P, I64, P, I, I64, I64, I64, I64, VP]
    L.tx_dot_acc.restype = I
    L.tx_dot_fp8_scaled.argtypes = [P, I, I64, P, P, I, I64, P, P, I64, I64, I64, I64, VP]
    L.tx_dot_fp8_scaled.restype = I
    L.tx_dot_fp8_scaled_ex.argtypes = [P, I, I64, P, P, I, I64, P, P, I, P, I, ctypes.c_float,
                                       I64, I64, I64, I64, VP]
    L.tx_dot_fp8_scaled_ex.restype = I
    L.tx_dot_fp8_scaled_grouped.argtypes = [P, I, I64, P, P, I, I64, I64, P, I64, P, I64, I, P, I, ctypes.c_float,
                                            I64, P, I64, I64, I64, I64, P]
    L.tx_dot_fp8_scaled_grouped.restype = I
    L.tx_dot_fp8_scaled_grouped_noalloc.argtypes = [P, I, I64, P, P, I, I64, I64, P, I64, P, I64, I, P, I, ctypes.c_float,
                                            I64, P, I64, I64, I64, I64, P]
    L.tx_dot_fp8_scaled_grouped_noalloc.restype = I
    L.tx_dot_fp8_scaled_batched.argtypes = [P, I, I64, I64, P, I64, P, I, I64, I64, P, I64, P, I64, I64, I64,
                                            I64, I64, I64, P]
    L.tx_dot_fp8_scaled_batched.restype = I
    L.tx_dot_scaled_mx.argtypes = [P, I, I64, P, I64, P, I, I64, P, I64, P, I, I64, I64, I64, I64, VP]
    L.tx_dot_scaled_mx.restype = I
    L.tx_quantize_mx.argtypes = [P, I, I64, P, I, I64, P, I64, I64, I64, VP]
    L.tx_quantize_mx.restype = I
    L.tx_quantize_rowwise.argtypes = [P, I, I64, P, I, I64, P, I64, I64, VP]
    L.tx_quantize_rowwise.restype = I
    L.tx_gemv_fp8_dequant.argtypes = [P, I64, P, I, I64, P, I64, I64, P, I64, I64, I64, I64, VP]
    L.tx_gemv_fp8_dequant.restype = I
    return L


lib = _load()


def last_error() -> str:
    m = lib.txGetLastError()
    return m.decode() if m else ""


def check(status: int) -> None:
    if status != SUCCESS:
        raise TxError(status, last_error())
