"""C ABI checks that need no GPU: the library loads, exports every symbol
include/tx_plugin.h declares, serves the plugin table, and turns bad calls
into status codes (never an abort)."""
import ctypes
import os
import re

import pytest
import torch

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# Several checks below pass stand-in device addresses (0x40, 0x100) that the
# call must reject before touching memory.  On a machine with a GPU, a request
# that validation accepts (for instance after the library starts serving a
# conversion it used to refuse) would launch a kernel on them and fault the
# card, so there they are skipped: they belong to the CPU suite.
stand_in_addresses = pytest.mark.skipif(torch.cuda.is_available(),
                                        reason="stand-in device addresses: CPU-only checks")


def declared_symbols():
    with open(os.path.join(REPO, "include", "tx_plugin.h")) as f:
        text = f.read()
    return sorted(set(re.findall(r"TX_API\s+[\w\s\*]+?\b(tx\w+)\s*\(", text)))


def test_exports_every_declared_symbol(tx):
    names = declared_symbols()
    assert len(names) >= 13
    lib = ctypes.CDLL(tx._lib.LIB_PATH)
    for n in names:
        assert hasattr(lib, n), n
    assert sorted(tx._lib.EXPORTED) == names


def test_plugin_table(tx):
    name, version, target, ops = tx.plugin_info()
    assert name == "txamd" and target == "gfx950" and version == tx.version()
    names = [o[0] for o in ops]
    assert {"tt.fp_to_fp", "tt.atomic_rmw", "tt.dot", "tt.dot_scaled.rowcol",
            "tx.gemv_fp8_dequant"} <= set(names)
    assert len(names) == len(set(names))
    # each call returns a fresh table that txReleasePluginInfo frees
    for _ in range(100):
        p = tx.lib.txGetPluginInfo()
        assert p and p.contents.api_version == 1
        tx.lib.txReleasePluginInfo(p)
    tx.lib.txReleasePluginInfo(None)


def test_find_and_invoke_unknown_op(tx):
    assert not tx.lib.txFindOp(b"tt.nope")
    assert tx.lib.txFindOp(b"tt.dot")
    vals = (tx._lib.TxValue * 1)()
    st = tx.lib.txInvokeOp(b"tt.nope", vals, 0, None)
    assert st == tx._lib.UNKNOWN_OP and "tt.nope" in tx._lib.last_error()


def test_table_operand_validation(tx):
    vals = (tx._lib.TxValue * 3)()
    st = tx.lib.txInvokeOp(b"tt.fp_to_fp", vals, 3, None)
    assert st == tx._lib.INVALID_ARGUMENT and "expected 7 or 8 operands" in tx._lib.last_error()
    ops = [tx._lib.TxValue.int(0)] + [tx._lib.TxValue.ptr(None)] * 6
    arr = (tx._lib.TxValue * 7)(*ops)
    st = tx.lib.txInvokeOp(b"tt.fp_to_fp", arr, 7, None)
    assert st == tx._lib.INVALID_ARGUMENT and "must be a pointer" in tx._lib.last_error()


def test_null_operand_array_is_rejected(tx):
    """A NULL operand array with a nonzero count is an argument error for
    every op of the table, at every count (including each op's own, e.g. 9
    and 12 for tt.dot, 7 and 8 for tt.fp_to_fp), never a dereference."""
    for name, _sig in tx.plugin_info()[3]:
        for count in range(1, 26):
            st = tx.lib.txInvokeOp(name.encode(), None, count, None)
            assert st == tx._lib.INVALID_ARGUMENT, (name, count, st)
            assert "operand array is NULL" in tx._lib.last_error()


@pytest.mark.parametrize("call", [
    lambda L: L.tx_fp_to_fp(None, 0, None, 1, -1, 0, 0, None),
    lambda L: L.tx_fp_to_fp(None, 0, None, 1, 10, 0, 0, None),
    lambda L: L.tx_atomic_rmw_scatter(None, 4, 10, None, None, None, 5, 0, None, None),
    lambda L: L.tx_atomic_rmw_scatter(None, 4, 10, None, None, None, 5, 42, None, None),
    lambda L: L.tx_dot_bf16(None, 4, None, 4, None, 4, -1, 4, 4, None),
    lambda L: L.tx_dot_bf16(None, 4, None, 4, None, 4, 4, 4, 4, None),
    lambda L: L.tx_dot_bf16(ctypes.c_void_p(64), 2, ctypes.c_void_p(64), 4, ctypes.c_void_p(64),
                            4, 4, 4, 4, None),
    lambda L: L.tx_dot_fp8_scaled(None, 0, 4, None, None, 1, 4, None, None, 4, 4, 4, 4, None),
    lambda L: L.tx_gemv_fp8_dequant(None, 128, None, 2, 128, None, 1, 0, None, 4, 1, 4, 128, None),
])
@stand_in_addresses
def test_bad_arguments_are_status_codes(tx, call):
    st = call(tx.lib)
    assert st == tx._lib.INVALID_ARGUMENT, (st, tx._lib.last_error())
    assert tx._lib.last_error()


@stand_in_addresses
def test_unsupported_requests(tx):
    L = tx.lib
    st = L.tx_gemv_fp8_dequant(None, 100, None, 2, 100, None, 1, 128, None, 4, 65, 4, 100, None)
    assert st == tx._lib.UNSUPPORTED
    # int32 -> fp32 is no tt.fp_to_fp conversion (served pairs are refused
    # only by type, never reached here)
    st = L.tx_fp_to_fp(ctypes.c_void_p(64), 4, ctypes.c_void_p(64), 0, 10, 0, 0, None)
    assert st == tx._lib.UNSUPPORTED and "is not served" in tx._lib.last_error()
    st = L.tx_fp_to_fp(ctypes.c_void_p(64), 0, ctypes.c_void_p(64), 1, 10, 2, 0, None)
    assert st == tx._lib.UNSUPPORTED and "random bits" in tx._lib.last_error()


def test_no_device_is_reported(tx):
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    with pytest.raises(tx.TxError, match="NO_DEVICE"):
        tx.init()
    st = tx.lib.tx_fp_to_fp(ctypes.c_void_p(64), 0, ctypes.c_void_p(64), 1, 4096, 0, 0, None)
    assert st == tx._lib.NO_DEVICE


def test_zero_sized_calls_succeed_without_device(tx):
    L = tx.lib
    assert L.tx_fp_to_fp(None, 0, None, 1, 0, 0, 0, None) == 0
    assert L.tx_dot_bf16(None, 0, None, 0, None, 0, 0, 5, 5, None) == 0
    assert L.tx_atomic_rmw_scatter(None, 4, 0, None, None, None, 0, 0, None, None) == 0


def test_python_mirror_rejects_cpu_tensors(tx):
    with pytest.raises(ValueError, match="GPU tensors only"):
        tx.fp_to_fp(torch.zeros(4), torch.float8_e4m3fn)
    assert tx.get_fp8_format_name(torch.float8_e5m2) == "e5m2"
    assert tx.get_fp8_format_name(torch.float8_e4m3fn) == "e4m3"
    with pytest.raises(AssertionError):
        tx.get_fp8_format_name(torch.float16)


def test_gemv_wrapper_validates_shapes_and_out(tx):
    """The GEMV mirror checks out, scales and operand shapes before the
    device, so a short or mistyped out can never reach the kernel."""
    x = torch.zeros((4, 256), dtype=torch.bfloat16)
    w = torch.zeros((32, 256), dtype=torch.float8_e5m2)
    s = torch.ones((32, 2), dtype=torch.float32)
    with pytest.raises(ValueError, match="out must be"):
        tx.gemv_fp8_dequant(x, w, s, out=torch.empty((3, 32), dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="out must be"):
        tx.gemv_fp8_dequant(x, w, s, out=torch.empty((4, 32), dtype=torch.float32))
    with pytest.raises(ValueError, match="out must be"):
        tx.gemv_fp8_dequant(x, w, s, out=torch.empty((32, 4), dtype=torch.bfloat16).t())
    with pytest.raises(ValueError, match="incompatible shapes"):
        tx.gemv_fp8_dequant(x, w, torch.ones((32, 1), dtype=torch.float32))
    with pytest.raises(ValueError, match="incompatible shapes"):
        tx.gemv_fp8_dequant(x, w[:, :128], s)
    with pytest.raises(ValueError, match="2-D"):
        tx.gemv_fp8_dequant(x.reshape(-1), w, s)
    with pytest.raises(ValueError, match="GPU tensors only"):
        tx.gemv_fp8_dequant(x, w, s)


_P = ctypes.c_void_p(256)   # a non-NULL, 256-byte aligned stand-in: these calls fail before any access


@pytest.mark.parametrize("call,status,msg", [
    # fused epilogue options: unknown activation, output type, fp8 output scale
    (lambda L: L.tx_dot_fp8_scaled_ex(_P, 1, 16, _P, _P, 1, 16, _P, None, 9, _P, 3, 1.0, 16, 16, 16, 16, None),
     "INVALID_ARGUMENT", "activation"),
    (lambda L: L.tx_dot_fp8_scaled_ex(_P, 1, 16, _P, _P, 1, 16, _P, None, 0, _P, 4, 1.0, 16, 16, 16, 16, None),
     "INVALID_ARGUMENT", "output type"),
    (lambda L: L.tx_dot_fp8_scaled_ex(_P, 1, 16, _P, _P, 1, 16, _P, None, 0, _P, 1, 0.0, 16, 16, 16, 16, None),
     "INVALID_ARGUMENT", "c_scale"),
    # MX dot: fp4 needs an even K; operand and output types; scale strides
    (lambda L: L.tx_dot_scaled_mx(_P, 7, 64, _P, 4, _P, 7, 64, _P, 4, _P, 0, 16, 16, 16, 127, None),
     "INVALID_ARGUMENT", "even K"),
    (lambda L: L.tx_dot_scaled_mx(_P, 3, 128, _P, 4, _P, 1, 128, _P, 4, _P, 0, 16, 16, 16, 128, None),
     "INVALID_ARGUMENT", "fp8 or fp4"),
    (lambda L: L.tx_dot_scaled_mx(_P, 1, 128, _P, 4, _P, 7, 64, _P, 4, _P, 4, 16, 16, 16, 128, None),
     "INVALID_ARGUMENT", "output type"),
    (lambda L: L.tx_dot_scaled_mx(_P, 1, 128, _P, 3, _P, 1, 128, _P, 4, _P, 0, 16, 16, 16, 128, None),
     "INVALID_ARGUMENT", "scale stride"),
    (lambda L: L.tx_dot_scaled_mx(_P, 1, 128, _P, 4, _P, 7, 32, _P, 4, _P, 0, 16, 16, 16, 128, None),
     "INVALID_ARGUMENT", "stride smaller"),
    # grouped / batched fp8 dot
    (lambda L: L.tx_dot_fp8_scaled_grouped(_P, 1, 128, _P, _P, 1, 128, 128 * 64, _P, 64, None, 0, 0, _P, 3,
                                          1.0, 64, None, 2, 100, 64, 128, None),
     "INVALID_ARGUMENT", "offsets"),
    (lambda L: L.tx_dot_fp8_scaled_grouped(_P, 1, 128, _P, _P, 1, 128, 128 * 64, _P, 64, None, 0, 0, _P, 3,
                                          1.0, 64, _P, -1, 100, 64, 128, None),
     "INVALID_ARGUMENT", "negative group"),
    (lambda L: L.tx_dot_fp8_scaled_grouped(_P, 1, 128, _P, _P, 1, 128, 128 * 64, _P, 64, None, 0, 5, _P, 3,
                                          1.0, 64, _P, 2, 100, 64, 128, None),
     "INVALID_ARGUMENT", "activation"),
    (lambda L: L.tx_dot_fp8_scaled_grouped(_P, 1, 120, _P, _P, 1, 120, 120 * 64, _P, 64, None, 0, 0, _P, 3,
                                          1.0, 64, _P, 2, 100, 64, 120, None),
     "UNSUPPORTED", "16-byte"),
    (lambda L: L.tx_dot_fp8_scaled_batched(_P, 6, 128, 128 * 64, _P, 64, _P, 1, 128, 128 * 64, _P, 64, _P, 64,
                                          64 * 64, 2, 64, 64, 128, None),
     "INVALID_ARGUMENT", "fp8"),
    # tt.atomic_rmw on 64-bit and 16-bit bins
    (lambda L: L.tx_atomic_rmw_scatter(_P, 6, 10, _P, _P, None, 5, 0, None, None),
     "INVALID_ARGUMENT", "fadd only"),
    (lambda L: L.tx_atomic_rmw_scatter(_P, 8, 10, _P, _P, None, 5, 1, None, None),
     "INVALID_ARGUMENT", "floating-point bins"),
    (lambda L: L.tx_atomic_rmw_scatter(_P, 10, 10, _P, _P, None, 5, 2, None, None),
     "INVALID_ARGUMENT", "fadd or xchg"),
    (lambda L: L.tx_atomic_rmw_scatter(_P, 8, 10, _P, ctypes.c_void_p(260), None, 5, 0, None, None),
     "INVALID_ARGUMENT", "8-byte aligned"),
    # tt.dot with its accumulator operand
    (lambda L: L.tx_dot_acc(_P, 3, 64, None, _P, 1, 0, 64, None, None, 0, _P, 0, 64, 64, 64, 64, None),
     "INVALID_ARGUMENT", "operands must be"),
    (lambda L: L.tx_dot_acc(_P, 1, 64, _P, _P, 1, 1, 64, _P, None, 0, _P, 0, 64, 64, 64, 64, None),
     "UNSUPPORTED", "N x K"),
    (lambda L: L.tx_dot_acc(_P, 3, 64, None, _P, 3, 0, 64, None, None, 0, _P, 1, 64, 64, 64, 64, None),
     "INVALID_ARGUMENT", "output type"),
    (lambda L: L.tx_dot_acc(_P, 1, 64, None, _P, 2, 0, 64, None, None, 0, _P, 0, 64, 64, 64, 64, None),
     "INVALID_ARGUMENT", "scale vectors"),
    (lambda L: L.tx_dot_acc(_P, 6, 64, _P, _P, 6, 0, 64, _P, None, 0, _P, 0, 64, 64, 64, 64, None),
     "INVALID_ARGUMENT", "scale vectors are for fp8"),
    (lambda L: L.tx_dot_acc(_P, 3, 64, None, _P, 3, 0, 64, None, _P, 64, _P, 3, 64, 64, 64, 64, None),
     "INVALID_ARGUMENT", "only for an fp32 / int32 D"),
    (lambda L: L.tx_dot_acc(_P, 3, 64, None, _P, 3, 0, 64, None, _P, 32, _P, 0, 64, 64, 64, 64, None),
     "INVALID_ARGUMENT", "ldc >= N"),
    # quantisers: K a multiple of the 32-element block; input and code types
    (lambda L: L.tx_quantize_mx(_P, 0, 100, _P, 1, 100, _P, 4, 4, 100, None), "INVALID_ARGUMENT", "multiple"),
    (lambda L: L.tx_quantize_mx(_P, 6, 128, _P, 1, 128, _P, 4, 4, 128, None), "INVALID_ARGUMENT", "fp32 or bf16"),
    (lambda L: L.tx_quantize_rowwise(_P, 0, 128, _P, 3, 128, _P, 4, 128, None), "INVALID_ARGUMENT", "fp8"),
])
@stand_in_addresses
def test_new_entry_points_validate_arguments(tx, call, status, msg):
    """Argument errors of the epilogue, MX, grouped / batched and quantiser
    entry points come back as status codes with a message, before any device
    access."""
    st = call(tx.lib)
    assert st == getattr(tx._lib, status), (st, tx._lib.last_error())
    assert msg in tx._lib.last_error(), tx._lib.last_error()


def test_new_entry_points_zero_sized(tx):
    L = tx.lib
    assert L.tx_dot_fp8_scaled_grouped(None, 1, 0, None, None, 1, 0, 0, None, 0, None, 0, 0, None, 3, 1.0, 0,
                                       None, 0, 0, 0, 0, None) == 0
    assert L.tx_dot_fp8_scaled_batched(None, 1, 0, 0, None, 0, None, 1, 0, 0, None, 0, None, 0, 0, 0, 0, 0, 0,
                                       None) == 0
    assert L.tx_dot_scaled_mx(None, 7, 0, None, 0, None, 7, 0, None, 0, None, 0, 0, 0, 0, 0, None) == 0
    assert L.tx_quantize_mx(None, 0, 0, None, 1, 0, None, 0, 0, 0, None) == 0
