"""GPU: tx_dot_fp8_scaled_grouped_noalloc (the grouped fp8 dot whose group
tile prefix lives in the library's fixed device array instead of allocated
scratch) against tx_dot_fp8_scaled_grouped, through the C ABI.

Both entry points run the same kernels in the same order, so the outputs
must be bit-identical.  Three calls in a row on a stream the library has not
seen: the second smaller than the first (fewer groups and rows, and the
fused epilogue), so it reads a prefix array that still holds the first
call's longer contents; the third large enough for the persistent grouped
kernel (256 x 256 tiles on every CU, K a whole number of 128-byte steps).
Across the three, the library's scratch allocation counter and torch's
reserved memory must not move (the allocating entry point, run afterwards
on another new stream, does move the counter).
"""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _codes(g, *shape):
    c = g.integers(0, 0x7F, size=shape, dtype=np.uint8)   # finite e4m3fn magnitudes
    return c | (g.integers(0, 2, size=shape, dtype=np.uint8) << 7)


def _problem(dev, seed, groups, M, N, K):
    g = np.random.default_rng(seed)
    sizes = g.multinomial(M, np.ones(groups) / groups)
    sizes[groups // 2] = 0                          # an empty group
    sizes[0] += M - sizes.sum()
    off = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)
    t = dict(
        A=torch.from_numpy(_codes(g, M, K)).to(dev).view(torch.float8_e4m3fn),
        B=torch.from_numpy(_codes(g, groups, N, K)).to(dev).view(torch.float8_e4m3fn),
        sa=torch.from_numpy(g.uniform(0.5, 2, M).astype(np.float32) * 1e-3).to(dev),
        sb=torch.from_numpy(g.uniform(0.5, 2, (groups, N)).astype(np.float32) * 1e-3).to(dev),
        bias=torch.from_numpy(g.standard_normal((groups, N)).astype(np.float32)).to(dev),
        off=torch.from_numpy(off).to(dev),
    )
    return t, groups, M, N, K


def _noalloc(tx, t, groups, M, N, K, out, bias, act, c_type, c_scale):
    L, lib = tx.lib, tx._lib
    st = L.tx_dot_fp8_scaled_grouped_noalloc(
        ctypes.c_void_p(t["A"].data_ptr()), lib.FP8E4M3FN, K, ctypes.c_void_p(t["sa"].data_ptr()),
        ctypes.c_void_p(t["B"].data_ptr()), lib.FP8E4M3FN, K, N * K, ctypes.c_void_p(t["sb"].data_ptr()), N,
        None if bias is None else ctypes.c_void_p(bias.data_ptr()), 0 if bias is None else N, act,
        ctypes.c_void_p(out.data_ptr()), c_type, c_scale, N, ctypes.c_void_p(t["off"].data_ptr()),
        groups, M, N, K, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == 0, (st, lib.last_error())


def test_noalloc_grouped_matches_the_allocating_entry(tx, dev):
    tx.init()
    calls = [  # (problem, bias, activation, output dtype, c_scale)
        (_problem(dev, 1, 6, 1000, 384, 256), False, "none", torch.bfloat16, 1.0),
        (_problem(dev, 2, 3, 300, 384, 256), True, "gelu_tanh", torch.float8_e4m3fn, 0.25),
        (_problem(dev, 4, 8, 4096, 4096, 256), False, "none", torch.bfloat16, 1.0),
    ]
    acts = {"none": tx._lib.ACT_NONE, "gelu_tanh": tx._lib.ACT_GELU_TANH}
    ctypes_out = {torch.bfloat16: tx._lib.BF16, torch.float8_e4m3fn: tx._lib.FP8E4M3FN}
    outs = [torch.zeros((M, N), dtype=odt, device=dev) for (_t, _G, M, N, _K), _b, _a, odt, _c in calls]
    torch.cuda.synchronize()
    allocs0, reserved0 = tx.lib.txScratchAllocations(), torch.cuda.memory_reserved(dev)
    s_na = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(s_na):
        for ((t, G, M, N, K), use_bias, act, odt, cs), out in zip(calls, outs):
            _noalloc(tx, t, G, M, N, K, out, t["bias"] if use_bias else None, acts[act], ctypes_out[odt], cs)
    torch.cuda.synchronize()
    assert tx.lib.txScratchAllocations() == allocs0
    assert torch.cuda.memory_reserved(dev) == reserved0
    s_ref = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(s_ref):
        refs = [tx.dot_scaled_rowcol_grouped(t["A"], t["sa"], t["B"], t["sb"], t["off"],
                                             bias=t["bias"] if use_bias else None,
                                             activation=None if act == "none" else act, out_dtype=odt,
                                             out_scale=cs)
                for (t, G, M, N, K), use_bias, act, odt, cs in calls]
    torch.cuda.synchronize()
    assert tx.lib.txScratchAllocations() > allocs0  # the allocating entry's prefix lease on a new stream
    for out, ref in zip(outs, refs):
        assert torch.equal(out.view(torch.uint8), ref.view(torch.uint8))
        assert torch.count_nonzero(out.view(torch.uint8)) > 0


def test_noalloc_grouped_rejects_too_many_groups(tx, dev):
    t, G, M, N, K = _problem(dev, 3, 4, 64, 64, 128)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    st = tx.lib.tx_dot_fp8_scaled_grouped_noalloc(
        ctypes.c_void_p(t["A"].data_ptr()), tx._lib.FP8E4M3FN, K, ctypes.c_void_p(t["sa"].data_ptr()),
        ctypes.c_void_p(t["B"].data_ptr()), tx._lib.FP8E4M3FN, K, N * K, ctypes.c_void_p(t["sb"].data_ptr()), N,
        None, 0, 0, ctypes.c_void_p(out.data_ptr()), tx._lib.BF16, 1.0, N, ctypes.c_void_p(t["off"].data_ptr()),
        16384, M, N, K, None)
    assert st == tx._lib.UNSUPPORTED and "16383" in tx._lib.last_error()
