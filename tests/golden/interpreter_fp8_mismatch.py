"""Mismatch report: the oracle's fp32 -> fp8 round-to-nearest-even (the GPU
kernels' target) against the CPU path of the reference's stack, Triton's
interpreter (`_convert_float` in triton/runtime/interpreter.py of the
installed Triton 3.6.0; the reference pins Triton 7a5d6a3d, ci/triton-hash.txt),
on the convert workload's inputs.

Every mismatch is put in exactly one class, in this order (from reading
_convert_float):
  inf_nan    : +-Inf or NaN input (not special-cased there: e4m3fn +Inf -> 0x78)
  overflow   : |x| above the largest finite value (the exponent is clamped,
               the mantissa kept: no NaN / Inf / saturation)
  subnormal  : |x| below the smallest normal (subnormal outputs truncated)
  tie        : x exactly halfway between two codes (rounded half up there)
  lost_carry : rounding up carries out of the mantissa into an exponent field
               whose lowest bit is 1 (OR-ed, not added, there: 1.9375 -> 1.0)
  other      : none of the above (expected to be empty)

Usage: python tests/golden/interpreter_fp8_mismatch.py [--n N]  (prints markdown)
Test infrastructure: it imports the oracle as the parity reference.
"""
from __future__ import annotations

import argparse
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
for p in (os.path.join(REPO, "oracle"), os.path.join(REPO, "triton-ext_amd"), os.path.join(REPO, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

CLASSES = ["inf_nan", "overflow", "subnormal", "tie", "lost_carry", "other"]
MBITS = {1: 3, 2: 2}
BIAS = {1: 7, 2: 15}
MAXV = {1: 448.0, 2: 57344.0}


def interpreter_rne(x: np.ndarray, fmt: int) -> np.ndarray:
    import triton.language as tl
    from triton._C.libtriton import ir
    from triton.runtime.interpreter import _convert_float
    dt = tl.float8e4nv if fmt == 1 else tl.float8e5
    return np.asarray(_convert_float(x, tl.float32, dt, ir.ROUNDING_MODE.RTNE), np.uint8)


def classify(x: np.ndarray, fmt: int):
    """Returns (mismatch count per class, number of inputs)."""
    import oracle
    o = oracle.encode(x, fmt, False)
    t = interpreter_rne(x, fmt)
    mis = o != t
    a = np.abs(x.astype(np.float64))
    finite = np.isfinite(x)
    c = oracle.encode_rtz(x, fmt, True) & 0x7F  # truncated magnitude code
    lo = oracle.decode(c.astype(np.uint8), fmt).astype(np.float64)
    hi = oracle.decode(np.minimum(c + 1, 0x7F).astype(np.uint8), fmt).astype(np.float64)
    m = MBITS[fmt]
    min_normal = 2.0 ** (1 - BIAS[fmt])
    om = (o & 0x7F).astype(np.int64)
    cls = np.full(x.size, len(CLASSES) - 1, np.int8)
    rest = mis.copy()

    def take(mask, k):
        nonlocal rest
        sel = rest & mask
        cls[sel] = k
        rest &= ~sel

    with np.errstate(invalid="ignore"):
        take(~finite, 0)
        take(finite & (a > MAXV[fmt]), 1)
        take(finite & (a < min_normal), 2)
        take(finite & (2 * a == lo + hi), 3)
        carry = ((c & ((1 << m) - 1)) == (1 << m) - 1) & (om == c + 1) & (((c >> m) & 1) == 1)
        take(finite & carry, 4)
    counts = {k: int(np.count_nonzero(mis & (cls == i))) for i, k in enumerate(CLASSES)}
    return counts, x.size


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--n", type=int, default=16_777_216)
    args = ap.parse_args()
    import workloads
    x = workloads.fp8_input(args.n)
    print(f"# fp32 -> fp8 RNE: oracle vs Triton interpreter, {x.size:,} convert-workload inputs\n")
    print("| format | " + " | ".join(CLASSES) + " | total mismatches | share |")
    print("|---" * (len(CLASSES) + 3) + "|")
    for fmt, name in ((1, "e4m3fn"), (2, "e5m2")):
        counts, n = classify(x, fmt)
        tot = sum(counts.values())
        print(f"| {name} | " + " | ".join(f"{counts[k]:,}" for k in CLASSES) + f" | {tot:,} | {100 * tot / n:.3f}% |")


if __name__ == "__main__":
    main()
