"""The oracle's fp32 -> fp8 RNE differs from the reference stack's CPU path
(Triton's interpreter, `_convert_float`) only in that path's known defects:
Inf/NaN not special-cased, no overflow handling, truncated subnormals,
ties rounded half up, and mantissa carries lost into odd exponent fields.
CPU only; skipped where Triton is not importable."""
import os
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))


@pytest.mark.parametrize("fmt", [1, 2])
def test_every_mismatch_has_a_known_cause(oracle, fmt):
    pytest.importorskip("triton")
    import interpreter_fp8_mismatch as M
    import workloads
    x = workloads.fp8_input(1 << 20, seed_stream=3)
    counts, n = M.classify(x, fmt)
    assert counts["other"] == 0, counts
    assert counts["inf_nan"] > 0 and counts["subnormal"] > 0 and counts["lost_carry"] > 0, counts
