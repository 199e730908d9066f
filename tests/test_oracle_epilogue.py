"""Pins the oracle's fp8 GEMM epilogue activations against PyTorch's own
float64 implementations (relu, gelu with approximate="tanh", silu), and the
bias broadcast over columns."""
import numpy as np
import pytest
import torch


@pytest.mark.parametrize("act,fn", [(1, torch.nn.functional.relu),
                                    (2, lambda t: torch.nn.functional.gelu(t, approximate="tanh")),
                                    (3, torch.nn.functional.silu)])
def test_activations_match_torch(oracle, act, fn):
    g = np.random.default_rng(act)
    y = np.concatenate([g.standard_normal(1000) * 10, [0.0, -0.0, 1e-30, -1e-30, 50.0, -50.0]])
    want = fn(torch.from_numpy(y)).numpy()
    got = oracle.activation(y, act)
    # gelu's 1 + tanh(.) cancels for large negative y (results near 1e-14
    # carry ~1e-16 absolute error in either formula): an absolute floor
    assert np.allclose(got, want, rtol=1e-12, atol=1e-14)


def test_relu_keeps_nan_and_bias_broadcasts(oracle):
    assert np.isnan(oracle.activation(np.array([np.nan]), 1))[0]
    acc = np.arange(6, dtype=np.float64).reshape(2, 3)
    bias = np.array([10.0, -20.0, 0.5])
    assert np.array_equal(oracle.gemm_fp8_epilogue(acc, bias, 0), acc + bias[None, :])
