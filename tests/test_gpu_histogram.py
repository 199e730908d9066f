"""GPU parity: tt.histogram (tx_histogram; passed through beside the atomics
at uTLXConversionPatterns.cpp:605, Triton's tl.histogram(x, num_bins, mask))
against numpy's bincount, bit for bit: values outside [0, num_bins) and
masked-off ones are not counted, and the counts are overwritten.  Bin
counts cover one LDS window, several windows (with the skewed one-pass and
spill path) and the hash-table path; sizes include 0, 1 and ragged ones."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _ref(x, nbins, mask=None):
    live = (x >= 0) & (x < nbins)
    if mask is not None:
        live &= mask != 0
    return np.bincount(x[live], minlength=nbins).astype(np.int32)


@pytest.mark.parametrize("nbins,n,skew", [(1, 1000, False), (100, 4097, False), (36864, 1_000_003, False),
                                          (65536, 16_777_216, True), (65536, 3_000_000, False),
                                          (200_000, 2_000_000, True), (5000, 0, False), (7, 1, False)])
@pytest.mark.parametrize("masked", [False, True])
def test_histogram_matches_bincount(tx, dev, nbins, n, skew, masked):
    g = np.random.default_rng(nbins + n + masked)
    if skew:
        x = ((g.zipf(1.1, n) - 1) % (nbins + 10)).astype(np.int32)
    else:
        x = g.integers(-5, nbins + 5, n).astype(np.int32)
    mask = (g.random(n) > 0.3).astype(np.uint8) if masked else None
    counts = tx.histogram(torch.from_numpy(x).to(dev), nbins,
                          mask=None if mask is None else torch.from_numpy(mask).to(dev))
    assert np.array_equal(counts.cpu().numpy(), _ref(x, nbins, mask))


def test_histogram_overwrites_and_table_op(tx, dev):
    g = np.random.default_rng(2)
    x = torch.from_numpy(g.integers(0, 300, 100_000).astype(np.int32)).to(dev)
    counts = torch.full((300,), 12345, dtype=torch.int32, device=dev)
    V = tx._lib.TxValue
    ops = [V.ptr(counts.data_ptr()), V.ptr(x.data_ptr()), V.ptr(None), V.int(x.numel()), V.int(300)]
    arr = (V * 5)(*ops)
    assert tx.lib.txInvokeOp(b"tt.histogram", arr, 5, None) == 0, tx._lib.last_error()
    torch.cuda.synchronize()
    assert torch.equal(counts, tx.histogram(x, 300))
    assert np.array_equal(counts.cpu().numpy(), _ref(x.cpu().numpy(), 300))
