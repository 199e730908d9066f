"""GPU parity: tt.atomic_rmw scatter-reduce vs the oracle.

int32 results are bit-exact (addition modulo 2^32 is order independent);
fp32 sums must satisfy |gpu_b - ref_b| <= 1e-5 * sum_{i->b} |v_i| per bin
(ref_b summed in fp64), the order tolerance for atomic fp32 sums.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

F32_TOL = 1e-5


def _run(tx, dev, op, bins_np, idx_np, val_np, mask_np=None, return_old=False):
    # unsigned data travels as int32 bit patterns (the op decides signedness)
    udt = bins_np.dtype == np.uint32
    bins = torch.from_numpy(bins_np.view(np.int32) if udt else bins_np.copy()).clone().to(dev)
    idx = torch.from_numpy(idx_np).to(dev)
    val = torch.from_numpy(val_np.view(np.int32) if udt else val_np).to(dev)
    mask = None if mask_np is None else torch.from_numpy(mask_np).to(dev)
    old = tx.atomic_rmw(op, bins, idx, val, mask=mask, return_old=return_old)
    torch.cuda.synchronize()
    out = bins.cpu().numpy()
    if udt:
        out = out.view(np.uint32)
    if return_old:
        return out, old.cpu().numpy()
    return out


def _check_f32(got, init, nbins, idx, val, oracle, mask=None):
    s, a = oracle.scatter_add_f32_ref(nbins, idx, val, mask)
    ref = init.astype(np.float64) + s
    err = np.abs(got.astype(np.float64) - ref) / np.maximum(a + np.abs(init), 1e-30)
    assert err.max() <= F32_TOL, f"max order error {err.max():.3g} at bin {err.argmax()}"


@pytest.mark.parametrize("nbins", [1, 7, 1000, 36864, 36865, 65536, 1 << 20])
def test_int32_add_random(tx, oracle, dev, nbins):
    g = np.random.default_rng(nbins)
    n = 300_001
    idx = g.integers(-3, nbins + 3, size=n, dtype=np.int64).astype(np.int32)  # some out of range
    val = g.integers(-2 ** 31, 2 ** 31, size=n, dtype=np.int64).astype(np.int32)
    init = g.integers(-1000, 1000, size=nbins, dtype=np.int32)
    got = _run(tx, dev, "add", init, idx, val)
    assert np.array_equal(got, oracle.scatter_add_i32(init, idx, val))


def test_int32_add_masked(tx, oracle, dev):
    g = np.random.default_rng(5)
    n, nbins = 123_457, 50_000
    idx = g.integers(0, nbins, size=n, dtype=np.int32)
    val = g.integers(0, 1000, size=n, dtype=np.int32)
    mask = (g.random(n) < 0.5).astype(np.uint8)
    init = np.zeros(nbins, np.int32)
    got = _run(tx, dev, "add", init, idx, val, mask)
    assert np.array_equal(got, oracle.scatter_add_i32(init, idx, val, mask))


@pytest.mark.parametrize("nbins", [100, 65536, 1 << 20])
def test_fp32_add_random(tx, oracle, dev, nbins):
    g = np.random.default_rng(nbins + 1)
    n = 500_000
    idx = g.integers(0, nbins, size=n, dtype=np.int32)
    val = g.standard_normal(n).astype(np.float32)
    init = g.standard_normal(nbins).astype(np.float32)
    got = _run(tx, dev, "fadd", init, idx, val)
    _check_f32(got, init, nbins, idx, val, oracle)


@pytest.mark.parametrize("nbins", [1000, 1 << 20])
def test_fp32_signed_zeros(tx, dev, nbins):
    """Zero signs follow sequential IEEE addition: -0 updates leave a bin as
    it was, a +0 update turns -0 into +0, untouched bins keep their bits."""
    init = np.where(np.arange(nbins) % 2 == 0, -0.0, 0.0).astype(np.float32)
    idx = np.concatenate([np.repeat(np.arange(0, 100), 3), np.repeat(np.arange(100, 200), 3)])
    val = np.concatenate([np.full(300, -0.0), np.full(300, 0.0)]).astype(np.float32)
    perm = np.random.default_rng(3).permutation(idx.size)
    idx, val = idx[perm].astype(np.int32), val[perm]
    got = _run(tx, dev, "fadd", init, idx, val)
    ref = init.copy()
    np.add.at(ref, idx, val)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    assert np.signbit(got[0]) and not np.signbit(got[100]) and not np.signbit(got[1])


@pytest.mark.parametrize("op,ufunc,dtype", [
    ("max", np.maximum, np.int32), ("min", np.minimum, np.int32),
    ("umax", np.maximum, np.uint32), ("umin", np.minimum, np.uint32),
    ("and", np.bitwise_and, np.uint32), ("or", np.bitwise_or, np.uint32),
    ("xor", np.bitwise_xor, np.uint32)])
@pytest.mark.parametrize("nbins", [2000, 65536])
def test_other_integer_ops(tx, dev, op, ufunc, dtype, nbins):
    # numpy's unbuffered ufunc.at is a sequential restatement of the scatter
    g = np.random.default_rng(nbins)
    n = 200_000
    idx = g.integers(0, nbins, size=n, dtype=np.int32)
    info = np.iinfo(dtype)
    val = g.integers(info.min, info.max, size=n, dtype=np.int64, endpoint=True).astype(dtype)
    init = g.integers(info.min, info.max, size=nbins, dtype=np.int64, endpoint=True).astype(dtype)
    ref = init.copy()
    ufunc.at(ref, idx, val)
    got = _run(tx, dev, op, init, idx, val)
    assert np.array_equal(got, ref)


def _skewed_keys(g, n, nbins, hot_lo, hot_frac):
    """hot_frac of the keys uniform in one 36,864-bin window starting at
    hot_lo (so the single-pass path takes it), the rest uniform over all
    bins, with 1% of the keys out of range (negative or >= nbins)."""
    hot = g.random(n) < hot_frac
    idx = np.where(hot, hot_lo + g.integers(0, 36864, n), g.integers(0, nbins, n)).astype(np.int32)
    bad = g.random(n) < 0.01
    idx[bad] = np.where(g.random(int(bad.sum())) < 0.5, -1 - g.integers(0, 5, int(bad.sum())),
                        nbins + g.integers(0, 5, int(bad.sum()))).astype(np.int32)
    return idx


@pytest.mark.parametrize("nbins,hot_lo", [(65536, 0), (65536, 20480), (100_000, 61440), (147_456, 55296),
                                          (73_728, 36864)])
@pytest.mark.parametrize("op", ["add", "fadd", "max", "xor"])
def test_single_window_with_spill(tx, oracle, dev, nbins, hot_lo, op):
    """More than one window and skewed keys: the one-pass path (the best
    window in LDS, every other in-range update by a global atomic), with
    masked and out-of-range updates, on windows that do not start at 0."""
    g = np.random.default_rng(nbins + hot_lo)
    n = 3_000_000
    idx = _skewed_keys(g, n, nbins, hot_lo, 0.9)
    mask = (g.random(n) < 0.95).astype(np.uint8)
    if op == "fadd":
        val = g.standard_normal(n).astype(np.float32)
        init = g.standard_normal(nbins).astype(np.float32)
        got = _run(tx, dev, op, init, idx, val, mask)
        _check_f32(got, init, nbins, idx, val, oracle, mask)
        return
    ufunc = {"add": np.add, "max": np.maximum, "xor": np.bitwise_xor}[op]
    dtype = np.uint32 if op == "xor" else np.int32
    info = np.iinfo(dtype)
    val = g.integers(info.min, info.max, size=n, dtype=np.int64, endpoint=True).astype(dtype)
    init = g.integers(info.min, info.max, size=nbins, dtype=np.int64, endpoint=True).astype(dtype)
    ref = init.copy()
    live = (idx >= 0) & (idx < nbins) & (mask != 0)
    with np.errstate(over="ignore"):
        ufunc.at(ref, idx[live], val[live])
    got = _run(tx, dev, op, init, idx, val, mask)
    assert np.array_equal(got, ref)


def test_return_old_counter(tx, dev):
    """tt.atomic_rmw's result: each update sees a distinct prior value, as in
    the reference's counter tests (test_tlx.py:7672-7723)."""
    n, nbins = 50_000, 7
    g = np.random.default_rng(9)
    idx = g.integers(0, nbins, size=n, dtype=np.int32)
    val = np.ones(n, np.int32)
    bins, old = _run(tx, dev, "add", np.zeros(nbins, np.int32), idx, val, return_old=True)
    for b in range(nbins):
        sel = np.sort(old[idx == b])
        assert np.array_equal(sel, np.arange(sel.size, dtype=np.int32))
        assert bins[b] == sel.size


def test_empty_and_degenerate(tx, oracle, dev):
    z = np.zeros(0, np.int32)
    got = _run(tx, dev, "add", np.arange(5, dtype=np.int32), z, z)
    assert np.array_equal(got, np.arange(5))
    # nbins = 0: every update is dropped
    bins = torch.zeros(0, dtype=torch.int32, device=dev)
    tx.atomic_rmw("add", bins, torch.zeros(10, dtype=torch.int32, device=dev),
                  torch.ones(10, dtype=torch.int32, device=dev))
    with pytest.raises(tx.TxError, match="INVALID_ARGUMENT"):
        tx.atomic_rmw("fadd", torch.zeros(4, dtype=torch.int32, device=dev),
                      torch.zeros(4, dtype=torch.int32, device=dev),
                      torch.zeros(4, dtype=torch.int32, device=dev))


def test_table_entry_point(tx, oracle, dev):
    g = np.random.default_rng(1)
    idx = torch.from_numpy(g.integers(0, 300, size=10_000, dtype=np.int32)).to(dev)
    val = torch.from_numpy(g.integers(0, 100, size=10_000, dtype=np.int32)).to(dev)
    bins = torch.zeros(300, dtype=torch.int32, device=dev)
    tx.invoke("tt.atomic_rmw", [bins, idx, val, None, None, 300, 10_000, 4, 0])
    ref = oracle.scatter_add_i32(np.zeros(300, np.int32), idx.cpu().numpy(), val.cpu().numpy())
    assert np.array_equal(bins.cpu().numpy(), ref)


@pytest.mark.parametrize("kind", ["i32", "f32"])
def test_zipf_config_full_size(tx, oracle, dev, kind):
    """67,108,864 Zipf(1.1) updates into 65,536 bins."""
    import workloads
    idx, val = workloads.scatter_input(kind=kind)
    nbins = 65536
    init = np.zeros(nbins, np.int32 if kind == "i32" else np.float32)
    got = _run(tx, dev, "add" if kind == "i32" else "fadd", init, idx, val)
    if kind == "i32":
        assert np.array_equal(got, oracle.scatter_add_i32(init, idx, val))
    else:
        _check_f32(got, init, nbins, idx, val, oracle)
