"""GPU parity: tt.atomic_rmw xchg and tt.atomic_cas (scatter form) vs the oracle.

Unique indices: bit-exact against the oracle's sequential form.  Repeated
indices: the device picks the order, so the results are checked by the
oracle's order-free checkers (every bin's exchanges form one chain;
first-writer-wins; the CAS ticket chain).  Masked-off and out-of-range
updates return 0 and change nothing."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DT = {"i32": (torch.int32, np.int32), "u32": (torch.uint32, np.uint32), "f32": (torch.float32, np.float32)}


def _bits(g, n):
    return g.integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32)


def _dev(a, dev, tdt=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t.view(tdt) if tdt is not None else t


def _np(t):
    return t.view(torch.int32).cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("kind", ["i32", "u32", "f32"])
def test_xchg_unique_indices_exact(tx, oracle, dev, kind):
    tdt, _ = DT[kind]
    g = np.random.default_rng(1)
    nb, n = 100_003, 70_001
    init = _bits(g, nb)        # every bit pattern, NaN payloads included
    idx = g.permutation(nb)[:n].astype(np.int32)
    val = _bits(g, n)
    bins = _dev(init.view(np.int32), dev).view(tdt)
    old = tx.atomic_rmw("xchg", bins, _dev(idx, dev), _dev(val.view(np.int32), dev).view(tdt),
                        return_old=True)
    fin, rold = oracle.atomic_xchg_seq(init, idx, val)
    assert np.array_equal(_np(bins), fin) and np.array_equal(_np(old), rold)


def test_xchg_repeated_indices_chain(tx, oracle, dev):
    g = np.random.default_rng(2)
    nb, n = 4096, 1 << 20
    init = _bits(g, nb)
    idx = (g.zipf(1.2, n) % nb).astype(np.int32)
    val = _bits(g, n)
    mask = (g.random(n) < 0.9).astype(np.uint8)
    idx[::97] = -5
    idx[1::97] = nb + 3
    bins = _dev(init.view(np.int32), dev)
    old = tx.atomic_rmw("xchg", bins, _dev(idx, dev), _dev(val.view(np.int32), dev), mask=_dev(mask, dev),
                        return_old=True)
    assert oracle.atomic_xchg_consistent(init, _np(bins), idx, val, _np(old), mask)
    # without old values: every touched bin ends with one of its updates' values
    bins2 = _dev(init.view(np.int32), dev)
    tx.atomic_rmw("xchg", bins2, _dev(idx, dev), _dev(val.view(np.int32), dev), mask=_dev(mask, dev))
    fin = _np(bins2)
    live = (idx >= 0) & (idx < nb) & (mask != 0)
    pairs = set(zip(idx[live].tolist(), val[live].tolist()))
    touched = np.zeros(nb, bool)
    touched[idx[live]] = True
    assert all((b, int(fin[b])) in pairs for b in np.flatnonzero(touched))
    assert np.array_equal(fin[~touched], init[~touched])


@pytest.mark.parametrize("kind", ["i32", "u32", "f32"])
def test_cas_unique_indices_exact(tx, oracle, dev, kind):
    tdt, _ = DT[kind]
    g = np.random.default_rng(3)
    nb, n = 65_537, 50_000
    init = _bits(g, nb)
    idx = g.permutation(nb)[:n].astype(np.int32)
    cmp = np.where(g.random(n) < 0.5, init[idx], _bits(g, n))   # about half match
    val = _bits(g, n)
    bins = _dev(init.view(np.int32), dev).view(tdt)
    old = tx.atomic_cas(bins, _dev(idx, dev), _dev(cmp.view(np.int32), dev).view(tdt),
                        _dev(val.view(np.int32), dev).view(tdt))
    fin, rold = oracle.atomic_cas_seq(init, idx, cmp, val)
    assert np.array_equal(_np(bins), fin) and np.array_equal(_np(old), rold)


def test_cas_fp32_compares_bits(tx, oracle, dev):
    init = np.array([0.0, np.nan, -0.0, 1.5], np.float32)
    idx = np.array([0, 1, 2, 3], np.int32)
    cmp = np.array([-0.0, np.nan, -0.0, 1.5], np.float32)
    val = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    bins = _dev(init, dev)
    old = tx.atomic_cas(bins, _dev(idx, dev), _dev(cmp, dev), _dev(val, dev))
    fin, rold = oracle.atomic_cas_seq(init, idx, cmp, val)
    assert np.array_equal(_np(bins), fin.view(np.uint32)) and np.array_equal(_np(old), rold.view(np.uint32))


def test_cas_first_writer_wins(tx, oracle, dev):
    g = np.random.default_rng(4)
    nb, n = 4096, 1 << 20
    idx = (g.zipf(1.1, n) % nb).astype(np.int32)
    cmp = np.zeros(n, np.int32)
    val = (np.arange(n) + 1).astype(np.int32)
    bins = torch.zeros(nb, dtype=torch.int32, device=dev)
    old = tx.atomic_cas(bins, _dev(idx, dev), _dev(cmp, dev), _dev(val, dev))
    assert oracle.atomic_cas_first_wins_consistent(0, _np(bins), idx, val.view(np.uint32), _np(old), nb)


def test_cas_ticket_chain(tx, oracle, dev):
    g = np.random.default_rng(5)
    nb = 20_000
    k = g.integers(1, 64, nb)
    idx = np.repeat(np.arange(nb), k).astype(np.int32)
    cmp = np.concatenate([g.permutation(kk) for kk in k]).astype(np.int32)
    order = g.permutation(idx.size)
    idx, cmp = idx[order], cmp[order]
    val = (cmp + 1).astype(np.int32)
    bins = torch.zeros(nb, dtype=torch.int32, device=dev)
    old = tx.atomic_cas(bins, _dev(idx, dev), _dev(cmp, dev), _dev(val, dev))
    assert oracle.atomic_cas_ticket_consistent(bins.cpu().numpy(), idx, cmp, old.cpu().numpy(), nb)


def test_cas_mask_range_table_and_errors(tx, oracle, dev):
    init = np.arange(16, dtype=np.int32)
    idx = np.array([0, 16, -1, 3, 5, 5], np.int32)
    cmp = np.array([0, 0, 0, 3, 5, 5], np.int32)
    val = np.array([100, 101, 102, 103, 104, 105], np.int32)
    mask = np.array([1, 1, 1, 0, 1, 1], np.uint8)
    bins = _dev(init, dev)
    old = torch.empty(6, dtype=torch.int32, device=dev)
    tx.invoke("tt.atomic_cas", [bins, _dev(idx, dev), _dev(cmp, dev), _dev(val, dev), _dev(mask, dev), old,
                                16, 6, 4])
    fin, rold = oracle.atomic_cas_seq(init, idx, cmp, val, mask)
    o = old.cpu().numpy()
    assert np.array_equal(o[:4], rold[:4]) and sorted(o[4:].tolist()) == [5, 104]
    b = bins.cpu().numpy()
    assert b[0] == 100 and b[3] == 3 and b[5] in (104, 105)
    # tt.atomic_rmw op 9 is xchg
    bins2 = _dev(init, dev)
    tx.invoke("tt.atomic_rmw", [bins2, _dev(idx[:1], dev), _dev(val[:1], dev), None, None, 16, 1, 4, 9])
    assert bins2.cpu().numpy()[0] == 100
    with pytest.raises(tx.TxError, match="INVALID_ARGUMENT"):
        tx.invoke("tt.atomic_cas", [bins, _dev(idx, dev), _dev(cmp, dev), _dev(val, dev), None, None,
                                    16, 6, 3])  # bf16 bins
    with pytest.raises(ValueError):
        tx.atomic_cas(bins, _dev(idx, dev), _dev(cmp, dev), _dev(val.astype(np.float32), dev))
