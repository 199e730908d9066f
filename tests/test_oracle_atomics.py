"""CPU pins of the oracle's tt.atomic_rmw xchg and tt.atomic_cas.

The sequential forms are pinned by their closed forms where indices are
unique (a plain assignment / a masked select).  Where indices repeat the
result depends on the order the updates apply in; the order-free checkers
(atomic_xchg_consistent, atomic_cas_first_wins_consistent,
atomic_cas_ticket_consistent) must accept the sequential result for many
different orders and reject results with a planted mistake (an exchange
that breaks the chain, a CAS that ignores its compare)."""
import numpy as np

import oracle


def _apply_in_order(fn, perm, idx, *arrays):
    """Run fn on the updates in the order `perm`, return (bins, old) with old
    back in the original update order."""
    out_bins, old_p = fn(idx[perm], *[a[perm] for a in arrays])
    old = np.empty_like(old_p)
    old[perm] = old_p
    return out_bins, old


def test_xchg_unique_indices_is_assignment():
    g = np.random.default_rng(1)
    init = g.integers(-2**31, 2**31 - 1, 1000, dtype=np.int64).astype(np.int32)
    idx = g.permutation(1000)[:700].astype(np.int32)
    val = g.integers(-2**31, 2**31 - 1, 700, dtype=np.int64).astype(np.int32)
    fin, old = oracle.atomic_xchg_seq(init, idx, val)
    exp = init.copy()
    exp[idx] = val
    assert np.array_equal(fin, exp) and np.array_equal(old, init[idx])


def test_xchg_mask_and_range():
    init = np.arange(10, dtype=np.int32)
    idx = np.array([0, 11, -1, 3, 3], np.int32)
    val = np.array([100, 101, 102, 103, 104], np.int32)
    mask = np.array([1, 1, 1, 0, 1], np.uint8)
    fin, old = oracle.atomic_xchg_seq(init, idx, val, mask)
    assert list(old) == [0, 0, 0, 0, 3] and fin[0] == 100 and fin[3] == 104
    assert oracle.atomic_xchg_consistent(init, fin, idx, val, old, mask)


def test_xchg_checker_accepts_every_order_and_rejects_mistakes():
    g = np.random.default_rng(2)
    nb, n = 50, 2000
    init = g.integers(0, 1 << 30, nb).astype(np.uint32)
    idx = (g.zipf(1.3, n) % nb).astype(np.int32)
    val = g.integers(0, 1 << 30, n).astype(np.uint32)
    for s in range(5):
        perm = np.random.default_rng(s).permutation(n)
        fin, old = _apply_in_order(lambda i, v: oracle.atomic_xchg_seq(init, i, v), perm, idx, val)
        assert oracle.atomic_xchg_consistent(init, fin, idx, val, old)
    fin, old = oracle.atomic_xchg_seq(init, idx, val)
    bad = old.copy()
    bad[5] = bad[6]                       # one update handed back another's old value
    assert not oracle.atomic_xchg_consistent(init, fin, idx, val, bad)
    bad_fin = fin.copy()
    bad_fin[idx[0]] ^= 1                  # a bin ends with a value nobody wrote
    assert not oracle.atomic_xchg_consistent(init, bad_fin, idx, val, old)
    # an oracle that adds instead of exchanging fails the check
    b = init.copy()
    o = np.empty(n, np.uint32)
    with np.errstate(over="ignore"):
        for i in range(n):
            o[i] = b[idx[i]]
            b[idx[i]] = b[idx[i]] + val[i]
    assert not oracle.atomic_xchg_consistent(init, b, idx, val, o)


def test_cas_unique_indices_is_select():
    g = np.random.default_rng(3)
    init = g.integers(0, 4, 500).astype(np.int32)
    idx = g.permutation(500)[:400].astype(np.int32)
    cmp = g.integers(0, 4, 400).astype(np.int32)
    val = g.integers(100, 200, 400).astype(np.int32)
    fin, old = oracle.atomic_cas_seq(init, idx, cmp, val)
    exp = init.copy()
    exp[idx] = np.where(init[idx] == cmp, val, init[idx])
    assert np.array_equal(fin, exp) and np.array_equal(old, init[idx])


def test_cas_compares_bit_patterns():
    init = np.array([0.0, np.nan, -0.0], np.float32)
    idx = np.array([0, 1, 2], np.int32)
    cmp = np.array([-0.0, np.nan, -0.0], np.float32)   # -0 != +0 bitwise; NaN == same NaN bits
    val = np.array([1.0, 2.0, 3.0], np.float32)
    fin, old = oracle.atomic_cas_seq(init, idx, cmp, val)
    assert fin.view(np.uint32)[0] == np.float32(0.0).view(np.uint32) and fin[1] == 2.0 and fin[2] == 3.0


def _first_wins_case(seed, nb=64, n=3000):
    g = np.random.default_rng(seed)
    idx = g.integers(0, nb, n).astype(np.int32)
    cmp = np.zeros(n, np.uint32)
    val = (np.arange(n) + 1).astype(np.uint32)
    return idx, cmp, val


def test_cas_first_wins_checker():
    nb = 64
    idx, cmp, val = _first_wins_case(4, nb)
    init = np.zeros(nb, np.uint32)
    for s in range(5):
        perm = np.random.default_rng(10 + s).permutation(idx.size)
        fin, old = _apply_in_order(lambda i, c, v: oracle.atomic_cas_seq(init, i, c, v), perm, idx, cmp, val)
        assert oracle.atomic_cas_first_wins_consistent(0, fin, idx, val, old, nb)
    # a CAS that ignores its compare (always swaps) fails the check
    fin, old = oracle.atomic_xchg_seq(init, idx, val)
    assert not oracle.atomic_cas_first_wins_consistent(0, fin, idx, val, old, nb)


def _ticket_case(seed, nb=200):
    g = np.random.default_rng(seed)
    k = g.integers(1, 40, nb)
    idx = np.repeat(np.arange(nb), k).astype(np.int32)
    cmp = np.concatenate([g.permutation(kk) for kk in k]).astype(np.int32)
    order = g.permutation(idx.size)
    return idx[order], cmp[order], (cmp[order] + 1).astype(np.int32)


def test_cas_ticket_checker():
    nb = 200
    idx, cmp, val = _ticket_case(5, nb)
    init = np.zeros(nb, np.int32)
    for s in range(5):
        perm = np.random.default_rng(20 + s).permutation(idx.size)
        fin, old = _apply_in_order(lambda i, c, v: oracle.atomic_cas_seq(init, i, c, v), perm, idx, cmp, val)
        assert oracle.atomic_cas_ticket_consistent(fin, idx, cmp, old, nb)
    fin, old = oracle.atomic_cas_seq(init, idx, cmp, val)
    # plant: one success reported as a failure
    bad = old.copy()
    j = np.flatnonzero(old == cmp)[0]
    bad[j] = cmp[j] + 1
    assert not oracle.atomic_cas_ticket_consistent(fin, idx, cmp, bad, nb)
    # a CAS that ignores its compare fails
    fin2, old2 = oracle.atomic_xchg_seq(init, idx, val)
    assert not oracle.atomic_cas_ticket_consistent(fin2, idx, cmp, old2, nb)
