"""GPU parity: tt.atomic_rmw scatter on 64-bit bins (int64 / uint64 integer
ops, fp64 fadd, 64-bit xchg) and fp16 / bf16 fadd bins.

The plugin passes every tt.atomic_rmw through (uTLXConversionPatterns.cpp:611),
whatever its element type.  Integer results are order-independent and
checked bit for bit against numpy's sequential ufunc.at (add wraps modulo
2^64).  fp64 sums are held to 1e-12 of the sum of |v| per bin.  fp16 / bf16
bins are checked bit for bit where every partial sum is exact (integer
values) or where a bin takes one update (round(b0 + v) once), and otherwise
within (updates + 1) roundings of the exact sum.  Both the LDS-table path
(bins that fit one table, updates at least twice the bins) and the one
atomic per update path run.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

I64_OPS = {"add": np.add, "max": np.maximum, "min": np.minimum, "umax": np.maximum, "umin": np.minimum,
           "and": np.bitwise_and, "or": np.bitwise_or, "xor": np.bitwise_xor}


def _keys(g, n, nbins, skew=True):
    k = (g.zipf(1.3, n) - 1) % nbins if skew else g.integers(0, nbins, n)
    k = k.astype(np.int32)
    k[g.integers(0, n, n // 50)] = -3            # out of range below
    k[g.integers(0, n, n // 50)] = nbins + 7     # and above
    return k


@pytest.mark.parametrize("op", list(I64_OPS))
@pytest.mark.parametrize("nbins,n", [(1000, 200_000), (18432, 1_000_000), (100_000, 300_000), (5000, 6000)])
def test_i64_ops_exact(tx, dev, op, nbins, n):
    g = np.random.default_rng(nbins + n + len(op))
    unsigned = op in ("umax", "umin")
    k = _keys(g, n, nbins)
    vals = g.integers(-2**63, 2**63 - 1, n, dtype=np.int64, endpoint=True)
    if op == "add":
        vals[: n // 2] = g.integers(-1000, 1000, n // 2)   # small ones too, and wrap-around from the large
    mask = (g.random(n) > 0.1).astype(np.uint8)
    b0 = g.integers(-2**63, 2**63 - 1, nbins, dtype=np.int64, endpoint=True)
    # int64 tensors throughout: the op (umax / umin) carries the unsigned compare
    bins = torch.from_numpy(b0.copy()).to(dev)
    tx.atomic_rmw(op, bins, torch.from_numpy(k).to(dev), torch.from_numpy(vals).to(dev),
                  mask=torch.from_numpy(mask).to(dev))
    live = (k >= 0) & (k < nbins) & (mask != 0)
    npdt = np.uint64 if unsigned else np.int64
    ref = b0.view(npdt).copy()
    with np.errstate(over="ignore"):
        I64_OPS[op].at(ref, k[live], vals.view(npdt)[live])
    got = bins.cpu().numpy().view(npdt)
    assert np.array_equal(got, ref), np.flatnonzero(got != ref)[:5]


def test_i64_add_returns_old_in_some_order(tx, dev):
    """With old values: per bin, the updates sorted by their old value form
    one sequential chain from the initial value to the final one (positive
    values, no wrap)."""
    g = np.random.default_rng(1)
    nbins, n = 300, 50_000
    k = g.integers(0, nbins, n).astype(np.int32)
    vals = g.integers(1, 1000, n).astype(np.int64)
    b0 = g.integers(0, 10**12, nbins).astype(np.int64)
    bins = torch.from_numpy(b0.copy()).to(dev)
    old = tx.atomic_rmw("add", bins, torch.from_numpy(k).to(dev), torch.from_numpy(vals).to(dev),
                        return_old=True).cpu().numpy()
    final = bins.cpu().numpy()
    for b in range(nbins):
        sel = np.flatnonzero(k == b)
        o = old[sel]
        order = np.argsort(o)
        chain = o[order]
        assert chain[0] == b0[b]
        assert np.array_equal(chain[1:], chain[:-1] + vals[sel][order][:-1])
        assert final[b] == chain[-1] + vals[sel][order][-1]


@pytest.mark.parametrize("nbins,n", [(2000, 400_000), (50_000, 200_000)])
def test_f64_fadd(tx, oracle, dev, nbins, n):
    g = np.random.default_rng(nbins)
    k = _keys(g, n, nbins)
    vals = g.standard_normal(n)
    b0 = g.standard_normal(nbins)
    bins = torch.from_numpy(b0.copy()).to(dev)
    tx.atomic_rmw("fadd", bins, torch.from_numpy(k).to(dev), torch.from_numpy(vals).to(dev))
    live = (k >= 0) & (k < nbins)
    exact = b0.copy()
    np.add.at(exact, k[live], vals[live])
    mag = np.abs(b0).copy()
    np.add.at(mag, k[live], np.abs(vals[live]))
    got = bins.cpu().numpy()
    assert np.all(np.abs(got - exact) <= 1e-12 * mag)


def _half(x, dt):
    return torch.from_numpy(np.asarray(x, np.float32)).to(dt)


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("nbins,n", [(3000, 60_000), (36864, 200_000), (50_000, 120_000)])
def test_half_fadd_exact_sums(tx, dev, dt, nbins, n):
    """Integer values whose every partial sum is exact in the format: the
    result is the exact sum whatever the order or the rounding points."""
    g = np.random.default_rng(nbins + n)
    k = g.integers(0, nbins, n).astype(np.int32)
    k[g.integers(0, n, n // 50)] = nbins + 1
    vals = g.integers(-2, 3, n).astype(np.float32)
    b0 = g.integers(-20, 21, nbins).astype(np.float32)
    bins = _half(b0, dt).to(dev)
    tx.atomic_rmw("fadd", bins, torch.from_numpy(k).to(dev), _half(vals, dt).to(dev))
    live = k < nbins
    exact = b0.astype(np.float64).copy()
    np.add.at(exact, k[live], vals[live])
    assert np.abs(exact).max() <= 256
    assert np.array_equal(bins.float().cpu().numpy(), exact.astype(np.float32))


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("nbins", [4000, 40_000])
def test_half_fadd_one_update_per_bin_rounds_once(tx, dev, dt, nbins):
    """A bin that takes one update ends at round(b0 + v) (the fp32 sum rounded
    to nearest even once), bit for bit; the others keep their bits.  nbins =
    4000 takes the LDS table (1.5 nbins masked-off updates make the count),
    40000 one atomic per update."""
    g = np.random.default_rng(nbins + 1)
    perm = g.permutation(nbins)[: nbins // 2].astype(np.int32)
    b0 = _half(g.standard_normal(nbins) * 4, dt)
    v = _half(g.standard_normal(perm.size) * np.exp2(g.integers(-12, 4, perm.size)), dt)
    # 1.5 nbins more updates, all masked off: the LDS-table path where the bins fit one
    extra = g.integers(0, nbins, 3 * nbins // 2).astype(np.int32)
    k = np.concatenate([perm, extra])
    vals = torch.cat([v, _half(g.standard_normal(extra.size), dt)])
    mask = np.concatenate([np.ones(perm.size, np.uint8), np.zeros(extra.size, np.uint8)])
    bins = b0.clone().to(dev)
    tx.atomic_rmw("fadd", bins, torch.from_numpy(k).to(dev), vals.to(dev), mask=torch.from_numpy(mask).to(dev))
    want = b0.clone()
    want[torch.from_numpy(perm).long()] = (b0[torch.from_numpy(perm).long()].float() + v.float()).to(dt)
    assert torch.equal(bins.cpu().view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("dt,u", [(torch.float16, 2.0 ** -11), (torch.bfloat16, 2.0 ** -8)])
@pytest.mark.parametrize("nbins,n", [(2000, 300_000), (60_000, 100_000)])
def test_half_fadd_normal_values(tx, dev, dt, u, nbins, n):
    """N(0,1) updates, Zipf keys: within (updates of the bin + 1) roundings
    of the exact sum, each at most u (|b0| + sum |v|)."""
    g = np.random.default_rng(nbins)
    k = _keys(g, n, nbins)
    vals = _half(g.standard_normal(n), dt)
    b0 = _half(g.standard_normal(nbins), dt)
    bins = b0.clone().to(dev)
    tx.atomic_rmw("fadd", bins, torch.from_numpy(k).to(dev), vals.to(dev))
    live = (k >= 0) & (k < nbins)
    v64 = vals.double().numpy()
    exact = b0.double().numpy().copy()
    np.add.at(exact, k[live], v64[live])
    mag = np.abs(b0.double().numpy())
    np.add.at(mag, k[live], np.abs(v64[live]))
    cnt = np.bincount(k[live], minlength=nbins)
    got = bins.double().cpu().numpy()
    # plus the fp32 rounding of the in-workgroup partial sums
    assert np.all(np.abs(got - exact) <= (cnt + 1) * (u + 2.0 ** -23) * mag)


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float64])
def test_wide_fadd_return_old_unique(tx, dev, dt):
    g = np.random.default_rng(3)
    nbins = 10_000
    perm = g.permutation(nbins).astype(np.int32)
    b0 = torch.from_numpy(g.standard_normal(nbins)).to(dt)
    v = torch.from_numpy(g.standard_normal(nbins)).to(dt)
    bins = b0.clone().to(dev)
    old = tx.atomic_rmw("fadd", bins, torch.from_numpy(perm).to(dev), v.to(dev), return_old=True).cpu()
    assert torch.equal(old, b0[torch.from_numpy(perm).long()])


@pytest.mark.parametrize("dt", [torch.int64, torch.float64])
def test_xchg_64bit(tx, dev, dt):
    """Unique indices: every bin takes its value, old is the initial one;
    repeated ones: each bin ends at one of its updates' values."""
    g = np.random.default_rng(4)
    nbins = 20_000
    perm = g.permutation(nbins).astype(np.int32)
    b0 = torch.from_numpy(g.integers(-2**62, 2**62, nbins)).view(dt) if dt == torch.int64 else \
        torch.from_numpy(g.standard_normal(nbins))
    v = torch.from_numpy(g.integers(-2**62, 2**62, nbins)).view(dt) if dt == torch.int64 else \
        torch.from_numpy(g.standard_normal(nbins))
    bins = b0.clone().to(dev)
    old = tx.atomic_rmw("xchg", bins, torch.from_numpy(perm).to(dev), v.to(dev), return_old=True).cpu()
    assert torch.equal(old.view(torch.int64), b0[torch.from_numpy(perm).long()].view(torch.int64))
    want = b0.clone()
    want[torch.from_numpy(perm).long()] = v
    assert torch.equal(bins.cpu().view(torch.int64), want.view(torch.int64))
    k = g.integers(0, 100, 5000).astype(np.int32)
    w = torch.from_numpy(g.integers(0, 2**40, 5000)).view(dt) if dt == torch.int64 else \
        torch.from_numpy(g.standard_normal(5000))
    bins2 = torch.zeros(100, dtype=dt, device=dev)
    tx.atomic_rmw("xchg", bins2, torch.from_numpy(k).to(dev), w.to(dev))
    got = bins2.cpu().view(torch.int64).numpy()
    wb = w.view(torch.int64).numpy()
    for b in range(100):
        assert got[b] in set(wb[k == b].tolist())


@pytest.mark.parametrize("dt", [torch.int64, torch.float64])
def test_cas_64bit(tx, dev, dt):
    """tt.atomic_cas on 64-bit bins: unique indices give the closed form
    (swap where the bin equals cmp, bit for bit: -0 != +0 for fp64); a ticket
    chain on repeated indices (cmp = the previous ticket) advances each bin
    exactly once per ticket taken."""
    g = np.random.default_rng(7)
    nbins = 20_000
    perm = g.permutation(nbins).astype(np.int32)
    b0 = g.integers(-2**62, 2**62, nbins)
    hit = g.random(nbins) < 0.5
    cmp = np.where(hit, b0[perm], b0[perm] ^ 1)
    val = g.integers(-2**62, 2**62, nbins)
    T = lambda x: torch.from_numpy(np.ascontiguousarray(x)).view(dt)
    bins = T(b0).to(dev)
    old = tx.atomic_cas(bins, torch.from_numpy(perm).to(dev), T(cmp).to(dev), T(val).to(dev)).cpu()
    assert torch.equal(old.view(torch.int64), torch.from_numpy(b0[perm]))
    want = b0.copy()
    want[perm[hit]] = val[hit]
    assert np.array_equal(bins.cpu().view(torch.int64).numpy(), want)
    # ticket chain: every update of a bin tries to move it from t to t + 1 for
    # t = 0 .. count - 1; each bin ends at the number of successful tries, and
    # the successes are exactly the tickets 0 .. final - 1, each once
    k = g.integers(0, 50, 4000).astype(np.int32)
    tickets = np.concatenate([np.arange(np.sum(k == b)) for b in range(50)])
    order = np.concatenate([np.flatnonzero(k == b) for b in range(50)])
    kk = k[order]
    cmpi = tickets.astype(np.int64)
    vali = cmpi + 1
    if dt == torch.float64:
        cmpi, vali = cmpi.astype(np.float64).view(np.int64), vali.astype(np.float64).view(np.int64)
    bins2 = torch.zeros(50, dtype=dt, device=dev)
    old2 = tx.atomic_cas(bins2, torch.from_numpy(kk).to(dev), T(cmpi).to(dev), T(vali).to(dev)).cpu()
    fin = bins2.cpu().numpy()
    for b in range(50):
        ok = old2.numpy()[kk == b] == (T(cmpi).numpy()[kk == b])
        assert fin[b] == ok.sum()
