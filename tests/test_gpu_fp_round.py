"""GPU parity: tt.fp_to_fp to fp16 / bf16 and stochastic rounding (rounding
"rs" with random bits, utlx_fp_to_fp_with_rbits) vs the oracle, bit-exact."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

E4, E5, BF16, F16 = 1, 2, 3, 6
TD = {E4: torch.float8_e4m3fn, E5: torch.float8_e5m2, BF16: torch.bfloat16, F16: torch.float16}
UINT = {E4: torch.uint8, E5: torch.uint8, BF16: torch.int16, F16: torch.int16}
NPU = {E4: np.uint8, E5: np.uint8, BF16: np.uint16, F16: np.uint16}


def inputs(seed, n):
    """All fp32 classes: random bit patterns, scaled normals over a wide
    exponent range (subnormal results included), specials, values at and
    around each format's largest finite value."""
    g = np.random.default_rng(seed)
    raw = g.integers(0, 2 ** 32, size=n // 2, dtype=np.uint64).astype(np.uint32).view(np.float32)
    sc = (g.standard_normal(n - n // 2) * np.exp2(g.integers(-40, 20, size=n - n // 2))).astype(np.float32)
    sp = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 65504.0, 65520.0, 448.0, 464.0, 57344.0,
                   61440.0, 3.3895313892515355e38, 3.4e38, 5.96e-8, 1e-45, -1e-40], np.float32)
    x = np.concatenate([raw, sc, sp, -sp])
    return x


def _codes(t, fmt):
    return t.view(UINT[fmt]).cpu().numpy().view(NPU[fmt])


@pytest.mark.parametrize("fmt", [E4, E5, BF16, F16])
@pytest.mark.parametrize("n", [1_000_003, 130, 65, 17])
def test_stochastic_rounding_matches_oracle(tx, oracle, dev, fmt, n):
    """Vector kernel plus tail at 1,000,003 elements; the reference's ragged
    sizes 130, 65 and 17 (test_tlx.py:5254-5256) on the tail kernel alone."""
    x = inputs(fmt * 1000 + n, n)[:n] if n < 1000 else inputs(fmt, n)
    r = np.random.default_rng(n).integers(0, 2 ** 32, size=x.size, dtype=np.uint64).astype(np.uint32)
    xt = torch.from_numpy(x).to(dev)
    rt = torch.from_numpy(r.view(np.int32)).to(dev)
    got = _codes(tx.stoch_round(xt, TD[fmt], rt), fmt)
    assert np.array_equal(got, oracle.round_rs(x, r, fmt))


@pytest.mark.parametrize("fmt", [BF16, F16])
@pytest.mark.parametrize("rounding", ["rtne", "rtz"])
@pytest.mark.parametrize("sat", [False, True])
def test_fp16_bf16_conversions_match_oracle(tx, oracle, dev, fmt, rounding, sat):
    x = inputs(fmt + 7, 1_000_003)
    got = _codes(tx.fp_to_fp(torch.from_numpy(x).to(dev), TD[fmt], rounding=rounding, saturate=sat), fmt)
    assert np.array_equal(got, oracle.encode_fmt(x, fmt, rtz=rounding == "rtz", sat=sat))


def test_fp16_bf16_rne_agree_with_torch(tx, dev):
    """Finite inputs: the same bits as torch's own conversions on the GPU."""
    x = torch.randn(1 << 20, device=dev) * torch.exp2(torch.randint(-30, 16, (1 << 20,), device=dev).float())
    for dt in (torch.float16, torch.bfloat16):
        assert torch.equal(tx.fp_to_fp(x, dt).view(torch.int16), x.to(dt).view(torch.int16))


@pytest.mark.parametrize("fmt", [E4, E5, BF16, F16])
def test_rs_other_roundings_ignore_rbits(tx, oracle, dev, fmt):
    x = inputs(3, 4099)
    xt = torch.from_numpy(x).to(dev)
    rt = torch.randint(-2 ** 31, 2 ** 31 - 1, (x.size,), dtype=torch.int32, device=dev)
    for rnd in ("rtne", "rtz"):
        a = _codes(tx.fp_to_fp(xt, TD[fmt], rounding=rnd, saturate=True, rbits=rt), fmt)
        b = _codes(tx.fp_to_fp(xt, TD[fmt], rounding=rnd, saturate=True), fmt)
        assert np.array_equal(a, b)


@pytest.mark.parametrize("fmt", [E5, F16])
def test_different_seeds_give_different_results(tx, dev, fmt):
    """As the reference's entropy check (test_tlx.py:5333-5371): values that
    need rounding come out differently for at least 10% of the elements."""
    x = torch.randn(256, device=dev) * 10.0
    g = torch.Generator(device=dev)
    r1 = torch.randint(-2 ** 31, 2 ** 31 - 1, (256,), dtype=torch.int32, device=dev, generator=g.manual_seed(12345))
    r2 = torch.randint(-2 ** 31, 2 ** 31 - 1, (256,), dtype=torch.int32, device=dev, generator=g.manual_seed(67890))
    a = tx.stoch_round(x, TD[fmt], r1).float()
    b = tx.stoch_round(x, TD[fmt], r2).float()
    assert (a != b).sum().item() > 256 * 0.1


def test_rs_rejects_unsupported_types(tx, dev):
    x = torch.randn(128, device=dev)
    r = torch.zeros(128, dtype=torch.int32, device=dev)
    # fp8 source, int32 destination and a missing rbits are errors
    with pytest.raises(tx.TxError, match="INVALID_ARGUMENT"):
        tx.stoch_round(x.to(torch.bfloat16), torch.float16, r)
    with pytest.raises((tx.TxError, ValueError)):
        tx.stoch_round(x, torch.int32, r)
    with pytest.raises(tx.TxError, match="UNSUPPORTED"):
        tx.fp_to_fp(x, torch.float16, rounding="rs")


def test_table_entry_with_rbits_operand(tx, oracle, dev):
    x = inputs(5, 5000)
    r = np.random.default_rng(5).integers(0, 2 ** 32, size=x.size, dtype=np.uint64).astype(np.uint32)
    xt = torch.from_numpy(x).to(dev)
    rt = torch.from_numpy(r.view(np.int32)).to(dev)
    out = torch.empty(x.size, dtype=torch.bfloat16, device=dev)
    tx.invoke("tt.fp_to_fp", [out, xt, x.size, 0, BF16, 2, 1, rt])
    assert np.array_equal(_codes(out, BF16), oracle.round_rs(x, r, BF16))
