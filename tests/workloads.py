"""Seeded synthetic inputs for the five measured configurations.

Host-side numpy generators (identical bytes on any host for a given seed), used
by bench.py and the tests.  Each returns numpy arrays; callers copy them to
the GPU.  Base seed 20261201; config c uses seed ``BASE ^ (c << 32)``.

  c=1 fp8 round trip: 16,777,216 fp32 values z * 2^u (z ~ N(0,1), u ~ U[-10, 9])
      with 1 % of positions replaced by special values.
  c=2 scatter-reduce: 67,108,864 updates into 65,536 bins, bin = Zipf(1.1) rank - 1;
      int32 values U[0, 1000) or fp32 values N(0, 1).
  c=3 bf16 GEMM: A M x K and B N x K (B column-major K x N), U(-1, 1) -> bf16 RNE.
  c=4 fp8 scaled GEMM: A, B ~ N(0, 1); per-row / per-column absmax scales,
      e4m3fn RNE with saturation of x * (448 / absmax).
  c=5 dequant GEMV: x bf16 N(0, 1) M x K; W ~ N(0, 0.02) N x K quantised to
      e5m2 with one fp32 scale per 128 consecutive k (absmax / 57344).
  c=6 MX-scaled dot: A, B ~ N(0, 1); one e8m0 scale per 32 consecutive k of
      each row, absmax / fmax rounded up to a power of two, then fp8 RNE with
      saturation (the reference's MX quantiser, mxfp8_utils.py:17-38).
"""
from __future__ import annotations

import numpy as np
import torch

BASE_SEED = 20261201


def rng(config: int, stream: int = 0) -> np.random.Generator:
    return np.random.default_rng([BASE_SEED ^ (config << 32), stream])


# ----------------------------------------------------------------- fp8 (c=1)
def fp8_specials() -> np.ndarray:
    """The special fp32 values mixed into the fp8 conversion input."""
    def f(bits):
        return np.array(bits, dtype=np.uint32).view(np.float32)

    def around(v):
        b = np.array([v], dtype=np.float32).view(np.uint32)[0]
        return [b - 1, b, b + 1]

    bits = [0x00000000, 0x80000000, 0x7F800000, 0xFF800000,       # +-0, +-Inf
            0x7FC00000, 0xFFC00000, 0x7F800001, 0xFF800001,       # NaNs
            0x00000001, 0x007FFFFF, 0x80000001, 0x807FFFFF]       # fp32 denormals
    edges = [448.0, 464.0, 480.0, 57344.0, 61440.0, 65536.0,
             2.0 ** -6, 2.0 ** -9, 2.0 ** -10, 1.5 * 2.0 ** -9,  # e4m3fn min normal / subnormal
             2.0 ** -14, 2.0 ** -16, 2.0 ** -17, 1.5 * 2.0 ** -16]  # e5m2
    for e in edges:
        for s in (1.0, -1.0):
            bits += around(np.float32(s * e))
    return f(bits)


def fp8_input(n: int = 16_777_216, seed_stream: int = 0) -> np.ndarray:
    g = rng(1, seed_stream)
    z = g.standard_normal(n, dtype=np.float32)
    u = g.uniform(-10.0, 9.0, n).astype(np.float32)
    x = (z * np.exp2(u)).astype(np.float32)
    sp = fp8_specials()
    nspec = max(1, n // 100) if n >= 100 else 0
    if nspec:
        pos = g.choice(n, size=nspec, replace=False)
        rand_den = g.integers(1, 1 << 23, size=nspec, dtype=np.uint32).view(np.float32)
        vals = np.resize(sp, nspec).copy()
        # every fourth special is a random fp32 denormal
        vals[3::4] = rand_den[3::4]
        x[pos] = vals
    return x


# ------------------------------------------------------------- scatter (c=2)
def zipf_cdf(nbins: int = 65536, s: float = 1.1) -> np.ndarray:
    w = np.arange(1, nbins + 1, dtype=np.float64) ** (-s)
    c = np.cumsum(w)
    return c / c[-1]


def scatter_input(n: int = 67_108_864, nbins: int = 65536, kind: str = "i32",
                  s: float = 1.1, seed_stream: int = 0):
    """Returns (idx int32[n], val int32|float32[n])."""
    g = rng(2, seed_stream)
    cdf = zipf_cdf(nbins, s)
    idx = np.searchsorted(cdf, g.random(n), side="right").astype(np.int32)
    np.minimum(idx, nbins - 1, out=idx)
    if kind == "i32":
        val = g.integers(0, 1000, size=n, dtype=np.int32)
    elif kind == "f32":
        val = g.standard_normal(n, dtype=np.float32)
    else:
        raise ValueError(kind)
    return idx, val


# ------------------------------------------------------------- bf16 (c=3)
def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 RNE bits via torch's CPU conversion."""
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16) \
        .view(torch.int16).numpy().view(np.uint16)


def bf16_gemm_input(M: int, N: int, K: int, seed_stream: int = 0):
    """Returns (A bits uint16[M,K], B bits uint16[N,K])."""
    g = rng(3, seed_stream)
    a = g.uniform(-1.0, 1.0, size=(M, K)).astype(np.float32)
    b = g.uniform(-1.0, 1.0, size=(N, K)).astype(np.float32)
    return to_bf16_bits(a), to_bf16_bits(b)


def matmul16_input(M: int, N: int, K: int, fp16: bool = True, seed_stream: int = 0):
    """The reference matmul test's operands (test_amd_gemm_pipelined.py:338-343:
    torch.randn a (M x K) and b (K x N), fp16): returns (A bits uint16[M,K],
    B bits uint16[K,N], row-major), fp16 or bf16 (RNE) codes of N(0,1) values."""
    g = rng(7, seed_stream)
    a = g.standard_normal((M, K), dtype=np.float32)
    b = g.standard_normal((K, N), dtype=np.float32)
    if fp16:
        return a.astype(np.float16).view(np.uint16), b.astype(np.float16).view(np.uint16)
    return to_bf16_bits(a), to_bf16_bits(b)


# -------------------------------------------------------------- fp8 (c=4)
def _quant_rows(x: np.ndarray, fmax: float, dtype):
    absmax = np.abs(x).max(axis=1).astype(np.float32)
    absmax = np.where(absmax > 0, absmax, np.float32(1.0))
    q = (x * (np.float32(fmax) / absmax)[:, None]).astype(np.float32)
    q = np.clip(q, -fmax, fmax)
    codes = torch.from_numpy(q).to(dtype).view(torch.uint8).numpy()
    return codes, (absmax / np.float32(fmax)).astype(np.float32)


def fp8_gemm_input(M: int, N: int, K: int, seed_stream: int = 0):
    """Returns (Aq uint8[M,K], sa f32[M], Bq uint8[N,K], sb f32[N]), e4m3fn codes."""
    g = rng(4, seed_stream)
    a = g.standard_normal((M, K), dtype=np.float32)
    aq, sa = _quant_rows(a, 448.0, torch.float8_e4m3fn)
    del a
    b = g.standard_normal((N, K), dtype=np.float32)
    bq, sb = _quant_rows(b, 448.0, torch.float8_e4m3fn)
    return aq, sa, bq, sb


# -------------------------------------------------------------- gemv (c=5)
def gemv_input(M: int, N: int = 14336, K: int = 4096, group: int = 128, seed_stream: int = 0):
    """Returns (x bf16 bits uint16[M,K], Wq e5m2 uint8[N,K], s f32[N, K/group])."""
    g = rng(5, seed_stream)
    x = to_bf16_bits(g.standard_normal((M, K), dtype=np.float32))
    w = (g.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    wg = w.reshape(N, K // group, group)
    absmax = np.abs(wg).max(axis=2).astype(np.float32)
    absmax = np.where(absmax > 0, absmax, np.float32(1.0))
    s = (absmax / np.float32(57344.0)).astype(np.float32)
    q = np.clip(wg / s[:, :, None], -57344.0, 57344.0).astype(np.float32).reshape(N, K)
    wq = torch.from_numpy(q).to(torch.float8_e5m2).view(torch.uint8).numpy()
    return x, wq, s


# ----------------------------------------------------------------- MX (c=6)
def quant_mx(x: np.ndarray, fmt: str = "e4m3fn"):
    """MX quantisation of x (rows x K, K a multiple of 32), following the
    reference's _compute_scale_and_quantize (mxfp8_utils.py:17-38): per block
    of 32, descale = absmax / fmax rounded up to a power of two (adding
    0x007FFFFF to the fp32 bits and keeping the exponent field), e8m0 code =
    that exponent field, data = clamp(x / descale, +-fmax) cast to fp8 RNE.
    Returns (codes uint8 rows x K, e8m0 uint8 rows x K/32)."""
    fmax, dt = (448.0, torch.float8_e4m3fn) if fmt == "e4m3fn" else (57344.0, torch.float8_e5m2)
    R, K = x.shape
    xb = x.reshape(R, K // 32, 32).astype(np.float32)
    descale = (np.abs(xb).max(axis=2) / np.float32(fmax)).astype(np.float32)
    e = ((descale.view(np.uint32) + np.uint32(0x007FFFFF)) & np.uint32(0x7F800000))
    rounded = e.view(np.float32)
    quant = np.where(rounded == 0, np.float32(0), np.float32(1) / np.where(rounded == 0, 1, rounded))
    q = np.clip(xb * quant[:, :, None].astype(np.float32), -fmax, fmax).astype(np.float32)
    codes = torch.from_numpy(q.reshape(R, K)).to(dt).view(torch.uint8).numpy()
    return codes, (e >> np.uint32(23)).astype(np.uint8)


E2M1_GRID = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], np.float32)


def quant_mx_fp4(x: np.ndarray):
    """MX fp4 (e2m1) quantisation of x (rows x K, K a multiple of 32) by the
    OCP Microscaling spec v1.0 rule: shared exponent floor(log2(absmax)) - 2
    (e2m1's largest exponent), clamped to the e8m0 range; elements
    x / 2^shared rounded to the nearest e2m1 value (ties to the even code),
    saturating at 6, the sign kept on zeros (as triton's MXFP4Tensor
    rounds).  Returns (packed uint8 rows x K/2, the even K index in the low
    nibble; e8m0 uint8 rows x K/32); all-zero blocks get scale 2^0."""
    R, K = x.shape
    xb = x.reshape(R, K // 32, 32).astype(np.float32)
    amax = np.abs(xb).max(axis=2)
    with np.errstate(divide="ignore"):
        shared = np.where(amax > 0, np.floor(np.log2(np.where(amax > 0, amax, 1))) - 2, 0)
    shared = np.clip(shared, -127, 127).astype(np.int32)
    v = np.abs(xb) * np.exp2(-shared.astype(np.float32))[:, :, None]
    mid = (E2M1_GRID[1:] + E2M1_GRID[:-1]) / 2
    code = np.searchsorted(mid, v, side="left").astype(np.uint8)         # v <= mid[i] -> i
    tie = (code < 7) & (v == mid[np.minimum(code, 6)])
    code = np.where(tie & (code % 2 == 1), code + 1, code).astype(np.uint8)  # ties to even
    code |= np.signbit(xb).astype(np.uint8) << 3                          # -0 kept
    code = code.reshape(R, K)
    packed = (code[:, 0::2] | (code[:, 1::2] << 4)).astype(np.uint8)
    return packed, (shared + 127).astype(np.uint8)


def mx_fp4_gemm_input(M: int, N: int, K: int, seed_stream: int = 0):
    """Returns (Aq packed fp4 uint8[M,K/2], sa e8m0 uint8[M,K/32], Bq uint8[N,K/2], sb)."""
    g = rng(6, seed_stream + 1)
    aq, sa = quant_mx_fp4(g.standard_normal((M, K), dtype=np.float32))
    bq, sb = quant_mx_fp4(g.standard_normal((N, K), dtype=np.float32))
    return aq, sa, bq, sb


def mx_gemm_input(M: int, N: int, K: int, seed_stream: int = 0, fa: str = "e4m3fn",
                  fb: str = "e4m3fn"):
    """Returns (Aq uint8[M,K], sa e8m0 uint8[M,K/32], Bq uint8[N,K], sb e8m0 uint8[N,K/32])."""
    g = rng(6, seed_stream)
    aq, sa = quant_mx(g.standard_normal((M, K), dtype=np.float32), fa)
    bq, sb = quant_mx(g.standard_normal((N, K), dtype=np.float32), fb)
    return aq, sa, bq, sb


# ----------------------------------------------------- grouped (MoE) fp8 GEMM
def moe_group_sizes(total: int, groups: int, seed_stream: int = 0) -> np.ndarray:
    """Rows per expert for `total` routed rows: a multinomial draw with
    expert weights proportional to 1 / (i + 1)^0.8 (a skewed router), so
    groups are uneven and rarely multiples of the 256-row tile."""
    g = rng(7, seed_stream)
    w = 1.0 / np.arange(1, groups + 1) ** 0.8
    return g.multinomial(total, w / w.sum()).astype(np.int64)
