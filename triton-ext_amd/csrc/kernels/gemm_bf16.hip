// tt.dot, 16-bit operands (bf16 or fp16), fp32 accumulation, bf16 or fp16
// output (round to nearest even), on gfx950.
// Kernel names: tx_gemm_<operands>_<tile>[_out_<output>], the output suffix
// present when the output type differs from the operands'.
// Generic variants: tile 256x256 (4 wavefronts of 128x128) for large shapes
// and 128x128 (4 wavefronts of 64x64) for shapes with few tiles, each with
// a global load width of 16, 8 or 2 bytes chosen by the host from the
// operand alignment (see gemm_common.h for the layout contract).
#include "gemm_tile.h"

using namespace txg;

#define TX_GEMM16(PFX, EL, SFX, OUT, NAME, BM, BN, WM, WN, VEC)                               \
  TX_KERNEL void __launch_bounds__(64 * WM * WN) tx_gemm_##PFX##_##NAME##_v##VEC##SFX(        \
      const tx_gemm_args a) {                                                                 \
    gemm_tile<GemmCfg<EL, EL, BM, BN, WM, WN, VEC>, OUT>(a);                                  \
  }

#define TX_GEMM16_GENERIC(PFX, EL, SFX, OUT)                          \
  TX_GEMM16(PFX, EL, SFX, OUT, 256x256, 256, 256, 2, 2, 16)           \
  TX_GEMM16(PFX, EL, SFX, OUT, 256x256, 256, 256, 2, 2, 8)            \
  TX_GEMM16(PFX, EL, SFX, OUT, 256x256, 256, 256, 2, 2, 2)            \
  TX_GEMM16(PFX, EL, SFX, OUT, 128x128, 128, 128, 2, 2, 16)           \
  TX_GEMM16(PFX, EL, SFX, OUT, 128x128, 128, 128, 2, 2, 8)            \
  TX_GEMM16(PFX, EL, SFX, OUT, 128x128, 128, 128, 2, 2, 2)

// fp32 and int8 tt.dot (tx_dot_acc): tx_gemm_{f32,i8}_128x128_v<load width>
// (the 256 x 256 tile's accumulators and 32-bit fragments spill)
#define TX_GEMM32_GENERIC(PFX, EL, OUT, V0, V1, V2)            \
  TX_GEMM16(PFX, EL, , OUT, 128x128, 128, 128, 2, 2, V0)      \
  TX_GEMM16(PFX, EL, , OUT, 128x128, 128, 128, 2, 2, V1)      \
  TX_GEMM16(PFX, EL, , OUT, 128x128, 128, 128, 2, 2, V2)
TX_GEMM32_GENERIC(f32, EL_F32, OUT_F32, 16, 8, 4)
TX_GEMM32_GENERIC(i8, EL_I8, OUT_I32, 16, 4, 1)

TX_GEMM16_GENERIC(bf16, EL_BF16, , OUT_BF16)
TX_GEMM16_GENERIC(bf16, EL_BF16, _out_f16, OUT_F16)
TX_GEMM16_GENERIC(f16, EL_F16, , OUT_F16)
TX_GEMM16_GENERIC(f16, EL_F16, _out_bf16, OUT_BF16)

#include "gemm_fast.h"

#define TX_GEMM16_FAST(PFX, EL, SFX, OUT)                                                    \
  TX_KERNEL void __launch_bounds__(512) tx_gemm_##PFX##_fast##SFX(const tx_gemm_args a) {     \
    gemm_fast_tile<GemmCfg<EL, EL, 256, 256, 2, 2, 16>, 256, fast::kWaves, false, OUT>(a);    \
  }                                                                                          \
  TX_KERNEL void __launch_bounds__(512) tx_gemm_##PFX##_fast##SFX##_n128(const tx_gemm_args a) { \
    gemm_fast_tile<GemmCfg<EL, EL, 256, 128, 2, 2, 16>, 128, fast::kWaves, false, OUT>(a);    \
  }

TX_GEMM16_FAST(bf16, EL_BF16, , OUT_BF16)
TX_GEMM16_FAST(bf16, EL_BF16, _out_f16, OUT_F16)
TX_GEMM16_FAST(f16, EL_F16, , OUT_F16)
TX_GEMM16_FAST(f16, EL_F16, _out_bf16, OUT_BF16)

// The persistent 4-wavefront tile (one workgroup per CU; see gemm_persist.h)
// for products of at least one 256 x 256 tile per CU whose K is a whole
// number (>= 2) of 64-element steps, N a multiple of 8 and C 16-byte aligned;
// _persist_kt: any K of at least 128 elements, rows of A and B 4-byte
// aligned, C rows of any alignment; _persist_kn: B row-major K x N (ldb
// elements per K row), K a whole number of 64-element steps, B and its rows
// 16-byte aligned; _persist128[_kn] / _persist64[_kn]: the same on 128 x 128
// / 64 x 64 tiles, for products with fewer 256 x 256 / 128 x 128 tiles than
// CUs.
#include "gemm_persist.h"

#define TX_GEMM16_PERSIST(PFX, EL, SFX, OUT)                                                              \
  TX_KERNEL void __launch_bounds__(256) tx_gemm_##PFX##_fast##SFX##_persist(const tx_gemm_args a) {    \
    gemm_persist<GemmCfg<EL, EL, 256, 256, 2, 2, 16>, OUT>(a);                                             \
  }                                                                                                       \
  TX_KERNEL void __launch_bounds__(256) tx_gemm_##PFX##_fast##SFX##_persist_kt(const tx_gemm_args a) { \
    gemm_persist<GemmCfg<EL, EL, 256, 256, 2, 2, 16>, OUT, false, true>(a);                                \
  }                                                                                                       \
  TX_KERNEL void __launch_bounds__(256) tx_gemm_##PFX##_fast##SFX##_persist_kn(const tx_gemm_args a) { \
    gemm_persist<GemmCfg<EL, EL, 256, 256, 2, 2, 16>, OUT, false, false, true>(a);                         \
  }                                                                                                       \
  TX_KERNEL void __launch_bounds__(256) tx_gemm_##PFX##_fast##SFX##_persist128(const tx_gemm_args a) { \
    gemm_persist<GemmCfg<EL, EL, 256, 256, 2, 2, 16>, OUT, false, false, false, 128>(a);                   \
  }                                                                                                       \
  TX_KERNEL void __launch_bounds__(256) tx_gemm_##PFX##_fast##SFX##_persist128_kn(const tx_gemm_args a) { \
    gemm_persist<GemmCfg<EL, EL, 256, 256, 2, 2, 16>, OUT, false, false, true, 128>(a);                    \
  }                                                                                                       \
  TX_KERNEL void __launch_bounds__(256) tx_gemm_##PFX##_fast##SFX##_persist64(const tx_gemm_args a) {  \
    gemm_persist<GemmCfg<EL, EL, 256, 256, 2, 2, 16>, OUT, false, false, false, 64>(a);                    \
  }                                                                                                       \
  TX_KERNEL void __launch_bounds__(256) tx_gemm_##PFX##_fast##SFX##_persist64_kn(const tx_gemm_args a) { \
    gemm_persist<GemmCfg<EL, EL, 256, 256, 2, 2, 16>, OUT, false, false, true, 64>(a);                     \
  }

TX_GEMM16_PERSIST(bf16, EL_BF16, , OUT_BF16)
TX_GEMM16_PERSIST(bf16, EL_BF16, _out_f16, OUT_F16)
TX_GEMM16_PERSIST(f16, EL_F16, , OUT_F16)
TX_GEMM16_PERSIST(f16, EL_F16, _out_bf16, OUT_BF16)

// Column strip of a 16-bit product: C[:, 0 .. N) with N <= W (1, 2, 4 or
// 8), the few columns past the last 256-column block of a larger product
// (whose 256-row tiles would spend a whole tile of MFMAs on each).  VALU dot
// products: a wavefront per row, lane l the 16-byte chunks l, l + 64, .. of
// K, kStripUnroll of them loaded before any is used, read through buffer
// resources (rows 4-byte aligned); the ragged end of K (K mod 8 elements,
// K >= 8) as the row's last 16 bytes with the elements before it skipped;
// fp32 sums reduced across the wave and rounded to nearest even.
constexpr int kStripWaves = 4, kStripUnroll = 4;

template <int EL>
__device__ __forceinline__ void widen8(const txd::u32x4 &w, float (&x)[8]) {
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    if constexpr (EL == EL_BF16) {
      x[2 * d] = __uint_as_float(w[d] << 16);
      x[2 * d + 1] = __uint_as_float(w[d] & 0xFFFF0000u);
    } else {
      x[2 * d] = float(__builtin_bit_cast(_Float16, uint16_t(w[d] & 0xFFFFu)));
      x[2 * d + 1] = float(__builtin_bit_cast(_Float16, uint16_t(w[d] >> 16)));
    }
  }
}

template <int EL, int OUT, int W>
__device__ __forceinline__ void gemm16_strip(const tx_gemm_args &a) {
  constexpr int U = kStripUnroll;
  const int lane = threadIdx.x & 63;
  const int row = int(blockIdx.x) * kStripWaves + int(threadIdx.x >> 6);
  if (row >= a.M) return;
  const uint32_t lda_b = uint32_t(a.lda) * 2u, ldb_b = uint32_t(a.ldb) * 2u, kb = uint32_t(a.K) * 2u;
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(a.A, uint32_t(a.M - 1) * lda_b + kb);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(a.B, uint32_t(a.N - 1) * ldb_b + kb);
  const uint32_t arow = uint32_t(row) * lda_b;
  uint32_t bcol[W];
#pragma unroll
  for (int j = 0; j < W; ++j) bcol[j] = uint32_t(min(j, a.N - 1)) * ldb_b;  // columns past N: discarded
  float acc[W];
#pragma unroll
  for (int j = 0; j < W; ++j) acc[j] = 0.0f;
  auto fma8 = [&](const txd::u32x4 &av, const txd::u32x4 (&bv)[W], int first) {
    float x[8];
    widen8<EL>(av, x);
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (e < first) x[e] = 0.0f;
#pragma unroll
    for (int j = 0; j < W; ++j) {
      float b[8];
      widen8<EL>(bv[j], b);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[j] = fmaf(x[e], b[e], acc[j]);
    }
  };
  auto ld = [&](__amdgpu_buffer_rsrc_t r, uint32_t o) {
    return __builtin_bit_cast(txd::u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, o, 0, 0));
  };
  const int whole = a.K / 8, rest = a.K % 8;
  for (int c0 = lane; c0 < whole; c0 += 64 * U) {
    txd::u32x4 av[U], bv[U][W];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + 64 * u;
      // chunks past the row end read out of the buffers' range (zeros) and are not used
      const uint32_t ko = c < whole ? uint32_t(c) * 16u : 0x80000000u;
      av[u] = ld(ra, arow + ko);
#pragma unroll
      for (int j = 0; j < W; ++j) bv[u][j] = ld(rb, bcol[j] + ko);
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (c0 + 64 * u < whole) fma8(av[u], bv[u], 0);
  }
  if (rest && lane == (whole & 63)) {
    txd::u32x4 bv[W];
#pragma unroll
    for (int j = 0; j < W; ++j) bv[j] = ld(rb, bcol[j] + kb - 16u);
    fma8(ld(ra, arow + kb - 16u), bv, 8 - rest);
  }
  // wave sums; lane j then stores column j
  float out = 0.0f;
#pragma unroll
  for (int j = 0; j < W; ++j) {
    float v = acc[j];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    if (lane == j) out = v;
  }
  if (lane < W && lane < a.N) {
    const uint32_t bits = OUT == OUT_F16 ? txd::pack_f16x2(out, 0.0f) & 0xFFFFu : txd::f32_to_bf16_bits(out);
    static_cast<uint16_t *>(a.C)[int64_t(row) * a.ldc + lane] = uint16_t(bits);
  }
}

#define TX_GEMM16_STRIP_W(PFX, EL, SFX, OUT, W)                                                                  \
  TX_KERNEL void __launch_bounds__(64 * kStripWaves) tx_gemm_##PFX##_strip##W##SFX(const tx_gemm_args a) { \
    gemm16_strip<EL, OUT, W>(a);                                                                             \
  }
#define TX_GEMM16_STRIP(PFX, EL, SFX, OUT)   \
  TX_GEMM16_STRIP_W(PFX, EL, SFX, OUT, 1)    \
  TX_GEMM16_STRIP_W(PFX, EL, SFX, OUT, 2)    \
  TX_GEMM16_STRIP_W(PFX, EL, SFX, OUT, 4)    \
  TX_GEMM16_STRIP_W(PFX, EL, SFX, OUT, 8)

TX_GEMM16_STRIP(bf16, EL_BF16, , OUT_BF16)
TX_GEMM16_STRIP(bf16, EL_BF16, _out_f16, OUT_F16)
TX_GEMM16_STRIP(f16, EL_F16, , OUT_F16)
TX_GEMM16_STRIP(f16, EL_F16, _out_bf16, OUT_BF16)

// Split-K reductions, by output type.
TX_KERNEL void __launch_bounds__(256) tx_gemm_bf16_splitk_reduce(const tx_gemm_args a) {
  splitk_reduce<false>(a);
}
TX_KERNEL void __launch_bounds__(256) tx_gemm_f16_splitk_reduce(const tx_gemm_args a) {
  splitk_reduce<false, OUT_F16>(a);
}

// Zero-padded copies of rows of 16-bit elements (either type).
TX_KERNEL void __launch_bounds__(256) tx_gemm_bf16_pad_rows(const tx_pad_args a) { pad_rows<2>(a); }

// Row-major K x N operands of 16-bit elements (either type) -> N rows of K.
TX_KERNEL void __launch_bounds__(256) tx_gemm_16_transpose_kn_v16(const tx_pad_args a) {
  transpose_kn<true>(a);
}
TX_KERNEL void __launch_bounds__(256) tx_gemm_16_transpose_kn_v2(const tx_pad_args a) {
  transpose_kn<false>(a);
}
