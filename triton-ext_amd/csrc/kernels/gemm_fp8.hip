// tt.dot on fp8 operands with the per-row / per-column fp32 scale epilogue,
// bf16 output, on gfx950 (v_mfma_f32_16x16x128_f8f6f4).  Variants: tile
// 256x256 and 128x128, operand formats e4m3fn/e5m2 for A and B, global load
// width 16, 4 or 1 bytes (1-byte loads only with the 128x128 tile, where
// their extra registers fit; see gemm_common.h for the layout contract).
#include "gemm_tile.h"

using namespace txg;

#define TX_GEMM_FP8(FA, FB, ELA, ELB, NAME, BM, BN, WM, WN, VEC)                         \
  TX_KERNEL void __launch_bounds__(64 * WM * WN) tx_gemm_fp8_##FA##_##FB##_##NAME##_v##VEC( \
      const tx_gemm_args a) {                                                           \
    gemm_tile<GemmCfg<ELA, ELB, BM, BN, WM, WN, VEC>>(a);                               \
  }

#define TX_GEMM_FP8_FORMATS(NAME, BM, BN, WM, WN, VEC)                             \
  TX_GEMM_FP8(e4m3fn, e4m3fn, EL_E4M3, EL_E4M3, NAME, BM, BN, WM, WN, VEC)         \
  TX_GEMM_FP8(e5m2, e5m2, EL_E5M2, EL_E5M2, NAME, BM, BN, WM, WN, VEC)             \
  TX_GEMM_FP8(e4m3fn, e5m2, EL_E4M3, EL_E5M2, NAME, BM, BN, WM, WN, VEC)           \
  TX_GEMM_FP8(e5m2, e4m3fn, EL_E5M2, EL_E4M3, NAME, BM, BN, WM, WN, VEC)

TX_GEMM_FP8_FORMATS(256x256, 256, 256, 2, 2, 16)
TX_GEMM_FP8_FORMATS(256x256, 256, 256, 2, 2, 4)
TX_GEMM_FP8_FORMATS(128x128, 128, 128, 2, 2, 16)
TX_GEMM_FP8_FORMATS(128x128, 128, 128, 2, 2, 4)
TX_GEMM_FP8_FORMATS(128x128, 128, 128, 2, 2, 1)

#include "gemm_fast.h"

#define TX_GEMM_FP8_FAST(FA, FB, ELA, ELB)                                                      \
  TX_KERNEL void __launch_bounds__(512) tx_gemm_fp8_##FA##_##FB##_fast(const tx_gemm_args a) {      \
    gemm_fast_tile<GemmCfg<ELA, ELB, 256, 256, 2, 2, 16>, 256>(a);                                  \
  }                                                                                                 \
  TX_KERNEL void __launch_bounds__(512) tx_gemm_fp8_##FA##_##FB##_fast_n128(const tx_gemm_args a) { \
    gemm_fast_tile<GemmCfg<ELA, ELB, 256, 128, 2, 2, 16>, 128>(a);                                  \
  }

TX_KERNEL void __launch_bounds__(256) tx_gemm_fp8_splitk_reduce(const tx_gemm_args a) {
  splitk_reduce<true>(a);
}

TX_GEMM_FP8_FAST(e4m3fn, e4m3fn, EL_E4M3, EL_E4M3)
TX_GEMM_FP8_FAST(e5m2, e5m2, EL_E5M2, EL_E5M2)
TX_GEMM_FP8_FAST(e4m3fn, e5m2, EL_E4M3, EL_E5M2)
TX_GEMM_FP8_FAST(e5m2, e4m3fn, EL_E5M2, EL_E4M3)

// The same tiles with the fused epilogue (bias, activation, output type).
#define TX_GEMM_FP8_FAST_EPI(FA, FB, ELA, ELB)                                                        \
  TX_KERNEL void __launch_bounds__(512) tx_gemm_fp8_##FA##_##FB##_fast_epi(const tx_gemm_args a) {      \
    gemm_fast_tile<GemmCfg<ELA, ELB, 256, 256, 2, 2, 16>, 256, fast::kWaves, false, OUT_BF16, true>(a);  \
  }                                                                                                     \
  TX_KERNEL void __launch_bounds__(512) tx_gemm_fp8_##FA##_##FB##_fast_epi_n128(const tx_gemm_args a) { \
    gemm_fast_tile<GemmCfg<ELA, ELB, 256, 128, 2, 2, 16>, 128, fast::kWaves, false, OUT_BF16, true>(a);  \
  }

TX_GEMM_FP8_FAST_EPI(e4m3fn, e4m3fn, EL_E4M3, EL_E4M3)
TX_GEMM_FP8_FAST_EPI(e5m2, e5m2, EL_E5M2, EL_E5M2)
TX_GEMM_FP8_FAST_EPI(e4m3fn, e5m2, EL_E4M3, EL_E5M2)
TX_GEMM_FP8_FAST_EPI(e5m2, e4m3fn, EL_E5M2, EL_E4M3)

#include "gemm_skinny.h"

// Kernel names: tx_gemm_fp8_<a>_<b>_skinny_w<waves>_m<16-row blocks of M>
// (the small-grid variant with 4 blocks of M has 8 wavefronts: 16 would not
// fit its registers in 128 VGPRs).
#define TX_GEMM_FP8_SKINNY(FA, FB, ELA, ELB, W, MB)                                       \
  TX_KERNEL void __launch_bounds__(64 * W) tx_gemm_fp8_##FA##_##FB##_skinny_w##W##_m##MB( \
      const tx_gemm_args a) {                                                            \
    skinny_fp8_tile<ELA, ELB, W, MB>(a);                                                 \
  }
#define TX_GEMM_FP8_SKINNY_ALL(FA, FB, ELA, ELB)                                               \
  TX_GEMM_FP8_SKINNY(FA, FB, ELA, ELB, 4, 1) TX_GEMM_FP8_SKINNY(FA, FB, ELA, ELB, 4, 2)       \
  TX_GEMM_FP8_SKINNY(FA, FB, ELA, ELB, 4, 4) TX_GEMM_FP8_SKINNY(FA, FB, ELA, ELB, 16, 1)      \
  TX_GEMM_FP8_SKINNY(FA, FB, ELA, ELB, 16, 2) TX_GEMM_FP8_SKINNY(FA, FB, ELA, ELB, 8, 4)

TX_GEMM_FP8_SKINNY_ALL(e4m3fn, e4m3fn, EL_E4M3, EL_E4M3)
TX_GEMM_FP8_SKINNY_ALL(e5m2, e5m2, EL_E5M2, EL_E5M2)
TX_GEMM_FP8_SKINNY_ALL(e4m3fn, e5m2, EL_E4M3, EL_E5M2)
TX_GEMM_FP8_SKINNY_ALL(e5m2, e4m3fn, EL_E5M2, EL_E4M3)

TX_KERNEL void __launch_bounds__(256) tx_gemm_fp8_pad_rows(const tx_pad_args a) { pad_rows<1>(a); }

// Epilogue pass of the skinny and generic kernels: their scaled fp32 sums
// (a.part, M x N) through bias, activation and the output conversion into C.
TX_KERNEL void __launch_bounds__(256) tx_gemm_fp8_epilogue(const tx_gemm_args a) {
  const int64_t total = int64_t(a.M) * a.N;
  for (int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
       t += int64_t(gridDim.x) * blockDim.x) {
    const int64_t m = t / a.N;
    const int n = int(t % a.N);
    epi_store1(a, m, n, epi_value(a, a.part[t], n));
  }
}
