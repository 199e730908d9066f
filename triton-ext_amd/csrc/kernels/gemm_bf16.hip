// tt.dot, bf16 operands, fp32 accumulation, bf16 output, on gfx950.
// Kernel variants: tile 256x256 (4 wavefronts of 128x128) for large shapes
// and 128x128 (4 wavefronts of 64x64) for shapes with few tiles, each with
// a global load width of 16, 8 or 2 bytes chosen by the host from the
// operand alignment (see gemm_common.h for the layout contract).
#include "gemm_tile.h"

using namespace txg;

#define TX_GEMM_BF16(NAME, BM, BN, WM, WN, VEC)                                         \
  TX_KERNEL void __launch_bounds__(64 * WM * WN) tx_gemm_bf16_##NAME##_v##VEC(        \
      const tx_gemm_args a) {                                                         \
    gemm_tile<GemmCfg<EL_BF16, EL_BF16, BM, BN, WM, WN, VEC>>(a);                     \
  }

TX_GEMM_BF16(256x256, 256, 256, 2, 2, 16)
TX_GEMM_BF16(256x256, 256, 256, 2, 2, 8)
TX_GEMM_BF16(256x256, 256, 256, 2, 2, 2)
TX_GEMM_BF16(128x128, 128, 128, 2, 2, 16)
TX_GEMM_BF16(128x128, 128, 128, 2, 2, 8)
TX_GEMM_BF16(128x128, 128, 128, 2, 2, 2)

#include "gemm_fast.h"

TX_KERNEL void __launch_bounds__(512) tx_gemm_bf16_fast(const tx_gemm_args a) {
  gemm_fast_tile<GemmCfg<EL_BF16, EL_BF16, 256, 256, 2, 2, 16>, 256>(a);
}
TX_KERNEL void __launch_bounds__(512) tx_gemm_bf16_fast_n128(const tx_gemm_args a) {
  gemm_fast_tile<GemmCfg<EL_BF16, EL_BF16, 256, 128, 2, 2, 16>, 128>(a);
}
TX_KERNEL void __launch_bounds__(256) tx_gemm_bf16_splitk_reduce(const tx_gemm_args a) {
  splitk_reduce<false>(a);
}

TX_KERNEL void __launch_bounds__(256) tx_gemm_bf16_pad_rows(const tx_pad_args a) { pad_rows<2>(a); }
