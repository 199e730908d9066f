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
// aligned, C rows of any alignment.
#include "gemm_persist.h"

#define TX_GEMM16_PERSIST(PFX, EL, SFX, OUT)                                                              \
  TX_KERNEL void __launch_bounds__(256) tx_gemm_##PFX##_fast##SFX##_persist(const tx_gemm_args a) {    \
    gemm_persist<GemmCfg<EL, EL, 256, 256, 2, 2, 16>, OUT>(a);                                             \
  }                                                                                                       \
  TX_KERNEL void __launch_bounds__(256) tx_gemm_##PFX##_fast##SFX##_persist_kt(const tx_gemm_args a) { \
    gemm_persist<GemmCfg<EL, EL, 256, 256, 2, 2, 16>, OUT, false, true>(a);                                \
  }

TX_GEMM16_PERSIST(bf16, EL_BF16, , OUT_BF16)
TX_GEMM16_PERSIST(bf16, EL_BF16, _out_f16, OUT_F16)
TX_GEMM16_PERSIST(f16, EL_F16, , OUT_F16)
TX_GEMM16_PERSIST(f16, EL_F16, _out_bf16, OUT_BF16)

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
