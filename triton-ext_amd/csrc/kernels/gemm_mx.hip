// tt.dot_scaled with MX block scales on gfx950: fp8 (e4m3fn / e5m2)
// operands, one e8m0 scale per 32 K elements of each row of A and each
// column of B, fp32 accumulation in v_mfma_scale_f32_32x32x64_f8f6f4 (the
// scales enter the MFMA itself), output bf16, fp16 or fp32.  The tile is the
// fast path's 256 x 256 (or 256 x 128) LDS-DMA pipeline with 4 wavefronts;
// see gemm_fast.h.
#include "gemm_common.h"
#include "gemm_fast.h"

using namespace txg;

#define TX_GEMM_MX(FA, FB, ELA, ELB, ON, OUT)                                                      \
  TX_KERNEL void __launch_bounds__(256) tx_gemm_mx_##FA##_##FB##_##ON(const tx_gemm_args a) {      \
    gemm_fast_tile<GemmCfg<ELA, ELB, 256, 256, 2, 2, 16>, 256, 4, true, OUT>(a);                    \
  }                                                                                                \
  TX_KERNEL void __launch_bounds__(256) tx_gemm_mx_##FA##_##FB##_##ON##_n128(const tx_gemm_args a) { \
    gemm_fast_tile<GemmCfg<ELA, ELB, 256, 128, 2, 2, 16>, 128, 4, true, OUT>(a);                    \
  }
#define TX_GEMM_MX_OUTS(FA, FB, ELA, ELB)      \
  TX_GEMM_MX(FA, FB, ELA, ELB, bf16, OUT_BF16) \
  TX_GEMM_MX(FA, FB, ELA, ELB, f16, OUT_F16)   \
  TX_GEMM_MX(FA, FB, ELA, ELB, f32, OUT_F32)

TX_GEMM_MX_OUTS(e4m3fn, e4m3fn, EL_E4M3, EL_E4M3)
TX_GEMM_MX_OUTS(e5m2, e5m2, EL_E5M2, EL_E5M2)
TX_GEMM_MX_OUTS(e4m3fn, e5m2, EL_E4M3, EL_E5M2)
TX_GEMM_MX_OUTS(e5m2, e4m3fn, EL_E5M2, EL_E4M3)

// Operand rows into zero-padded, 16-byte aligned rows (as the fp8 GEMM's).
TX_KERNEL void __launch_bounds__(256) tx_gemm_mx_pad_rows(const tx_pad_args a) { pad_rows<1>(a); }

// Scales into the step-major layout the tile reads (see tx_mx_pack_args):
// one thread per output dword, consecutive threads on consecutive rows.
TX_KERNEL void __launch_bounds__(256) tx_gemm_mx_pack_scales(const tx_mx_pack_args a) {
  const int64_t total = int64_t(a.steps) * a.rows_pad;
  uint32_t *dst = reinterpret_cast<uint32_t *>(a.dst);
  for (int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
       t += int64_t(gridDim.x) * blockDim.x) {
    const int s = int(t / a.rows_pad);
    const int r = int(t % a.rows_pad);
    uint32_t w = 0x7F7F7F7Fu;
    if (r < a.rows) {
      const uint8_t *src = a.src + int64_t(r) * a.src_ld;
      w = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int c = 4 * s + i;
        const uint32_t b = c < a.cols ? uint32_t(src[c]) : 127u;
        w |= b << (8 * i);
      }
    }
    dst[t] = w;
  }
}
