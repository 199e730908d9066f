// tt.dot_scaled with MX block scales on gfx950: fp8 (e4m3fn / e5m2) or
// fp4 (e2m1, two per byte along K) operands, one e8m0 scale per 32 K elements of each row of A and each
// column of B, fp32 accumulation in v_mfma_scale_f32_32x32x64_f8f6f4 (the
// scales enter the MFMA itself), output bf16, fp16 or fp32.  The tile is the
// fast path's LDS-DMA pipeline: 256 x 256 with 4 wavefronts, 256 x 128 with
// 8; see gemm_fast.h.
#include "gemm_common.h"
#include "gemm_fast.h"

using namespace txg;

#define TX_GEMM_MX(FA, FB, ELA, ELB, ON, OUT)                                                      \
  TX_KERNEL void __launch_bounds__(256) tx_gemm_mx_##FA##_##FB##_##ON(const tx_gemm_args a) {      \
    gemm_fast_tile<GemmCfg<ELA, ELB, 256, 256, 2, 2, 16>, 256, 4, true, OUT>(a);                    \
  }                                                                                                \
  TX_KERNEL void __launch_bounds__(512) tx_gemm_mx_##FA##_##FB##_##ON##_n128(const tx_gemm_args a) { \
    gemm_fast_tile<GemmCfg<ELA, ELB, 256, 128, 2, 2, 16>, 128, 8, true, OUT>(a);                    \
  }
#define TX_GEMM_MX_OUTS(FA, FB, ELA, ELB)      \
  TX_GEMM_MX(FA, FB, ELA, ELB, bf16, OUT_BF16) \
  TX_GEMM_MX(FA, FB, ELA, ELB, f16, OUT_F16)   \
  TX_GEMM_MX(FA, FB, ELA, ELB, f32, OUT_F32)

TX_GEMM_MX_OUTS(e4m3fn, e4m3fn, EL_E4M3, EL_E4M3)
TX_GEMM_MX_OUTS(e5m2, e5m2, EL_E5M2, EL_E5M2)
TX_GEMM_MX_OUTS(e4m3fn, e5m2, EL_E4M3, EL_E5M2)
TX_GEMM_MX_OUTS(e5m2, e4m3fn, EL_E5M2, EL_E4M3)
TX_GEMM_MX_OUTS(e2m1, e2m1, EL_E2M1, EL_E2M1)

// Split-K: sums of the K splits' fp32 planes, rounded to the output type.
TX_KERNEL void __launch_bounds__(256) tx_gemm_mx_splitk_reduce_bf16(const tx_gemm_args a) {
  splitk_reduce<false, OUT_BF16>(a);
}
TX_KERNEL void __launch_bounds__(256) tx_gemm_mx_splitk_reduce_f16(const tx_gemm_args a) {
  splitk_reduce<false, OUT_F16>(a);
}
TX_KERNEL void __launch_bounds__(256) tx_gemm_mx_splitk_reduce_f32(const tx_gemm_args a) {
  splitk_reduce<false, OUT_F32>(a);
}

// Operand rows into zero-padded, 16-byte aligned rows (as the fp8 GEMM's).
TX_KERNEL void __launch_bounds__(256) tx_gemm_mx_pad_rows(const tx_pad_args a) { pad_rows<1>(a); }

// fp4 (e2m1) operand rows, two values a byte with the even K index in the
// low nibble, into e4m3fn rows of dst_ld bytes (cols = source bytes, i.e.
// K / 2; dst_cols = the zero-filled destination row length), so that an fp4
// operand can meet an fp8 one in the fp8 x fp8 tile.  Every e2m1 value is
// exact in e4m3fn: magnitude nibble (e, m) = (bits 2:1, bit 0) is 0.5 m for
// e = 0 and 2^(e-1) (1 + m/2) otherwise, i.e. code ((e + 6) << 3) | (m << 2)
// (0x30 for 0.5, 0 for 0), sign to bit 7.  Thread unit: 4 source bytes ->
// 8 destination bytes.
__device__ __forceinline__ uint32_t e2m1x4_to_e4m3(uint32_t nibs16) {  // 4 nibbles in bits 0..15
  uint32_t out = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t n = (nibs16 >> (4 * i)) & 15u, mag = n & 7u, e = mag >> 1, m = mag & 1u;
    const uint32_t code = e ? (((e + 6u) << 3) | (m << 2)) : (m ? 0x30u : 0u);
    out |= (code | ((n & 8u) << 4)) << (8 * i);
  }
  return out;
}

TX_KERNEL void __launch_bounds__(256) tx_gemm_mx_fp4_to_e4m3(const tx_pad_args a) {
  const uint8_t *src = static_cast<const uint8_t *>(a.src);
  uint8_t *dst = static_cast<uint8_t *>(a.dst);
  const int64_t units_row = (int64_t(a.dst_cols) + 7) / 8;  // 8 destination bytes each
  const int64_t total = int64_t(a.rows) * units_row;
  const bool words = (reinterpret_cast<uintptr_t>(src) & 3) == 0 && (a.src_ld & 3) == 0;
  for (int64_t u = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; u < total;
       u += int64_t(gridDim.x) * blockDim.x) {
    const int64_t r = u / units_row;
    const int c = int(u - r * units_row) * 4;  // first source byte
    const uint8_t *row = src + r * a.src_ld;
    uint32_t v = 0;
    if (words && c + 3 < a.cols) {
      v = *reinterpret_cast<const uint32_t *>(row + c);
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (c + k < a.cols) v |= uint32_t(row[c + k]) << (8 * k);
    }
    const txd::u32x2 o = {e2m1x4_to_e4m3(v & 0xFFFFu), e2m1x4_to_e4m3(v >> 16)};
    // dst rows are whole 8-byte units (dst_ld and dst_cols multiples of 8)
    *reinterpret_cast<txd::u32x2 *>(dst + r * a.dst_ld + 2 * c) = o;
  }
}

// Scales of A and B into the step-major layout the tile reads (see
// tx_mx_pack_args), through LDS: workgroup b of an operand transposes rows
// 64 * (b % R) .. +63 (R = rows_pad / 64) for source dword columns
// 32 * (b / R) .. +31 (128 blocks), reading each source row's bytes
// contiguously (dwords when the rows are 4-byte aligned, every load issued
// before the first is used) and writing runs of consecutive rows' dwords.
TX_KERNEL void __launch_bounds__(256) tx_gemm_mx_pack_scales(const tx_mx_pack2_args both) {
  __shared__ uint32_t t[64][33];  // [row][dword of 4 blocks], odd pitch against bank conflicts
  const bool second = int(blockIdx.x) >= both.blocks0;
  const tx_mx_pack_args &a = both.op[second ? 1 : 0];
  const int b = int(blockIdx.x) - (second ? both.blocks0 : 0);
  const int nrb = a.rows_pad / 64;
  const int r0 = (b % nrb) * 64;
  const int d0 = (b / nrb) * 32;  // first dword column (4 blocks each)
  const int c0 = 4 * d0;
  const int tid = threadIdx.x;
  const bool words = (reinterpret_cast<uintptr_t>(a.src) & 3) == 0 && (a.src_ld & 3) == 0;
  uint32_t w[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int i = tid + 256 * j;  // tile dword: row i / 32, blocks 4 (i % 32) .. +3
    const int r = i >> 5, c = c0 + 4 * (i & 31);
    uint32_t v = 0x7F7F7F7Fu;
    if (r0 + r < a.rows) {
      const uint8_t *row = a.src + int64_t(r0 + r) * a.src_ld;
      if (words && c + 3 < a.cols) {
        v = *reinterpret_cast<const uint32_t *>(row + c);
      } else {
        v = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) v |= (c + k < a.cols ? uint32_t(row[c + k]) : 127u) << (8 * k);
      }
    }
    w[j] = v;
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int i = tid + 256 * j;
    t[i >> 5][i & 31] = w[j];
  }
  __syncthreads();
  uint32_t *dst = reinterpret_cast<uint32_t *>(a.dst);
  const int r = tid & 63;
  const int ndw = a.steps * a.sd;  // dword columns in all
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int cl = (tid >> 6) + 4 * j;  // dword column within the tile
    const int d = d0 + cl;
    if (d < ndw) {
      const int s = d / a.sd, q = d % a.sd;
      dst[(int64_t(s) * a.rows_pad + r0 + r) * a.sd + q] = t[r][cl];
    }
  }
}
