// fp8 weight-only dequant GEMV / skinny GEMM on gfx950:
//   y[m,n] = bf16_rne( sum_g s[n,g] * sum_{k in g} x[m,k] * W[n,k] )
// x bf16 (M <= 64 rows), W fp8 N x K row-major, s fp32 N x (K/group).
//
// HBM-bound on W.  A workgroup owns 16 columns (rows of W) and splits K over
// its 4 wavefronts; each lane streams 32 contiguous bytes of one W row per
// 128-element slice with two 128-bit loads, several slices in flight.
//
// Dequantisation is bit placement, not arithmetic: an fp8 code's magnitude
// bits shifted so its mantissa lands at the top of the bf16 mantissa
// ((c & 0x7F) << (7 - m)), with its sign at bit 15, form a bf16 whose value
// is exactly W * 2^-(127 - fp8 bias) for every finite code (normal codes keep
// their exponent field; subnormal codes become bf16 subnormals of the same
// scaled value).  The factor 2^(127 - bias) is applied once per group partial
// sum in fp32, before the group scale, so no per-element multiply is needed.
// Weights are expected finite (saturating quantisation): Inf/NaN codes are
// not propagated as such.  The products run on the bf16 MFMA
// v_mfma_f32_16x16x32_bf16 with fp32 accumulation; each 128-wide (group)
// partial sum is scaled in fp32 before it joins the running sum.
#include "tx_device.h"

namespace {

constexpr int kWaves = 4;
constexpr int kBlock = 64 * kWaves;
constexpr int kCols = 16;       // W rows (output columns) per workgroup
constexpr int kSlice = 128;     // K elements per lane-group load step (2 x 16 B per lane)
constexpr int kUnroll = 4;      // slices in flight per wave

// Four fp8 codes (one 32-bit word) -> four bf16 (two words) holding W*2^-OFF.
template <int FMT>
__device__ __forceinline__ void fp8x4_to_bf16x4_scaled(uint32_t w, uint32_t &lo, uint32_t &hi) {
  // spread bytes: p0 = b0 | b1 << 16, p1 = b2 | b3 << 16
  const uint32_t p0 = __builtin_amdgcn_perm(0u, w, 0x0c010c00u);
  const uint32_t p1 = __builtin_amdgcn_perm(0u, w, 0x0c030c02u);
  constexpr int SH = (FMT == 2) ? 5 : 4;  // mantissa lands in bf16 bits 6..(7-m)
  lo = ((p0 & 0x00800080u) << 8) | ((p0 & 0x007F007Fu) << SH);
  hi = ((p1 & 0x00800080u) << 8) | ((p1 & 0x007F007Fu) << SH);
}

template <int FMT>
__device__ __forceinline__ void gemv_body(const tx_gemv_args &a) {
  // bf16 exponent bias 127 vs the fp8 bias: the bit-placed value is
  // W * 2^-(127 - bias).
  constexpr float kUnfold = (FMT == 2) ? 5.192296858534828e+33f   /* 2^112 */
                                       : 1.329227995784916e+36f;  /* 2^120 */
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = blockIdx.x * kCols;
  const int col = lane & 15, g = lane >> 4;
  const int n = n0 + col;
  const bool n_ok = n < a.N;
  const uint8_t *wrow = a.W + int64_t(n_ok ? n : 0) * a.ldw;
  const int nslices = a.K / kSlice;  // host guarantees K % 128 == 0
  const int per_wave = (nslices + kWaves - 1) / kWaves;
  const int s_begin = wave * per_wave;
  const int s_end = min(nslices, s_begin + per_wave);
  const int mblocks = (a.M + 15) >> 4;
  const int slices_per_group = a.group / kSlice;  // host: group % 128 == 0

  txd::f32x4 acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = txd::f32x4{0.f, 0.f, 0.f, 0.f};
  txd::f32x4 part[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) part[i] = txd::f32x4{0.f, 0.f, 0.f, 0.f};

  for (int s0 = s_begin; s0 < s_end; s0 += kUnroll) {
    txd::u32x4 wv[kUnroll][2];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int s = s0 + u;
      if (s < s_end && n_ok) {
        const txd::u32x4 *p = reinterpret_cast<const txd::u32x4 *>(wrow + s * kSlice + 32 * g);
        wv[u][0] = __builtin_nontemporal_load(p);
        wv[u][1] = __builtin_nontemporal_load(p + 1);
      } else {
        wv[u][0] = txd::u32x4{0u, 0u, 0u, 0u};
        wv[u][1] = txd::u32x4{0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int s = s0 + u;
      if (s >= s_end) break;
      // 32 codes of this lane -> 4 MFMA operands of 8 bf16
      uint32_t wb[16];
      const uint32_t words[8] = {wv[u][0].x, wv[u][0].y, wv[u][0].z, wv[u][0].w,
                                 wv[u][1].x, wv[u][1].y, wv[u][1].z, wv[u][1].w};
#pragma unroll
      for (int q = 0; q < 8; ++q) fp8x4_to_bf16x4_scaled<FMT>(words[q], wb[2 * q], wb[2 * q + 1]);
      const int kbase = s * kSlice + 32 * g;
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        if (mb >= mblocks) break;
        const int m = mb * 16 + col;
        const uint16_t *xrow = a.x + int64_t(m < a.M ? m : 0) * a.ldx + kbase;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          txd::u32x4 xv = {0u, 0u, 0u, 0u};
          if (m < a.M) xv = *reinterpret_cast<const txd::u32x4 *>(xrow + 8 * i);
          const txd::u32x4 wq = {wb[4 * i], wb[4 * i + 1], wb[4 * i + 2], wb[4 * i + 3]};
          part[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(txd::bf16x8, xv), __builtin_bit_cast(txd::bf16x8, wq), part[mb], 0, 0, 0);
        }
      }
      // close the group when its last slice is done
      if ((s + 1) % slices_per_group == 0 || s + 1 == nslices) {
        const int grp = s / slices_per_group;
        const float sc = n_ok ? a.scales[int64_t(n) * a.ld_scales + grp] : 0.0f;
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
          acc[mb] += (part[mb] * kUnfold) * sc;
          part[mb] = txd::f32x4{0.f, 0.f, 0.f, 0.f};
        }
      }
    }
  }
  // A group split across two waves leaves a partial in both; scale it here.
  if (s_end > s_begin && (s_end % slices_per_group) != 0) {
    const int grp = (s_end - 1) / slices_per_group;
    const float sc = n_ok ? a.scales[int64_t(n) * a.ld_scales + grp] : 0.0f;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) acc[mb] += (part[mb] * kUnfold) * sc;
  }

  // Cross-wave reduction in LDS: red[wave][mb][lane] (f32x4).
  __shared__ txd::f32x4 red[kWaves][4][64];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) red[wave][mb][lane] = acc[mb];
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      if (mb >= mblocks) break;
      txd::f32x4 t = red[0][mb][lane];
#pragma unroll
      for (int w = 1; w < kWaves; ++w) t += red[w][mb][lane];
      // MFMA result layout: lane holds D[m = 4*(lane/16) + r][n = lane % 16]
      const float v[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = mb * 16 + 4 * g + r;
        if (m < a.M && n_ok) a.y[int64_t(m) * a.ldy + n] = uint16_t(txd::f32_to_bf16_bits(v[r]));
      }
    }
  }
}

}  // namespace

TX_KERNEL void __launch_bounds__(kBlock) tx_gemv_fp8_e5m2(const tx_gemv_args a) { gemv_body<2>(a); }
TX_KERNEL void __launch_bounds__(kBlock) tx_gemv_fp8_e4m3fn(const tx_gemv_args a) { gemv_body<1>(a); }
