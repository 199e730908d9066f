// fp8 weight-only dequant GEMV / skinny GEMM on gfx950:
//   y[m,n] = bf16_rne( sum_g s[n,g] * sum_{k in g} x[m,k] * W[n,k] )
// x bf16 (M <= 64 rows), W fp8 N x K row-major, s fp32 N x (K/group).
//
// HBM-bound on W.  A workgroup owns 32 columns (rows of W) as two 16-row
// blocks and splits K over its 4 wavefronts; each lane streams two 16-byte
// pieces of each of its two W rows per 128-element slice (128-bit loads,
// several slices in flight), and each x fragment feeds both blocks' MFMAs.
//
// Dequantisation is bit placement, not arithmetic: an fp8 code's magnitude
// bits shifted so its mantissa lands at the top of the bf16 mantissa, with
// its sign at bit 15, form a bf16 whose value
// is exactly W * 2^-(127 - fp8 bias) for every finite code (normal codes keep
// their exponent field; subnormal codes become bf16 subnormals of the same
// scaled value).  The factor 2^(127 - bias) is applied once per group partial
// sum in fp32, before the group scale, so no per-element multiply is needed.
// Weights are expected finite (saturating quantisation): Inf/NaN codes are
// not propagated as such.  The products run on the bf16 MFMA
// v_mfma_f32_16x16x32_bf16 with fp32 accumulation; each 128-wide (group)
// partial sum is scaled in fp32 before it joins the running sum.
#include <type_traits>

#include "tx_device.h"

namespace {

constexpr int kNB = 2;                 // 16-row W blocks per wavefront
constexpr int kCols = 16 * kNB;        // W rows (output columns) per workgroup
constexpr int kSlice = 128;     // K elements per lane-group load step (2 x 16 B per lane)

// Four fp8 codes (one 32-bit word) -> four bf16 (two words) holding
// W * 2^-(127 - bias), by bit placement only:
//  1. v_perm puts code b0 in the high byte of the low 16-bit half and b1 in
//     the high byte of the high half (low bytes zero): sign at bit 15,
//     magnitude at bits 14..8;
//  2. a packed 16-bit arithmetic shift right by (8 - e), e = exponent bits,
//     moves the exponent field into the low e bits of bf16's exponent field
//     (bits 6+e .. 7) and the mantissa to the top of bf16's mantissa, and
//     smears the sign over the bits above;
//  3. one AND keeps the sign bit, clears the smeared copies and the low bits.
template <int FMT>
__device__ __forceinline__ void fp8x4_to_bf16x4_scaled(uint32_t w, uint32_t &lo, uint32_t &hi) {
  constexpr int SH = (FMT == 2) ? 3 : 4;                             // 8 - exponent bits
  constexpr uint32_t KEEP = (FMT == 2) ? 0x8FE08FE0u : 0x87F087F0u;  // sign | magnitude
  typedef short s16x2 __attribute__((ext_vector_type(2)));
  const uint32_t p0 = __builtin_amdgcn_perm(0u, w, 0x010c000cu);   // b1<<24 | b0<<8
  const uint32_t p1 = __builtin_amdgcn_perm(0u, w, 0x030c020cu);   // b3<<24 | b2<<8
  const s16x2 sh = {SH, SH};
  const s16x2 q0 = __builtin_bit_cast(s16x2, p0) >> sh;
  const s16x2 q1 = __builtin_bit_cast(s16x2, p1) >> sh;
  lo = __builtin_bit_cast(uint32_t, q0) & KEEP;
  hi = __builtin_bit_cast(uint32_t, q1) & KEEP;
}

template <int FMT, int kWaves, int kUnroll, int MB>
__device__ __forceinline__ void gemv_body(const tx_gemv_args &a) {
  // The bit-placed weights are W * 2^-(127 - bias); the factor is split in
  // two halves: one folded into every group scale (safe for any scale below
  // 2^64), the other applied once to the final sum.
  constexpr float kHalf = (FMT == 2) ? 7.205759403792794e+16f   /* 2^56 */
                                     : 1.152921504606847e+18f;  /* 2^60 */
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = blockIdx.x * kCols;
  const int col = lane & 15, g = lane >> 4;
  const int nslices = a.K / kSlice;  // host guarantees K % 128 == 0
  const int per_wave = (nslices + kWaves - 1) / kWaves;
  const int s_begin = min(nslices, wave * per_wave);
  const int s_end = min(nslices, s_begin + per_wave);
  const int slices_per_group = a.group / kSlice;  // host: group % 128 == 0

  // The wave's NB blocks of 16 W rows (output columns).  Rows past N read
  // row N-1 (always valid) and are never stored: no branch.
  const uint8_t *wrow[kNB];
  const float *srow[kNB];
#pragma unroll
  for (int b = 0; b < kNB; ++b) {
    const int n = n0 + 16 * b + col;
    const int nn = n < a.N ? n : a.N - 1;
    wrow[b] = a.W + int64_t(nn) * a.ldw + 16 * g;
    srow[b] = a.scales + int64_t(nn) * a.ld_scales;
  }
  // Group scales of this wave's slices, loaded once (up to 8 groups; longer
  // ranges fall back to a load per group).
  const int g_first = s_begin / slices_per_group;
  float scl[kNB][8];
#pragma unroll
  for (int b = 0; b < kNB; ++b)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int gi = g_first + j;
      scl[b][j] = (gi * slices_per_group < nslices) ? srow[b][gi] : 0.0f;
    }
  auto scale_of = [&](int b, int grp) -> float {
    const int j = grp - g_first;
    float v = (j >= 0 && j < 8) ? scl[b][0] : srow[b][grp];
#pragma unroll
    for (int t = 1; t < 8; ++t) v = (j == t) ? scl[b][t] : v;
    return v;
  };

  // x rows past M read row M-1: MFMA output rows are independent and rows
  // past M are never stored, so no masking is needed.
  const uint16_t *xrow[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int m = mb * 16 + col;
    xrow[mb] = a.x + int64_t(m < a.M ? m : a.M - 1) * a.ldx + 16 * g;
  }

  txd::f32x4 acc[kNB][MB], part[kNB][MB];
#pragma unroll
  for (int b = 0; b < kNB; ++b)
#pragma unroll
    for (int i = 0; i < MB; ++i) acc[b][i] = part[b][i] = txd::f32x4{0.f, 0.f, 0.f, 0.f};
  bool fresh = true;  // the next MFMA chain starts from zero

  // Lane group g holds bytes [16g, 16g+16) and [64+16g, 64+16g+16) of each
  // 128-byte slice, so a load instruction covers contiguous 64-byte halves of
  // the 16 rows' lines; MFMA i of a slice takes k = 64 (i/2) + 16g + 8 (i%2) + 0..7
  // for both x and W.  Each x fragment feeds the MFMAs of all kNB W blocks.
  auto slice = [&](int s, const txd::u32x4 (&w)[kNB][2]) {
    uint32_t wb[kNB][16];
#pragma unroll
    for (int b = 0; b < kNB; ++b) {
      const uint32_t words[8] = {w[b][0].x, w[b][0].y, w[b][0].z, w[b][0].w,
                                 w[b][1].x, w[b][1].y, w[b][1].z, w[b][1].w};
#pragma unroll
      for (int q = 0; q < 8; ++q) fp8x4_to_bf16x4_scaled<FMT>(words[q], wb[b][2 * q], wb[b][2 * q + 1]);
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const uint16_t *xp = xrow[mb] + s * kSlice;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const txd::u32x4 xv = *reinterpret_cast<const txd::u32x4 *>(xp + (i >> 1) * 64 + (i & 1) * 8);
#pragma unroll
        for (int b = 0; b < kNB; ++b) {
          const txd::u32x4 wq = {wb[b][4 * i], wb[b][4 * i + 1], wb[b][4 * i + 2], wb[b][4 * i + 3]};
          const txd::f32x4 c = (i == 0 && fresh) ? txd::f32x4{0.f, 0.f, 0.f, 0.f} : part[b][mb];
          part[b][mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(txd::bf16x8, xv), __builtin_bit_cast(txd::bf16x8, wq), c, 0, 0, 0);
        }
      }
    }
    fresh = false;
    // close the group when its last slice is done (uniform)
    if ((s + 1) % slices_per_group == 0 || s + 1 == nslices) {
      const int grp = s / slices_per_group;
#pragma unroll
      for (int b = 0; b < kNB; ++b) {
        const float sc = scale_of(b, grp) * kHalf;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[b][mb] += part[b][mb] * sc;
      }
      fresh = true;
    }
  };

  int s0 = s_begin;
  for (; s0 + kUnroll <= s_end; s0 += kUnroll) {
    txd::u32x4 wv[kUnroll][kNB][2];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
#pragma unroll
      for (int b = 0; b < kNB; ++b) {
        const txd::u32x4 *p = reinterpret_cast<const txd::u32x4 *>(wrow[b] + (s0 + u) * kSlice);
        wv[u][b][0] = __builtin_nontemporal_load(p);
        wv[u][b][1] = __builtin_nontemporal_load(p + 4);
      }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) slice(s0 + u, wv[u]);
  }
  for (; s0 < s_end; ++s0) {
    txd::u32x4 wv[kNB][2];
#pragma unroll
    for (int b = 0; b < kNB; ++b) {
      const txd::u32x4 *p = reinterpret_cast<const txd::u32x4 *>(wrow[b] + s0 * kSlice);
      wv[b][0] = __builtin_nontemporal_load(p);
      wv[b][1] = __builtin_nontemporal_load(p + 4);
    }
    slice(s0, wv);
  }
  // A group split across two waves leaves a partial in both; scale it here.
  if (!fresh) {
    const int grp = (s_end - 1) / slices_per_group;
#pragma unroll
    for (int b = 0; b < kNB; ++b) {
      const float sc = scale_of(b, grp) * kHalf;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) acc[b][mb] += part[b][mb] * sc;
    }
  }

  // Cross-wave reduction in LDS, one (W block, 16-row block of M) at a time.
  __shared__ txd::f32x4 red[kWaves][64];
#pragma unroll
  for (int b = 0; b < kNB; ++b)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      red[wave][lane] = acc[b][mb];
      __syncthreads();
      if (wave == 0) {
        txd::f32x4 t = red[0][lane];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) t += red[w][lane];
        t *= kHalf;
        // MFMA result layout: lane holds D[m = 4*(lane/16) + r][n = lane % 16]
        const int n = n0 + 16 * b + col;
        const float v[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = mb * 16 + 4 * g + r;
          if (m < a.M && n < a.N) a.y[int64_t(m) * a.ldy + n] = uint16_t(txd::f32_to_bf16_bits(v[r]));
        }
      }
      __syncthreads();
    }
}

}  // namespace

// Kernel names: tx_gemv_fp8_<w format>_w<waves>_m<16-row blocks of M>.
#define TX_GEMV(NAME, FMT, W, U, MB)                                                      \
  TX_KERNEL void __launch_bounds__(64 * W) tx_gemv_fp8_##NAME##_w##W##_m##MB(const tx_gemv_args a) { \
    gemv_body<FMT, W, U, MB>(a);                                                          \
  }
#define TX_GEMV_MB(NAME, FMT, W, U) \
  TX_GEMV(NAME, FMT, W, U, 1) TX_GEMV(NAME, FMT, W, U, 2) TX_GEMV(NAME, FMT, W, U, 4)
TX_GEMV_MB(e5m2, 2, 4, 4)
TX_GEMV_MB(e4m3fn, 1, 4, 4)
