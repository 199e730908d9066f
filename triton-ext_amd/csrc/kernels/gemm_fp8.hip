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

// The persistent 4-wavefront tile (one workgroup per CU; see gemm_persist.h)
// for products of at least one 256 x 256 tile per CU whose K is a whole
// number (>= 2) of 128-byte steps, N a multiple of 8 and C 16-byte aligned.
#include "gemm_persist.h"

#define TX_GEMM_FP8_PERSIST(FA, FB, ELA, ELB)                                                               \
  TX_KERNEL void __launch_bounds__(256) tx_gemm_fp8_##FA##_##FB##_fast_persist(const tx_gemm_args a) {    \
    gemm_persist<GemmCfg<ELA, ELB, 256, 256, 2, 2, 16>>(a);                                                  \
  }                                                                                                         \
  TX_KERNEL void __launch_bounds__(256) tx_gemm_fp8_##FA##_##FB##_grouped_persist(const tx_grouped_args q) { \
    gemm_persist<GemmCfg<ELA, ELB, 256, 256, 2, 2, 16>, OUT_BF16, true>(q.g, &q);                            \
  }

TX_GEMM_FP8_PERSIST(e4m3fn, e4m3fn, EL_E4M3, EL_E4M3)
TX_GEMM_FP8_PERSIST(e5m2, e5m2, EL_E5M2, EL_E5M2)
TX_GEMM_FP8_PERSIST(e4m3fn, e5m2, EL_E4M3, EL_E5M2)
TX_GEMM_FP8_PERSIST(e5m2, e4m3fn, EL_E5M2, EL_E4M3)

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
// fit its registers in 128 VGPRs).  The 4-wave kernel for one block of M
// is held to 4 workgroups per CU (128 registers): its grid at N = 14336 is
// 3.5 workgroups per CU, which must all be resident at once.
#define TX_GEMM_FP8_SKINNY(FA, FB, ELA, ELB, W, MB)                                            \
  TX_KERNEL void __launch_bounds__(64 * W, (W == 4 && MB == 1) ? 4 : 1)                        \
      tx_gemm_fp8_##FA##_##FB##_skinny_w##W##_m##MB(                                           \
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

// ---------------------------------------------------------------------------
// Grouped / batched fp8 GEMM (see tx_grouped_args): the fast tile, one
// workgroup per (problem, tile), no K split.
//
// Tile prefix of a grouped product: one workgroup scans the groups' m-tile
// counts ceil(rows / 256) in chunks of 256 (rows from the clamped offsets).
TX_KERNEL void __launch_bounds__(256) tx_gemm_fp8_grouped_prefix(const tx_grouped_args q) {
  __shared__ int sc[256];
  const int t = threadIdx.x;
  const int total = q.g.M;
  int carry = 0;
  if (t == 0) q.tile_prefix[0] = 0;
  for (int base = 0; base < q.groups; base += 256) {
    const int p = base + t;
    int c = 0;
    if (p < q.groups) {
      const int r1 = min(max(q.offsets[p + 1], 0), total);
      const int r0 = min(max(q.offsets[p], 0), r1);
      c = (r1 - r0 + q.tile_rows - 1) / q.tile_rows;
    }
    sc[t] = c;
    __syncthreads();
    for (int d = 1; d < 256; d *= 2) {  // inclusive scan
      const int v = t >= d ? sc[t - d] : 0;
      __syncthreads();
      sc[t] += v;
      __syncthreads();
    }
    if (p < q.groups) q.tile_prefix[p + 1] = carry + sc[t];
    carry += sc[255];
    __syncthreads();
  }
}

// Tile of workgroup wg among the real_m x tiles_n tiles of a grouped
// product (real_m = the prefix total, known only on the device; the grid
// is larger).  Workgroups reach the 8 XCDs round robin, so XCD x = wg % 8
// takes the x-th eighth of the real tiles in its own dispatch order (the
// same contiguous, L2-sharing ranges as tile_coords) and the rest of its
// workgroups leave: every XCD gets an equal share of the real work, which
// tile_coords over the padded grid would give mostly to the first XCDs.
__device__ __forceinline__ bool grouped_tile(int wg, int real_m, int tiles_n, int *tm, int *tn) {
  const int total = real_m * tiles_n;
  const int per = total / 8, rem = total % 8;
  const int x = wg % 8, i = wg / 8;
  if (i >= per + (x < rem ? 1 : 0)) return false;
  const int pid = x * per + (x < rem ? x : rem) + i;
  const int group_m = real_m < 8 ? real_m : 8;
  const int in_group = group_m * tiles_n;
  const int first_m = (pid / in_group) * group_m;
  const int gsz = (real_m - first_m) < group_m ? (real_m - first_m) : group_m;
  const int r = pid % in_group;
  *tm = first_m + r % gsz;
  *tn = r / gsz;
  return true;
}

template <class C, int BN, bool EPI>
__device__ __forceinline__ void gemm_fp8_grouped(const tx_grouped_args &q) {
  // bytes per C element: bf16, or the fused epilogue's output type
  const int ce = !EPI ? 2 : q.g.out_kind == EPI_OUT_F32 ? 4 : q.g.out_kind >= EPI_OUT_E4M3FN ? 1 : 2;
  int vm, tn;
  tx_gemm_args a = q.g;
  int p, tm;
  if (q.offsets) {
    const int32_t *T = q.tile_prefix;
    // uniform: a workgroup without a real tile leaves as a whole
    if (!grouped_tile(int(blockIdx.x), T[q.groups], q.g.tiles_n, &vm, &tn)) return;
    int lo = 0, hi = q.groups - 1;  // the last problem p with T[p] <= vm
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (T[mid] <= vm) lo = mid;
      else hi = mid - 1;
    }
    p = lo;
    tm = vm - T[p];
    const int r1 = min(max(q.offsets[p + 1], 0), q.g.M);
    const int r0 = min(max(q.offsets[p], 0), r1);
    a.M = r1 - r0;
    a.A = static_cast<const uint8_t *>(q.g.A) + int64_t(r0) * q.g.lda;
    a.C = static_cast<uint8_t *>(q.g.C) + int64_t(r0) * q.g.ldc * ce;
    a.scale_a = q.g.scale_a + r0;
  } else {
    tile_coords(int(blockIdx.x), q.mtiles, q.g.tiles_n, q.g.group_m, &vm, &tn);
    p = vm / q.tiles_per;
    tm = vm - p * q.tiles_per;
    if (p >= q.groups) return;
    a.A = static_cast<const uint8_t *>(q.g.A) + int64_t(p) * q.stride_a;
    a.C = static_cast<uint8_t *>(q.g.C) + int64_t(p) * q.stride_c * ce;
    a.scale_a = q.g.scale_a + int64_t(p) * q.stride_sa;
  }
  a.B = static_cast<const uint8_t *>(q.g.B) + int64_t(p) * q.stride_b;
  a.scale_b = q.g.scale_b + int64_t(p) * q.stride_sb;
  if (EPI && q.g.bias) a.bias = q.g.bias + int64_t(p) * q.stride_bias;
  gemm_fast_tile_at<C, BN, fast::kWaves, false, OUT_BF16, EPI>(a, tm, tn, 0);
}

// Groups of few rows: the roles swapped, so that a group's rows fill the
// tile's 128-wide side instead of a fraction of its 256 rows.  The tile's A
// operand is expert p's B (N rows), its B operand the group's rows of A
// (m tiles of 128 rows in the prefix), and the bf16 tile is stored
// transposed into C's rows.
template <class C>
__device__ __forceinline__ void gemm_fp8_grouped_t(const tx_grouped_args &q) {
  int vt, tf;  // 128-row tile of A (over all groups), 256-column tile of C
  const int32_t *T = q.tile_prefix;
  if (!grouped_tile(int(blockIdx.x), T[q.groups], q.g.tiles_n, &vt, &tf)) return;
  int lo = 0, hi = q.groups - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (T[mid] <= vt) lo = mid;
    else hi = mid - 1;
  }
  const int p = lo;
  const int r1 = min(max(q.offsets[p + 1], 0), q.g.M);
  const int r0 = min(max(q.offsets[p], 0), r1);
  tx_gemm_args a = q.g;
  a.A = static_cast<const uint8_t *>(q.g.B) + int64_t(p) * q.stride_b;
  a.lda = q.g.ldb;
  a.scale_a = q.g.scale_b + int64_t(p) * q.stride_sb;
  a.M = q.g.N;
  a.B = static_cast<const uint8_t *>(q.g.A) + int64_t(r0) * q.g.lda;
  a.ldb = q.g.lda;
  a.scale_b = q.g.scale_a + r0;
  a.N = r1 - r0;
  a.C = static_cast<uint16_t *>(q.g.C) + int64_t(r0) * q.g.ldc;
  gemm_fast_tile_at<C, 128, fast::kWaves, false, OUT_BF16, false, true>(a, tf, vt - T[p], 0);
}

#define TX_GEMM_FP8_GROUPED(FA, FB, ELA, ELB)                                                    \
  TX_KERNEL void __launch_bounds__(512) tx_gemm_fp8_##FA##_##FB##_grouped(const tx_grouped_args q) { \
    gemm_fp8_grouped<GemmCfg<ELA, ELB, 256, 256, 2, 2, 16>, 256, false>(q);                       \
  }                                                                                              \
  TX_KERNEL void __launch_bounds__(512) tx_gemm_fp8_##FA##_##FB##_grouped_n128(const tx_grouped_args q) { \
    gemm_fp8_grouped<GemmCfg<ELA, ELB, 256, 128, 2, 2, 16>, 128, false>(q);                       \
  }                                                                                              \
  TX_KERNEL void __launch_bounds__(512) tx_gemm_fp8_##FA##_##FB##_grouped_t(const tx_grouped_args q) { \
    gemm_fp8_grouped_t<GemmCfg<ELB, ELA, 256, 128, 2, 2, 16>>(q);                                 \
  }                                                                                              \
  TX_KERNEL void __launch_bounds__(512) tx_gemm_fp8_##FA##_##FB##_grouped_epi(const tx_grouped_args q) { \
    gemm_fp8_grouped<GemmCfg<ELA, ELB, 256, 256, 2, 2, 16>, 256, true>(q);                        \
  }                                                                                              \
  TX_KERNEL void __launch_bounds__(512) tx_gemm_fp8_##FA##_##FB##_grouped_epi_n128(const tx_grouped_args q) { \
    gemm_fp8_grouped<GemmCfg<ELA, ELB, 256, 128, 2, 2, 16>, 128, true>(q);                        \
  }

TX_GEMM_FP8_GROUPED(e4m3fn, e4m3fn, EL_E4M3, EL_E4M3)
TX_GEMM_FP8_GROUPED(e5m2, e5m2, EL_E5M2, EL_E5M2)
TX_GEMM_FP8_GROUPED(e4m3fn, e5m2, EL_E4M3, EL_E5M2)
TX_GEMM_FP8_GROUPED(e5m2, e4m3fn, EL_E5M2, EL_E4M3)
