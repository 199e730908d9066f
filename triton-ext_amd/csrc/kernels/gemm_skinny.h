// Skinny fp8 scaled GEMM (M <= 64) on gfx950:
//   C[m,n] = bf16_rne( scale_a[m] * scale_b[n] * sum_k A[m,k] * B[n,k] )
// A (M x K) and B (N x K) fp8, both K-contiguous, as tt.dot_scaled's
// row/column-scaled case with a decode-sized M.
//
// HBM-bound on B, which is read once.  A workgroup owns 16 rows of B (16
// output columns) and splits K over its wavefronts.  Each wave streams its
// 16 rows through a private LDS stage (double-buffered when its K range spans
// several chunks; a single stage keeps two workgroups per CU) with gfx950's
// `buffer_load_dwordx4 ... lds` (one instruction fills 1 KiB = 1024 / KC rows
// of a KC-byte chunk, so the 64 lanes read whole contiguous lines of B), and
// reads the MFMA fragments back from LDS.  The stage stores 16-byte chunk c of
// row r at chunk c ^ (r & 15): the 16 lanes of a ds_read_b128 phase read one
// logical chunk of 16 consecutive rows, which this places in 16 different
// 16-byte bank groups.  Per 128-byte K slice a lane (row r = lane % 16,
// group g = lane / 16) takes bytes [32g, 32g + 32) of the slice for both B and
// A (A is a few KiB per slice for the whole grid, read from cache), and one
// v_mfma_f32_16x16x128_f8f6f4 per 16-row block of A.  The per-wave partial
// sums are reduced across the workgroup in LDS and the scales applied once,
// in fp32, before the bf16 rounding.
#pragma once

#include "gemm_fast.h"

namespace txg {

template <int ELA, int ELB, int kWaves, int MB, int KC, int kStages>
__device__ __forceinline__ void skinny_fp8_tile(const tx_gemm_args &a) {
  static_assert(kStages == 1 || kStages == 2, "one or two stages per wave");
  constexpr int kSlice = 128;             // K bytes per MFMA
  constexpr int kSpc = KC / kSlice;       // slices per chunk
  constexpr int kStage = 16 * KC;         // one wave's stage: 16 rows x KC bytes
  constexpr int kRpi = 1024 / KC;         // rows per load instruction
  constexpr int kCpr = KC / 16;           // 16-byte chunks per row
  constexpr int kLoads = 16 / kRpi;       // load instructions per stage
  static_assert(kCpr >= 16 && kLoads >= 1, "chunk of 256 bytes or more");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kWaves * kStages * kStage];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n0 = blockIdx.x * 16;
  const int r = lane & 15, g = lane >> 4;
  const int nslices = a.K / kSlice;  // host guarantees K % 128 == 0
  const int per_wave = (nslices + kWaves - 1) / kWaves;
  const int s_begin = min(nslices, wave * per_wave);
  const int s_end = min(nslices, s_begin + per_wave);
  const int nchunks = (s_end - s_begin + kSpc - 1) / kSpc;

  // Loads: instruction j covers rows kRpi*j .. kRpi*j + kRpi - 1; lane i lands
  // in row kRpi*j + i / kCpr, physical chunk i % kCpr, and fetches logical
  // chunk (i % kCpr) ^ (row & 15).  Rows past N read as zero (never stored).
  const uint32_t kb_end = uint32_t(a.K);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(a.B, uint32_t(a.N - 1) * uint32_t(a.ldb) + kb_end);
  uint32_t vo[kLoads], lc[kLoads];
#pragma unroll
  for (int j = 0; j < kLoads; ++j) {
    const int row = kRpi * j + lane / kCpr;
    lc[j] = uint32_t((lane % kCpr) ^ (row & 15));
    vo[j] = n0 + row < a.N ? uint32_t(n0 + row) * uint32_t(a.ldb) + 16u * lc[j] : kOob;
  }
  uint8_t *my = lds + wave * kStages * kStage;
  auto issue = [&](int c) {
    const int s = s_begin + c * kSpc;
    const uint32_t kb = uint32_t(s) * kSlice;
    const uint32_t valid = uint32_t(min(kSpc, s_end - s)) * kSlice;  // bytes of this chunk in range
    uint8_t *st = my + (kStages == 2 ? (c & 1) * kStage : 0);
#pragma unroll
    for (int j = 0; j < kLoads; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void *)(st + 1024 * j), 16,
                                               16u * lc[j] < valid ? vo[j] : kOob, kb, 0, 0);
  };

  // A rows past M read the last valid row and are never stored.
  const uint8_t *arow[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int m = mb * 16 + r;
    arow[mb] = reinterpret_cast<const uint8_t *>(a.A) + int64_t(m < a.M ? m : a.M - 1) * a.lda + 32 * g;
  }
  // Read offsets of this lane's two 16-byte pieces of slice u (logical chunks
  // 8u + 2g and 8u + 2g + 1 of row r).
  int ro[kSpc][2];
#pragma unroll
  for (int u = 0; u < kSpc; ++u)
#pragma unroll
    for (int e = 0; e < 2; ++e) ro[u][e] = r * KC + (((8 * u + 2 * g + e) ^ r) << 4);

  txd::f32x4 acc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = txd::f32x4{0.f, 0.f, 0.f, 0.f};

  if (nchunks > 0) issue(0);
  for (int c = 0; c < nchunks; ++c) {
    const int s = s_begin + c * kSpc;
    const int ns = min(kSpc, s_end - s);
    // A pieces of this chunk (cache-resident); issued before the next chunk's
    // loads so that loads completing in order lets the wait below leave only
    // those in flight.
    txd::u32x4 xa[kSpc][MB][2];
#pragma unroll
    for (int u = 0; u < kSpc; ++u)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const txd::u32x4 *xp = reinterpret_cast<const txd::u32x4 *>(arow[mb] + (s + (u < ns ? u : 0)) * kSlice);
        xa[u][mb][0] = xp[0];
        xa[u][mb][1] = xp[1];
      }
    if (kStages == 2 && c + 1 < nchunks) {
      issue(c + 1);
      __builtin_amdgcn_s_waitcnt((kLoads & 15) | (7 << 4) | (0xF << 8) | ((kLoads >> 4) << 14));
    } else {
      __builtin_amdgcn_s_waitcnt((7 << 4) | (0xF << 8));  // vmcnt(0)
    }
    asm volatile("" ::: "memory");
    const uint8_t *st = my + (kStages == 2 ? (c & 1) * kStage : 0);
#pragma unroll
    for (int u = 0; u < kSpc; ++u) {
      if (u < ns) {
        const txd::i32x4 w0 = *reinterpret_cast<const txd::i32x4 *>(st + ro[u][0]);
        const txd::i32x4 w1 = *reinterpret_cast<const txd::i32x4 *>(st + ro[u][1]);
        const i32x8 wv = __builtin_shufflevector(w0, w1, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          const i32x8 xv = __builtin_bit_cast(i32x8, __builtin_shufflevector(xa[u][mb][0], xa[u][mb][1], 0, 1, 2, 3, 4, 5, 6, 7));
          // src0 = A rows (output rows m), src1 = B rows (output columns n)
          acc[mb] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(xv, wv, acc[mb], F8Code<ELA>::v,
                                                                     F8Code<ELB>::v, 0, 0, 0, 0);
        }
      }
    }
    // The stage just read is refilled by the next load: its reads must be
    // complete first.
    __builtin_amdgcn_s_waitcnt((0xF) | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0)
    asm volatile("" ::: "memory");
    if (kStages == 1 && c + 1 < nchunks) issue(c + 1);
  }

  // Cross-wave reduction in LDS (reusing the stage memory); MFMA result
  // layout: lane holds D[m = 4 * (lane / 16) + i][n = lane % 16].
  __syncthreads();
  txd::f32x4 *red = reinterpret_cast<txd::f32x4 *>(lds);  // [kWaves][MB][64]
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) red[(wave * MB + mb) * 64 + lane] = acc[mb];
  __syncthreads();
  if (wave < MB) {
    const int mb = wave;
    txd::f32x4 t = red[mb * 64 + lane];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) t += red[(w * MB + mb) * 64 + lane];
    const int n = n0 + r;
    if (n < a.N) {
      const float sb = a.scale_b[n];
      const float v[4] = {t.x, t.y, t.z, t.w};
      uint16_t *Cb = reinterpret_cast<uint16_t *>(a.C);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = mb * 16 + 4 * g + i;
        if (m < a.M) Cb[int64_t(m) * a.ldc + n] = uint16_t(txd::f32_to_bf16_bits(v[i] * a.scale_a[m] * sb));
      }
    }
  }
}

}  // namespace txg
