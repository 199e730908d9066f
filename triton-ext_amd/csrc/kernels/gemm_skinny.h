// Skinny fp8 scaled GEMM (M <= 64) on gfx950:
//   C[m,n] = bf16_rne( scale_a[m] * scale_b[n] * sum_k A[m,k] * B[n,k] )
// A (M x K) and B (N x K) fp8, both K-contiguous, as tt.dot_scaled's
// row/column-scaled case with a decode-sized M.
//
// HBM-bound on B, which is read once.  A workgroup owns 16 rows of B (16
// output columns) and splits K over its wavefronts.  A wave streams its 16
// rows in rounds of 256 bytes per row (two 128-byte K slices): each of the 4
// loads of a round reads 4 whole 256-byte row segments (16 lanes x 16 bytes
// per row), and two rounds are in flight in registers.  The MFMA wants lane
// (r = lane % 16, g = lane / 16) to hold 32 bytes of row r, so each round is
// transposed through a private 4 KiB LDS tile: 16-byte chunk c of row r is
// stored at chunk c ^ (r & 15), which keeps both the writes (16 lanes of one
// row) and the fragment reads (16 rows, one logical chunk) in 16 different
// 16-byte bank groups.  Per slice a lane takes bytes [32g, 32g + 32) of the
// slice for both B and A (A is a few KiB per slice for the whole grid, read
// from cache), and one v_mfma_f32_16x16x128_f8f6f4 runs per 16-row block of
// A.  The per-wave partial sums are reduced across the workgroup in LDS and
// the scales applied once, in fp32, before the bf16 rounding.
#pragma once

#include "gemm_fast.h"

namespace txg {

template <int ELA, int ELB, int kWaves, int MB>
__device__ __forceinline__ void skinny_fp8_tile(const tx_gemm_args &a) {
  constexpr int kSlice = 128;        // K bytes per MFMA
  constexpr int kRound = 2;          // slices per round: 256 bytes per row
  constexpr int kDepth = 2;          // rounds in flight
  constexpr int kTile = 16 * 256;    // one wave's transpose tile
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kWaves * kTile];
  static_assert(kWaves * MB * 1024 <= kWaves * kTile, "reduction fits in the tiles");

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n0 = blockIdx.x * 16;
  const int r = lane & 15, g = lane >> 4;
  const int nslices = a.K / kSlice;  // host guarantees K % 128 == 0
  const int per_wave = (nslices + kWaves - 1) / kWaves;
  const int s_begin = min(nslices, wave * per_wave);
  const int s_end = min(nslices, s_begin + per_wave);
  const int nrounds = (s_end - s_begin + kRound - 1) / kRound;

  // Load j (0..3) of a round: row 4j + lane / 16 of the block, bytes
  // 16 (lane % 16) of that row's 256-byte segment.  Rows past N read the
  // last row (valid memory) and are never stored.
  // Buffer loads with 32-bit lane offsets from one resource per operand (the
  // host keeps 16 ldb and 64 lda below 2^31), which leaves the registers of
  // 64-bit row pointers to the loads in flight.
  constexpr int kNt = 2;  // buffer load cache policy: non-temporal
  const int rows_valid = min(16, a.N - n0);
  const __amdgpu_buffer_rsrc_t brs =
      make_rsrc(reinterpret_cast<const uint8_t *>(a.B) + int64_t(n0) * a.ldb,
                uint32_t(rows_valid - 1) * uint32_t(a.ldb) + uint32_t(a.K));
  uint32_t boff[4];
  int wpos[4];
  uint8_t *tile = lds + wave * kTile;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = 4 * j + (lane >> 4);
    boff[j] = uint32_t(min(row, rows_valid - 1)) * uint32_t(a.ldb);
    wpos[j] = row * 256 + (((lane & 15) ^ (row & 15)) << 4);
  }
  // Fragment read offsets: slice u of a round, pieces e = 0, 1 (logical
  // chunks 8u + 2g + e of row r).
  int rpos[kRound][2];
#pragma unroll
  for (int u = 0; u < kRound; ++u)
#pragma unroll
    for (int e = 0; e < 2; ++e) rpos[u][e] = r * 256 + (((8 * u + 2 * g + e) ^ r) << 4);
  // A rows past M read the last valid row and are never stored.
  const __amdgpu_buffer_rsrc_t ars = make_rsrc(a.A, uint32_t(a.M - 1) * uint32_t(a.lda) + uint32_t(a.K));
  uint32_t aoff[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int m = mb * 16 + r;
    aoff[mb] = uint32_t(m < a.M ? m : a.M - 1) * uint32_t(a.lda) + 32 * g;
  }

  // A round's B loads and (one 16-row block of A, 4 waves) its A fragments,
  // loaded together two rounds ahead of use: the CU serves vector loads in
  // order, so A loaded where it is used (a cache hit) would wait behind the
  // B round in flight.  With more blocks of A the fragments would not fit
  // the registers and are loaded where used.
  constexpr bool kAAhead = MB == 1;
  struct Round {
    txd::u32x4 w[4];
    txd::u32x4 xa[kAAhead ? kRound : 1][MB][2];
  };
  auto a_frags = [&](int s, int u, int ns, txd::u32x4 (&xa)[MB][2]) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const uint32_t o = aoff[mb] + uint32_t(s + (u < ns ? u : 0)) * kSlice;
      xa[mb][0] = __builtin_bit_cast(txd::u32x4, __builtin_amdgcn_raw_buffer_load_b128(ars, int(o), 0, 0));
      xa[mb][1] = __builtin_bit_cast(txd::u32x4, __builtin_amdgcn_raw_buffer_load_b128(ars, int(o + 16), 0, 0));
    }
  };
  // Round q's loads.  Every lane loads (no per-lane select: its merge would
  // make the wave wait for the load right away); in a round with one slice
  // left, lanes 8..15 re-read the slice's last chunk into the unused half of
  // the tile.
  auto fetch = [&](int q, Round &f) {
    const int s = s_begin + q * kRound;
    const int valid = min(kRound, s_end - s) * kSlice;
    if constexpr (kAAhead) {
#pragma unroll
      for (int u = 0; u < kRound; ++u) a_frags(s, u, valid / kSlice, f.xa[u]);
    }
    const uint32_t off = uint32_t(s * kSlice + min(16 * (lane & 15), valid - 16));
#pragma unroll
    for (int j = 0; j < 4; ++j)
      f.w[j] = __builtin_bit_cast(txd::u32x4, __builtin_amdgcn_raw_buffer_load_b128(brs, int(boff[j] + off), 0, kNt));
  };
  txd::f32x4 acc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = txd::f32x4{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](int q, const Round &f) {
    const int s = s_begin + q * kRound;
    const int ns = min(kRound, s_end - s);
    txd::u32x4 xa[kRound][MB][2];
#pragma unroll
    for (int u = 0; u < kRound; ++u) {
      if constexpr (kAAhead) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) xa[u][mb][0] = f.xa[u][mb][0], xa[u][mb][1] = f.xa[u][mb][1];
      } else {
        a_frags(s, u, ns, xa[u]);
      }
    }
    // Transpose through the wave's tile (LDS operations of one wave complete
    // in order, so the reads see the writes and the next round's writes
    // follow these reads).
#pragma unroll
    for (int j = 0; j < 4; ++j) *reinterpret_cast<txd::u32x4 *>(tile + wpos[j]) = f.w[j];
    asm volatile("" ::: "memory");
#pragma unroll
    for (int u = 0; u < kRound; ++u) {
      if (u < ns) {
        const txd::i32x4 w0 = *reinterpret_cast<const txd::i32x4 *>(tile + rpos[u][0]);
        const txd::i32x4 w1 = *reinterpret_cast<const txd::i32x4 *>(tile + rpos[u][1]);
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
    asm volatile("" ::: "memory");
  };

  // Two rounds in flight.  With A loaded ahead, no load is issued on a
  // conditional path: the compiler's wait counts merge over branches and
  // would otherwise wait for every outstanding load at the loop head.  So
  // that schedule takes two rounds per loop iteration and always fetches,
  // the last one to three rounds are straight-line tails, and the prologue's
  // second round re-reads round 0 when the wave has only one.  (The other
  // variants load A where used, which waits for the B round in flight anyway;
  // they keep the shorter loop, which needs fewer registers.)
  static_assert(kDepth == 2, "the schedules below keep two rounds in flight");
  if constexpr (kAAhead) {
    if (nrounds > 0) {
      Round b0, b1;
      fetch(0, b0);
      fetch(min(1, nrounds - 1), b1);
      int q = 0;
      for (; q + 3 < nrounds; q += 2) {
        compute(q, b0);
        fetch(q + 2, b0);
        compute(q + 1, b1);
        fetch(q + 3, b1);
      }
      const int rem = nrounds - q;  // 1, 2 or 3
      if (rem == 3) {
        compute(q, b0);
        fetch(q + 2, b0);
        compute(q + 1, b1);
        compute(q + 2, b0);
      } else if (rem == 2) {
        compute(q, b0);
        compute(q + 1, b1);
      } else {
        compute(q, b0);
      }
    }
  } else {
    // Round slots are compile-time registers: slot d holds rounds congruent
    // to d mod kDepth, refilled right after its round is consumed.
    Round buf[kDepth];
#pragma unroll
    for (int d = 0; d < kDepth; ++d)
      if (d < nrounds) fetch(d, buf[d]);
    for (int q0 = 0; q0 < nrounds; q0 += kDepth) {
#pragma unroll
      for (int d = 0; d < kDepth; ++d) {
        const int q = q0 + d;
        if (q < nrounds) {
          compute(q, buf[d]);
          if (q + kDepth < nrounds) fetch(q + kDepth, buf[d]);
        }
      }
    }
  }

  // Cross-wave reduction in LDS (reusing the tiles); MFMA result layout:
  // lane holds D[m = 4 * (lane / 16) + i][n = lane % 16].
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
        if (m >= a.M) continue;
        if (a.epi) a.part[int64_t(m) * a.N + n] = v[i] * a.scale_a[m] * sb;  // epilogue pass follows
        else Cb[int64_t(m) * a.ldc + n] = uint16_t(txd::f32_to_bf16_bits(v[i] * a.scale_a[m] * sb));
      }
    }
  }
}

}  // namespace txg
