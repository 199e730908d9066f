// fp8 weight-only dequant GEMV / skinny GEMM on gfx950:
//   y[m,n] = bf16_rne( sum_g s[n,g] * sum_{k in g} x[m,k] * W[n,k] )
// x bf16 (M <= 64 rows), W fp8 N x K row-major, s fp32 N x (K/group).
//
// HBM-bound on W, which is read once.  A workgroup owns up to 16 or 32 rows
// of W (one or two 16-row blocks, 16 output columns each; the host spreads
// the rows evenly over a whole number of workgroups per CU) and splits K over
// its wavefronts.  A wave streams its rows in rounds of 256 bytes per row:
// each of the 4 loads of a round reads 4 whole 256-byte row segments, two
// rounds are in flight in registers, and a round is transposed through a
// private 4 KiB LDS tile per block (chunk c of row r at chunk c ^ (r & 15))
// into MFMA fragments.  Each round's x fragments and group scales are loaded
// with its W, two rounds ahead: the CU serves vector loads in order, so x
// loaded where it is used (an L2 hit) would wait behind the W round in
// flight.  No load sits on a conditional path (see the schedule below).  The
// per-wave partial sums are reduced across the workgroup in LDS.
//
// Dequantisation is gfx950's scaled fp8 -> bf16 pair conversion
// (v_cvt_scalef32_pk_bf16_bf8 / _fp8, scale 1): two instructions per four
// codes, exact for every code (bf16 holds every e4m3fn and e5m2 value,
// subnormals included), with NaN codes giving NaN and e5m2 Inf giving Inf,
// so the products propagate them as fp32 arithmetic on the decoded values
// would.  The products run on the bf16 MFMA
// v_mfma_f32_16x16x32_bf16 with fp32 accumulation; each 128-wide (group)
// partial sum is scaled in fp32 before it joins the running sum.
#include <type_traits>

#include "tx_device.h"

namespace {

constexpr int kSlice = 128;     // K elements per slice (one group-scale unit)

// Four fp8 codes (one 32-bit word) -> four bf16 (two words): codes 0, 1 into
// lo (code 0 in the low half), codes 2, 3 into hi.
template <int FMT>
__device__ __forceinline__ void fp8x4_to_bf16x4(uint32_t w, uint32_t &lo, uint32_t &hi) {
  if constexpr (FMT == 2) {
    lo = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w, 1.0f, false));
    hi = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w, 1.0f, true));
  } else {
    lo = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false));
    hi = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true));
  }
}

template <int FMT, int kWaves, int MB, int NB>
__device__ __forceinline__ void gemv_body(const tx_gemv_args &a) {
  constexpr int kRound = 2;          // slices per round: 256 bytes per W row
  constexpr int kDepth = 2;          // rounds in flight
  constexpr int kTile = 16 * 256;    // one wave's transpose tile
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kWaves * NB * kTile];
  static_assert(MB * NB * 1024 <= NB * kTile, "reduction fits in the tiles");

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // This workgroup's W rows: [n0, n_end), at most 16 NB of them (the host
  // sizes rows_per_wg so that every CU gets the same number of rows).
  const int n0 = blockIdx.x * a.rows_per_wg;
  const int n_end = min(a.N, n0 + a.rows_per_wg);
  const int r = lane & 15, g = lane >> 4;
  const int nslices = a.K / kSlice;  // host guarantees K % 128 == 0
  const int per_wave = (nslices + kWaves - 1) / kWaves;
  const int s_begin = min(nslices, wave * per_wave);
  const int s_end = min(nslices, s_begin + per_wave);
  const int nrounds = (s_end - s_begin + kRound - 1) / kRound;
  const int slices_per_group = a.group / kSlice;  // host: group % 128 == 0

  // Load j (0..3) of a round of block b: W row 16b + 4j + lane / 16, bytes
  // 16 (lane % 16) of that row's 256-byte segment.  Rows past the
  // workgroup's range read its last row (the same addresses in one load, so
  // no extra traffic) and are never stored.
  const uint8_t *wp[NB][4];
  int wpos[4];
  uint8_t *tile = lds + wave * NB * kTile;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = 4 * j + (lane >> 4);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int n = n0 + 16 * b + row;
      wp[b][j] = a.W + int64_t(n < n_end ? n : n_end - 1) * a.ldw;
    }
    wpos[j] = row * 256 + (((lane & 15) ^ (row & 15)) << 4);
  }
  // Fragment reads: MFMA i of slice u takes codes 32 i + 8 g .. + 7 of row r,
  // 8 bytes at chunk 8 u + 2 i + g / 2 of the row's 256-byte segment.
  auto rpos = [&](int u, int i) { return r * 256 + (((8 * u + 2 * i + (g >> 1)) ^ r) << 4) + 8 * (g & 1); };

  // This lane's output columns (W rows 16b + r); their group scales travel
  // with each round's x fragments.
  const float *srow[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int nc = n0 + 16 * b + r;
    srow[b] = a.scales + int64_t(nc < n_end ? nc : n_end - 1) * a.ld_scales;
  }
  // x rows past M read row M-1: MFMA output rows are independent and rows
  // past M are never stored, so no masking is needed.
  const uint16_t *xrow[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int m = mb * 16 + r;
    xrow[mb] = a.x + int64_t(m < a.M ? m : a.M - 1) * a.ldx + 8 * g;
  }

  struct Round {
    txd::u32x4 w[NB][4];
  };
  // Every lane loads (no per-lane select, whose merge would make the wave
  // wait for the load right away): in a round with one slice left, lanes 8..15
  // re-read the slice's last chunk, which lands in the unused half of the tile.
  auto fetch = [&](int q, Round &f) {
    const int s = s_begin + q * kRound;
    const int valid = min(kRound, s_end - s) * kSlice;
    const int off = s * kSlice + min(16 * (lane & 15), valid - 16);
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        f.w[b][j] = __builtin_nontemporal_load(reinterpret_cast<const txd::u32x4 *>(wp[b][j] + off));
  };
  // x fragments and group scales of round q (slices past the wave's range
  // repeat its last one), loaded just before the round's W, two rounds ahead
  // of use: waiting for them (memory counters retire in order) then waits only
  // for loads issued before them, never for a later W round.
  // With more than one 16-row block of x, or 16 wavefronts (128 registers
  // each), two rounds of fragments would not fit the registers: those kernels
  // load x where it is used (and wait for the W round in flight before it).
  constexpr bool kXAhead = MB == 1 && kWaves <= 4;
  struct XRound {
    txd::u32x4 v[kXAhead ? kRound : 1][MB][4];
    float sc[kRound][NB];  // group scale of each slice's group
  };
  auto x_frags = [&](int su, txd::u32x4 (&xv)[MB][4]) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        xv[mb][i] = *reinterpret_cast<const txd::u32x4 *>(xrow[mb] + su * kSlice + 32 * i);
  };
  auto load_x = [&](int q, XRound &xr) {
#pragma unroll
    for (int u = 0; u < kRound; ++u) {
      const int su = min(s_begin + q * kRound + u, s_end - 1);
      if constexpr (kXAhead) x_frags(su, xr.v[u]);
#pragma unroll
      for (int b = 0; b < NB; ++b) xr.sc[u][b] = srow[b][su / slices_per_group];
    }
  };

  txd::f32x4 acc[NB][MB], part[NB][MB];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int i = 0; i < MB; ++i) acc[b][i] = part[b][i] = txd::f32x4{0.f, 0.f, 0.f, 0.f};
  bool fresh = true;  // the next MFMA chain starts from zero

  // Slice s: MFMA i takes k = 32 i + 8 g .. + 7 of the slice in lane (r, g),
  // of both W and x (so that a lane group's x loads read 64 contiguous bytes
  // of each row: 16 cache-line halves per load instead of 32 lines).
  auto compute = [&](int q, const Round &f, const XRound &xr) {
    const int s = s_begin + q * kRound;
    const int ns = min(kRound, s_end - s);
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int j = 0; j < 4; ++j) *reinterpret_cast<txd::u32x4 *>(tile + b * kTile + wpos[j]) = f.w[b][j];
    asm volatile("" ::: "memory");
#pragma unroll
    for (int u = 0; u < kRound; ++u) {
      if (u < ns) {
        const int su = s + u;
        txd::u32x4 xv[MB][4];
        if constexpr (kXAhead) {
#pragma unroll
          for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int i = 0; i < 4; ++i) xv[mb][i] = xr.v[u][mb][i];
        } else {
          x_frags(su, xv);
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          uint32_t wb[16];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const txd::u32x2 c = *reinterpret_cast<const txd::u32x2 *>(tile + b * kTile + rpos(u, i));
            fp8x4_to_bf16x4<FMT>(c.x, wb[4 * i], wb[4 * i + 1]);
            fp8x4_to_bf16x4<FMT>(c.y, wb[4 * i + 2], wb[4 * i + 3]);
          }
#pragma unroll
          for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const txd::u32x4 wq = {wb[4 * i], wb[4 * i + 1], wb[4 * i + 2], wb[4 * i + 3]};
              const txd::f32x4 c = (i == 0 && fresh) ? txd::f32x4{0.f, 0.f, 0.f, 0.f} : part[b][mb];
              part[b][mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                  __builtin_bit_cast(txd::bf16x8, xv[mb][i]), __builtin_bit_cast(txd::bf16x8, wq), c, 0, 0, 0);
            }
        }
        fresh = false;
        // close the group when its last slice is done (uniform)
        if ((su + 1) % slices_per_group == 0 || su + 1 == nslices) {
#pragma unroll
          for (int b = 0; b < NB; ++b) {
            const float sc = xr.sc[u][b];
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) acc[b][mb] += part[b][mb] * sc;
          }
          fresh = true;
        }
      }
    }
    asm volatile("" ::: "memory");
  };

  // Two rounds in flight, each with its x fragments and scales (requested
  // just before its W).  No load is issued on a conditional path: the
  // compiler's wait counts merge over branches and would otherwise wait for
  // every outstanding load at the loop head.  So the steady-state loop takes
  // two rounds per iteration and always fetches, the last one to three rounds
  // are straight-line tails, and the prologue's second round re-reads round 0
  // when the wave has only one.
  static_assert(kDepth == 2, "the schedule below keeps two rounds in flight");
  if (nrounds > 0) {
    Round b0, b1;
    XRound x0, x1;
    load_x(0, x0);
    fetch(0, b0);
    load_x(min(1, nrounds - 1), x1);
    fetch(min(1, nrounds - 1), b1);
    int q = 0;
    for (; q + 3 < nrounds; q += 2) {
      compute(q, b0, x0);
      load_x(q + 2, x0);
      fetch(q + 2, b0);
      compute(q + 1, b1, x1);
      load_x(q + 3, x1);
      fetch(q + 3, b1);
    }
    const int rem = nrounds - q;  // 1, 2 or 3
    bool last0 = true;            // the last round's scales are in x0
    if (rem == 3) {
      compute(q, b0, x0);
      load_x(q + 2, x0);
      fetch(q + 2, b0);
      compute(q + 1, b1, x1);
      compute(q + 2, b0, x0);
    } else if (rem == 2) {
      compute(q, b0, x0);
      compute(q + 1, b1, x1);
      last0 = false;
    } else {
      compute(q, b0, x0);
    }
    // A group split across two waves leaves a partial in both; scale it
    // here with the scale of the wave's last slice.
    if (!fresh) {
      const int ul = (s_end - 1 - s_begin) % kRound;
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const float s0 = ul == 0 ? x0.sc[0][b] : x0.sc[kRound - 1][b];
        const float s1 = ul == 0 ? x1.sc[0][b] : x1.sc[kRound - 1][b];
        const float sc = last0 ? s0 : s1;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[b][mb] += part[b][mb] * sc;
      }
    }
  }

  // Cross-wave reduction in LDS (reusing the tiles), one W block at a time;
  // MFMA result layout: lane holds D[m = 4 * (lane / 16) + i][n = lane % 16].
  txd::f32x4 *red = reinterpret_cast<txd::f32x4 *>(lds);  // [kWaves][MB][64]
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    __syncthreads();
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) red[(wave * MB + mb) * 64 + lane] = acc[b][mb];
    __syncthreads();
    if (wave < MB) {
      const int mb = wave;
      txd::f32x4 t = red[mb * 64 + lane];
#pragma unroll
      for (int w = 1; w < kWaves; ++w) t += red[(w * MB + mb) * 64 + lane];
      const int ncol = n0 + 16 * b + r;
      if (ncol < n_end) {
        const float v[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = mb * 16 + 4 * g + i;
          if (m < a.M) a.y[int64_t(m) * a.ldy + ncol] = uint16_t(txd::f32_to_bf16_bits(v[i]));
        }
      }
    }
  }
}

// One row of x (M = 1, batch-1 decode): a plain streaming dot on the VALU.  Wave w of
// workgroup b owns W rows 2 (4 b + w) and 2 (4 b + w) + 1 and walks them in
// 1 KiB slices (lane l: bytes 16 l .. 16 l + 15 of the slice, so one load
// instruction reads 1 KiB of one row, contiguous, non-temporal), two
// slices of both rows in flight at a time.  x (M x K bf16, at most
// kLinMaxX bytes) is staged in LDS once per workgroup, in dynamic LDS of
// exactly its size, which keeps the registers to the W stream (54) and the
// occupancy at 8 waves per SIMD.  Small workgroups of 4 wavefronts (8 W
// rows) spread the rows evenly over the CUs (14336 rows: 7 workgroups per
// CU; 8 wavefronts and 16 rows per workgroup left 3 or 4 per CU and ran
// 14.4 against 11.9 us).  The codes become fp32 through gfx950's packed
// conversions (exact for every finite code), each lane's 16 products are
// summed in fp32 and scaled by their group's scale (16 consecutive K never
// cross a group: group % 128 == 0), and the lanes' sums meet in a butterfly
// reduction.
constexpr int kLinMaxX = 32768;
constexpr int kLinWaves = 4;

template <int FMT, int MB>
__device__ __forceinline__ void gemv_lin(const tx_gemv_args &a) {
  constexpr int RPW = 2, CB = 2;  // rows per wave, 1 KiB slices per batch
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];  // MB x K, K * MB * 2 <= kLinMaxX
  // the wave index is uniform: row bases stay scalar, loads take a 32-bit lane offset
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // x rows into LDS (row pitch K), 16 bytes per thread and step
  for (int e = 8 * int(threadIdx.x); e < MB * a.K; e += 8 * 64 * kLinWaves) {
    const int m = e / a.K, k = e - m * a.K;
    *reinterpret_cast<txd::u32x4 *>(xs + e) =
        m < a.M ? *reinterpret_cast<const txd::u32x4 *>(a.x + int64_t(m) * a.ldx + k) : txd::u32x4{0, 0, 0, 0};
  }
  __syncthreads();
  const int row0 = (int(blockIdx.x) * kLinWaves + wave) * RPW;
  if (row0 >= a.N) return;  // whole wave, after the only barrier
  const int nslices = (a.K + 1023) / 1024;
  float acc[RPW][MB];
#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int m = 0; m < MB; ++m) acc[r][m] = 0.0f;
  for (int c0 = 0; c0 < nslices; c0 += CB) {
    txd::u32x4 w[CB][RPW];
    float sc[CB][RPW];
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      const int k = (c0 + c) * 1024 + 16 * lane;
      const bool in = c0 + c < nslices && k < a.K;
#pragma unroll
      for (int r = 0; r < RPW; ++r) {
        const bool ok = in && row0 + r < a.N;
        const uint8_t *wrow = a.W + int64_t(row0 + r) * a.ldw;  // uniform
        const float *srow = a.scales + int64_t(row0 + r) * a.ld_scales;
        w[c][r] = ok ? __builtin_nontemporal_load(reinterpret_cast<const txd::u32x4 *>(wrow + uint32_t(k)))
                     : txd::u32x4{0, 0, 0, 0};
        sc[c][r] = ok ? srow[uint32_t(k) / uint32_t(a.group)] : 0.0f;
      }
    }
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      const int k = (c0 + c) * 1024 + 16 * lane;
      if (c0 + c >= nslices || k >= a.K) continue;  // that lane's slice is empty (w = 0 as well)
#pragma unroll
      for (int r = 0; r < RPW; ++r) {
        float t[MB];
#pragma unroll
        for (int m = 0; m < MB; ++m) t[m] = 0.0f;
        // four codes at a time: their fp32 values and the four x values
        // (8 bytes of LDS) meet in four fused multiply-adds
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const int code4 = int(w[c][r][d]);
          const auto lo = FMT == 2 ? __builtin_amdgcn_cvt_pk_f32_bf8(code4, false)
                                   : __builtin_amdgcn_cvt_pk_f32_fp8(code4, false);
          const auto hi = FMT == 2 ? __builtin_amdgcn_cvt_pk_f32_bf8(code4, true)
                                   : __builtin_amdgcn_cvt_pk_f32_fp8(code4, true);
#pragma unroll
          for (int m = 0; m < MB; ++m) {
            const txd::u32x2 xw = *reinterpret_cast<const txd::u32x2 *>(xs + m * a.K + k + 4 * d);
            t[m] = fmaf(__uint_as_float(xw.x << 16), lo[0], t[m]);
            t[m] = fmaf(__uint_as_float(xw.x & 0xFFFF0000u), lo[1], t[m]);
            t[m] = fmaf(__uint_as_float(xw.y << 16), hi[0], t[m]);
            t[m] = fmaf(__uint_as_float(xw.y & 0xFFFF0000u), hi[1], t[m]);
          }
        }
#pragma unroll
        for (int m = 0; m < MB; ++m) acc[r][m] = fmaf(t[m], sc[c][r], acc[r][m]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int m = 0; m < MB; ++m)
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) acc[r][m] += __shfl_xor(acc[r][m], o);
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
      for (int m = 0; m < MB; ++m)
        if (row0 + r < a.N && m < a.M)
          a.y[int64_t(m) * a.ldy + row0 + r] = uint16_t(txd::f32_to_bf16_bits(acc[r][m]));
  }
}


}  // namespace

// Streaming VALU kernels for M = 1: tx_gemv_fp8_<w format>_lin_m1 (at M = 2 the
// MFMA kernel is faster: 17.4 against ~16 us at 14336 x 4096).
#define TX_GEMV_LIN(NAME, FMT, MB)                                                                      \
  TX_KERNEL void __launch_bounds__(64 * kLinWaves, 8) tx_gemv_fp8_##NAME##_lin_m##MB(const tx_gemv_args a) { \
    gemv_lin<FMT, MB>(a);                                                                        \
  }
TX_GEMV_LIN(e5m2, 2, 1)
TX_GEMV_LIN(e4m3fn, 1, 1)

// Kernel names: tx_gemv_fp8_<w format>_w<waves>_m<16-row blocks of M>_b<W
// blocks per wave>.  Two W blocks per wave share each x fragment (for M above
// a few rows the x reads from cache would otherwise outweigh the W stream);
// the small-grid variants with 2 or 4 blocks of M have 8 wavefronts (16 would
// not fit their registers in 128 VGPRs).
#define TX_GEMV(NAME, FMT, W, MB, NB)                                                         \
  TX_KERNEL void __launch_bounds__(64 * W) tx_gemv_fp8_##NAME##_w##W##_m##MB##_b##NB(         \
      const tx_gemv_args a) {                                                                 \
    gemv_body<FMT, W, MB, NB>(a);                                                             \
  }
#define TX_GEMV_ALL(NAME, FMT)                                                                   \
  TX_GEMV(NAME, FMT, 4, 1, 1) TX_GEMV(NAME, FMT, 4, 1, 2) TX_GEMV(NAME, FMT, 4, 2, 2)           \
  TX_GEMV(NAME, FMT, 4, 4, 2) TX_GEMV(NAME, FMT, 16, 1, 1) TX_GEMV(NAME, FMT, 8, 2, 1)          \
  TX_GEMV(NAME, FMT, 8, 4, 1)
TX_GEMV_ALL(e5m2, 2)
TX_GEMV_ALL(e4m3fn, 1)
