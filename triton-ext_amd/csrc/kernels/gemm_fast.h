// Fast-path GEMM body for aligned operands (both K-contiguous, 16-byte
// aligned rows, K * element size a multiple of 16 bytes), 256 x 256 tile,
// 8 wavefronts of 128 x 64 (two per SIMD) or 4 of 128 x 128.
//
// Pipeline (per 64-byte K step, i.e. 32 bf16 or 64 fp8 of K):
//  * LDS holds 4 stages of (256 A rows + 256 B rows) x 64 bytes = 4 x 32 KiB.
//    Rows are 4 chunks of 16 bytes stored at chunk ^ ((row >> 2) & 3): a
//    ds_read_b128 is served 16 lanes at a time over 256 bytes of banks, the
//    fragment reads have 16 lanes read one logical chunk of 16 consecutive
//    rows, and this swizzle spreads those over the 16 bank groups.
//  * global -> LDS bypasses registers: gfx950's `buffer_load_dwordx4 ... lds`
//    writes each lane's 16 bytes at M0 + 16 * lane, so one instruction fills a
//    1 KiB block = 16 rows; lane i lands in row i / 4, physical chunk i % 4 and
//    therefore fetches logical chunk (i % 4) ^ (i / 16).  Out-of-range rows and
//    the K tail use an offset past the buffer's range, which reads as zero.
//  * loads run 4 steps ahead: at the top of step k every wave waits until its
//    loads of step k+1 landed (vmcnt), one barrier publishes them, and the
//    wave issues step k+4 into the stage that held step k (already copied to
//    registers).  A load therefore has three steps of MFMA time to arrive.
//  * LDS -> registers runs one step ahead: the MFMAs of step k consume
//    fragments read during step k-1, while the fragments of step k+1 are read
//    between them.
//  * MFMA: v_mfma_f32_32x32x64_f8f6f4 (fp8) or 2 x v_mfma_f32_32x32x16_bf16.
//    The B tile feeds the MFMA A operand, so lane l, accumulator register j
//    holds C[m0 + l % 32][n0 + 8 * (j / 4) + 4 * (l / 32) + j % 4].
#pragma once

#include <type_traits>

#include "gemm_tile.h"

namespace txg {

constexpr uint32_t kOob = 0x80000000u;  // buffer offset beyond any num_records used here

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  // word 3 = 0x00020000: raw (untyped) buffer, 32-bit data format, on gfx9 parts
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

typedef __attribute__((address_space(3))) void lds_void;

namespace fast {
constexpr int kStep = 64;                  // K bytes per step
constexpr int kStages = 4;
constexpr int kRows = 512;                 // 256 A rows + 256 B rows
constexpr int kStageBytes = kRows * kStep;  // 32 KiB
constexpr int kAhead = kStages;            // steps in flight

__device__ __forceinline__ int off(int row, int chunk) {
  return row * kStep + ((chunk ^ ((row >> 2) & 3)) << 4);
}
}  // namespace fast

// One 32x32 block product over a 64-byte K step.  Operands are i32x8 tuples
// (32 bytes per lane: chunks 2g and 2g+1 of the lane's row).
template <class C>
__device__ __forceinline__ void mfma32(txd::f32x16 &acc, const i32x8 &mb, const i32x8 &ma) {
  if constexpr (!C::FP8) {
    const txd::bf16x8 b0 = __builtin_bit_cast(txd::bf16x8, __builtin_shufflevector(mb, mb, 0, 1, 2, 3));
    const txd::bf16x8 b1 = __builtin_bit_cast(txd::bf16x8, __builtin_shufflevector(mb, mb, 4, 5, 6, 7));
    const txd::bf16x8 a0 = __builtin_bit_cast(txd::bf16x8, __builtin_shufflevector(ma, ma, 0, 1, 2, 3));
    const txd::bf16x8 a1 = __builtin_bit_cast(txd::bf16x8, __builtin_shufflevector(ma, ma, 4, 5, 6, 7));
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b0, a0, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b1, a1, acc, 0, 0, 0);
  } else {
    acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(mb, ma, acc, F8Code<C::EL_B_>::v,
                                                          F8Code<C::EL_A_>::v, 0, 0, 0, 0);
  }
}

// Two 16-byte LDS reads forming one operand tuple.
__device__ __forceinline__ i32x8 lds_pair(const uint8_t *p0, const uint8_t *p1) {
  const txd::i32x4 lo = *reinterpret_cast<const txd::i32x4 *>(p0);
  const txd::i32x4 hi = *reinterpret_cast<const txd::i32x4 *>(p1);
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Wait until at most N vector-memory loads of this wave are outstanding and
// all its LDS operations are done, then meet the workgroup at a barrier.
// (A plain __syncthreads() would also wait for every outstanding load, which
// would drain the prefetch pipeline.)  The inline asm is a compiler memory
// barrier so no LDS access moves across it.
template <int N>
__device__ __forceinline__ void wait_and_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  // gfx9 s_waitcnt: vmcnt[3:0] | expcnt[6:4] (7 = no wait) | lgkmcnt[11:8] | vmcnt[5:4] at [15:14]
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (0 << 8) | ((N >> 4) << 14));
  asm volatile("s_barrier" ::: "memory");
}

template <class C, int WAVES>
__device__ __forceinline__ void gemm_fast_tile(const tx_gemm_args &a) {
  static_assert(WAVES == 4 || WAVES == 8, "4 or 8 wavefronts");
  using namespace fast;
  constexpr int WN = WAVES / 2;          // waves along N (2 along M)
  constexpr int TN = 256 / WN;           // wave tile: 128 x TN
  constexpr int FN = TN / 32;            // 32-column blocks per wave
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kStages * kStageBytes];

  int tm, tn;
  tile_coords(blockIdx.x, a.tiles_m, a.tiles_n, a.group_m, &tm, &tn);
  const int m0 = tm * 256, n0 = tn * 256;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  constexpr int BLK = 16 / WAVES;  // A (and B) 1 KiB blocks per wave per step
  static_assert(BLK * WAVES == 16, "16 blocks per operand per stage");
  constexpr int ES = C::FP8 ? 1 : 2;
  const uint32_t kb_end = uint32_t(a.K) * ES;
  const int ksteps = int((kb_end + kStep - 1) / kStep);
  const uint32_t lda_b = uint32_t(a.lda) * ES, ldb_b = uint32_t(a.ldb) * ES;
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(a.A, uint32_t(a.M - 1) * lda_b + kb_end);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(a.B, uint32_t(a.N - 1) * ldb_b + kb_end);

  // DMA assignment: wave w fills A blocks BLK*w .. BLK*w+BLK-1 and the same B
  // blocks (16 rows each); this lane's row in block j is 16 (BLK w + j) + lane / 4.
  const uint32_t kch = 16u * uint32_t((lane & 3) ^ (lane >> 4));
  uint32_t voa[BLK], vob[BLK];
#pragma unroll
  for (int j = 0; j < BLK; ++j) {
    const int row = 16 * (BLK * wave + j) + (lane >> 2);
    const int gm = m0 + row, gn = n0 + row;
    voa[j] = gm < a.M ? uint32_t(gm) * lda_b + kch : kOob;
    vob[j] = gn < a.N ? uint32_t(gn) * ldb_b + kch : kOob;
  }
  auto issue = [&](int ks) {
    const uint32_t so = uint32_t(ks) * kStep;
    const bool past = so + kch >= kb_end;  // K tail: this lane's chunk is past the row end
    uint8_t *As = lds + (ks % kStages) * kStageBytes;
    uint8_t *Bs = As + 256 * kStep;
#pragma unroll
    for (int j = 0; j < BLK; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void *)(As + (BLK * wave + j) * 1024), 16,
                                               past ? kOob : voa[j], so, 0, 0);
#pragma unroll
    for (int j = 0; j < BLK; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void *)(Bs + (BLK * wave + j) * 1024), 16,
                                               past ? kOob : vob[j], so, 0, 0);
  };

  // Fragment reads: lane l holds row l % 32 of a 32-row block, chunks 2g, 2g+1
  // (g = l / 32).  Blocks 32 rows apart share the swizzle ((row >> 2) & 3 does
  // not change by 32 rows), so they are one base plus 2 KiB steps.
  const int frow = lane & 31, fg = lane >> 5;
  const int a0 = off(wm * 128 + frow, 2 * fg), a1 = off(wm * 128 + frow, 2 * fg + 1);
  const int b0 = 256 * kStep + off(wn * TN + frow, 2 * fg);
  const int b1 = 256 * kStep + off(wn * TN + frow, 2 * fg + 1);
  i32x8 fa[2][4], fb[2][FN];  // [register buffer][32-row block]
  auto read = [&](int ks, auto buf_tag) {
    constexpr int buf = decltype(buf_tag)::value;
    const uint8_t *S = lds + (ks % kStages) * kStageBytes;
#pragma unroll
    for (int f = 0; f < 4; ++f) fa[buf][f] = lds_pair(S + a0 + 2048 * f, S + a1 + 2048 * f);
#pragma unroll
    for (int f = 0; f < FN; ++f) fb[buf][f] = lds_pair(S + b0 + 2048 * f, S + b1 + 2048 * f);
  };

  txd::f32x16 acc[FN][4];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // Prologue: steps 0..3 in flight (steps past the end read as zeros), step 0
  // landed and in registers.
#pragma unroll
  for (int s = 0; s < kAhead; ++s) issue(s);
  wait_and_barrier<(kAhead - 1) * 2 * BLK>();
  read(0, std::integral_constant<int, 0>{});

  // One K step; CUR is the register buffer holding step ks (compile-time, so
  // the fragment arrays stay in registers).  Every step has the same shape:
  // loads past the last step are still issued and fill a free stage with
  // zeros, so the wait count is always "two steps may stay in flight".
  auto step = [&](int ks, auto cur_tag) {
    constexpr int CUR = decltype(cur_tag)::value;
    // this wave's step ks+1 landed, then everyone's did, and stage ks % 4 is
    // free (its contents are in registers)
    wait_and_barrier<(kAhead - 2) * 2 * BLK>();
    issue(ks + kAhead);
    read(ks + 1, std::integral_constant<int, CUR ^ 1>{});
#pragma unroll
    for (int fn = 0; fn < FN; ++fn)
#pragma unroll
      for (int fm = 0; fm < 4; ++fm) mfma32<C>(acc[fn][fm], fb[CUR][fn], fa[CUR][fm]);
  };
  int ks = 0;
  for (; ks + 1 < ksteps; ks += 2) {
    step(ks, std::integral_constant<int, 0>{});
    step(ks + 1, std::integral_constant<int, 1>{});
  }
  if (ks < ksteps) step(ks, std::integral_constant<int, 0>{});
  // Drain the trailing (zero-fill) loads before the workgroup's LDS is released.
  wait_and_barrier<0>();

  // Epilogue: lane owns, per (fm, fn, jj), C[m][n .. n+3] with
  // m = m0 + wm*128 + fm*32 + l%32, n = n0 + wn*128 + fn*32 + 8*jj + 4*(l/32).
  uint16_t *Cb = reinterpret_cast<uint16_t *>(a.C);
  const bool cvec = ((reinterpret_cast<uintptr_t>(a.C) & 7) == 0) && ((a.ldc & 3) == 0);
#pragma unroll
  for (int fm = 0; fm < 4; ++fm) {
    const int m = m0 + wm * 128 + fm * 32 + frow;
    if (m >= a.M) continue;
    float sa = 1.0f;
    if constexpr (C::FP8) sa = a.scale_a[m];
#pragma unroll
    for (int fn = 0; fn < FN; ++fn)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int n = n0 + wn * TN + fn * 32 + 8 * jj + 4 * fg;
        float v[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) v[t] = acc[fn][fm][4 * jj + t];
        if constexpr (C::FP8) {
#pragma unroll
          for (int t = 0; t < 4; ++t) v[t] = v[t] * sa * (n + t < a.N ? a.scale_b[n + t] : 0.0f);
        }
        uint16_t *dst = Cb + int64_t(m) * a.ldc + n;
        if (cvec && n + 3 < a.N) {
          txd::u32x2 p = {txd::pack_bf16x2(v[0], v[1]), txd::pack_bf16x2(v[2], v[3])};
          *reinterpret_cast<txd::u32x2 *>(dst) = p;
        } else {
#pragma unroll
          for (int t = 0; t < 4; ++t)
            if (n + t < a.N) dst[t] = uint16_t(txd::f32_to_bf16_bits(v[t]));
        }
      }
  }
}

}  // namespace txg
