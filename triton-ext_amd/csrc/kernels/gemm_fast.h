// Fast-path GEMM body for K-contiguous operands (16-byte aligned rows and
// K * element size a multiple of 16 bytes; 16-bit operands in 256 x 128
// tiles also with 4-byte aligned rows and any K of at least two steps, see
// fast::KTail): 256 x 256 tile,
// 8 wavefronts (two per SIMD), each owning a 128 x 64 block of C (64 x 64 in
// the 256 x 128 variant).
//
// Pipeline (per 128-byte K step, i.e. 64 bf16 or 128 fp8 of K):
//  * LDS is a ring of 5 slots of 32 KiB (all of gfx950's 160 KiB); a slot
//    holds one operand of one step, 256 rows x 128 bytes.  Operand-step u
//    (A of step k is u = 2k, B is u = 2k + 1) lives in slot u % 5.
//    Rows are 8 chunks of 16 bytes stored at chunk ^ ((row >> 1) & 7): a
//    ds_read_b128 is served 16 lanes at a time over 256 bytes of banks, the
//    fragment reads have 16 lanes read one logical chunk of 16 consecutive
//    rows, and this swizzle puts those 16 reads in 16 different 16-byte bank
//    groups (row parity picks the half of the bank window, (row >> 1) & 7 the
//    chunk within it).
//  * global -> LDS bypasses registers: gfx950's `buffer_load_dwordx4 ... lds`
//    writes each lane's 16 bytes at M0 + 16 * lane, so one instruction fills a
//    1 KiB block = 8 rows of 128 bytes; lane i lands in row i / 8, physical
//    chunk i % 8, and therefore fetches logical chunk (i % 8) ^ ((row >> 1) & 7).
//    The 8 lanes of a row fetch one whole 128-byte line.  Out-of-range rows
//    and the K tail use an offset past the buffer's range, which reads as zero.
//  * A step is consumed in two K halves of 64 bytes (one 32x32x64 fp8 MFMA,
//    or two 32x32x16 bf16 MFMAs, per 32 x 32 block).  Fragments run one half
//    ahead in registers: while the MFMAs of half 0 of step k run, half 1 is
//    read.  Then every wave waits for its loads of step k+1, and one barrier
//    publishes them to the workgroup and frees the two slots of step k (both
//    halves are in registers).  While the MFMAs of half 1 run, the wave reads
//    half 0 of step k+1 and loads B of step k+2 and A of step k+3 into the
//    freed slots ((2k + 5) % 5 and (2k + 6) % 5 are the slots of A and B of
//    step k).  B loads have one step of MFMA time to arrive, A loads two.
//  * The instruction order inside each half is fixed in the source and
//    pinned with scheduling barriers: after each MFMA, a share of the LDS
//    reads (all of them within the first half of the MFMAs, in the order the
//    next half consumes them) and, in the second half, one of the loads.
//  * MFMA roles: the B tile feeds the MFMA A operand, so lane l, accumulator
//    register j holds C[m0 + l % 32][n0 + 8 * (j / 4) + 4 * (l / 32) + j % 4].
//  * The 32x32x64 fp8 MFMA takes a lane's 32 operand bytes as two 16-byte
//    pieces: bytes 0-15 are K 16g .. 16g+15 of the 64, bytes 16-31 are
//    K 32+16g .. 32+16g+15 (g = lane / 32).  Lane g therefore reads chunks g
//    and g + 2 of a 64-byte K half, so that K block b (bytes 32b .. 32b+31 of
//    the half) is piece b of both lane halves: the block an MX scale of lane
//    32b + row covers.  (bf16 reads chunks 2g and 2g + 1; the order of K
//    inside a product does not change an unscaled sum.)
//  * MX (block-scaled) variant: one e8m0 scale per 32 K elements of each row
//    of A and B.  A 128-byte step holds blocks 4s .. 4s+3 of a row, one
//    dword; the host repacks the scales step-major (dword [s][row]), so the
//    32 rows of a fragment are one 128-byte line per step.  Each lane loads
//    the dword of its row for each of its fragments and, when the step
//    begins, shifts it right by 8g so that byte 2h is the block of K half h
//    it multiplies (op_sel picks the byte).  The loads of step k+1 are issued
//    at the start of the second half of step k, ahead of that half's LDS-DMA
//    loads: loads complete in issue order, so a scale load issued behind the
//    DMA loads would make its first use wait for operand loads that the
//    pipeline otherwise gives two steps.  In the 256 x 256 tile only 4
//    wavefronts (one per SIMD) leave the registers for this; the 256 x 128
//    tile keeps 8.
#pragma once

#include <type_traits>
#include <utility>

#include "gemm_tile.h"

namespace txg {

constexpr uint32_t kOob = 0x80000000u;  // buffer offset beyond any num_records used here

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  // word 3 = 0x00020000: raw (untyped) buffer, 32-bit data format, on gfx9 parts
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) uint8_t lds_u8;

// Compile-time loop: f(integral_constant<int, 0>) ... f(integral_constant<int, N-1>).
template <class F, int... Is>
__device__ __forceinline__ void static_for_impl(F &&f, std::integer_sequence<int, Is...>) {
  (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F &&f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

namespace fast {
constexpr int kStep = 128;                   // K bytes per step
constexpr int kSlotBytes = 256 * kStep;      // one operand of one step: 32 KiB
constexpr int kSlots = 5;
constexpr int kWaves = 8;

__device__ __forceinline__ int off(int row, int chunk) {
  return row * kStep + ((chunk ^ ((row >> 1) & 7)) << 4);
}

// n items spread evenly over the first `over` MFMAs of a half: items
// [spread_lo, spread_hi) follow MFMA i.
__host__ __device__ constexpr int spread_lo(int i, int n, int over) {
  return i >= over ? n : (i * n) / over;
}
__host__ __device__ constexpr int spread_hi(int i, int n, int over) {
  return i >= over ? n : ((i + 1) * n) / over;
}

// Ragged K of 16-bit operands (rows 4-byte aligned, K bytes kb_end not a
// whole number of 16-byte chunks, r = kb_end mod 16 > 0, at least two K
// steps): the last chunk of each row, logical chunk cp of the last K step,
// is fetched as the row's last 16 bytes [kb_end - 16, kb_end), so nothing
// past the row is read; its first 16 - r bytes repeat the chunk before and
// are cleared in both operands' fragments before that step's MFMAs (the
// duplicated K positions then add 0 x 0, whatever the values).  The loads of
// the last step take scalar offset - 16 and lane offset + 16 (+ r for the
// partial chunk), which keeps every lane offset non-negative; chunks past
// the row use an out-of-range offset and read as zero.
struct KTail {
  uint32_t keep[4];  // bytes of the partial chunk kept, per dword
  int cp;            // the partial chunk of the last step; 8: none
};
__device__ __forceinline__ KTail make_ktail(uint32_t kb_end) {
  KTail t;
  const int clear = (kb_end & 15u) ? 16 - int(kb_end & 15u) : 0;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const int nz = min(max(clear - 4 * d, 0), 4);
    t.keep[d] = nz >= 4 ? 0u : (0xFFFFFFFFu << (8 * nz));
  }
  t.cp = (kb_end & 15u) ? int((kb_end & 127u) >> 4) : 8;
  return t;
}
// Clear the repeated bytes in the fragments of K half h (16-bit operands:
// lane l holds chunks 4h + 2g and 4h + 2g + 1 of the step, g = l / 32).
template <int NF>
__device__ __forceinline__ void ktail_clear(txd::i32x4 (&fr)[NF][2], int h, int g, const KTail &t) {
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const bool hit = 4 * h + 2 * g + e == t.cp;
    int m[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) m[d] = hit ? int(t.keep[d]) : -1;
#pragma unroll
    for (int f = 0; f < NF; ++f)
#pragma unroll
      for (int d = 0; d < 4; ++d) fr[f][e][d] &= m[d];
  }
}
}  // namespace fast

// One 32x32 block product over a 64-byte K half.  Operands are i32x8 tuples
// (32 bytes per lane: chunks 2g and 2g+1 of the half, g = lane / 32).
template <class C>
__device__ __forceinline__ void mfma32(txd::f32x16 &acc, const i32x8 &mb, const i32x8 &ma) {
  if constexpr (C::F16) {
    const txd::f16x8 b0 = __builtin_bit_cast(txd::f16x8, __builtin_shufflevector(mb, mb, 0, 1, 2, 3));
    const txd::f16x8 b1 = __builtin_bit_cast(txd::f16x8, __builtin_shufflevector(mb, mb, 4, 5, 6, 7));
    const txd::f16x8 a0 = __builtin_bit_cast(txd::f16x8, __builtin_shufflevector(ma, ma, 0, 1, 2, 3));
    const txd::f16x8 a1 = __builtin_bit_cast(txd::f16x8, __builtin_shufflevector(ma, ma, 4, 5, 6, 7));
    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(b0, a0, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(b1, a1, acc, 0, 0, 0);
  } else if constexpr (!C::FP8) {
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

// The same product with MX block scales: byte OPSEL of scale_b (scale_a)
// scales the 32 K values of this lane's row of the B (A) block.
template <class C, int OPSEL>
__device__ __forceinline__ void mfma32_mx(txd::f32x16 &acc, const i32x8 &mb, const i32x8 &ma,
                                          uint32_t scale_b, uint32_t scale_a) {
  acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(mb, ma, acc, F8Code<C::EL_B_>::v, F8Code<C::EL_A_>::v,
                                                        OPSEL, int(scale_b), OPSEL, int(scale_a));
}

// fp4 (e2m1) operands: one 16-byte piece per lane is 32 K values, so a
// 64-byte K half is two MFMAs of K = 64 (the instruction reads the first 4
// registers of each operand).
template <class C, int OPSEL>
__device__ __forceinline__ void mfma32_mx_fp4(txd::f32x16 &acc, const txd::i32x4 &pb, const txd::i32x4 &pa,
                                              uint32_t scale_b, uint32_t scale_a) {
  const i32x8 mb = __builtin_shufflevector(pb, pb, 0, 1, 2, 3, 0, 1, 2, 3);
  const i32x8 ma = __builtin_shufflevector(pa, pa, 0, 1, 2, 3, 0, 1, 2, 3);
  acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(mb, ma, acc, 4, 4, OPSEL, int(scale_b), OPSEL,
                                                        int(scale_a));
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


// The tile (tm, tn) of C (256 x BN elements at row 256 tm, column BN tn),
// split `split` of a.splits along K.  TRANS (bf16 out, no split): the tile
// is stored transposed, element (i, j) at C[j * ldc + i].
template <class C, int BN, int NW = fast::kWaves, bool MX = false, int OUT = OUT_BF16, bool EPI = false,
          bool TRANS = false>
__device__ __forceinline__ void gemm_fast_tile_at(const tx_gemm_args &a, int tm, int tn, int split) {
  using namespace fast;
  static_assert(BN == 256 || BN == 128, "tile 256 x 256 or 256 x 128");
  static_assert(NW == 8 || NW == 4, "8 or 4 wavefronts");
  static_assert(!MX || (C::FP8 && (NW == 4 || BN == 128)), "MX scales: fp8 operands; 256x256: 4 wavefronts");
  constexpr bool FP4 = C::EL_A_ == EL_E2M1;
  static_assert(!FP4 || (MX && C::EL_B_ == EL_E2M1), "fp4: MX-scaled, both operands");
  constexpr int SD = FP4 ? 2 : 1;  // MX scale dwords per row and K step (4 blocks each)
  static_assert(OUT == OUT_BF16 || MX || (OUT == OUT_F16 && !C::FP8),
                "fp16 output: MX or 16-bit operands; fp32 output: MX only");
  static_assert(!EPI || (C::FP8 && !MX && OUT == OUT_BF16), "fused epilogue: row/column-scaled fp8");
  static_assert(!TRANS || (!EPI && OUT == OUT_BF16), "transposed store: plain bf16 output");
  // Wave grid WM x WN.  256x128 tiles with 8 waves take 4 x 2 (64 x 64 per
  // wave): LDS reads per step are then (64 + 64) x 8 rows instead of
  // (128 + 32) x 8, which matters because narrow tiles are LDS-bound.
  constexpr int WM = (BN == 128 && NW == 8) ? 4 : 2;
  constexpr int WN = NW / WM;
  constexpr int TM = 256 / WM;       // wave tile: TM x TN
  constexpr int TN = BN / WN;
  constexpr int FM = TM / 32;        // 32-row blocks per wave
  constexpr int FN = TN / 32;        // 32-column blocks per wave
  constexpr int NM = FM * FN;        // mfma32 calls per K half
  constexpr int NF = FM + FN;        // fragments per K half: A 0..FM-1, B FM..
  constexpr int NR = 2 * NF;         // ds_read_b128 per K half
  constexpr int BLKA = 32 / NW;      // 1 KiB blocks of A per wave per step
  constexpr int BLKB = BN / 8 / NW;  // ... of B
  constexpr int ND = BLKA + BLKB;    // loads per wave per step
  static_assert(BLKA % 2 == 0 && BLKB % 2 == 0, "a wave's first block must have an even index");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kSlots * kSlotBytes];

  const int splits = a.splits > 1 ? a.splits : 1;
  const int m0 = tm * 256, n0 = tn * BN;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: keeps LDS addresses scalar
  const int wm = wave % WM, wn = wave / WM;
  constexpr int ES = C::FP8 ? 1 : 2;
  const uint32_t kb_end = uint32_t(a.K) * ES;
  const int ksteps_all = int((kb_end + kStep - 1) / kStep);
  const int kfirst = splits > 1 ? split * a.ksteps_split : 0;  // first K step of this split
  const int ksteps = splits > 1 ? min(a.ksteps_split, ksteps_all - kfirst) : ksteps_all;
  const uint32_t kbase = uint32_t(kfirst) * kStep;
  const uint32_t lda_b = uint32_t(a.lda) * ES, ldb_b = uint32_t(a.ldb) * ES;
  // (K = 0: empty ranges, so the prologue's loads read nothing at all)
  const __amdgpu_buffer_rsrc_t rsrc[2] = {make_rsrc(a.A, kb_end ? uint32_t(a.M - 1) * lda_b + kb_end : 0u),
                                          make_rsrc(a.B, kb_end ? uint32_t(a.N - 1) * ldb_b + kb_end : 0u)};
  // Loads of steps past the last one (the pipeline's look-ahead at the end of
  // the K loop) go through an empty range: every lane is out of range
  // whatever its offsets, so they read zeros and touch no memory.
  const __amdgpu_buffer_rsrc_t rnull[2] = {make_rsrc(a.A, 0u), make_rsrc(a.B, 0u)};

  // DMA assignment: wave w fills blocks BLKA*w .. of A and BLKB*w .. of B.
  // Lane i of block q covers row 8q + i/8 and logical chunk
  // (i % 8) ^ ((row >> 1) & 7) = (i % 8) ^ ((4q + i/16) & 7), which depends on
  // the parity of q only (a wave's first block index is even, so it is the
  // parity of j).
  const uint32_t kch[2] = {16u * uint32_t((lane & 7) ^ ((lane >> 4) & 7)),
                           16u * uint32_t((lane & 7) ^ ((4 + (lane >> 4)) & 7))};
  uint32_t vo[2][BLKA > BLKB ? BLKA : BLKB];
#pragma unroll
  for (int j = 0; j < BLKA; ++j) {
    const int row = 8 * (BLKA * wave + j) + (lane >> 3);
    const int gm = m0 + row;
    vo[0][j] = gm < a.M ? uint32_t(gm) * lda_b + kch[j & 1] : kOob;
  }
#pragma unroll
  for (int j = 0; j < BLKB; ++j) {
    const int row = 8 * (BLKB * wave + j) + (lane >> 3);
    const int gn = n0 + row;
    vo[1][j] = gn < a.N ? uint32_t(gn) * ldb_b + kch[j & 1] : kOob;
  }
  // Source of operand op for (split-local) step ks: its buffer range and K
  // offset.  Steps past the split's end are loaded but never multiplied;
  // those past the operand's last step read through the empty range (scalar
  // selects, once per step and operand).
  struct Src {
    __amdgpu_buffer_rsrc_t rs;
    uint32_t so;
  };
  auto src = [&](int ks, int op) {
    const bool live = kfirst + ks < ksteps_all;
    return Src{live ? rsrc[op] : rnull[op], live ? kbase + uint32_t(ks) * kStep : 0u};
  };
  // Load block j of operand op from `sr` into the LDS operand buffer at byte
  // `base`.  With TAIL (K * element size not a multiple of the step), a lane
  // whose chunk lies past the row end reads zeros; otherwise no chunk ever
  // does, and the load takes its per-lane offset as it is (no vector
  // instructions per load).
  // A ragged K (fast::KTail) is served by the 256 x 128 tile with 16-bit
  // operands (the 256 x 256 one has no registers to spare for it):
  // the last step's offsets (klast = 0 with a single step, which the host
  // never sends with a ragged K).
  constexpr bool RAGGED = !C::FP8 && BN == 128;
  const KTail kt = make_ktail(kb_end);
  const uint32_t kb16 = kb_end & ~15u, kr = kb_end & 15u;
  const uint32_t kbz = kr ? kb16 + 16u : kb_end;  // chunks from here on read as zero
  const uint32_t klast = uint32_t(ksteps_all - 1) * kStep;
  auto load_op = [&](const Src &sr, int base, auto op_tag, auto j_tag, auto tail_tag) {
    constexpr int op = decltype(op_tag)::value, j = decltype(j_tag)::value;
    constexpr int blk = op == 0 ? BLKA : BLKB;
    uint32_t voff = vo[op][j], so = sr.so;
    if constexpr (decltype(tail_tag)::value) {
      const uint32_t cs = sr.so + kch[j & 1];  // the lane's chunk, in bytes from the row start
      if constexpr (RAGGED) {
        if (klast != 0u && sr.so == klast) {
          // (the empty asm keeps the compiler from holding adjusted copies
          // of every lane offset in registers across the K loop)
          asm volatile("" : "+v"(voff));
          so -= 16u;
          voff = cs >= kbz ? kOob : voff + (cs == kb16 ? kr : 16u);
        } else if (cs >= kb_end) {
          voff = kOob;
        }
      } else {
        if (cs >= kb_end) voff = kOob;
      }
    }
    uint8_t *dst = lds + base + (blk * wave + j) * 1024;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(sr.rs, (lds_void *)dst, 16, voff, so, 0, 0);
  };
  using OpA = std::integral_constant<int, 0>;
  using OpB = std::integral_constant<int, 1>;
  // Load d of the second half of a step: B (d < BLKB) from srb into the
  // buffer at byte dst_b, then A from sra into dst_a.
  auto load = [&](const Src &srb, const Src &sra, int dst_b, int dst_a, auto d_tag, auto tail_tag) {
    constexpr int d = decltype(d_tag)::value;
    if constexpr (d < BLKB) load_op(srb, dst_b, OpB{}, std::integral_constant<int, d>{}, tail_tag);
    else load_op(sra, dst_a, OpA{}, std::integral_constant<int, d - BLKB>{}, tail_tag);
  };

  // Fragment reads: lane l holds row l % 32 of a 32-row block and, for K half
  // h, chunks 4h + g and 4h + g + 2 (fp8) or 4h + 2g and 4h + 2g + 1 (bf16),
  // g = l / 32.  Blocks 32 rows apart share the swizzle ((row >> 1) & 7 does
  // not change by 32 rows), so they are one base plus 4 KiB steps.
  const int frow = lane & 31, fg = lane >> 5;
  int ro[2][2][2];  // [operand][K half][piece]
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int chunk = 4 * h + (C::FP8 ? fg + 2 * e : 2 * fg + e);
      ro[0][h][e] = off(wm * TM + frow, chunk);
      ro[1][h][e] = off(wn * TN + frow, chunk);
    }

  // MX scales, step-major: the SD dwords of row r for K step s (blocks
  // 4 SD s .. +4 SD - 1; fp8: 4 blocks of 32 bytes, fp4: 8 blocks of 16) at
  // byte s * ld_mx + 4 SD r; rows are padded to whole tiles (with finite
  // codes), and the load one step past the end reads past the buffer's
  // range (zeros, never used).  scn: the raw dwords of the next step, in
  // flight; scc: this step's, shifted by 8g.
  constexpr int NS = MX ? NF * SD : 1;
  uint32_t scc[NS], scn[NS];
  __amdgpu_buffer_rsrc_t srs[2];
  uint32_t svb[2] = {0u, 0u};
  if constexpr (MX) {
    srs[0] = make_rsrc(a.mx_a, uint32_t(ksteps_all) * uint32_t(a.ld_mxa));
    srs[1] = make_rsrc(a.mx_b, uint32_t(ksteps_all) * uint32_t(a.ld_mxb));
    svb[0] = 4u * SD * uint32_t(m0 + wm * TM + frow);
    svb[1] = 4u * SD * uint32_t(n0 + wn * TN + frow);
  }
  auto load_scales = [&](int ks, uint32_t(&dst)[NS]) {
    if constexpr (MX) {
      const int s = kfirst + ks;
#pragma unroll
      for (int f = 0; f < NF; ++f) {
        const int op = f < FM ? 0 : 1;
        const int fb = f < FM ? f : f - FM;
        const int soff = s * int(op == 0 ? a.ld_mxa : a.ld_mxb) + 128 * SD * fb;
        if constexpr (SD == 1) {
          dst[f] = uint32_t(__builtin_amdgcn_raw_buffer_load_b32(srs[op], int(svb[op]), soff, 0));
        } else {
          const txd::u32x2 d = __builtin_bit_cast(
              txd::u32x2, __builtin_amdgcn_raw_buffer_load_b64(srs[op], int(svb[op]), soff, 0));
          dst[2 * f] = d.x;
          dst[2 * f + 1] = d.y;
        }
      }
    }
  };
  txd::i32x4 fr[2][NF][2];  // [K half][fragment][16-byte piece]
  // Read r of a K half: fragments in the order the MFMAs consume them
  // (A0, B0, A1 .. A(FM-1), B1 .., two 16-byte pieces each.
  // (base_a, base_b: the step's A and B buffers in LDS, in bytes)
  auto read = [&](int base_a, int base_b, auto h_tag, auto r_tag) {
    constexpr int h = decltype(h_tag)::value, r = decltype(r_tag)::value, e = r % 2, o = r / 2;
    constexpr int f = o == 0 ? 0 : o == 1 ? FM : o <= FM ? o - 1 : o;
    const uint8_t *S = lds + (f < FM ? base_a : base_b);
    const int byte = f < FM ? ro[0][h][e] + 4096 * f : ro[1][h][e] + 4096 * (f - FM);
    fr[h][f][e] = *reinterpret_cast<const txd::i32x4 *>(S + byte);
  };

  txd::f32x16 acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  // MFMA i of a K half: B block i / FM against A block i % FM.
  auto mma = [&](auto h_tag, auto i_tag) {
    constexpr int h = decltype(h_tag)::value, i = decltype(i_tag)::value, fn = i / FM, fm = i % FM;
    const i32x8 va = __builtin_shufflevector(fr[h][fm][0], fr[h][fm][1], 0, 1, 2, 3, 4, 5, 6, 7);
    const i32x8 vb = __builtin_shufflevector(fr[h][FM + fn][0], fr[h][FM + fn][1], 0, 1, 2, 3, 4, 5, 6, 7);
    if constexpr (FP4) {
      // K half h holds blocks 4h .. 4h + 3 (dword h of the step's two):
      // piece e is blocks 4h + 2e + g, byte 2e after the 8g shift
      mfma32_mx_fp4<C, 0>(acc[fn][fm], fr[h][FM + fn][0], fr[h][fm][0], scc[2 * (FM + fn) + h], scc[2 * fm + h]);
      mfma32_mx_fp4<C, 2>(acc[fn][fm], fr[h][FM + fn][1], fr[h][fm][1], scc[2 * (FM + fn) + h], scc[2 * fm + h]);
    } else if constexpr (MX) {
      mfma32_mx<C, 2 * h>(acc[fn][fm], vb, va, scc[FM + fn], scc[fm]);
    } else {
      mfma32<C>(acc[fn][fm], vb, va);
    }
  };
  using H0 = std::integral_constant<int, 0>;
  using H1 = std::integral_constant<int, 1>;
  constexpr int RW = NM / 2;  // reads follow the first RW MFMAs of a half

  // The prologue and the K loop, with or without the K-tail zero fill.
  // Ring of LDS operand buffers.  Standard: 5 slots of one operand of one
  // step (32 KiB), A of step k in slot 2k mod 5 and B in 2k + 1 mod 5; during
  // the second half of step k, B of step k+2 and A of step k+3 go into the
  // two slots step k frees, so B has one step to arrive and A two.  HS (256 x
  // 128 tiles without MX scales): 3 stages of one whole step (A 32 KiB, then
  // B 16 KiB), step k in stage k mod 3, and the second half of step k loads
  // both operands of step k+3 into its stage: two steps for each, which the
  // tiles that stream B from HBM (products with few rows) need.
  constexpr bool HS = BN == 128 && !MX;
  constexpr int kStage = (256 + BN) * kStep;  // HS stage: A, then B
  static_assert(!HS || 3 * kStage <= kSlots * kSlotBytes, "HS stages fit in LDS");
  auto pipeline = [&](auto tail) {
    if constexpr (HS) {
      // Prologue: steps 0, 1 and 2 in flight, step 0 landed, half 0 of step
      // 0 in registers.
      static_for<3>([&](auto s_tag) {
        constexpr int st = decltype(s_tag)::value;
        const Src as = src(st, 0), bs = src(st, 1);
        static_for<BLKA>([&](auto j) { load_op(as, st * kStage, OpA{}, j, tail); });
        static_for<BLKB>([&](auto j) { load_op(bs, st * kStage + 256 * kStep, OpB{}, j, tail); });
      });
      wait_and_barrier<2 * ND>();
      static_for<NR>([&](auto r) { read(0, 256 * kStep, H0{}, r); });
      int st = 0;  // stage of step ks (uniform)
      for (int ks = 0; ks < ksteps; ++ks) {
        const int nt = st == 2 ? 0 : st + 1;
        const int ca = st * kStage, cb = ca + 256 * kStep, xa = nt * kStage, xb = xa + 256 * kStep;
        const bool clear = RAGGED && decltype(tail)::value && kt.cp < 8 && kfirst + ks == ksteps_all - 1;
        if (clear) ktail_clear<NF>(fr[0], 0, fg, kt);
        static_for<NM>([&](auto I) {
          constexpr int i = decltype(I)::value;
          mma(H0{}, I);
          __builtin_amdgcn_sched_barrier(0);
          constexpr int r0 = spread_lo(i, NR, RW), r1 = spread_hi(i, NR, RW);
          static_for<r1 - r0>([&](auto R) {
            read(ca, cb, H1{}, std::integral_constant<int, r0 + decltype(R)::value>{});
          });
          __builtin_amdgcn_sched_barrier(0);
        });
        // step ks+1 landed for every wave (step ks+2 may still be in flight);
        // the stage of step ks is free
        wait_and_barrier<ND>();
        __builtin_amdgcn_sched_barrier(0);
        if (clear) ktail_clear<NF>(fr[1], 1, fg, kt);
        const Src srb = src(ks + 3, 1), sra = src(ks + 3, 0);
        static_for<NM>([&](auto I) {
          constexpr int i = decltype(I)::value;
          mma(H1{}, I);
          __builtin_amdgcn_sched_barrier(0);
          constexpr int d0 = spread_lo(i, ND, NM), d1 = spread_hi(i, ND, NM);
          static_for<d1 - d0>([&](auto D) {
            load(srb, sra, cb, ca, std::integral_constant<int, d0 + decltype(D)::value>{}, tail);
          });
          constexpr int r0 = spread_lo(i, NR, RW), r1 = spread_hi(i, NR, RW);
          static_for<r1 - r0>([&](auto R) {
            read(xa, xb, H0{}, std::integral_constant<int, r0 + decltype(R)::value>{});
          });
          __builtin_amdgcn_sched_barrier(0);
        });
        st = nt;
      }
      return;
    }
    // Prologue: A0 B0 A1 B1 A2 in flight (steps past the end read as zeros),
    // step 0 landed, half 0 of step 0 in registers.  The MX scales of step 0
    // go first, so the same wait covers them.
    load_scales(0, scn);
    {
      const Src a0 = src(0, 0), b0 = src(0, 1), a1 = src(1, 0), b1 = src(1, 1), a2 = src(2, 0);
      static_for<BLKA>([&](auto j) { load_op(a0, 0 * kSlotBytes, OpA{}, j, tail); });
      static_for<BLKB>([&](auto j) { load_op(b0, 1 * kSlotBytes, OpB{}, j, tail); });
      static_for<BLKA>([&](auto j) { load_op(a1, 2 * kSlotBytes, OpA{}, j, tail); });
      static_for<BLKB>([&](auto j) { load_op(b1, 3 * kSlotBytes, OpB{}, j, tail); });
      static_for<BLKA>([&](auto j) { load_op(a2, 4 * kSlotBytes, OpA{}, j, tail); });
    }
    wait_and_barrier<2 * BLKA + BLKB>();
    static_for<NR>([&](auto r) { read(0, kSlotBytes, H0{}, r); });

    int sa = 0, sb = 1;  // slots of A and B of step ks (uniform)
    for (int ks = 0; ks < ksteps; ++ks) {
      const int na = sa >= 3 ? sa - 3 : sa + 2, nb = sb >= 3 ? sb - 3 : sb + 2;  // step ks+1
      const bool clear = RAGGED && decltype(tail)::value && kt.cp < 8 && kfirst + ks == ksteps_all - 1;
      if (clear) ktail_clear<NF>(fr[0], 0, fg, kt);
      if constexpr (MX) {
        // this step's scales (loaded during the previous half) into place
#pragma unroll
        for (int f = 0; f < NS; ++f) scc[f] = scn[f] >> (8 * fg);
      }
      static_for<NM>([&](auto I) {
        constexpr int i = decltype(I)::value;
        mma(H0{}, I);
        __builtin_amdgcn_sched_barrier(0);
        constexpr int r0 = spread_lo(i, NR, RW), r1 = spread_hi(i, NR, RW);
        static_for<r1 - r0>([&](auto R) {
          read(sa * kSlotBytes, sb * kSlotBytes, H1{}, std::integral_constant<int, r0 + decltype(R)::value>{});
        });
        __builtin_amdgcn_sched_barrier(0);
      });
      // A and B of step ks+1 landed for every wave (the BLKA loads of A of step
      // ks+2, issued last, may still be in flight); the slots of step ks are free.
      wait_and_barrier<BLKA>();
      __builtin_amdgcn_sched_barrier(0);
      if (clear) ktail_clear<NF>(fr[1], 1, fg, kt);
      load_scales(ks + 1, scn);  // MX: ahead of this half's DMA loads
      const Src srb = src(ks + 2, 1), sra = src(ks + 3, 0);
      static_for<NM>([&](auto I) {
        constexpr int i = decltype(I)::value;
        mma(H1{}, I);
        __builtin_amdgcn_sched_barrier(0);
        constexpr int d0 = spread_lo(i, ND, NM), d1 = spread_hi(i, ND, NM);
        static_for<d1 - d0>([&](auto D) {
          load(srb, sra, sa * kSlotBytes, sb * kSlotBytes, std::integral_constant<int, d0 + decltype(D)::value>{},
               tail);
        });
        constexpr int r0 = spread_lo(i, NR, RW), r1 = spread_hi(i, NR, RW);
        static_for<r1 - r0>([&](auto R) {
          read(na * kSlotBytes, nb * kSlotBytes, H0{}, std::integral_constant<int, r0 + decltype(R)::value>{});
        });
        __builtin_amdgcn_sched_barrier(0);
      });
      sa = na;
      sb = nb;
    }
  };
  if (kb_end % kStep == 0) pipeline(std::false_type{});
  else pipeline(std::true_type{});
  // Drain the trailing (zero-fill) loads before the workgroup's LDS is released.
  wait_and_barrier<0>();

  // Epilogue: lane owns, per (fm, fn, jj), C[m][n .. n+3] with
  // m = m0 + wm*TM + fm*32 + l%32, n = n0 + wn*TN + fn*32 + 8*jj + 4*(l/32).
  // With partial planes (K split, or one plane for a reduce that adds tt.dot's
  // accumulator operand), the unscaled fp32 sums go to the split's plane
  // (row-major M x N); a reduction kernel combines the planes.  An fp32
  // output (MX variant) is stored the same way, straight into C.
  const bool to_part = a.part != nullptr;
  if (!TRANS && (to_part || OUT == OUT_F32)) {
    float *P = to_part ? a.part + int64_t(split) * a.M * a.N : static_cast<float *>(a.C);
    const int64_t ldp = to_part ? a.N : a.ldc;
    const bool pvec = to_part ? (a.N & 3) == 0
                              : ((reinterpret_cast<uintptr_t>(a.C) & 15) == 0 && (a.ldc & 3) == 0);
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      const int m = m0 + wm * TM + fm * 32 + frow;
      if (m >= a.M) continue;
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int n = n0 + wn * TN + fn * 32 + 8 * jj + 4 * fg;
          float *dst = P + int64_t(m) * ldp + n;
          if (pvec && n + 3 < a.N) {
            *reinterpret_cast<txd::f32x4 *>(dst) =
                txd::f32x4{acc[fn][fm][4 * jj], acc[fn][fm][4 * jj + 1], acc[fn][fm][4 * jj + 2], acc[fn][fm][4 * jj + 3]};
          } else {
#pragma unroll
            for (int t = 0; t < 4; ++t)
              if (n + t < a.N) dst[t] = acc[fn][fm][4 * jj + t];
          }
        }
    }
    return;
  }
  // Fused epilogue (bias, activation, output type): two 32-row blocks of its
  // tile at a time, each wave stages its raw sums in LDS (rows padded by 16
  // bytes against bank conflicts), then walks a block four rows at a time
  // with lane l on row l / 16 and columns 4 (l % 16) .. +3 of the wave's 64:
  // the columns' scales and bias stay in registers, the row's scale comes
  // from lane r by a lane shuffle, and each lane stores its four outputs at
  // once (8-, 16- or 4-byte stores).  Staging is expanded at compile time
  // (the accumulators need constant indices); the walk is a plain loop with
  // one copy of the epilogue code per activation.
  if constexpr (EPI) {
    static_assert(TN == 64, "16 lanes x 4 columns per row of the wave tile");
    constexpr int SP = TN + 4;     // staged row pitch, floats
    constexpr int NB = FM < 2 ? FM : 2;  // blocks staged at once
    static_assert(FM % NB == 0, "whole groups of staged blocks");
    static_assert(NW * NB * 32 * SP * 4 <= kSlots * kSlotBytes, "epilogue staging fits in LDS");
    float *ws = reinterpret_cast<float *>(lds) + wave * NB * 32 * SP;
    const int c4 = 4 * (lane & 15), rq = lane >> 4;
    const int n = n0 + wn * TN + c4;
    float sb4[4], bias4[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      sb4[t] = n + t < a.N ? a.scale_b[n + t] : 0.0f;
      bias4[t] = (n + t < a.N && a.bias) ? a.bias[n + t] : 0.0f;
    }
    static_for<FM / NB>([&](auto g_tag) {
      constexpr int G = decltype(g_tag)::value;
      static_for<NB>([&](auto q_tag) {
        constexpr int q = decltype(q_tag)::value, fm = G * NB + q;
        static_for<FN>([&](auto fn_tag) {
          constexpr int fn = decltype(fn_tag)::value;
          static_for<4>([&](auto jj_tag) {
            constexpr int jj = decltype(jj_tag)::value;
            *reinterpret_cast<txd::f32x4 *>(ws + (q * 32 + frow) * SP + fn * 32 + 8 * jj + 4 * fg) =
                txd::f32x4{acc[fn][fm][4 * jj], acc[fn][fm][4 * jj + 1], acc[fn][fm][4 * jj + 2],
                           acc[fn][fm][4 * jj + 3]};
          });
        });
      });
      __syncthreads();
      with_act(a.act, [&](auto act_tag) {
        constexpr int ACT = decltype(act_tag)::value;
        for (int q = 0; q < NB; ++q) {
          const int mb = m0 + wm * TM + (G * NB + q) * 32;
          const float sa_lane = mb + frow < a.M ? a.scale_a[mb + frow] : 0.0f;  // lanes 0..31: rows
          const float *wq = ws + q * 32 * SP;
          txd::f32x4 v[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) v[i] = *reinterpret_cast<const txd::f32x4 *>(wq + (4 * i + rq) * SP + c4);
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const int r = 4 * i + rq;
            const float sa_r = __shfl(sa_lane, r);
            const int m = mb + r;
            const float x[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
            float y[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) y[t] = epi_act_t<ACT>(x[t] * sa_r * sb4[t] + bias4[t]);
            if (m < a.M) {
              if (n + 3 < a.N) {
                epi_store4(a, m, n, y);
              } else {
#pragma unroll
                for (int t = 0; t < 4; ++t)
                  if (n + t < a.N) epi_store1(a, m, n + t, y[t]);
              }
            }
          }
        }
      });
      __syncthreads();
    });
    return;
  }
  // Epilogue: scale (fp8 with row / column scales), round to bf16 (fp16)
  // and stage the whole tile in LDS (the ring is free after the drain
  // above), then write whole row segments of C with 16-byte stores.
  // Staged 16-byte chunk c of tile row r sits at chunk
  // c ^ (r % CH): the 32 rows of a fragment column write 32 (BN 256) or 16
  // twice-used (BN 128) different chunks, the minimum two passes for 512
  // bytes, and the CH lanes reading one row cover every chunk once.
  constexpr int CH = BN / 8;        // 16-byte chunks per staged row
  constexpr int ROWB = BN * 2;      // staged row bytes
  constexpr int RPI = 64 / CH;      // rows per store instruction
  static_assert(256 * ROWB <= kSlots * kSlotBytes, "staged tile fits in LDS");
  constexpr bool ROWCOL = C::FP8 && !MX;  // per-row / per-column fp32 scales
  float sav[FM], sbv[FN][4][4];
  if constexpr (ROWCOL) {
    // all scale loads in one batch ahead of their use
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      const int m = m0 + wm * TM + fm * 32 + frow;
      sav[fm] = m < a.M ? a.scale_a[m] : 0.0f;
    }
#pragma unroll
    for (int fn = 0; fn < FN; ++fn)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int n = n0 + wn * TN + fn * 32 + 8 * jj + 4 * fg + t;
          sbv[fn][jj][t] = n < a.N ? a.scale_b[n] : 0.0f;
        }
  }
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) {
    const int row = wm * TM + fm * 32 + frow;
#pragma unroll
    for (int fn = 0; fn < FN; ++fn)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        float v[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          v[t] = acc[fn][fm][4 * jj + t];
          if constexpr (ROWCOL) v[t] = v[t] * sav[fm] * sbv[fn][jj][t];
        }
        const int c = (wn * TN + fn * 32 + 8 * jj) / 8;
        *reinterpret_cast<txd::u32x2 *>(lds + row * ROWB + ((c ^ (row & (CH - 1))) << 4) + 8 * fg) =
            OUT == OUT_F16 ? txd::u32x2{txd::pack_f16x2(v[0], v[1]), txd::pack_f16x2(v[2], v[3])}
                           : txd::u32x2{txd::pack_bf16x2(v[0], v[1]), txd::pack_bf16x2(v[2], v[3])};
      }
  }
  __syncthreads();
  uint16_t *Cb = reinterpret_cast<uint16_t *>(a.C);
  if constexpr (TRANS) {
    // Unit u: staged column c = u % BN (C row n0 + c) and staged rows 8 s ..
    // 8 s + 7 (C columns m0 + 8 s ..), s = u / BN: a wave reads one staged
    // row segment of 64 columns at a time and each lane stores 16 bytes.
    const bool tvec = ((reinterpret_cast<uintptr_t>(a.C) & 15) == 0) && ((a.ldc & 7) == 0);
#pragma unroll
    for (int i = 0; i < 256 * BN / 8 / (64 * NW); ++i) {
      const int u = tid + 64 * NW * i;
      const int c = u % BN, s8 = 8 * (u / BN);
      uint32_t h[4];
#pragma unroll
      for (int t = 0; t < 8; t += 2) {
        const uint32_t lo = *reinterpret_cast<const uint16_t *>(
            lds + (s8 + t) * ROWB + (((c >> 3) ^ ((s8 + t) & (CH - 1))) << 4) + 2 * (c & 7));
        const uint32_t hi = *reinterpret_cast<const uint16_t *>(
            lds + (s8 + t + 1) * ROWB + (((c >> 3) ^ ((s8 + t + 1) & (CH - 1))) << 4) + 2 * (c & 7));
        h[t / 2] = lo | (hi << 16);
      }
      const int orow = n0 + c, ocol = m0 + s8;
      if (orow < a.N && ocol < a.M) {
        uint16_t *dst = Cb + int64_t(orow) * a.ldc + ocol;
        if (tvec && ocol + 7 < a.M) {
          *reinterpret_cast<txd::u32x4 *>(dst) = txd::u32x4{h[0], h[1], h[2], h[3]};
        } else {
#pragma unroll
          for (int t = 0; t < 8; ++t)
            if (ocol + t < a.M) dst[t] = uint16_t(h[t / 2] >> (16 * (t % 2)));
        }
      }
    }
    return;
  }
  const bool cvec = ((reinterpret_cast<uintptr_t>(a.C) & 15) == 0) && ((a.ldc & 7) == 0);
  const int sc = lane % CH;
  const int n = n0 + 8 * sc;
#pragma unroll
  for (int i = 0; i < 256 / NW / RPI; ++i) {
    const int row = wave * (256 / NW) + i * RPI + lane / CH;
    const int m = m0 + row;
    const txd::u32x4 w = *reinterpret_cast<const txd::u32x4 *>(lds + row * ROWB + ((sc ^ (row & (CH - 1))) << 4));
    if (m < a.M && n < a.N) {
      uint16_t *dst = Cb + int64_t(m) * a.ldc + n;
      if (cvec && n + 7 < a.N) {
        *reinterpret_cast<txd::u32x4 *>(dst) = w;
      } else {
        const uint32_t h[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int t = 0; t < 8; ++t)
          if (n + t < a.N) dst[t] = uint16_t(h[t / 2] >> (16 * (t % 2)));
      }
    }
  }
}

// Split-K reduction: C[m, n] = out(scale_a[m] * scale_b[n] * sum_s P[s][m][n])
// (ROWCOL: the fp8 row / column scales; out: bf16 or fp16 round to nearest
// even, or fp32), four consecutive n per thread.
// One workgroup per tile of a single product, or per (tile, split) pair
// with K split (split_coords).
template <class C, int BN, int NW = fast::kWaves, bool MX = false, int OUT = OUT_BF16, bool EPI = false>
__device__ __forceinline__ void gemm_fast_tile(const tx_gemm_args &a) {
  int tm, tn, split = 0;
  if (a.splits > 1) split_coords(int(blockIdx.x), a.tiles_m, a.tiles_n, a.splits, a.group_m, &tm, &tn, &split);
  else tile_coords(int(blockIdx.x), a.tiles_m, a.tiles_n, a.group_m, &tm, &tn);
  gemm_fast_tile_at<C, BN, NW, MX, OUT, EPI>(a, tm, tn, split);
}

constexpr int kReduceBatch = 16;  // splits whose loads are in flight together

template <bool ROWCOL, int OUT = OUT_BF16>
__device__ __forceinline__ void splitk_reduce(const tx_gemm_args &a) {
  // 16-bit output, no fused epilogue, N and ldc multiples of 8, C (and the
  // column scales) 16-byte aligned, at most 8 splits: eight consecutive n
  // per thread (the partial planes are 32-byte aligned then), every
  // split's 32 bytes loaded before the adds (same order of additions as the
  // general loop below), scales as vectors, one 16-byte store.
  if constexpr (OUT != OUT_F32) {
    if (!a.epi && (a.N & 7) == 0 && (a.ldc & 7) == 0 && (reinterpret_cast<uintptr_t>(a.C) & 15) == 0 &&
        a.splits <= 8 && (!ROWCOL || (reinterpret_cast<uintptr_t>(a.scale_b) & 15) == 0)) {
      const int64_t octs_per_row = a.N / 8;
      const int64_t total = int64_t(a.M) * octs_per_row;
      const int64_t plane = int64_t(a.M) * a.N;
      for (int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
           t += int64_t(gridDim.x) * blockDim.x) {
        const int m = int(t / octs_per_row);
        const int n = int(t % octs_per_row) * 8;
        const float *p = a.part + int64_t(m) * a.N + n;
        txd::f32x4 x[8][2];
#pragma unroll
        for (int s = 0; s < 8; ++s)
          if (s < a.splits) {
            x[s][0] = *reinterpret_cast<const txd::f32x4 *>(p + s * plane);
            x[s][1] = *reinterpret_cast<const txd::f32x4 *>(p + s * plane + 4);
          }
        float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 8; ++s)
          if (s < a.splits)
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] += x[s][i / 4][i % 4];
        if constexpr (ROWCOL) {
          const float sa = a.scale_a[m];
          const txd::f32x4 sb0 = *reinterpret_cast<const txd::f32x4 *>(a.scale_b + n);
          const txd::f32x4 sb1 = *reinterpret_cast<const txd::f32x4 *>(a.scale_b + n + 4);
#pragma unroll
          for (int i = 0; i < 8; ++i) v[i] = v[i] * sa * (i < 4 ? sb0[i] : sb1[i - 4]);
        }
        txd::u32x4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          o[i] = OUT == OUT_F16 ? txd::pack_f16x2(v[2 * i], v[2 * i + 1]) : txd::pack_bf16x2(v[2 * i], v[2 * i + 1]);
        *reinterpret_cast<txd::u32x4 *>(reinterpret_cast<uint16_t *>(a.C) + int64_t(m) * a.ldc + n) = o;
      }
      return;
    }
  }
  const int64_t quads_per_row = (a.N + 3) / 4;
  const int64_t total = int64_t(a.M) * quads_per_row;
  const int64_t plane = int64_t(a.M) * a.N;
  uint16_t *Cb = reinterpret_cast<uint16_t *>(a.C);
  for (int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
       t += int64_t(gridDim.x) * blockDim.x) {
    const int m = int(t / quads_per_row);
    const int n = int(t % quads_per_row) * 4;
    const float *p = a.part + int64_t(m) * a.N + n;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    // Splits in batches of kReduceBatch, each batch's loads issued before
    // its adds (in split order, so the sum is the same as one at a time).
    for (int s0 = 0; s0 < a.splits; s0 += kReduceBatch) {
      txd::f32x4 x[kReduceBatch];
#pragma unroll
      for (int j = 0; j < kReduceBatch; ++j) {
        const int s = s0 + j;
        if (s < a.splits) {
          if ((a.N & 3) == 0) {
            x[j] = *reinterpret_cast<const txd::f32x4 *>(p + s * plane);
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) x[j][i] = n + i < a.N ? p[s * plane + i] : 0.0f;
          }
        }
      }
#pragma unroll
      for (int j = 0; j < kReduceBatch; ++j)
        if (s0 + j < a.splits) {
          v[0] += x[j].x; v[1] += x[j].y; v[2] += x[j].z; v[3] += x[j].w;
        }
    }
    float sa = 1.0f;
    if constexpr (ROWCOL) sa = a.scale_a[m];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (n + i >= a.N) break;
      float r = v[i];
      if constexpr (ROWCOL) r = r * sa * a.scale_b[n + i];
      if (a.epi) {  // fused epilogue (uniform branch), after tt.dot's accumulator operand
        if (a.acc) r += a.acc[int64_t(m) * a.ld_acc + n + i];
        epi_store1(a, m, n + i, epi_value(a, r, n + i));
        continue;
      }
      if constexpr (OUT == OUT_F32) static_cast<float *>(a.C)[int64_t(m) * a.ldc + n + i] = r;
      else if constexpr (OUT == OUT_F16) Cb[int64_t(m) * a.ldc + n + i] = uint16_t(txd::pack_f16x2(r, 0.0f));
      else Cb[int64_t(m) * a.ldc + n + i] = uint16_t(txd::f32_to_bf16_bits(r));
    }
  }
}

}  // namespace txg
