// Persistent 4-wavefront GEMM for aligned operands whose K is a whole number
// of 128-byte steps (KTAIL, 16-bit operands: rows 4-byte aligned, any K of
// at least two steps, read as fast::KTail describes, and C rows of any
// alignment): one workgroup per CU walks its share of the BT x BT tiles
// (BT = 256; 128 or 64 for products with fewer 256 x 256 / 128 x 128 tiles
// than CUs),
// and the LDS-DMA pipeline of gemm_fast.h runs as one continuous
// stream of (tile, K step) pairs, so the first steps of the next tile are
// loaded while the current one finishes and no tile pays a pipeline fill.
//
// Layout per workgroup: 4 wavefronts (one per SIMD) in a 2 x 2 grid, each
// owning a BT / 2 square block of the tile; its accumulator blocks of 32 x 32
// (BT = 256: 16 blocks, 256 registers) live in AGPRs.  Against the
// 8-wavefront tile this reads a
// third less from LDS per MFMA (1 KiB instead of 1.5), which the power-
// limited clock turns into speed.
//
// The K loop is that of gemm_fast_tile_at (ring of 5 LDS slots of BT x 128 bytes,
// B of step s+2 and A of step s+3 loaded during the second half of step s,
// fragments one 64-byte half ahead in registers, one barrier per step), with
// s counting steps over all tiles of the workgroup.  Each operand's loads go
// through a buffer resource for the tile they belong to: base at the tile's
// first row, range ending after its last valid row, so rows past M / N read
// as zero; steps past the workgroup's last tile use an empty range.
//
// Tile order: the tiles of the transposed grid in the XCD-contiguous order of
// tile_coords, so each XCD's round of 32 concurrent tiles covers 8 column
// panels (B), kept from one round to the next, and 4 row panels (A), new in
// every round.  With inputs that are not yet in the Infinity Cache the new
// panels come from HBM, and A, loaded three steps ahead, hides that latency
// where B, two steps ahead, did not (8192^3 fp8 from HBM-resident inputs:
// 2530 -> 2290 cycles per K step; 2146 with cached inputs either way).
//
// Epilogue: the scales load just before the tile's last K step, whose A
// loads of step s+3 are deferred so that their LDS slot stages the output:
// per 32 x 32 block the accumulators are scaled, rounded to bf16 / fp16
// (RNE), and lanes l and l + 32 exchange halves (v_permlane32_swap); each
// wave writes its 32 x BT / 2 block to its own quarter of that slot, reads
// back whole rows (BT = 256: 4 of 256 bytes) per instruction and stores them
// through a buffer
// resource for C (stores past M / N are dropped).  The first K step of each
// tile starts its MFMAs from a zero accumulator operand, so the accumulators
// are never cleared explicitly.
#pragma once

#include "gemm_fast.h"

namespace txg {

namespace persist {
constexpr int kWaves = 4;

// Chunk swizzle of a K-major B slot (row-major K x N operand), by K row mod
// 4, for K rows of krb bytes: 256 or more, (0, 6, 12, 10); 128 (8 chunks,
// two rows per 256 bytes of banks), (0, 2, 4, 6).
__device__ __forceinline__ constexpr int kn_swz(int rho, int krb) {
  return krb >= 256 ? ((rho << 1) ^ (rho << 2)) & 14 : rho << 1;
}

// s_waitcnt lgkmcnt(N) that the two fragments depend on (their values come
// from LDS reads issued in inline asm, which the compiler does not wait for).
template <int N>
__device__ __forceinline__ void lgkm_wait_tie(txd::i32x4 &x, txd::i32x4 &y) {
  asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(x), "+v"(y) : "n"(N));
}
// The same dependency on a wait already made (the barrier's).
__device__ __forceinline__ void tie(txd::i32x4 &x, txd::i32x4 &y) { asm volatile("" : "+v"(x), "+v"(y)); }

// Buffer resource for rows r0 .. r0 + BT - 1 of an operand with `rows` rows of
// `ld_b` bytes, K step bytes kb_end: rows past the operand's end are outside
// the range.
template <int BT>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const void *base, int r0, int rows, uint32_t ld_b,
                                                            uint32_t kb_end) {
  const int valid = min(BT, rows - r0);
  return make_rsrc(static_cast<const uint8_t *>(base) + int64_t(r0) * ld_b, uint32_t(valid - 1) * ld_b + kb_end);
}
}  // namespace persist

// GROUPED: the tiles of a grouped product (tx_grouped_args with offsets;
// the m-tile prefix already written by tx_gemm_fp8_grouped_prefix), a the
// shared fields q->g: tile t of the workgroup is (problem p, m tile, n tile)
// of expert p's rows offsets[p] .. offsets[p + 1] of A, C and scale_a against
// B + p stride_b and scale_b + p stride_sb.
//
// BKN: B is row-major K x N (16-bit operands, K a whole number of steps).  A
// step of B is then 64 K rows of the tile's BT columns (2 BT bytes each),
// DMA'd into a K-major slot whose 16-byte chunk c of K row k sits at
// c ^ kn_swz(k mod 4, 2 BT), and each B fragment is two transposing LDS reads
// (ds_read_b64_tr_b16): in each 16-lane group, lane s reads 4 columns at K
// row s / 4 and lane d receives column d's 4 K values, the register layout
// the MFMA takes.  The swizzle keeps a group's 4 rows x 2 chunks on 8
// distinct 16-byte bank groups of 128 bytes, and a 32-lane half's 4 rows x
// 4 chunks on 16 of 256 bytes (for 128-byte rows, two to 256 bytes of
// banks: on 8 of 128 and on 16 half-row positions).
template <class C, int OUT = OUT_BF16, bool GROUPED = false, bool KTAIL = false, bool BKN = false, int BT = 256>
__device__ __forceinline__ void gemm_persist(const tx_gemm_args &a, const tx_grouped_args *q = nullptr) {
  using namespace fast;
  static_assert(OUT == OUT_BF16 || (OUT == OUT_F16 && !C::FP8), "bf16 output, or fp16 out of 16-bit operands");
  static_assert(!KTAIL || (!C::FP8 && !GROUPED), "ragged K: 16-bit operands, one product");
  static_assert(!BKN || (!C::FP8 && !GROUPED && !KTAIL), "row-major B: 16-bit operands, whole K steps");
  static_assert(BT == 256 || BT == 128 || BT == 64, "tile 256, 128 or 64 square");
  constexpr int NW = persist::kWaves;
  constexpr int TM = BT / 2, TN = BT / 2, FM = TM / 32, FN = TN / 32;
  constexpr int NM = FM * FN, NF = FM + FN, NR = 2 * NF;
  constexpr int SB = BT * kStep;  // one operand of one K step
  constexpr int BLKA = SB / 1024 / NW, BLKB = BLKA, ND = BLKA + BLKB;
  constexpr int RW = NM >= 2 ? NM / 2 : 1;
  constexpr bool ROWCOL = C::FP8;
  // BKN: bytes of a K row of the B tile, and K rows per 1 KiB DMA block
  constexpr int KRB = 2 * BT, RPB = 1024 / KRB, CPR = KRB / 16;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kSlots * SB];

  // m tiles: the grouped product's real count is only on the device
  const int tiles_m = GROUPED ? q->tile_prefix[q->groups] : a.tiles_m;
  const int total = tiles_m * a.tiles_n;
  const int G = int(gridDim.x);
  const int w = int(blockIdx.x);
  const int T = w < total ? (total - w + G - 1) / G : 0;  // tiles of this workgroup
  if (T == 0) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % 2, wn = wave / 2;
  constexpr int ES = C::FP8 ? 1 : 2;
  const uint32_t kb_end = uint32_t(a.K) * ES;
  const int KS = int(KTAIL ? (kb_end + kStep - 1) / kStep : kb_end / kStep);  // K steps per tile (>= 2)
  const int S = T * KS;                // steps of the workgroup
  const uint32_t lda_b = uint32_t(a.lda) * ES, ldb_b = uint32_t(a.ldb) * ES;

  // Per-lane DMA offsets within a tile: row * ld + chunk for the wave's
  // first two blocks (the chunk swizzle depends on the block's parity only);
  // block j adds 8 j rows, and the K step, in the scalar offset.
  const uint32_t kch[2] = {16u * uint32_t((lane & 7) ^ ((lane >> 4) & 7)),
                           16u * uint32_t((lane & 7) ^ ((4 + (lane >> 4)) & 7))};
  uint32_t vo[2][2];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    vo[0][e] = uint32_t(8 * (BLKA * wave + e) + (lane >> 3)) * lda_b + kch[e];
    if constexpr (BKN) {
      // block j: K rows RPB (BLKB wave + j) .. + RPB - 1 of the step, lane p
      // filling chunk position p mod CPR of row + p / CPR (row mod 4
      // depends on the block's parity only)
      const int kr = RPB * (BLKB * wave + e) + lane / CPR;
      vo[1][e] = uint32_t(kr) * ldb_b + 16u * uint32_t((lane % CPR) ^ persist::kn_swz(kr & 3, KRB));
    } else {
      vo[1][e] = uint32_t(8 * (BLKB * wave + e) + (lane >> 3)) * ldb_b + kch[e];
    }
  }
  const uint32_t ld8[2] = {8u * lda_b, (BKN ? uint32_t(RPB) : 8u) * ldb_b};
  // bytes of an operand's K step in its rows
  const uint32_t kstep_b[2] = {uint32_t(kStep), BKN ? 64u * ldb_b : uint32_t(kStep)};
  // KTAIL: the lane offsets of the last K step (scalar offset - 16 there)
  const KTail kt = make_ktail(kb_end);
  uint32_t vl[2][2];
  if constexpr (KTAIL) {
    const uint32_t kb16 = kb_end & ~15u, kr = kb_end & 15u, kbz = kr ? kb16 + 16u : kb_end;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const uint32_t cs = uint32_t(KS - 1) * kStep + kch[e];  // the lane's chunk, from the row start
#pragma unroll
      for (int op = 0; op < 2; ++op) vl[op][e] = cs >= kbz ? kOob : vo[op][e] + (cs == kb16 ? kr : 16u);
    }
  }
  using OpA = std::integral_constant<int, 0>;
  using OpB = std::integral_constant<int, 1>;
  // Tile t of the workgroup: its operands and output (for a grouped product,
  // those of its problem) and its m / n tile.
  struct TileDesc {
    const uint8_t *A, *B;
    uint8_t *out;  // C
    const float *sa, *sb;
    int rows, tm, tn;
  };
  auto desc = [&](int t) {
    TileDesc d;
    int vm;
    tile_coords(w + t * G, a.tiles_n, tiles_m, min(8, a.tiles_n), &d.tn, &vm);  // transposed grid
    d.A = static_cast<const uint8_t *>(a.A);
    d.B = static_cast<const uint8_t *>(a.B);
    d.out = static_cast<uint8_t *>(a.C);
    d.sa = a.scale_a;
    d.sb = a.scale_b;
    d.rows = a.M;
    d.tm = vm;
    if constexpr (GROUPED) {
      const int32_t *Tp = q->tile_prefix;
      int lo = 0, hi = q->groups - 1;  // the last problem p with Tp[p] <= vm
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (Tp[mid] <= vm) lo = mid;
        else hi = mid - 1;
      }
      const int r1 = min(max(q->offsets[lo + 1], 0), a.M);
      const int r0 = min(max(q->offsets[lo], 0), r1);
      d.A += int64_t(r0) * a.lda;
      d.B += int64_t(lo) * q->stride_b;
      d.out += int64_t(r0) * a.ldc * 2;
      d.sa += r0;
      d.sb += int64_t(lo) * q->stride_sb;
      d.rows = r1 - r0;
      d.tm = vm - Tp[lo];
    }
    return d;
  };

  // Load cursor of one operand: the step it is at and the buffer resource of
  // that step's tile (an empty range past the last tile).  Steps advance
  // one at a time.
  struct Cursor {
    int t, k;
    __amdgpu_buffer_rsrc_t rs;
  };
  auto set_tile = [&](Cursor &c, auto op_tag) {
    constexpr int op = decltype(op_tag)::value;
    if (c.t < T) {
      const TileDesc d = desc(c.t);
      if constexpr (BKN && op == 1) {
        // columns BT tn .. of all K rows, the range ending at the last
        // row's last column (columns past N in earlier rows read that
        // row's padding or the next row: their products are not stored)
        c.rs = make_rsrc(d.B + int64_t(d.tn) * KRB, uint32_t(a.K - 1) * ldb_b + uint32_t(a.N - d.tn * BT) * 2u);
      } else {
        c.rs = op == 0 ? persist::tile_rsrc<BT>(d.A, d.tm * BT, d.rows, lda_b, kb_end)
                       : persist::tile_rsrc<BT>(d.B, d.tn * BT, a.N, ldb_b, kb_end);
      }
    } else {
      c.rs = make_rsrc(op == 0 ? a.A : a.B, 0u);
    }
  };
  auto advance = [&](Cursor &c, auto op_tag) {
    if (++c.k == KS) {
      c.k = 0;
      ++c.t;
      set_tile(c, op_tag);
    }
  };
  auto load_op = [&](const Cursor &c, int slot, auto op_tag, auto j_tag) {
    constexpr int op = decltype(op_tag)::value, j = decltype(j_tag)::value;
    constexpr int blk = op == 0 ? BLKA : BLKB;
    uint8_t *dst = lds + slot * SB + (blk * wave + j) * 1024;
    const bool lk = KTAIL && c.k == KS - 1;  // (c.k >= 1 there)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(c.rs, (lds_void *)dst, 16, lk ? vl[op][j & 1] : vo[op][j & 1],
                                             uint32_t(c.k) * kstep_b[op] + uint32_t(j & ~1) * ld8[op] -
                                                 (lk ? 16u : 0u),
                                             0, 0);
  };

  const int frow = lane & 31, fg = lane >> 5;
  int ro[2][2][2];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int chunk = 4 * h + (C::FP8 ? fg + 2 * e : 2 * fg + e);
      ro[0][h][e] = off(wm * TM + frow, chunk);
      ro[1][h][e] = off(wn * TN + frow, chunk);
    }
  // BKN: the B fragment reads' lane offsets in a slot, per 32-column block
  // fn, for K row 16 g + s / 4 (g = lane / 32, s = lane mod 16) and columns
  // 32 fn + 16 ((lane / 16) mod 2) + 4 (s mod 4) .. + 3 of the wave's; half
  // h, piece e and read r add K rows 32 h + 8 e + 4 r (a multiple of 4, so
  // the swizzle is the lane's).
  int bko[BKN ? FN : 1];
  const uint32_t lds_base = uint32_t(reinterpret_cast<uintptr_t>((lds_u8 *)lds));
  if constexpr (BKN) {
    const int s16 = lane & 15, rho = s16 >> 2;
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) {
      const int n = wn * TN + 32 * fn + 16 * ((lane >> 4) & 1) + 4 * (s16 & 3);
      bko[fn] = (16 * fg + rho) * KRB + (((n >> 3) ^ persist::kn_swz(rho, KRB)) << 4) + 8 * ((n >> 2) & 1);
    }
  }
  txd::i32x4 fr[2][NF][2];
  auto read = [&](int slot_a, int slot_b, auto h_tag, auto r_tag) {
    constexpr int h = decltype(h_tag)::value, r = decltype(r_tag)::value, e = r % 2, o = r / 2;
    constexpr int f = o == 0 ? 0 : o == 1 ? FM : o <= FM ? o - 1 : o;
    const uint8_t *Sp = lds + (f < FM ? slot_a : slot_b) * SB;
    if constexpr (BKN && f >= FM) {
      // Inline asm: the compiler puts a vmcnt(0) (a drain of every operand
      // load in flight) before the intrinsic form of this read whenever an
      // LDS-DMA load is pending.  Its results are waited for explicitly:
      // kn_wait in the K step's first half, the barrier in the second.
      constexpr int c0 = (32 * h + 8 * e) * KRB;
      const uint32_t addr = lds_base + uint32_t(slot_b * SB + bko[f - FM]);
      txd::u32x2 lo, hi;
      asm volatile("ds_read_b64_tr_b16 %0, %2 offset:%3\n\tds_read_b64_tr_b16 %1, %2 offset:%4"
                   : "=&v"(lo), "=&v"(hi)
                   : "v"(addr), "i"(c0), "i"(c0 + 4 * KRB)
                   : "memory");
      fr[h][f][e] = txd::i32x4{int(lo[0]), int(lo[1]), int(hi[0]), int(hi[1])};
    } else {
      const int byte = f < FM ? ro[0][h][e] + 4096 * f : ro[1][h][e] + 4096 * (f - FM);
      fr[h][f][e] = *reinterpret_cast<const txd::i32x4 *>(Sp + byte);
    }
  };
  // BKN: wait for the first half's B block fn before its first MFMA.  The
  // half's reads are issued in the order of `read`: A0 (2 LDS operations),
  // B0 (4), A1 .. A(FM-1) (2 each), B1 .. B(FN-1) (4 each); LDS operations complete
  // in order, so at most the operations issued after B fn may be left
  // outstanding (capped at lgkmcnt's 15; extra scalar loads in flight only
  // make the wait longer).  The asm ties the fragments to the wait.
  auto kn_wait = [&](auto fn_tag) {
    constexpr int fn = decltype(fn_tag)::value;
    constexpr int after = fn == 0 ? 2 * (FM - 1) + 4 * (FN - 1) : 4 * (FN - 1 - fn);
    constexpr int n = after > 15 ? 15 : after;
    persist::lgkm_wait_tie<n>(fr[0][FM + fn][0], fr[0][FM + fn][1]);
  };
  txd::f32x16 acc[FN][FM];
  // MFMA i of a K half: B block i / FM against A block i % FM; FIRST: the
  // tile's first step, from a zero accumulator.
  auto mma = [&](auto h_tag, auto i_tag, auto first_tag) {
    constexpr int h = decltype(h_tag)::value, i = decltype(i_tag)::value, fn = i / FM, fm = i % FM;
    const i32x8 va = __builtin_shufflevector(fr[h][fm][0], fr[h][fm][1], 0, 1, 2, 3, 4, 5, 6, 7);
    const i32x8 vb = __builtin_shufflevector(fr[h][FM + fn][0], fr[h][FM + fn][1], 0, 1, 2, 3, 4, 5, 6, 7);
    if constexpr (decltype(first_tag)::value && h == 0) acc[fn][fm] = txd::f32x16{};
    mfma32<C>(acc[fn][fm], vb, va);
  };
  using H0 = std::integral_constant<int, 0>;
  using H1 = std::integral_constant<int, 1>;

  // Prologue: steps 0, 0, 1, 1, 2 (A0 B0 A1 B1 A2) of the first tile.
  Cursor ca, cb;
  ca.t = ca.k = cb.t = cb.k = 0;
  set_tile(ca, OpA{});
  set_tile(cb, OpB{});
  static_for<BLKA>([&](auto j) { load_op(ca, 0, OpA{}, j); });
  static_for<BLKB>([&](auto j) { load_op(cb, 1, OpB{}, j); });
  advance(ca, OpA{});
  advance(cb, OpB{});
  static_for<BLKA>([&](auto j) { load_op(ca, 2, OpA{}, j); });
  static_for<BLKB>([&](auto j) { load_op(cb, 3, OpB{}, j); });
  advance(ca, OpA{});
  advance(cb, OpB{});  // next B load: step 2
  static_for<BLKA>([&](auto j) { load_op(ca, 4, OpA{}, j); });
  advance(ca, OpA{});  // next A load: step 3
  wait_and_barrier<2 * BLKA + BLKB>();
  static_for<NR>([&](auto r) { read(0, 1, H0{}, r); });

  // One K step: half 0 (reads of half 1), barrier, half 1 (loads of B s+2
  // and A s+3, reads of half 0 of step s+1).  FIRST: the tile's first step
  // (MFMAs from a zero accumulator); VM: loads and stores allowed in flight
  // at the barrier (the next step's operands are older than the last VM);
  // LAST: the tile's last step, whose A s+3 loads wait until after the
  // epilogue (their slot stages the output tile), as do the reads of the
  // next step's first half (their registers hold the column scales).
  int sa = 0, sb = 1;
  auto step = [&](auto first_tag, auto vm_tag, auto last_tag) {
    constexpr int VM = decltype(vm_tag)::value;
    constexpr bool LAST = decltype(last_tag)::value;
    const int na = sa >= 3 ? sa - 3 : sa + 2, nb = sb >= 3 ? sb - 3 : sb + 2;
    const bool clear = KTAIL && LAST && kt.cp < 8;
    if (clear) ktail_clear<NF>(fr[0], 0, fg, kt);
    static_for<NM>([&](auto I) {
      constexpr int i = decltype(I)::value;
      if constexpr (BKN && i % FM == 0) kn_wait(std::integral_constant<int, i / FM>{});
      mma(H0{}, I, first_tag);
      __builtin_amdgcn_sched_barrier(0);
      constexpr int r0 = spread_lo(i, NR, RW), r1 = spread_hi(i, NR, RW);
      static_for<r1 - r0>([&](auto R) { read(sa, sb, H1{}, std::integral_constant<int, r0 + decltype(R)::value>{}); });
      __builtin_amdgcn_sched_barrier(0);
    });
    wait_and_barrier<VM>();
    if constexpr (BKN) {
      // the barrier's lgkmcnt(0) completed the second half's B reads
      static_for<FN>([&](auto fn) { persist::tie(fr[1][FM + decltype(fn)::value][0], fr[1][FM + decltype(fn)::value][1]); });
    }
    __builtin_amdgcn_sched_barrier(0);
    if (clear) ktail_clear<NF>(fr[1], 1, fg, kt);
    static_for<NM>([&](auto I) {
      constexpr int i = decltype(I)::value;
      mma(H1{}, I, std::false_type{});
      __builtin_amdgcn_sched_barrier(0);
      constexpr int d0 = spread_lo(i, ND, NM), d1 = spread_hi(i, ND, NM);
      static_for<d1 - d0>([&](auto D) {
        constexpr int d = d0 + decltype(D)::value;
        if constexpr (d < BLKB) load_op(cb, sa, OpB{}, std::integral_constant<int, d>{});
        else if constexpr (!LAST) load_op(ca, sb, OpA{}, std::integral_constant<int, d - BLKB>{});
      });
      constexpr int r0 = spread_lo(i, NR, RW), r1 = spread_hi(i, NR, RW);
      if constexpr (!LAST)
        static_for<r1 - r0>([&](auto R) { read(na, nb, H0{}, std::integral_constant<int, r0 + decltype(R)::value>{}); });
      __builtin_amdgcn_sched_barrier(0);
    });
    advance(cb, OpB{});
    if constexpr (!LAST) advance(ca, OpA{});
    sa = na;
    sb = nb;
  };
  using VmStep = std::integral_constant<int, BLKA>;
  // The epilogue issues exactly kEpiStores stores per wave, then the last
  // step's deferred BLKA loads of A; the next tile's first barrier may
  // leave all of them in flight.
  // staging geometry: the wave's 32 x TN block as 32 rows of SRB bytes
  // (CH 16-byte chunks), read back SPI rows per instruction
  constexpr int SRB = 2 * TN, CH = SRB / 16, SPI = 64 / CH;
  constexpr int kEpiStores = FM * (32 / SPI);
  using VmAfterEpi = std::integral_constant<int, BLKB + kEpiStores>;
  static_assert(BLKB + kEpiStores < 64, "vmcnt range");
  // Scale loads issued before the last step (row scales, 16 column-scale
  // vectors) that its barrier leaves in flight with the step's own A loads.
  constexpr int kScaleLoads = ROWCOL ? FM + 4 * FN : 0;
  using VmLast = std::integral_constant<int, BLKA + kScaleLoads>;
  static_assert(BLKA + kScaleLoads < 64, "vmcnt range");

  // Staging: wave w owns bytes 32 SRB w .. + 32 SRB of the slot its last
  // step's A s+3 loads would have filled (the same bytes those loads fill
  // once the epilogue is done, so no other wave ever touches them): 32 rows
  // of SRB bytes, 16-byte chunk c of row r at c ^ (r % CH).
  for (int t = 0; t < T; ++t) {
    const TileDesc d = desc(t);
    const int m0 = d.tm * BT, n0 = d.tn * BT;
    // C as a buffer: a store whose row or column block lies past M / N gets
    // an offset past the range and is dropped (N is a multiple of 8, so a
    // 16-byte column block is wholly in or out).  KTAIL: rows of C may have
    // any alignment; the buffer starts at the 16-byte boundary below C.
    const uint32_t cmis = KTAIL ? uint32_t(reinterpret_cast<uintptr_t>(d.out) & 15u) : 0u;
    const __amdgpu_buffer_rsrc_t crs =
        make_rsrc(d.out - cmis, uint32_t((int64_t(d.rows - 1) * a.ldc + a.N) * 2) + cmis);
    if (t == 0) step(std::true_type{}, VmStep{}, std::false_type{});
    else step(std::true_type{}, VmAfterEpi{}, std::false_type{});
    for (int k = 1; k < KS - 1; ++k) step(std::false_type{}, VmStep{}, std::false_type{});
    // Scales load just before the last step and are waited for after it
    // with vmcnt(BLKB), leaving its B loads in flight.  Loads and waits are
    // written out: the compiler does not count the LDS-DMA loads when it
    // places waits, so its own wait here would be vmcnt(0), a full drain of
    // the next tile's operand loads (vector-memory operations complete in
    // order, so vmcnt(n) with n = the operations issued since guarantees a
    // load).  Rows past M read row M - 1 and columns past N the last four;
    // their stores are dropped.
    float sav[FM];
    txd::f32x4 sb4[FN][4];  // columns 32 fn + 8 jj + 4 g .. + 3 of the wave's
    if constexpr (ROWCOL) {
      const int nl = n0 + wn * TN + 4 * fg;
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        const float *ps = d.sa + min(m0 + wm * TM + fm * 32 + frow, d.rows - 1);
        asm volatile("global_load_dword %0, %1, off" : "=v"(sav[fm]) : "v"(ps) : "memory");
      }
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const float *ps = d.sb + min(nl + 32 * fn + 8 * jj, a.N - 4);
          asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(sb4[fn][jj]) : "v"(ps) : "memory");
        }
    }
    const int stage_slot = sb;  // the last step's B slot: its A s+3 loads go there
    step(std::false_type{}, VmLast{}, std::true_type{});  // the last step (KS >= 2)
    if constexpr (ROWCOL) {
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(BLKB) : "memory");
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) asm volatile("" : "+v"(sav[fm]));
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
        asm volatile("" : "+v"(sb4[fn][0]), "+v"(sb4[fn][1]), "+v"(sb4[fn][2]), "+v"(sb4[fn][3]));
    }
    // Epilogue, per 32-row block fm: scale, round, and exchange halves so
    // that lane l < 32 holds columns 16 p .. 16 p + 7 and lane l + 32
    // columns 16 p + 8 .. + 15 of row l % 32 (p = 2 fn + pr); stage the
    // wave's 32 x TN block, then store SPI rows of SRB bytes per instruction.
    // The accumulators are read below in inline asm, for which the compiler
    // inserts no wait states after the MFMAs that write them: the last step's
    // final MFMAs stay above this point, and 32 wait states (a 16-pass MFMA's
    // result needs about 19) pass before the first read.
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    uint8_t *stg = lds + stage_slot * SB + wave * (32 * SRB);
    // The lane's staging offsets are recomputed for each tile from an opaque
    // copy of the lane index: hoisted out of the tile loop, they would hold
    // registers through the whole K loop (fp8: 238 -> 206 VGPRs).
    int el = lane;
    asm volatile("" : "+v"(el));
    const int efrow = el & 31, efg = el >> 5;
    const int srow = el / CH, schunk = el % CH;  // read-back: row SPI i + srow, chunk schunk
    const int n_st = n0 + wn * TN + 8 * schunk;
    const uint32_t coloff = n_st < a.N ? uint32_t(n_st) * 2u + cmis : kOob;
    static_for<FM>([&](auto fm_tag) {
      constexpr int fm = decltype(fm_tag)::value;
      static_for<FN>([&](auto fn_tag) {
        constexpr int fn = decltype(fn_tag)::value;
#pragma unroll
        for (int pr = 0; pr < 2; ++pr) {
          uint32_t pk[2][2];
#pragma unroll
          for (int jl = 0; jl < 2; ++jl) {
            float v[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              // read the accumulator where it is used (the compiler would
              // otherwise copy whole tiles out of the AGPRs at once)
              asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(v[q]) : "a"(acc[fn][fm][4 * (2 * pr + jl) + q]));
              if constexpr (ROWCOL) v[q] = v[q] * sav[fm] * sb4[fn][2 * pr + jl][q];
            }
            pk[jl][0] = OUT == OUT_F16 ? txd::pack_f16x2(v[0], v[1]) : txd::pack_bf16x2(v[0], v[1]);
            pk[jl][1] = OUT == OUT_F16 ? txd::pack_f16x2(v[2], v[3]) : txd::pack_bf16x2(v[2], v[3]);
          }
          uint32_t o[4];
#pragma unroll
          for (int d = 0; d < 2; ++d) {
            const auto sw = __builtin_amdgcn_permlane32_swap(pk[0][d], pk[1][d], false, false);
            o[d] = sw[0];
            o[2 + d] = sw[1];
          }
          const int chunk = 2 * (2 * fn + pr) + efg;
          *reinterpret_cast<txd::u32x4 *>(stg + efrow * SRB + ((chunk ^ (efrow & (CH - 1))) << 4)) =
              txd::u32x4{o[0], o[1], o[2], o[3]};
        }
      });
#pragma unroll
      for (int i = 0; i < 32 / SPI; ++i) {
        const int r = SPI * i + srow;
        const txd::u32x4 w = *reinterpret_cast<const txd::u32x4 *>(stg + r * SRB + ((schunk ^ (r & (CH - 1))) << 4));
        const int m = m0 + wm * TM + fm * 32 + r;
        const uint32_t voff = (m >= d.rows || coloff == kOob) ? kOob : uint32_t(m) * uint32_t(a.ldc) * 2u + coloff;
        __builtin_amdgcn_raw_buffer_store_b128(w, crs, voff, 0, 0);
      }
    });
    // the deferred A s+3 loads (after this wave's last staging reads) and
    // the next step's first-half fragments
    __builtin_amdgcn_s_waitcnt((63 & 15) | (7 << 4) | (0 << 8) | ((63 >> 4) << 14));
    static_for<BLKA>([&](auto j) { load_op(ca, stage_slot, OpA{}, j); });
    advance(ca, OpA{});
    static_for<NR>([&](auto r) { read(sa, sb, H0{}, r); });
  }
  // Drain the trailing (empty-range) loads before the workgroup's LDS is released.
  wait_and_barrier<0>();
}

}  // namespace txg
