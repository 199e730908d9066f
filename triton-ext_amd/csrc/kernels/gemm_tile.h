// Tiled MFMA GEMM body shared by the bf16 and fp8 tt.dot kernels.
// See gemm_common.h for the layout contract and LDS organisation.
#pragma once

#include "gemm_common.h"

namespace txg {

// Operand element kinds for the MFMA selection.
enum { EL_BF16 = 0, EL_E4M3 = 1, EL_E5M2 = 2, EL_E2M1 = 4, EL_F16 = 5, EL_F32 = 6, EL_I8 = 7 };  // e2m1: fp4, two per byte along K

// Output element types of the tiles (16-bit kinds round to nearest even;
// int32: the int8 dot's exact sums, wrapping modulo 2^32).
enum GemmOut { OUT_BF16 = 0, OUT_F16 = 1, OUT_F32 = 2, OUT_I32 = 3 };

template <int EL_A, int EL_B, int BM_, int BN_, int WM_, int WN_, int VEC_>
struct GemmCfg {
  static constexpr int EL_A_ = EL_A, EL_B_ = EL_B;
  static constexpr bool FP8 = EL_A == EL_E4M3 || EL_A == EL_E5M2 || EL_A == EL_E2M1;  // the f8f6f4 MFMA
  static constexpr bool F16 = EL_A == EL_F16;
  static constexpr bool F32 = EL_A == EL_F32;  // fp32 operands (v_mfma_f32_16x16x4_f32)
  static constexpr bool I8 = EL_A == EL_I8;    // int8 operands (v_mfma_i32_16x16x64_i8)
  static constexpr int ES = F32 ? 4 : (FP8 || I8) ? 1 : 2;  // operand bytes per element
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, VEC = VEC_;
  static constexpr int T = 64 * WM * WN;
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int FM = WTM / 16, FN = WTN / 16;
  static constexpr int A_CH = BM * kChunks / T, B_CH = BN * kChunks / T;
  static constexpr int STAGE_BYTES = (BM + BN) * kRowBytes;
  static_assert(BM * kChunks % T == 0 && BN * kChunks % T == 0, "chunk split");
  static_assert(WTM % 16 == 0 && WTN % 16 == 0, "wave tile");
};

// f8f6f4 operand format codes of the gfx950 MFMA (0 = fp8 e4m3, 1 = bf8 e5m2,
// 4 = fp4 e2m1).
template <int EL> struct F8Code { static constexpr int v = EL == EL_E5M2 ? 1 : EL == EL_E2M1 ? 4 : 0; };

template <class C>
__device__ __forceinline__ f32x4 mfma_step(f32x4 acc, const u32x4 (&mfa)[2], const u32x4 (&mfb)[2]) {
  if constexpr (C::F32) {
    // 8 fp32 K values per lane: one 4-K instruction per value (lane group g
    // holds K 8g .. 8g + 7 of the step, so instruction j sums K j, 8 + j, ...)
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(mfa[h][j]), __uint_as_float(mfb[h][j]), acc,
                                                   0, 0, 0);
  } else if constexpr (C::I8) {
    // the int32 accumulators live in the fp32 registers' bits
    txd::i32x4 c = __builtin_bit_cast(txd::i32x4, acc);
    c = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(txd::i32x4, mfa[0]),
                                              __builtin_bit_cast(txd::i32x4, mfb[0]), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(txd::i32x4, mfa[1]),
                                              __builtin_bit_cast(txd::i32x4, mfb[1]), c, 0, 0, 0);
    acc = __builtin_bit_cast(f32x4, c);
  } else if constexpr (C::F16) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(txd::f16x8, mfa[0]),
                                                 __builtin_bit_cast(txd::f16x8, mfb[0]), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(txd::f16x8, mfa[1]),
                                                 __builtin_bit_cast(txd::f16x8, mfb[1]), acc, 0, 0, 0);
  } else if constexpr (!C::FP8) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(txd::bf16x8, mfa[0]),
                                                  __builtin_bit_cast(txd::bf16x8, mfb[0]), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(txd::bf16x8, mfa[1]),
                                                  __builtin_bit_cast(txd::bf16x8, mfb[1]), acc, 0, 0, 0);
  } else {
    const i32x8 a8 = {int(mfa[0].x), int(mfa[0].y), int(mfa[0].z), int(mfa[0].w),
                      int(mfa[1].x), int(mfa[1].y), int(mfa[1].z), int(mfa[1].w)};
    const i32x8 b8 = {int(mfb[0].x), int(mfb[0].y), int(mfb[0].z), int(mfb[0].w),
                      int(mfb[1].x), int(mfb[1].y), int(mfb[1].z), int(mfb[1].w)};
    // MFMA "A" operand is the B tile, MFMA "B" operand is the A tile.
    acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a8, b8, acc, F8Code<C::EL_B_>::v,
                                                           F8Code<C::EL_A_>::v, 0, 0, 0, 0);
  }
  return acc;
}

template <class C, int OUT = OUT_BF16>
__device__ __forceinline__ void gemm_tile(const tx_gemm_args &a) {
  static_assert((C::F32 && OUT == OUT_F32) || (C::I8 && OUT == OUT_I32) ||
                    (!C::F32 && !C::I8 && (OUT == OUT_BF16 || (OUT == OUT_F16 && !C::FP8))),
                "generic tile: bf16 out, fp16 out of 16-bit operands, fp32 out of fp32, int32 out of int8");
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * C::STAGE_BYTES];

  int tm, tn;
  tile_coords(blockIdx.x, a.tiles_m, a.tiles_n, a.group_m, &tm, &tn);
  const int m0 = tm * C::BM, n0 = tn * C::BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % C::WM, wn = wave / C::WM;
  constexpr int ES = C::ES;
  const int kb_end = a.K * ES;
  const int ksteps = (kb_end + kRowBytes - 1) / kRowBytes;
  const uint8_t *Ab = reinterpret_cast<const uint8_t *>(a.A);
  const uint8_t *Bb = reinterpret_cast<const uint8_t *>(a.B);
  const int64_t lda_b = a.lda * ES, ldb_b = a.ldb * ES;

  // Global -> register staging assignment: chunk `ch` of rows r_base + i*T/8.
  const int ch = tid & 7, r_base = tid >> 3;
  constexpr int RSTEP = C::T / 8;
  const uint8_t *a_row[C::A_CH];
  bool a_ok[C::A_CH];
  const uint8_t *b_row[C::B_CH];
  bool b_ok[C::B_CH];
#pragma unroll
  for (int i = 0; i < C::A_CH; ++i) {
    const int gm = m0 + r_base + i * RSTEP;
    a_ok[i] = gm < a.M;
    a_row[i] = Ab + int64_t(a_ok[i] ? gm : 0) * lda_b;
  }
#pragma unroll
  for (int i = 0; i < C::B_CH; ++i) {
    const int gn = n0 + r_base + i * RSTEP;
    b_ok[i] = gn < a.N;
    b_row[i] = Bb + int64_t(b_ok[i] ? gn : 0) * ldb_b;
  }
  u32x4 ra[C::A_CH], rb[C::B_CH];
  auto gload = [&](int ks) {
    const int kb = ks * kRowBytes + ch * 16;
#pragma unroll
    for (int i = 0; i < C::A_CH; ++i) ra[i] = load_chunk<C::VEC>(a_row[i], kb, kb_end, a_ok[i]);
#pragma unroll
    for (int i = 0; i < C::B_CH; ++i) rb[i] = load_chunk<C::VEC>(b_row[i], kb, kb_end, b_ok[i]);
  };
  auto lstore = [&](int buf) {
    uint8_t *As = lds + buf * C::STAGE_BYTES;
    uint8_t *Bs = As + C::BM * kRowBytes;
#pragma unroll
    for (int i = 0; i < C::A_CH; ++i)
      *reinterpret_cast<u32x4 *>(As + lds_off(r_base + i * RSTEP, ch)) = ra[i];
#pragma unroll
    for (int i = 0; i < C::B_CH; ++i)
      *reinterpret_cast<u32x4 *>(Bs + lds_off(r_base + i * RSTEP, ch)) = rb[i];
  };

  f32x4 acc[C::FN][C::FM];
#pragma unroll
  for (int i = 0; i < C::FN; ++i)
#pragma unroll
    for (int j = 0; j < C::FM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (ksteps > 0) {
    gload(0);
    lstore(0);
  }
  __syncthreads();

  const int frow = lane & 15, fg = lane >> 4;  // fragment row / lane group
  for (int ks = 0; ks < ksteps; ++ks) {
    const int buf = ks & 1;
    if (ks + 1 < ksteps) gload(ks + 1);
    const uint8_t *As = lds + buf * C::STAGE_BYTES;
    const uint8_t *Bs = As + C::BM * kRowBytes;
    u32x4 fa[C::FM][2];
#pragma unroll
    for (int fm = 0; fm < C::FM; ++fm) {
      const int r = wm * C::WTM + fm * 16 + frow;
      fa[fm][0] = *reinterpret_cast<const u32x4 *>(As + lds_off(r, 2 * fg));
      fa[fm][1] = *reinterpret_cast<const u32x4 *>(As + lds_off(r, 2 * fg + 1));
    }
#pragma unroll
    for (int fn = 0; fn < C::FN; ++fn) {
      const int r = wn * C::WTN + fn * 16 + frow;
      u32x4 fb[2];
      fb[0] = *reinterpret_cast<const u32x4 *>(Bs + lds_off(r, 2 * fg));
      fb[1] = *reinterpret_cast<const u32x4 *>(Bs + lds_off(r, 2 * fg + 1));
#pragma unroll
      for (int fm = 0; fm < C::FM; ++fm) acc[fn][fm] = mfma_step<C>(acc[fn][fm], fb, fa[fm]);
    }
    if (ks + 1 < ksteps) lstore(buf ^ 1);
    __syncthreads();
  }

  // Epilogue: lane owns C[m][n .. n+3] of every 16x16 block.
  if constexpr (OUT == OUT_F32 || OUT == OUT_I32) {
    // 32-bit outputs (fp32 and int8 operands), plus tt.dot's accumulator
    // operand when given (fp32, or int32 bits for int8: added modulo 2^32)
#pragma unroll
    for (int fm = 0; fm < C::FM; ++fm) {
      const int m = m0 + wm * C::WTM + fm * 16 + frow;
      if (m >= a.M) continue;
#pragma unroll
      for (int fn = 0; fn < C::FN; ++fn) {
        const int n = n0 + wn * C::WTN + fn * 16 + 4 * fg;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (n + j >= a.N) continue;
          const int64_t ci = int64_t(m) * a.ldc + n + j, ai = int64_t(m) * a.ld_acc + n + j;
          if constexpr (OUT == OUT_I32) {
            uint32_t r = __float_as_uint(acc[fn][fm][j]);
            if (a.acc) r += reinterpret_cast<const uint32_t *>(a.acc)[ai];
            static_cast<uint32_t *>(a.C)[ci] = r;
          } else {
            float r = acc[fn][fm][j];
            if (a.acc) r += a.acc[ai];
            static_cast<float *>(a.C)[ci] = r;
          }
        }
      }
    }
    return;
  }
  uint16_t *Cb = reinterpret_cast<uint16_t *>(a.C);
  const bool cvec = ((reinterpret_cast<uintptr_t>(a.C) & 7) == 0) && ((a.ldc & 3) == 0);
#pragma unroll
  for (int fm = 0; fm < C::FM; ++fm) {
    const int m = m0 + wm * C::WTM + fm * 16 + frow;
    if (m >= a.M) continue;
    float sa = 1.0f;
    if constexpr (C::FP8) sa = a.scale_a[m];
#pragma unroll
    for (int fn = 0; fn < C::FN; ++fn) {
      const int n = n0 + wn * C::WTN + fn * 16 + 4 * fg;
      float v[4] = {acc[fn][fm].x, acc[fn][fm].y, acc[fn][fm].z, acc[fn][fm].w};
      if constexpr (C::FP8) {
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = v[j] * sa * (n + j < a.N ? a.scale_b[n + j] : 0.0f);
      }
      if (C::FP8 && a.epi) {  // epilogue requested: scaled fp32 sums to a.part (M x N)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (n + j < a.N) a.part[int64_t(m) * a.N + n + j] = v[j];
      } else {
        uint16_t *dst = Cb + int64_t(m) * a.ldc + n;
        if (cvec && n + 3 < a.N) {
          txd::u32x2 p = OUT == OUT_F16
                             ? txd::u32x2{txd::pack_f16x2(v[0], v[1]), txd::pack_f16x2(v[2], v[3])}
                             : txd::u32x2{txd::pack_bf16x2(v[0], v[1]), txd::pack_bf16x2(v[2], v[3])};
          *reinterpret_cast<txd::u32x2 *>(dst) = p;
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (n + j < a.N)
              dst[j] = OUT == OUT_F16 ? uint16_t(txd::pack_f16x2(v[j], 0.0f))
                                      : uint16_t(txd::f32_to_bf16_bits(v[j]));
        }
      }
    }
  }
}

}  // namespace txg
