// fp32 -> fp8 / fp16 / bf16 integer encoders shared by the codec kernels and
// the GEMM epilogues (rounding rules: see fp8_codec.hip's header).
#pragma once

#include "tx_device.h"

namespace txf {

// Format ids as tx_dtype.
enum { E4M3FN = 1, E5M2 = 2, BF16 = 3, F16 = 6 };

template <int FMT>
struct Fp8Format {
  static constexpr int M = FMT == E4M3FN ? 3 : FMT == E5M2 ? 2 : FMT == BF16 ? 7 : 10;  // mantissa bits
  static constexpr int BIAS = FMT == E4M3FN ? 7 : FMT == BF16 ? 127 : 15;
  static constexpr int W = (FMT == BF16 || FMT == F16) ? 16 : 8;                    // code bits
  static constexpr uint32_t MAXC = FMT == E4M3FN ? 0x7Eu : FMT == E5M2 ? 0x7Bu : FMT == BF16 ? 0x7F7Fu : 0x7BFFu;
  static constexpr uint32_t OVF = FMT == E4M3FN ? 0x7Fu : FMT == E5M2 ? 0x7Cu : FMT == BF16 ? 0x7F80u : 0x7C00u;
  static constexpr uint32_t NANC = W == 8 ? 0x7Fu : FMT == BF16 ? 0x7FC0u : 0x7E00u;
  static constexpr int SH = 23 - M;                           // dropped bits
  static constexpr uint32_t MIN_NORM_BITS = uint32_t(128 - BIAS) << 23;
  static constexpr uint32_t REBIAS = uint32_t(127 - BIAS) << 23;
  static constexpr uint32_t MAGIC_BITS = uint32_t(127 + 24 - BIAS - M) << 23;
  static __device__ __forceinline__ uint32_t sign(uint32_t u) { return (u >> (32 - W)) & (1u << (W - 1)); }
};

// fp32 bits -> fp8 code, round to nearest even.
template <int FMT, bool SAT>
__device__ __forceinline__ uint32_t encode_rtne(uint32_t u) {
  using F = Fp8Format<FMT>;
  const uint32_t a = u & 0x7FFFFFFFu;
  const uint32_t lsb = (a >> F::SH) & 1u;
  const uint32_t nrm = (a - F::REBIAS + ((1u << (F::SH - 1)) - 1u) + lsb) >> F::SH;
  const float f = __uint_as_float(a) + __uint_as_float(F::MAGIC_BITS);
  const uint32_t sub = __float_as_uint(f) - F::MAGIC_BITS;
  uint32_t code = (a < F::MIN_NORM_BITS) ? sub : nrm;
  code = min(code, SAT ? F::MAXC : F::OVF);
  code = (a > 0x7F800000u) ? F::NANC : code;
  return code | F::sign(u);
}

// fp32 bits -> fp8 code, round toward zero.
template <int FMT, bool SAT>
__device__ __forceinline__ uint32_t encode_rtz(uint32_t u) {
  using F = Fp8Format<FMT>;
  const uint32_t a = u & 0x7FFFFFFFu;
  const uint32_t nrm = (a - F::REBIAS) >> F::SH;
  const uint32_t e = a >> 23;
  const uint32_t sig = (a & 0x7FFFFFu) | (e ? 0x800000u : 0u);
  const uint32_t s = uint32_t(151 - F::BIAS - F::M) - (e ? e : 1u);
  const uint32_t sub = (s > 31u) ? 0u : (sig >> s);
  uint32_t code = (a < F::MIN_NORM_BITS) ? sub : nrm;
  code = min(code, F::MAXC);  // finite values never round away from zero
  if (a == 0x7F800000u) code = SAT ? F::MAXC : F::OVF;
  if (a > 0x7F800000u) code = F::NANC;
  return code | F::sign(u);
}

// Four fp32 values already clamped to +-max (NaN allowed) -> four fp8 codes
// (byte i = value i), round to nearest even, with gfx950's packed convert
// instructions.  Over all 2^32 fp32 patterns clamped to +-max they return
// encode_rtne's codes (checked exhaustively on the device); NaN inputs are
// set to encode_rtne's NaN code (0x7F with the input's sign) explicitly.
template <int FMT>
__device__ __forceinline__ uint32_t encode_clamped4_hw(const float (&x)[4]) {
  static_assert(FMT == E4M3FN || FMT == E5M2, "fp8 formats");
  int w;
  if constexpr (FMT == E4M3FN) {
    w = __builtin_amdgcn_cvt_pk_fp8_f32(x[0], x[1], 0, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(x[2], x[3], w, true);
  } else {
    w = __builtin_amdgcn_cvt_pk_bf8_f32(x[0], x[1], 0, false);
    w = __builtin_amdgcn_cvt_pk_bf8_f32(x[2], x[3], w, true);
  }
  uint32_t c = uint32_t(w);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (x[i] != x[i]) {
      const uint32_t nanc = 0x7Fu | ((__float_as_uint(x[i]) >> 24) & 0x80u);
      c = (c & ~(0xFFu << (8 * i))) | (nanc << (8 * i));
    }
  }
  return c;
}

}  // namespace txf
