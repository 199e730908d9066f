// tt.fp_to_fp for fp32 <-> fp8 (OCP E4M3FN and E5M2) on gfx950.
//
// Streaming kernels: every load is a 128-bit, wave-contiguous global load and
// every store is wave-contiguous, so each wave instruction moves whole cache
// lines.  The conversion from or to fp32 is integer bit manipulation on the
// fp32 encoding, so the rounding, saturation and NaN rules are exactly the
// ones written here.  Between bf16 / fp16 and fp8 (round to nearest even,
// and every fp8 -> 16-bit decode) the finite values take gfx950's packed
// fp8 conversions, which give the same codes as these encoders for every
// 16-bit source value, and the special values are set explicitly to what
// the encoders give (fp8x4_to_16, f16x4_to_fp8_rtne):
//
//  encode (fp32 -> fp8), round to nearest even:
//   * normal range (|x| >= 2^(1-bias)): re-bias the fp32 exponent field to
//     the fp8 bias, add half an fp8 ulp minus one plus the lowest kept bit
//     (ties-to-even), and keep the top bits.  A carry out of the mantissa
//     moves into the exponent field by itself.
//   * subnormal range: add the power of two 2^k whose fp32 ulp equals the fp8
//     subnormal quantum 2^(1-bias-m) (k = 24 - bias - m); the fp32 adder
//     rounds to nearest even at exactly that position, and the low bits of
//     the sum are the fp8 code (the 'magic number' method of rounding by
//     addition).  fp32 denormal inputs round to zero with either denormal
//     mode.
//   * overflow: codes above the largest finite code are clamped to max
//     (saturating, and round-toward-zero) or to the overflow code (NaN 0x7F
//     for e4m3fn, Inf 0x7C for e5m2); NaN input gives 0x7F; the sign bit is
//     OR-ed in last.
//  decode (fp8 -> fp32), exact: normal codes are re-biased by a shift and an
//  add; subnormal codes are mant * 2^(1-bias-m), computed as an exact
//  int->float conversion times a power of two; NaN codes give 0x7FC00000
//  and e5m2 Inf codes give Inf, each with the code's sign.
//
// The same integer encoders, with the format's parameters, also produce
// fp16 and bf16 (fp16: quantum 2^-24 below 2^-14; bf16: fp32's exponent
// range, so only fp32 denormals take the subnormal path).  fp16 / bf16 NaN
// outputs are the canonical quiet NaN (0x7E00 / 0x7FC0) with the input's
// sign.
//
//  stochastic rounding (rounding "rs", fp32 source, one 32-bit word r of
//  random bits per element, always saturating): the round-toward-zero code,
//  moved one step away from zero iff r + floor(frac * 2^32) carries out of
//  32 bits, frac being the dropped fraction of an ulp.  frac * 2^32 is read
//  straight off the dropped bits: in the normal range they are the low
//  23 - m bits of the fp32 encoding, in the subnormal range the low s bits
//  of the 24-bit significand (s bits below the quantum).  Codes at max,
//  +-Inf and |x| above max give +-max; NaN gives NaN.
//
// Semantics follow tt.fp_to_fp (semantic.py:807-827, default RTNE at :809;
// rounding operand 0 rtne, 1 rtz, 2 rs with random bits,
// createFpToFpWithRbits at ops/NewOps.cpp:249-303) and the reference's
// saturating idiom clamp-then-convert (mxfp8_utils.py:17-21, 36-38).
#include "fp8_encode.h"
#include "tx_device.h"

namespace {

using namespace txf;

// fp32 bits -> code, stochastic rounding with random word r (saturating).
template <int FMT>
__device__ __forceinline__ uint32_t round_rs(uint32_t u, uint32_t r) {
  using F = Fp8Format<FMT>;
  const uint32_t a = u & 0x7FFFFFFFu;
  const uint32_t code = encode_rtz<FMT, true>(u) & ~(1u << (F::W - 1));
  // floor(frac * 2^32) from the dropped bits
  uint32_t thr;
  if (a >= F::MIN_NORM_BITS) {
    thr = (a & ((1u << F::SH) - 1u)) << (32 - F::SH);
  } else {
    const uint32_t e = a >> 23;
    const uint64_t sig = (a & 0x7FFFFFu) | (e ? 0x800000u : 0u);
    const uint32_t s = uint32_t(151 - F::BIAS - F::M) - (e ? e : 1u);  // >= 24 - M
    thr = s <= 32u ? uint32_t((sig & ((uint64_t(1) << s) - 1u)) << (32u - s))
                   : (s - 32u < 24u ? uint32_t(sig >> (s - 32u)) : 0u);
  }
  const bool up = (uint64_t(r) + thr) >> 32 != 0 && code < F::MAXC && a < 0x7F800000u;
  return (code + (up ? 1u : 0u)) | F::sign(u);
}

template <int FMT, bool SAT, bool RTZ>
__device__ __forceinline__ uint32_t encode(uint32_t u) {
  if constexpr (RTZ) return encode_rtz<FMT, SAT>(u);
  else return encode_rtne<FMT, SAT>(u);
}

// fp8 code (0..255) -> fp32 bits, exact.
template <int FMT>
__device__ __forceinline__ uint32_t decode(uint32_t c) {
  using F = Fp8Format<FMT>;
  const uint32_t mag = c & 0x7Fu;
  const uint32_t nrm = (mag << F::SH) + F::REBIAS;
  // subnormal quantum 2^(1-bias-m) as fp32 bits
  constexpr uint32_t QBITS = uint32_t(127 + 1 - F::BIAS - F::M) << 23;
  const uint32_t sub = __float_as_uint(float(mag) * __uint_as_float(QBITS));
  uint32_t r = (mag < (1u << F::M)) ? sub : nrm;
  if constexpr (FMT == E4M3FN) {
    r = (mag == 0x7Fu) ? 0x7FC00000u : r;
  } else {
    r = (mag >= 0x7Cu) ? ((mag == 0x7Cu) ? 0x7F800000u : 0x7FC00000u) : r;
  }
  return r | ((c & 0x80u) << 24);
}

constexpr int kBlock = 256;
constexpr int kVecPerThread = 4;                         // float4 loads per thread
constexpr int kChunk = kBlock * kVecPerThread * 4;       // elements per block step

// Four fp32 values -> four fp8 codes (code i in byte i), round to nearest
// even, not saturating, by gfx950's packed converts: without clamping,
// v_cvt_pk_fp8_f32 / v_cvt_pk_bf8_f32 give exactly encode_rtne<FMT, false>'s
// code for every fp32 input that is not a NaN (a device sweep over all 2^32
// patterns found no difference: ties, subnormals, overflow to NaN / Inf and
// Inf included).  NaN inputs differ: e4m3fn gives 0xFF for every NaN (0x7F |
// sign wanted), so positive NaNs are first replaced by +Inf, whose code is
// 0x7F (a signed min with 0x7F800000 leaves every other pattern alone);
// e5m2 gives 0xFE for every NaN, a code no other input produces, so those
// bytes are rewritten to 0x7F | the input's sign.
template <int FMT>
__device__ __forceinline__ uint32_t encode4_rtne_hw(const txd::u32x4 &v) {
  if constexpr (FMT == E4M3FN) {
    auto fix = [](uint32_t u) { return __int_as_float(min(int(u), 0x7F800000)); };
    int w = __builtin_amdgcn_cvt_pk_fp8_f32(fix(v.x), fix(v.y), 0, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(fix(v.z), fix(v.w), w, true);
    return uint32_t(w);
  } else {
    int w = __builtin_amdgcn_cvt_pk_bf8_f32(__uint_as_float(v.x), __uint_as_float(v.y), 0, false);
    w = __builtin_amdgcn_cvt_pk_bf8_f32(__uint_as_float(v.z), __uint_as_float(v.w), w, true);
    const uint32_t t = uint32_t(w) ^ 0xFEFEFEFEu;                      // zero bytes: NaN inputs
    // bit 7 of each zero byte of t; the borrow can also flag a byte of t equal
    // to 0x01 above a zero byte, i.e. a code 0xFF, which the converter never
    // gives (a NaN gives 0xFE, every other input its encode_rtne code)
    const uint32_t nan7 = (t - 0x01010101u) & ~t & 0x80808080u;
    if (nan7 == 0u) return uint32_t(w);
    // byte i of `sign` holds byte 3 (sign and top exponent bits) of value i
    const uint32_t sign = __builtin_amdgcn_perm(v.y, v.x, 0x0c0c0703u) | __builtin_amdgcn_perm(v.w, v.z, 0x07030c0cu);
    const uint32_t mask = (nan7 >> 7) * 0xFFu;
    return (uint32_t(w) & ~mask) | ((sign & 0x80808080u) | 0x7F7F7F7Fu) & mask;
  }
}

// Vector encode: [start, n) with (n - start) a multiple of kChunk, src 16-byte
// aligned, dst 4-byte aligned, start a multiple of 4.
template <int FMT, bool SAT, bool RTZ>
__device__ __forceinline__ void encode_vec(const tx_fp8_codec_args &a) {
  const txd::u32x4 *src = reinterpret_cast<const txd::u32x4 *>(a.src) + a.start / 4;
  uint32_t *dst = reinterpret_cast<uint32_t *>(a.dst) + a.start / 4;
  const int64_t nchunks = (a.n - a.start) / kChunk;
  for (int64_t c = blockIdx.x; c < nchunks; c += gridDim.x) {
    const int64_t w0 = c * (kChunk / 4) + threadIdx.x;
    txd::u32x4 v[kVecPerThread];
#pragma unroll
    for (int j = 0; j < kVecPerThread; ++j)
      v[j] = __builtin_nontemporal_load(src + w0 + j * kBlock);
#pragma unroll
    for (int j = 0; j < kVecPerThread; ++j) {
      if constexpr (!SAT && !RTZ) {
        __builtin_nontemporal_store(encode4_rtne_hw<FMT>(v[j]), dst + w0 + j * kBlock);
      } else {
        const uint32_t b0 = encode<FMT, SAT, RTZ>(v[j].x);
        const uint32_t b1 = encode<FMT, SAT, RTZ>(v[j].y);
        const uint32_t b2 = encode<FMT, SAT, RTZ>(v[j].z);
        const uint32_t b3 = encode<FMT, SAT, RTZ>(v[j].w);
        __builtin_nontemporal_store(b0 | (b1 << 8) | (b2 << 16) | (b3 << 24), dst + w0 + j * kBlock);
      }
    }
  }
}

template <int FMT, bool SAT, bool RTZ>
__device__ __forceinline__ void encode_tail(const tx_fp8_codec_args &a) {
  const uint32_t *src = reinterpret_cast<const uint32_t *>(a.src);
  uint8_t *dst = reinterpret_cast<uint8_t *>(a.dst);
  for (int64_t i = a.start + int64_t(blockIdx.x) * kBlock + threadIdx.x; i < a.n;
       i += int64_t(gridDim.x) * kBlock)
    dst[i] = uint8_t(encode<FMT, SAT, RTZ>(src[i]));
}

// Vector decode: [start, n) with (n - start) a multiple of kChunk, src 4-byte
// aligned, dst 16-byte aligned, start a multiple of 4.
template <int FMT>
__device__ __forceinline__ void decode_vec(const tx_fp8_codec_args &a) {
  const uint32_t *src = reinterpret_cast<const uint32_t *>(a.src) + a.start / 4;
  txd::u32x4 *dst = reinterpret_cast<txd::u32x4 *>(a.dst) + a.start / 4;
  const int64_t nchunks = (a.n - a.start) / kChunk;
  for (int64_t c = blockIdx.x; c < nchunks; c += gridDim.x) {
    const int64_t w0 = c * (kChunk / 4) + threadIdx.x;
    uint32_t v[kVecPerThread];
#pragma unroll
    for (int j = 0; j < kVecPerThread; ++j)
      v[j] = __builtin_nontemporal_load(src + w0 + j * kBlock);
#pragma unroll
    for (int j = 0; j < kVecPerThread; ++j) {
      txd::u32x4 o;
      o.x = decode<FMT>(v[j] & 0xFFu);
      o.y = decode<FMT>((v[j] >> 8) & 0xFFu);
      o.z = decode<FMT>((v[j] >> 16) & 0xFFu);
      o.w = decode<FMT>(v[j] >> 24);
      __builtin_nontemporal_store(o, dst + w0 + j * kBlock);
    }
  }
}

template <int FMT>
__device__ __forceinline__ void decode_tail(const tx_fp8_codec_args &a) {
  const uint8_t *src = reinterpret_cast<const uint8_t *>(a.src);
  uint32_t *dst = reinterpret_cast<uint32_t *>(a.dst);
  for (int64_t i = a.start + int64_t(blockIdx.x) * kBlock + threadIdx.x; i < a.n;
       i += int64_t(gridDim.x) * kBlock)
    dst[i] = decode<FMT>(src[i]);
}

// fp32 bits -> code of format FMT; MODE 0 rtne, 1 rtz, 2 rs (r random bits).
template <int FMT, int MODE, bool SAT>
__device__ __forceinline__ uint32_t convert(uint32_t u, uint32_t r) {
  if constexpr (MODE == 2) return round_rs<FMT>(u, r);
  else if constexpr (MODE == 1) return encode_rtz<FMT, SAT>(u);
  else return encode_rtne<FMT, SAT>(u);
}

// Vector conversion: [start, n) with (n - start) a multiple of kChunk, src
// (and for rs the random bits) 16-byte aligned, dst 4-byte (8-bit codes) or
// 8-byte (16-bit codes) aligned, start a multiple of 4.
template <int FMT, int MODE, bool SAT>
__device__ __forceinline__ void cvt_vec(const tx_fp8_codec_args &a) {
  using F = Fp8Format<FMT>;
  const txd::u32x4 *src = reinterpret_cast<const txd::u32x4 *>(a.src) + a.start / 4;
  const txd::u32x4 *rb = reinterpret_cast<const txd::u32x4 *>(a.rbits) + a.start / 4;
  const int64_t nchunks = (a.n - a.start) / kChunk;
  for (int64_t c = blockIdx.x; c < nchunks; c += gridDim.x) {
    const int64_t w0 = c * (kChunk / 4) + threadIdx.x;
    txd::u32x4 v[kVecPerThread], r[kVecPerThread];
#pragma unroll
    for (int j = 0; j < kVecPerThread; ++j) {
      v[j] = __builtin_nontemporal_load(src + w0 + j * kBlock);
      if constexpr (MODE == 2) r[j] = __builtin_nontemporal_load(rb + w0 + j * kBlock);
      else r[j] = txd::u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int j = 0; j < kVecPerThread; ++j) {
      const uint32_t c0 = convert<FMT, MODE, SAT>(v[j].x, r[j].x);
      const uint32_t c1 = convert<FMT, MODE, SAT>(v[j].y, r[j].y);
      const uint32_t c2 = convert<FMT, MODE, SAT>(v[j].z, r[j].z);
      const uint32_t c3 = convert<FMT, MODE, SAT>(v[j].w, r[j].w);
      if constexpr (F::W == 8) {
        uint32_t *dst = reinterpret_cast<uint32_t *>(a.dst) + a.start / 4;
        __builtin_nontemporal_store(c0 | (c1 << 8) | (c2 << 16) | (c3 << 24), dst + w0 + j * kBlock);
      } else {
        txd::u32x2 *dst = reinterpret_cast<txd::u32x2 *>(a.dst) + a.start / 4;
        __builtin_nontemporal_store(txd::u32x2{c0 | (c1 << 16), c2 | (c3 << 16)}, dst + w0 + j * kBlock);
      }
    }
  }
}

template <int FMT, int MODE, bool SAT>
__device__ __forceinline__ void cvt_tail(const tx_fp8_codec_args &a) {
  using F = Fp8Format<FMT>;
  const uint32_t *src = reinterpret_cast<const uint32_t *>(a.src);
  for (int64_t i = a.start + int64_t(blockIdx.x) * kBlock + threadIdx.x; i < a.n;
       i += int64_t(gridDim.x) * kBlock) {
    const uint32_t code = convert<FMT, MODE, SAT>(src[i], MODE == 2 ? a.rbits[i] : 0u);
    if constexpr (F::W == 8) reinterpret_cast<uint8_t *>(a.dst)[i] = uint8_t(code);
    else reinterpret_cast<uint16_t *>(a.dst)[i] = uint16_t(code);
  }
}

// ------------------------------------ conversions between any two formats
// Source codes of fp32 (bits), bf16, fp16, e4m3fn or e5m2 widen to fp32
// exactly (every bf16, fp16 and fp8 value is an fp32 value), then take the
// encoders above, so each result is the source value rounded once.
constexpr int F32 = 0;  // tx_dtype of fp32

template <int T>
struct Bytes {
  static constexpr int v = T == F32 ? 4 : (T == BF16 || T == F16) ? 2 : 1;
};

// code -> fp32 bits, exact.  fp16: normal codes re-biased (exponent + 112),
// subnormal codes mant * 2^-24 (an exact int -> float conversion times a
// power of two), Inf / NaN kept (NaN stays NaN).
template <int SRC>
__device__ __forceinline__ uint32_t widen(uint32_t c) {
  if constexpr (SRC == F32) {
    return c;
  } else if constexpr (SRC == BF16) {
    return c << 16;
  } else if constexpr (SRC == F16) {
    const uint32_t e = (c >> 10) & 0x1Fu, m = c & 0x3FFu;
    const uint32_t nrm = ((e + 112u) << 23) | (m << 13);
    const uint32_t sub = __float_as_uint(float(m) * 0x1p-24f);
    const uint32_t r = e == 0u ? sub : (e == 31u ? (0x7F800000u | (m << 13)) : nrm);
    return r | ((c & 0x8000u) << 16);
  } else {
    return decode<SRC>(c);
  }
}

// fp32 bits -> code of DST (fp32: the bits), MODE 0 rtne, 1 rtz.
template <int DST, int MODE, bool SAT>
__device__ __forceinline__ uint32_t narrow(uint32_t u) {
  if constexpr (DST == F32) return u;
  else if constexpr (MODE == 1) return encode_rtz<DST, SAT>(u);
  else return encode_rtne<DST, SAT>(u);
}

template <int B> struct Unit;  // a B-byte memory access
template <> struct Unit<4> { using T = uint32_t; };
template <> struct Unit<8> { using T = txd::u32x2; };
template <> struct Unit<16> { using T = txd::u32x4; };

template <int B>
__device__ __forceinline__ void unit_words(const typename Unit<B>::T &v, uint32_t (&w)[4]) {
  if constexpr (B == 4) { w[0] = v; w[1] = w[2] = w[3] = 0u; }
  else if constexpr (B == 8) { w[0] = v.x; w[1] = v.y; w[2] = w[3] = 0u; }
  else { w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w; }
}
template <int B>
__device__ __forceinline__ typename Unit<B>::T words_unit(const uint32_t (&w)[4]) {
  if constexpr (B == 4) return w[0];
  else if constexpr (B == 8) return txd::u32x2{w[0], w[1]};
  else return txd::u32x4{w[0], w[1], w[2], w[3]};
}

// fp8 -> bf16 / fp16 for the four codes of one word: every fp8 value is a
// bf16 and an fp16 value, so no rounding mode matters.  Finite codes go
// through gfx950's packed fp8 -> fp32 conversion (exact) and keep the top
// half of the fp32 bits (bf16) or convert to fp16 (exact, so truncation
// is as good as rounding); e5m2 -> fp16 is byte placement (e5m2 is the top
// byte of fp16).  Inf and NaN codes are then set to the encoders' results:
// NaN to the format's NaN code with the sign, e5m2 Inf to Inf, or to the
// largest finite value when saturating.  Out: o[0] = values 0, 1, o[1] =
// values 2, 3.
template <int SRC, int DST, bool SAT>
__device__ __forceinline__ void fp8x4_to_16(uint32_t w, uint32_t (&o)[2]) {
  using FD = Fp8Format<DST>;
  if constexpr (SRC == E5M2 && DST == F16) {
    o[0] = __builtin_amdgcn_perm(0u, w, 0x010c000cu);  // b1 << 24 | b0 << 8
    o[1] = __builtin_amdgcn_perm(0u, w, 0x030c020cu);  // b3 << 24 | b2 << 8
  } else {
    const auto lo = SRC == E4M3FN ? __builtin_amdgcn_cvt_pk_f32_fp8(int(w), false)
                                  : __builtin_amdgcn_cvt_pk_f32_bf8(int(w), false);
    const auto hi = SRC == E4M3FN ? __builtin_amdgcn_cvt_pk_f32_fp8(int(w), true)
                                  : __builtin_amdgcn_cvt_pk_f32_bf8(int(w), true);
    if constexpr (DST == BF16) {
      o[0] = __builtin_amdgcn_perm(__float_as_uint(lo[1]), __float_as_uint(lo[0]), 0x07060302u);
      o[1] = __builtin_amdgcn_perm(__float_as_uint(hi[1]), __float_as_uint(hi[0]), 0x07060302u);
    } else {
      o[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo[0], lo[1]));
      o[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(hi[0], hi[1]));
    }
  }
  constexpr uint32_t SPEC = SRC == E4M3FN ? 0x7Fu : 0x7Cu;  // magnitude bits set in Inf / NaN codes
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t c = (w >> (8 * j)) & 0xFFu;
    const uint32_t mag = c & 0x7Fu;
    const uint32_t inf = SAT ? FD::MAXC : FD::OVF;
    const uint32_t sv = ((SRC == E5M2 && mag == 0x7Cu) ? inf : FD::NANC) | ((c & 0x80u) << 8);
    const int sh = 16 * (j & 1);
    uint32_t &r = o[j >> 1];
    r = (mag & SPEC) == SPEC ? (r & ~(0xFFFFu << sh)) | (sv << sh) : r;
  }
}

// bf16 / fp16 -> fp8, round to nearest even, for the four values of two
// words: the values widen to fp32 exactly and, clamped to the format's
// largest finite value, take gfx950's packed conversion, which returns
// encode_rtne's codes for every clamped bf16 / fp16 value (the conversion
// tests run every 16-bit source code).  What clamping changes is set explicitly, as
// encode_rtne has it: NaN to the NaN code with the sign; without
// saturation, magnitudes that round past the largest finite value (above
// 464 for e4m3fn: the tie at 464 goes to the even 448; from 61440 up for
// e5m2: the tie between 57344 and 65536 goes to the even 65536, which
// overflows) to the overflow code (NaN / Inf) with the sign.
template <int SRC, int DST, bool SAT>
__device__ __forceinline__ uint32_t f16x4_to_fp8_rtne(uint32_t w0, uint32_t w1) {
  using F = Fp8Format<DST>;
  float x[4];
  if constexpr (SRC == BF16) {
    x[0] = __uint_as_float(w0 << 16);
    x[1] = __uint_as_float(w0 & 0xFFFF0000u);
    x[2] = __uint_as_float(w1 << 16);
    x[3] = __uint_as_float(w1 & 0xFFFF0000u);
  } else {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 a = __builtin_bit_cast(h2, w0), b = __builtin_bit_cast(h2, w1);
    x[0] = float(a[0]);
    x[1] = float(a[1]);
    x[2] = float(b[0]);
    x[3] = float(b[1]);
  }
  constexpr float FMAX = DST == E4M3FN ? 448.0f : 57344.0f;
  float c[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) c[i] = fminf(fmaxf(x[i], -FMAX), FMAX);
  int p;
  if constexpr (DST == E4M3FN) {
    p = __builtin_amdgcn_cvt_pk_fp8_f32(c[0], c[1], 0, false);
    p = __builtin_amdgcn_cvt_pk_fp8_f32(c[2], c[3], p, true);
  } else {
    p = __builtin_amdgcn_cvt_pk_bf8_f32(c[0], c[1], 0, false);
    p = __builtin_amdgcn_cvt_pk_bf8_f32(c[2], c[3], p, true);
  }
  uint32_t code = uint32_t(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t s = (__float_as_uint(x[i]) >> 24) & 0x80u;
    const float m = fabsf(x[i]);
    const bool ovf = !SAT && (DST == E4M3FN ? m > 464.0f : m >= 61440.0f);
    const bool nan = x[i] != x[i];
    const uint32_t v = (nan ? F::NANC : F::OVF) | s;
    code = (nan || ovf) ? (code & ~(0xFFu << (8 * i))) | (v << (8 * i)) : code;
  }
  return code;
}

// One unit of E elements: the source unit's words in, the destination
// unit's words out.
template <int SRC, int DST, int MODE, bool SAT, int E>
__device__ __forceinline__ void cvt_unit(const uint32_t (&w)[4], uint32_t (&o)[4]) {
  if constexpr ((SRC == BF16 || SRC == F16) && (DST == E4M3FN || DST == E5M2) && MODE == 0) {
    static_assert(E == 8, "16 bytes in, 8 codes out");
    o[0] = f16x4_to_fp8_rtne<SRC, DST, SAT>(w[0], w[1]);
    o[1] = f16x4_to_fp8_rtne<SRC, DST, SAT>(w[2], w[3]);
    o[2] = o[3] = 0u;
    return;
  }
  if constexpr ((SRC == E4M3FN || SRC == E5M2) && (DST == BF16 || DST == F16)) {
    static_assert(E == 8, "8 codes in, 16 bytes out");
    uint32_t h[2];
    fp8x4_to_16<SRC, DST, SAT>(w[0], h);
    o[0] = h[0];
    o[1] = h[1];
    fp8x4_to_16<SRC, DST, SAT>(w[1], h);
    o[2] = h[0];
    o[3] = h[1];
    return;
  }
  constexpr int S = Bytes<SRC>::v, D = Bytes<DST>::v;
  constexpr uint32_t SM = S == 4 ? 0xFFFFFFFFu : (1u << (8 * S)) - 1u;
  constexpr uint32_t DM = D == 4 ? 0xFFFFFFFFu : (1u << (8 * D)) - 1u;
  o[0] = o[1] = o[2] = o[3] = 0u;
#pragma unroll
  for (int i = 0; i < E; ++i) {
    const uint32_t c = (w[(i * S) / 4] >> (8 * ((i * S) % 4))) & SM;
    const uint32_t y = narrow<DST, MODE, SAT>(widen<SRC>(c)) & DM;
    o[(i * D) / 4] |= y << (8 * ((i * D) % 4));
  }
}

// Chunks per block step of the generic vector conversion: two where a value
// moves 3 bytes or fewer, so every lane keeps at least 64 bytes of loads
// and stores in flight (the host sizes its vector range to match).
template <int SRC, int DST>
struct Steps {
  static constexpr int v = Bytes<SRC>::v + Bytes<DST>::v <= 3 ? 2 : 1;
};

// Vector conversion: [start, n) with (n - start) a multiple of R * kChunk.
// Each thread converts 16 * R elements per block step in units of
// E = 16 / max(S, D) elements, so the wider side of the conversion moves 16
// bytes per lane and both sides are wave-contiguous; src aligned to E * S
// bytes, dst to E * D bytes.  All loads of a step are issued before the
// first conversion.
template <int SRC, int DST, int MODE, bool SAT, int R = Steps<SRC, DST>::v>
__device__ __forceinline__ void cvt2_vec(const tx_fp8_codec_args &a) {
  constexpr int S = Bytes<SRC>::v, D = Bytes<DST>::v;
  constexpr int E = 16 / (S > D ? S : D), U = 16 / E;  // elements per unit, units per chunk
  constexpr int LB = E * S, SB = E * D;
  static_assert(kBlock * U * E == kChunk, "16 elements per thread and chunk");
  using LT = typename Unit<LB>::T;
  using ST = typename Unit<SB>::T;
  const LT *src = reinterpret_cast<const LT *>(static_cast<const uint8_t *>(a.src) + a.start * S);
  ST *dst = reinterpret_cast<ST *>(static_cast<uint8_t *>(a.dst) + a.start * D);
  const int64_t nsteps = (a.n - a.start) / (int64_t(R) * kChunk);
  for (int64_t c = blockIdx.x; c < nsteps; c += gridDim.x) {
    const int64_t w0 = c * (kBlock * U * R) + threadIdx.x;
    LT v[U * R];
#pragma unroll
    for (int u = 0; u < U * R; ++u) v[u] = __builtin_nontemporal_load(src + w0 + u * kBlock);
#pragma unroll
    for (int u = 0; u < U * R; ++u) {
      uint32_t w[4], o[4];
      unit_words<LB>(v[u], w);
      cvt_unit<SRC, DST, MODE, SAT, E>(w, o);
      __builtin_nontemporal_store(words_unit<SB>(o), dst + w0 + u * kBlock);
    }
  }
}

template <int SRC, int DST, int MODE, bool SAT>
__device__ __forceinline__ void cvt2_tail(const tx_fp8_codec_args &a) {
  constexpr int S = Bytes<SRC>::v, D = Bytes<DST>::v;
  const uint8_t *src = static_cast<const uint8_t *>(a.src);
  uint8_t *dst = static_cast<uint8_t *>(a.dst);
  for (int64_t i = a.start + int64_t(blockIdx.x) * kBlock + threadIdx.x; i < a.n;
       i += int64_t(gridDim.x) * kBlock) {
    uint32_t c;
    if constexpr (S == 4) c = reinterpret_cast<const uint32_t *>(src)[i];
    else if constexpr (S == 2) c = reinterpret_cast<const uint16_t *>(src)[i];
    else c = src[i];
    const uint32_t y = narrow<DST, MODE, SAT>(widen<SRC>(c));
    if constexpr (D == 4) reinterpret_cast<uint32_t *>(dst)[i] = y;
    else if constexpr (D == 2) reinterpret_cast<uint16_t *>(dst)[i] = uint16_t(y);
    else dst[i] = uint8_t(y);
  }
}

// ----------------------------------------------------------- quantisers
// x element i of a row as fp32 (XT 0: fp32, 1: bf16 bits).
template <int XT>
__device__ __forceinline__ float load_x(const void *row, int64_t i) {
  if constexpr (XT == 0) return static_cast<const float *>(row)[i];
  else return __uint_as_float(uint32_t(static_cast<const uint16_t *>(row)[i]) << 16);
}

// max(m, |v|) ignoring a NaN v (a comparison with NaN is false, for quiet
// and signalling NaNs alike).
__device__ __forceinline__ float absmax_step(float m, float v) {
  const float a = fabsf(v);
  return a > m ? a : m;
}

// clamp(v, -max, max) with NaN kept (comparisons with NaN are false).
template <int FMT>
__device__ __forceinline__ float clamp_keep_nan(float v) {
  constexpr float FMAX = FMT == E4M3FN ? 448.0f : 57344.0f;
  return v > FMAX ? FMAX : (v < -FMAX ? -FMAX : v);
}

// Lanes per 32-element block of the MX quantiser: 4 for fp32 input (8
// elements, two 16-byte loads each), 2 for bf16 (16 elements, two 16-byte
// loads: four lanes of 8 bf16 moved half as many bytes per instruction, and
// that path ran at 0.58 of HBM against the fp32 one's 0.69).
template <int XT>
constexpr int MxLanes = XT == 0 ? 4 : 2;

// One thread's E = 32 / MxLanes elements of a block.
template <int XT>
__device__ __forceinline__ void mx_load(const tx_quant_args &a, int64_t t, int64_t nb, float (&v)[32 / MxLanes<XT>]) {
  constexpr int L = MxLanes<XT>, E = 32 / L;
  const int64_t blk = t / L;
  const int64_t r = blk / nb;
  const int64_t col = (blk % nb) * 32 + (t % L) * E;
  const uint8_t *xrow = static_cast<const uint8_t *>(a.x) + r * a.ldx * (XT == 0 ? 4 : 2);
  if (a.vec) {
    if constexpr (XT == 0) {
      const txd::f32x4 p0 = *reinterpret_cast<const txd::f32x4 *>(xrow + 4 * col);
      const txd::f32x4 p1 = *reinterpret_cast<const txd::f32x4 *>(xrow + 4 * col + 16);
      v[0] = p0.x; v[1] = p0.y; v[2] = p0.z; v[3] = p0.w;
      v[4] = p1.x; v[5] = p1.y; v[6] = p1.z; v[7] = p1.w;
    } else {
      const txd::u32x4 p0 = *reinterpret_cast<const txd::u32x4 *>(xrow + 2 * col);
      const txd::u32x4 p1 = *reinterpret_cast<const txd::u32x4 *>(xrow + 2 * col + 16);
      const uint32_t w[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        v[2 * i] = __uint_as_float(w[i] << 16);
        v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < E; ++i) v[i] = load_x<XT>(xrow, col + i);
  }
}

// Block amax over the block's lanes, the e8m0 scale, codes, stores.
template <int FMT, int XT>
__device__ __forceinline__ void mx_store(const tx_quant_args &a, int64_t t, int64_t nb, const float (&v)[32 / MxLanes<XT>]) {
  constexpr int L = MxLanes<XT>, E = 32 / L;
  constexpr float FMAX = FMT == E4M3FN ? 448.0f : 57344.0f;
  const int64_t blk = t / L;
  const int64_t r = blk / nb, cb = blk % nb;
  const int64_t col = cb * 32 + (t % L) * E;
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < E; ++i) amax = absmax_step(amax, v[i]);
#pragma unroll
  for (int o = 1; o < L; o <<= 1) amax = absmax_step(amax, __shfl_xor(amax, o));
  const float descale = amax / FMAX;
  const uint32_t e = ((__float_as_uint(descale) + 0x007FFFFFu) & 0x7F800000u) >> 23;
  const float rounded = __uint_as_float(e << 23);
  const float quant = e == 0 ? 0.0f : 1.0f / rounded;
  uint32_t code[E / 4];
#pragma unroll
  for (int k = 0; k < E / 4; ++k) {
    float c[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) c[i] = clamp_keep_nan<FMT>(v[4 * k + i] * quant);
    code[k] = encode_clamped4_hw<FMT>(c);
  }
  uint8_t *qrow = a.q + r * a.ldq;
  if (a.vec) {
#pragma unroll
    for (int k = 0; k < E / 8; ++k)
      *reinterpret_cast<txd::u32x2 *>(qrow + col + 8 * k) = txd::u32x2{code[2 * k], code[2 * k + 1]};
  } else {
#pragma unroll
    for (int i = 0; i < E; ++i) qrow[col + i] = uint8_t((code[i / 4] >> (8 * (i % 4))) & 0xFFu);
  }
  if (t % L == 0) static_cast<uint8_t *>(a.scales)[r * a.ld_s + cb] = uint8_t(e);
}

// MX quantiser, following the reference's _compute_scale_and_quantize
// (mxfp8_utils.py:17-38) for each block of 32 consecutive elements of a row:
//   amax     = max |x| over the block, NaN ignored (tl.max combines with
//              tl.maximum, whose default propagate_nan is NONE)
//   descale  = amax / fmax (fp32, rounded to nearest)
//   e        = ((bits(descale) + 0x007FFFFF) & 0x7F800000) >> 23   -> the e8m0 scale
//   q        = fp8_rne(clamp(x * (1 / 2^(e-127)), +-fmax))  (x * 0 when e = 0;
//              NaN inputs stay NaN), converted by encode_clamped4_hw
// MxLanes<XT> lanes share a block; the block's amax is combined with one
// (bf16) or two (fp32) lane exchanges.  (Taking two or four blocks per trip,
// their loads issued together, measured 7-16% slower at 8192 x 8192.)
template <int FMT, int XT>
__device__ __forceinline__ void quant_mx(const tx_quant_args &a) {
  constexpr int L = MxLanes<XT>;
  const int64_t nb = a.K / 32;
  const int64_t total = a.rows * nb * L;
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  // total and stride are multiples of L, so the lanes of a block are always
  // active together
  for (int64_t t0 = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; t0 < total; t0 += stride) {
    float v[32 / L];
    mx_load<XT>(a, t0, nb, v);
    mx_store<FMT, XT>(a, t0, nb, v);
  }
}

// Codes of the 4 (fp32) or 8 (bf16) elements of one 16-byte x vector,
// stored at q + 4i or q + 8i.
template <int FMT, int XT>
__device__ __forceinline__ void row_codes(const txd::u32x4 &p, float mult, uint8_t *qrow, int64_t i) {
  const uint32_t w[4] = {p.x, p.y, p.z, p.w};
  if constexpr (XT == 0) {
    float y[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) y[j] = clamp_keep_nan<FMT>(__uint_as_float(w[j]) * mult);
    *reinterpret_cast<uint32_t *>(qrow + 4 * i) = encode_clamped4_hw<FMT>(y);
  } else {
    float y0[4], y1[4];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      y0[2 * j] = clamp_keep_nan<FMT>(__uint_as_float(w[j] << 16) * mult);
      y0[2 * j + 1] = clamp_keep_nan<FMT>(__uint_as_float(w[j] & 0xFFFF0000u) * mult);
      y1[2 * j] = clamp_keep_nan<FMT>(__uint_as_float(w[j + 2] << 16) * mult);
      y1[2 * j + 1] = clamp_keep_nan<FMT>(__uint_as_float(w[j + 2] & 0xFFFF0000u) * mult);
    }
    *reinterpret_cast<txd::u32x2 *>(qrow + 8 * i) = txd::u32x2{encode_clamped4_hw<FMT>(y0), encode_clamped4_hw<FMT>(y1)};
  }
}

template <int XT>
__device__ __forceinline__ float vec_absmax(const txd::u32x4 &p, float amax) {
  const uint32_t w[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if constexpr (XT == 0) {
      amax = absmax_step(amax, __uint_as_float(w[j]));
    } else {
      amax = absmax_step(amax, __uint_as_float(w[j] << 16));
      amax = absmax_step(amax, __uint_as_float(w[j] & 0xFFFF0000u));
    }
  }
  return amax;
}

// Workgroup-wide absmax (NaN never enters: absmax_step drops it).
__device__ __forceinline__ float block_absmax(float amax, float *red) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) amax = absmax_step(amax, __shfl_xor(amax, o));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < kBlock / 64; ++w) amax = absmax_step(amax, red[w]);
  __syncthreads();  // red is reused by the next row
  return amax;
}

// Rows of at most RowRegs<XT> 16-byte vectors per thread (fp32: 16, K <=
// 16384; bf16: 4, K <= 8192) stay in registers between the absmax and the
// codes, so each row is read from memory once.  (fp32: 5% faster at 8192 x
// 8192 than a second pass from cache.  bf16 with the fp32 budget of 16
// vectors, 64 registers for 4 used, measured 30% slower than two passes.)
template <int XT>
constexpr int RowRegs = XT == 0 ? 8 : 4;

// Row-wise absmax quantiser (the fp8 GEMM's per-row / per-column scales):
//   amax = max |x| over the row (NaN ignored), 1 if that is 0
//   q = fp8_rne(clamp(x * (fmax / amax), +-fmax)),  scale = amax / fmax
// (fp32 throughout; NaN inputs stay NaN).  One workgroup per row; fp32 rows
// that fit are read once into registers, other rows take a pass for amax
// and a second pass (from cache) for the codes.
template <int FMT, int XT>
__device__ __forceinline__ void quant_row(const tx_quant_args &a) {
  constexpr float FMAX = FMT == E4M3FN ? 448.0f : 57344.0f;
  constexpr int VE = XT == 0 ? 4 : 8;  // elements per 16-byte load
  __shared__ float red[kBlock / 64];
  float *scales = static_cast<float *>(a.scales);
  const int tid = threadIdx.x;
  constexpr int RR = RowRegs<XT>;
  const bool in_regs = a.vec && a.K % VE == 0 && a.K / VE <= int64_t(kBlock) * RR;
  if (in_regs) {
    const int nvec = int(a.K / VE);
    for (int64_t r = blockIdx.x; r < a.rows; r += gridDim.x) {
      const uint8_t *xrow = static_cast<const uint8_t *>(a.x) + r * a.ldx * (XT == 0 ? 4 : 2);
      txd::u32x4 p[RR];
#pragma unroll
      for (int j = 0; j < RR; ++j) {
        const int i = tid + kBlock * j;
        if (i < nvec) p[j] = *reinterpret_cast<const txd::u32x4 *>(xrow + 16 * int64_t(i));
      }
      float amax = 0.0f;
#pragma unroll
      for (int j = 0; j < RR; ++j)
        if (tid + kBlock * j < nvec) amax = vec_absmax<XT>(p[j], amax);
      amax = block_absmax(amax, red);
      if (amax == 0.0f) amax = 1.0f;
      const float mult = FMAX / amax;
      if (tid == 0) scales[r] = amax / FMAX;
      uint8_t *qrow = a.q + r * a.ldq;
#pragma unroll
      for (int j = 0; j < RR; ++j) {
        const int i = tid + kBlock * j;
        if (i < nvec) row_codes<FMT, XT>(p[j], mult, qrow, i);
      }
    }
    return;
  }
  for (int64_t r = blockIdx.x; r < a.rows; r += gridDim.x) {
    const uint8_t *xrow = static_cast<const uint8_t *>(a.x) + r * a.ldx * (XT == 0 ? 4 : 2);
    uint8_t *qrow = a.q + r * a.ldq;
    const int64_t nvec = a.vec ? a.K / VE : 0;
    float amax = 0.0f;
    for (int64_t i = tid; i < nvec; i += kBlock)
      amax = vec_absmax<XT>(*reinterpret_cast<const txd::u32x4 *>(xrow + 16 * i), amax);
    for (int64_t i = nvec * VE + tid; i < a.K; i += kBlock) amax = absmax_step(amax, load_x<XT>(xrow, i));
    amax = block_absmax(amax, red);
    if (amax == 0.0f) amax = 1.0f;
    const float mult = FMAX / amax;
    if (tid == 0) scales[r] = amax / FMAX;
    for (int64_t i = tid; i < nvec; i += kBlock)
      row_codes<FMT, XT>(*reinterpret_cast<const txd::u32x4 *>(xrow + 16 * i), mult, qrow, i);
    for (int64_t i = nvec * VE + tid; i < a.K; i += kBlock)
      qrow[i] = uint8_t(encode_rtne<FMT, false>(__float_as_uint(clamp_keep_nan<FMT>(load_x<XT>(xrow, i) * mult))));
  }
}

}  // namespace

// absmax + fp8 quantisers (MX block scales and row-wise scales).
#define TX_QUANT_KERNELS(FN, FMT, XN, XT)                                                   \
  TX_KERNEL void __launch_bounds__(kBlock) tx_quant_mx_##FN##_##XN(const tx_quant_args a) {  \
    quant_mx<FMT, XT>(a);                                                                   \
  }                                                                                         \
  TX_KERNEL void __launch_bounds__(kBlock) tx_quant_row_##FN##_##XN(const tx_quant_args a) { \
    quant_row<FMT, XT>(a);                                                                  \
  }

TX_QUANT_KERNELS(e4m3fn, E4M3FN, f32, 0)
TX_QUANT_KERNELS(e4m3fn, E4M3FN, bf16, 1)
TX_QUANT_KERNELS(e5m2, E5M2, f32, 0)
TX_QUANT_KERNELS(e5m2, E5M2, bf16, 1)

// fp32 -> fp16 / bf16 (rtne, rtz, saturating or not) and fp32 -> any of the
// four formats with stochastic rounding.
#define TX_CVT_KERNELS(NAME, FMT, MODE, SAT)                                                    \
  TX_KERNEL void __launch_bounds__(kBlock) tx_cvt_f32_##NAME##_vec(const tx_fp8_codec_args a) {  \
    cvt_vec<FMT, MODE, SAT>(a);                                                                 \
  }                                                                                             \
  TX_KERNEL void __launch_bounds__(kBlock) tx_cvt_f32_##NAME##_tail(const tx_fp8_codec_args a) { \
    cvt_tail<FMT, MODE, SAT>(a);                                                                \
  }

TX_CVT_KERNELS(bf16_rtne, BF16, 0, false)
TX_CVT_KERNELS(bf16_rtne_sat, BF16, 0, true)
TX_CVT_KERNELS(bf16_rtz, BF16, 1, false)
TX_CVT_KERNELS(bf16_rtz_sat, BF16, 1, true)
TX_CVT_KERNELS(f16_rtne, F16, 0, false)
TX_CVT_KERNELS(f16_rtne_sat, F16, 0, true)
TX_CVT_KERNELS(f16_rtz, F16, 1, false)
TX_CVT_KERNELS(f16_rtz_sat, F16, 1, true)
TX_CVT_KERNELS(e4m3fn_rs, E4M3FN, 2, true)
TX_CVT_KERNELS(e5m2_rs, E5M2, 2, true)
TX_CVT_KERNELS(bf16_rs, BF16, 2, true)
TX_CVT_KERNELS(f16_rs, F16, 2, true)

#define TX_ENCODE_KERNELS(NAME, FMT, SAT, RTZ)                                      \
  TX_KERNEL void __launch_bounds__(kBlock) tx_fp8_encode_##NAME##_vec(              \
      const tx_fp8_codec_args a) {                                                  \
    encode_vec<FMT, SAT, RTZ>(a);                                                   \
  }                                                                                 \
  TX_KERNEL void __launch_bounds__(kBlock) tx_fp8_encode_##NAME##_tail(             \
      const tx_fp8_codec_args a) {                                                  \
    encode_tail<FMT, SAT, RTZ>(a);                                                  \
  }

TX_ENCODE_KERNELS(e4m3fn_rtne, E4M3FN, false, false)
TX_ENCODE_KERNELS(e4m3fn_rtne_sat, E4M3FN, true, false)
TX_ENCODE_KERNELS(e4m3fn_rtz, E4M3FN, false, true)
TX_ENCODE_KERNELS(e4m3fn_rtz_sat, E4M3FN, true, true)
TX_ENCODE_KERNELS(e5m2_rtne, E5M2, false, false)
TX_ENCODE_KERNELS(e5m2_rtne_sat, E5M2, true, false)
TX_ENCODE_KERNELS(e5m2_rtz, E5M2, false, true)
TX_ENCODE_KERNELS(e5m2_rtz_sat, E5M2, true, true)

// HBM ceiling kernels with the vector encoder's exact shape (block, chunk,
// loads per thread, non-temporal hints, grid), for measurement only
// (txStreamCeiling): the same bytes as the fp32 -> fp8 encode with no
// conversion work.  copy41 stores each value's low byte (4 B read, 1 B
// written per value); read loads every value and stores one word per
// thread only if the XOR of its 16 words is the improbable a.n (so the
// loads cannot be dropped).
__device__ __forceinline__ void stream_copy41(const tx_fp8_codec_args &a) {
  const txd::u32x4 *src = reinterpret_cast<const txd::u32x4 *>(a.src) + a.start / 4;
  uint32_t *dst = reinterpret_cast<uint32_t *>(a.dst) + a.start / 4;
  const int64_t nchunks = (a.n - a.start) / kChunk;
  for (int64_t c = blockIdx.x; c < nchunks; c += gridDim.x) {
    const int64_t w0 = c * (kChunk / 4) + threadIdx.x;
    txd::u32x4 v[kVecPerThread];
#pragma unroll
    for (int j = 0; j < kVecPerThread; ++j) v[j] = __builtin_nontemporal_load(src + w0 + j * kBlock);
#pragma unroll
    for (int j = 0; j < kVecPerThread; ++j)
      __builtin_nontemporal_store(__builtin_amdgcn_perm(v[j].y, v[j].x, 0x0c0c0400u) |
                                      __builtin_amdgcn_perm(v[j].w, v[j].z, 0x04000c0cu),
                                  dst + w0 + j * kBlock);
  }
}

__device__ __forceinline__ void stream_read(const tx_fp8_codec_args &a) {
  const txd::u32x4 *src = reinterpret_cast<const txd::u32x4 *>(a.src) + a.start / 4;
  uint32_t *dst = reinterpret_cast<uint32_t *>(a.dst) + a.start / 4;
  const int64_t nchunks = (a.n - a.start) / kChunk;
  for (int64_t c = blockIdx.x; c < nchunks; c += gridDim.x) {
    const int64_t w0 = c * (kChunk / 4) + threadIdx.x;
    txd::u32x4 v[kVecPerThread];
#pragma unroll
    for (int j = 0; j < kVecPerThread; ++j) v[j] = __builtin_nontemporal_load(src + w0 + j * kBlock);
    uint32_t x = 0;
#pragma unroll
    for (int j = 0; j < kVecPerThread; ++j) x ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
    if (x == uint32_t(a.n)) dst[w0] = x;
  }
}

TX_KERNEL void __launch_bounds__(kBlock) tx_stream_copy41_vec(const tx_fp8_codec_args a) { stream_copy41(a); }
TX_KERNEL void __launch_bounds__(kBlock) tx_stream_read_vec(const tx_fp8_codec_args a) { stream_read(a); }

TX_KERNEL void __launch_bounds__(kBlock) tx_fp8_decode_e4m3fn_vec(const tx_fp8_codec_args a) {
  decode_vec<E4M3FN>(a);
}
TX_KERNEL void __launch_bounds__(kBlock) tx_fp8_decode_e4m3fn_tail(const tx_fp8_codec_args a) {
  decode_tail<E4M3FN>(a);
}
TX_KERNEL void __launch_bounds__(kBlock) tx_fp8_decode_e5m2_vec(const tx_fp8_codec_args a) {
  decode_vec<E5M2>(a);
}
TX_KERNEL void __launch_bounds__(kBlock) tx_fp8_decode_e5m2_tail(const tx_fp8_codec_args a) {
  decode_tail<E5M2>(a);
}

// Conversions with a bf16, fp16 or fp8 source: tx_cvt_<src>_<dst>_<rounding>[_sat].
// Rounding ones come in rtne / rtz, saturating or not; exact ones (to a
// format that holds every source value) once, as _exact, plus _exact_sat
// where the source has infinities and the destination a saturating form.
#define TX_CVT2(NAME, SRC, DST, MODE, SAT)                                                  \
  TX_KERNEL void __launch_bounds__(kBlock) tx_cvt_##NAME##_vec(const tx_fp8_codec_args a) {  \
    cvt2_vec<SRC, DST, MODE, SAT>(a);                                                       \
  }                                                                                         \
  TX_KERNEL void __launch_bounds__(kBlock) tx_cvt_##NAME##_tail(const tx_fp8_codec_args a) { \
    cvt2_tail<SRC, DST, MODE, SAT>(a);                                                      \
  }
#define TX_CVT2_ROUNDING(S, D, SRC, DST)            \
  TX_CVT2(S##_##D##_rtne, SRC, DST, 0, false)       \
  TX_CVT2(S##_##D##_rtne_sat, SRC, DST, 0, true)    \
  TX_CVT2(S##_##D##_rtz, SRC, DST, 1, false)        \
  TX_CVT2(S##_##D##_rtz_sat, SRC, DST, 1, true)

TX_CVT2_ROUNDING(bf16, e4m3fn, BF16, E4M3FN)
TX_CVT2_ROUNDING(bf16, e5m2, BF16, E5M2)
TX_CVT2_ROUNDING(bf16, f16, BF16, F16)
TX_CVT2_ROUNDING(f16, e4m3fn, F16, E4M3FN)
TX_CVT2_ROUNDING(f16, e5m2, F16, E5M2)
TX_CVT2_ROUNDING(f16, bf16, F16, BF16)
TX_CVT2_ROUNDING(e4m3fn, e5m2, E4M3FN, E5M2)
TX_CVT2_ROUNDING(e5m2, e4m3fn, E5M2, E4M3FN)
TX_CVT2(bf16_f32_exact, BF16, F32, 0, false)
TX_CVT2(f16_f32_exact, F16, F32, 0, false)
TX_CVT2(e4m3fn_bf16_exact, E4M3FN, BF16, 0, false)
TX_CVT2(e4m3fn_f16_exact, E4M3FN, F16, 0, false)
TX_CVT2(e5m2_bf16_exact, E5M2, BF16, 0, false)
TX_CVT2(e5m2_f16_exact, E5M2, F16, 0, false)
// e5m2 holds +-Inf: saturating makes them +-max of the destination
TX_CVT2(e5m2_bf16_exact_sat, E5M2, BF16, 0, true)
TX_CVT2(e5m2_f16_exact_sat, E5M2, F16, 0, true)
