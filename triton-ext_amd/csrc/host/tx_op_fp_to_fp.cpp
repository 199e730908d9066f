// tt.fp_to_fp entry points (fp32 <-> fp8, fp32 -> fp16 / bf16, bf16 / fp16 /
// fp8 to any other of these formats, stochastic rounding with random bits)
// and their table registration.
//
// Reference: tt.fp_to_fp is emitted by semantic.cast (semantic.py:807-827,
// default rounding RTNE at :809), passed through the plugin's conversion
// (uTLXConversionPatterns.cpp:577) and re-created with a rounding operand by
// createFpToFpWithRbits (ops/NewOps.cpp:249-303; rounding 0 rtne, 1 rtz,
// 2 rs at :270-286).  The saturating variant is the reference's
// clamp-then-convert idiom (mxfp8_utils.py:17-21, 36-38).
#include <algorithm>
#include <cstdio>

#include "tx_kernel_args.h"
#include "tx_ops.h"

namespace tx {
namespace {

constexpr unsigned kBlock = 256;
constexpr int64_t kChunk = 4096;  // elements per block step of the vector kernels

const char *fmt_name(tx_dtype t) {
  switch (t) {
    case TX_FP8E4M3FN: return "e4m3fn";
    case TX_FP8E5M2: return "e5m2";
    case TX_BF16: return "bf16";
    case TX_F16: return "f16";
    default: return nullptr;
  }
}

bool is_fp8(tx_dtype t) { return t == TX_FP8E4M3FN || t == TX_FP8E5M2; }
bool is_16(tx_dtype t) { return t == TX_BF16 || t == TX_F16; }

// The vector kernel covers the largest multiple of `step` elements (its
// block step) of [0, n); the tail kernel the rest.
tx_status run(const char *vec_name, const char *tail_name, const void *src,
              void *dst, int64_t n, bool vec_ok, hipStream_t stream,
              const uint32_t *rbits = nullptr, int64_t step = kChunk) {
  tx_fp8_codec_args args{src, dst, 0, n, rbits};
  int64_t n_vec = vec_ok ? (n / step) * step : 0;
  const int cus = cu_count();
  if (n_vec > 0) {
    hipFunction_t fn;
    TX_TRY(get_kernel(CodeObject::Fp8Codec, vec_name, &fn));
    args.start = 0;
    args.n = n_vec;
    // One block per step, capped at 32 resident blocks per CU; the kernels
    // loop over the remaining steps.
    int64_t grid = std::min<int64_t>(n_vec / step, int64_t(cus) * 32);
    TX_TRY(launch(fn, unsigned(grid), 1, kBlock, stream, &args, sizeof args, vec_name));
  }
  if (n_vec < n) {
    hipFunction_t fn;
    TX_TRY(get_kernel(CodeObject::Fp8Codec, tail_name, &fn));
    args.start = n_vec;
    args.n = n;
    int64_t grid = std::min<int64_t>((n - n_vec + kBlock - 1) / kBlock, int64_t(cus) * 32);
    TX_TRY(launch(fn, unsigned(grid), 1, kBlock, stream, &args, sizeof args, tail_name));
  }
  return TX_SUCCESS;
}

}  // namespace

static tx_status fp_to_fp(const void *src, tx_dtype src_type, void *dst,
                          tx_dtype dst_type, int64_t n, tx_rounding rounding,
                          int saturate, tx_stream_t stream) {
  if (n < 0) return fail(TX_INVALID_ARGUMENT, "tx_fp_to_fp: n = %lld < 0", (long long)n);
  if (n == 0) return TX_SUCCESS;
  if (!src || !dst) return fail(TX_INVALID_ARGUMENT, "tx_fp_to_fp: NULL buffer");
  const bool src_fp8 = is_fp8(src_type);
  const bool dst_fp8 = is_fp8(dst_type);
  hipStream_t s = static_cast<hipStream_t>(stream);
  char vec[64], tail[64];
  if (src_type == TX_F32 && (dst_fp8 || is_16(dst_type))) {
    if (rounding == TX_RS)
      return fail(TX_UNSUPPORTED,
                  "tx_fp_to_fp: stochastic rounding needs random bits "
                  "(tx_fp_to_fp_with_rbits)");
    if (rounding != TX_RTNE && rounding != TX_RTZ)
      return fail(TX_INVALID_ARGUMENT, "tx_fp_to_fp: rounding %d", int(rounding));
    const char *r = rounding == TX_RTZ ? "rtz" : "rtne";
    const char *sat = saturate ? "_sat" : "";
    const char *kind = dst_fp8 ? "fp8_encode" : "cvt_f32";
    std::snprintf(vec, sizeof vec, "tx_%s_%s_%s%s_vec", kind, fmt_name(dst_type), r, sat);
    std::snprintf(tail, sizeof tail, "tx_%s_%s_%s%s_tail", kind, fmt_name(dst_type), r, sat);
    const bool vec_ok = aligned(src, 16) && aligned(dst, dst_fp8 ? 4 : 8);
    return run(vec, tail, src, dst, n, vec_ok, s);
  }
  if (src_fp8 && dst_type == TX_F32) {
    std::snprintf(vec, sizeof vec, "tx_fp8_decode_%s_vec", fmt_name(src_type));
    std::snprintf(tail, sizeof tail, "tx_fp8_decode_%s_tail", fmt_name(src_type));
    const bool vec_ok = aligned(src, 4) && aligned(dst, 16);
    return run(vec, tail, src, dst, n, vec_ok, s);
  }
  // bf16 / fp16 / fp8 sources: widened to fp32 exactly, then rounded once.
  // Destinations that hold every source value (fp8 -> bf16 / fp16, bf16 /
  // fp16 -> fp32) are exact whatever the rounding; saturation there only
  // maps e5m2's +-Inf to the 16-bit format's +-max (an fp32 destination,
  // as in the fp8 -> fp32 decode, keeps infinities).
  if ((src_fp8 || is_16(src_type)) && (dst_fp8 || is_16(dst_type) || dst_type == TX_F32) &&
      src_type != dst_type) {
    if (rounding == TX_RS)
      return fail(TX_UNSUPPORTED, "tx_fp_to_fp: stochastic rounding takes a float32 source (got %d)",
                  int(src_type));
    if (rounding != TX_RTNE && rounding != TX_RTZ)
      return fail(TX_INVALID_ARGUMENT, "tx_fp_to_fp: rounding %d", int(rounding));
    const bool exact = dst_type == TX_F32 || (src_fp8 && is_16(dst_type));
    const char *sn = fmt_name(src_type), *dn = dst_type == TX_F32 ? "f32" : fmt_name(dst_type);
    if (!sn || !dn) return fail(TX_UNSUPPORTED, "tx_fp_to_fp: conversion %d -> %d", int(src_type), int(dst_type));
    char mode[16];
    std::snprintf(mode, sizeof mode, "%s", exact ? "exact" : rounding == TX_RTZ ? "rtz" : "rtne");
    const bool sat_matters = !exact || (src_type == TX_FP8E5M2 && is_16(dst_type));
    const char *sat = (sat_matters && saturate) ? "_sat" : "";
    std::snprintf(vec, sizeof vec, "tx_cvt_%s_%s_%s%s_vec", sn, dn, mode, sat);
    std::snprintf(tail, sizeof tail, "tx_cvt_%s_%s_%s%s_tail", sn, dn, mode, sat);
    // units of 16 / max(sizes) elements: 16-byte accesses on the wider side
    const int ss = src_fp8 ? 1 : 2, ds = dst_type == TX_F32 ? 4 : dst_fp8 ? 1 : 2;
    const int e = 16 / std::max(ss, ds);
    const bool vec_ok = aligned(src, size_t(e * ss)) && aligned(dst, size_t(e * ds));
    // two chunks per block step where a value moves 3 bytes or fewer
    const int64_t step = kChunk * (ss + ds <= 3 ? 2 : 1);
    return run(vec, tail, src, dst, n, vec_ok, s, nullptr, step);
  }
  return fail(TX_UNSUPPORTED, "tx_fp_to_fp: conversion %d -> %d is not served",
              int(src_type), int(dst_type));
}

// Stochastic rounding takes a float32 source and an fp16, bf16, e5m2 or
// e4m3fn destination (the reference's stoch_round accepts exactly these and
// raises otherwise, test_tlx.py:5291-5329) and one 32-bit word of random
// bits per element; it always saturates (the reference lowers it to
// cvt.rs.satfinite, test_tlx.py:5182).  Other roundings ignore rbits.
static tx_status fp_to_fp_rbits(const void *src, tx_dtype src_type, void *dst,
                                tx_dtype dst_type, const uint32_t *rbits, int64_t n,
                                tx_rounding rounding, int saturate, tx_stream_t stream) {
  if (rounding != TX_RS)
    return fp_to_fp(src, src_type, dst, dst_type, n, rounding, saturate, stream);
  if (n < 0) return fail(TX_INVALID_ARGUMENT, "tx_fp_to_fp_with_rbits: n = %lld < 0", (long long)n);
  if (src_type != TX_F32)
    return fail(TX_INVALID_ARGUMENT,
                "tx_fp_to_fp_with_rbits: stochastic rounding takes a float32 source (got %d)",
                int(src_type));
  if (!is_fp8(dst_type) && !is_16(dst_type))
    return fail(TX_INVALID_ARGUMENT,
                "tx_fp_to_fp_with_rbits: stochastic rounding is supported to fp16, bf16, e5m2 "
                "and e4m3fn only (got %d)", int(dst_type));
  if (n == 0) return TX_SUCCESS;
  if (!src || !dst || !rbits)
    return fail(TX_INVALID_ARGUMENT, "tx_fp_to_fp_with_rbits: NULL buffer");
  char vec[64], tail[64];
  std::snprintf(vec, sizeof vec, "tx_cvt_f32_%s_rs_vec", fmt_name(dst_type));
  std::snprintf(tail, sizeof tail, "tx_cvt_f32_%s_rs_tail", fmt_name(dst_type));
  const bool vec_ok = aligned(src, 16) && aligned(rbits, 16) && aligned(dst, is_fp8(dst_type) ? 4 : 8);
  return run(vec, tail, src, dst, n, vec_ok, static_cast<hipStream_t>(stream), rbits);
}

// Table form: operands = {dst (result slot), src, n, src_type, dst_type,
// rounding, saturate[, rbits]}; rbits as in createFpToFpWithRbits, an
// optional operand (ops/NewOps.cpp:253-257).
static tx_status fp_to_fp_op(tx_value *v, size_t count, tx_stream_t stream) {
  Operands o{v, count, "tt.fp_to_fp"};
  TX_TRY(o.need_either(7, 8));
  void *dst, *src, *rbits = nullptr;
  int64_t n, st, dt, rnd, sat;
  TX_TRY(o.ptr(0, &dst));
  TX_TRY(o.ptr(1, &src));
  TX_TRY(o.integer(2, &n));
  TX_TRY(o.integer(3, &st));
  TX_TRY(o.integer(4, &dt));
  TX_TRY(o.integer(5, &rnd));
  TX_TRY(o.integer(6, &sat));
  if (count == 8) TX_TRY(o.ptr(7, &rbits));
  return fp_to_fp_rbits(src, tx_dtype(st), dst, tx_dtype(dt), static_cast<const uint32_t *>(rbits),
                        n, tx_rounding(rnd), int(sat), stream);
}

static const bool registered = register_op(
    "tt.fp_to_fp", fp_to_fp_op,
    "dst(result), src, n:i64, src_type:i32, dst_type:i32, rounding:i32, saturate:i32"
    "[, rbits:u32*]");

}  // namespace tx

extern "C" TX_API tx_status tx_fp_to_fp_with_rbits(const void *src, tx_dtype src_type,
                                                   void *dst, tx_dtype dst_type,
                                                   const uint32_t *rbits, int64_t n,
                                                   tx_rounding rounding, int saturate,
                                                   tx_stream_t stream) {
  tx::clear_error();
  return tx::fp_to_fp_rbits(src, src_type, dst, dst_type, rbits, n, rounding, saturate, stream);
}

extern "C" TX_API tx_status tx_fp_to_fp(const void *src, tx_dtype src_type,
                                        void *dst, tx_dtype dst_type, int64_t n,
                                        tx_rounding rounding, int saturate,
                                        tx_stream_t stream) {
  tx::clear_error();
  return tx::fp_to_fp(src, src_type, dst, dst_type, n, rounding, saturate, stream);
}

extern "C" TX_API tx_status txStreamCeiling(int kind, const void *src, void *dst, int64_t n,
                                            tx_stream_t stream) {
  tx::clear_error();
  if (kind != 0 && kind != 1) return tx::fail(TX_INVALID_ARGUMENT, "txStreamCeiling: kind %d", kind);
  if (n < 0 || n % tx::kChunk != 0)
    return tx::fail(TX_INVALID_ARGUMENT, "txStreamCeiling: n = %lld is not a multiple of %lld", (long long)n,
                    (long long)tx::kChunk);
  if (n == 0) return TX_SUCCESS;
  if (!src || !dst || !tx::aligned(src, 16) || !tx::aligned(dst, 4))
    return tx::fail(TX_INVALID_ARGUMENT, "txStreamCeiling: src must be 16-byte and dst 4-byte aligned");
  const char *name = kind == 0 ? "tx_stream_copy41_vec" : "tx_stream_read_vec";
  return tx::run(name, name, src, dst, n, true, static_cast<hipStream_t>(stream));
}
