// absmax + fp8 quantiser entry points (MX block scales, row-wise scales)
// and their table registrations: the producer step in front of the fp8 and
// MX-scaled GEMMs.
//
// Reference: the MX quantiser is _compute_scale_and_quantize /
// _to_mxfp8_block (extensions/utlx/python/utlx_plugin/mxfp8_utils.py:10-56),
// emitted into TLX kernels; the row-wise form is the per-row absmax scaling
// the fp8 scaled dot consumes (one fp32 scale per row of A / column of B).
#include <algorithm>
#include <climits>
#include <cstdio>

#include "tx_kernel_args.h"
#include "tx_ops.h"

namespace tx {
namespace {

const char *q_name(tx_dtype t) {
  return t == TX_FP8E4M3FN ? "e4m3fn" : (t == TX_FP8E5M2 ? "e5m2" : nullptr);
}
const char *x_name(tx_dtype t) {
  return t == TX_F32 ? "f32" : (t == TX_BF16 ? "bf16" : nullptr);
}

tx_status check_quant(const char *what, const void *x, tx_dtype x_type, int64_t ldx, const void *q,
                      tx_dtype q_type, int64_t ldq, const void *scales, int64_t rows, int64_t K) {
  if (!x_name(x_type))
    return fail(TX_INVALID_ARGUMENT, "%s: x must be fp32 or bf16 (got %d)", what, int(x_type));
  if (!q_name(q_type))
    return fail(TX_INVALID_ARGUMENT, "%s: q must be an fp8 type (got %d)", what, int(q_type));
  if (rows < 0 || K < 0)
    return fail(TX_INVALID_ARGUMENT, "%s: negative size (rows=%lld K=%lld)", what, (long long)rows,
                (long long)K);
  if (rows == 0 || K == 0) return TX_SUCCESS;
  if (!x || !q || !scales) return fail(TX_INVALID_ARGUMENT, "%s: NULL buffer", what);
  if (ldx < K || ldq < K)
    return fail(TX_INVALID_ARGUMENT, "%s: stride smaller than the row (ldx=%lld ldq=%lld)", what,
                (long long)ldx, (long long)ldq);
  const size_t xs = x_type == TX_F32 ? 4 : 2;
  if (!aligned(x, xs)) return fail(TX_INVALID_ARGUMENT, "%s: x not %zu-byte aligned", what, xs);
  return TX_SUCCESS;
}

// The vector paths: 16-byte x loads (fp32: 4, bf16: 8 elements), q stores
// of `qbytes` (4 or 8) bytes, so rows and pitches must keep that alignment.
bool quant_vec(const void *x, tx_dtype x_type, int64_t ldx, const void *q, int64_t ldq,
               int64_t K, int64_t qbytes) {
  const int64_t ve = x_type == TX_F32 ? 4 : 8;
  return aligned(x, 16) && ldx % ve == 0 && K % ve == 0 && aligned(q, size_t(qbytes)) &&
         ldq % qbytes == 0;
}

tx_status quantize_mx(const void *x, tx_dtype x_type, int64_t ldx, void *q, tx_dtype q_type,
                      int64_t ldq, uint8_t *scales, int64_t ld_scales, int64_t rows, int64_t K,
                      tx_stream_t stream) {
  const char *what = "tx_quantize_mx";
  TX_TRY(check_quant(what, x, x_type, ldx, q, q_type, ldq, scales, rows, K));
  if (rows == 0 || K == 0) return TX_SUCCESS;
  if (K % 32)
    return fail(TX_INVALID_ARGUMENT, "%s: K = %lld is not a multiple of the 32-element block", what,
                (long long)K);
  if (ld_scales < K / 32)
    return fail(TX_INVALID_ARGUMENT, "%s: scale stride %lld < K / 32", what, (long long)ld_scales);
  char kname[64];
  std::snprintf(kname, sizeof kname, "tx_quant_mx_%s_%s", q_name(q_type), x_name(x_type));
  hipFunction_t fn;
  TX_TRY(get_kernel(CodeObject::Fp8Codec, kname, &fn));
  // 8-byte q stores at multiples of 8 elements; x loads as for the row path
  tx_quant_args a{x, static_cast<uint8_t *>(q), scales, ldx, ldq, ld_scales, rows, K,
                  quant_vec(x, x_type, ldx, q, ldq, K, 8) ? 1 : 0, 0};
  const int64_t threads = rows * (K / 32) * (x_type == TX_F32 ? 4 : 2);  // lanes per 32-element block
  const int64_t grid = std::min<int64_t>((threads + 255) / 256, int64_t(cu_count()) * 32);
  return launch(fn, unsigned(grid), 1, 256, static_cast<hipStream_t>(stream), &a, sizeof a, kname);
}

tx_status quantize_rowwise(const void *x, tx_dtype x_type, int64_t ldx, void *q, tx_dtype q_type,
                           int64_t ldq, float *scales, int64_t rows, int64_t K,
                           tx_stream_t stream) {
  const char *what = "tx_quantize_rowwise";
  TX_TRY(check_quant(what, x, x_type, ldx, q, q_type, ldq, scales, rows, K));
  if (rows == 0 || K == 0) return TX_SUCCESS;
  if (!aligned(scales, 4)) return fail(TX_INVALID_ARGUMENT, "%s: scales not 4-byte aligned", what);
  char kname[64];
  std::snprintf(kname, sizeof kname, "tx_quant_row_%s_%s", q_name(q_type), x_name(x_type));
  hipFunction_t fn;
  TX_TRY(get_kernel(CodeObject::Fp8Codec, kname, &fn));
  tx_quant_args a{x, static_cast<uint8_t *>(q), scales, ldx, ldq, 0, rows, K,
                  quant_vec(x, x_type, ldx, q, ldq, K, x_type == TX_F32 ? 4 : 8) ? 1 : 0, 0};
  const int64_t grid = std::min<int64_t>(rows, int64_t(cu_count()) * 16);
  return launch(fn, unsigned(grid), 1, 256, static_cast<hipStream_t>(stream), &a, sizeof a, kname);
}

// tx.quantize_mx: {q (result), scales (result), x, rows, K, ldx, ldq, ld_scales, x_type, q_type}
tx_status quant_mx_op(tx_value *v, size_t count, tx_stream_t stream) {
  Operands o{v, count, "tx.quantize_mx"};
  TX_TRY(o.need(10));
  void *q, *s, *x;
  int64_t rows, K, ldx, ldq, lds, xt, qt;
  TX_TRY(o.ptr(0, &q));
  TX_TRY(o.ptr(1, &s));
  TX_TRY(o.ptr(2, &x));
  TX_TRY(o.integer(3, &rows));
  TX_TRY(o.integer(4, &K));
  TX_TRY(o.integer(5, &ldx));
  TX_TRY(o.integer(6, &ldq));
  TX_TRY(o.integer(7, &lds));
  TX_TRY(o.integer(8, &xt));
  TX_TRY(o.integer(9, &qt));
  return quantize_mx(x, tx_dtype(xt), ldx, q, tx_dtype(qt), ldq, static_cast<uint8_t *>(s), lds,
                     rows, K, stream);
}

// tx.quantize_rowwise: {q (result), scales (result), x, rows, K, ldx, ldq, x_type, q_type}
tx_status quant_row_op(tx_value *v, size_t count, tx_stream_t stream) {
  Operands o{v, count, "tx.quantize_rowwise"};
  TX_TRY(o.need(9));
  void *q, *s, *x;
  int64_t rows, K, ldx, ldq, xt, qt;
  TX_TRY(o.ptr(0, &q));
  TX_TRY(o.ptr(1, &s));
  TX_TRY(o.ptr(2, &x));
  TX_TRY(o.integer(3, &rows));
  TX_TRY(o.integer(4, &K));
  TX_TRY(o.integer(5, &ldx));
  TX_TRY(o.integer(6, &ldq));
  TX_TRY(o.integer(7, &xt));
  TX_TRY(o.integer(8, &qt));
  return quantize_rowwise(x, tx_dtype(xt), ldx, q, tx_dtype(qt), ldq, static_cast<float *>(s), rows,
                          K, stream);
}

const bool reg_quant_mx = register_op(
    "tx.quantize_mx", quant_mx_op,
    "q:fp8*(result), scales:e8m0*(result, rows x K/32), x:f32|bf16*, rows, K, ldx, ldq, "
    "ld_scales, x_type:i32, q_type:i32");
const bool reg_quant_row = register_op(
    "tx.quantize_rowwise", quant_row_op,
    "q:fp8*(result), scales:f32*(result, rows), x:f32|bf16*, rows, K, ldx, ldq, x_type:i32, "
    "q_type:i32");

}  // namespace
}  // namespace tx

extern "C" {

TX_API tx_status tx_quantize_mx(const void *x, tx_dtype x_type, int64_t ldx, void *q,
                                tx_dtype q_type, int64_t ldq, uint8_t *scales, int64_t ld_scales,
                                int64_t rows, int64_t K, tx_stream_t stream) {
  tx::clear_error();
  return tx::quantize_mx(x, x_type, ldx, q, q_type, ldq, scales, ld_scales, rows, K, stream);
}

TX_API tx_status tx_quantize_rowwise(const void *x, tx_dtype x_type, int64_t ldx, void *q,
                                     tx_dtype q_type, int64_t ldq, float *scales, int64_t rows,
                                     int64_t K, tx_stream_t stream) {
  tx::clear_error();
  return tx::quantize_rowwise(x, x_type, ldx, q, q_type, ldq, scales, rows, K, stream);
}

}  // extern "C"
