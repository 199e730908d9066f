// Internal helpers shared by the op entry points: registration and operand
// decoding for the generic (table) calling convention.
#pragma once

#include <cstddef>
#include <cstdint>

#include "tx_plugin.h"
#include "tx_runtime.h"

namespace tx {

// Add an op to the registry (static-initialisation time, like exportOp at
// support/Export.cpp:38-42).  Always returns true so it can initialise a
// static bool.
bool register_op(const char *name, tx_op_fn fn, const char *signature);

// Operand access for table callbacks.  The reference's ops check the operand
// count and return without a result when it is wrong (uTLXPlugin.cpp:59-60);
// here a wrong count or kind is a TX_INVALID_ARGUMENT with a message.
struct Operands {
  tx_value *v;
  size_t n;
  const char *op;

  tx_status need(size_t count) const {
    if (!v && n) return fail(TX_INVALID_ARGUMENT, "%s: operand array is NULL", op);
    if (n != count)
      return fail(TX_INVALID_ARGUMENT, "%s: expected %zu operands, got %zu", op,
                  count, n);
    return TX_SUCCESS;
  }
  // Either of two operand counts (an op with optional trailing operands).
  tx_status need_either(size_t a, size_t b) const {
    if (!v && n) return fail(TX_INVALID_ARGUMENT, "%s: operand array is NULL", op);
    if (n != a && n != b)
      return fail(TX_INVALID_ARGUMENT, "%s: expected %zu or %zu operands, got %zu", op, a, b, n);
    return TX_SUCCESS;
  }
  tx_status ptr(size_t i, void **out) const {
    if (v[i].kind != TX_VALUE_PTR)
      return fail(TX_INVALID_ARGUMENT, "%s: operand %zu must be a pointer", op, i);
    *out = v[i].u.ptr;
    return TX_SUCCESS;
  }
  tx_status integer(size_t i, int64_t *out) const {
    if (v[i].kind != TX_VALUE_INT)
      return fail(TX_INVALID_ARGUMENT, "%s: operand %zu must be an integer constant",
                  op, i);
    *out = v[i].u.i;
    return TX_SUCCESS;
  }
};

// The grouped fp8 dot (tx_dot_fp8_scaled_grouped) with an optional caller
// workspace for its group tile prefix (groups + 1 int32 on the device);
// NULL uses the library's stream scratch.  `what` names the entry point in
// error messages.
tx_status dot_fp8_scaled_grouped_ws(const char *what, const void *A, tx_dtype a_type, int64_t lda,
                                    const float *sa, const void *B, tx_dtype b_type, int64_t ldb,
                                    int64_t stride_b, const float *sb, int64_t stride_sb, const float *bias,
                                    int64_t stride_bias, int activation, void *C, tx_dtype c_type,
                                    float c_scale, int64_t ldc, const int32_t *offsets, int64_t groups,
                                    int64_t M, int64_t N, int64_t K, tx_stream_t stream, int32_t *prefix_ws);

#define TX_TRY(expr)                      \
  do {                                    \
    tx_status _s = (expr);                \
    if (_s != TX_SUCCESS) return _s;      \
  } while (0)

}  // namespace tx
