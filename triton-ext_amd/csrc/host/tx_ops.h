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

#define TX_TRY(expr)                      \
  do {                                    \
    tx_status _s = (expr);                \
    if (_s != TX_SUCCESS) return _s;      \
  } while (0)

}  // namespace tx
