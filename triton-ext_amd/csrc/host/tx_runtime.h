// Internal host runtime of libtxamd.so: last-error plumbing, per-device
// code-object loading and the launch helper.  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>

#include "tx_plugin.h"

namespace tx {

// The gfx950 code objects embedded in the library, one per kernel source.
enum class CodeObject : int {
  Fp8Codec = 0,
  Scatter = 1,
  GemmBf16 = 2,
  GemmFp8 = 3,
  Gemv = 4,
  Count = 5
};

// Record `status` and a printf-style message as the calling thread's last
// error and return `status`.
tx_status fail(tx_status status, const char *fmt, ...)
    __attribute__((format(printf, 2, 3)));

// Clear the calling thread's last error (every entry point starts with it).
void clear_error();

// Resolve kernel `name` of code object `co` on the current device, loading
// that device's code objects on first use.
tx_status get_kernel(CodeObject co, const char *name, hipFunction_t *out);

// Enqueue `fn` with one by-value argument block of `args_size` bytes.
tx_status launch(hipFunction_t fn, unsigned grid_x, unsigned grid_y,
                 unsigned block_x, hipStream_t stream, void *args,
                 size_t args_size, const char *what);

// Number of compute units of the current device (cached per device).
int cu_count();

// True if p is aligned to `bytes`.
inline bool aligned(const void *p, size_t bytes) {
  return (reinterpret_cast<uintptr_t>(p) & (bytes - 1)) == 0;
}

}  // namespace tx
