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
  GemmMx = 5,
  Count = 6
};

// Record `status` and a printf-style message as the calling thread's last
// error and return `status`.
tx_status fail(tx_status status, const char *fmt, ...)
    __attribute__((format(printf, 2, 3)));

// Clear the calling thread's last error (every entry point starts with it).
void clear_error();

// Resolve kernel `name` of code object `co` on the current device, loading
// that device's code objects on first use.  Every kernel handle is resolved
// at load time into a table that is only read afterwards: no lock, no scan.
tx_status get_kernel(CodeObject co, const char *name, hipFunction_t *out);

// Enqueue `fn` with one by-value argument block of `args_size` bytes.
tx_status launch(hipFunction_t fn, unsigned grid_x, unsigned grid_y,
                 unsigned block_x, hipStream_t stream, void *args,
                 size_t args_size, const char *what, unsigned shared_bytes = 0);

// The current device's copy of the no-allocation entry point's workspace
// (tx_noalloc.hip), its address looked up once per device.
tx_status noalloc_scratch(void **out);

// Number of compute units of the current device (cached per device).
int cu_count();

// Stream-ordered device scratch for the ops that need a workspace.  The
// library keeps one buffer per (device, stream, slot), up to kKeptScratch
// bytes, and later calls on that stream reuse it, so steady-state calls
// allocate nothing.  Growing a kept buffer frees the old one and allocates
// the new one in stream order (hipFreeAsync / hipMallocAsync on the stream):
// work already enqueued keeps its memory.  Larger requests get a buffer of
// their own, freed in stream order when the lease ends.  A lease holds the
// lock of its (stream, slot) buffer from acquire() until it is destroyed,
// so the caller enqueues every launch that uses the buffer while holding
// it: two calls on one stream from different threads never see one buffer
// change under them, and calls on other streams or slots never wait for
// it.  A thread asking for a slot it already holds gets an error.  (A
// stream handle that is destroyed and handed out again keeps its
// predecessor's buffer; its work must have finished, as for any reuse of
// memory.)  txShutdown frees the kept buffers.
constexpr size_t kKeptScratch = size_t(512) << 20;

class ScratchLease {
 public:
  ScratchLease() = default;
  ScratchLease(const ScratchLease &) = delete;
  ScratchLease &operator=(const ScratchLease &) = delete;
  ~ScratchLease();
  // `slot` (0, 1 or 2) separates the buffers one call needs at the same time.
  tx_status acquire(hipStream_t stream, int slot, size_t bytes);
  void *ptr() const { return ptr_; }

 private:
  void *ptr_ = nullptr;
  hipStream_t stream_ = nullptr;
  bool own_ = false;    // a per-call buffer, freed by the destructor
  void *lock_ = nullptr;  // the (stream, slot) buffer whose lock this lease holds
};

// Free every kept scratch buffer of every device (txShutdown).
void release_all_scratch();

// True if p is aligned to `bytes`.
inline bool aligned(const void *p, size_t bytes) {
  return (reinterpret_cast<uintptr_t>(p) & (bytes - 1)) == 0;
}

}  // namespace tx
