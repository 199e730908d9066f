// tx_dot_fp8_scaled_grouped_noalloc: the grouped fp8 dot for callers that
// cannot allocate device memory (code under HIP graph capture, serving
// loops, harnesses that forbid hipMalloc).  It has no counterpart in the
// reference.
//
// The grouped product needs one workspace: the m-tile prefix sums of its
// groups (groups + 1 int32), written by a one-workgroup scan before the
// product reads them.  Here that workspace is a file-scope device array of
// kNoAllocScratchBytes, one copy per GPU, alive until the process ends.  Its
// device address is looked up once per device with hipGetSymbolAddress (at
// txInit, or on the entry point's first call on that device) and only that
// address is ever handed to a kernel: in host code the array's name is a
// host-side stand-in, not a device address.
//
// Every call on one GPU shares that GPU's array and the array keeps the last
// call's contents; the prefix scan writes every entry a call reads, so
// nothing needs clearing.  Calls that overlap on one GPU (different streams,
// or threads that do not order their calls) race on the array.
#include <hip/hip_runtime.h>

#include <mutex>

#include "tx_ops.h"

namespace {

constexpr size_t kNoAllocScratchBytes = size_t(64) << 10;
// largest group count whose tile prefix fits the array
constexpr int64_t kNoAllocMaxGroups = int64_t(kNoAllocScratchBytes / sizeof(int32_t)) - 1;

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;

struct DeviceScratch {
  std::once_flag once;
  hipError_t err = hipSuccess;
  void *ptr = nullptr;  // this device's copy of `scratch`
};
DeviceScratch g_scratch[kMaxDevices];

}  // namespace

namespace tx {

// The current device's copy of the array (its address looked up once, with
// that device current).
tx_status noalloc_scratch(void **out) {
  int dev = 0;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(TX_NO_DEVICE, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(TX_NO_DEVICE, "device index %d out of range", dev);
  DeviceScratch &d = g_scratch[dev];
  std::call_once(d.once, [&] {
    d.err = hipGetSymbolAddress(&d.ptr, HIP_SYMBOL(scratch));
    if (d.err != hipSuccess) {
      (void)hipGetLastError();
      d.ptr = nullptr;
    }
  });
  if (d.err != hipSuccess || !d.ptr)
    return fail(TX_GENERIC_FAILURE, "no-allocation scratch of device %d: hipGetSymbolAddress: %s", dev,
                hipGetErrorString(d.err));
  *out = d.ptr;
  return TX_SUCCESS;
}

}  // namespace tx

extern "C" {

TX_API tx_status tx_dot_fp8_scaled_grouped_noalloc(const void *A, tx_dtype a_type, int64_t lda,
                                                   const float *scale_a, const void *B, tx_dtype b_type,
                                                   int64_t ldb, int64_t stride_b, const float *scale_b,
                                                   int64_t stride_scale_b, const float *bias,
                                                   int64_t stride_bias, int activation, void *C,
                                                   tx_dtype c_type, float c_scale, int64_t ldc,
                                                   const int32_t *group_offsets, int64_t groups, int64_t M,
                                                   int64_t N, int64_t K, tx_stream_t stream) {
  const char *what = "tx_dot_fp8_scaled_grouped_noalloc";
  tx::clear_error();
  if (groups > kNoAllocMaxGroups)
    return tx::fail(TX_UNSUPPORTED, "%s: %lld groups exceed the %lld its %zu-byte workspace holds", what,
                    (long long)groups, (long long)kNoAllocMaxGroups, kNoAllocScratchBytes);
  void *ws = nullptr;
  if (groups > 0 && M > 0 && N > 0) TX_TRY(tx::noalloc_scratch(&ws));
  return tx::dot_fp8_scaled_grouped_ws(what, A, a_type, lda, scale_a, B, b_type, ldb, stride_b, scale_b,
                                       stride_scale_b, bias, stride_bias, activation, C, c_type, c_scale, ldc,
                                       group_offsets, groups, M, N, K, stream, static_cast<int32_t *>(ws));
}

}  // extern "C"
