// Host runtime: errors, code-object loading, launches.
//
// The reference's plugin is loaded by Triton with dlopen and hands Triton MLIR
// callbacks (support/Export.cpp:58-97); the device code is then produced by
// Triton's own backend.  Here the device code is prebuilt: each kernel source
// is compiled ahead of time to a gfx950 code object, the code objects are
// embedded in this library's read-only data, and they are loaded into a
// device with hipModuleLoadData the first time an op runs there.
#include "tx_runtime.h"

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <utility>

// Embedded code objects (see the generated tx_embedded.S).
extern "C" {
extern const unsigned char tx_co_fp8_codec_begin[], tx_co_fp8_codec_end[];
extern const unsigned char tx_co_scatter_begin[], tx_co_scatter_end[];
extern const unsigned char tx_co_gemm_bf16_begin[], tx_co_gemm_bf16_end[];
extern const unsigned char tx_co_gemm_fp8_begin[], tx_co_gemm_fp8_end[];
extern const unsigned char tx_co_gemv_begin[], tx_co_gemv_end[];
extern const unsigned char tx_co_gemm_mx_begin[], tx_co_gemm_mx_end[];
}

namespace tx {
namespace {

thread_local std::string g_last_error;

struct CodeObjectImage {
  const char *name;
  const unsigned char *begin;
  const unsigned char *end;
};

const CodeObjectImage kImages[static_cast<int>(CodeObject::Count)] = {
    {"fp8_codec", tx_co_fp8_codec_begin, tx_co_fp8_codec_end},
    {"scatter", tx_co_scatter_begin, tx_co_scatter_end},
    {"gemm_bf16", tx_co_gemm_bf16_begin, tx_co_gemm_bf16_end},
    {"gemm_fp8", tx_co_gemm_fp8_begin, tx_co_gemm_fp8_end},
    {"gemv", tx_co_gemv_begin, tx_co_gemv_end},
    {"gemm_mx", tx_co_gemm_mx_begin, tx_co_gemm_mx_end},
};

constexpr int kMaxDevices = 64;
constexpr int kMaxKernels = 96;

constexpr size_t kMaxKernelName = 96;

struct KernelSlot {
  char name[kMaxKernelName];  // a copy: callers pass transient buffers
  int co;
  hipFunction_t fn;
};

struct KeptScratch {
  void *ptr = nullptr;
  size_t bytes = 0;
};

struct DeviceState {
  std::once_flag once;
  tx_status status = TX_GENERIC_FAILURE;
  std::string error;
  int cus = 0;
  hipModule_t modules[static_cast<int>(CodeObject::Count)] = {};
  std::mutex mu;
  KernelSlot kernels[kMaxKernels] = {};
  int num_kernels = 0;
  // kept scratch buffers, keyed by (stream, slot); recursive so that one
  // call can hold a lease on each slot
  std::recursive_mutex scratch_mu;
  std::map<std::pair<hipStream_t, int>, KeptScratch> scratch;
};

DeviceState g_devices[kMaxDevices];

void load_device(int dev, DeviceState &st) {
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, dev);
  if (e != hipSuccess) {
    st.status = TX_NO_DEVICE;
    st.error = std::string("hipGetDeviceProperties: ") + hipGetErrorString(e);
    return;
  }
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    st.status = TX_NO_DEVICE;
    st.error = std::string("device ") + std::to_string(dev) + " is " +
               prop.gcnArchName + "; this library carries gfx950 code only";
    return;
  }
  st.cus = prop.multiProcessorCount;
  for (int i = 0; i < static_cast<int>(CodeObject::Count); ++i) {
    const CodeObjectImage &img = kImages[i];
    if (img.end <= img.begin) {
      st.status = TX_CODE_OBJECT_ERROR;
      st.error = std::string("code object '") + img.name + "' is empty";
      return;
    }
    e = hipModuleLoadData(&st.modules[i], img.begin);
    if (e != hipSuccess) {
      st.status = TX_CODE_OBJECT_ERROR;
      st.error = std::string("hipModuleLoadData(") + img.name +
                 "): " + hipGetErrorString(e);
      for (int j = 0; j < i; ++j) {
        hipModuleUnload(st.modules[j]);
        st.modules[j] = nullptr;
      }
      return;
    }
  }
  st.status = TX_SUCCESS;
}

tx_status device_state(DeviceState **out) {
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count <= 0)
    return fail(TX_NO_DEVICE, "no HIP device available (%s)",
                e == hipSuccess ? "count is 0" : hipGetErrorString(e));
  int dev = 0;
  e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return fail(TX_NO_DEVICE, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(TX_NO_DEVICE, "device index %d out of range", dev);
  DeviceState &st = g_devices[dev];
  std::call_once(st.once, [&] { load_device(dev, st); });
  if (st.status != TX_SUCCESS) return fail(st.status, "%s", st.error.c_str());
  *out = &st;
  return TX_SUCCESS;
}

}  // namespace

tx_status fail(tx_status status, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return status;
}

void clear_error() { g_last_error.clear(); }

tx_status get_kernel(CodeObject co, const char *name, hipFunction_t *out) {
  DeviceState *st = nullptr;
  tx_status s = device_state(&st);
  if (s != TX_SUCCESS) return s;
  const int ci = static_cast<int>(co);
  std::lock_guard<std::mutex> lock(st->mu);
  for (int i = 0; i < st->num_kernels; ++i) {
    const KernelSlot &k = st->kernels[i];
    if (k.co == ci && std::strcmp(k.name, name) == 0) {
      *out = k.fn;
      return TX_SUCCESS;
    }
  }
  hipFunction_t fn = nullptr;
  hipError_t e = hipModuleGetFunction(&fn, st->modules[ci], name);
  if (e != hipSuccess)
    return fail(TX_CODE_OBJECT_ERROR, "kernel '%s' not found in code object '%s': %s",
                name, kImages[ci].name, hipGetErrorString(e));
  if (st->num_kernels < kMaxKernels && std::strlen(name) < kMaxKernelName) {
    KernelSlot &slot = st->kernels[st->num_kernels++];
    std::memcpy(slot.name, name, std::strlen(name) + 1);
    slot.co = ci;
    slot.fn = fn;
  }
  *out = fn;
  return TX_SUCCESS;
}

tx_status ScratchLease::acquire(hipStream_t stream, int slot, size_t bytes) {
  DeviceState *st = nullptr;
  tx_status s = device_state(&st);
  if (s != TX_SUCCESS) return s;
  if (lock_) return fail(TX_GENERIC_FAILURE, "scratch lease acquired twice");
  st->scratch_mu.lock();
  lock_ = &st->scratch_mu;
  stream_ = stream;
  if (bytes > kKeptScratch) {
    hipError_t e = hipMallocAsync(&ptr_, bytes, stream);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      ptr_ = nullptr;
      return fail(TX_GENERIC_FAILURE, "scratch of %zu bytes: %s", bytes, hipGetErrorString(e));
    }
    own_ = true;
    return TX_SUCCESS;
  }
  KeptScratch &k = st->scratch[{stream, slot}];
  if (k.bytes < bytes) {
    if (k.ptr && hipFreeAsync(k.ptr, stream) != hipSuccess) (void)hipGetLastError();
    k.ptr = nullptr;
    k.bytes = 0;
    // round up so that slowly growing requests do not reallocate every call
    const size_t want = std::min(kKeptScratch, (bytes + (size_t(4) << 20) - 1) / (size_t(4) << 20) * (size_t(4) << 20));
    hipError_t e = hipMallocAsync(&k.ptr, want, stream);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      k.ptr = nullptr;
      return fail(TX_GENERIC_FAILURE, "scratch of %zu bytes: %s", want, hipGetErrorString(e));
    }
    k.bytes = want;
  }
  ptr_ = k.ptr;
  return TX_SUCCESS;
}

ScratchLease::~ScratchLease() {
  if (own_ && ptr_ && hipFreeAsync(ptr_, stream_) != hipSuccess) (void)hipGetLastError();
  if (lock_) static_cast<std::recursive_mutex *>(lock_)->unlock();
}

void release_all_scratch() {
  for (int d = 0; d < kMaxDevices; ++d) {
    DeviceState &st = g_devices[d];
    std::lock_guard<std::recursive_mutex> lock(st.scratch_mu);
    if (st.scratch.empty()) continue;
    int cur = 0;
    if (hipGetDevice(&cur) != hipSuccess || hipSetDevice(d) != hipSuccess) continue;
    for (auto &kv : st.scratch)
      if (kv.second.ptr && hipFree(kv.second.ptr) != hipSuccess) (void)hipGetLastError();
    st.scratch.clear();
    hipSetDevice(cur);
  }
}

int cu_count() {
  DeviceState *st = nullptr;
  if (device_state(&st) != TX_SUCCESS) return 0;
  return st->cus;
}

tx_status launch(hipFunction_t fn, unsigned grid_x, unsigned grid_y,
                 unsigned block_x, hipStream_t stream, void *args,
                 size_t args_size, const char *what) {
  if (grid_x == 0 || grid_y == 0) return TX_SUCCESS;
  void *config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, args,
                    HIP_LAUNCH_PARAM_BUFFER_SIZE, &args_size,
                    HIP_LAUNCH_PARAM_END};
  hipError_t e = hipModuleLaunchKernel(fn, grid_x, grid_y, 1, block_x, 1, 1, 0,
                                       stream, nullptr, config);
  if (e != hipSuccess)
    return fail(TX_LAUNCH_ERROR, "launch of %s failed: %s", what,
                hipGetErrorString(e));
  return TX_SUCCESS;
}

}  // namespace tx

extern "C" {

TX_API const char *txGetLastError(void) { return tx::g_last_error.c_str(); }

TX_API tx_status txInit(void) {
  tx::clear_error();
  hipFunction_t fn;
  // Loading happens inside device_state; resolving one kernel proves the
  // code objects are usable.
  return tx::get_kernel(tx::CodeObject::Fp8Codec, "tx_fp8_decode_e4m3fn_vec",
                        &fn);
}

TX_API void txShutdown(void) {
  tx::release_all_scratch();
  for (int d = 0; d < tx::kMaxDevices; ++d) {
    tx::DeviceState &st = tx::g_devices[d];
    if (st.status != TX_SUCCESS) continue;
    int cur = 0;
    if (hipGetDevice(&cur) != hipSuccess) return;
    if (hipSetDevice(d) != hipSuccess) continue;
    std::lock_guard<std::mutex> lock(st.mu);
    for (auto &m : st.modules) {
      if (m) hipModuleUnload(m);
      m = nullptr;
    }
    st.num_kernels = 0;
    // The once_flag cannot be reset; mark the device unusable after shutdown.
    st.status = TX_CODE_OBJECT_ERROR;
    st.error = "txShutdown() was called; code objects are unloaded";
    hipSetDevice(cur);
  }
}

}  // extern "C"
