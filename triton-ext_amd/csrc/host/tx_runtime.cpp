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
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <utility>
#include <vector>

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
// device allocations made for stream scratch (txScratchAllocations)
std::atomic<uint64_t> g_scratch_allocs{0};

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

// ------------------------------------------------------------ kernel table
// Every kernel of a code object is resolved once, when the device's code
// objects are loaded, into an open-addressing hash table that is never
// written afterwards: a launch looks its kernel up without a lock.  Kernel
// names come from the code object itself (the `<name>.kd` kernel
// descriptor symbols of its ELF symbol table), so the table always matches
// what was embedded.

// FNV-1a, 64-bit.
uint64_t name_hash(const char *s) {
  uint64_t h = 1469598103934665603ull;
  for (; *s; ++s) h = (h ^ uint8_t(*s)) * 1099511628211ull;
  return h;
}

struct KernelTable {
  struct Entry {
    uint64_t hash = 0;
    const char *name = nullptr;  // into `names`
    hipFunction_t fn = nullptr;
  };
  std::vector<std::string> names;
  std::vector<Entry> slots;  // power-of-two size, at most half full
  hipFunction_t find(const char *name) const {
    if (slots.empty()) return nullptr;
    const uint64_t h = name_hash(name);
    const size_t mask = slots.size() - 1;
    for (size_t i = size_t(h) & mask;; i = (i + 1) & mask) {
      const Entry &e = slots[i];
      if (!e.name) return nullptr;
      if (e.hash == h && std::strcmp(e.name, name) == 0) return e.fn;
    }
  }
};

// The gfx950 ELF inside an embedded image: hipcc --genco writes a clang
// offload bundle (magic, entry count, then per entry offset, size, target
// triple); a bare ELF is taken as it is.
bool find_device_elf(const unsigned char *img, size_t size, const unsigned char **elf, size_t *elf_size) {
  static const char kMagic[] = "__CLANG_OFFLOAD_BUNDLE__";
  const size_t ml = sizeof kMagic - 1;
  auto u64 = [&](size_t off, uint64_t *v) {
    if (off + 8 > size) return false;
    std::memcpy(v, img + off, 8);
    return true;
  };
  if (size >= 4 && std::memcmp(img, "\x7f" "ELF", 4) == 0) {
    *elf = img;
    *elf_size = size;
    return true;
  }
  if (size < ml + 8 || std::memcmp(img, kMagic, ml) != 0) return false;
  uint64_t n = 0;
  if (!u64(ml, &n)) return false;
  size_t off = ml + 8;
  for (uint64_t i = 0; i < n; ++i) {
    uint64_t eo, es, tl;
    if (!u64(off, &eo) || !u64(off + 8, &es) || !u64(off + 16, &tl) || off + 24 + tl > size) return false;
    const std::string triple(reinterpret_cast<const char *>(img + off + 24), size_t(tl));
    off += 24 + size_t(tl);
    if (triple.find("amdgcn") != std::string::npos && eo + es <= size) {
      *elf = img + eo;
      *elf_size = size_t(es);
      return true;
    }
  }
  return false;
}

// Kernel names of a 64-bit little-endian ELF: symbols `<name>.kd`.
bool elf_kernel_names(const unsigned char *elf, size_t size, std::vector<std::string> *out) {
  auto rd = [&](size_t off, size_t n, void *dst) {
    if (off + n > size) return false;
    std::memcpy(dst, elf + off, n);
    return true;
  };
  uint64_t shoff = 0;
  uint16_t shentsize = 0, shnum = 0;
  if (size < 64 || elf[4] != 2 /* ELFCLASS64 */ || !rd(0x28, 8, &shoff) || !rd(0x3A, 2, &shentsize) ||
      !rd(0x3C, 2, &shnum) || shentsize < 64)
    return false;
  for (uint16_t i = 0; i < shnum; ++i) {
    const size_t sh = size_t(shoff) + size_t(i) * shentsize;
    uint32_t type = 0, link = 0;
    uint64_t off = 0, sz = 0, entsize = 0;
    if (!rd(sh + 4, 4, &type) || !rd(sh + 24, 8, &off) || !rd(sh + 32, 8, &sz) || !rd(sh + 40, 4, &link) ||
        !rd(sh + 56, 8, &entsize))
      return false;
    if (type != 2 /* SHT_SYMTAB */ || entsize < 24) continue;
    const size_t strsh = size_t(shoff) + size_t(link) * shentsize;
    uint64_t stroff = 0, strsz = 0;
    if (link >= shnum || !rd(strsh + 24, 8, &stroff) || !rd(strsh + 32, 8, &strsz) || stroff + strsz > size)
      return false;
    for (uint64_t k = 0; k + entsize <= sz; k += entsize) {
      uint32_t nm = 0;
      if (!rd(size_t(off + k), 4, &nm) || nm >= strsz) continue;
      const char *name = reinterpret_cast<const char *>(elf + stroff + nm);
      const size_t len = strnlen(name, size_t(strsz - nm));
      if (len > 3 && std::strcmp(name + len - 3, ".kd") == 0) out->emplace_back(name, len - 3);
    }
  }
  std::sort(out->begin(), out->end());
  out->erase(std::unique(out->begin(), out->end()), out->end());
  return !out->empty();
}

// Kept scratch buffer of one (stream, slot); its mutex is held by a lease.
struct KeptScratch {
  std::mutex mu;
  std::atomic<std::thread::id> owner{};  // the thread holding mu (a second lease from it is an error)
  void *ptr = nullptr;
  size_t bytes = 0;
};

struct DeviceState {
  std::once_flag once;
  tx_status status = TX_GENERIC_FAILURE;
  std::string error;
  int cus = 0;
  hipModule_t modules[static_cast<int>(CodeObject::Count)] = {};
  KernelTable kernels[static_cast<int>(CodeObject::Count)];
  // kept scratch buffers, keyed by (stream, slot); map_mu guards the map
  // itself only (never held while a lease is)
  std::mutex map_mu;
  std::map<std::pair<hipStream_t, int>, std::unique_ptr<KeptScratch>> scratch;
};

DeviceState g_devices[kMaxDevices];

tx_status build_table(const CodeObjectImage &img, hipModule_t mod, KernelTable *t, std::string *err) {
  const unsigned char *elf = nullptr;
  size_t elf_size = 0;
  std::vector<std::string> names;
  if (!find_device_elf(img.begin, size_t(img.end - img.begin), &elf, &elf_size) ||
      !elf_kernel_names(elf, elf_size, &names)) {
    *err = std::string("code object '") + img.name + "': no kernel symbols found";
    return TX_CODE_OBJECT_ERROR;
  }
  t->names = std::move(names);
  size_t cap = 16;
  while (cap < 2 * t->names.size()) cap *= 2;
  t->slots.assign(cap, KernelTable::Entry{});
  for (const std::string &n : t->names) {
    hipFunction_t fn = nullptr;
    const hipError_t e = hipModuleGetFunction(&fn, mod, n.c_str());
    if (e != hipSuccess) {
      *err = std::string("hipModuleGetFunction(") + n + "): " + hipGetErrorString(e);
      return TX_CODE_OBJECT_ERROR;
    }
    const uint64_t h = name_hash(n.c_str());
    size_t i = size_t(h) & (cap - 1);
    while (t->slots[i].name) i = (i + 1) & (cap - 1);
    t->slots[i] = KernelTable::Entry{h, n.c_str(), fn};
  }
  return TX_SUCCESS;
}

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
    tx_status ts = TX_SUCCESS;
    if (img.end <= img.begin) {
      ts = TX_CODE_OBJECT_ERROR;
      st.error = std::string("code object '") + img.name + "' is empty";
    } else if ((e = hipModuleLoadData(&st.modules[i], img.begin)) != hipSuccess) {
      ts = TX_CODE_OBJECT_ERROR;
      st.modules[i] = nullptr;
      st.error = std::string("hipModuleLoadData(") + img.name + "): " + hipGetErrorString(e);
    } else {
      ts = build_table(img, st.modules[i], &st.kernels[i], &st.error);
    }
    if (ts != TX_SUCCESS) {
      st.status = ts;
      for (int j = 0; j <= i; ++j) {
        if (st.modules[j]) (void)hipModuleUnload(st.modules[j]);
        st.modules[j] = nullptr;
        st.kernels[j] = KernelTable{};
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
  hipFunction_t fn = st->kernels[ci].find(name);
  if (!fn)
    return fail(TX_CODE_OBJECT_ERROR, "kernel '%s' not found in code object '%s'", name, kImages[ci].name);
  *out = fn;
  return TX_SUCCESS;
}

tx_status ScratchLease::acquire(hipStream_t stream, int slot, size_t bytes) {
  DeviceState *st = nullptr;
  tx_status s = device_state(&st);
  if (s != TX_SUCCESS) return s;
  if (lock_) return fail(TX_GENERIC_FAILURE, "scratch lease acquired twice");
  stream_ = stream;
  if (bytes > kKeptScratch) {
    hipError_t e = hipMallocAsync(&ptr_, bytes, stream);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      ptr_ = nullptr;
      return fail(TX_GENERIC_FAILURE, "scratch of %zu bytes: %s", bytes, hipGetErrorString(e));
    }
    g_scratch_allocs.fetch_add(1, std::memory_order_relaxed);
    own_ = true;
    return TX_SUCCESS;
  }
  KeptScratch *k;
  {
    std::lock_guard<std::mutex> g(st->map_mu);
    std::unique_ptr<KeptScratch> &slot_ptr = st->scratch[{stream, slot}];
    if (!slot_ptr) slot_ptr.reset(new KeptScratch);
    k = slot_ptr.get();
  }
  // only calls on this stream and slot wait here
  if (k->owner.load(std::memory_order_relaxed) == std::this_thread::get_id())
    return fail(TX_GENERIC_FAILURE, "scratch slot %d of this stream is already leased by this thread", slot);
  k->mu.lock();
  k->owner.store(std::this_thread::get_id(), std::memory_order_relaxed);
  lock_ = k;
  if (k->bytes < bytes) {
    if (k->ptr && hipFreeAsync(k->ptr, stream) != hipSuccess) (void)hipGetLastError();
    k->ptr = nullptr;
    k->bytes = 0;
    // round up so that slowly growing requests do not reallocate every call
    const size_t want = std::min(kKeptScratch, (bytes + (size_t(4) << 20) - 1) / (size_t(4) << 20) * (size_t(4) << 20));
    hipError_t e = hipMallocAsync(&k->ptr, want, stream);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      k->ptr = nullptr;
      return fail(TX_GENERIC_FAILURE, "scratch of %zu bytes: %s", want, hipGetErrorString(e));
    }
    g_scratch_allocs.fetch_add(1, std::memory_order_relaxed);
    k->bytes = want;
  }
  ptr_ = k->ptr;
  return TX_SUCCESS;
}

ScratchLease::~ScratchLease() {
  if (own_ && ptr_ && hipFreeAsync(ptr_, stream_) != hipSuccess) (void)hipGetLastError();
  if (lock_) {
    KeptScratch *k = static_cast<KeptScratch *>(lock_);
    k->owner.store(std::thread::id(), std::memory_order_relaxed);
    k->mu.unlock();
  }
}

void release_all_scratch() {
  for (int d = 0; d < kMaxDevices; ++d) {
    DeviceState &st = g_devices[d];
    std::lock_guard<std::mutex> g(st.map_mu);
    if (st.scratch.empty()) continue;
    int cur = 0;
    if (hipGetDevice(&cur) != hipSuccess || hipSetDevice(d) != hipSuccess) continue;
    for (auto &kv : st.scratch) {
      std::lock_guard<std::mutex> kg(kv.second->mu);
      if (kv.second->ptr && hipFree(kv.second->ptr) != hipSuccess) (void)hipGetLastError();
      kv.second->ptr = nullptr;
      kv.second->bytes = 0;
    }
    st.scratch.clear();
    (void)hipSetDevice(cur);
  }
}

int cu_count() {
  DeviceState *st = nullptr;
  if (device_state(&st) != TX_SUCCESS) return 0;
  return st->cus;
}

tx_status launch(hipFunction_t fn, unsigned grid_x, unsigned grid_y,
                 unsigned block_x, hipStream_t stream, void *args,
                 size_t args_size, const char *what, unsigned shared_bytes) {
  if (grid_x == 0 || grid_y == 0) return TX_SUCCESS;
  void *config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, args,
                    HIP_LAUNCH_PARAM_BUFFER_SIZE, &args_size,
                    HIP_LAUNCH_PARAM_END};
  hipError_t e = hipModuleLaunchKernel(fn, grid_x, grid_y, 1, block_x, 1, 1, shared_bytes,
                                       stream, nullptr, config);
  if (e != hipSuccess)
    return fail(TX_LAUNCH_ERROR, "launch of %s failed: %s", what,
                hipGetErrorString(e));
  return TX_SUCCESS;
}

}  // namespace tx

extern "C" {

TX_API const char *txGetLastError(void) { return tx::g_last_error.c_str(); }

TX_API uint64_t txScratchAllocations(void) { return tx::g_scratch_allocs.load(std::memory_order_relaxed); }

TX_API tx_status txInit(void) {
  tx::clear_error();
  hipFunction_t fn;
  // Loading happens inside device_state; resolving one kernel proves the
  // code objects are usable.  The no-allocation entry point's workspace is
  // looked up here too, so that entry point allocates nothing later.
  tx_status s = tx::get_kernel(tx::CodeObject::Fp8Codec, "tx_fp8_decode_e4m3fn_vec", &fn);
  if (s != TX_SUCCESS) return s;
  void *ws = nullptr;
  return tx::noalloc_scratch(&ws);
}

TX_API void txShutdown(void) {
  tx::release_all_scratch();
  for (int d = 0; d < tx::kMaxDevices; ++d) {
    tx::DeviceState &st = tx::g_devices[d];
    if (st.status != TX_SUCCESS) continue;
    int cur = 0;
    if (hipGetDevice(&cur) != hipSuccess) return;
    if (hipSetDevice(d) != hipSuccess) continue;
    for (int i = 0; i < static_cast<int>(tx::CodeObject::Count); ++i) {
      if (st.modules[i]) (void)hipModuleUnload(st.modules[i]);
      st.modules[i] = nullptr;
      st.kernels[i] = tx::KernelTable{};
    }
    // The once_flag cannot be reset; mark the device unusable after shutdown.
    st.status = TX_CODE_OBJECT_ERROR;
    st.error = "txShutdown() was called; code objects are unloaded";
    (void)hipSetDevice(cur);
  }
}

}  // extern "C"
