// A native caller of the plugin library: C++ against include/tx_plugin.h and
// libtxamd.so only (no Python, no torch), the way a Triton-extension host or
// a C++ serving stack would drive the ops.  It prints the registration
// table (txGetPluginInfo), runs each hot-path entry point once on device
// buffers it allocates, calls tt.fp_to_fp, tt.dot and tt.atomic_rmw again
// through the table (txFindOp / txInvokeOp, the OpInfo operand convention),
// and checks the results against closed forms: inputs
// are chosen so that every output is exactly representable, so the checks
// are bit-exact.  Without --check it then times the fp8 scaled GEMM at 8192^3
// and the 16 Mi fp32 -> e4m3fn convert with HIP events, after enough untimed
// launches (about 20 ms of work) for the clocks to settle.
//
// Exit status: 0 when every check passed, 1 otherwise, 2 on an API error.
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "tx_plugin.h"

#define HIP_CHECK(x)                                                                  \
  do {                                                                                \
    hipError_t e_ = (x);                                                              \
    if (e_ != hipSuccess) {                                                           \
      std::fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_)); \
      std::exit(2);                                                                   \
    }                                                                                 \
  } while (0)

#define TX_CHECK(x)                                                              \
  do {                                                                           \
    tx_status s_ = (x);                                                          \
    if (s_ != TX_SUCCESS) {                                                      \
      std::fprintf(stderr, "%s:%d %s: status %d: %s\n", __FILE__, __LINE__, #x,  \
                   int(s_), txGetLastError());                                   \
      std::exit(2);                                                              \
    }                                                                            \
  } while (0)

namespace {

int g_failures = 0;

void expect(bool ok, const char *what) {
  std::printf("  %-64s %s\n", what, ok ? "ok" : "FAILED");
  if (!ok) ++g_failures;
}

// Device buffer holding a host vector's bytes.
template <class T>
T *to_device(const std::vector<T> &h) {
  T *d = nullptr;
  HIP_CHECK(hipMalloc(&d, h.size() * sizeof(T)));
  HIP_CHECK(hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice));
  return d;
}

template <class T>
std::vector<T> to_host(const T *d, size_t n) {
  std::vector<T> h(n);
  HIP_CHECK(hipMemcpy(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost));
  return h;
}

template <class T>
bool all_equal(const std::vector<T> &v, T x) {
  for (const T &e : v)
    if (e != x) return false;
  return true;
}

float bits_f32(uint32_t b) {
  float f;
  std::memcpy(&f, &b, 4);
  return f;
}

// tt.fp_to_fp: every finite e4m3fn code decodes to fp32 and encodes back to
// itself (RNE, non-saturating); known codes decode to their values.
void check_fp_to_fp() {
  std::printf("tx_fp_to_fp\n");
  std::vector<uint8_t> codes(256);
  for (int i = 0; i < 256; ++i) codes[i] = uint8_t(i);
  uint8_t *dc = to_device(codes);
  float *df = nullptr;
  uint8_t *dr = nullptr;
  HIP_CHECK(hipMalloc(&df, 256 * sizeof(float)));
  HIP_CHECK(hipMalloc(&dr, 256));
  TX_CHECK(tx_fp_to_fp(dc, TX_FP8E4M3FN, df, TX_F32, 256, TX_RTNE, 0, nullptr));
  TX_CHECK(tx_fp_to_fp(df, TX_F32, dr, TX_FP8E4M3FN, 256, TX_RTNE, 0, nullptr));
  HIP_CHECK(hipDeviceSynchronize());
  const std::vector<float> f = to_host(df, 256);
  const std::vector<uint8_t> r = to_host(dr, 256);
  bool round_trip = true;
  for (int i = 0; i < 256; ++i)
    if ((i & 0x7F) != 0x7F && r[i] != codes[i]) round_trip = false;
  expect(round_trip, "e4m3fn -> fp32 -> e4m3fn keeps every finite code");
  expect(f[0x38] == 1.0f && f[0x7E] == 448.0f && f[0xC0] == -2.0f && f[0x01] == std::ldexp(1.0f, -9) &&
             std::isnan(f[0x7F]),
         "codes 0x38, 0x7E, 0xC0, 0x01, 0x7F decode to 1, 448, -2, 2^-9, NaN");
  HIP_CHECK(hipFree(dc));
  HIP_CHECK(hipFree(df));
  HIP_CHECK(hipFree(dr));
}

// tt.atomic_rmw scatter: 2^20 int32 ones into 1024 bins, bin i % 1024 each.
void check_scatter() {
  std::printf("tx_atomic_rmw_scatter\n");
  const int64_t n = int64_t(1) << 20, nbins = 1024;
  std::vector<int32_t> idx(n), val(n, 1);
  for (int64_t i = 0; i < n; ++i) idx[i] = int32_t((i * 7) % nbins);
  int32_t *didx = to_device(idx), *dval = to_device(val);
  int32_t *dbins = to_device(std::vector<int32_t>(nbins, 0));
  TX_CHECK(tx_atomic_rmw_scatter(dbins, TX_I32, nbins, didx, dval, nullptr, n, TX_RMW_ADD, nullptr, nullptr));
  HIP_CHECK(hipDeviceSynchronize());
  expect(all_equal(to_host(dbins, nbins), int32_t(n / nbins)), "every bin counts 1024 updates");
  HIP_CHECK(hipFree(didx));
  HIP_CHECK(hipFree(dval));
  HIP_CHECK(hipFree(dbins));
}

// fp8 scaled dot: A and B all 1.0 (e4m3fn 0x38), scales 0.5: C = 0.25 K.
void check_dot_fp8() {
  std::printf("tx_dot_fp8_scaled\n");
  const int64_t M = 256, N = 256, K = 256;
  uint8_t *dA = to_device(std::vector<uint8_t>(M * K, 0x38)), *dB = to_device(std::vector<uint8_t>(N * K, 0x38));
  float *dsa = to_device(std::vector<float>(M, 0.5f)), *dsb = to_device(std::vector<float>(N, 0.5f));
  uint16_t *dC = nullptr;
  HIP_CHECK(hipMalloc(&dC, M * N * 2));
  TX_CHECK(tx_dot_fp8_scaled(dA, TX_FP8E4M3FN, K, dsa, dB, TX_FP8E4M3FN, K, dsb, dC, N, M, N, K, nullptr));
  HIP_CHECK(hipDeviceSynchronize());
  expect(all_equal(to_host(dC, M * N), uint16_t(0x4280)), "256^3, operands 1, scales 0.5: every output bf16 64");
  HIP_CHECK(hipFree(dA));
  HIP_CHECK(hipFree(dB));
  HIP_CHECK(hipFree(dsa));
  HIP_CHECK(hipFree(dsb));
  HIP_CHECK(hipFree(dC));
}

// 16-bit dot with a row-major K x N B (the reference's matmul operand): A
// all 1.0, B all 0.5 in fp16: C = 0.5 K.
void check_dot16_kn() {
  std::printf("tx_dot (fp16, B row-major K x N)\n");
  const int64_t M = 512, N = 512, K = 512;
  uint16_t *dA = to_device(std::vector<uint16_t>(M * K, 0x3C00));
  uint16_t *dB = to_device(std::vector<uint16_t>(K * N, 0x3800));
  uint16_t *dC = nullptr;
  HIP_CHECK(hipMalloc(&dC, M * N * 2));
  TX_CHECK(tx_dot(dA, TX_F16, K, dB, TX_B_KN, N, dC, TX_F16, N, M, N, K, nullptr));
  HIP_CHECK(hipDeviceSynchronize());
  expect(all_equal(to_host(dC, M * N), uint16_t(0x5C00)), "512^3, A 1, B 0.5: every output fp16 256");
  HIP_CHECK(hipFree(dA));
  HIP_CHECK(hipFree(dB));
  HIP_CHECK(hipFree(dC));
}

// fp8 dequant GEMV: x 1.0 (bf16), W 1.0 (e5m2 0x3C), group scales 0.25 per
// 128 K: y = 0.25 K.
void check_gemv() {
  std::printf("tx_gemv_fp8_dequant\n");
  const int64_t M = 1, N = 1024, K = 4096, G = 128;
  uint16_t *dx = to_device(std::vector<uint16_t>(M * K, 0x3F80));
  uint8_t *dW = to_device(std::vector<uint8_t>(N * K, 0x3C));
  float *ds = to_device(std::vector<float>(N * (K / G), 0.25f));
  uint16_t *dy = nullptr;
  HIP_CHECK(hipMalloc(&dy, M * N * 2));
  TX_CHECK(tx_gemv_fp8_dequant(dx, K, dW, TX_FP8E5M2, K, ds, K / G, G, dy, N, M, N, K, nullptr));
  HIP_CHECK(hipDeviceSynchronize());
  expect(all_equal(to_host(dy, M * N), uint16_t(0x4480)), "M = 1, K = 4096, scales 0.25: every output bf16 1024");
  HIP_CHECK(hipFree(dx));
  HIP_CHECK(hipFree(dW));
  HIP_CHECK(hipFree(ds));
  HIP_CHECK(hipFree(dy));
}

tx_value ptr_v(const void *p) {
  tx_value v{};
  v.kind = TX_VALUE_PTR;
  v.u.ptr = const_cast<void *>(p);
  return v;
}

tx_value int_v(int64_t i) {
  tx_value v{};
  v.kind = TX_VALUE_INT;
  v.u.i = i;
  return v;
}

// The same ops through the registration table, as Triton's loader reaches a
// plugin's ops: txFindOp / txInvokeOp with the OpInfo operand convention
// (operands[0] the result slot, inputs after it, options as integers).
void check_table_ops() {
  std::printf("txFindOp / txInvokeOp\n");
  const tx_op_info *dot = txFindOp("tt.dot");
  expect(dot && dot->fn && dot->signature && std::strncmp(dot->signature, "C:", 2) == 0,
         "tt.dot is registered with its operand signature");
  expect(txFindOp("tt.no_such_op") == nullptr, "an unknown name is not found");
  expect(txInvokeOp("tt.no_such_op", nullptr, 0, nullptr) == TX_UNKNOWN_OP, "invoking it returns TX_UNKNOWN_OP");

  {  // tt.fp_to_fp: e4m3fn 0x38 (1.0) -> fp32
    const int64_t n = 4096;
    uint8_t *src = to_device(std::vector<uint8_t>(n, 0x38));
    float *dst = nullptr;
    HIP_CHECK(hipMalloc(&dst, n * sizeof(float)));
    tx_value ops[7] = {ptr_v(dst), ptr_v(src), int_v(n), int_v(TX_FP8E4M3FN), int_v(TX_F32), int_v(TX_RTNE), int_v(0)};
    TX_CHECK(txInvokeOp("tt.fp_to_fp", ops, 7, nullptr));
    HIP_CHECK(hipDeviceSynchronize());
    expect(all_equal(to_host(dst, n), 1.0f), "tt.fp_to_fp (7 operands): 4096 codes 0x38 decode to 1");
    HIP_CHECK(hipFree(src));
    HIP_CHECK(hipFree(dst));
  }
  {  // tt.dot, 9 operands: bf16, B N x K; A 1, B 0.5 -> C = 0.5 K
    const int64_t M = 256, N = 256, K = 256;
    uint16_t *dA = to_device(std::vector<uint16_t>(M * K, 0x3F80));
    uint16_t *dB = to_device(std::vector<uint16_t>(N * K, 0x3F00));
    uint16_t *dC = nullptr;
    HIP_CHECK(hipMalloc(&dC, M * N * 2));
    tx_value ops[9] = {ptr_v(dC), ptr_v(dA), ptr_v(dB), int_v(M), int_v(N), int_v(K), int_v(K), int_v(K), int_v(N)};
    TX_CHECK(txInvokeOp("tt.dot", ops, 9, nullptr));
    HIP_CHECK(hipDeviceSynchronize());
    expect(all_equal(to_host(dC, M * N), uint16_t(0x4300)), "tt.dot (9 operands): 256^3 bf16, every output 128");
    HIP_CHECK(hipFree(dA));
    HIP_CHECK(hipFree(dB));
    HIP_CHECK(hipFree(dC));
  }
  {  // tt.atomic_rmw: 2^16 int32 ones into 1024 bins, (3 i) mod 1024
    const int64_t n = int64_t(1) << 16, nbins = 1024;
    std::vector<int32_t> idx(n);
    for (int64_t i = 0; i < n; ++i) idx[i] = int32_t((3 * i) % nbins);
    int32_t *didx = to_device(idx), *dval = to_device(std::vector<int32_t>(n, 1));
    int32_t *dbins = to_device(std::vector<int32_t>(nbins, 0));
    tx_value ops[9] = {ptr_v(dbins), ptr_v(didx), ptr_v(dval), ptr_v(nullptr), ptr_v(nullptr),
                       int_v(nbins), int_v(n),    int_v(TX_I32), int_v(TX_RMW_ADD)};
    TX_CHECK(txInvokeOp("tt.atomic_rmw", ops, 9, nullptr));
    HIP_CHECK(hipDeviceSynchronize());
    expect(all_equal(to_host(dbins, nbins), int32_t(n / nbins)), "tt.atomic_rmw (9 operands): every bin counts 64");
    HIP_CHECK(hipFree(didx));
    HIP_CHECK(hipFree(dval));
    HIP_CHECK(hipFree(dbins));
  }
}

// Average milliseconds of `iters` launches of f after `warm` untimed ones.
template <class F>
float time_ms(F &&f, int warm, int iters) {
  for (int i = 0; i < warm; ++i) f();
  hipEvent_t a, b;
  HIP_CHECK(hipEventCreate(&a));
  HIP_CHECK(hipEventCreate(&b));
  HIP_CHECK(hipEventRecord(a, nullptr));
  for (int i = 0; i < iters; ++i) f();
  HIP_CHECK(hipEventRecord(b, nullptr));
  HIP_CHECK(hipEventSynchronize(b));
  float ms = 0.0f;
  HIP_CHECK(hipEventElapsedTime(&ms, a, b));
  HIP_CHECK(hipEventDestroy(a));
  HIP_CHECK(hipEventDestroy(b));
  return ms / float(iters);
}

void bench() {
  std::printf("timings (one buffer set, inputs reused)\n");
  const int64_t S = 8192;
  std::vector<uint8_t> codes(S * S);
  uint32_t x = 12345u;
  for (auto &c : codes) {  // finite e4m3fn codes of either sign
    x = x * 1664525u + 1013904223u;
    c = uint8_t((x >> 24) % 0x7F) | uint8_t((x >> 16) & 0x80);
  }
  uint8_t *dA = to_device(codes), *dB = to_device(codes);
  float *dsa = to_device(std::vector<float>(S, 1.0f / 256)), *dsb = to_device(std::vector<float>(S, 1.0f / 256));
  uint16_t *dC = nullptr;
  HIP_CHECK(hipMalloc(&dC, S * S * 2));
  const float gemm_ms = time_ms(
      [&] { TX_CHECK(tx_dot_fp8_scaled(dA, TX_FP8E4M3FN, S, dsa, dB, TX_FP8E4M3FN, S, dsb, dC, S, S, S, S, nullptr)); },
      50, 100);
  std::printf("  fp8 scaled GEMM 8192^3: %.1f us, %.0f TFLOP/s\n", gemm_ms * 1e3, 2.0 * S * S * S / (gemm_ms * 1e-3) / 1e12);
  const int64_t n = int64_t(1) << 24;
  std::vector<float> src(n);
  for (int64_t i = 0; i < n; ++i) src[i] = bits_f32(0x3F000000u | uint32_t((i * 2654435761u) & 0x7FFFFFu));
  float *dsrc = to_device(src);
  uint8_t *ddst = nullptr;
  HIP_CHECK(hipMalloc(&ddst, n));
  const float cvt_ms = time_ms([&] { TX_CHECK(tx_fp_to_fp(dsrc, TX_F32, ddst, TX_FP8E4M3FN, n, TX_RTNE, 0, nullptr)); }, 200, 500);
  std::printf("  fp32 -> e4m3fn 16 Mi: %.1f us, %.0f GB/s\n", cvt_ms * 1e3, 5.0 * n / (cvt_ms * 1e-3) / 1e9);
  HIP_CHECK(hipFree(dA));
  HIP_CHECK(hipFree(dB));
  HIP_CHECK(hipFree(dsa));
  HIP_CHECK(hipFree(dsb));
  HIP_CHECK(hipFree(dC));
  HIP_CHECK(hipFree(dsrc));
  HIP_CHECK(hipFree(ddst));
}

}  // namespace

int main(int argc, char **argv) {
  const bool check_only = argc > 1 && std::strcmp(argv[1], "--check") == 0;
  TX_CHECK(txInit());
  const tx_plugin_info *info = txGetPluginInfo();
  std::printf("%s %s (target %s, api %u): %zu ops\n", info->name, info->version, info->target, info->api_version,
              info->num_ops);
  for (size_t i = 0; i < info->num_ops; ++i) std::printf("  %s\n", info->ops[i].name);
  txReleasePluginInfo(info);
  check_fp_to_fp();
  check_scatter();
  check_dot_fp8();
  check_dot16_kn();
  check_gemv();
  check_table_ops();
  if (!check_only && g_failures == 0) bench();
  std::printf("%d check(s) failed\n", g_failures);
  txShutdown();
  return g_failures ? 1 : 0;
}
