// tt.dot entry points (bf16, fp8 with row/column scales, fp8 with MX block
// scales), the fp8 dequant GEMV, and their table registrations.
//
// Reference: tt.dot is converted by TritonDotPattern
// (uTLXConversionPatterns.cpp:227-296) and lowered to MFMA by Triton's AMD
// backend (accelerate_matmul, custom_stages.py:84-85); the only AMD kernel in
// the tree is matmul_kernel_pipelined_mi300 with its host wrapper
// (test_amd_gemm_pipelined.py:184-331): grouped tile rasterisation
// (:204-212), fp32 accumulation (:259-292), cast and masked store (:294-300).
#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdio>
#include <cstring>

#include "tx_kernel_args.h"
#include "tx_ops.h"

namespace tx {
namespace {

constexpr int kGroupM = 8;

// Largest load width (bytes) that every operand row start and the row length
// are aligned to, among `widths` (descending).
int pick_vec(const void *A, int64_t lda_b, const void *B, int64_t ldb_b, int64_t k_b,
             const int *widths, int nw) {
  for (int i = 0; i < nw; ++i) {
    const int w = widths[i];
    if (aligned(A, w) && aligned(B, w) && lda_b % w == 0 && ldb_b % w == 0 && k_b % w == 0)
      return w;
  }
  return widths[nw - 1];
}

tx_status check_gemm(const char *what, const void *A, int64_t lda, const void *B, int64_t ldb,
                     const void *C, int64_t ldc, int64_t M, int64_t N, int64_t K,
                     size_t c_align = 2) {
  if (M < 0 || N < 0 || K < 0)
    return fail(TX_INVALID_ARGUMENT, "%s: negative size (M=%lld N=%lld K=%lld)", what,
                (long long)M, (long long)N, (long long)K);
  if (M > INT32_MAX / 2 || N > INT32_MAX / 2 || K > INT32_MAX / 4)
    return fail(TX_UNSUPPORTED, "%s: size exceeds 32-bit tile indexing", what);
  if (M == 0 || N == 0) return TX_SUCCESS;
  if (!C || (K > 0 && (!A || !B))) return fail(TX_INVALID_ARGUMENT, "%s: NULL buffer", what);
  if (lda < K || ldb < K || ldc < N)
    return fail(TX_INVALID_ARGUMENT, "%s: stride smaller than row length (lda=%lld ldb=%lld ldc=%lld)",
                what, (long long)lda, (long long)ldb, (long long)ldc);
  if (!aligned(C, c_align))
    return fail(TX_INVALID_ARGUMENT, "%s: C must be %zu-byte aligned", what, c_align);
  return TX_SUCCESS;
}

// Pick the tile: 256x256 when it still yields at least one tile per CU,
// otherwise 128x128.
bool use_big_tile(int64_t M, int64_t N) {
  const int64_t big = ((M + 255) / 256) * ((N + 255) / 256);
  return big >= cu_count();
}

tx_status launch_gemm(const char *kname, CodeObject co, tx_gemm_args &args, int tile_m, int tile_n,
                      hipStream_t s, unsigned threads = 256, int splits = 1) {
  args.tiles_m = int32_t((args.M + tile_m - 1) / tile_m);
  args.tiles_n = int32_t((args.N + tile_n - 1) / tile_n);
  args.group_m = std::min<int32_t>(kGroupM, args.tiles_m);
  hipFunction_t fn;
  TX_TRY(get_kernel(co, kname, &fn));
  const int64_t grid = int64_t(args.tiles_m) * args.tiles_n * splits;
  if (grid > INT32_MAX) return fail(TX_UNSUPPORTED, "%s: too many tiles", kname);
  return launch(fn, unsigned(grid), 1, threads, s, &args, sizeof args, kname);
}

// Wavefronts per workgroup of the fast path (two per SIMD) and of its
// persistent variant (one per SIMD).
constexpr int kFastWaves = 8;
constexpr int kPersistWaves = 4;
// Largest M served by the skinny fp8 kernel (4 blocks of 16 rows).
constexpr int64_t kSkinnyMaxM = 64;
// Split K only while every split keeps at least this many 128-byte K steps.
constexpr int64_t kMinStepsPerSplit = 4;
constexpr int64_t kMaxSplits = 16;

// The LDS-DMA fast path needs 16-byte aligned rows and a row length that is a
// multiple of 16 bytes, and operands small enough that a 32-bit buffer offset
// with the top bit clear addresses them (out-of-range lanes use 0x80000000).
bool fast_ok(const void *A, int64_t lda_b, const void *B, int64_t ldb_b, int64_t k_b, int64_t M,
             int64_t N) {
  if (!aligned(A, 16) || !aligned(B, 16) || lda_b % 16 || ldb_b % 16 || k_b % 16) return false;
  const int64_t lim = int64_t(1) << 31;
  return (M - 1) * lda_b + k_b < lim && (N - 1) * ldb_b + k_b < lim;
}

// 16-bit operands the fast path also reads in place (fast::KTail in
// gemm_fast.h, the persistent and the 256 x 128 tiles): rows 4-byte
// aligned, a row length of whole 4-byte words (the last chunk of a row is
// fetched as the row's last 16 bytes, which must stay 4-byte aligned for the
// buffer loads), and one that is not a whole number of 16-byte chunks only
// with at least two K steps.  An odd K takes the padded copies.
bool fast16_ragged_ok(const void *A, int64_t lda_b, const void *B, int64_t ldb_b, int64_t k_b, int64_t M,
                      int64_t N) {
  if (!aligned(A, 16) || !aligned(B, 16) || lda_b % 4 || ldb_b % 4 || k_b % 4 || (k_b % 16 && k_b <= 128))
    return false;
  const int64_t lim = int64_t(1) << 31;
  return (M - 1) * lda_b + k_b + 16 < lim && (N - 1) * ldb_b + k_b + 16 < lim;
}

// Launch the fast path (kernel `base`, or `base`_n128): 256x256 tiles while
// they give at least one tile per CU (see kStripMaxN for a narrow column
// tail); otherwise 256x128 tiles, and when those
// still leave CUs idle, K is split (at most 16 ways, at least 4 K steps per
// split) into fp32 partial planes in the library's stream scratch
// (ScratchLease, slot 1) that the `reduce` kernel sums, scales and rounds
// into C.
// A narrow tail of columns past the last full 256-column block (at most
// kStripMaxN) that would cost a whole extra round of 256x256 tiles is a
// separate, second fast-path product (few tiles, so 256x128 with K split).
constexpr int64_t kStripMaxN = 64;
// The 16-bit strip kernel (gemm_bf16.hip): up to 8 columns, a row per
// wavefront, 4 per workgroup of 256 threads.
constexpr int64_t kStripKernelCols = 8, kStripKernelRows = 4;

// The persistent 4-wavefront kernel (gemm_persist.h) takes the 256 x 256
// products it was built for: no fused epilogue or K split, at least two
// 128-byte K steps, N a multiple of 8, C addressable with 32-bit byte
// offsets.  `base`_persist: K a whole number of steps, C rows 16-byte
// aligned; `base`_persist_kt (16-bit operands, es == 2): any K and any C
// alignment.  Returns the kernel suffix, or nullptr.
const char *persist_variant(const tx_gemm_args &args, int64_t k_bytes, int es) {
  if (args.epi || args.splits > 1 || k_bytes < 256 || args.N % 8 != 0) return nullptr;
  const int64_t c_bytes = ((int64_t(args.M) - 1) * args.ldc + args.N) * 2;
  if (c_bytes + 16 >= (int64_t(1) << 31)) return nullptr;
  if (k_bytes % 128 == 0 && aligned(args.C, 16) && args.ldc % 8 == 0) return "_persist";
  return es == 2 && aligned(args.C, 2) ? "_persist_kt" : nullptr;
}

// The persistent tile's edge for a product with fewer 256 x 256 tiles than
// CUs: 128 with at least one 128 x 128 tile per CU, else 64 with at least one
// 64 x 64 tile per CU, or with fewer when a tile is at most kSmallMaxSteps
// 128-byte K steps (one short launch beats the K split and its reduce);
// else 0 (the 256 x 128 tile with K split).
constexpr int64_t kSmallMaxSteps = 32;
int small_persist_tile(int64_t M, int64_t N, int64_t k_bytes, int64_t cus) {
  for (int bt : {128, 64})
    if (((M + bt - 1) / bt) * ((N + bt - 1) / bt) >= cus) return bt;
  return (k_bytes + 127) / 128 <= kSmallMaxSteps ? 64 : 0;
}

// `narrow` sends the whole product to the 256 x 128 tile (the column tail
// of a wide product: at most kStripMaxN columns, and any K the 256 x 128
// tile takes, decided before the main part is launched).
tx_status launch_fast(const char *base, const char *reduce, CodeObject co, tx_gemm_args &args,
                      int64_t k_bytes, int es, hipStream_t s, bool persist = false, bool narrow = false) {
  const int64_t cus = cu_count();
  const int64_t tiles_m = (args.M + 255) / 256;
  char kname[96];
  // 256 x 256 tiles: the persistent kernel when it applies, else one
  // workgroup per tile
  auto launch_big = [&](tx_gemm_args &ga) -> tx_status {
    const char *pv = persist ? persist_variant(ga, k_bytes, es) : nullptr;
    if (pv) {
      std::snprintf(kname, sizeof kname, "%s%s", base, pv);
      ga.tiles_m = int32_t((ga.M + 255) / 256);
      ga.tiles_n = int32_t((ga.N + 255) / 256);
      ga.group_m = std::min<int32_t>(kGroupM, ga.tiles_m);
      hipFunction_t fn;
      TX_TRY(get_kernel(co, kname, &fn));
      const int64_t grid = std::min<int64_t>(int64_t(ga.tiles_m) * ga.tiles_n, cus);
      return launch(fn, unsigned(grid), 1, 64 * kPersistWaves, s, &ga, sizeof ga, kname);
    }
    // a ragged K (16-bit operands): the persistent and the 256 x 128 tiles only
    if (k_bytes % 16 != 0) return TX_UNSUPPORTED;
    std::snprintf(kname, sizeof kname, "%s", base);
    return launch_gemm(kname, co, ga, 256, 256, s, 64 * kFastWaves);
  };
  if (!narrow && tiles_m * ((args.N + 255) / 256) >= cus) {
    std::snprintf(kname, sizeof kname, "%s", base);
    const int64_t full = args.N / 256, tail = args.N % 256;
    const int64_t rounds_all = (tiles_m * (full + (tail > 0)) + cus - 1) / cus;
    const int64_t rounds_main = (tiles_m * full + cus - 1) / cus;
    if (full > 0 && tail > 0 && tail <= kStripMaxN && rounds_main < rounds_all) {
      tx_gemm_args strip_args = args;
      const int64_t n0 = full * 256;
      strip_args.B = static_cast<const uint8_t *>(args.B) + n0 * args.ldb * es;
      const int64_t ce = !args.epi ? 2 : args.out_kind == EPI_OUT_F32 ? 4 : args.out_kind >= EPI_OUT_E4M3FN ? 1 : 2;
      strip_args.C = static_cast<uint8_t *>(args.C) + n0 * ce;
      if (args.scale_b) strip_args.scale_b = args.scale_b + n0;
      if (args.bias) strip_args.bias = args.bias + n0;
      strip_args.N = int32_t(tail);
      args.N = int32_t(n0);
      TX_TRY(launch_big(args));
      const char *fast = std::strstr(base, "_fast");
      if (es == 2 && tail <= kStripKernelCols && k_bytes >= 16 && k_bytes % 4 == 0 && fast &&
          (args.lda * 2) % 4 == 0 &&
          (args.ldb * 2) % 4 == 0 && aligned(args.A, 4) && aligned(strip_args.B, 4)) {
        // 16-bit operands, at most 8 columns: the VALU strip kernel for
        // W >= tail columns (tx_gemm_<operands>_strip<W>[_out_<output>])
        const int w = tail <= 1 ? 1 : tail <= 2 ? 2 : tail <= 4 ? 4 : 8;
        std::snprintf(kname, sizeof kname, "%.*s_strip%d%s", int(fast - base), base, w, fast + 5);
        hipFunction_t fn;
        TX_TRY(get_kernel(co, kname, &fn));
        const int64_t grid = (int64_t(args.M) + kStripKernelRows - 1) / kStripKernelRows;
        return launch(fn, unsigned(grid), 1, 256, s, &strip_args, sizeof strip_args, kname);
      }
      return launch_fast(base, reduce, co, strip_args, k_bytes, es, s, persist, true);
    }
    return launch_big(args);
  }
  if (!narrow && persist && es == 2) {
    // fewer 256 x 256 tiles than CUs: the persistent tile at the edge
    // small_persist_tile picks (16-bit operands), no K split
    const char *pv = persist_variant(args, k_bytes, es);
    const int bt = small_persist_tile(args.M, args.N, k_bytes, cus);
    if (bt && pv && std::strcmp(pv, "_persist") == 0) {
      std::snprintf(kname, sizeof kname, "%s_persist%d", base, bt);
      args.tiles_m = int32_t((args.M + bt - 1) / bt);
      args.tiles_n = int32_t((args.N + bt - 1) / bt);
      args.group_m = std::min<int32_t>(kGroupM, args.tiles_m);
      hipFunction_t fn;
      TX_TRY(get_kernel(co, kname, &fn));
      const int64_t grid = std::min<int64_t>(int64_t(args.tiles_m) * args.tiles_n, cus);
      return launch(fn, unsigned(grid), 1, 64 * kPersistWaves, s, &args, sizeof args, kname);
    }
  }
  std::snprintf(kname, sizeof kname, "%s_n128", base);
  const int64_t tiles = tiles_m * ((args.N + 127) / 128);
  const int64_t ksteps = (k_bytes + 127) / 128;
  int64_t splits = std::min({kMaxSplits, cus / tiles, ksteps / kMinStepsPerSplit});
  ScratchLease part;  // held until every launch using it is enqueued
  if (splits >= 2) {
    const int64_t per = (ksteps + splits - 1) / splits;
    splits = (ksteps + per - 1) / per;  // no empty split
    const size_t bytes = size_t(splits) * size_t(args.M) * size_t(args.N) * sizeof(float);
    if (part.acquire(s, 1, bytes) != TX_SUCCESS) {
      clear_error();  // no workspace: run unsplit
    } else {
      args.splits = int32_t(splits);
      args.ksteps_split = int32_t(per);
      args.part = static_cast<float *>(part.ptr());
    }
  }
  if (!part.ptr()) return launch_gemm(kname, co, args, 256, 128, s, 64 * kFastWaves);
  TX_TRY(launch_gemm(kname, co, args, 256, 128, s, 64 * kFastWaves, int(args.splits)));
  hipFunction_t fn;
  TX_TRY(get_kernel(co, reduce, &fn));
  // a thread per 4 columns, or per 8 where the reduce's vector path takes N
  const int64_t units = args.M * (args.N % 8 == 0 ? args.N / 8 : (args.N + 3) / 4);
  const int64_t grid = std::min<int64_t>((units + 255) / 256, cus * 16);
  return launch(fn, unsigned(grid), 1, 256, s, &args, sizeof args, reduce);
}

// Operands the fast path cannot take (rows not 16-byte aligned or K * size
// not a multiple of 16 bytes) in a product of at least kPadMinWork
// multiply-adds are first copied into zero-padded rows in the library's
// stream scratch (ScratchLease, slot 0).  K is rounded up to a whole
// 128-byte step: the zeros add nothing to the sums, every row starts on a
// 128-byte line (a row segment of a step is then one cache line, not two),
// and no step needs the K-tail fill.
// Returns TX_UNSUPPORTED without launching anything when that is not
// possible, and the caller takes the generic kernel.
constexpr int64_t kPadMinWork = int64_t(1) << 30;

// Widest source load (8, 4, 2 or 1 bytes) that divides the base address,
// the row pitch and the row length of a padded copy's source.
int pad_load_bytes(const void *src, int64_t ld_bytes, int64_t row_bytes) {
  for (int w = 8; w > 1; w /= 2)
    if (aligned(src, w) && ld_bytes % w == 0 && row_bytes % w == 0) return w;
  return 1;
}

// Copy A and B into zero-padded rows of kp (K rounded up to a whole
// 128-byte step) in `ws` (stream scratch slot 0) and point args at them.
// TX_UNSUPPORTED (nothing launched) when an operand would exceed the GEMM's
// 31-bit buffer offsets or the scratch cannot be had.
tx_status pad_operands(const char *pad, CodeObject co, tx_gemm_args &args, int es, hipStream_t s,
                       ScratchLease &ws) {
  const int64_t per = 16 / es, step = 128 / es;
  const int64_t kp = (int64_t(args.K) + step - 1) / step * step;
  if ((int64_t(std::max(args.M, args.N)) * kp) * es >= (int64_t(1) << 31)) return TX_UNSUPPORTED;
  const size_t a_bytes = size_t(args.M) * size_t(kp) * es;
  const size_t b_bytes = size_t(args.N) * size_t(kp) * es;
  if (ws.acquire(s, 0, a_bytes + b_bytes) != TX_SUCCESS) {
    clear_error();
    return TX_UNSUPPORTED;
  }
  hipFunction_t fn;
  TX_TRY(get_kernel(co, pad, &fn));
  const int64_t cus = cu_count();
  uint8_t *wa = static_cast<uint8_t *>(ws.ptr()), *wb = wa + a_bytes;
  tx_pad_args pa{args.A, wa, args.lda, kp, args.M, args.K, int32_t(kp),
                 pad_load_bytes(args.A, args.lda * es, int64_t(args.K) * es)};
  const int64_t ga = std::min<int64_t>((int64_t(args.M) * kp / per + 255) / 256, cus * 16);
  TX_TRY(launch(fn, unsigned(ga), 1, 256, s, &pa, sizeof pa, pad));
  tx_pad_args pb{args.B, wb, args.ldb, kp, args.N, args.K, int32_t(kp),
                 pad_load_bytes(args.B, args.ldb * es, int64_t(args.K) * es)};
  const int64_t gb = std::min<int64_t>((int64_t(args.N) * kp / per + 255) / 256, cus * 16);
  TX_TRY(launch(fn, unsigned(gb), 1, 256, s, &pb, sizeof pb, pad));
  args.A = wa;
  args.lda = kp;
  args.B = wb;
  args.ldb = kp;
  args.K = int32_t(kp);
  return TX_SUCCESS;
}

tx_status launch_padded(const char *base, const char *reduce, const char *pad, CodeObject co,
                        tx_gemm_args &args, int es, hipStream_t s) {
  if (int64_t(args.M) * args.N * args.K < kPadMinWork) return TX_UNSUPPORTED;
  ScratchLease ws;  // held until every launch using it is enqueued
  TX_TRY(pad_operands(pad, co, args, es, s, ws));
  return launch_fast(base, reduce, co, args, int64_t(args.K) * es, es, s, true);
}

// tt.dot with its accumulator operand: the 256 x 128 tile writes the fp32
// sums to partial planes in stream scratch (slot 1; K split while the tiles
// leave CUs idle, at least one plane), and the split-K reduce sums them,
// applies the fp8 scales, adds the accumulator and rounds to the output type
// (its epilogue path, args.epi / out_kind / acc).  K = 0: the reduce alone.
tx_status launch_acc(const char *base, const char *reduce, CodeObject co, tx_gemm_args &args, int64_t k_bytes,
                     hipStream_t s) {
  const int64_t cus = cu_count();
  ScratchLease part;  // held until the reduce is enqueued
  if (k_bytes > 0) {
    const int64_t tiles = ((int64_t(args.M) + 255) / 256) * ((int64_t(args.N) + 127) / 128);
    const int64_t ksteps = (k_bytes + 127) / 128;
    int64_t splits = std::max<int64_t>(1, std::min({kMaxSplits, cus / tiles, ksteps / kMinStepsPerSplit}));
    const int64_t per = (ksteps + splits - 1) / splits;
    splits = (ksteps + per - 1) / per;  // no empty split
    TX_TRY(part.acquire(s, 1, size_t(splits) * size_t(args.M) * size_t(args.N) * sizeof(float)));
    args.splits = int32_t(splits);
    args.ksteps_split = int32_t(per);
    args.part = static_cast<float *>(part.ptr());
    char kname[96];
    std::snprintf(kname, sizeof kname, "%s_n128", base);
    TX_TRY(launch_gemm(kname, co, args, 256, 128, s, 64 * kFastWaves, int(splits)));
  } else {
    args.splits = 0;  // no plane: D = round(C)
    args.part = nullptr;
  }
  hipFunction_t fn;
  TX_TRY(get_kernel(co, reduce, &fn));
  const int64_t units = int64_t(args.M) * ((int64_t(args.N) + 3) / 4);
  const int64_t grid = std::min<int64_t>((units + 255) / 256, cus * 16);
  return launch(fn, unsigned(grid), 1, 256, s, &args, sizeof args, reduce);
}

const char *fp8_name(tx_dtype t) {
  return t == TX_FP8E4M3FN ? "e4m3fn" : (t == TX_FP8E5M2 ? "e5m2" : nullptr);
}

}  // namespace

// A row-major K x N B (the reference's matmul operand) for the 16-bit dot:
// B^T into stream scratch `ws` (slot 0): N rows of kp = K rounded up to a
// whole 64-element (128-byte) step, zero-filled; A is copied into
// zero-padded rows of kp too when the fast path cannot read it as is.
// args.B / ldb (and A / lda / K) then describe the copies.
static tx_status transpose_kn(const char *what, tx_gemm_args &args, hipStream_t s, ScratchLease &ws) {
  const int64_t M = args.M, N = args.N, K = args.K;
  const void *A = args.A, *B = args.B;
  const int64_t lda = args.lda, ldb = args.ldb;
  const int64_t kp = (K + 63) / 64 * 64;
  const bool a_pad = !(aligned(A, 16) && (lda * 2) % 16 == 0 && (K * 2) % 16 == 0);
  const int64_t lim = int64_t(1) << 31;
  if (N * kp * 2 >= lim || (a_pad ? M * kp * 2 : (M - 1) * lda * 2 + K * 2) >= lim)
    return fail(TX_UNSUPPORTED, "%s: an operand exceeds the 2 GiB range of the GEMM's buffer loads", what);
  if (kp / 64 > 65535)
    return fail(TX_UNSUPPORTED, "%s: K = %lld too large for the transpose grid", what, (long long)K);
  const size_t bt_bytes = size_t(N) * size_t(kp) * 2;
  const size_t a_bytes = a_pad ? size_t(M) * size_t(kp) * 2 : 0;
  TX_TRY(ws.acquire(s, 0, bt_bytes + a_bytes));
  uint16_t *wb = static_cast<uint16_t *>(ws.ptr());
  uint16_t *wa = wb + size_t(N) * size_t(kp);
  const bool tvec = aligned(B, 16) && (ldb * 2) % 16 == 0;
  const char *tname = tvec ? "tx_gemm_16_transpose_kn_v16" : "tx_gemm_16_transpose_kn_v2";
  hipFunction_t fn;
  TX_TRY(get_kernel(CodeObject::GemmBf16, tname, &fn));
  tx_pad_args ta{B, wb, ldb, kp, int32_t(K), int32_t(N), int32_t(kp), 0};
  TX_TRY(launch(fn, unsigned((N + 63) / 64), unsigned(kp / 64), 256, s, &ta, sizeof ta, tname));
  args.B = wb;
  args.ldb = kp;
  if (a_pad) {
    TX_TRY(get_kernel(CodeObject::GemmBf16, "tx_gemm_bf16_pad_rows", &fn));
    tx_pad_args pa{A, wa, lda, kp, int32_t(M), int32_t(K), int32_t(kp), pad_load_bytes(A, lda * 2, K * 2)};
    const int64_t ga = std::min<int64_t>((M * kp / 8 + 255) / 256, int64_t(cu_count()) * 16);
    TX_TRY(launch(fn, unsigned(ga), 1, 256, s, &pa, sizeof pa, "tx_gemm_bf16_pad_rows"));
    args.A = wa;
    args.lda = kp;
    args.K = int32_t(kp);
  }
  return TX_SUCCESS;
}

// A row-major K x N B read in place by the persistent tile: the tile edge
// (256: `base`_persist_kn, 128 / 64: `base`_persist128_kn / _persist64_kn)
// launch_fast would give the product (256: at least one 256 x 256 tile per
// CU and no column strip split off; else small_persist_tile), under the
// `_persist` conditions (K a whole number of 64-element
// steps, N a multiple of 8, C rows 16-byte aligned), with A and B and their
// rows 16-byte aligned and both addressable with 32-bit byte offsets (B: its
// K rows plus a tile of columns).  0: the transpose pass instead.
static int persist_kn_tile(const tx_gemm_args &args) {
  const int64_t M = args.M, N = args.N, K = args.K, cus = cu_count();
  const int64_t tiles_m = (M + 255) / 256, full = N / 256, tail = N % 256;
  int bt = 256;
  if (tiles_m * ((N + 255) / 256) < cus) {
    bt = small_persist_tile(M, N, K * 2, cus);
    if (!bt) return 0;
  } else {
    const int64_t rounds_all = (tiles_m * (full + (tail > 0)) + cus - 1) / cus;
    const int64_t rounds_main = (tiles_m * full + cus - 1) / cus;
    if (full > 0 && tail > 0 && tail <= kStripMaxN && rounds_main < rounds_all) return 0;
  }
  const char *pv = persist_variant(args, K * 2, 2);
  if (!pv || std::strcmp(pv, "_persist") != 0) return 0;
  const int64_t lim = int64_t(1) << 31;
  const bool ok = aligned(args.A, 16) && (args.lda * 2) % 16 == 0 && (M - 1) * args.lda * 2 + K * 2 + 16 < lim &&
                  aligned(args.B, 16) && (args.ldb * 2) % 16 == 0 && (K - 1) * args.ldb * 2 + N * 2 + 512 < lim;
  return ok ? bt : 0;
}

// tt.dot with 16-bit operands (bf16 / fp16) and a 16-bit output.  Kernel
// names: tx_gemm_<operands>_<variant>[_out_<output>]; the split-K reduce
// is the output type's.
static tx_status dot16(const char *what, const void *A, tx_dtype ab, int64_t lda, const void *B,
                       tx_b_layout layout, int64_t ldb, void *C, tx_dtype ct, int64_t ldc,
                       int64_t M, int64_t N, int64_t K, tx_stream_t stream) {
  if (ab != TX_BF16 && ab != TX_F16)
    return fail(TX_INVALID_ARGUMENT, "%s: operand type must be bf16 or fp16 (got %d)", what, int(ab));
  if (ct != TX_BF16 && ct != TX_F16)
    return fail(TX_INVALID_ARGUMENT, "%s: output type must be bf16 or fp16 (got %d)", what, int(ct));
  if (layout != TX_B_NK && layout != TX_B_KN)
    return fail(TX_INVALID_ARGUMENT, "%s: B layout %d", what, int(layout));
  const bool kn = layout == TX_B_KN && K > 0;
  // B's row-length check is the layout's: K (N x K storage) or N (K x N)
  TX_TRY(check_gemm(what, A, lda, B, kn ? K : ldb, C, ldc, M, N, K));
  if (kn && ldb < N)
    return fail(TX_INVALID_ARGUMENT, "%s: stride smaller than row length (ldb=%lld < N=%lld)", what,
                (long long)ldb, (long long)N);
  if (M == 0 || N == 0) return TX_SUCCESS;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const char *pfx = ab == TX_BF16 ? "bf16" : "f16";
  const char *sfx = ct == ab ? "" : (ct == TX_F16 ? "_out_f16" : "_out_bf16");
  const char *reduce = ct == TX_BF16 ? "tx_gemm_bf16_splitk_reduce" : "tx_gemm_f16_splitk_reduce";
  char base[64];
  std::snprintf(base, sizeof base, "tx_gemm_%s_fast%s", pfx, sfx);
  tx_gemm_args args{A, B, C, nullptr, nullptr, lda, ldb, ldc, int32_t(M), int32_t(N),
                    int32_t(K), 0, 0, 0};
  if (kn) {
    if (const int bt = persist_kn_tile(args)) {
      // the persistent tile reads the row-major B itself (no transpose pass)
      char kname[96];
      if (bt == 256) std::snprintf(kname, sizeof kname, "%s_persist_kn", base);
      else std::snprintf(kname, sizeof kname, "%s_persist%d_kn", base, bt);
      args.tiles_m = int32_t((M + bt - 1) / bt);
      args.tiles_n = int32_t((N + bt - 1) / bt);
      args.group_m = std::min<int32_t>(kGroupM, args.tiles_m);
      hipFunction_t fn;
      TX_TRY(get_kernel(CodeObject::GemmBf16, kname, &fn));
      const int64_t grid = std::min<int64_t>(int64_t(args.tiles_m) * args.tiles_n, cu_count());
      return launch(fn, unsigned(grid), 1, 64 * kPersistWaves, s, &args, sizeof args, kname);
    }
    ScratchLease ws;  // held until every launch using it is enqueued
    TX_TRY(transpose_kn(what, args, s, ws));
    return launch_fast(base, reduce, CodeObject::GemmBf16, args, int64_t(args.K) * 2, 2, s, true);
  }
  if (layout == TX_B_KN) args.ldb = K;  // K = 0: B is never read
  if (fast_ok(A, lda * 2, B, args.ldb * 2, K * 2, M, N))
    return launch_fast(base, reduce, CodeObject::GemmBf16, args, K * 2, 2, s, true);
  if (fast16_ragged_ok(A, lda * 2, B, args.ldb * 2, K * 2, M, N)) {
    // TX_UNSUPPORTED (nothing launched): a shape only the 256 x 256 tile takes
    tx_gemm_args direct = args;
    const tx_status st = launch_fast(base, reduce, CodeObject::GemmBf16, direct, K * 2, 2, s, true);
    if (st != TX_UNSUPPORTED) return st;
    clear_error();
  }
  {
    tx_gemm_args padded = args;
    const tx_status st = launch_padded(base, reduce, "tx_gemm_bf16_pad_rows", CodeObject::GemmBf16,
                                       padded, 2, s);
    if (st != TX_UNSUPPORTED) return st;
    clear_error();
  }
  static const int widths[] = {16, 8, 2};
  const int vec = pick_vec(A, lda * 2, B, args.ldb * 2, K * 2, widths, 3);
  const int tile = use_big_tile(M, N) ? 256 : 128;
  char kname[64];
  std::snprintf(kname, sizeof kname, "tx_gemm_%s_%dx%d_v%d%s", pfx, tile, tile, vec, sfx);
  return launch_gemm(kname, CodeObject::GemmBf16, args, tile, tile, s);
}

static tx_status dot_bf16(const void *A, int64_t lda, const void *B, int64_t ldb, void *C,
                          int64_t ldc, int64_t M, int64_t N, int64_t K, tx_stream_t stream) {
  return dot16("tx_dot_bf16", A, TX_BF16, lda, B, TX_B_NK, ldb, C, TX_BF16, ldc, M, N, K, stream);
}

// The fp8 GEMM's optional epilogue (tx_dot_fp8_scaled_ex).
struct Epilogue {
  const float *bias = nullptr;
  int act = EPI_ACT_NONE;
  int out_kind = EPI_OUT_BF16;
  float out_mul = 1.0f;
  bool on() const { return bias || act != EPI_ACT_NONE || out_kind != EPI_OUT_BF16; }
};

// Skinny and generic kernels write scaled fp32 sums to a.part (stream
// scratch slot 1) when an epilogue is requested; this pass finishes them.
tx_status epilogue_pass(tx_gemm_args &args, hipStream_t s) {
  hipFunction_t fn;
  TX_TRY(get_kernel(CodeObject::GemmFp8, "tx_gemm_fp8_epilogue", &fn));
  const int64_t total = int64_t(args.M) * args.N;
  const int64_t grid = std::min<int64_t>((total + 255) / 256, int64_t(cu_count()) * 16);
  return launch(fn, unsigned(grid), 1, 256, s, &args, sizeof args, "tx_gemm_fp8_epilogue");
}

static tx_status dot_fp8_impl(const char *what, const void *A, tx_dtype a_type, int64_t lda,
                              const float *sa, const void *B, tx_dtype b_type, int64_t ldb,
                              const float *sb, void *C, int64_t ldc, int64_t M, int64_t N, int64_t K,
                              const Epilogue &epi, tx_stream_t stream) {
  const size_t ce = epi.out_kind == EPI_OUT_F32 ? 4 : epi.out_kind >= EPI_OUT_E4M3FN ? 1 : 2;
  TX_TRY(check_gemm(what, A, lda, B, ldb, C, ldc, M, N, K, ce));
  const char *fa = fp8_name(a_type), *fb = fp8_name(b_type);
  if (!fa || !fb)
    return fail(TX_INVALID_ARGUMENT, "%s: operand types must be fp8 (got %d, %d)", what,
                int(a_type), int(b_type));
  if (M == 0 || N == 0) return TX_SUCCESS;
  if (!sa || !sb) return fail(TX_INVALID_ARGUMENT, "%s: NULL scale vector", what);
  if (!aligned(sa, 4) || !aligned(sb, 4) || !aligned(epi.bias, 4))
    return fail(TX_INVALID_ARGUMENT, "%s: scales and bias must be 4-byte aligned", what);
  hipStream_t s = static_cast<hipStream_t>(stream);
  tx_gemm_args args{A, B, C, sa, sb, lda, ldb, ldc, int32_t(M), int32_t(N), int32_t(K), 0, 0, 0};
  const bool with_epi = epi.on();
  if (with_epi) {
    args.bias = epi.bias;
    args.act = epi.act;
    args.out_kind = epi.out_kind;
    args.out_mul = epi.out_mul;
    args.epi = 1;
  }
  // skinny / generic kernels with an epilogue: scaled sums into scratch first
  ScratchLease sums;
  auto with_sums = [&]() -> tx_status {
    TX_TRY(sums.acquire(s, 1, size_t(M) * size_t(N) * sizeof(float)));
    args.part = static_cast<float *>(sums.ptr());
    return TX_SUCCESS;
  };
  char kname[96];
  // Decode-sized M: stream B once with the skinny kernel (16 columns per
  // workgroup, K split over its wavefronts).
  if (M <= kSkinnyMaxM && K % 128 == 0 && aligned(A, 16) && aligned(B, 16) && lda % 16 == 0 &&
      ldb % 16 == 0 && ldb <= INT32_MAX / 16 && lda <= INT32_MAX / 64) {  // 32-bit buffer offsets
    const int mb = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
    const int64_t grid = (N + 15) / 16;
    // Many column blocks: 4 wavefronts each, with long K ranges per wave;
    // few: 16 (8 with 4 blocks of M) to keep enough loads in flight.
    const int waves = grid >= 2 * int64_t(cu_count()) ? 4 : (mb == 4 ? 8 : 16);
    std::snprintf(kname, sizeof kname, "tx_gemm_fp8_%s_%s_skinny_w%d_m%d", fa, fb, waves, mb);
    hipFunction_t fn;
    TX_TRY(get_kernel(CodeObject::GemmFp8, kname, &fn));
    if (with_epi) TX_TRY(with_sums());
    TX_TRY(launch(fn, unsigned(grid), 1, unsigned(64 * waves), s, &args, sizeof args, kname));
    return with_epi ? epilogue_pass(args, s) : TX_SUCCESS;
  }
  std::snprintf(kname, sizeof kname, "tx_gemm_fp8_%s_%s_fast%s", fa, fb, with_epi ? "_epi" : "");
  if (fast_ok(A, lda, B, ldb, K, M, N))
    return launch_fast(kname, "tx_gemm_fp8_splitk_reduce", CodeObject::GemmFp8, args, K, 1, s, true);
  {
    tx_gemm_args padded = args;
    const tx_status st = launch_padded(kname, "tx_gemm_fp8_splitk_reduce", "tx_gemm_fp8_pad_rows",
                                       CodeObject::GemmFp8, padded, 1, s);
    if (st != TX_UNSUPPORTED) return st;
    clear_error();
  }
  static const int widths[] = {16, 4, 1};
  const int vec = pick_vec(A, lda, B, ldb, K, widths, 3);
  const int tile = (vec != 1 && use_big_tile(M, N)) ? 256 : 128;
  std::snprintf(kname, sizeof kname, "tx_gemm_fp8_%s_%s_%dx%d_v%d", fa, fb, tile, tile, vec);
  if (with_epi) TX_TRY(with_sums());
  TX_TRY(launch_gemm(kname, CodeObject::GemmFp8, args, tile, tile, s));
  return with_epi ? epilogue_pass(args, s) : TX_SUCCESS;
}

static tx_status dot_fp8_scaled(const void *A, tx_dtype a_type, int64_t lda, const float *sa,
                                const void *B, tx_dtype b_type, int64_t ldb, const float *sb,
                                void *C, int64_t ldc, int64_t M, int64_t N, int64_t K,
                                tx_stream_t stream) {
  return dot_fp8_impl("tx_dot_fp8_scaled", A, a_type, lda, sa, B, b_type, ldb, sb, C, ldc, M, N, K,
                      Epilogue{}, stream);
}

// tt.dot with its accumulator operand c: TritonDotPattern keeps it as an
// operand (uTLXConversionPatterns.cpp:273, 290-291) and the reference's AMD
// kernel chains it through its K loop (accumulator = tl.dot(a, b,
// accumulator), test_amd_gemm_pipelined.py:274, 292):
//   D = A.B (times scale_a[m] scale_b[n] for fp8 operands) + C
// in fp32, rounded once to D's type (fp32, bf16 or fp16, nearest even).
static tx_status dot_acc(const void *A, tx_dtype a_type, int64_t lda, const float *sa, const void *B,
                         tx_dtype b_type, tx_b_layout layout, int64_t ldb, const float *sb, const float *Cacc,
                         int64_t ld_acc, void *D, tx_dtype d_type, int64_t ldd, int64_t M, int64_t N, int64_t K,
                         tx_stream_t stream) {
  const char *what = "tx_dot_acc";
  const char *fa = fp8_name(a_type), *fb = fp8_name(b_type);
  const bool fp8 = fa && fb;
  const bool b16 = (a_type == TX_BF16 || a_type == TX_F16) && b_type == a_type;
  const bool f32 = a_type == TX_F32 && b_type == TX_F32, i8 = a_type == TX_I8 && b_type == TX_I8;
  if (!fp8 && !b16 && !f32 && !i8)
    return fail(TX_INVALID_ARGUMENT,
                "%s: operands must be bf16, fp16, fp32 or int8 (both the same) or fp8 (got %d, %d)", what,
                int(a_type), int(b_type));
  if (layout != TX_B_NK && layout != TX_B_KN)
    return fail(TX_INVALID_ARGUMENT, "%s: B layout %d", what, int(layout));
  if (!b16 && layout != TX_B_NK)
    return fail(TX_UNSUPPORTED, "%s: fp8, fp32 and int8 operands take B stored N x K", what);
  if (f32 || i8) {
    if (d_type != (f32 ? TX_F32 : TX_I32))
      return fail(TX_INVALID_ARGUMENT, "%s: %s operands give %s output (got type %d)", what, f32 ? "fp32" : "int8",
                  f32 ? "fp32" : "int32", int(d_type));
  } else if (d_type != TX_F32 && d_type != TX_BF16 && d_type != TX_F16) {
    return fail(TX_INVALID_ARGUMENT, "%s: output type must be fp32, bf16 or fp16 (got %d)", what, int(d_type));
  }
  const size_t de = (d_type == TX_F32 || d_type == TX_I32) ? 4 : 2;
  const bool kn = layout == TX_B_KN && K > 0;
  TX_TRY(check_gemm(what, A, lda, B, kn ? K : ldb, D, ldd, M, N, K, de));
  if (kn && ldb < N)
    return fail(TX_INVALID_ARGUMENT, "%s: stride smaller than row length (ldb=%lld < N=%lld)", what,
                (long long)ldb, (long long)N);
  if (M == 0 || N == 0) return TX_SUCCESS;
  if (fp8 && (!sa || !sb)) return fail(TX_INVALID_ARGUMENT, "%s: fp8 operands need both scale vectors", what);
  if (!fp8 && (sa || sb)) return fail(TX_INVALID_ARGUMENT, "%s: scale vectors are for fp8 operands", what);
  if (!aligned(sa, 4) || !aligned(sb, 4))
    return fail(TX_INVALID_ARGUMENT, "%s: scales must be 4-byte aligned", what);
  if (Cacc) {
    if (ld_acc < N || !aligned(Cacc, 4))
      return fail(TX_INVALID_ARGUMENT, "%s: C needs ldc >= N and 4-byte alignment", what);
    if (static_cast<const void *>(Cacc) == D && !(de == 4 && ld_acc == ldd))
      return fail(TX_INVALID_ARGUMENT, "%s: C may be D itself only for an fp32 / int32 D with the same stride",
                  what);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (f32 || i8) {
    // the generic 128 x 128 tile with 32-bit outputs; its epilogue adds C
    const int es = f32 ? 4 : 1;
    static const int wf[] = {16, 8, 4}, wi[] = {16, 4, 1};
    const int vec = pick_vec(A, lda * es, B, ldb * es, K * es, f32 ? wf : wi, 3);
    tx_gemm_args g{A, B, D, nullptr, nullptr, lda, ldb, ldd, int32_t(M), int32_t(N), int32_t(K), 0, 0, 0};
    g.acc = Cacc;
    g.ld_acc = ld_acc;
    char kname[48];
    std::snprintf(kname, sizeof kname, "tx_gemm_%s_128x128_v%d", f32 ? "f32" : "i8", vec);
    return launch_gemm(kname, CodeObject::GemmBf16, g, 128, 128, s);
  }
  tx_gemm_args args{A, B, D, sa, sb, lda, ldb, ldd, int32_t(M), int32_t(N), int32_t(K), 0, 0, 0};
  args.epi = 1;
  args.act = EPI_ACT_NONE;
  args.out_mul = 1.0f;
  args.out_kind = d_type == TX_F32 ? EPI_OUT_F32 : d_type == TX_F16 ? EPI_OUT_F16 : EPI_OUT_BF16;
  args.acc = Cacc;
  args.ld_acc = ld_acc;
  const int es = fp8 ? 1 : 2;
  const CodeObject co = fp8 ? CodeObject::GemmFp8 : CodeObject::GemmBf16;
  char base[64];
  if (fp8) std::snprintf(base, sizeof base, "tx_gemm_fp8_%s_%s_fast", fa, fb);
  else std::snprintf(base, sizeof base, "tx_gemm_%s_fast", a_type == TX_BF16 ? "bf16" : "f16");
  const char *reduce = fp8 ? "tx_gemm_fp8_splitk_reduce" : "tx_gemm_bf16_splitk_reduce";
  if (K == 0) return launch_acc(base, reduce, co, args, 0, s);
  ScratchLease ws;  // operand copies (slot 0), held until the product is enqueued
  if (kn) {
    TX_TRY(transpose_kn(what, args, s, ws));
  } else if (!fast_ok(A, lda * es, B, ldb * es, K * es, M, N) &&
             !(b16 && fast16_ragged_ok(A, lda * es, B, ldb * es, K * es, M, N))) {
    const tx_status st =
        pad_operands(fp8 ? "tx_gemm_fp8_pad_rows" : "tx_gemm_bf16_pad_rows", co, args, es, s, ws);
    if (st == TX_UNSUPPORTED)
      return fail(TX_UNSUPPORTED, "%s: operands too large for the zero-padded copies", what);
    TX_TRY(st);
  }
  return launch_acc(base, reduce, co, args, int64_t(args.K) * es, s);
}

// The fused epilogue's options (bias, tx_activation, output type and, for
// fp8 outputs, the scale the output is divided by) into an Epilogue; *es =
// bytes per output element.
tx_status make_epilogue(const char *what, const float *bias, int activation, tx_dtype c_type,
                        float c_scale, Epilogue *e, size_t *es) {
  e->bias = bias;
  if (activation < TX_ACT_NONE || activation > TX_ACT_SILU)
    return fail(TX_INVALID_ARGUMENT, "%s: unknown activation %d", what, activation);
  e->act = activation;
  switch (c_type) {
    case TX_BF16: e->out_kind = EPI_OUT_BF16; *es = 2; break;
    case TX_F16: e->out_kind = EPI_OUT_F16; *es = 2; break;
    case TX_F32: e->out_kind = EPI_OUT_F32; *es = 4; break;
    case TX_FP8E4M3FN: e->out_kind = EPI_OUT_E4M3FN; *es = 1; break;
    case TX_FP8E5M2: e->out_kind = EPI_OUT_E5M2; *es = 1; break;
    default:
      return fail(TX_INVALID_ARGUMENT, "%s: output type must be bf16, fp16, fp32 or fp8 (got %d)", what,
                  int(c_type));
  }
  if (*es == 1) {
    if (!(c_scale > 0.0f) || !std::isfinite(c_scale))
      return fail(TX_INVALID_ARGUMENT, "%s: fp8 output needs a positive finite c_scale", what);
    e->out_mul = 1.0f / c_scale;
  }
  return TX_SUCCESS;
}

static tx_status dot_fp8_scaled_ex(const void *A, tx_dtype a_type, int64_t lda, const float *sa,
                                   const void *B, tx_dtype b_type, int64_t ldb, const float *sb,
                                   const float *bias, int activation, void *C, tx_dtype c_type,
                                   float c_scale, int64_t ldc, int64_t M, int64_t N, int64_t K,
                                   tx_stream_t stream) {
  const char *what = "tx_dot_fp8_scaled_ex";
  Epilogue e;
  size_t es;
  TX_TRY(make_epilogue(what, bias, activation, c_type, c_scale, &e, &es));
  return dot_fp8_impl(what, A, a_type, lda, sa, B, b_type, ldb, sb, C, ldc, M, N, K, e, stream);
}

// tt.dot_scaled with MX block scales (fp8 operands, or fp4 (e2m1) packed two
// per byte, e8m0 scales per 32 K elements).  The kernel walks operand bytes
// (fp4: a 128-byte step is 256 K values and 8 scale blocks, two scale dwords
// per row), and reads its operands through the fast path's LDS-DMA
// pipeline, so rows that are not 16-byte aligned (or K not a multiple of 16)
// are first copied into zero-padded rows (stream scratch slot 0, K rounded up
// to a 128-byte step).  The scales are always repacked step-major (slot 2),
// the layout in which a fragment's scales for one K step are one cache line.
static tx_status dot_scaled_mx(const void *A, tx_dtype a_type, int64_t lda, const uint8_t *sa,
                               int64_t ld_sa, const void *B, tx_dtype b_type, int64_t ldb,
                               const uint8_t *sb, int64_t ld_sb, void *C, tx_dtype c_type,
                               int64_t ldc, int64_t M, int64_t N, int64_t K, tx_stream_t stream) {
  const char *what = "tx_dot_scaled_mx";
  const bool fa4 = a_type == TX_FP4E2M1, fb4 = b_type == TX_FP4E2M1;
  const bool fp4 = fa4 && fb4;    // the fp4 x fp4 tile
  const bool mixed = fa4 != fb4;  // fp4 operand expanded to e4m3fn, then the fp8 tile
  if ((fa4 || fb4) && K % 2)
    return fail(TX_INVALID_ARGUMENT, "%s: fp4 operands need an even K (two values per byte)", what);
  const int64_t ka = fa4 ? K / 2 : K, kbb = fb4 ? K / 2 : K;  // operand row bytes
  const int64_t kb = std::min(ka, kbb);
  TX_TRY(check_gemm(what, A, lda, B, ldb, C, ldc, M, N, kb));
  if (M > 0 && N > 0 && (lda < ka || ldb < kbb))
    return fail(TX_INVALID_ARGUMENT, "%s: stride smaller than row length (lda=%lld ldb=%lld)", what,
                (long long)lda, (long long)ldb);
  const char *fa = fp4 ? "e2m1" : fa4 ? "e4m3fn" : fp8_name(a_type);
  const char *fb = fp4 ? "e2m1" : fb4 ? "e4m3fn" : fp8_name(b_type);
  if (!fa || !fb)
    return fail(TX_INVALID_ARGUMENT, "%s: operand types must be fp8 or fp4 (got %d, %d)", what,
                int(a_type), int(b_type));
  const char *fo = c_type == TX_BF16 ? "bf16" : c_type == TX_F16 ? "f16" : c_type == TX_F32 ? "f32" : nullptr;
  if (!fo)
    return fail(TX_INVALID_ARGUMENT, "%s: output type must be bf16, fp16 or fp32 (got %d)", what,
                int(c_type));
  if (c_type == TX_F32 && !aligned(C, 4))
    return fail(TX_INVALID_ARGUMENT, "%s: fp32 C must be 4-byte aligned", what);
  if (M == 0 || N == 0) return TX_SUCCESS;
  const int64_t nblk = (K + 31) / 32;
  if (K > 0 && (!sa || !sb)) return fail(TX_INVALID_ARGUMENT, "%s: NULL scale matrix", what);
  if (ld_sa < nblk || ld_sb < nblk)
    return fail(TX_INVALID_ARGUMENT, "%s: scale stride smaller than ceil(K / 32) (ld_sa=%lld ld_sb=%lld)",
                what, (long long)ld_sa, (long long)ld_sb);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t cus = cu_count();
  // the kernel walks operand bytes (fp4: K / 2 of them per row)
  tx_gemm_args args{A, B, C, nullptr, nullptr, lda, ldb, ldc, int32_t(M), int32_t(N), int32_t(kb), 0, 0, 0};

  // operands: as given, or zero-padded to whole 128-byte steps
  ScratchLease ws, wsc;  // held until every launch using them is enqueued
  int64_t kk = kb;       // row bytes the kernel runs over
  if (mixed && K > 0) {
    // the fp4 operand into e4m3fn rows of kp bytes (zeros past K); the fp8
    // one as given when the fast path can read it, else padded likewise
    const int64_t kp = (K + 127) / 128 * 128;
    const void *src4 = fa4 ? A : B, *src8 = fa4 ? B : A;
    const int64_t ld4 = fa4 ? lda : ldb, ld8 = fa4 ? ldb : lda;
    const int64_t rows4 = fa4 ? M : N, rows8 = fa4 ? N : M;
    const bool direct8 = aligned(src8, 16) && ld8 % 16 == 0 && K % 16 == 0 &&
                         (rows8 - 1) * ld8 + K < (int64_t(1) << 31);
    if (std::max(rows4, direct8 ? int64_t(0) : rows8) * kp >= (int64_t(1) << 31))
      return fail(TX_UNSUPPORTED, "%s: expanded operands exceed 32-bit offsets", what);
    const size_t b4 = size_t(rows4) * size_t(kp), b8 = direct8 ? 0 : size_t(rows8) * size_t(kp);
    TX_TRY(ws.acquire(s, 0, b4 + b8));
    uint8_t *w4 = static_cast<uint8_t *>(ws.ptr()), *w8 = w4 + b4;
    hipFunction_t fn;
    TX_TRY(get_kernel(CodeObject::GemmMx, "tx_gemm_mx_fp4_to_e4m3", &fn));
    tx_pad_args px{src4, w4, ld4, kp, int32_t(rows4), int32_t(K / 2), int32_t(kp), 0};
    TX_TRY(launch(fn, unsigned(std::min<int64_t>((rows4 * kp / 8 + 255) / 256, cus * 16)), 1, 256, s,
                  &px, sizeof px, "tx_gemm_mx_fp4_to_e4m3"));
    if (!direct8) {
      TX_TRY(get_kernel(CodeObject::GemmMx, "tx_gemm_mx_pad_rows", &fn));
      tx_pad_args pp{src8, w8, ld8, kp, int32_t(rows8), int32_t(K), int32_t(kp), pad_load_bytes(src8, ld8, K)};
      TX_TRY(launch(fn, unsigned(std::min<int64_t>((rows8 * kp / 16 + 255) / 256, cus * 16)), 1, 256, s,
                    &pp, sizeof pp, "tx_gemm_mx_pad_rows"));
    }
    const void *d8 = direct8 ? src8 : w8;
    const int64_t l8 = direct8 ? ld8 : kp;
    args.A = fa4 ? static_cast<const void *>(w4) : d8;
    args.lda = fa4 ? kp : l8;
    args.B = fa4 ? d8 : static_cast<const void *>(w4);
    args.ldb = fa4 ? l8 : kp;
    kk = direct8 ? K : kp;
    args.K = int32_t(kk);
  } else if (!fast_ok(A, lda, B, ldb, kb, M, N)) {
    const int64_t kp = (kb + 127) / 128 * 128;
    if (std::max(M, N) * kp >= (int64_t(1) << 31))
      return fail(TX_UNSUPPORTED, "%s: padded operands exceed 32-bit offsets", what);
    const size_t a_bytes = size_t(M) * size_t(kp), b_bytes = size_t(N) * size_t(kp);
    TX_TRY(ws.acquire(s, 0, a_bytes + b_bytes));
    hipFunction_t fn;
    TX_TRY(get_kernel(CodeObject::GemmMx, "tx_gemm_mx_pad_rows", &fn));
    uint8_t *wa = static_cast<uint8_t *>(ws.ptr()), *wb = wa + a_bytes;
    tx_pad_args pa{A, wa, lda, kp, int32_t(M), int32_t(kb), int32_t(kp), pad_load_bytes(A, lda, kb)};
    TX_TRY(launch(fn, unsigned(std::min<int64_t>((M * kp / 16 + 255) / 256, cus * 16)), 1, 256, s,
                  &pa, sizeof pa, "tx_gemm_mx_pad_rows"));
    tx_pad_args pb{B, wb, ldb, kp, int32_t(N), int32_t(kb), int32_t(kp), pad_load_bytes(B, ldb, kb)};
    TX_TRY(launch(fn, unsigned(std::min<int64_t>((N * kp / 16 + 255) / 256, cus * 16)), 1, 256, s,
                  &pb, sizeof pb, "tx_gemm_mx_pad_rows"));
    args.A = wa;
    args.lda = kp;
    args.B = wb;
    args.ldb = kp;
    args.K = int32_t(kp);
    kk = kp;
  }
  // scales: repacked step-major (one or two 128-byte lines per fragment and
  // step: a 128-byte step holds 4 blocks of fp8, 8 of fp4), rows padded to
  // whole tiles, blocks past ceil(K / 32) set to 2^0
  const int64_t steps = (kk + 127) / 128;
  const int64_t sd = fp4 ? 2 : 1;  // scale dwords per row and step
  const int64_t rows_a = (M + 255) / 256 * 256, rows_b = (N + 255) / 256 * 256;
  if (steps * 4 * sd * std::max(rows_a, rows_b) >= (int64_t(1) << 31))
    return fail(TX_UNSUPPORTED, "%s: scale matrices exceed 32-bit offsets", what);
  if (steps > 0) {
    const size_t pa_bytes = size_t(steps * sd) * size_t(rows_a) * 4, pb_bytes = size_t(steps * sd) * size_t(rows_b) * 4;
    TX_TRY(wsc.acquire(s, 2, pa_bytes + pb_bytes));
    hipFunction_t fn;
    TX_TRY(get_kernel(CodeObject::GemmMx, "tx_gemm_mx_pack_scales", &fn));
    uint8_t *p = static_cast<uint8_t *>(wsc.ptr());
    // one workgroup per 64 rows x 32 scale dwords (128 blocks)
    const int64_t dcols = (steps * sd + 31) / 32;
    const int64_t ga = (rows_a / 64) * dcols, gb = (rows_b / 64) * dcols;
    if (ga + gb > INT32_MAX) return fail(TX_UNSUPPORTED, "%s: scale repack grid too large", what);
    tx_mx_pack2_args pk{{{sa, p, ld_sa, int32_t(M), int32_t(nblk), int32_t(steps), int32_t(rows_a), int32_t(sd), 0},
                         {sb, p + pa_bytes, ld_sb, int32_t(N), int32_t(nblk), int32_t(steps), int32_t(rows_b),
                          int32_t(sd), 0}},
                        int32_t(ga), 0};
    TX_TRY(launch(fn, unsigned(ga + gb), 1, 256, s, &pk, sizeof pk, "tx_gemm_mx_pack_scales"));
    args.mx_a = p;
    args.ld_mxa = rows_a * 4 * sd;
    args.mx_b = p + pa_bytes;
    args.ld_mxb = rows_b * 4 * sd;
  }

  // 256x256 tiles while they give every CU one, else 256x128, with K split
  // into fp32 partial planes (slot 1) while tiles still leave CUs idle
  const bool big = ((M + 255) / 256) * ((N + 255) / 256) >= cus;
  char kname[80];
  std::snprintf(kname, sizeof kname, "tx_gemm_mx_%s_%s_%s%s", fa, fb, fo, big ? "" : "_n128");
  if (big) return launch_gemm(kname, CodeObject::GemmMx, args, 256, 256, s, 256);
  const int64_t tiles = ((M + 255) / 256) * ((N + 127) / 128);
  int64_t splits = std::min({kMaxSplits, cus / tiles, steps / kMinStepsPerSplit});
  ScratchLease part;
  if (splits >= 2) {
    const int64_t per = (steps + splits - 1) / splits;
    splits = (steps + per - 1) / per;  // no empty split
    const size_t bytes = size_t(splits) * size_t(M) * size_t(N) * sizeof(float);
    if (part.acquire(s, 1, bytes) != TX_SUCCESS) {
      clear_error();  // no workspace: run unsplit
    } else {
      args.splits = int32_t(splits);
      args.ksteps_split = int32_t(per);
      args.part = static_cast<float *>(part.ptr());
    }
  }
  if (!part.ptr()) return launch_gemm(kname, CodeObject::GemmMx, args, 256, 128, s, 512);
  TX_TRY(launch_gemm(kname, CodeObject::GemmMx, args, 256, 128, s, 512, int(args.splits)));
  char rname[64];
  std::snprintf(rname, sizeof rname, "tx_gemm_mx_splitk_reduce_%s", fo);
  hipFunction_t fn;
  TX_TRY(get_kernel(CodeObject::GemmMx, rname, &fn));
  const int64_t quads = M * ((N + 3) / 4);
  const int64_t grid = std::min<int64_t>((quads + 255) / 256, cus * 16);
  return launch(fn, unsigned(grid), 1, 256, s, &args, sizeof args, rname);
}

// Grouped (offsets != NULL) or batched fp8 scaled dot, bf16 out: the fast
// tile over every (problem, tile) pair in one launch (tx_grouped_args).  The
// group sizes stay on the device: a one-workgroup scan turns the offsets
// into m-tile prefix sums (stream scratch slot 1), and the grid covers
// ceil(M / 256) + groups m tiles, of which the ones past the last problem
// exit at once.  Operands must be what the fast path reads in place
// (16-byte aligned rows, K a multiple of 16 bytes).
static tx_status dot_fp8_grouped_impl(const char *what, const void *A, tx_dtype a_type, int64_t lda,
                                      int64_t stride_a, const float *sa, int64_t stride_sa,
                                      const void *B, tx_dtype b_type, int64_t ldb, int64_t stride_b,
                                      const float *sb, int64_t stride_sb, void *C, int64_t ldc,
                                      int64_t stride_c, const int32_t *offsets, int64_t groups,
                                      int64_t M, int64_t N, int64_t K, tx_stream_t stream,
                                      const Epilogue &e = Epilogue{}, size_t es = 2,
                                      int64_t stride_bias = 0, int32_t *prefix_ws = nullptr) {
  const char *fa = fp8_name(a_type), *fb = fp8_name(b_type);
  if (!fa || !fb)
    return fail(TX_INVALID_ARGUMENT, "%s: operand types must be fp8 (got %d, %d)", what, int(a_type),
                int(b_type));
  if (groups < 0) return fail(TX_INVALID_ARGUMENT, "%s: negative group count", what);
  if (groups > INT32_MAX / 2) return fail(TX_UNSUPPORTED, "%s: too many groups", what);
  TX_TRY(check_gemm(what, A, lda, B, ldb, C, ldc, M, N, K, es));
  if (groups == 0 || M == 0 || N == 0) return TX_SUCCESS;
  if (!sa || !sb) return fail(TX_INVALID_ARGUMENT, "%s: NULL scale vector", what);
  if (e.bias && (!aligned(e.bias, 4) || stride_bias < 0))
    return fail(TX_INVALID_ARGUMENT, "%s: bias must be 4-byte aligned with a non-negative stride", what);
  if (!aligned(sa, 4) || !aligned(sb, 4))
    return fail(TX_INVALID_ARGUMENT, "%s: scales must be 4-byte aligned", what);
  const bool grouped = offsets != nullptr;
  if (stride_b < 0 || stride_sb < 0 || (!grouped && (stride_a < 0 || stride_sa < 0 || stride_c < 0)))
    return fail(TX_INVALID_ARGUMENT, "%s: negative stride", what);
  if (K > 0 && (!aligned(A, 16) || !aligned(B, 16) || lda % 16 || ldb % 16 || K % 16 || stride_b % 16 ||
                (!grouped && stride_a % 16)))
    return fail(TX_UNSUPPORTED,
                "%s: needs 16-byte aligned operand rows and problems (A, B, lda, ldb, K, strides)", what);
  if ((M - 1) * lda + K >= (int64_t(1) << 31) || (N - 1) * ldb + K >= (int64_t(1) << 31))
    return fail(TX_UNSUPPORTED, "%s: a problem's operands exceed 32-bit offsets", what);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t cus = cu_count();
  // Groups averaging under 192 rows: the transposed tile (a group's rows on
  // the tile's 128-wide side, so a 100-row group wastes 28 rows, not 156).
  const bool trans = grouped && !e.on() && M < 192 * groups;
  const int64_t tile_rows = trans ? 128 : 256;
  const int64_t rt = (M + tile_rows - 1) / tile_rows;
  const int64_t mtiles = grouped ? rt + groups : groups * rt;
  const bool big = !trans && (grouped ? rt : mtiles) * ((N + 255) / 256) >= cus;
  const int64_t bn = big || trans ? 256 : 128;  // C columns per tile
  const int64_t tiles_n = (N + bn - 1) / bn;
  if (mtiles * tiles_n > INT32_MAX) return fail(TX_UNSUPPORTED, "%s: too many tiles", what);

  tx_grouped_args q{};
  q.g = tx_gemm_args{A, B, C, sa, sb, lda, ldb, ldc, int32_t(M), int32_t(N), int32_t(K),
                     int32_t(mtiles), int32_t(tiles_n), int32_t(std::min<int64_t>(kGroupM, mtiles)), 1, 0,
                     nullptr};
  q.offsets = offsets;
  q.stride_a = stride_a;
  q.stride_sa = stride_sa;
  q.stride_c = stride_c;
  q.stride_b = stride_b;
  q.stride_sb = stride_sb;
  q.stride_bias = stride_bias;
  if (e.on()) {
    q.g.bias = e.bias;
    q.g.act = e.act;
    q.g.out_kind = e.out_kind;
    q.g.out_mul = e.out_mul;
    q.g.epi = 1;
  }
  q.groups = int32_t(groups);
  q.mtiles = int32_t(mtiles);
  q.tiles_per = int32_t(rt);
  q.tile_rows = int32_t(tile_rows);
  ScratchLease pre;  // held until the product is enqueued
  hipFunction_t fn;
  if (grouped) {
    if (prefix_ws) {  // the caller's workspace (the no-allocation entry point)
      q.tile_prefix = prefix_ws;
    } else {
      TX_TRY(pre.acquire(s, 1, size_t(groups + 1) * sizeof(int32_t)));
      q.tile_prefix = static_cast<int32_t *>(pre.ptr());
    }
    TX_TRY(get_kernel(CodeObject::GemmFp8, "tx_gemm_fp8_grouped_prefix", &fn));
    TX_TRY(launch(fn, 1, 1, 256, s, &q, sizeof q, "tx_gemm_fp8_grouped_prefix"));
  }
  char kname[80];
  // 256 x 256 tiles of a grouped product without an epilogue: the
  // persistent kernel (one workgroup per CU walking the real tiles, whose
  // count it reads from the prefix) when K is a whole number (>= 2) of
  // 128-byte steps and C rows are 16-byte aligned.
  if (grouped && big && !e.on() && K % 128 == 0 && K >= 256 && N % 8 == 0 && aligned(C, 16) && ldc % 8 == 0 &&
      ((M - 1) * ldc + N) * 2 < (int64_t(1) << 31)) {
    std::snprintf(kname, sizeof kname, "tx_gemm_fp8_%s_%s_grouped_persist", fa, fb);
    TX_TRY(get_kernel(CodeObject::GemmFp8, kname, &fn));
    return launch(fn, unsigned(std::min<int64_t>(mtiles * tiles_n, cus)), 1, 64 * kPersistWaves, s, &q, sizeof q,
                  kname);
  }
  if (trans) std::snprintf(kname, sizeof kname, "tx_gemm_fp8_%s_%s_grouped_t", fa, fb);
  else std::snprintf(kname, sizeof kname, "tx_gemm_fp8_%s_%s_grouped%s%s", fa, fb, e.on() ? "_epi" : "",
                     big ? "" : "_n128");
  TX_TRY(get_kernel(CodeObject::GemmFp8, kname, &fn));
  return launch(fn, unsigned(mtiles * tiles_n), 1, 64 * kFastWaves, s, &q, sizeof q, kname);
}

// The grouped product with an optional caller workspace for the group tile
// prefix (groups + 1 int32); NULL: the library's stream scratch.
tx_status dot_fp8_scaled_grouped_ws(const char *what, const void *A, tx_dtype a_type, int64_t lda,
                                    const float *sa, const void *B, tx_dtype b_type, int64_t ldb,
                                    int64_t stride_b, const float *sb, int64_t stride_sb, const float *bias,
                                    int64_t stride_bias, int activation, void *C, tx_dtype c_type,
                                    float c_scale, int64_t ldc, const int32_t *offsets, int64_t groups,
                                    int64_t M, int64_t N, int64_t K, tx_stream_t stream, int32_t *prefix_ws) {
  if (!offsets && groups > 0 && M > 0 && N > 0)
    return fail(TX_INVALID_ARGUMENT, "%s: NULL group offsets", what);
  Epilogue e;
  size_t es;
  TX_TRY(make_epilogue(what, bias, activation, c_type, c_scale, &e, &es));
  return dot_fp8_grouped_impl(what, A, a_type, lda, 0, sa, 0, B, b_type, ldb, stride_b, sb, stride_sb, C,
                              ldc, 0, offsets, groups, M, N, K, stream, e, es, stride_bias, prefix_ws);
}

static tx_status dot_fp8_scaled_grouped(const void *A, tx_dtype a_type, int64_t lda, const float *sa,
                                        const void *B, tx_dtype b_type, int64_t ldb, int64_t stride_b,
                                        const float *sb, int64_t stride_sb, const float *bias,
                                        int64_t stride_bias, int activation, void *C, tx_dtype c_type,
                                        float c_scale, int64_t ldc, const int32_t *offsets, int64_t groups,
                                        int64_t M, int64_t N, int64_t K, tx_stream_t stream) {
  return dot_fp8_scaled_grouped_ws("tx_dot_fp8_scaled_grouped", A, a_type, lda, sa, B, b_type, ldb,
                                       stride_b, sb, stride_sb, bias, stride_bias, activation, C, c_type,
                                       c_scale, ldc, offsets, groups, M, N, K, stream, nullptr);
}

static tx_status gemv_fp8_dequant(const void *x, int64_t ldx, const void *W, tx_dtype w_type,
                                  int64_t ldw, const float *scales, int64_t ld_scales,
                                  int64_t group, void *y, int64_t ldy, int64_t M, int64_t N,
                                  int64_t K, tx_stream_t stream) {
  const char *what = "tx_gemv_fp8_dequant";
  const char *fw = fp8_name(w_type);
  if (!fw) return fail(TX_INVALID_ARGUMENT, "%s: W must be fp8 (got %d)", what, int(w_type));
  if (M < 0 || N < 0 || K < 0 || group <= 0)
    return fail(TX_INVALID_ARGUMENT, "%s: bad size (M=%lld N=%lld K=%lld group=%lld)", what,
                (long long)M, (long long)N, (long long)K, (long long)group);
  if (M > 64) return fail(TX_UNSUPPORTED, "%s: M = %lld > 64 (use tx_dot_fp8_scaled)", what, (long long)M);
  if (N > INT32_MAX / 2 || K > INT32_MAX / 2)
    return fail(TX_UNSUPPORTED, "%s: size exceeds 32-bit indexing", what);
  if (M == 0 || N == 0) return TX_SUCCESS;
  if (K % 128 != 0 || group % 128 != 0)
    return fail(TX_UNSUPPORTED, "%s: K (%lld) and group (%lld) must be multiples of 128", what,
                (long long)K, (long long)group);
  if (!y || (K > 0 && (!x || !W || !scales)))
    return fail(TX_INVALID_ARGUMENT, "%s: NULL buffer", what);
  const int64_t ngroups = (K + group - 1) / group;
  if (ldx < K || ldw < K || ldy < N || ld_scales < ngroups)
    return fail(TX_INVALID_ARGUMENT, "%s: stride smaller than row length", what);
  if (!aligned(x, 16) || ldx % 8 != 0 || !aligned(W, 16) || ldw % 16 != 0 ||
      !aligned(scales, 4) || !aligned(y, 2))
    return fail(TX_UNSUPPORTED,
                "%s: needs 16-byte aligned x and W rows (ldx %% 8 == 0, ldw %% 16 == 0)", what);
  tx_gemv_args args{static_cast<const uint16_t *>(x), static_cast<const uint8_t *>(W), scales,
                    static_cast<uint16_t *>(y), ldx, ldw, ld_scales, ldy, int32_t(M), int32_t(N),
                    int32_t(K), int32_t(group), 0, 0};
  char kname[48];
  hipFunction_t fn;
  if (M == 1 && K * 2 <= 32768) {  // x fits the kernel's LDS stage
    // streaming VALU kernel: two W rows per wavefront, 4 wavefronts, x in
    // K * 2 bytes of dynamic LDS
    std::snprintf(kname, sizeof kname, "tx_gemv_fp8_%s_lin_m1", fw);
    TX_TRY(get_kernel(CodeObject::Gemv, kname, &fn));
    return launch(fn, unsigned((N + 7) / 8), 1, 256, static_cast<hipStream_t>(stream), &args, sizeof args,
                  kname, unsigned(K * 2));
  }
  // Up to 16 or 32 W rows per workgroup, K split over its wavefronts.  Many
  // column blocks: 4 wavefronts, each with two 16-row W blocks sharing its x
  // reads, and the rows spread evenly over a whole number of workgroups per
  // CU (N = 14336: 512 workgroups of 28 rows, where 448 of 32 left 64 CUs with
  // half the bytes of the others and the rest finishing 3-5 us later).  Few:
  // one W block per workgroup and 16 wavefronts (8 with 2 or 4 blocks of M)
  // to keep enough loads in flight.
  const int mblocks = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  const int64_t cus = cu_count();
  const bool wide = (N + 15) / 16 >= 2 * cus;
  const int waves = wide ? 4 : (mblocks == 1 ? 16 : 8);
  const int nb = wide ? 2 : 1;
  int64_t rows = 16 * nb;
  if (wide) {
    const int64_t nwg = ((N + rows - 1) / rows + cus - 1) / cus * cus;
    rows = (N + nwg - 1) / nwg;
  }
  args.rows_per_wg = int32_t(rows);
  const int64_t grid = (N + rows - 1) / rows;
  std::snprintf(kname, sizeof kname, "tx_gemv_fp8_%s_w%d_m%d_b%d", fw, waves, mblocks, nb);
  TX_TRY(get_kernel(CodeObject::Gemv, kname, &fn));
  return launch(fn, unsigned(grid), 1, unsigned(64 * waves), static_cast<hipStream_t>(stream), &args,
                sizeof args, kname);
}

// Table forms.
// tt.dot: {C (result), A, B, M, N, K, lda, ldb, ldc[, ab_type, c_type,
// b_layout[, acc, ld_acc, scale_a, scale_b, b_type]]} -- without the last
// eight, bf16 operands and output and B stored N x K; with the last five,
// tt.dot's accumulator operand (acc fp32 M x N or NULL; c_type fp32, bf16 or
// fp16; fp8 operands with scale_a / scale_b, 16-bit ones with NULL scales;
// tx_dot_acc).
static tx_status dot_op(tx_value *v, size_t count, tx_stream_t stream) {
  Operands o{v, count, "tt.dot"};
  if (count != 17) TX_TRY(o.need_either(9, 12));
  else TX_TRY(o.need(17));
  void *C, *A, *B;
  int64_t M, N, K, lda, ldb, ldc;
  TX_TRY(o.ptr(0, &C));
  TX_TRY(o.ptr(1, &A));
  TX_TRY(o.ptr(2, &B));
  TX_TRY(o.integer(3, &M));
  TX_TRY(o.integer(4, &N));
  TX_TRY(o.integer(5, &K));
  TX_TRY(o.integer(6, &lda));
  TX_TRY(o.integer(7, &ldb));
  TX_TRY(o.integer(8, &ldc));
  int64_t ab = TX_BF16, ct = TX_BF16, layout = TX_B_NK;
  if (count >= 12) {
    TX_TRY(o.integer(9, &ab));
    TX_TRY(o.integer(10, &ct));
    TX_TRY(o.integer(11, &layout));
  }
  if (count == 17) {
    void *acc, *sa, *sb;
    int64_t ld_acc, bt;
    TX_TRY(o.ptr(12, &acc));
    TX_TRY(o.integer(13, &ld_acc));
    TX_TRY(o.ptr(14, &sa));
    TX_TRY(o.ptr(15, &sb));
    TX_TRY(o.integer(16, &bt));
    return dot_acc(A, tx_dtype(ab), lda, static_cast<const float *>(sa), B, tx_dtype(bt), tx_b_layout(layout),
                   ldb, static_cast<const float *>(sb), static_cast<const float *>(acc), ld_acc, C, tx_dtype(ct),
                   ldc, M, N, K, stream);
  }
  return dot16("tt.dot", A, tx_dtype(ab), lda, B, tx_b_layout(layout), ldb, C, tx_dtype(ct), ldc, M,
               N, K, stream);
}

// tt.dot_scaled.rowcol: {C (result), A, B, scale_a, scale_b, M, N, K, lda, ldb,
// ldc, a_type, b_type}
static tx_status dot_fp8_op(tx_value *v, size_t count, tx_stream_t stream) {
  Operands o{v, count, "tt.dot_scaled.rowcol"};
  TX_TRY(o.need(13));
  void *C, *A, *B, *sa, *sb;
  int64_t M, N, K, lda, ldb, ldc, at, bt;
  TX_TRY(o.ptr(0, &C));
  TX_TRY(o.ptr(1, &A));
  TX_TRY(o.ptr(2, &B));
  TX_TRY(o.ptr(3, &sa));
  TX_TRY(o.ptr(4, &sb));
  TX_TRY(o.integer(5, &M));
  TX_TRY(o.integer(6, &N));
  TX_TRY(o.integer(7, &K));
  TX_TRY(o.integer(8, &lda));
  TX_TRY(o.integer(9, &ldb));
  TX_TRY(o.integer(10, &ldc));
  TX_TRY(o.integer(11, &at));
  TX_TRY(o.integer(12, &bt));
  return dot_fp8_scaled(A, tx_dtype(at), lda, static_cast<const float *>(sa), B, tx_dtype(bt), ldb,
                        static_cast<const float *>(sb), C, ldc, M, N, K, stream);
}

// tx.dot_fp8_scaled_grouped: {C (result), A, B, scale_a, scale_b, offsets,
// bias (or NULL), groups, M, N, K, lda, ldb, ldc, stride_b, stride_scale_b,
// stride_bias, a_type, b_type, c_type, activation, c_scale (fp32 bits)}
static tx_status dot_fp8_grouped_op(tx_value *v, size_t count, tx_stream_t stream) {
  Operands o{v, count, "tx.dot_fp8_scaled_grouped"};
  TX_TRY(o.need(22));
  void *C, *A, *B, *sa, *sb, *off, *bias;
  int64_t G, M, N, K, lda, ldb, ldc, stb, stsb, stbias, at, bt, ct, act, cs;
  TX_TRY(o.ptr(0, &C));
  TX_TRY(o.ptr(1, &A));
  TX_TRY(o.ptr(2, &B));
  TX_TRY(o.ptr(3, &sa));
  TX_TRY(o.ptr(4, &sb));
  TX_TRY(o.ptr(5, &off));
  TX_TRY(o.ptr(6, &bias));
  TX_TRY(o.integer(7, &G));
  TX_TRY(o.integer(8, &M));
  TX_TRY(o.integer(9, &N));
  TX_TRY(o.integer(10, &K));
  TX_TRY(o.integer(11, &lda));
  TX_TRY(o.integer(12, &ldb));
  TX_TRY(o.integer(13, &ldc));
  TX_TRY(o.integer(14, &stb));
  TX_TRY(o.integer(15, &stsb));
  TX_TRY(o.integer(16, &stbias));
  TX_TRY(o.integer(17, &at));
  TX_TRY(o.integer(18, &bt));
  TX_TRY(o.integer(19, &ct));
  TX_TRY(o.integer(20, &act));
  TX_TRY(o.integer(21, &cs));
  float c_scale;
  const uint32_t bits = uint32_t(cs);
  std::memcpy(&c_scale, &bits, sizeof c_scale);
  return dot_fp8_scaled_grouped(A, tx_dtype(at), lda, static_cast<const float *>(sa), B, tx_dtype(bt), ldb,
                                stb, static_cast<const float *>(sb), stsb, static_cast<const float *>(bias),
                                stbias, int(act), C, tx_dtype(ct), c_scale, ldc,
                                static_cast<const int32_t *>(off), G, M, N, K, stream);
}

// tx.dot_fp8_scaled_batched: {C (result), A, B, scale_a, scale_b, batch, M,
// N, K, lda, ldb, ldc, stride_a, stride_scale_a, stride_b, stride_scale_b,
// stride_c, a_type, b_type}
static tx_status dot_fp8_batched_op(tx_value *v, size_t count, tx_stream_t stream) {
  Operands o{v, count, "tx.dot_fp8_scaled_batched"};
  TX_TRY(o.need(19));
  void *C, *A, *B, *sa, *sb;
  int64_t G, M, N, K, lda, ldb, ldc, sta, stsa, stb, stsb, stc, at, bt;
  TX_TRY(o.ptr(0, &C));
  TX_TRY(o.ptr(1, &A));
  TX_TRY(o.ptr(2, &B));
  TX_TRY(o.ptr(3, &sa));
  TX_TRY(o.ptr(4, &sb));
  TX_TRY(o.integer(5, &G));
  TX_TRY(o.integer(6, &M));
  TX_TRY(o.integer(7, &N));
  TX_TRY(o.integer(8, &K));
  TX_TRY(o.integer(9, &lda));
  TX_TRY(o.integer(10, &ldb));
  TX_TRY(o.integer(11, &ldc));
  TX_TRY(o.integer(12, &sta));
  TX_TRY(o.integer(13, &stsa));
  TX_TRY(o.integer(14, &stb));
  TX_TRY(o.integer(15, &stsb));
  TX_TRY(o.integer(16, &stc));
  TX_TRY(o.integer(17, &at));
  TX_TRY(o.integer(18, &bt));
  return dot_fp8_grouped_impl("tx_dot_fp8_scaled_batched", A, tx_dtype(at), lda, sta,
                              static_cast<const float *>(sa), stsa, B, tx_dtype(bt), ldb, stb,
                              static_cast<const float *>(sb), stsb, C, ldc, stc, nullptr, G, M, N, K, stream);
}

// tx.gemv_fp8_dequant: {y (result), x, W, scales, M, N, K, group, ldx, ldw,
// ld_scales, ldy, w_type}
static tx_status gemv_op(tx_value *v, size_t count, tx_stream_t stream) {
  Operands o{v, count, "tx.gemv_fp8_dequant"};
  TX_TRY(o.need(13));
  void *y, *x, *W, *s;
  int64_t M, N, K, group, ldx, ldw, lds, ldy, wt;
  TX_TRY(o.ptr(0, &y));
  TX_TRY(o.ptr(1, &x));
  TX_TRY(o.ptr(2, &W));
  TX_TRY(o.ptr(3, &s));
  TX_TRY(o.integer(4, &M));
  TX_TRY(o.integer(5, &N));
  TX_TRY(o.integer(6, &K));
  TX_TRY(o.integer(7, &group));
  TX_TRY(o.integer(8, &ldx));
  TX_TRY(o.integer(9, &ldw));
  TX_TRY(o.integer(10, &lds));
  TX_TRY(o.integer(11, &ldy));
  TX_TRY(o.integer(12, &wt));
  return gemv_fp8_dequant(x, ldx, W, tx_dtype(wt), ldw, static_cast<const float *>(s), lds, group,
                          y, ldy, M, N, K, stream);
}

// tt.dot_scaled: {C (result), A, B, scale_a, scale_b, M, N, K, lda, ldb, ldc,
// ld_scale_a, ld_scale_b, a_type, b_type, c_type}
static tx_status dot_mx_op(tx_value *v, size_t count, tx_stream_t stream) {
  Operands o{v, count, "tt.dot_scaled"};
  TX_TRY(o.need(16));
  void *C, *A, *B, *sa, *sb;
  int64_t M, N, K, lda, ldb, ldc, ldsa, ldsb, at, bt, ct;
  TX_TRY(o.ptr(0, &C));
  TX_TRY(o.ptr(1, &A));
  TX_TRY(o.ptr(2, &B));
  TX_TRY(o.ptr(3, &sa));
  TX_TRY(o.ptr(4, &sb));
  TX_TRY(o.integer(5, &M));
  TX_TRY(o.integer(6, &N));
  TX_TRY(o.integer(7, &K));
  TX_TRY(o.integer(8, &lda));
  TX_TRY(o.integer(9, &ldb));
  TX_TRY(o.integer(10, &ldc));
  TX_TRY(o.integer(11, &ldsa));
  TX_TRY(o.integer(12, &ldsb));
  TX_TRY(o.integer(13, &at));
  TX_TRY(o.integer(14, &bt));
  TX_TRY(o.integer(15, &ct));
  return dot_scaled_mx(A, tx_dtype(at), lda, static_cast<const uint8_t *>(sa), ldsa, B, tx_dtype(bt),
                       ldb, static_cast<const uint8_t *>(sb), ldsb, C, tx_dtype(ct), ldc, M, N, K,
                       stream);
}

// tx.dot_fp8_scaled_ex: {C (result), A, B, scale_a, scale_b, bias (may be NULL), M, N, K,
// lda, ldb, ldc, a_type, b_type, c_type, activation, c_scale_bits (fp32 bits of c_scale)}
static tx_status dot_fp8_ex_op(tx_value *v, size_t count, tx_stream_t stream) {
  Operands o{v, count, "tx.dot_fp8_scaled_ex"};
  TX_TRY(o.need(17));
  void *C, *A, *B, *sa, *sb, *bias;
  int64_t M, N, K, lda, ldb, ldc, at, bt, ct, act, csb;
  TX_TRY(o.ptr(0, &C));
  TX_TRY(o.ptr(1, &A));
  TX_TRY(o.ptr(2, &B));
  TX_TRY(o.ptr(3, &sa));
  TX_TRY(o.ptr(4, &sb));
  TX_TRY(o.ptr(5, &bias));
  TX_TRY(o.integer(6, &M));
  TX_TRY(o.integer(7, &N));
  TX_TRY(o.integer(8, &K));
  TX_TRY(o.integer(9, &lda));
  TX_TRY(o.integer(10, &ldb));
  TX_TRY(o.integer(11, &ldc));
  TX_TRY(o.integer(12, &at));
  TX_TRY(o.integer(13, &bt));
  TX_TRY(o.integer(14, &ct));
  TX_TRY(o.integer(15, &act));
  TX_TRY(o.integer(16, &csb));
  const uint32_t bits = uint32_t(csb);
  float c_scale;
  std::memcpy(&c_scale, &bits, sizeof c_scale);
  return dot_fp8_scaled_ex(A, tx_dtype(at), lda, static_cast<const float *>(sa), B, tx_dtype(bt), ldb,
                           static_cast<const float *>(sb), static_cast<const float *>(bias), int(act),
                           C, tx_dtype(ct), c_scale, ldc, M, N, K, stream);
}

static const bool reg_dot = register_op(
    "tt.dot", dot_op,
    "C:bf16|f16|f32*(result), A:bf16|f16|fp8*, B:bf16|f16|fp8* (N x K, or K x N with b_layout 1), M, "
    "N, K, lda, ldb, ldc[, ab_type:i32, c_type:i32, b_layout:i32[, acc:f32*|NULL, ld_acc, "
    "scale_a:f32*|NULL, scale_b:f32*|NULL, b_type:i32]]");
static const bool reg_dot_fp8 = register_op(
    "tt.dot_scaled.rowcol", dot_fp8_op,
    "C:bf16*(result), A:fp8*, B:fp8* (N x K), scale_a:f32*, scale_b:f32*, M, N, K, lda, ldb, "
    "ldc, a_type:i32, b_type:i32");
static const bool reg_dot_fp8_ex = register_op(
    "tx.dot_fp8_scaled_ex", dot_fp8_ex_op,
    "C:bf16|f16|f32|fp8*(result), A:fp8*, B:fp8* (N x K), scale_a:f32*, scale_b:f32*, "
    "bias:f32*|NULL, M, N, K, lda, ldb, ldc, a_type:i32, b_type:i32, c_type:i32, activation:i32, "
    "c_scale:f32 bits");
static const bool reg_dot_mx = register_op(
    "tt.dot_scaled", dot_mx_op,
    "C:bf16|f16|f32*(result), A:fp8|fp4x2*, B:fp8|fp4x2* (N x K), scale_a:e8m0* (M x ceil(K/32)), "
    "scale_b:e8m0* (N x ceil(K/32)), M, N, K, lda, ldb, ldc, ld_scale_a, ld_scale_b, a_type:i32, "
    "b_type:i32, c_type:i32");
static const bool reg_dot_fp8_grouped = register_op(
    "tx.dot_fp8_scaled_grouped", dot_fp8_grouped_op,
    "C:bf16|f16|f32|fp8*(result, M x N), A:fp8* (M x K), B:fp8* (groups x N x K), scale_a:f32* (M), "
    "scale_b:f32* (groups x N), offsets:i32* (groups + 1 rows of A), bias:f32*|NULL (groups x N), "
    "groups, M, N, K, lda, ldb, ldc, stride_b, stride_scale_b, stride_bias, a_type:i32, b_type:i32, "
    "c_type:i32, activation:i32, c_scale:f32 bits");
static const bool reg_dot_fp8_batched = register_op(
    "tx.dot_fp8_scaled_batched", dot_fp8_batched_op,
    "C:bf16*(result, batch x M x N), A:fp8*, B:fp8* (N x K each), scale_a:f32*, scale_b:f32*, batch, "
    "M, N, K, lda, ldb, ldc, stride_a, stride_scale_a, stride_b, stride_scale_b, stride_c, a_type:i32, "
    "b_type:i32");
static const bool reg_gemv = register_op(
    "tx.gemv_fp8_dequant", gemv_op,
    "y:bf16*(result), x:bf16*, W:fp8* (N x K), scales:f32* (N x K/group), M, N, K, group, ldx, "
    "ldw, ld_scales, ldy, w_type:i32");

}  // namespace tx

extern "C" {

TX_API tx_status tx_dot(const void *A, tx_dtype ab_type, int64_t lda, const void *B,
                        tx_b_layout b_layout, int64_t ldb, void *C, tx_dtype c_type, int64_t ldc,
                        int64_t M, int64_t N, int64_t K, tx_stream_t stream) {
  tx::clear_error();
  return tx::dot16("tx_dot", A, ab_type, lda, B, b_layout, ldb, C, c_type, ldc, M, N, K, stream);
}

TX_API tx_status tx_dot_acc(const void *A, tx_dtype a_type, int64_t lda, const float *scale_a, const void *B,
                            tx_dtype b_type, tx_b_layout b_layout, int64_t ldb, const float *scale_b,
                            const float *C, int64_t ldc, void *D, tx_dtype d_type, int64_t ldd, int64_t M,
                            int64_t N, int64_t K, tx_stream_t stream) {
  tx::clear_error();
  return tx::dot_acc(A, a_type, lda, scale_a, B, b_type, b_layout, ldb, scale_b, C, ldc, D, d_type, ldd, M, N, K,
                     stream);
}

TX_API tx_status tx_dot_bf16(const void *A, int64_t lda, const void *B, int64_t ldb, void *C,
                             int64_t ldc, int64_t M, int64_t N, int64_t K, tx_stream_t stream) {
  tx::clear_error();
  return tx::dot_bf16(A, lda, B, ldb, C, ldc, M, N, K, stream);
}

TX_API tx_status tx_dot_fp8_scaled(const void *A, tx_dtype a_type, int64_t lda,
                                   const float *scale_a, const void *B, tx_dtype b_type,
                                   int64_t ldb, const float *scale_b, void *C, int64_t ldc,
                                   int64_t M, int64_t N, int64_t K, tx_stream_t stream) {
  tx::clear_error();
  return tx::dot_fp8_scaled(A, a_type, lda, scale_a, B, b_type, ldb, scale_b, C, ldc, M, N, K,
                            stream);
}

TX_API tx_status tx_dot_fp8_scaled_ex(const void *A, tx_dtype a_type, int64_t lda,
                                      const float *scale_a, const void *B, tx_dtype b_type,
                                      int64_t ldb, const float *scale_b, const float *bias,
                                      int activation, void *C, tx_dtype c_type, float c_scale,
                                      int64_t ldc, int64_t M, int64_t N, int64_t K,
                                      tx_stream_t stream) {
  tx::clear_error();
  return tx::dot_fp8_scaled_ex(A, a_type, lda, scale_a, B, b_type, ldb, scale_b, bias, activation,
                               C, c_type, c_scale, ldc, M, N, K, stream);
}

TX_API tx_status tx_dot_fp8_scaled_grouped(const void *A, tx_dtype a_type, int64_t lda,
                                           const float *scale_a, const void *B, tx_dtype b_type,
                                           int64_t ldb, int64_t stride_b, const float *scale_b,
                                           int64_t stride_scale_b, const float *bias,
                                           int64_t stride_bias, int activation, void *C,
                                           tx_dtype c_type, float c_scale, int64_t ldc,
                                           const int32_t *group_offsets, int64_t groups, int64_t M,
                                           int64_t N, int64_t K, tx_stream_t stream) {
  tx::clear_error();
  return tx::dot_fp8_scaled_grouped(A, a_type, lda, scale_a, B, b_type, ldb, stride_b, scale_b,
                                    stride_scale_b, bias, stride_bias, activation, C, c_type, c_scale, ldc,
                                    group_offsets, groups, M, N, K, stream);
}

TX_API tx_status tx_dot_fp8_scaled_batched(const void *A, tx_dtype a_type, int64_t lda, int64_t stride_a,
                                           const float *scale_a, int64_t stride_scale_a, const void *B,
                                           tx_dtype b_type, int64_t ldb, int64_t stride_b,
                                           const float *scale_b, int64_t stride_scale_b, void *C,
                                           int64_t ldc, int64_t stride_c, int64_t batch, int64_t M,
                                           int64_t N, int64_t K, tx_stream_t stream) {
  tx::clear_error();
  return tx::dot_fp8_grouped_impl("tx_dot_fp8_scaled_batched", A, a_type, lda, stride_a, scale_a,
                                  stride_scale_a, B, b_type, ldb, stride_b, scale_b, stride_scale_b, C, ldc,
                                  stride_c, nullptr, batch, M, N, K, stream);
}

TX_API tx_status tx_dot_scaled_mx(const void *A, tx_dtype a_type, int64_t lda,
                                  const uint8_t *scale_a, int64_t ld_scale_a, const void *B,
                                  tx_dtype b_type, int64_t ldb, const uint8_t *scale_b,
                                  int64_t ld_scale_b, void *C, tx_dtype c_type, int64_t ldc,
                                  int64_t M, int64_t N, int64_t K, tx_stream_t stream) {
  tx::clear_error();
  return tx::dot_scaled_mx(A, a_type, lda, scale_a, ld_scale_a, B, b_type, ldb, scale_b, ld_scale_b,
                           C, c_type, ldc, M, N, K, stream);
}

TX_API tx_status tx_gemv_fp8_dequant(const void *x, int64_t ldx, const void *W, tx_dtype w_type,
                                     int64_t ldw, const float *scales, int64_t ld_scales,
                                     int64_t group, void *y, int64_t ldy, int64_t M, int64_t N,
                                     int64_t K, tx_stream_t stream) {
  tx::clear_error();
  return tx::gemv_fp8_dequant(x, ldx, W, w_type, ldw, scales, ld_scales, group, y, ldy, M, N, K,
                              stream);
}

}  // extern "C"
