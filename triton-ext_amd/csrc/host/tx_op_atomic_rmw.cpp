// tt.atomic_rmw and tt.atomic_cas scatter entry points and their table
// registrations.
//
// Reference: tl.atomic_add / tl.atomic_max ... lower to tt.atomic_rmw, which
// the plugin passes through unchanged (uTLXConversionPatterns.cpp:611); the
// reference's only uses are counters that check the returned old values
// (test_tlx.py:7627-7629, 7672-7723).  The scatter form bins[idx[i]] op= v[i]
// is the data-parallel op this entry point serves.
#include <algorithm>
#include <climits>
#include <cstdio>

#include "tx_kernel_args.h"
#include "tx_ops.h"

namespace tx {
namespace {

constexpr int kAggBlock = 1024;     // threads of the aggregating kernels
constexpr int64_t kAggStep = 4 * kAggBlock;
constexpr int64_t kWinStep = 3 * kAggStep;  // windowed kernel: its pipelined loop takes 3 steps at a time
constexpr int64_t kDirectSlots = 36864;  // bins per LDS window
constexpr int64_t kMaxWindows = 4;       // beyond this the hash-table kernel is used
// Spill buffer of the windowed kernel's one-pass path: records per
// wavefront region (16 wavefronts per workgroup), and the chunk of records
// per workgroup of the second launch that folds them into the bins.
constexpr int64_t kSpillWave = 512;
constexpr int64_t kSpillChunk = 3 * kWinStep;

const char *op_name(tx_rmw_op op) {
  switch (op) {
    case TX_RMW_ADD: return "add";
    case TX_RMW_FADD: return "fadd";
    case TX_RMW_MAX: return "max";
    case TX_RMW_MIN: return "min";
    case TX_RMW_UMAX: return "umax";
    case TX_RMW_UMIN: return "umin";
    case TX_RMW_AND: return "and";
    case TX_RMW_OR: return "or";
    case TX_RMW_XOR: return "xor";
    case TX_RMW_XCHG: return "xchg";
  }
  return nullptr;
}

// One thread per update (grid-stride beyond 64 workgroups per CU).
unsigned direct_grid(int64_t n) {
  return unsigned(std::min<int64_t>((n + 255) / 256, int64_t(cu_count()) * 64));
}

}  // namespace

// The aggregating forms (no old values, 32-bit bins): LDS windows or the
// hash table; args.val == NULL adds 1 per update (tt.histogram).
static tx_status aggregate(tx_scatter_args args, const char *name, hipStream_t s) {
  const int64_t n = args.n, nbins = args.nbins;
  const int cus = cu_count();
  char kname[64];
  const int64_t windows = (nbins + kDirectSlots - 1) / kDirectSlots;
  hipFunction_t fn;
  if (windows <= kMaxWindows) {
    std::snprintf(kname, sizeof kname, "tx_scatter_%s_windowed", name);
    TX_TRY(get_kernel(CodeObject::Scatter, kname, &fn));
    // One workgroup per CU at a time (the table fills a CU's LDS) and one
    // chunk of updates per workgroup; the workgroup itself makes one pass
    // per window, or a single pass when its chunk's keys are skewed.
    int64_t chunks = std::max<int64_t>(8, cus);
    int64_t per = (n + chunks - 1) / chunks;
    per = (per + kWinStep - 1) / kWinStep * kWinStep;
    if (per > INT32_MAX) per = INT32_MAX / kWinStep * kWinStep;
    chunks = (n + per - 1) / per;
    args.per_block = int32_t(per);
    args.splits = int32_t(windows);
    args.window = int32_t(kDirectSlots);
    if (windows == 1) return launch(fn, unsigned(chunks), 1, kAggBlock, s, &args, sizeof args, kname);
    // Several windows: a workgroup whose keys are skewed makes one pass with
    // its best window and writes the in-range updates outside it to its
    // wavefronts' regions of a spill buffer in stream scratch (slot 0); a
    // second launch of the same kernel folds those records (unused ones are
    // marked out of range) into the bins, with direct global atomics for
    // whatever spills again.  Without the buffer the first launch sends its
    // spills to global atomics itself.
    const int64_t records = chunks * (kAggBlock / 64) * kSpillWave;
    ScratchLease sp;  // held until both launches are enqueued
    if (sp.acquire(s, 0, size_t(records) * 8) != TX_SUCCESS) {
      clear_error();
      return launch(fn, unsigned(chunks), 1, kAggBlock, s, &args, sizeof args, kname);
    }
    args.spill_keys = static_cast<uint32_t *>(sp.ptr());
    args.spill_vals = args.spill_keys + records;
    args.spill_wave = int32_t(kSpillWave);
    TX_TRY(launch(fn, unsigned(chunks), 1, kAggBlock, s, &args, sizeof args, kname));
    tx_scatter_args fold{args.bins, reinterpret_cast<const int32_t *>(args.spill_keys), args.spill_vals, nullptr,
                         nullptr, records, int32_t(nbins), int32_t(kSpillChunk), int32_t(windows),
                         int32_t(kDirectSlots)};
    const int64_t fold_chunks = (records + kSpillChunk - 1) / kSpillChunk;
    return launch(fn, unsigned(fold_chunks), 1, kAggBlock, s, &fold, sizeof fold, kname);
  }
  std::snprintf(kname, sizeof kname, "tx_scatter_%s_hashed", name);
  TX_TRY(get_kernel(CodeObject::Scatter, kname, &fn));
  int64_t per = (n + cus - 1) / cus;
  per = (per + kAggStep - 1) / kAggStep * kAggStep;
  if (per > INT32_MAX) per = INT32_MAX / kAggStep * kAggStep;
  args.per_block = int32_t(per);
  const int64_t grid = (n + per - 1) / per;
  return launch(fn, unsigned(grid), 1, kAggBlock, s, &args, sizeof args, kname);
}

// 64-bit and 16-bit float bins (tx_scatter_<type>_<op>_{table,direct,old},
// tx_scatter_i64_xchg in scatter.hip): an LDS table per workgroup when the
// bins fit one (and the updates are at least twice the bins), one global
// atomic per update otherwise and for the returning-old and xchg forms.
constexpr int64_t kWideSlots64 = 18432, kWideSlots16 = 36864;
constexpr unsigned kWideBlock = 1024;

static tx_status atomic_rmw_wide(void *bins, tx_dtype bins_type, int64_t nbins, const int32_t *idx,
                                 const void *val, const uint8_t *mask, int64_t n, tx_rmw_op op, void *old,
                                 hipStream_t s) {
  const char *what = "tx_atomic_rmw_scatter";
  const bool i64 = bins_type == TX_I64 || bins_type == TX_U64;
  const bool half = bins_type == TX_F16 || bins_type == TX_BF16;
  if (half && op != TX_RMW_FADD)
    return fail(TX_INVALID_ARGUMENT, "%s: fp16 / bf16 bins take fadd only", what);
  if (bins_type == TX_F64 && op != TX_RMW_FADD && op != TX_RMW_XCHG)
    return fail(TX_INVALID_ARGUMENT, "%s: fp64 bins take fadd or xchg", what);
  if (i64 && op == TX_RMW_FADD) return fail(TX_INVALID_ARGUMENT, "%s: fadd needs floating-point bins", what);
  if (n == 0) return TX_SUCCESS;
  if (!idx || !val || (!bins && nbins > 0)) return fail(TX_INVALID_ARGUMENT, "%s: NULL buffer", what);
  const size_t es = half ? 2 : 8;
  if (!aligned(idx, 4) || !aligned(val, es) || (bins && !aligned(bins, es)) || (old && !aligned(old, es)))
    return fail(TX_INVALID_ARGUMENT, "%s: idx must be 4-byte and bins / val / old %zu-byte aligned", what, es);
  tx_scatter_args args{bins, idx, val, mask, old, n, int32_t(nbins), 0, 0, 0};
  const char *tn = i64 ? "i64" : bins_type == TX_F64 ? "f64" : bins_type == TX_F16 ? "f16" : "bf16";
  char kname[64];
  hipFunction_t fn;
  if (op == TX_RMW_XCHG) {
    TX_TRY(get_kernel(CodeObject::Scatter, "tx_scatter_i64_xchg", &fn));
    return launch(fn, direct_grid(n), 1, 256, s, &args, sizeof args, "tx_scatter_i64_xchg");
  }
  const int64_t slots = half ? kWideSlots16 : kWideSlots64;
  if (!old && nbins == 0) return TX_SUCCESS;  // every update is out of range
  if (!old && nbins <= slots && n >= 2 * nbins) {
    std::snprintf(kname, sizeof kname, "tx_scatter_%s_%s_table", tn, op_name(op));
    TX_TRY(get_kernel(CodeObject::Scatter, kname, &fn));
    const int64_t chunks = std::max<int64_t>(1, std::min<int64_t>(cu_count(), n / (4 * kWideBlock)));
    int64_t per = (n + chunks - 1) / chunks;
    if (per > INT32_MAX) per = INT32_MAX;
    args.per_block = int32_t(per);
    return launch(fn, unsigned((n + per - 1) / per), 1, kWideBlock, s, &args, sizeof args, kname);
  }
  std::snprintf(kname, sizeof kname, "tx_scatter_%s_%s_%s", tn, op_name(op), old ? "old" : "direct");
  TX_TRY(get_kernel(CodeObject::Scatter, kname, &fn));
  return launch(fn, direct_grid(n), 1, 256, s, &args, sizeof args, kname);
}

static tx_status atomic_rmw_scatter(void *bins, tx_dtype bins_type, int64_t nbins,
                                    const int32_t *idx, const void *val,
                                    const uint8_t *mask, int64_t n, tx_rmw_op op,
                                    void *old, tx_stream_t stream) {
  const char *name = op_name(op);
  if (!name) return fail(TX_INVALID_ARGUMENT, "tx_atomic_rmw_scatter: unknown op %d", int(op));
  if (n < 0 || nbins < 0)
    return fail(TX_INVALID_ARGUMENT, "tx_atomic_rmw_scatter: n = %lld, nbins = %lld",
                (long long)n, (long long)nbins);
  if (nbins > INT32_MAX)
    return fail(TX_UNSUPPORTED, "tx_atomic_rmw_scatter: nbins %lld exceeds int32 indexing",
                (long long)nbins);
  if (bins_type == TX_I64 || bins_type == TX_U64 || bins_type == TX_F64 || bins_type == TX_F16 ||
      bins_type == TX_BF16)
    return atomic_rmw_wide(bins, bins_type, nbins, idx, val, mask, n, op, old, static_cast<hipStream_t>(stream));
  if (op == TX_RMW_FADD) {
    if (bins_type != TX_F32)
      return fail(TX_INVALID_ARGUMENT, "tx_atomic_rmw_scatter: fadd needs TX_F32, TX_F64, TX_F16 or TX_BF16 bins");
  } else if (op == TX_RMW_XCHG) {
    if (bins_type != TX_I32 && bins_type != TX_U32 && bins_type != TX_F32)
      return fail(TX_INVALID_ARGUMENT, "tx_atomic_rmw_scatter: xchg needs 32- or 64-bit bins");
  } else if (bins_type != TX_I32 && bins_type != TX_U32) {
    return fail(TX_INVALID_ARGUMENT,
                "tx_atomic_rmw_scatter: integer ops need TX_I32, TX_U32, TX_I64 or TX_U64 bins");
  }
  if (n == 0) return TX_SUCCESS;
  if (!idx || !val || (!bins && nbins > 0))
    return fail(TX_INVALID_ARGUMENT, "tx_atomic_rmw_scatter: NULL buffer");
  if (!aligned(idx, 4) || !aligned(val, 4) || (bins && !aligned(bins, 4)) ||
      (old && !aligned(old, 4)))
    return fail(TX_INVALID_ARGUMENT, "tx_atomic_rmw_scatter: buffers must be 4-byte aligned");

  hipStream_t s = static_cast<hipStream_t>(stream);
  const int cus = cu_count();
  tx_scatter_args args{bins, idx, val, mask, old, n, int32_t(nbins), 0, 0, 0};
  char kname[64];
  if (op == TX_RMW_XCHG) {
    hipFunction_t fn;
    TX_TRY(get_kernel(CodeObject::Scatter, "tx_scatter_xchg", &fn));
    return launch(fn, direct_grid(n), 1, 256, s, &args, sizeof args, "tx_scatter_xchg");
  }
  if (old) {
    std::snprintf(kname, sizeof kname, "tx_scatter_%s_old", name);
    hipFunction_t fn;
    TX_TRY(get_kernel(CodeObject::Scatter, kname, &fn));
    const int64_t grid = std::min<int64_t>((n + 255) / 256, int64_t(cus) * 64);
    return launch(fn, unsigned(grid), 1, 256, s, &args, sizeof args, kname);
  }
  if (nbins == 0) return TX_SUCCESS;  // every update is out of range
  return aggregate(args, name, s);
}

// Table form: operands = {bins (result slot), idx, val, mask, old, nbins, n,
// bins_type, op}.  mask and old may be NULL pointers.
static tx_status atomic_rmw_op(tx_value *v, size_t count, tx_stream_t stream) {
  Operands o{v, count, "tt.atomic_rmw"};
  TX_TRY(o.need(9));
  void *bins, *idx, *val, *mask, *old;
  int64_t nbins, n, bt, op;
  TX_TRY(o.ptr(0, &bins));
  TX_TRY(o.ptr(1, &idx));
  TX_TRY(o.ptr(2, &val));
  TX_TRY(o.ptr(3, &mask));
  TX_TRY(o.ptr(4, &old));
  TX_TRY(o.integer(5, &nbins));
  TX_TRY(o.integer(6, &n));
  TX_TRY(o.integer(7, &bt));
  TX_TRY(o.integer(8, &op));
  return atomic_rmw_scatter(bins, tx_dtype(bt), nbins, static_cast<const int32_t *>(idx), val,
                            static_cast<const uint8_t *>(mask), n, tx_rmw_op(op), old, stream);
}

static tx_status atomic_cas_scatter(void *bins, tx_dtype bins_type, int64_t nbins,
                                    const int32_t *idx, const void *cmp, const void *val,
                                    const uint8_t *mask, int64_t n, void *old,
                                    tx_stream_t stream) {
  if (n < 0 || nbins < 0)
    return fail(TX_INVALID_ARGUMENT, "tx_atomic_cas_scatter: n = %lld, nbins = %lld",
                (long long)n, (long long)nbins);
  if (nbins > INT32_MAX)
    return fail(TX_UNSUPPORTED, "tx_atomic_cas_scatter: nbins %lld exceeds int32 indexing",
                (long long)nbins);
  const bool w64 = bins_type == TX_I64 || bins_type == TX_U64 || bins_type == TX_F64;
  if (bins_type != TX_I32 && bins_type != TX_U32 && bins_type != TX_F32 && !w64)
    return fail(TX_INVALID_ARGUMENT, "tx_atomic_cas_scatter: bins must be 32- or 64-bit (got type %d)",
                int(bins_type));
  if (n == 0) return TX_SUCCESS;
  if (!idx || !cmp || !val || (!bins && nbins > 0))
    return fail(TX_INVALID_ARGUMENT, "tx_atomic_cas_scatter: NULL buffer");
  const size_t es = w64 ? 8 : 4;
  if (!aligned(idx, 4) || !aligned(cmp, es) || !aligned(val, es) || (bins && !aligned(bins, es)) ||
      (old && !aligned(old, es)))
    return fail(TX_INVALID_ARGUMENT, "tx_atomic_cas_scatter: idx must be 4-byte and bins / cmp / val / old "
                "%zu-byte aligned", es);
  tx_cas_args args{bins, idx, static_cast<const uint32_t *>(cmp), static_cast<const uint32_t *>(val),
                   mask, static_cast<uint32_t *>(old), n, int32_t(nbins), 0};
  const char *kname = w64 ? "tx_scatter_cas64" : "tx_scatter_cas";
  hipFunction_t fn;
  TX_TRY(get_kernel(CodeObject::Scatter, kname, &fn));
  return launch(fn, direct_grid(n), 1, 256, static_cast<hipStream_t>(stream), &args, sizeof args, kname);
}

// Table form: operands = {bins (result slot), idx, cmp, val, mask, old, nbins,
// n, bins_type}.  mask and old may be NULL pointers.
static tx_status atomic_cas_op(tx_value *v, size_t count, tx_stream_t stream) {
  Operands o{v, count, "tt.atomic_cas"};
  TX_TRY(o.need(9));
  void *bins, *idx, *cmp, *val, *mask, *old;
  int64_t nbins, n, bt;
  TX_TRY(o.ptr(0, &bins));
  TX_TRY(o.ptr(1, &idx));
  TX_TRY(o.ptr(2, &cmp));
  TX_TRY(o.ptr(3, &val));
  TX_TRY(o.ptr(4, &mask));
  TX_TRY(o.ptr(5, &old));
  TX_TRY(o.integer(6, &nbins));
  TX_TRY(o.integer(7, &n));
  TX_TRY(o.integer(8, &bt));
  return atomic_cas_scatter(bins, tx_dtype(bt), nbins, static_cast<const int32_t *>(idx), cmp, val,
                            static_cast<const uint8_t *>(mask), n, old, stream);
}

// tt.histogram (passed through beside the atomics,
// uTLXConversionPatterns.cpp:605; Triton's tl.histogram(x, num_bins) with
// its optional mask): counts[b] = #{i < n : mask[i] != 0, x[i] == b} for
// 0 <= b < num_bins, values outside the range not counted.  counts is
// overwritten: a zero-fill launch, then the aggregating integer-add scatter
// with one per update (no value array is read).
static tx_status histogram(const int32_t *x, const uint8_t *mask, int64_t n, int32_t *counts, int64_t num_bins,
                           tx_stream_t stream) {
  const char *what = "tx_histogram";
  if (n < 0 || num_bins < 0)
    return fail(TX_INVALID_ARGUMENT, "%s: n = %lld, num_bins = %lld", what, (long long)n, (long long)num_bins);
  if (num_bins > INT32_MAX) return fail(TX_UNSUPPORTED, "%s: num_bins exceeds int32 indexing", what);
  if (num_bins == 0) return TX_SUCCESS;
  if (!counts || (n > 0 && !x)) return fail(TX_INVALID_ARGUMENT, "%s: NULL buffer", what);
  if (!aligned(counts, 4) || !aligned(x, 4))
    return fail(TX_INVALID_ARGUMENT, "%s: x and counts must be 4-byte aligned", what);
  hipStream_t s = static_cast<hipStream_t>(stream);
  tx_scatter_args zero{counts, nullptr, nullptr, nullptr, nullptr, num_bins, 0, 0, 0, 0};
  hipFunction_t fn;
  TX_TRY(get_kernel(CodeObject::Scatter, "tx_scatter_zero_bins", &fn));
  TX_TRY(launch(fn, direct_grid(num_bins), 1, 256, s, &zero, sizeof zero, "tx_scatter_zero_bins"));
  if (n == 0) return TX_SUCCESS;
  tx_scatter_args args{counts, x, nullptr, mask, nullptr, n, int32_t(num_bins), 0, 0, 0};
  return aggregate(args, "add", s);
}

// Table form: operands = {counts (result slot, int32[num_bins]), x:i32*,
// mask:u8*|NULL, n, num_bins}.
static tx_status histogram_op(tx_value *v, size_t count, tx_stream_t stream) {
  Operands o{v, count, "tt.histogram"};
  TX_TRY(o.need(5));
  void *counts, *x, *mask;
  int64_t n, nb;
  TX_TRY(o.ptr(0, &counts));
  TX_TRY(o.ptr(1, &x));
  TX_TRY(o.ptr(2, &mask));
  TX_TRY(o.integer(3, &n));
  TX_TRY(o.integer(4, &nb));
  return histogram(static_cast<const int32_t *>(x), static_cast<const uint8_t *>(mask), n,
                   static_cast<int32_t *>(counts), nb, stream);
}

static const bool registered_histogram = register_op(
    "tt.histogram", histogram_op, "counts:i32*(result, num_bins), x:i32*, mask:u8*|null, n:i64, num_bins:i64");
static const bool registered = register_op(
    "tt.atomic_rmw", atomic_rmw_op,
    "bins(result), idx:i32*, val, mask:u8*|null, old|null, nbins:i64, n:i64, "
    "bins_type:i32, op:i32");
static const bool registered_cas = register_op(
    "tt.atomic_cas", atomic_cas_op,
    "bins(result), idx:i32*, cmp, val, mask:u8*|null, old|null, nbins:i64, n:i64, bins_type:i32");

}  // namespace tx

extern "C" TX_API tx_status tx_atomic_rmw_scatter(void *bins, tx_dtype bins_type,
                                                  int64_t nbins, const int32_t *idx,
                                                  const void *val, const uint8_t *mask,
                                                  int64_t n, tx_rmw_op op, void *old,
                                                  tx_stream_t stream) {
  tx::clear_error();
  return tx::atomic_rmw_scatter(bins, bins_type, nbins, idx, val, mask, n, op, old, stream);
}

extern "C" TX_API tx_status tx_atomic_cas_scatter(void *bins, tx_dtype bins_type, int64_t nbins,
                                                  const int32_t *idx, const void *cmp,
                                                  const void *val, const uint8_t *mask, int64_t n,
                                                  void *old, tx_stream_t stream) {
  tx::clear_error();
  return tx::atomic_cas_scatter(bins, bins_type, nbins, idx, cmp, val, mask, n, old, stream);
}

extern "C" TX_API tx_status tx_histogram(const int32_t *x, const uint8_t *mask, int64_t n, int32_t *counts,
                                         int64_t num_bins, tx_stream_t stream) {
  tx::clear_error();
  return tx::histogram(x, mask, n, counts, num_bins, stream);
}
