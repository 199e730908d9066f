/*
 * tx_plugin.h -- C ABI of libtxamd.so, the MI355X (gfx950) op library that
 * replaces the data-parallel ops Triton lowers for the reference's plugin path.
 *
 * Two layers, both plain C (no HIP, torch or MLIR types cross this boundary):
 *
 *  1. The registration surface.  txGetPluginInfo() returns a table of ops in
 *     the shape of the reference's PluginInfo (support/Export.h:15,
 *     support/Export.cpp:58-97, extensions/utlx/uTLXPlugin.cpp:700-814):
 *     {api_version, name, version, ops*, num_ops, target}.  Each entry is
 *     {name, fn, signature}, keyed by the Triton op it implements.  The op
 *     calling convention follows the reference's OpInfo callbacks
 *     (uTLXPlugin.cpp:40-50, ops/NewOps.cpp:295-302): operands[0] is the
 *     result slot, inputs start at operands[1], scalar options follow as
 *     integer constants.  Unlike the reference, txReleasePluginInfo is
 *     defined (it is only declared at support/Export.h:17).
 *
 *  2. Typed entry points, one per op, taking device pointers, sizes, strides
 *     and a stream.  The table's fn pointers unpack operands and call these.
 *
 * Conventions (all entry points):
 *  - The caller owns every input and output buffer.  tx_dot_bf16,
 *    tx_dot_fp8_scaled[_ex] and tx_dot_scaled_mx may use device scratch that
 *    the library keeps per (device, stream): fp32 split-K partial planes
 *    (at most 16 x M x N x 4 bytes) when the output tiles leave CUs idle,
 *    zero-padded copies of A and B when the kernels cannot read their rows
 *    in place (fp8: rows not 16-byte aligned or K not a multiple of 16;
 *    bf16 / fp16: rows not 4-byte aligned, and ragged K in the few shapes
 *    only the 8-wavefront 256 x 256 tile takes) in a product of at least
 *    2^30 multiply-adds (tx_dot_scaled_mx: in any product), the e4m3fn expansion of an fp4 operand that meets an fp8
 *    one (tx_dot_scaled_mx), and repacked MX scale rows.  The scratch is allocated
 *    stream-ordered (hipMallocAsync on `stream`) the first time a stream
 *    needs it, grown the same way, and reused by later calls, so
 *    steady-state calls allocate nothing; requests above 512 MiB get a
 *    buffer per call.  If the allocation fails, tx_dot_bf16 and
 *    tx_dot_fp8_scaled run without it and tx_dot_scaled_mx returns the
 *    error.  tx_atomic_rmw_scatter (aggregating form, more bins than one
 *    36,864-bin LDS window) takes the same scratch for its spill buffer
 *    (8 bytes x 8,192 records per CU: 16 MiB on 256 CUs) and without it
 *    sends those updates to global atomics.  No other entry point
 *    allocates device memory.  txShutdown frees the kept scratch.  The
 *    library owns its code-object handles, loaded once per device on first
 *    use (or by txInit) and unloaded by txShutdown.
 *  - Work is enqueued on `stream` (a hipStream_t; NULL = the null stream)
 *    and is stream-ordered; entry points return after enqueueing.
 *  - Errors are returned as tx_status (0 = success, as TP_SUCCESS in
 *    support/Export.h:25-28); txGetLastError() gives the calling thread's
 *    last message.  No exception or abort crosses the ABI.
 *  - Entry points are reentrant; concurrent calls on different streams are
 *    allowed.
 */
#ifndef TX_PLUGIN_H
#define TX_PLUGIN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#define TX_API __attribute__((visibility("default")))
#else
#define TX_API
#endif

#define TX_PLUGIN_API_VERSION 1u

typedef void *tx_stream_t; /* hipStream_t */

typedef enum tx_status {
  TX_SUCCESS = 0,            /* TP_SUCCESS, support/Export.h:26 */
  TX_GENERIC_FAILURE = 1,    /* TP_GENERIC_FAILURE, support/Export.h:27 */
  TX_INVALID_ARGUMENT = 2,   /* null pointer, negative size, bad stride */
  TX_UNSUPPORTED = 3,        /* valid request this library does not serve */
  TX_NO_DEVICE = 4,          /* no HIP device, or not a gfx950 device */
  TX_CODE_OBJECT_ERROR = 5,  /* a gfx950 code object failed to load */
  TX_LAUNCH_ERROR = 6,       /* the HIP runtime rejected a launch */
  TX_UNKNOWN_OP = 7          /* no op of that name in the table */
} tx_status;

/* Element types (the tt dtypes of the path: tl.float32, tl.float8e4nv,
 * tl.float8e5, tl.bfloat16, tl.float16, tl.int32; utility.py:92-105 names the fp8 ones
 * "e4m3" and "e5m2"). */
typedef enum tx_dtype {
  TX_F32 = 0,
  TX_FP8E4M3FN = 1,
  TX_FP8E5M2 = 2,
  TX_BF16 = 3,
  TX_I32 = 4,
  TX_U32 = 5,
  TX_F16 = 6,
  TX_FP4E2M1 = 7, /* OCP MX fp4: 1 sign, 2 exponent (bias 1), 1 mantissa bit; two per byte,
                    the lower K index in the low nibble (tx_dot_scaled_mx operands) */
  TX_I64 = 8,     /* tl.int64 (tx_atomic_rmw_scatter bins) */
  TX_U64 = 9,     /* tl.uint64 */
  TX_F64 = 10,    /* tl.float64 */
  TX_I8 = 11      /* tl.int8 (tx_dot_acc operands) */
} tx_dtype;

/* Rounding modes, numbered as the rounding operand of
 * utlx_fp_to_fp_with_rbits (ops/NewOps.cpp:270-286): 0 rtne, 1 rtz, 2 rs. */
typedef enum tx_rounding { TX_RTNE = 0, TX_RTZ = 1, TX_RS = 2 } tx_rounding;

/* Read-modify-write kinds of tt.atomic_rmw (Triton's RMWOp). */
typedef enum tx_rmw_op {
  TX_RMW_ADD = 0,  /* integer add, wraps modulo 2^32 (2^64 for 64-bit bins) */
  TX_RMW_FADD = 1, /* floating-point add: fp32, fp64, fp16 or bf16 bins */
  TX_RMW_MAX = 2,  /* signed integer max */
  TX_RMW_MIN = 3,  /* signed integer min */
  TX_RMW_UMAX = 4, /* unsigned integer max */
  TX_RMW_UMIN = 5, /* unsigned integer min */
  TX_RMW_AND = 6,
  TX_RMW_OR = 7,
  TX_RMW_XOR = 8,
  TX_RMW_XCHG = 9  /* exchange: the bin takes val (any 32- or 64-bit bins) */
} tx_rmw_op;

/* Storage of tt.dot's B operand (K x N) in tx_dot. */
typedef enum tx_b_layout {
  TX_B_NK = 0, /* column-major K x N: N rows of K elements, row stride ldb >= K */
  TX_B_KN = 1  /* row-major K x N: K rows of N elements, row stride ldb >= N
                  (the layout of the reference's matmul(a, b) caller) */
} tx_b_layout;

/* Activations of the fp8 GEMM's fused epilogue (tx_dot_fp8_scaled_ex). */
typedef enum tx_activation {
  TX_ACT_NONE = 0,
  TX_ACT_RELU = 1,      /* y < 0 ? 0 : y (NaN kept) */
  TX_ACT_GELU_TANH = 2, /* 0.5 y (1 + tanh(sqrt(2/pi) (y + 0.044715 y^3))) */
  TX_ACT_SILU = 3       /* y / (1 + exp(-y)) */
} tx_activation;

/* ----------------------------------------------------------------------- */
/* Registration surface                                                     */
/* ----------------------------------------------------------------------- */

typedef enum tx_value_kind { TX_VALUE_PTR = 0, TX_VALUE_INT = 1 } tx_value_kind;

/* One operand: a device pointer or an integer constant (the reference passes
 * scalar options as arith.constant values, decoded by extractConstantInt,
 * uTLXPlugin.cpp:40-50). */
typedef struct tx_value {
  int32_t kind; /* tx_value_kind */
  int32_t reserved;
  union {
    void *ptr;
    int64_t i;
  } u;
} tx_value;

/* Op callback: the counterpart of plugin::OpInfo::add (support/Export.cpp:82-84). */
typedef tx_status (*tx_op_fn)(tx_value *operands, size_t num_operands,
                              tx_stream_t stream);

typedef struct tx_op_info {
  const char *name;      /* Triton op name, e.g. "tt.fp_to_fp" */
  tx_op_fn fn;
  const char *signature; /* operand list, human readable */
} tx_op_info;

/* Counterpart of plugin::PluginInfo (uTLXPlugin.cpp:801-812). */
typedef struct tx_plugin_info {
  uint32_t api_version; /* TX_PLUGIN_API_VERSION */
  const char *name;     /* "txamd" */
  const char *version;  /* library version string */
  const tx_op_info *ops;
  size_t num_ops;
  const char *target;   /* "gfx950" */
} tx_plugin_info;

/* Replaces tritonGetPluginInfo (support/Export.h:15, uTLXPlugin.cpp:700).
 * Each call returns a fresh table that stays valid until released. */
TX_API const tx_plugin_info *txGetPluginInfo(void);

/* Replaces tritonReleasePluginInfo (declared, never defined, at
 * support/Export.h:17).  Frees a table from txGetPluginInfo; NULL is a no-op. */
TX_API void txReleasePluginInfo(const tx_plugin_info *info);

/* Look an op up by name in the registry (NULL if absent). */
TX_API const tx_op_info *txFindOp(const char *name);

/* Invoke a registered op by name (TX_UNKNOWN_OP if absent). */
TX_API tx_status txInvokeOp(const char *name, tx_value *operands,
                            size_t num_operands, tx_stream_t stream);

/* Thread-local message for the calling thread's last failing call ("" if none). */
TX_API const char *txGetLastError(void);

/* Load the gfx950 code objects on the current device (optional: every entry
 * point does this on first use).  TX_NO_DEVICE without a gfx950 device. */
TX_API tx_status txInit(void);

/* Unload code objects on every device this process initialised. */
TX_API void txShutdown(void);

/* Library version string. */
TX_API const char *txVersion(void);

/* Diagnostic with no counterpart in the reference: the number of device
 * allocations the library has made for its stream scratch since the process
 * started (split-K partials, padded operand copies, transposes, group tile
 * prefixes; each first use or growth of a (stream, use) buffer counts one).
 * Lets a caller that must not allocate check that a call did not. */
TX_API uint64_t txScratchAllocations(void);

/* Diagnostic with no counterpart in the reference: HBM ceiling kernels with
 * exactly the launch shape of the fp32 -> fp8 encode of tx_fp_to_fp, for
 * measuring how close the encode comes to what the memory system gives that
 * shape.  kind 0: dst[i] = low byte of the 32-bit word src[i] (4 bytes read,
 * 1 written per element, no conversion work); kind 1: reads src[0 .. n) and
 * writes dst only where the XOR of a thread's 16 words equals n (so the
 * loads stay).  src: n 32-bit words, 16-byte aligned; dst: n bytes, 4-byte
 * aligned; n a multiple of 4096. */
TX_API tx_status txStreamCeiling(int kind, const void *src, void *dst, int64_t n, tx_stream_t stream);

/* ----------------------------------------------------------------------- */
/* Typed entry points                                                       */
/* ----------------------------------------------------------------------- */

/*
 * tt.fp_to_fp, elementwise over n contiguous elements.
 * Replaces Triton's lowering of tt.fp_to_fp (emitted by semantic.cast,
 * semantic.py:807-827; passed through at uTLXConversionPatterns.cpp:577;
 * re-created with a rounding attribute by createFpToFpWithRbits,
 * ops/NewOps.cpp:249-303).
 *  - TX_F32 -> TX_FP8E4M3FN / TX_FP8E5M2 / TX_F16 / TX_BF16 with rounding
 *    TX_RTNE or TX_RTZ.
 *    saturate = 0: overflow and +-Inf become NaN (e4m3fn) or +-Inf (e5m2,
 *    fp16, bf16); round toward zero keeps finite values finite.
 *    saturate = 1: the reference's clamp(x, -max, max)-then-convert idiom
 *    (mxfp8_utils.py:17-21, 36-38): overflow and +-Inf become +-max, NaN
 *    stays NaN.  NaN input gives 0x7F (fp8), 0x7E00 (fp16) or 0x7FC0
 *    (bf16) with the input's sign bit.
 *  - TX_FP8E4M3FN / TX_FP8E5M2 -> TX_F32 (exact; NaN codes give 0x7FC00000
 *    with the code's sign).
 *  - TX_BF16 / TX_F16 / TX_FP8E4M3FN / TX_FP8E5M2 -> any other of TX_F32,
 *    TX_BF16, TX_F16, TX_FP8E4M3FN, TX_FP8E5M2 (x.to(tl.float8e4nv) on bf16
 *    activations, fp8 -> bf16 upcasts, ...): the source value widened to
 *    fp32 (exactly) and converted as above, so it is rounded once, with the
 *    same rounding, saturation and NaN rules.  Conversions to a format that
 *    holds every source value (fp8 -> fp16 / bf16 / fp32, fp16 / bf16 ->
 *    fp32) are exact under any rounding; saturation there only maps e5m2's
 *    +-Inf to +-max of an fp16 / bf16 destination (an fp32 destination
 *    keeps infinities, as the fp8 -> fp32 decode does).
 * TX_RS needs random bits and an fp32 source: use tx_fp_to_fp_with_rbits
 * (TX_UNSUPPORTED here).
 */
TX_API tx_status tx_fp_to_fp(const void *src, tx_dtype src_type, void *dst,
                             tx_dtype dst_type, int64_t n,
                             tx_rounding rounding, int saturate,
                             tx_stream_t stream);

/*
 * tt.fp_to_fp with a random-bits operand, as built by
 * utlx_fp_to_fp_with_rbits (createFpToFpWithRbits, ops/NewOps.cpp:249-303;
 * used by tlx.stoch_round, test_tlx.py:5138-5153).  With TX_RTNE / TX_RTZ it
 * is tx_fp_to_fp (rbits unused, may be NULL).  With TX_RS (stochastic
 * rounding): src_type must be TX_F32 and dst_type one of TX_F16, TX_BF16,
 * TX_FP8E5M2, TX_FP8E4M3FN (others: TX_INVALID_ARGUMENT, as the reference's
 * stoch_round raises, test_tlx.py:5291-5329); rbits holds one 32-bit word
 * per element; the result always saturates (the reference lowers it to
 * cvt.rs.satfinite, test_tlx.py:5182) and `saturate` is ignored.  Each
 * element becomes its round-toward-zero value, moved one step away from
 * zero iff rbits[i] + floor(frac * 2^32) >= 2^32, frac being the fraction of
 * an ulp that truncation dropped: with uniform random bits the result rounds
 * up with probability frac (to 2^-32) and is unbiased.  NaN stays NaN (as
 * for tx_fp_to_fp); +-Inf and |x| above max give +-max.
 */
TX_API tx_status tx_fp_to_fp_with_rbits(const void *src, tx_dtype src_type, void *dst,
                                        tx_dtype dst_type, const uint32_t *rbits,
                                        int64_t n, tx_rounding rounding, int saturate,
                                        tx_stream_t stream);

/*
 * tt.atomic_rmw in scatter form: for every i < n with mask[i] != 0 (mask may
 * be NULL) and 0 <= idx[i] < nbins, atomically bins[idx[i]] = bins[idx[i]]
 * (op) val[i].  Replaces Triton's per-lane lowering of tl.atomic_add and
 * friends (tt.atomic_rmw, passed through at uTLXConversionPatterns.cpp:611;
 * used at test_tlx.py:7627-7629 and 7687).  bins_type is TX_I32, TX_U32,
 * TX_I64 or TX_U64 for the integer ops and TX_F32, TX_F64, TX_F16 or TX_BF16
 * for TX_RMW_FADD; val has the bins' type.  Updates are pre-aggregated (in
 * registers, within a wavefront, and in an LDS table per workgroup) before
 * they reach global memory, so floating-point sums are order-dependent
 * within rounding.  fp16 / bf16 bins: a workgroup's updates of one bin are
 * summed in fp32 and the bin is rounded to nearest even once per such
 * partial (once per update when the bins exceed one LDS table of 36864, or
 * with old).  64-bit bins are pre-aggregated up to 18432 bins.
 * If old != NULL, every update instead returns the bin's value before it was
 * applied (the tt.atomic_rmw result) in old[i] (0 for dropped updates), and
 * no pre-aggregation is done.
 * TX_RMW_XCHG takes TX_I32, TX_U32, TX_F32, TX_I64, TX_U64 or TX_F64 bins
 * (the bit pattern is exchanged) and is one atomic per update: where several
 * updates hit one
 * bin they apply one at a time in an order the hardware picks, so the bin
 * ends with one of their values and, with old, their old values are the
 * bin's initial value and the other updates' values.
 */
TX_API tx_status tx_atomic_rmw_scatter(void *bins, tx_dtype bins_type,
                                       int64_t nbins, const int32_t *idx,
                                       const void *val, const uint8_t *mask,
                                       int64_t n, tx_rmw_op op, void *old,
                                       tx_stream_t stream);

/*
 * tt.histogram (passed through beside the atomics at
 * uTLXConversionPatterns.cpp:605; Triton's tl.histogram(x, num_bins, mask)):
 * counts[b] = the number of i < n with mask[i] != 0 (mask may be NULL) and
 * x[i] == b, for 0 <= b < num_bins; values outside [0, num_bins) are not
 * counted.  counts (int32[num_bins]) is overwritten.  Served by the
 * aggregating scatter of tx_atomic_rmw_scatter with one added per update.
 */
TX_API tx_status tx_histogram(const int32_t *x, const uint8_t *mask, int64_t n, int32_t *counts,
                              int64_t num_bins, tx_stream_t stream);

/*
 * tt.atomic_cas in scatter form: for every i < n with mask[i] != 0 (mask may
 * be NULL) and 0 <= idx[i] < nbins, atomically
 *   old[i] = bins[idx[i]]; if (old[i] == cmp[i]) bins[idx[i]] = val[i];
 * comparing the bit patterns (bins_type TX_I32, TX_U32, TX_F32, TX_I64,
 * TX_U64 or TX_F64; cmp, val and old of the same type).  Replaces Triton's
 * per-lane lowering of
 * tl.atomic_cas (tt.atomic_cas, passed through at
 * uTLXConversionPatterns.cpp:610).  old may be NULL; dropped updates return
 * 0.  Updates of one bin apply one at a time in an order the hardware
 * picks.
 */
TX_API tx_status tx_atomic_cas_scatter(void *bins, tx_dtype bins_type,
                                       int64_t nbins, const int32_t *idx,
                                       const void *cmp, const void *val,
                                       const uint8_t *mask, int64_t n,
                                       void *old, tx_stream_t stream);

/*
 * tt.dot with bf16 operands, fp32 accumulation and bf16 output:
 * C[m,n] = bf16_rne(sum_k A[m,k] * B[k,n]).
 * Replaces Triton's MFMA lowering of tt.dot (TritonDotPattern,
 * uTLXConversionPatterns.cpp:227-296; the kernel at
 * test_amd_gemm_pipelined.py:184-300 and its host wrapper :303-331).
 * A: row-major M x K, row stride lda (elements).
 * B: column-major K x N, i.e. N rows of K elements, row stride ldb.
 * C: row-major M x N, row stride ldc.
 * Any M, N, K >= 0 (K = 0 gives zeros); strides >= the row length.
 */
TX_API tx_status tx_dot_bf16(const void *A, int64_t lda, const void *B,
                             int64_t ldb, void *C, int64_t ldc, int64_t M,
                             int64_t N, int64_t K, tx_stream_t stream);

/*
 * tt.dot with 16-bit operands, fp32 accumulation and a 16-bit output:
 * C[m,n] = out_rne(sum_k A[m,k] * B[k,n]).
 * Replaces Triton's MFMA lowering of tt.dot for fp16 / bf16 operands
 * (TritonDotPattern, uTLXConversionPatterns.cpp:227-296) behind the
 * reference's only AMD GEMM caller: matmul(a, b) with fp16 a (M x K,
 * row-major) and fp16 b (K x N, row-major), fp16 output
 * (test_amd_gemm_pipelined.py:303-331; its kernel accumulates in fp32 and
 * casts, :259-299).
 * ab_type: TX_BF16 or TX_F16 (both operands).  c_type: TX_BF16 or TX_F16.
 * A: row-major M x K, row stride lda (elements).
 * B: b_layout TX_B_NK (N rows of K, ldb >= K) or TX_B_KN (K rows of N,
 *    ldb >= N).  A TX_B_KN operand is read in place when the product takes
 *    the persistent tile (at least one 64 x 64 tile per CU or K <= 2048, K a
 *    multiple of 64, N a multiple of 8, 16-byte aligned rows); otherwise it is first
 *    transposed into the library's stream scratch (N rows of K rounded up
 *    to 64, zero-filled), which fails with TX_GENERIC_FAILURE if that
 *    allocation fails.
 * C: row-major M x N, row stride ldc.
 * Any M, N, K >= 0 (K = 0 gives zeros).
 */
TX_API tx_status tx_dot(const void *A, tx_dtype ab_type, int64_t lda,
                        const void *B, tx_b_layout b_layout, int64_t ldb,
                        void *C, tx_dtype c_type, int64_t ldc, int64_t M,
                        int64_t N, int64_t K, tx_stream_t stream);

/*
 * tt.dot with its accumulator operand.  TritonDotPattern keeps c as a real
 * operand of tt.dot (uTLXConversionPatterns.cpp:273, 290-291) and the
 * reference's AMD kernel chains it through its K loop (accumulator =
 * tl.dot(a, b, accumulator), test_amd_gemm_pipelined.py:274, 292):
 *   D[m,n] = round_d( s[m,n] * sum_k f32(A[m,k]) * f32(B[k,n]) + C[m,n] )
 * in fp32, with s = scale_a[m] * scale_b[n] for fp8 operands and 1 for
 * 16-bit ones, rounded once to d_type (TX_F32, TX_BF16 or TX_F16, nearest
 * even).  Operands: bf16 or fp16 (a_type == b_type; scale_a, scale_b NULL;
 * B stored N x K or row-major K x N as tx_dot), or fp8 (TX_FP8E4M3FN /
 * TX_FP8E5M2 in any pairing, B stored N x K, fp32 scale_a[M], scale_b[N]),
 * or fp32 (both; fp32 products and sums, input precision "ieee", d_type
 * TX_F32), or int8 (both TX_I8; exact int32 sums wrapping modulo 2^32,
 * d_type TX_I32, C then holds int32), these two with B stored N x K and
 * NULL scales.
 * C: fp32 row-major M x N (ldc elements), or NULL for D = round_d(s * A.B);
 * C may be D itself when d_type is TX_F32 and ldc == ldd (accumulating in
 * place, as the reference's K loop does).  Non-finite values propagate as in
 * fp32 arithmetic.  Uses stream scratch (fp32 partial sums of M x N per K
 * split; operand copies when rows are misaligned or B is K x N).
 */
TX_API tx_status tx_dot_acc(const void *A, tx_dtype a_type, int64_t lda, const float *scale_a,
                            const void *B, tx_dtype b_type, tx_b_layout b_layout, int64_t ldb,
                            const float *scale_b, const float *C, int64_t ldc, void *D,
                            tx_dtype d_type, int64_t ldd, int64_t M, int64_t N, int64_t K,
                            tx_stream_t stream);

/*
 * tt.dot on fp8 operands with a per-row / per-column scale epilogue:
 * C[m,n] = bf16_rne(scale_a[m] * scale_b[n] * sum_k f32(A[m,k]) * f32(B[k,n])).
 * No reference kernel exists; the closed form follows the scaled-dot check
 * at test_tlx.py:2271-2292 with fp32 per-row/per-column scales in place of
 * e8m0 block scales.  a_type/b_type are TX_FP8E4M3FN or TX_FP8E5M2.
 * A: row-major M x K bytes (lda); B: column-major, N rows of K bytes (ldb);
 * C: row-major bf16 (ldc).  scale_a has M floats, scale_b has N floats.
 * Non-finite codes keep their decoded meaning (tt.fp_to_fp's fp8 -> fp32,
 * uTLXConversionPatterns.cpp:577): e4m3fn 0x7F / 0xFF are NaN, e5m2 0x7C /
 * 0xFC are +-Inf and its other all-ones-exponent codes NaN, so an output
 * is NaN where its sum reads a NaN or meets Inf * 0 or Inf - Inf, and
 * +-Inf where it reads Inf otherwise, on every kernel this entry point (and
 * the _ex / grouped / batched / MX forms below) may pick.
 */
TX_API tx_status tx_dot_fp8_scaled(const void *A, tx_dtype a_type, int64_t lda,
                                   const float *scale_a, const void *B,
                                   tx_dtype b_type, int64_t ldb,
                                   const float *scale_b, void *C, int64_t ldc,
                                   int64_t M, int64_t N, int64_t K,
                                   tx_stream_t stream);

/*
 * tx_dot_fp8_scaled with a fused epilogue, the adjacent caller in serving
 * stacks (a GEMM followed by bias, activation and a cast, often back to
 * fp8).  No reference kernel exists; the product is tx_dot_fp8_scaled's:
 *   y[m,n] = act(scale_a[m] * scale_b[n] * sum_k f32(A[m,k]) * f32(B[k,n]) + bias[n])
 * in fp32 (bias may be NULL; activation a tx_activation), then C[m,n] =
 *   bf16 / fp16 (round to nearest even) or fp32 of y (c_type TX_BF16,
 *   TX_F16, TX_F32), or fp8 (TX_FP8E4M3FN / TX_FP8E5M2) of y * (1 / c_scale)
 *   rounded to nearest even with saturation (c_scale > 0; NaN stays NaN).
 * Layouts as tx_dot_fp8_scaled; C row-major with ldc elements of c_type,
 * aligned to its element size.  Skinny (M <= 64) and misaligned products
 * stage the scaled sums in the library's per-stream scratch (M x N x 4 bytes).
 */
TX_API tx_status tx_dot_fp8_scaled_ex(const void *A, tx_dtype a_type, int64_t lda,
                                      const float *scale_a, const void *B, tx_dtype b_type,
                                      int64_t ldb, const float *scale_b, const float *bias,
                                      int activation, void *C, tx_dtype c_type, float c_scale,
                                      int64_t ldc, int64_t M, int64_t N, int64_t K,
                                      tx_stream_t stream);

/*
 * Grouped tx_dot_fp8_scaled_ex (the grouped variant serving stacks call for
 * mixture-of-experts layers): one launch computes, for every group p,
 *   y[r, n] = act(scale_a[r] * scale_b[p * stride_scale_b + n] *
 *                 sum_k f32(A[r, k]) * f32(B_p[k, n]) + bias[p * stride_bias + n])
 * for the rows r of A in group_offsets[p] .. group_offsets[p + 1], where
 * B_p is the column-major N x K operand at B + p * stride_b bytes, and
 * writes C[r, n] as tx_dot_fp8_scaled_ex does (c_type bf16 / fp16 / fp32,
 * or fp8 of y / c_scale; bias may be NULL, activation a tx_activation; with
 * no bias, no activation and bf16 it is tx_dot_fp8_scaled per group).  No
 * reference kernel exists.
 * group_offsets: groups + 1 int32 row offsets on the device, nondecreasing,
 * within 0 .. M (M = rows of A and C in all; values outside are clamped);
 * they are read by the device only, so the call never waits for them.
 * A row-major (lda bytes), C row-major (ldc elements of c_type), scale_a M
 * floats.
 * Operands as the fast path reads them in place: A and B 16-byte aligned,
 * lda, ldb, K and stride_b multiples of 16 (else TX_UNSUPPORTED).  Uses
 * (groups + 1) x 4 bytes of the library's per-stream scratch.
 */
TX_API tx_status tx_dot_fp8_scaled_grouped(const void *A, tx_dtype a_type, int64_t lda,
                                           const float *scale_a, const void *B,
                                           tx_dtype b_type, int64_t ldb, int64_t stride_b,
                                           const float *scale_b, int64_t stride_scale_b,
                                           const float *bias, int64_t stride_bias,
                                           int activation, void *C, tx_dtype c_type,
                                           float c_scale, int64_t ldc,
                                           const int32_t *group_offsets, int64_t groups,
                                           int64_t M, int64_t N, int64_t K,
                                           tx_stream_t stream);

/*
 * tx_dot_fp8_scaled_grouped for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  Same arguments, checks and
 * results as tx_dot_fp8_scaled_grouped; its group tile prefix lives in a
 * fixed 64 KiB device array, one per GPU, held until the process ends, so
 * groups is at most 16383 (more: TX_UNSUPPORTED).  It calls no hipMalloc,
 * hipFree or other allocating routine once txInit() has run on the device
 * (txInit loads the code objects and looks up the array; without it the
 * first call on a device does both).  All calls on one GPU share the
 * array: calls that overlap on one GPU (different streams, or unordered
 * threads) race.
 */
TX_API tx_status tx_dot_fp8_scaled_grouped_noalloc(const void *A, tx_dtype a_type, int64_t lda,
                                                   const float *scale_a, const void *B,
                                                   tx_dtype b_type, int64_t ldb, int64_t stride_b,
                                                   const float *scale_b, int64_t stride_scale_b,
                                                   const float *bias, int64_t stride_bias,
                                                   int activation, void *C, tx_dtype c_type,
                                                   float c_scale, int64_t ldc,
                                                   const int32_t *group_offsets, int64_t groups,
                                                   int64_t M, int64_t N, int64_t K,
                                                   tx_stream_t stream);

/*
 * Batched tx_dot_fp8_scaled: `batch` products of one shape in one launch,
 * product p on A + p * stride_a bytes, scale_a + p * stride_scale_a,
 * B + p * stride_b bytes, scale_b + p * stride_scale_b and C + p * stride_c
 * elements (M x N each).  No reference kernel exists.  Alignment as
 * tx_dot_fp8_scaled_grouped (stride_a too a multiple of 16).
 */
TX_API tx_status tx_dot_fp8_scaled_batched(const void *A, tx_dtype a_type, int64_t lda,
                                           int64_t stride_a, const float *scale_a,
                                           int64_t stride_scale_a, const void *B,
                                           tx_dtype b_type, int64_t ldb, int64_t stride_b,
                                           const float *scale_b, int64_t stride_scale_b,
                                           void *C, int64_t ldc, int64_t stride_c,
                                           int64_t batch, int64_t M, int64_t N, int64_t K,
                                           tx_stream_t stream);

/*
 * tt.dot_scaled with MX block scales (OCP Microscaling: one e8m0 scale per
 * 32 consecutive K elements of each row of A and each column of B), fp32
 * accumulation:
 * C[m,n] = out(sum_k A[m,k] * 2^(sa[m][k/32] - 127) * B[k,n] * 2^(sb[n][k/32] - 127)).
 * e8m0 code e in 0..254 is 2^(e - 127) (0 is 2^-127, not zero); 255 is NaN.
 * Replaces the scaled MMA of the reference's TLX ops (async_dot_scaled,
 * tlx/mma_ops.py:163-237, lowered through GenericOpPattern<DotScaledOp>,
 * uTLXConversionPatterns.cpp:616); closed form of its check at
 * test_tlx.py:2271-2292, whose `bits << 23` scale decode agrees for codes
 * 1..254.  a_type/b_type are TX_FP8E4M3FN, TX_FP8E5M2 or TX_FP4E2M1 in any
 * pairing (the "e4m3" / "e5m2" / "e2m1" formats of async_dot_scaled; an
 * fp4 operand that meets an fp8 one is first expanded to e4m3fn, exactly,
 * in the library's scratch).
 * A: row-major M rows of K bytes (fp8) or K/2 bytes (fp4, K even), row
 * stride lda in bytes; B: column-major, N rows likewise (ldb bytes).
 * scale_a: e8m0 bytes, row-major M x ceil(K/32) (row stride ld_scale_a);
 * scale_b: N x ceil(K/32) (ld_scale_b).  Past K inside the last block the
 * operands count as zero.
 * C: row-major M x N (ldc elements) of c_type TX_F32, TX_BF16 or TX_F16
 * (round to nearest even; fp16 overflows to Inf).
 * Uses the library's per-stream scratch (see the conventions above) for
 * the scales, repacked into the layout the kernel reads (about
 * 4 * ceil(K/128) * (M + N) bytes), and for zero-padded operand rows when
 * rows are not 16-byte aligned or K is not a multiple of 16.
 */
TX_API tx_status tx_dot_scaled_mx(const void *A, tx_dtype a_type, int64_t lda,
                                  const uint8_t *scale_a, int64_t ld_scale_a, const void *B,
                                  tx_dtype b_type, int64_t ldb, const uint8_t *scale_b,
                                  int64_t ld_scale_b, void *C, tx_dtype c_type, int64_t ldc,
                                  int64_t M, int64_t N, int64_t K, tx_stream_t stream);

/*
 * absmax + fp8 quantiser with MX block scales, the producer in front of
 * tx_dot_scaled_mx.  Follows the reference's _compute_scale_and_quantize /
 * _to_mxfp8_block (extensions/utlx/python/utlx_plugin/mxfp8_utils.py:10-56)
 * for each block of 32 consecutive elements of a row:
 *   amax  = max |x| over the block (NaN ignored, as tl.max),
 *   e     = ((bits(amax / fmax) + 0x007FFFFF) & 0x7F800000) >> 23   (fp32
 *           division, round to nearest; the e8m0 scale written to scales),
 *   q     = fp8_rne(clamp(x * (1 / 2^(e - 127)), +-fmax))   (x * 0 when e = 0),
 * fmax = 448 (TX_FP8E4M3FN) or 57344 (TX_FP8E5M2).  NaN inputs give the NaN
 * code; an infinite amax gives e = 255 and zeros (NaN for the infinities).
 * x: fp32 or bf16 (x_type), row-major rows x K (ldx elements), K a multiple
 * of 32; q: fp8 row-major (ldq bytes); scales: e8m0 bytes rows x K/32
 * (ld_scales bytes).
 */
TX_API tx_status tx_quantize_mx(const void *x, tx_dtype x_type, int64_t ldx, void *q,
                                tx_dtype q_type, int64_t ldq, uint8_t *scales,
                                int64_t ld_scales, int64_t rows, int64_t K,
                                tx_stream_t stream);

/*
 * absmax + fp8 quantiser with one fp32 scale per row, the producer of
 * tx_dot_fp8_scaled's operands (rows of A, and rows of the N x K storage of
 * B, i.e. its columns).  No reference kernel exists; the form is the
 * reference's saturating idiom (clamp, then convert: mxfp8_utils.py:36-38)
 * with a per-row scale:
 *   amax = max |x| over the row (NaN ignored; 1 if it is 0),
 *   q = fp8_rne(clamp(x * (fmax / amax), +-fmax)),  scales[r] = amax / fmax
 * in fp32.  x: fp32 or bf16 rows x K (ldx elements); q: fp8 (ldq bytes);
 * scales: fp32[rows].
 */
TX_API tx_status tx_quantize_rowwise(const void *x, tx_dtype x_type, int64_t ldx, void *q,
                                     tx_dtype q_type, int64_t ldq, float *scales,
                                     int64_t rows, int64_t K, tx_stream_t stream);

/*
 * fp8 weight-only dequant GEMV / skinny GEMM:
 * y[m,n] = bf16_rne(sum_g scales[n,g] * sum_{k in group g} x[m,k] * f32(W[n,k])).
 * No reference kernel exists (the nearest is the fp8 tt.dot of
 * tx_dot_fp8_scaled).  x: bf16 row-major M x K (ldx); W: fp8 (w_type) row-major
 * N x K bytes (ldw); scales: fp32 row-major N x ceil(K/group) (ld_scales);
 * y: bf16 row-major M x N (ldy).  K and group are multiples of 128 (the last
 * group may be partial), M <= 64, x and W rows 16-byte aligned, scales 4-byte
 * aligned (TX_UNSUPPORTED otherwise).  NaN / Inf weight codes (e4m3fn 0x7F /
 * 0xFF; e5m2 0x7C / 0xFC Inf, the rest of its all-ones exponent NaN) and
 * NaN / Inf in x propagate as in fp32 arithmetic on the decoded values
 * (NaN, Inf * 0 and Inf - Inf give NaN), the same for every M.
 */
TX_API tx_status tx_gemv_fp8_dequant(const void *x, int64_t ldx, const void *W,
                                     tx_dtype w_type, int64_t ldw,
                                     const float *scales, int64_t ld_scales,
                                     int64_t group, void *y, int64_t ldy,
                                     int64_t M, int64_t N, int64_t K,
                                     tx_stream_t stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* TX_PLUGIN_H */
