/*
 * Kernel argument blocks, shared by the host launchers (csrc/host) and the
 * gfx950 kernels (csrc/kernels).  Each kernel takes exactly one of these
 * structs by value, so the kernarg segment is the struct itself.
 * Plain C layout only: fixed-width integers and raw pointers.
 */
#ifndef TX_KERNEL_ARGS_H
#define TX_KERNEL_ARGS_H

#include <stdint.h>

/* fp8 codec: n elements; vector kernels process n_vec = a multiple of their
 * block chunk, the tail kernel processes [start, n). */
typedef struct tx_fp8_codec_args {
  const void *src;
  void *dst;
  int64_t start; /* first element this launch handles */
  int64_t n;     /* one past the last element this launch handles */
  const uint32_t *rbits; /* stochastic rounding: one random word per element */
} tx_fp8_codec_args;

/* absmax + fp8 quantisers: x (fp32 or bf16) rows x K (ldx elements) ->
 * q fp8 rows x K (ldq bytes) and scales (MX: e8m0 bytes rows x K/32, ld_s
 * bytes; row-wise: fp32[rows]).  vec: rows and pitches allow the 16-byte
 * loads / 8-byte stores of the vector path. */
typedef struct tx_quant_args {
  const void *x;
  uint8_t *q;
  void *scales;
  int64_t ldx;
  int64_t ldq;
  int64_t ld_s;
  int64_t rows;
  int64_t K;
  int32_t vec;
  int32_t reserved;
} tx_quant_args;

/* scatter-reduce */
typedef struct tx_scatter_args {
  void *bins;
  const int32_t *idx;
  const void *val;
  const uint8_t *mask; /* may be NULL */
  void *old;           /* may be NULL (aggregating kernels ignore it) */
  int64_t n;
  int32_t nbins;
  int32_t per_block;   /* updates per chunk (multiple of 4 * blockDim) */
  int32_t splits;      /* windowed kernels: bin windows (workgroups per chunk) */
  int32_t window;      /* windowed kernels: bins per window */
  /* windowed kernels, one-pass path: in-range updates outside the window go
   * to the spill buffer (keys at spill_keys, values at spill_vals), region
   * (chunk * 16 + wavefront) of spill_wave records each, unused records
   * marked with key -1; a full region sends the rest to global atomics.
   * NULL: all of them go to global atomics. */
  uint32_t *spill_keys;
  uint32_t *spill_vals;
  int32_t spill_wave;
  int32_t reserved;
} tx_scatter_args;

/* tt.atomic_cas in scatter form: 32-bit bins, compared bit for bit */
typedef struct tx_cas_args {
  void *bins;
  const int32_t *idx;
  const uint32_t *cmp;
  const uint32_t *val;
  const uint8_t *mask; /* may be NULL */
  uint32_t *old;       /* may be NULL */
  int64_t n;
  int32_t nbins;
  int32_t pad;
} tx_cas_args;

/* GEMM, both operands K-contiguous ("A row-major, B column-major").
 * Element strides for bf16; byte strides for fp8. */
typedef struct tx_gemm_args {
  const void *A;
  const void *B;
  void *C;
  const float *scale_a; /* fp8 only */
  const float *scale_b; /* fp8 only */
  int64_t lda;
  int64_t ldb;
  int64_t ldc;
  int32_t M;
  int32_t N;
  int32_t K;
  int32_t tiles_m;   /* ceil(M / tile) */
  int32_t tiles_n;   /* ceil(N / tile) */
  int32_t group_m;   /* rasterisation group height in tiles */
  int32_t splits;    /* fast path: K splits (<= 1: none) */
  int32_t ksteps_split; /* fast path: 128-byte K steps per split */
  float *part;       /* fast path with splits > 1: splits x M x N fp32 partial sums */
  /* MX-scaled dot: e8m0 block scales (one byte per 32 K elements), packed
   * step-major: the scales of row r for 128-byte K step s are sd dwords
   * (low byte first) at byte s * ld_mx* + 4 sd r: blocks 4s .. 4s+3 for fp8
   * (sd = 1), 8s .. 8s+7 for fp4 (sd = 2), for every row of every tile (rows
   * past M / N hold finite codes). */
  const uint8_t *mx_a;
  const uint8_t *mx_b;
  int64_t ld_mxa;
  int64_t ld_mxb;
  /* fp8 GEMM epilogue (used when epi != 0): y = act(scaled sum + bias[n]),
   * written as out_kind (EPI_OUT_*); fp8 outputs are y * out_mul, rounded to
   * nearest even with saturation. */
  const float *bias;   /* NULL: none */
  int32_t act;         /* EPI_ACT_* */
  int32_t out_kind;    /* EPI_OUT_* */
  float out_mul;
  int32_t epi;
  /* tt.dot's accumulator operand (split-K reduce with epi only): fp32 M x N
   * (ld_acc elements) added to the scaled sum before the bias; NULL: none. */
  const float *acc;
  int64_t ld_acc;
} tx_gemm_args;

/* Grouped / batched fp8 GEMM (row/column scales, bf16 out) over the fast
 * tile.  g holds the shared fields (B, C, scales, strides, N, K, tiles_n,
 * group_m; A and C at problem 0).  Grouped (offsets != NULL): problem p is
 * rows offsets[p] .. offsets[p + 1] of A, C and scale_a (g.M = the rows of
 * A in all; offsets are clamped to 0 .. g.M), against B + p * stride_b and
 * scale_b + p * stride_sb; tile_prefix[p] = sum over q < p of
 * ceil(rows_q / 256) (written by tx_gemm_fp8_grouped_prefix).  Batched
 * (offsets == NULL): problem p is g.M rows at A + p * stride_a (elements),
 * scale_a + p * stride_sa, C + p * stride_c.  The grid covers mtiles x
 * tiles_n tiles; m tiles past the last problem's exit at once.  With g.epi
 * the fast tile's fused epilogue writes C as g.out_kind (strides in
 * elements of that type). */
typedef struct tx_grouped_args {
  tx_gemm_args g;
  const int32_t *offsets;
  int32_t *tile_prefix;
  int64_t stride_a;
  int64_t stride_sa;
  int64_t stride_c;
  int64_t stride_b;
  int64_t stride_sb;
  int64_t stride_bias;  /* fused epilogue (g.epi): bias of problem p at g.bias + p * stride_bias */
  int32_t groups;
  int32_t mtiles;       /* m tiles the grid covers */
  int32_t tiles_per;    /* batched: ceil(g.M / 256) */
  int32_t tile_rows;    /* grouped: rows of A per m tile (256; 128 in the transposed tile) */
} tx_grouped_args;

enum { EPI_ACT_NONE = 0, EPI_ACT_RELU = 1, EPI_ACT_GELU_TANH = 2, EPI_ACT_SILU = 3 };
enum { EPI_OUT_BF16 = 0, EPI_OUT_F16 = 1, EPI_OUT_F32 = 2, EPI_OUT_E4M3FN = 3, EPI_OUT_E5M2 = 4 };

/* Step-major repack of MX scales: with sd dwords per row and K step (1 for
 * fp8, 2 for fp4), dword j of row r for step s sits at byte
 * s * 4 * sd * rows_pad + 4 * (sd * r + j) and holds src[r][4 (sd s + j) .. +3],
 * with 127 (2^0) for r >= rows or a block >= cols. */
typedef struct tx_mx_pack_args {
  const uint8_t *src;
  uint8_t *dst;
  int64_t src_ld;   /* bytes between source rows */
  int32_t rows;
  int32_t cols;     /* scale blocks per source row, ceil(K / 32) */
  int32_t steps;    /* K steps of the kernel */
  int32_t rows_pad; /* rows of the packed matrix (whole tiles) */
  int32_t sd;       /* dwords per row and step */
  int32_t reserved;
} tx_mx_pack_args;

/* Both operands' repacks in one launch: workgroups [0, blocks0) pack op[0],
 * the rest op[1]. */
typedef struct tx_mx_pack2_args {
  tx_mx_pack_args op[2];
  int32_t blocks0;
  int32_t reserved;
} tx_mx_pack2_args;

/* Row copy into a zero-padded buffer: dst[r][c] = c < cols ? src[r][c] : 0
 * for c < dst_cols (elements of elem_bytes bytes; dst rows 16-byte aligned,
 * dst_cols a multiple of 16 / elem_bytes). */
typedef struct tx_pad_args {
  const void *src;
  void *dst;
  int64_t src_ld;    /* elements */
  int64_t dst_ld;    /* elements */
  int32_t rows;
  int32_t cols;
  int32_t dst_cols;
  int32_t load_bytes; /* source load width: 8, 4, 2 or 1 (see pad_rows) */
} tx_pad_args;

/* fp8 dequant GEMV */
typedef struct tx_gemv_args {
  const uint16_t *x; /* bf16 bits */
  const uint8_t *W;
  const float *scales;
  uint16_t *y;       /* bf16 bits */
  int64_t ldx;
  int64_t ldw;
  int64_t ld_scales;
  int64_t ldy;
  int32_t M;
  int32_t N;
  int32_t K;
  int32_t group;
  int32_t rows_per_wg; /* MFMA kernels: W rows per workgroup (at most 16 per W block) */
  int32_t pad_;
} tx_gemv_args;

#endif /* TX_KERNEL_ARGS_H */
