// Shared GEMM machinery for the bf16 and fp8 tt.dot kernels on gfx950.
//
// Layout contract (both operands K-contiguous, as tt.dot's A row-major /
// B column-major case at test_amd_gemm_pipelined.py:303-331 with B stored as
// N rows of K):
//   A: M rows of K elements (row stride lda), B: N rows of K (row stride ldb),
//   C: row-major M x N bf16 (row stride ldc).
//
// Tiling: a workgroup owns a BM x BN tile of C and walks K in steps of one
// 128-byte row slice (64 bf16 or 128 fp8 elements).  Each step stages the
// BM x 128 B slice of A and the BN x 128 B slice of B in LDS; every 128-byte
// LDS row holds 8 chunks of 16 bytes stored at chunk ^ ((row >> 1) & 7).
// gfx950's LDS serves a ds_read_b128 16 lanes at a time over 64 banks
// (256 bytes); the fragment reads have 16 lanes read the same logical chunk
// of 16 consecutive rows, and with this swizzle those 16 chunks fall in 16
// different 16-byte bank groups (row parity picks the half of the 256-byte
// bank window, (row >> 1) & 7 the chunk within it).  Two LDS stages are
// used: global loads for step k+1 are in flight (in registers) while step k
// is multiplied, then written to the other stage, with one barrier per step.
//
// MFMA roles: the B tile feeds the MFMA "A" operand and the A tile the MFMA
// "B" operand, so an MFMA result block is C^T: lane l, register j holds
// C[m0 + (l % 16)][n0 + 4 * (l / 16) + j].  Each lane therefore owns 4
// consecutive columns of one row, which the epilogue writes as one 8-byte
// store.  Within one MFMA the K order of the operand lanes is a free choice
// as long as both operands use the same one: lane group g = l / 16 holds the
// two 16-byte chunks 2g and 2g+1 of the 128-byte slice.
#pragma once

#include <type_traits>

#include "fp8_encode.h"
#include "tx_device.h"

namespace txg {

// ------------------------------------------------------------ epilogues
// y = act(v + bias[n]) for the fp8 GEMMs' fused epilogue (v already carries
// the row / column scales).  relu keeps NaN; gelu is the tanh form
// 0.5 y (1 + tanh(sqrt(2/pi) (y + 0.044715 y^3))) (Hendrycks & Gimpel),
// evaluated as y / (1 + e^(-2u)) with u the tanh argument (the identity
// 0.5 (1 + tanh u) = 1 / (1 + e^(-2u))); silu is y / (1 + e^-y).  Both use
// the hardware exp and reciprocal (a few ulp in fp32: the outputs are
// bf16 / fp16 / fp8 or an fp8 product's fp32 sum).
template <int ACT>
__device__ __forceinline__ float epi_act_t(float v) {
  if constexpr (ACT == EPI_ACT_RELU) return v < 0.0f ? 0.0f : v;
  else if constexpr (ACT == EPI_ACT_GELU_TANH)
    return __fdividef(v, 1.0f + __expf(-1.5957691216f * (v + 0.044715f * v * v * v)));
  else if constexpr (ACT == EPI_ACT_SILU) return __fdividef(v, 1.0f + __expf(-v));
  else return v;
}

__device__ __forceinline__ float epi_act(int act, float v) {
  switch (act) {
    case EPI_ACT_RELU: return epi_act_t<EPI_ACT_RELU>(v);
    case EPI_ACT_GELU_TANH: return epi_act_t<EPI_ACT_GELU_TANH>(v);
    case EPI_ACT_SILU: return epi_act_t<EPI_ACT_SILU>(v);
    default: return v;
  }
}

// f(integral_constant<int, ACT>) for the runtime activation `act`.
template <class F>
__device__ __forceinline__ void with_act(int act, F &&f) {
  switch (act) {
    case EPI_ACT_RELU: f(std::integral_constant<int, EPI_ACT_RELU>{}); break;
    case EPI_ACT_GELU_TANH: f(std::integral_constant<int, EPI_ACT_GELU_TANH>{}); break;
    case EPI_ACT_SILU: f(std::integral_constant<int, EPI_ACT_SILU>{}); break;
    default: f(std::integral_constant<int, EPI_ACT_NONE>{}); break;
  }
}

__device__ __forceinline__ float epi_value(const tx_gemm_args &a, float v, int n) {
  if (a.bias) v += a.bias[n];
  return epi_act(a.act, v);
}

// One output element of C (row-major, ldc elements) in the epilogue's type.
__device__ __forceinline__ void epi_store1(const tx_gemm_args &a, int64_t m, int64_t n, float y) {
  const int64_t i = m * a.ldc + n;
  switch (a.out_kind) {
    case EPI_OUT_F16: static_cast<uint16_t *>(a.C)[i] = uint16_t(txd::pack_f16x2(y, 0.0f)); break;
    case EPI_OUT_F32: static_cast<float *>(a.C)[i] = y; break;
    case EPI_OUT_E4M3FN:
      static_cast<uint8_t *>(a.C)[i] = uint8_t(txf::encode_rtne<txf::E4M3FN, true>(__float_as_uint(y * a.out_mul)));
      break;
    case EPI_OUT_E5M2:
      static_cast<uint8_t *>(a.C)[i] = uint8_t(txf::encode_rtne<txf::E5M2, true>(__float_as_uint(y * a.out_mul)));
      break;
    default: static_cast<uint16_t *>(a.C)[i] = uint16_t(txd::f32_to_bf16_bits(y)); break;
  }
}

// Four consecutive outputs C[m][n .. n+3] (n + 3 < N), one vector store when
// the row and pitch allow it.
__device__ __forceinline__ void epi_store4(const tx_gemm_args &a, int64_t m, int64_t n, const float (&y)[4]) {
  const int64_t i = m * a.ldc + n;
  const uintptr_t base = reinterpret_cast<uintptr_t>(a.C);
  switch (a.out_kind) {
    case EPI_OUT_F32:
      if (((base | uintptr_t(4 * i)) & 15) == 0) {
        *reinterpret_cast<txd::f32x4 *>(static_cast<float *>(a.C) + i) = txd::f32x4{y[0], y[1], y[2], y[3]};
        return;
      }
      break;
    case EPI_OUT_E4M3FN:
    case EPI_OUT_E5M2:
      if (((base | uintptr_t(i)) & 3) == 0) {
        // saturate (NaN kept), then the hardware's round-to-nearest-even
        const float fmax = a.out_kind == EPI_OUT_E4M3FN ? 448.0f : 57344.0f;
        float c[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float v = y[t] * a.out_mul;
          c[t] = v > fmax ? fmax : (v < -fmax ? -fmax : v);
        }
        *reinterpret_cast<uint32_t *>(static_cast<uint8_t *>(a.C) + i) =
            a.out_kind == EPI_OUT_E4M3FN ? txf::encode_clamped4_hw<txf::E4M3FN>(c)
                                         : txf::encode_clamped4_hw<txf::E5M2>(c);
        return;
      }
      break;
    default:
      if (((base | uintptr_t(2 * i)) & 7) == 0) {
        const bool h = a.out_kind == EPI_OUT_F16;
        *reinterpret_cast<txd::u32x2 *>(static_cast<uint16_t *>(a.C) + i) =
            h ? txd::u32x2{txd::pack_f16x2(y[0], y[1]), txd::pack_f16x2(y[2], y[3])}
              : txd::u32x2{txd::pack_bf16x2(y[0], y[1]), txd::pack_bf16x2(y[2], y[3])};
        return;
      }
      break;
  }
#pragma unroll
  for (int t = 0; t < 4; ++t) epi_store1(a, m, n + t, y[t]);
}

using txd::f32x4;
using txd::i32x8;
using txd::u32x4;

constexpr int kRowBytes = 128;  // one K step of one row, in bytes
constexpr int kChunks = 8;      // 16-byte chunks per row

__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row >> 1) & 7); }

// Byte offset of (row, chunk) inside one LDS operand stage.
__device__ __forceinline__ int lds_off(int row, int chunk) {
  return row * kRowBytes + swz(row, chunk) * 16;
}

// Load one 16-byte chunk of a K-contiguous row with pieces of VEC bytes,
// zero-filling pieces past the end of the row (kb_end bytes) or invalid rows.
template <int VEC>
__device__ __forceinline__ u32x4 load_chunk(const uint8_t *row_ptr, int kb, int kb_end, bool row_ok) {
  u32x4 v = {0u, 0u, 0u, 0u};
  if constexpr (VEC == 16) {
    if (row_ok && kb < kb_end) v = *reinterpret_cast<const u32x4 *>(row_ptr + kb);
  } else if constexpr (VEC == 8) {
    txd::u32x2 lo = {0u, 0u}, hi = {0u, 0u};
    if (row_ok && kb < kb_end) lo = *reinterpret_cast<const txd::u32x2 *>(row_ptr + kb);
    if (row_ok && kb + 8 < kb_end) hi = *reinterpret_cast<const txd::u32x2 *>(row_ptr + kb + 8);
    v.x = lo.x; v.y = lo.y; v.z = hi.x; v.w = hi.y;
  } else if constexpr (VEC == 4) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = (row_ok && kb + 4 * i < kb_end) ? *reinterpret_cast<const uint32_t *>(row_ptr + kb + 4 * i) : 0u;
    v.x = w[0]; v.y = w[1]; v.z = w[2]; v.w = w[3];
  } else if constexpr (VEC == 2) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t lo = (row_ok && kb + 4 * i < kb_end) ? *reinterpret_cast<const uint16_t *>(row_ptr + kb + 4 * i) : 0u;
      uint32_t hi = (row_ok && kb + 4 * i + 2 < kb_end) ? *reinterpret_cast<const uint16_t *>(row_ptr + kb + 4 * i + 2) : 0u;
      w[i] = lo | (hi << 16);
    }
    v.x = w[0]; v.y = w[1]; v.z = w[2]; v.w = w[3];
  } else {  // VEC == 1
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t acc = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int o = kb + 4 * i + b;
        const uint32_t byte = (row_ok && o < kb_end) ? row_ptr[o] : 0u;
        acc |= byte << (8 * b);
      }
      w[i] = acc;
    }
    v.x = w[0]; v.y = w[1]; v.z = w[2]; v.w = w[3];
  }
  return v;
}

// Tile id -> (tile_m, tile_n) in groups of group_m tile rows, so that
// neighbouring tiles share A and B panels.
__device__ __forceinline__ void raster_coords(int pid, int tiles_m, int tiles_n, int group_m, int *tm, int *tn) {
  const int in_group = group_m * tiles_n;
  const int gid = pid / in_group;
  const int first_m = gid * group_m;
  const int gsz = (tiles_m - first_m) < group_m ? (tiles_m - first_m) : group_m;
  const int r = pid % in_group;
  *tm = first_m + r % gsz;
  *tn = r / gsz;
}

// Regroup linear workgroup ids so that each of the 8 XCDs (workgroups are
// dispatched round-robin over XCDs) gets a contiguous range of `total` ids.
__device__ __forceinline__ int xcd_contiguous(int wg, int total) {
  const int per = total / 8, rem = total % 8;
  const int x = wg % 8, i = wg / 8;
  return x * per + (x < rem ? x : rem) + i;
}

// Map a linear workgroup id to a (tile_m, tile_n) pair: XCD-contiguous tile
// ids, rasterised in groups of group_m tile rows so that neighbouring tiles
// share A and B panels in the XCD's L2.
__device__ __forceinline__ void tile_coords(int wg, int tiles_m, int tiles_n, int group_m,
                                            int *tm, int *tn) {
  raster_coords(xcd_contiguous(wg, tiles_m * tiles_n), tiles_m, tiles_n, group_m, tm, tn);
}

// Split-K grids (tiles x splits workgroups): XCD-contiguous ids taken
// split-major, so the workgroups of one XCD run one split (one K range of A,
// which its L2 then holds) over neighbouring tiles, and the tiles that share
// a B column panel in that K range run on the same XCD at the same time.
__device__ __forceinline__ void split_coords(int wg, int tiles_m, int tiles_n, int splits, int group_m,
                                             int *tm, int *tn, int *split) {
  const int tiles = tiles_m * tiles_n;
  const int pid = xcd_contiguous(wg, tiles * splits);
  *split = pid / tiles;
  raster_coords(pid % tiles, tiles_m, tiles_n, group_m, tm, tn);
}

// Copy rows into a zero-padded buffer (see tx_pad_args): one 16-byte chunk of
// a destination row per thread.  The source is read LW bytes at a time, LW
// (a.load_bytes: 8, 4, 2 or 1) dividing the source base address, its row
// pitch and its row length in bytes, so every load lies wholly inside or
// wholly past the row (the source rows are what the fast path could not
// take: not 16-byte aligned).
template <int ES, int LW>
__device__ __forceinline__ void pad_rows_w(const tx_pad_args &a) {
  constexpr int PER = 16 / ES;  // elements per 16-byte chunk
  using L = typename std::conditional<
      LW == 8, uint64_t,
      typename std::conditional<LW == 4, uint32_t,
                                typename std::conditional<LW == 2, uint16_t, uint8_t>::type>::type>::type;
  const int64_t chunks_per_row = a.dst_cols / PER;
  const int64_t total = int64_t(a.rows) * chunks_per_row;
  const int64_t row_bytes = int64_t(a.cols) * ES;
  for (int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
       t += int64_t(gridDim.x) * blockDim.x) {
    const int64_t r = t / chunks_per_row;
    const int64_t b0 = (t % chunks_per_row) * 16;
    const uint8_t *s = reinterpret_cast<const uint8_t *>(a.src) + r * a.src_ld * ES;
    uint8_t chunk[16] __attribute__((aligned(16)));
#pragma unroll
    for (int i = 0; i < 16 / LW; ++i) {
      const int64_t off = b0 + i * LW;
      *reinterpret_cast<L *>(chunk + i * LW) = off < row_bytes ? *reinterpret_cast<const L *>(s + off) : L(0);
    }
    *reinterpret_cast<u32x4 *>(reinterpret_cast<uint8_t *>(a.dst) + r * a.dst_ld * ES + b0) =
        *reinterpret_cast<const u32x4 *>(chunk);
  }
}

template <int ES>
__device__ __forceinline__ void pad_rows(const tx_pad_args &a) {
  switch (a.load_bytes) {
    case 8: pad_rows_w<ES, 8>(a); break;
    case 4: pad_rows_w<ES, 4>(a); break;
    case 2: pad_rows_w<ES, 2>(a); break;
    default: pad_rows_w<ES, 1>(a); break;
  }
}

// A row-major K x N operand of 16-bit elements (`rows` = K source rows of
// `cols` = N elements, pitch src_ld) -> N rows of dst_cols (a multiple of
// 64, >= K) elements, pitch dst_ld: dst[n][k] = src[k][n], zero for k >= K.
// One workgroup of 256 threads per 64 (n) x 64 (k) tile, blockIdx.x the n
// tile, blockIdx.y the k tile.  Thread t loads 8 consecutive n of source
// rows k and k + 1 (k = 2 (t / 8), n = 8 (t % 8) within the tile; 16-byte
// loads when VEC) and writes them to LDS as 8 dwords (k, k + 1) in the rows
// of their n; then each thread writes two 16-byte runs of 8 k of one n.
// The LDS tile is 64 rows of 36 dwords with the dword column XORed by
// 8 (row / 8 mod 4): the 64 lanes' dword writes then fall at most two to a
// bank, and a 16-byte read of dwords 4q .. 4q + 3 stays contiguous.
template <bool VEC>
__device__ __forceinline__ void transpose_kn(const tx_pad_args &a) {
  constexpr int P = 36;  // LDS row pitch in dwords
  __shared__ __attribute__((aligned(16))) uint32_t t[64 * P];
  const int tid = threadIdx.x;
  const int n0 = blockIdx.x * 64, k0 = blockIdx.y * 64;
  const uint16_t *src = static_cast<const uint16_t *>(a.src);
  {
    const int p = tid >> 3, c = tid & 7;
    const int k = k0 + 2 * p, n = n0 + 8 * c;
    uint32_t lo[4] = {0u, 0u, 0u, 0u}, hi[4] = {0u, 0u, 0u, 0u};  // n pairs of rows k, k + 1
    auto load = [&](int kk, uint32_t (&w)[4]) {
      if (kk >= a.rows) return;
      const uint16_t *row = src + int64_t(kk) * a.src_ld + n;
      if (VEC && n + 8 <= a.cols) {
        const u32x4 v = *reinterpret_cast<const u32x4 *>(row);
        w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (n + j < a.cols) w[j / 2] |= uint32_t(row[j]) << (16 * (j % 2));
      }
    };
    load(k, lo);
    load(k + 1, hi);
    const int col = p ^ (8 * (c & 3));  // row 8c + j has (row / 8) mod 4 = c mod 4
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t e0 = (lo[j / 2] >> (16 * (j % 2))) & 0xFFFFu;
      const uint32_t e1 = (hi[j / 2] >> (16 * (j % 2))) & 0xFFFFu;
      t[(8 * c + j) * P + col] = e0 | (e1 << 16);
    }
  }
  __syncthreads();
  uint16_t *dst = static_cast<uint16_t *>(a.dst);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int u = tid + 256 * i;
    const int r = u >> 3, q = u & 7;  // tile row n0 + r, k run 8q .. 8q + 7
    const int d0 = (4 * q) ^ (8 * ((r >> 3) & 3));
    const u32x4 w = *reinterpret_cast<const u32x4 *>(&t[r * P + d0]);
    if (n0 + r < a.cols)
      *reinterpret_cast<u32x4 *>(dst + int64_t(n0 + r) * a.dst_ld + k0 + 8 * q) = w;
  }
}

}  // namespace txg
