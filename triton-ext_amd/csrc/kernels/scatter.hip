// tt.atomic_rmw in scatter form, bins[idx[i]] (op)= val[i], on gfx950.
//
// Triton lowers tl.atomic_add(bins + idx, v) to one global atomic per lane
// (tt.atomic_rmw, passed through at uTLXConversionPatterns.cpp:611), which
// serialises in L2 on hot bins.  These kernels reduce in three levels before
// global memory is touched:
//   1. registers: each lane loads 4 updates with one 128-bit load of indices
//      and one of values;
//   2. wavefront: runs of equal keys inside a wavefront are combined with a
//      ballot/read-lane loop before they reach a shared atomic (spill path);
//   3. workgroup: an LDS table owned by the workgroup.  Up to 4 x 36,864
//      bins the table is direct-mapped (slot = bin - window start), with the
//      bin range cut into windows that each fit in LDS, one workgroup per
//      chunk of updates making one pass per window -- or, when a sample of
//      the chunk finds one window holding most updates (skewed keys), a
//      single pass that privatises that window and sends the rest to global
//      atomics through per-wavefront LDS queues; beyond 4 windows it is an
//      open addressing hash
//      table (Fibonacci hash, bounded linear probing) keyed by bin, and
//      updates whose probe sequence is full spill to global atomics after a
//      wavefront-level combine.  At the end the table is flushed with one
//      global atomic per occupied slot.
// Every combine is an associative, commutative op, so integer results are
// exact and order independent; fp32 sums differ from a sequential sum only
// by rounding order.
#include "tx_device.h"

namespace {

enum Op { ADD = 0, FADD = 1, MAX = 2, MIN = 3, UMAX = 4, UMIN = 5, AND = 6, OR = 7, XOR = 8 };

constexpr int kBlock = 1024;
constexpr int64_t kIter = 4 * kBlock;       // updates per workgroup iteration
constexpr int kDepth = 3;                   // iterations of loads in flight (pipelined loop)
constexpr int kDirectSlots = 36864;          // 144 KiB of 4-byte counters
constexpr int kHashLog2 = 14;                // 16384 slots, 128 KiB keys + values
constexpr int kHashSlots = 1 << kHashLog2;
constexpr int kProbes = 4;
constexpr uint32_t kEmpty = 0xFFFFFFFFu;
// fp32 hot keys (see HotKeys): up to kHot keys, sampled in a 2048-slot table.
constexpr int kHot = 8;  // HotKeys::take names each of the kHot sums
constexpr int kSampleLog2 = 11;
constexpr int kSampleSlots = 1 << kSampleLog2;
constexpr uint32_t kHotMinCount = 16;        // of at most 4 x kBlock samples
// Per-wavefront spill queue of the one-pass window (see spill_push): kQueue
// keys and kQueue values per wavefront, in the LDS words the fp32 hot-key
// sample uses before the pass.
constexpr uint32_t kQueue = 128;
constexpr int kAuxWords = 2 * kSampleSlots;  // 16 KiB: the sample's keys and counts, or the queues
static_assert(kBlock / 64 * 2 * kQueue <= kAuxWords, "spill queues fit in the auxiliary LDS");

template <int OP> struct OpTraits;
template <> struct OpTraits<ADD> { using T = uint32_t; static __device__ T id() { return 0u; } };
// -0.0 is the exact identity of IEEE addition (x + -0 == x for every x,
// +0 included), so fp32 tables start at -0 and untouched slots can be skipped.
template <> struct OpTraits<FADD> { using T = float; static __device__ T id() { return -0.0f; } };
template <> struct OpTraits<MAX> { using T = int32_t; static __device__ T id() { return INT32_MIN; } };
template <> struct OpTraits<MIN> { using T = int32_t; static __device__ T id() { return INT32_MAX; } };
template <> struct OpTraits<UMAX> { using T = uint32_t; static __device__ T id() { return 0u; } };
template <> struct OpTraits<UMIN> { using T = uint32_t; static __device__ T id() { return 0xFFFFFFFFu; } };
template <> struct OpTraits<AND> { using T = uint32_t; static __device__ T id() { return 0xFFFFFFFFu; } };
template <> struct OpTraits<OR> { using T = uint32_t; static __device__ T id() { return 0u; } };
template <> struct OpTraits<XOR> { using T = uint32_t; static __device__ T id() { return 0u; } };

template <int OP, typename T>
__device__ __forceinline__ T combine(T a, T b) {
  if constexpr (OP == ADD || OP == FADD) return a + b;
  else if constexpr (OP == MAX || OP == UMAX) return a > b ? a : b;
  else if constexpr (OP == MIN || OP == UMIN) return a < b ? a : b;
  else if constexpr (OP == AND) return a & b;
  else if constexpr (OP == OR) return a | b;
  else return a ^ b;
}

// Atomic combine into LDS or global memory (the address space follows p).
template <int OP, typename T>
__device__ __forceinline__ void atomic_combine(T *p, T v) {
  if constexpr (OP == ADD || OP == FADD) atomicAdd(p, v);
  else if constexpr (OP == MAX || OP == UMAX) atomicMax(p, v);
  else if constexpr (OP == MIN || OP == UMIN) atomicMin(p, v);
  else if constexpr (OP == AND) atomicAnd(p, v);
  else if constexpr (OP == OR) atomicOr(p, v);
  else atomicXor(p, v);
}

// Slots still holding the identity are skipped when flushing.  For fp32 the
// test is on the bits: only -0 is an identity, +0 is not (it turns a -0 bin
// into +0).
// Combine one update per lane into an LDS table (`pend` marks the lanes with
// an update).  Integer ops use the native LDS atomics.  fp32 adds avoid
// ds_add_f32 where they can: on gfx950 it retires about 0.37 lanes per clock
// per CU, while ds_cmpst_rtn_b32 runs at 2.3 to 3.3 and ds_add_u32 at 4 to 6.
// Each lane tries one compare-and-swap (it compares bit patterns, so NaN and
// signed-zero slots behave like any other value); only the lanes that lose it
// (several lanes or wavefronts on one bin: hot keys) fall back to ds_add_f32,
// which never retries.
template <int OP, typename T>
__device__ __forceinline__ void wave_lds_combine(T *table, bool pend, uint32_t r, T v) {
  if constexpr (OP != FADD) {
    if (pend) atomic_combine<OP, T>(&table[r], v);
  } else {
    if (pend) {
      uint32_t *q = reinterpret_cast<uint32_t *>(table) + r;
      const uint32_t old = __atomic_load_n(q, __ATOMIC_RELAXED);
      if (atomicCAS(q, old, __float_as_uint(__uint_as_float(old) + v)) != old) atomicAdd(&table[r], v);
    }
  }
}

template <int OP, typename T>
__device__ __forceinline__ bool is_identity(T v) {
  if constexpr (OP == FADD) return __builtin_bit_cast(uint32_t, v) == 0x80000000u;
  else return v == OpTraits<OP>::id();
}

// Wavefront-level combine for the lanes in `pending` (a subset of active
// lanes): repeatedly take the lowest pending lane's key, gather every pending
// lane holding the same key, reduce their values across the wavefront, and
// let the leader issue one global atomic.
template <int OP, typename T>
__device__ __forceinline__ void wave_combine_global(T *bins, bool pending, uint32_t key, T v) {
  uint64_t todo = __ballot(pending);
  while (todo) {
    const int leader = __ffsll((unsigned long long)todo) - 1;
    const uint32_t lkey = __shfl(key, leader);
    const bool match = pending && key == lkey;
    const uint64_t mm = __ballot(match);
    T mine = match ? v : OpTraits<OP>::id();
    // butterfly reduction over the wavefront (identity for non-matching lanes)
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mine = combine<OP, T>(mine, __shfl_xor(mine, off));
    if (threadIdx.x % 64 == unsigned(leader)) atomic_combine<OP, T>(bins + lkey, mine);
    if (match) pending = false;
    todo &= ~mm;
  }
}

// Out-of-window updates of the one-pass window.  A global atomic inside the
// streaming loop would hold up the loads issued after it (vmcnt counts
// loads, stores and atomics together, in order), so each wavefront appends
// them to its queue in LDS (keys at q[0 .. kQueue), values at q[kQueue ..
// 2 kQueue); ballot + mbcnt give the slots) and sends the queue to global
// memory with whole-wavefront atomics only when it would overflow and at the
// end of the pass.  qn (the queue's fill) is wavefront-uniform.
template <int OP, typename T>
__device__ __forceinline__ void spill_flush(const uint32_t *q, uint32_t qn, T *bins) {
  for (uint32_t i = threadIdx.x & 63; i < qn; i += 64)
    atomic_combine<OP, T>(bins + q[i], __builtin_bit_cast(T, q[kQueue + i]));
}

// The wavefront's region of the spill buffer (see tx_scatter_args): `fill`
// records written of `cap` (both wavefront-uniform); keys == NULL: none.
struct SpillRegion {
  uint32_t *keys = nullptr, *vals = nullptr;
  uint32_t fill = 0, cap = 0;
  __device__ __forceinline__ void init(const tx_scatter_args &a) {
    if (!a.spill_keys) return;
    const int64_t r = (int64_t(blockIdx.x) * (kBlock / 64) + threadIdx.x / 64) * a.spill_wave;
    keys = a.spill_keys + r;
    vals = a.spill_vals + r;
    cap = uint32_t(a.spill_wave);
  }
  // mark the unused records (every lane of the wavefront takes part)
  __device__ __forceinline__ void close() {
    if (!keys) return;
    for (uint32_t i = fill + (threadIdx.x & 63); i < cap; i += 64) keys[i] = 0xFFFFFFFFu;
  }
};

// Send the queue's qn records to the region when they fit (whole-wavefront
// stores, read again by a second launch of the windowed kernel), else to the
// bins with global atomics.
template <int OP, typename T>
__device__ __forceinline__ void spill_out(const uint32_t *q, uint32_t qn, T *bins, SpillRegion &sr) {
  if (sr.keys && sr.fill + qn <= sr.cap) {
    for (uint32_t i = threadIdx.x & 63; i < qn; i += 64) {
      sr.keys[sr.fill + i] = q[i];
      sr.vals[sr.fill + i] = q[kQueue + i];
    }
    sr.fill += qn;
  } else {
    spill_flush<OP, T>(q, qn, bins);
  }
}

template <int OP, typename T>
__device__ __forceinline__ void spill_push(uint32_t *q, uint32_t &qn, T *bins, SpillRegion &sr, bool sp,
                                           uint32_t key, T v) {
  const uint64_t m = __ballot(sp);
  if (m == 0) return;
  const uint32_t cnt = uint32_t(__popcll(m));
  if (qn + cnt > kQueue) {
    spill_out<OP, T>(q, qn, bins, sr);
    qn = 0;
  }
  if (sp) {
    const uint32_t pos = qn + __builtin_amdgcn_mbcnt_hi(uint32_t(m >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(m), 0u));
    q[pos] = key;
    q[kQueue + pos] = __builtin_bit_cast(uint32_t, v);
  }
  qn += cnt;
}

// Hot keys of one workgroup's fp32 window.  ds_add_f32 retires about 0.3
// lanes per clock per CU however its addresses fall, so the compare-and-swap
// in wave_lds_combine carries fp32 adds; it loses whenever several lanes of
// an instruction, or several wavefronts at once, hit one bin, and skewed keys
// (Zipf: the top 8 of 65,536 bins draw a third of the updates) make that
// common.  (Integer ops do not use them: their native LDS atomics lose less
// to same-address lanes than the register accumulators cost.)  Each
// workgroup therefore samples the first 4 x kBlock
// updates of its chunk, counts the in-window keys in a small LDS hash table,
// and takes up to kHot keys seen at least kHotMinCount times.  Their updates
// never touch LDS: every lane combines them in registers (one accumulator
// per hot key), and the accumulators are reduced over the wavefront and
// combined into the table once, at the end of the chunk.  Which keys are
// chosen only moves work between the two paths; integer results are the
// same either way, fp32 sums up to rounding order.
template <int OP>
struct HotKeys {
  using T = typename OpTraits<OP>::T;
  int n = 0;            // number of hot keys (workgroup-uniform)
  uint32_t r[kHot];     // their window-relative slots (same in every lane); unused: kEmpty
  T acc[kHot];          // this lane's partial results

  // Route one update: a pending update on a hot slot is combined into that
  // slot's accumulator and stops pending.  Lanes that are not pending
  // combine the identity; no pending slot equals kEmpty (pending slots are
  // below the window size).
  __device__ __forceinline__ void take(bool &pend, uint32_t slot, T v) {
    const T x = pend ? v : OpTraits<OP>::id();
    bool hit = false;
#pragma unroll
    for (int t = 0; t < kHot; ++t) {
      const bool m = slot == r[t];
      acc[t] = combine<OP, T>(acc[t], m ? x : OpTraits<OP>::id());
      hit = hit || m;
    }
    // The accumulators are complete here, before any LDS atomic of this
    // update: left to itself the compiler sinks the combines past the
    // atomics and keeps all kHot compare masks alive in scalar registers
    // across them.
    asm volatile("" : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3]), "+v"(acc[4]),
                 "+v"(acc[5]), "+v"(acc[6]), "+v"(acc[7])::"memory");
    pend = pend && !hit;
  }
};

template <int OP>
struct Scatter {
  using T = typename OpTraits<OP>::T;

  // Load up to 4 updates for this lane starting at element e (e % 4 == 0).
  // `full` means all 4 are in range and the buffers are 16-byte aligned.
  static __device__ __forceinline__ void load4(const tx_scatter_args &a, int64_t e, int64_t end,
                                               bool vec, uint32_t key[4], T val[4],
                                               bool ok[4]) {
    const int32_t *idx = a.idx;
    const T *vals = reinterpret_cast<const T *>(a.val);
    if (vec && e + 4 <= end) {
      const txd::i32x4 k4 = __builtin_nontemporal_load(reinterpret_cast<const txd::i32x4 *>(idx + e));
      const txd::u32x4 v4 = vals ? __builtin_nontemporal_load(reinterpret_cast<const txd::u32x4 *>(vals + e))
                                 : txd::u32x4{1u, 1u, 1u, 1u};
      uint32_t mbits = 0xFFFFFFFFu;
      if (a.mask) mbits = *reinterpret_cast<const uint32_t *>(a.mask + e);
      const int32_t kk[4] = {k4.x, k4.y, k4.z, k4.w};
      const uint32_t vv[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        key[j] = uint32_t(kk[j]);
        val[j] = __builtin_bit_cast(T, vv[j]);
        ok[j] = kk[j] >= 0 && kk[j] < a.nbins && ((mbits >> (8 * j)) & 0xFFu) != 0;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t i = e + j;
        ok[j] = i < end;
        key[j] = 0;
        val[j] = OpTraits<OP>::id();
        if (ok[j]) {
          const int32_t k = idx[i];
          key[j] = uint32_t(k);
          val[j] = vals ? vals[i] : __builtin_bit_cast(T, 1u);
          ok[j] = k >= 0 && k < a.nbins && (!a.mask || a.mask[i] != 0);
        }
      }
    }
  }

  // One full iteration's worth of this lane's updates: 4 indices, 4 values
  // and (MASK) 4 mask bytes, each fetched with one load.
  template <bool MASK>
  static __device__ __forceinline__ void fetch(const tx_scatter_args &a, int64_t e, txd::i32x4 &k,
                                               txd::u32x4 &v, uint32_t &m) {
    k = __builtin_nontemporal_load(reinterpret_cast<const txd::i32x4 *>(a.idx + e));
    // no values: every update adds 1 (tt.histogram through the integer add)
    v = a.val ? __builtin_nontemporal_load(reinterpret_cast<const txd::u32x4 *>(a.val) + e / 4)
              : txd::u32x4{1u, 1u, 1u, 1u};
    if constexpr (MASK) m = *reinterpret_cast<const uint32_t *>(a.mask + e);
    else m = 0xFFFFFFFFu;
  }

  // Combine 4 updates into the LDS window [lo, lo + nb).  A key outside the
  // window (negative keys included: they wrap to large unsigned values) or
  // with a zero mask byte is dropped, or with SPILL, when it is in
  // [0, nbins), goes to the wavefront's spill queue q; lo + nb <= nbins <=
  // INT32_MAX.
  template <bool HOT, bool SPILL>
  static __device__ __forceinline__ void apply(T *table, uint32_t lo, uint32_t nb, T *bins, uint32_t nbins,
                                               uint32_t *q, uint32_t &qn, SpillRegion &sr, HotKeys<OP> &hot,
                                               const txd::i32x4 &k, const txd::u32x4 &v, uint32_t m) {
    const int32_t kk[4] = {k.x, k.y, k.z, k.w};
    const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t r = uint32_t(kk[j]) - lo;
      const bool live = ((m >> (8 * j)) & 0xFFu) != 0;
      bool pend = r < nb && live;
      const T x = __builtin_bit_cast(T, vv[j]);
      if constexpr (SPILL)
        spill_push<OP, T>(q, qn, bins, sr, live && !pend && uint32_t(kk[j]) < nbins, uint32_t(kk[j]), x);
      if constexpr (OP == FADD && HOT) hot.take(pend, r, x);
      wave_lds_combine<OP, T>(table, pend, r, x);
    }
  }

  // Pipelined pass over `groups` x kDepth full iterations starting at this
  // lane's element e0 (16-byte aligned index and value buffers): the loads of
  // the next kDepth iterations are in flight while an iteration's LDS atomics
  // run.  Slot d always holds an iteration congruent to d mod kDepth, so the
  // slots are compile-time registers; refills past the last iteration re-read
  // the last one (in range, never applied).
  template <bool MASK, bool HOT, bool SPILL>
  static __device__ __forceinline__ void stream(const tx_scatter_args &a, T *table, uint32_t lo,
                                                uint32_t nb, uint32_t *q, uint32_t &qn, SpillRegion &sr,
                                                HotKeys<OP> &hot, int64_t e0, int64_t groups) {
    T *bins = reinterpret_cast<T *>(a.bins);
    txd::i32x4 k[kDepth];
    txd::u32x4 v[kDepth];
    uint32_t m[kDepth];
#pragma unroll
    for (int d = 0; d < kDepth; ++d) fetch<MASK>(a, e0 + d * kIter, k[d], v[d], m[d]);
    const int64_t last = e0 + (groups * kDepth - 1) * kIter;
    for (int64_t g = 0; g < groups; ++g) {
      const int64_t eg = e0 + g * kDepth * kIter;
#pragma unroll
      for (int d = 0; d < kDepth; ++d) {
        apply<HOT, SPILL>(table, lo, nb, bins, uint32_t(a.nbins), q, qn, sr, hot, k[d], v[d], m[d]);
        const int64_t en = eg + (d + kDepth) * kIter;
        fetch<MASK>(a, en < last ? en : last, k[d], v[d], m[d]);
      }
    }
  }

  // The best single window for a chunk: counts the first 4 x kBlock updates
  // of the chunk per block of kWinBlock bins, and returns (workgroup-uniform)
  // the start of the `window`-bin window, at a multiple of kWinBlock, that
  // holds the most of them, with that count and the number sampled.  Every
  // workgroup of a chunk reads the same sample, so they all agree.  The
  // counts live in `cnt`, the first words of the workgroup's window table
  // (set up only afterwards).  Needs the whole workgroup; ends with a
  // barrier.
  static constexpr int kWinBlock = 2048;
  static constexpr int kMaxWinBlocks = 4 * kDirectSlots / kWinBlock;
  static __device__ __forceinline__ void pick_window(const tx_scatter_args &a, int64_t begin, int64_t end, bool vec,
                                     uint32_t window, uint32_t *cnt, uint32_t &base, uint32_t &hits,
                                     uint32_t &total) {
    for (int s = threadIdx.x; s < kMaxWinBlocks + 2; s += kBlock) cnt[s] = 0u;
    __syncthreads();
    {
      uint32_t key[4];
      T val[4];
      bool ok[4];
      load4(a, begin + 4 * int64_t(threadIdx.x), end, vec, key, val, ok);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (ok[j]) atomicAdd(&cnt[key[j] / kWinBlock], 1u);  // key < nbins <= 4 x kDirectSlots
    }
    __syncthreads();
    if (threadIdx.x < 64) {
      const int lane = threadIdx.x;
      const int nblk = int((uint32_t(a.nbins) + kWinBlock - 1) / kWinBlock);
      const int wblk = int(window / kWinBlock);
      const int ncand = nblk > wblk ? nblk - wblk + 1 : 1;
      uint32_t sum = 0u, all = 0u;
      if (lane < ncand)
        for (int i = lane; i < lane + wblk && i < nblk; ++i) sum += cnt[i];
      for (int i = lane; i < nblk; i += 64) all += cnt[i];
      // best candidate: most hits, then the lowest start
      uint32_t best = lane < ncand ? (sum << 8) | uint32_t(255 - lane) : 0u;
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) {
        const uint32_t o = __shfl_xor(best, off);
        best = o > best ? o : best;
        all += __shfl_xor(all, off);
      }
      if (lane == 0) {
        cnt[kMaxWinBlocks] = best;
        cnt[kMaxWinBlocks + 1] = all;
      }
    }
    __syncthreads();
    const uint32_t best = __builtin_amdgcn_readfirstlane(cnt[kMaxWinBlocks]);
    total = __builtin_amdgcn_readfirstlane(cnt[kMaxWinBlocks + 1]);
    hits = best >> 8;
    base = uint32_t(255 - (best & 0xFFu)) * kWinBlock;
    __syncthreads();
  }

  // Picks the workgroup's hot keys (HotKeys) from the first 4 x kBlock
  // updates of its chunk; on return every lane holds the same set, with
  // zeroed sums.  Needs the whole workgroup; ends with a barrier.
  static __device__ __forceinline__ void sample_hot(const tx_scatter_args &a, uint32_t lo, uint32_t nb, int64_t begin,
                                    int64_t end, bool vec, uint32_t *aux, HotKeys<OP> &hot) {
    uint32_t *skey = aux, *scnt = aux + kSampleSlots;
    for (int s = threadIdx.x; s < kSampleSlots; s += kBlock) {
      skey[s] = kEmpty;
      scnt[s] = 0u;
    }
    __syncthreads();
    {
      uint32_t key[4];
      T val[4];
      bool ok[4];
      load4(a, begin + 4 * int64_t(threadIdx.x), end, vec, key, val, ok);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t r = key[j] - lo;
        if (!(ok[j] && r < nb)) continue;
        const uint32_t h = (r * 2654435769u) >> (32 - kSampleLog2);
#pragma unroll
        for (int p = 0; p < kProbes; ++p) {
          const uint32_t slot = (h + p) & (kSampleSlots - 1);
          uint32_t k = __atomic_load_n(&skey[slot], __ATOMIC_RELAXED);
          if (k == kEmpty) k = atomicCAS(&skey[slot], kEmpty, r);
          if (k == kEmpty || k == r) {
            atomicAdd(&scnt[slot], 1u);
            break;
          }
        }
      }
    }
    __syncthreads();
    // Wavefront 0 takes the kHot largest counts (ties: lower slot first) and
    // then publishes them in the table's first slots: skey[0 .. kHot) holds
    // the keys, scnt[0] their number.
    if (threadIdx.x < 64) {
      uint32_t res[kHot];
      const int lane = threadIdx.x;
      auto best_of_lane = [&]() {
        uint64_t b = 0;
        for (int s = lane; s < kSampleSlots; s += 64) {
          const uint64_t c = (uint64_t(scnt[s]) << 32) | uint32_t(kSampleSlots - 1 - s);
          b = c > b ? c : b;
        }
        return b;
      };
      uint64_t mine = best_of_lane();
      int n = 0;
      for (int t = 0; t < kHot; ++t) {
        uint64_t b = mine;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
          const uint32_t lo32 = __shfl_xor(uint32_t(b), off), hi32 = __shfl_xor(uint32_t(b >> 32), off);
          const uint64_t o = (uint64_t(hi32) << 32) | lo32;
          b = o > b ? o : b;
        }
        if (uint32_t(b >> 32) < kHotMinCount) break;
        const int slot = kSampleSlots - 1 - int(uint32_t(b));
        res[t] = __builtin_amdgcn_readfirstlane(skey[slot]);
        if (slot % 64 == lane) {
          scnt[slot] = 0u;
          mine = best_of_lane();
        }
        n = t + 1;
      }
      if (lane == 0) {
#pragma unroll
        for (int t = 0; t < kHot; ++t)
          if (t < n) skey[t] = res[t];
        scnt[0] = uint32_t(n);
      }
    }
    __syncthreads();
    hot.n = int(__builtin_amdgcn_readfirstlane(scnt[0]));
#pragma unroll
    for (int t = 0; t < kHot; ++t) {
      // kept in vector registers: scalar registers are the scarcer resource
      // in the unrolled update loop
      hot.r[t] = t < hot.n ? skey[t] : kEmpty;
      hot.acc[t] = OpTraits<OP>::id();
    }
  }

  // One pass of a workgroup over its chunk with the LDS window [lo, lo + nb):
  // set the table to the identity, (fp32) pick the hot keys, stream the
  // chunk, then combine the hot keys' and the table's results into the bins
  // with one global atomic per touched slot.  With SPILL, in-range updates
  // outside the window go to the bins through the wavefront spill queues in
  // aux; without it they are left to the chunk's other passes.
  static __device__ __forceinline__ void pass(const tx_scatter_args &a, T *table, uint32_t *aux, uint32_t lo, uint32_t nb,
                              bool spill, int64_t begin, int64_t end, bool vec) {
    for (uint32_t s = threadIdx.x; s < nb; s += kBlock) table[s] = OpTraits<OP>::id();
    HotKeys<OP> hot;
    if constexpr (OP == FADD) sample_hot(a, lo, nb, begin, end, vec, aux, hot);
    __syncthreads();
    T *bins = reinterpret_cast<T *>(a.bins);
    uint32_t *q = aux + (threadIdx.x / 64) * 2 * kQueue;
    uint32_t qn = 0;
    SpillRegion sr;
    if (spill) sr.init(a);
    int64_t e = begin + 4 * int64_t(threadIdx.x);
    if (vec) {
      // Whole groups of kDepth full iterations go through the pipelined loop.
      const int64_t groups = (end - begin) / (kDepth * kIter);
      if (groups > 0) {
        const bool h = OP == FADD && hot.n > 0;
        if (spill) {
          if (h) {
            if (a.mask) stream<true, true, true>(a, table, lo, nb, q, qn, sr, hot, e, groups);
            else stream<false, true, true>(a, table, lo, nb, q, qn, sr, hot, e, groups);
          } else {
            if (a.mask) stream<true, false, true>(a, table, lo, nb, q, qn, sr, hot, e, groups);
            else stream<false, false, true>(a, table, lo, nb, q, qn, sr, hot, e, groups);
          }
        } else {
          if (h) {
            if (a.mask) stream<true, true, false>(a, table, lo, nb, q, qn, sr, hot, e, groups);
            else stream<false, true, false>(a, table, lo, nb, q, qn, sr, hot, e, groups);
          } else {
            if (a.mask) stream<true, false, false>(a, table, lo, nb, q, qn, sr, hot, e, groups);
            else stream<false, false, false>(a, table, lo, nb, q, qn, sr, hot, e, groups);
          }
        }
        e += groups * kDepth * kIter;
      }
    }
    // Remaining iterations: a uniform trip count (the combines need every
    // lane of the wavefront); lanes past `end` carry no update.
    const int64_t first = e - 4 * int64_t(threadIdx.x);
    for (int64_t eb = first; eb < end; eb += kIter) {
      uint32_t key[4];
      T val[4];
      bool ok[4];
      load4(a, eb + 4 * int64_t(threadIdx.x), end, vec, key, val, ok);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t r = key[j] - lo;  // wraps for keys below the window
        bool pend = ok[j] && r < nb;
        if (spill) spill_push<OP, T>(q, qn, bins, sr, ok[j] && !pend, key[j], val[j]);
        if constexpr (OP == FADD) {
          if (hot.n > 0) hot.take(pend, r, val[j]);
        }
        wave_lds_combine<OP, T>(table, pend, r, val[j]);
      }
    }
    if (spill) {
      spill_out<OP, T>(q, qn, bins, sr);
      sr.close();
    }
    // the hot keys' accumulators: one LDS combine per wavefront and key
#pragma unroll
    for (int t = 0; t < kHot; ++t) {
      if (t < hot.n) {
        T x = hot.acc[t];
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) x = combine<OP, T>(x, __shfl_xor(x, off));
        if ((threadIdx.x & 63) == 0) atomic_combine<OP, T>(&table[hot.r[t]], x);
      }
    }
    __syncthreads();
    for (uint32_t s = threadIdx.x; s < nb; s += kBlock) {
      const T v = table[s];
      if (!is_identity<OP, T>(v)) atomic_combine<OP, T>(bins + lo + s, v);
    }
    __syncthreads();  // the table and aux are reused by the next pass
  }

  // Windowed LDS privatisation, one workgroup per chunk of updates.  Up to
  // `window` bins the table holds them all and one pass does the chunk.
  // Beyond that the bin range is cut into `splits` windows of `window` bins
  // (each fits in LDS).  The chunk's first 4 x kBlock updates decide how:
  // when the best single window holds at least 3/4 of them (skewed keys) the
  // workgroup makes one pass with that window and spills the rest (one read
  // of the chunk); otherwise it makes one pass per window, each reading the
  // whole chunk.
  static __device__ __forceinline__ void windowed(const tx_scatter_args &a) {
    __shared__ T table[kDirectSlots];
    __shared__ uint32_t aux[kAuxWords];
    const int64_t begin = int64_t(blockIdx.x) * a.per_block;
    if (begin >= a.n) return;  // uniform: the whole workgroup leaves
    const int64_t end = begin + a.per_block < a.n ? begin + a.per_block : a.n;
    const bool vec = ((reinterpret_cast<uintptr_t>(a.idx) | reinterpret_cast<uintptr_t>(a.val)) & 15) == 0 &&
                     (!a.mask || (reinterpret_cast<uintptr_t>(a.mask) & 3) == 0);
    const uint32_t W = uint32_t(a.window), nbins = uint32_t(a.nbins);
    if (a.splits > 1) {
      uint32_t base, hits, total;
      pick_window(a, begin, end, vec, W, reinterpret_cast<uint32_t *>(table), base, hits, total);
      if (total > 0u && 4u * hits >= 3u * total) {
        pass(a, table, aux, base, min(W, nbins - base), true, begin, end, vec);
      } else {
        for (int w = 0; w < a.splits; ++w)
          pass(a, table, aux, uint32_t(w) * W, min(W, nbins - uint32_t(w) * W), false, begin, end, vec);
        SpillRegion sr;  // nothing spilled: every record of the regions unused
        sr.init(a);
        sr.close();
      }
      return;
    }
    pass(a, table, aux, 0u, min(W, nbins), false, begin, end, vec);
  }

  // Hash-table LDS cache with global spill.
  static __device__ void hashed(const tx_scatter_args &a) {
    __shared__ uint32_t keys[kHashSlots];
    __shared__ T vals[kHashSlots];
    for (int s = threadIdx.x; s < kHashSlots; s += kBlock) {
      keys[s] = kEmpty;
      vals[s] = OpTraits<OP>::id();
    }
    __syncthreads();
    T *bins = reinterpret_cast<T *>(a.bins);
    const int64_t begin = int64_t(blockIdx.x) * a.per_block;
    const int64_t end = begin + a.per_block < a.n ? begin + a.per_block : a.n;
    const bool vec = ((reinterpret_cast<uintptr_t>(a.idx) | reinterpret_cast<uintptr_t>(a.val)) & 15) == 0 &&
                     (!a.mask || (reinterpret_cast<uintptr_t>(a.mask) & 3) == 0);
    // Loop bound is uniform across the workgroup so that every lane takes part
    // in the wavefront-level combine of the spill path.
    const int64_t span = end > begin ? end - begin : 0;
    const int64_t iters = (span + 4 * kBlock - 1) / (4 * kBlock);
    for (int64_t it = 0; it < iters; ++it) {
      const int64_t e = begin + it * 4 * kBlock + 4 * int64_t(threadIdx.x);
      uint32_t key[4];
      T val[4];
      bool ok[4];
      load4(a, e, end, vec, key, val, ok);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        bool spill = false;
        if (ok[j]) {
          spill = true;
          const uint32_t h = (key[j] * 2654435769u) >> (32 - kHashLog2);
#pragma unroll
          for (int p = 0; p < kProbes; ++p) {
            const uint32_t slot = (h + p) & (kHashSlots - 1);
            uint32_t k = __atomic_load_n(&keys[slot], __ATOMIC_RELAXED);
            if (k == kEmpty) k = atomicCAS(&keys[slot], kEmpty, key[j]);
            if (k == kEmpty || k == key[j]) {
              atomic_combine<OP, T>(&vals[slot], val[j]);
              spill = false;
              break;
            }
          }
        }
        wave_combine_global<OP, T>(bins, spill, key[j], val[j]);
      }
    }
    __syncthreads();
    for (int s = threadIdx.x; s < kHashSlots; s += kBlock) {
      const uint32_t k = keys[s];
      const T v = vals[s];
      if (k != kEmpty && !is_identity<OP, T>(v)) atomic_combine<OP, T>(bins + k, v);
    }
  }

  // One returning atomic per update: old[i] is the bin's prior value.
  static __device__ void with_old(const tx_scatter_args &a) {
    T *bins = reinterpret_cast<T *>(a.bins);
    const T *vals = reinterpret_cast<const T *>(a.val);
    T *old = reinterpret_cast<T *>(a.old);
    for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < a.n; i += int64_t(gridDim.x) * 256) {
      const int32_t k = a.idx[i];
      T r = T(0);
      if (k >= 0 && k < a.nbins && (!a.mask || a.mask[i] != 0)) {
        T *p = bins + k;
        const T v = vals[i];
        if constexpr (OP == ADD || OP == FADD) r = atomicAdd(p, v);
        else if constexpr (OP == MAX || OP == UMAX) r = atomicMax(p, v);
        else if constexpr (OP == MIN || OP == UMIN) r = atomicMin(p, v);
        else if constexpr (OP == AND) r = atomicAnd(p, v);
        else if constexpr (OP == OR) r = atomicOr(p, v);
        else r = atomicXor(p, v);
      }
      old[i] = r;
    }
  }
};

}  // namespace

#define TX_SCATTER_KERNELS(NAME, OP)                                                   \
  TX_KERNEL void __launch_bounds__(kBlock) tx_scatter_##NAME##_windowed(const tx_scatter_args a) { \
    Scatter<OP>::windowed(a);                                                          \
  }                                                                                    \
  TX_KERNEL void __launch_bounds__(kBlock) tx_scatter_##NAME##_hashed(const tx_scatter_args a) { \
    Scatter<OP>::hashed(a);                                                            \
  }                                                                                    \
  TX_KERNEL void __launch_bounds__(256) tx_scatter_##NAME##_old(const tx_scatter_args a) { \
    Scatter<OP>::with_old(a);                                                          \
  }

TX_SCATTER_KERNELS(add, ADD)
TX_SCATTER_KERNELS(fadd, FADD)
TX_SCATTER_KERNELS(max, MAX)
TX_SCATTER_KERNELS(min, MIN)
TX_SCATTER_KERNELS(umax, UMAX)
TX_SCATTER_KERNELS(umin, UMIN)
TX_SCATTER_KERNELS(and, AND)
TX_SCATTER_KERNELS(or, OR)
TX_SCATTER_KERNELS(xor, XOR)

// tt.atomic_rmw xchg and tt.atomic_cas: one global atomic per update on the
// bin's 32-bit pattern (int32, uint32 and fp32 bins alike; CAS compares bit
// for bit).  The updates of one bin are applied one at a time in an order
// the hardware picks, so each update's old value is the bin's value after
// some set of that bin's earlier-applied updates.  Updates outside
// [0, nbins) or masked off return 0 and change nothing.
TX_KERNEL void __launch_bounds__(256) tx_scatter_xchg(const tx_scatter_args a) {
  uint32_t *bins = static_cast<uint32_t *>(a.bins);
  const uint32_t *vals = static_cast<const uint32_t *>(a.val);
  uint32_t *old = static_cast<uint32_t *>(a.old);
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < a.n; i += int64_t(gridDim.x) * 256) {
    const int32_t k = a.idx[i];
    uint32_t r = 0u;
    if (k >= 0 && k < a.nbins && (!a.mask || a.mask[i] != 0)) r = atomicExch(bins + k, vals[i]);
    if (old) old[i] = r;
  }
}

// 64-bit bins (int64 / uint64 / fp64 bit patterns): the same on 64-bit words.
TX_KERNEL void __launch_bounds__(256) tx_scatter_cas64(const tx_cas_args a) {
  unsigned long long *bins = static_cast<unsigned long long *>(a.bins);
  const unsigned long long *cmp = reinterpret_cast<const unsigned long long *>(a.cmp);
  const unsigned long long *val = reinterpret_cast<const unsigned long long *>(a.val);
  unsigned long long *old = reinterpret_cast<unsigned long long *>(a.old);
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < a.n; i += int64_t(gridDim.x) * 256) {
    const int32_t k = a.idx[i];
    unsigned long long r = 0ull;
    if (k >= 0 && k < a.nbins && (!a.mask || a.mask[i] != 0)) r = atomicCAS(bins + k, cmp[i], val[i]);
    if (old) old[i] = r;
  }
}

TX_KERNEL void __launch_bounds__(256) tx_scatter_cas(const tx_cas_args a) {
  uint32_t *bins = static_cast<uint32_t *>(a.bins);
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < a.n; i += int64_t(gridDim.x) * 256) {
    const int32_t k = a.idx[i];
    uint32_t r = 0u;
    if (k >= 0 && k < a.nbins && (!a.mask || a.mask[i] != 0)) r = atomicCAS(bins + k, a.cmp[i], a.val[i]);
    if (a.old) a.old[i] = r;
  }
}

// ---------------------------------------------------------------------------
// tt.atomic_rmw on 64-bit bins (int64 / uint64: add, max, min, umax, umin,
// and, or, xor, xchg; fp64: fadd, xchg) and 16-bit float bins (fp16 / bf16:
// fadd), the element types Triton's atomic_rmw accepts beside the 32-bit
// ones (the plugin passes every atomic_rmw through,
// uTLXConversionPatterns.cpp:611).
//
// When the bins fit one LDS table (64-bit: 18432 slots of 8 bytes; 16-bit
// fadd: 36864 fp32 slots), each workgroup combines its chunk of updates in
// the table with LDS atomics and then adds each touched slot to its bin
// with one global atomic (wide_table); otherwise every update is one global
// atomic (wide_direct), which also serves the returning-old and xchg forms.
// 16-bit fadd sums a workgroup's updates of one bin in fp32 and adds that
// partial to the bin with a compare-and-swap loop on the aligned 32-bit word
// that holds it (the other half is written back unchanged), rounding the
// bin to nearest even once per partial; wide_direct rounds once per update,
// as a per-element 16-bit atomic does.
namespace {

enum WideKind { W64I = 0, W64F = 1, WF16 = 2, WBF16 = 3 };
constexpr int kWideBlock = 1024;
constexpr int kWideSlots64 = 18432;   // 144 KiB of 8-byte slots
constexpr int kWideSlots16 = 36864;   // 144 KiB of fp32 partials

template <int KIND>
struct Wide;
template <>
struct Wide<W64I> {
  using Bin = unsigned long long;
  using Acc = unsigned long long;
  static constexpr int kSlots = kWideSlots64;
};
template <>
struct Wide<W64F> {
  using Bin = double;
  using Acc = double;
  static constexpr int kSlots = kWideSlots64;
};
template <>
struct Wide<WF16> {
  using Bin = uint16_t;
  using Acc = float;
  static constexpr int kSlots = kWideSlots16;
};
template <>
struct Wide<WBF16> {
  using Bin = uint16_t;
  using Acc = float;
  static constexpr int kSlots = kWideSlots16;
};

template <int KIND>
__device__ __forceinline__ float half_to_f32(uint32_t h) {
  if constexpr (KIND == WBF16) return txd::bf16_bits_to_f32(h);
  else return float(__builtin_bit_cast(_Float16, uint16_t(h)));
}

template <int KIND>
__device__ __forceinline__ uint32_t f32_to_half(float f) {
  if constexpr (KIND == WBF16) return txd::f32_to_bf16_bits(f);
  else return txd::pack_f16x2(f, 0.0f) & 0xFFFFu;
}

// The identity of each combine (fp adds start from -0, exact for IEEE add).
template <int KIND, int OP>
__device__ __forceinline__ typename Wide<KIND>::Acc wide_id() {
  if constexpr (KIND == W64I) {
    if constexpr (OP == MAX) return 0x8000000000000000ull;
    else if constexpr (OP == MIN) return 0x7FFFFFFFFFFFFFFFull;
    else if constexpr (OP == UMIN || OP == AND) return ~0ull;
    else return 0ull;
  } else {
    return typename Wide<KIND>::Acc(-0.0);
  }
}

template <int KIND, int OP>
__device__ __forceinline__ bool wide_is_id(typename Wide<KIND>::Acc v) {
  if constexpr (KIND == W64I) return v == wide_id<KIND, OP>();
  else if constexpr (KIND == W64F) return __builtin_bit_cast(uint64_t, v) == 0x8000000000000000ull;
  else return __builtin_bit_cast(uint32_t, v) == 0x80000000u;
}

// Combine v into *p (LDS or global, by the pointer's address space).
template <int KIND, int OP, typename P, typename V>
__device__ __forceinline__ void wide_atomic(P *p, V v) {
  if constexpr (KIND == W64I) {
    if constexpr (OP == ADD) atomicAdd(p, v);
    else if constexpr (OP == MAX) atomicMax(reinterpret_cast<long long *>(p), (long long)v);
    else if constexpr (OP == MIN) atomicMin(reinterpret_cast<long long *>(p), (long long)v);
    else if constexpr (OP == UMAX) atomicMax(p, v);
    else if constexpr (OP == UMIN) atomicMin(p, v);
    else if constexpr (OP == AND) atomicAnd(p, v);
    else if constexpr (OP == OR) atomicOr(p, v);
    else atomicXor(p, v);
  } else {
    atomicAdd(p, v);
  }
}

// bins16[s] = round(bins16[s] + x) through the aligned 32-bit word holding
// it; returns the bin's prior 16 bits.
template <int KIND>
__device__ __forceinline__ uint32_t half_add(uint16_t *bins16, int64_t s, float x) {
  uint16_t *h = bins16 + s;
  uint32_t *w = reinterpret_cast<uint32_t *>(reinterpret_cast<uintptr_t>(h) & ~uintptr_t(3));
  const int sh = (reinterpret_cast<uintptr_t>(h) & 2) ? 16 : 0;
  uint32_t old = __atomic_load_n(w, __ATOMIC_RELAXED), assumed;
  do {
    assumed = old;
    const uint32_t cur = (assumed >> sh) & 0xFFFFu;
    const uint32_t nh = f32_to_half<KIND>(half_to_f32<KIND>(cur) + x);
    old = atomicCAS(w, assumed, (assumed & ~(0xFFFFu << sh)) | (nh << sh));
  } while (old != assumed);
  return (assumed >> sh) & 0xFFFFu;
}

template <int KIND>
__device__ __forceinline__ typename Wide<KIND>::Acc wide_val(const void *val, int64_t i) {
  if constexpr (KIND == W64I) return static_cast<const unsigned long long *>(val)[i];
  else if constexpr (KIND == W64F) return static_cast<const double *>(val)[i];
  else return half_to_f32<KIND>(static_cast<const uint16_t *>(val)[i]);
}

__device__ __forceinline__ bool wide_live(const tx_scatter_args &a, int64_t i, int32_t k) {
  return k >= 0 && k < a.nbins && (!a.mask || a.mask[i] != 0);
}

// Chunk per workgroup, the bins in one LDS table.
template <int KIND, int OP>
__device__ __forceinline__ void wide_table(const tx_scatter_args &a) {
  using W = Wide<KIND>;
  using Acc = typename W::Acc;
  __shared__ Acc table[W::kSlots];
  const int64_t begin = int64_t(blockIdx.x) * a.per_block;
  if (begin >= a.n) return;  // uniform
  const int64_t end = min(begin + int64_t(a.per_block), a.n);
  for (int s = threadIdx.x; s < a.nbins; s += kWideBlock) table[s] = wide_id<KIND, OP>();
  __syncthreads();
  for (int64_t i = begin + threadIdx.x; i < end; i += kWideBlock) {
    const int32_t k = a.idx[i];
    if (wide_live(a, i, k)) {
      if constexpr (KIND == WF16 || KIND == WBF16) {
        wave_lds_combine<FADD, float>(table, true, uint32_t(k), wide_val<KIND>(a.val, i));
      } else {
        wide_atomic<KIND, OP>(&table[k], wide_val<KIND>(a.val, i));
      }
    }
  }
  __syncthreads();
  for (int s = threadIdx.x; s < a.nbins; s += kWideBlock) {
    const Acc v = table[s];
    if (wide_is_id<KIND, OP>(v)) continue;
    if constexpr (KIND == WF16 || KIND == WBF16) half_add<KIND>(static_cast<uint16_t *>(a.bins), s, v);
    else wide_atomic<KIND, OP>(static_cast<typename W::Bin *>(a.bins) + s, v);
  }
}

// One global atomic per update; OLD: each update's prior bin value to a.old
// (0 for updates out of range or masked off).  XCHG: the bin takes val.
template <int KIND, int OP, bool OLD, bool XCHG>
__device__ __forceinline__ void wide_direct(const tx_scatter_args &a) {
  using Bin = typename Wide<KIND>::Bin;
  Bin *bins = static_cast<Bin *>(a.bins);
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < a.n; i += int64_t(gridDim.x) * 256) {
    const int32_t k = a.idx[i];
    Bin r = Bin(0);
    if (wide_live(a, i, k)) {
      if constexpr (KIND == WF16 || KIND == WBF16) {
        r = Bin(half_add<KIND>(reinterpret_cast<uint16_t *>(bins), k, wide_val<KIND>(a.val, i)));
      } else if constexpr (XCHG) {
        const unsigned long long v = static_cast<const unsigned long long *>(a.val)[i];
        r = __builtin_bit_cast(Bin, atomicExch(reinterpret_cast<unsigned long long *>(bins + k), v));
      } else if constexpr (KIND == W64F) {
        r = atomicAdd(bins + k, wide_val<KIND>(a.val, i));
      } else {
        const unsigned long long v = wide_val<KIND>(a.val, i);
        unsigned long long *p = bins + k;
        if constexpr (OP == ADD) r = atomicAdd(p, v);
        else if constexpr (OP == MAX) r = (unsigned long long)atomicMax(reinterpret_cast<long long *>(p), (long long)v);
        else if constexpr (OP == MIN) r = (unsigned long long)atomicMin(reinterpret_cast<long long *>(p), (long long)v);
        else if constexpr (OP == UMAX) r = atomicMax(p, v);
        else if constexpr (OP == UMIN) r = atomicMin(p, v);
        else if constexpr (OP == AND) r = atomicAnd(p, v);
        else if constexpr (OP == OR) r = atomicOr(p, v);
        else r = atomicXor(p, v);
      }
    }
    if constexpr (OLD) static_cast<Bin *>(a.old)[i] = r;
  }
}

}  // namespace

// tx_scatter_<i64|f64|f16|bf16>_<op>_{table,direct,old}; xchg: _xchg (old optional).
#define TX_WIDE_KERNELS(TN, KIND, ON, OP)                                                                   \
  TX_KERNEL void __launch_bounds__(kWideBlock) tx_scatter_##TN##_##ON##_table(const tx_scatter_args a) {  \
    wide_table<KIND, OP>(a);                                                                                \
  }                                                                                                         \
  TX_KERNEL void __launch_bounds__(256) tx_scatter_##TN##_##ON##_direct(const tx_scatter_args a) {         \
    wide_direct<KIND, OP, false, false>(a);                                                                 \
  }                                                                                                         \
  TX_KERNEL void __launch_bounds__(256) tx_scatter_##TN##_##ON##_old(const tx_scatter_args a) {            \
    wide_direct<KIND, OP, true, false>(a);                                                                  \
  }
TX_WIDE_KERNELS(i64, W64I, add, ADD)
TX_WIDE_KERNELS(i64, W64I, max, MAX)
TX_WIDE_KERNELS(i64, W64I, min, MIN)
TX_WIDE_KERNELS(i64, W64I, umax, UMAX)
TX_WIDE_KERNELS(i64, W64I, umin, UMIN)
TX_WIDE_KERNELS(i64, W64I, and, AND)
TX_WIDE_KERNELS(i64, W64I, or, OR)
TX_WIDE_KERNELS(i64, W64I, xor, XOR)
TX_WIDE_KERNELS(f64, W64F, fadd, FADD)
TX_WIDE_KERNELS(f16, WF16, fadd, FADD)
TX_WIDE_KERNELS(bf16, WBF16, fadd, FADD)

TX_KERNEL void __launch_bounds__(256) tx_scatter_i64_xchg(const tx_scatter_args a) {
  if (a.old) wide_direct<W64I, ADD, true, true>(a);
  else wide_direct<W64I, ADD, false, true>(a);
}

// counts[0 .. n) = 0 before a histogram's scatter (a kernel rather than a
// memset, so that a captured graph holds no memset node).
TX_KERNEL void __launch_bounds__(256) tx_scatter_zero_bins(const tx_scatter_args a) {
  uint32_t *b = static_cast<uint32_t *>(a.bins);
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < a.n; i += int64_t(gridDim.x) * 256) b[i] = 0u;
}
