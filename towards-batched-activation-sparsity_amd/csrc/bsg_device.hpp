// bsg_device.hpp — device side of libbsgemm: buffer loads, MFMA element traits, the
// block-list staging and split-K hand-off pieces, and the three GEMM kernel templates.
// Each translation unit that instantiates a slice of the tile set includes it; the kernels
// live in an anonymous namespace (one private copy per unit), and the tile tables are the
// only symbols shared between units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

#include "bsgemm.h"

namespace bsgk {

struct GemmParams {
  const void* x;
  const void* wp;
  void* y;
  const int32_t* idx;
  const int32_t* na_dev;
  const uint8_t* bitmap;
  float* part;
  uint32_t* cnt;
  int64_t ldx;
  int64_t ldy;
  int32_t bt, K, N, npad, nblk, nbm, na, mode, split_k, n_tiles, x_bytes, y_fast;
  // MODE_TOPK: exact-L1 block scores (na = k), whether they fit the unique-key order, and where
  // work-group (0, 0) publishes the kept list and its count (null: not published)
  const uint64_t* scores;
  int32_t* idx_out;
  int32_t* na_out;
  int32_t keyed;
  // MODE_LIST: sort the list ascending while staging it (at most BSG_MAX_NBLK / 2 entries)
  int32_t sort_list;
  // 2-D sparsity: ascending active 64-column output blocks (null: every column), their count
  // (host value, or the device one when nn_dev is set), whether Y is compact (active blocks
  // side by side), and the width Y stores are bounded by (N, or nn * 64 when compact)
  const int32_t* nidx;
  const int32_t* nn_dev;
  int32_t nn, ncompact, ny;
  // Phase timeline of a profiling build (-DBSG_TIMELINE): 8 stamps per work-group, or null.  The
  // shipped build never reads it.
  uint64_t* tl;
};

typedef void (*GemmFn)(GemmParams);

enum { KIND_KSPLIT = 1, KIND_XLDS = 2, KIND_FMA = 3, KIND_XLDS_KH = 4, KIND_VT = 5, KIND_VT1 = 6, KIND_VT1X = 7 };

// 1-D and, for tiles of at most 64 columns per work-group, 2-D (active output blocks) entries.
// f16_sel: the fp16 1-D form compiled with the in-GEMM top-k (MODE_TOPK; on 16-row tiles also
// the self-scored MODE_TOPK_SELF), for the MFMA kinds (null for kind 3).  The other forms leave
// that code out: carried in every kernel it cost every plain launch 0.1-0.2 us.
struct KernelEntry {
  int kind, rows, nsub, wpg, depth;
  GemmFn f16, bf16, f16_2d, bf16_2d, f16_sel;
};

// A translation unit's slice of the instantiated tile set.
struct TileTable {
  const KernelEntry* e;
  int n;
};

extern const TileTable kTilesK1R16, kTilesK1R32, kTilesK1R64, kTilesK2, kTilesK4, kTilesK3, kTilesK5, kTilesK7;

}  // namespace bsgk

namespace {

using namespace bsgk;

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr int kOOB = (int)0x80000000u;  // buffer offset beyond any num_records we build
constexpr int kRsrcWord3 = 0x00020000;  // gfx9 raw buffer: 32-bit data format, no swizzle

// Phase timeline (a separate profiling build of the library, compiled with -DBSG_TIMELINE; in
// the shipped build these expand to nothing).  Wave 0 of each work-group keeps the 100 MHz wall
// clock at its phase boundaries in registers and writes them once at the end to
// p.tl[group * 8 + slot]: 0 entry, 1 block list staged, 2 first block's weights consumed,
// 3 main loop done, 4 outputs or partials issued, 5 end (own stores acknowledged),
// 6 = bit 0: this work-group stored Y (the last arriver under split-K); bits 1..: the latest
// main-loop end over the work-group's waves (every wave posts its own to LDS), 7 = XCC id << 32 |
// HW_ID.
#ifdef BSG_TIMELINE
#define BSG_TL_DECL                                        \
  uint64_t bsg_ts_[6] = {0, 0, 0, 0, 0, 0};                \
  __shared__ unsigned long long bsg_tl_last_;              \
  if (threadIdx.x == 0) bsg_tl_last_ = 0;
#define BSG_TL(i) (bsg_ts_[i] = wall_clock64())
#define BSG_TL_IF(i, cond) \
  if (cond) bsg_ts_[i] = wall_clock64()
#define BSG_TL_LOOP_END()                                                   \
  do {                                                                      \
    bsg_ts_[3] = wall_clock64();                                            \
    if ((threadIdx.x & 63) == 0) atomicMax(&bsg_tl_last_, (unsigned long long)bsg_ts_[3]); \
  } while (0)
#define BSG_TL_END(p, stored_y)                                                                         \
  do {                                                                                                 \
    __builtin_amdgcn_s_waitcnt(0x0F70);                                                                \
    bsg_ts_[5] = wall_clock64();                                                                       \
    __syncthreads();                                                                                   \
    if ((p).tl != nullptr && threadIdx.x == 0) {                                                       \
      uint64_t* t_ = (p).tl + ((size_t)blockIdx.y * gridDim.x + blockIdx.x) * 8;                      \
      for (int i_ = 0; i_ < 6; ++i_) t_[i_] = bsg_ts_[i_];                                             \
      t_[6] = ((stored_y) ? 1u : 0u) | ((uint64_t)bsg_tl_last_ << 1);                                  \
      t_[7] = ((uint64_t)__builtin_amdgcn_s_getreg((31 << 11) | 20) << 32) |                          \
              (uint64_t)__builtin_amdgcn_s_getreg((31 << 11) | 4);                                     \
    }                                                                                                  \
  } while (0)
#else
#define BSG_TL_DECL
#define BSG_TL(i) ((void)0)
#define BSG_TL_IF(i, cond) ((void)0)
#define BSG_TL_LOOP_END() ((void)0)
#define BSG_TL_END(p, stored_y) ((void)0)
#endif

// MODE_TOPK: the GEMM ranks block scores an earlier launch wrote.  MODE_TOPK_SELF: every
// work-group also computes those scores itself from x (fp16, at most BSG_SELF_MAX_ROWS rows).
enum { MODE_LIST = 0, MODE_BITMAP = 1, MODE_DENSE = 2, MODE_TOPK = 3, MODE_TOPK_SELF = 4 };
// A GEMM ranks block scores itself (MODE_TOPK) up to this many blocks: keys and ranks fit its
// block-list buffer, and a one-wave work-group flags at most 8 per thread.
#define BSG_TOPK_MAX_NBLK 512
#define BSG_SELF_MAX_ROWS 8

// Kind 3 activation staging: 1 KiB loads per wave, and the LDS it may take.
#define BSG_FMA_X_LOADS 16
#define BSG_FMA_LDS_MAX (96 * 1024)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int num_bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, num_bytes, kRsrcWord3);
}

__device__ __forceinline__ u32x4 ld16(__amdgpu_buffer_rsrc_t r, int voff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0);
}

#ifndef BSG_W_AUX
#define BSG_W_AUX 2  // weight stream: non-temporal (read once, keep X resident in L1/L2)
#endif

__device__ __forceinline__ u32x4 ld16_stream(__amdgpu_buffer_rsrc_t r, int voff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, BSG_W_AUX);
}

// fn(std::integral_constant<int, i>) for i = 0 .. N-1, in order.
template <typename Fn, int... I>
__device__ __forceinline__ void static_for_seq(Fn&& fn, std::integer_sequence<int, I...>) {
  (fn(std::integral_constant<int, I>{}), ...);
}
template <int N, typename Fn>
__device__ __forceinline__ void static_for(Fn&& fn) {
  static_for_seq(fn, std::make_integer_sequence<int, N>{});
}

// 16 bytes per lane straight into LDS: lane i's bytes land at lds + 16 i (an out-of-range offset
// writes zeros).  No register receives them, and the compiler's wait insertion does not order
// later LDS reads after such a load, so its users wait by count (vmem_wait).
__device__ __forceinline__ void ld16_lds(__amdgpu_buffer_rsrc_t r, void* lds, int voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, 0, 0, 0);
}

// Wait until at most N vector-memory loads of this wave are outstanding (s_waitcnt vmcnt, gfx9
// encoding; the expcnt and lgkmcnt fields at their maxima), fenced so that no instruction moves
// across it.  Loads complete in issue order, so every load issued N or more loads before is done.
template <int N>
__device__ __forceinline__ void vmem_wait() {
  constexpr int n = N < 63 ? N : 63;
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt((n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8));
  __builtin_amdgcn_sched_barrier(0);
}

template <typename T>
struct Elem;

template <>
struct Elem<_Float16> {
  static __device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint16_t bits(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
  }
  // a.lo*b.lo + a.hi*b.hi + c: fp16 products are exact in fp32, one fp32 rounding per add.
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c, false);
  }
};

template <>
struct Elem<__bf16> {
  static __device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint16_t bits(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);
  }
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
  }
};

// Exclusive prefix sum over the work-group; also returns the total.  `scratch` holds
// one int per wave.  Contains two barriers.
template <int NT>
__device__ __forceinline__ int wg_exclusive_scan(int v, int* scratch, int* total) {
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  int incl = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    int o = __shfl_up(incl, d, 64);
    if (lane >= d) incl += o;
  }
  if (lane == 63) scratch[w] = incl;
  __syncthreads();
  int base = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < NT / 64; ++i) {
    int s = scratch[i];
    if (i < w) base += s;
    tot += s;
  }
  __syncthreads();
  *total = tot;
  return base + incl - v;
}


// Rank of block j among nb scores in LDS, ordered (score desc, block id asc): the number of
// blocks ahead of it.  s_sc holds the nb scores followed by zeros up to a multiple of 16 (a pad
// is never ahead: its score is the lowest and its id >= nb).  The scores are read as LDS
// broadcasts into two 8-score buffers, each refilled while the other is compared, so the loop
// runs at the compare rate rather than the LDS round trip.  UNIQUE: the scores are distinct keys
// that already encode the id order, so one compare does.  Rolled on purpose: a work-group runs
// it once, so unrolled copies cost more in cold instruction fetch than they save.
template <bool UNIQUE, typename S>
__device__ __forceinline__ int rank_of(const S* s_sc, int nb, int j, S sj) {
  const int nb16 = (nb + 15) & ~15;
  int rank = 0;
  S a[8], b[8];
  auto count = [&](const S (&v)[8], int i0) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if constexpr (UNIQUE)
        rank += v[u] > sj;
      else
        rank += (v[u] > sj) | ((v[u] == sj) & (i0 + u < j));
    }
  };
#pragma unroll
  for (int u = 0; u < 8; ++u) a[u] = s_sc[u];
#pragma unroll 1
  for (int i0 = 0; i0 < nb16; i0 += 16) {
#pragma unroll
    for (int u = 0; u < 8; ++u) b[u] = s_sc[i0 + 8 + u];
    __builtin_amdgcn_sched_barrier(0);
    count(a, i0);
    const int in = i0 + 16 < nb16 ? i0 + 16 : 0;  // the last refill is a harmless re-read
#pragma unroll
    for (int u = 0; u < 8; ++u) a[u] = s_sc[in + u];
    __builtin_amdgcn_sched_barrier(0);
    count(b, i0 + 8);
  }
  return rank;
}

// Zero the pad of a score array after its nb entries, up to a multiple of 16 (rank_of).
template <typename S>
__device__ __forceinline__ void pad_scores(S* s_sc, int nb) {
  const int tid = threadIdx.x;
  if (tid < ((nb + 15) & ~15) - nb) s_sc[nb + tid] = S(0);
}

// Top-k of nb exact-L1 block scores (global memory, written by an earlier kernel on the
// stream): ranked (score desc, id asc), the first k kept, their ids handed to emit(position,
// id) in ascending id order.  keyed: every score is below 2^53, so (score << 11) | (2047 - id)
// is a unique key in the same order and one compare decides.  The nb^2 compares are spread over
// every wave of the work-group: a work item is (64 blocks, 16 scores), each lane counts the
// scores ahead of its block and adds the count to the block's rank in LDS.  s_key holds nb
// keys rounded up to 16, s_rank nb ints; per-wave ballots of the kept flags then give ascending
// positions.  Returns min(k, nb).  No thread reads s_key after the ranking barrier, so emit may
// overwrite s_key (not s_rank, which waves still read while others emit).
template <int NT, typename Emit>
__device__ __forceinline__ int topk_l1_list(const uint64_t* scores, int nb, int k, bool keyed, uint64_t* s_key,
                                            int* s_rank, Emit emit, bool staged = false) {
  constexpr int W = NT / 64;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nb16 = (nb + 15) & ~15;
  // staged: s_key already holds the keys and pads (self_score_keys)
  for (int i = tid; !staged && i < nb16; i += NT) {
    uint64_t key = 0;  // pads: lowest score, ids >= nb, never ahead
    if (i < nb) {
      const uint64_t v = scores[i];
      key = keyed ? (v << 11) | (uint64_t)(BSG_MAX_NBLK - 1 - i) : v;
    }
    s_key[i] = key;
  }
  for (int i = tid; i < nb; i += NT) s_rank[i] = 0;
  __syncthreads();
  const int C = nb16 / 16;
  const int items = ((nb + 63) / 64) * C;
#pragma unroll 1
  for (int it = w; it < items; it += W) {
    const int g = it / C;
    const int i0 = 16 * (it - g * C);
    const int j = 64 * g + lane;
    const uint64_t kj = j < nb ? s_key[j] : 0;
    uint64_t ki[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) ki[u] = s_key[i0 + u];
    int r = 0;
    if (keyed) {
#pragma unroll
      for (int u = 0; u < 16; ++u) r += ki[u] > kj;
    } else {
#pragma unroll
      for (int u = 0; u < 16; ++u) r += (ki[u] > kj) | ((ki[u] == kj) & (i0 + u < j));
    }
    if (j < nb && r != 0) atomicAdd(&s_rank[j], r);
  }
  __syncthreads();
  // Ascending positions of the kept blocks (rank < kk) without a scan: every wave ballots the
  // kept flags of each 64-block group in turn and keeps the running count, so the position of
  // block j is the kept count before its group plus the kept lanes below it; wave g % W emits
  // group g.  No barrier, and the only LDS reads are of s_rank.
  const int kk = k < nb ? k : nb;
  int before = 0;
#pragma unroll 1
  for (int g = 0; 64 * g < nb; ++g) {
    const int j = 64 * g + lane;
    const bool keep = j < nb && s_rank[j] < kk;
    const uint64_t m = __ballot(keep);
    if (g % W == w && keep) emit(before + __popcll(m & ((1ull << lane) - 1ull)), j);
    before += __popcll(m);
  }
  return kk;
}


// Split-K hand-off primitives.  Partials move with agent-scope relaxed atomics, which are
// device-coherent without touching the rest of L2 (an agent-scope fence would write back and
// invalidate the whole L2 of the XCD on every work-group).

__device__ __forceinline__ void part_store(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Components of one fragment lane sit 64 floats apart (see the partial layout).
__device__ __forceinline__ f32x4 part_load(const float* q) {
  f32x4 v;
  v.x = __hip_atomic_load(q + 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  v.y = __hip_atomic_load(q + 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  v.z = __hip_atomic_load(q + 128, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  v.w = __hip_atomic_load(q + 192, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return v;
}

// Every store of this wave has completed (at the scope it was issued with).
__device__ __forceinline__ void part_publish() {
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0), expcnt(7), lgkmcnt(15)
}

__device__ __forceinline__ unsigned counter_add(uint32_t* c) {
  return __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void counter_reset(uint32_t* c) {
  __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}


// ---------------------------------------------------------------------------------------
// Pieces shared by both GEMM kernel kinds.

// Work-group -> (column tile, split) with an XCD-aware order: hardware places work-group b
// on XCD b % 8, so consecutive logical ids (the split partners of a tile) share an XCD.
__device__ __forceinline__ void tile_of_group(int split_k, int* tile, int* sk) {
  const int nwg = gridDim.x;
  const int bid = blockIdx.x;
  const int lid = (nwg & 7) == 0 ? (bid & 7) * (nwg >> 3) + (bid >> 3) : bid;
  *tile = lid / split_k;
  *sk = lid - *tile * split_k;
}

// Columns of column tile `tile` (gc columns wide): n0 = first weight column it reads, n0y =
// first output column it writes.  N2D (2-D sparsity, a separate instantiation so the 1-D
// kernels carry none of it): tile t is piece t % (64/gc) of active 64-column block
// nidx[t / (64/gc)]; compact output packs the active blocks side by side.  Returns false when
// the tile has no block (past the device-side count): the whole work-group then returns
// before any barrier.  A block id outside [0, ceil(N/64)) reads past the packed columns (zero
// weights) and writes nothing.
template <bool N2D>
__device__ __forceinline__ bool tile_columns(const GemmParams& p, int tile, int gc, int* n0, int* n0y) {
  if constexpr (!N2D) {
    *n0 = *n0y = tile * gc;
    return true;
  }
  const int per = 64 / gc;
  const int bi = tile / per;
  int nn = p.nn;
  if (p.nn_dev != nullptr) {
    const int d = __builtin_amdgcn_readfirstlane(*p.nn_dev);
    nn = d < 0 ? 0 : (d < nn ? d : nn);
  }
  if (bi >= nn) return false;
  const int off = (tile - bi * per) * gc;
  const int nb = __builtin_amdgcn_readfirstlane(p.nidx[bi]);
  const bool ok = nb >= 0 && nb < (p.N + 63) / 64;
  *n0 = ok ? nb * 64 + off : p.npad;
  *n0y = p.ncompact ? bi * 64 + off : (ok ? *n0 : p.ny);
  return true;
}

// |x| of an fp16 value in units of 2^-24 (exact for every finite value; Inf/NaN map above
// every finite value, NaN above Inf).
__device__ __forceinline__ uint64_t f16_units(uint32_t hbits) {
  const uint32_t b = hbits & 0x7fffu;
  const uint32_t e = b >> 10, m = b & 0x3ffu;
  return e == 0 ? (uint64_t)m : ((uint64_t)(1024u | m) << (e - 1));
}

__device__ __forceinline__ uint64_t f16x8_units(u32x4 v) {
  return f16_units(v.x & 0xffffu) + f16_units(v.x >> 16) + f16_units(v.y & 0xffffu) + f16_units(v.y >> 16) +
         f16_units(v.z & 0xffffu) + f16_units(v.z >> 16) + f16_units(v.w & 0xffffu) + f16_units(v.w >> 16);
}

// sum |x| of 8 fp16 values as an fp64 value, exactly: every finite |x| is a multiple of 2^-24
// below 2^16, so every partial sum of up to 512 of them needs at most 50 significant bits and
// fp64 adds are exact.  A group holding Inf or NaN takes the integer units of f16x8_units (their
// mapping above every finite value), scaled by 2^-24 (exact), so either way the result times
// 2^24 is the integer sum of the units.
__device__ __forceinline__ double f16x8_abs_sum(u32x4 v) {
  auto nonfinite = [](uint32_t d) {  // a 16-bit half of d with exponent 31
    const uint32_t t = (d & 0x7c007c00u) ^ 0x7c007c00u;
    return ((t - 0x00010001u) & ~t & 0x80008000u) != 0u;
  };
  if (nonfinite(v.x) | nonfinite(v.y) | nonfinite(v.z) | nonfinite(v.w))
    return (double)f16x8_units(v) * 0x1p-24;
  auto h = [](uint32_t d, int hi) {
    return fabs((double)(float)__builtin_bit_cast(_Float16, (uint16_t)(hi ? d >> 16 : d & 0xffffu)));
  };
  return ((h(v.x, 0) + h(v.x, 1)) + (h(v.y, 0) + h(v.y, 1))) + ((h(v.z, 0) + h(v.z, 1)) + (h(v.w, 0) + h(v.w, 1)));
}

// One DPP row shift (row_shr:n = 0x110 + n) of a 64-bit value: lane i of each 16-lane row
// reads lane i - n of the same row, and 0 where that lane lies outside the row.
template <int CTRL>
__device__ __forceinline__ uint64_t u64_row_shr(uint64_t x) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)x, CTRL, 0xf, 0xf, true);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(x >> 32), CTRL, 0xf, 0xf, true);
  return ((uint64_t)hi << 32) | lo;
}

// The 64-bit value of lane `src` of the wave.
__device__ __forceinline__ uint64_t u64_lane(uint64_t x, int src) {
  const uint32_t lo = (uint32_t)__shfl((int)(uint32_t)x, src, 64);
  const uint32_t hi = (uint32_t)__shfl((int)(uint32_t)(x >> 32), src, 64);
  return ((uint64_t)hi << 32) | lo;
}

// MODE_TOPK_SELF: the exact-L1 score of every K-block of x[0, bt) (bt <= BSG_SELF_MAX_ROWS, fp16)
// computed by this work-group alone -- the integers bsg_score_l1_kernel writes: block j sums
// |x| over the rows and its channels in units of 2^-24 -- as top-k keys in s_key[0, nb16) (keyed
// order as topk_l1_list builds it, pads 0).  A segment of SEG = 8 x (rows rounded up to a power
// of two) consecutive lanes covers one block (lane s of the segment: row s / 8, channels
// 8 (s % 8) .. +7), so a pass of the work-group covers NT / SEG blocks.  The loads of up to U
// passes are in flight before any is summed; passes past the last block are skipped (a
// work-group-uniform test).  Segment sums: DPP row shifts give the sum of the 8 or 16 lanes up
// to each lane of a 16-lane row, and for 32- and 64-lane segments the last lane adds the other
// rows' totals.  x is read from L2 (every work-group of the launch reads the same bytes).
// Ends with a barrier.
template <int NT>
__device__ __forceinline__ void self_score_keys(const GemmParams& p, uint64_t* s_key) {
  constexpr int U = 8;
  const int tid = threadIdx.x, lane = tid & 63;
  const int rp2 = p.bt <= 1 ? 1 : p.bt <= 2 ? 2 : p.bt <= 4 ? 4 : 8;
  const int seg = 8 * rp2;  // 8, 16, 32 or 64 lanes
  const int per_pass = NT / seg;
  const int s = tid % seg, row = s >> 3, grp = s & 7;
  const int nb = p.nblk, nb16 = (nb + 15) & ~15;
  const uint16_t* x = (const uint16_t*)p.x;
  for (int j0 = 0; j0 < nb; j0 += U * per_pass) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = j0 + u * per_pass + tid / seg;
      const int col = 64 * j + 8 * grp;
      v[u] = u32x4{0u, 0u, 0u, 0u};
      if (row < p.bt && j < nb && col < p.K) v[u] = *(const u32x4*)(x + (size_t)row * (size_t)p.ldx + col);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (j0 + u * per_pass >= nb) break;  // uniform: no block in this pass or the next
      // exact fp64 sums (f16x8_abs_sum); the DPP steps move their bit patterns
      auto shr = [](double a, auto ctrl) {
        return a + __builtin_bit_cast(double, u64_row_shr<decltype(ctrl)::value>(__builtin_bit_cast(uint64_t, a)));
      };
      double a = f16x8_abs_sum(v[u]);
      a = shr(a, std::integral_constant<int, 0x111>{});
      a = shr(a, std::integral_constant<int, 0x112>{});
      a = shr(a, std::integral_constant<int, 0x114>{});
      if (seg >= 16) a = shr(a, std::integral_constant<int, 0x118>{});  // lane 15 of a row: its total
      if (seg >= 32) {
        const double r1 = __builtin_bit_cast(  // the previous row's total
            double, u64_lane(__builtin_bit_cast(uint64_t, a), ((lane | 15) - 16) & 63));
        if (lane & 16) a += r1;  // lanes 31, 63: their halves
      }
      if (seg == 64) {
        const double h = __builtin_bit_cast(double, u64_lane(__builtin_bit_cast(uint64_t, a), 31));
        if (lane == 63) a += h;
      }
      const int j = j0 + u * per_pass + tid / seg;
      if (s == seg - 1 && j < nb) {
        const uint64_t units = (uint64_t)(a * 0x1p24);  // an integer below 2^50: exact
        s_key[j] = p.keyed ? (units << 11) | (uint64_t)(BSG_MAX_NBLK - 1 - j) : units;
      }
    }
  }
  if (tid < nb16 - nb) s_key[nb + tid] = 0;  // pads: lowest score, never ahead
  __syncthreads();
}

// The first na block ids in ascending order, into s_ids[0, na) (na <= BSG_MAX_NBLK / 2): the
// sequence an ascending sort of the list gives (equal ids are equal, so their order does not
// show).  The ids go to LDS as unsigned keys 0x7fffffff - id (descending in the id).  A list that
// is already ascending is copied back; any other is ranked, each id's rank being the number of
// entries before it in (id asc, list position asc) order, written to
// s_ids[BSG_MAX_NBLK / 2 + rank] and copied back.  The rank loop reads the keys as LDS
// broadcasts and keeps no array, so the kernels' register allocation is not disturbed.  Leaves
// the copy-back unfenced; the caller's barrier follows.
template <int NT>
__device__ __forceinline__ void sort_block_list(const int32_t* ids, int na, int* s_ids) {
  const int tid = threadIdx.x;
  uint32_t* const s_key = (uint32_t*)s_ids;
  for (int i = tid; i < na; i += NT) s_key[i] = (uint32_t)(0x7fffffffLL - (long long)ids[i]);
  __syncthreads();
  int unsorted = 0;
  for (int i = tid; i + 1 < na; i += NT) unsorted |= s_key[i] < s_key[i + 1];
  if (__syncthreads_or(unsorted)) {
    int* const s_out = s_ids + BSG_MAX_NBLK / 2;
    for (int i = tid; i < na; i += NT) {
      const uint32_t ki = s_key[i];
      int r = 0;
#pragma unroll 8
      for (int j = 0; j < na; ++j) {
        const uint32_t kj = s_key[j];
        r += (kj > ki) | ((kj == ki) & (j < i));
      }
      s_out[r] = (int)(0x7fffffffLL - (long long)ki);
    }
    __syncthreads();
    for (int i = tid; i < na; i += NT) s_ids[i] = s_out[i];
  } else {
    // each thread rewrites only the entries it read
    for (int i = tid; i < na; i += NT) s_ids[i] = (int)(0x7fffffffLL - (long long)s_key[i]);
  }
}

// Stage this call's active-block list in LDS (list copy, bitmap compaction, top-k of block
// scores or identity) and return its length.  Ends with a barrier.  s_ids is 16-byte aligned
// and holds BSG_MAX_NBLK ids; the top-k stages its keys in the first half and its ranks in the
// second (up to 512 blocks).  ONE_D: the in-kernel sort of a 1-D list (p.sort_list) is compiled
// in (the 2-D forms have none).  SEL: the in-GEMM top-k (MODE_TOPK) is, and SELF_SCORE its
// self-scored form (MODE_TOPK_SELF): the selection instantiations only (KernelEntry::f16_sel),
// which alone are launched in those modes.
template <int NT, bool ONE_D, bool SEL = false, bool SELF_SCORE = false>
__device__ __forceinline__ int stage_block_list(const GemmParams& p, int* s_ids, int* s_scan) {
  const int tid = threadIdx.x;
  int na = 0;
  bool ranked = false;
  if constexpr (SEL) {
    if (p.mode == MODE_TOPK || (SELF_SCORE && p.mode == MODE_TOPK_SELF)) {
      // Every work-group ranks the scores itself (identically), so the list needs no other
      // launch; keys and ranks are staged in the list buffer and overwritten by the kept ids.
      // MODE_TOPK_SELF computes the scores here too, so the selection needs no launch of its own.
      const bool self = SELF_SCORE && p.mode == MODE_TOPK_SELF;
      if (self) self_score_keys<NT>(p, (uint64_t*)s_ids);
      na = topk_l1_list<NT>(p.scores, p.nblk, p.na, p.keyed != 0, (uint64_t*)s_ids, s_ids + BSG_MAX_NBLK / 2,
                            [&](int pos, int id) { s_ids[pos] = id; }, self);
      ranked = true;
    }
  }
  if (ranked) {
    // the kept list is staged
  } else if (p.mode == MODE_LIST) {
    na = p.na;
    if (p.na_dev != nullptr) {
      const int d = *p.na_dev;
      na = d < 0 ? 0 : (d < na ? d : na);
    }
    if (ONE_D && p.sort_list)
      sort_block_list<NT>(p.idx, __builtin_amdgcn_readfirstlane(na), s_ids);
    else
      for (int i = tid; i < na; i += NT) s_ids[i] = p.idx[i];
  } else if (p.mode == MODE_BITMAP) {
    const int per = (p.nbm + NT - 1) / NT;
    const int beg = tid * per < p.nbm ? tid * per : p.nbm;
    const int end = beg + per < p.nbm ? beg + per : p.nbm;
    int c = 0;
    for (int i = beg; i < end; ++i) c += p.bitmap[i] != 0;
    int total = 0;
    int o = wg_exclusive_scan<NT>(c, s_scan, &total);
    for (int i = beg; i < end; ++i)
      if (p.bitmap[i] != 0) s_ids[o++] = i;
    na = total;
  } else {
    na = p.nblk;
    for (int i = tid; i < na; i += NT) s_ids[i] = i;
  }
  na = __builtin_amdgcn_readfirstlane(na);
  __syncthreads();
  if (SEL && ranked && p.idx_out != nullptr && blockIdx.x == 0 && blockIdx.y == 0) {
    for (int i = tid; i < na; i += NT) p.idx_out[i] = s_ids[i];
    if (tid == 0) *p.na_out = na;
  }
  return na;
}

// Output fragment g = bi * CS + cs of a work-group whose columns start at n0 (CS 16-column
// subtiles): lane holds Y[y0 + 16 bi + lane%16][n0 + 16 cs + 4 (lane/16) + r], r = 0..3.
template <typename T, int CS>
__device__ __forceinline__ void store_y(const GemmParams& p, int y0, int n0, int g, f32x4 v) {
  const int lane = threadIdx.x & 63;
  const int bi = g / CS;
  const int cs = g - bi * CS;
  const int b = y0 + 16 * bi + (lane & 15);
  const int n = n0 + 16 * cs + 4 * (lane >> 4);
  if (b >= p.bt) return;
  uint16_t* yrow = (uint16_t*)p.y + (size_t)b * (size_t)p.ldy;
  if (p.y_fast) {
    if (n < p.ny) {
      u32x2 pk;
      pk.x = (uint32_t)Elem<T>::bits(v.x) | ((uint32_t)Elem<T>::bits(v.y) << 16);
      pk.y = (uint32_t)Elem<T>::bits(v.z) | ((uint32_t)Elem<T>::bits(v.w) << 16);
      *(u32x2*)(yrow + n) = pk;
    }
  } else {
    if (n + 0 < p.ny) yrow[n + 0] = Elem<T>::bits(v.x);
    if (n + 1 < p.ny) yrow[n + 1] = Elem<T>::bits(v.y);
    if (n + 2 < p.ny) yrow[n + 2] = Elem<T>::bits(v.z);
    if (n + 3 < p.ny) yrow[n + 3] = Elem<T>::bits(v.w);
  }
}

// Partials: [tile][split][fragment][component][lane] floats, so every dword store or load
// instruction of a wave covers 256 contiguous bytes.
template <int FT>
__device__ __forceinline__ void part_emit(const GemmParams& p, size_t tile_lin, int sk, int g, f32x4 v) {
  float* dst = (float*)p.part + ((tile_lin * p.split_k + sk) * FT + g) * 256 + (threadIdx.x & 63);
  part_store(dst + 0, v.x);
  part_store(dst + 64, v.y);
  part_store(dst + 128, v.z);
  part_store(dst + 192, v.w);
}

// Split-K hand-off: publish this work-group's partials, count arrivals; in the last work-group
// of the tile each wave that holds accumulators (every wave of kind 2, the first channel half
// of kind 4, wave 0 of kind 1 after its in-group reduction) reduces its own fragments in split
// order, taking this work-group's split from registers and loading only the other S - 1 (up to
// 16 fragment loads in flight per round trip), stores Y and re-arms the counter for the next
// launch (graph-replay safe).  Partials move through agent-scope (device-coherent) stores and
// loads, so no L2 write-back/invalidate is needed: each wave waits for its own stores, the
// barrier orders them before the counter update, and the last work-group loads only after it
// has seen the final count.  wc = the wave's column group, CS = 16-column subtiles per tile,
// FT = fragments per tile.
template <typename T, int BTT, int NSUB, int CS, int FT>
__device__ __forceinline__ void splitk_finish(const GemmParams& p, size_t tile_lin, int y0, int n0, int sk,
                                              int wc, bool holds, const f32x4 (&acc)[BTT][NSUB], int* s_flag) {
  const int S = p.split_k;
  const int lane = threadIdx.x & 63;
  part_publish();
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned prev = counter_add(&p.cnt[tile_lin]);
    *s_flag = prev == (unsigned)(S - 1);
  }
  __syncthreads();
  if (!*s_flag) return;
  if (holds) {
    constexpr int F = BTT * NSUB;
    constexpr int QB = F >= 16 ? 1 : 16 / F;  // splits per round trip
    const float* base = (const float*)p.part + (tile_lin * S) * FT * 256 + lane;
    f32x4 sum[BTT][NSUB];
#pragma unroll
    for (int bi = 0; bi < BTT; ++bi)
#pragma unroll
      for (int s = 0; s < NSUB; ++s) sum[bi][s] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int q0 = 0; q0 < S; q0 += QB) {
      f32x4 t[QB][BTT][NSUB];
#pragma unroll
      for (int qq = 0; qq < QB; ++qq) {
        const int q = q0 + qq;
        if (q < S && q != sk) {
#pragma unroll
          for (int bi = 0; bi < BTT; ++bi)
#pragma unroll
            for (int s = 0; s < NSUB; ++s)
              t[qq][bi][s] = part_load(base + ((size_t)q * FT + bi * CS + wc * NSUB + s) * 256);
        }
      }
#pragma unroll
      for (int qq = 0; qq < QB; ++qq) {
        const int q = q0 + qq;
        if (q < S) {
#pragma unroll
          for (int bi = 0; bi < BTT; ++bi)
#pragma unroll
            for (int s = 0; s < NSUB; ++s) sum[bi][s] += q == sk ? acc[bi][s] : t[qq][bi][s];
        }
      }
    }
#pragma unroll
    for (int bi = 0; bi < BTT; ++bi)
#pragma unroll
      for (int s = 0; s < NSUB; ++s) store_y<T, CS>(p, y0, n0, bi * CS + wc * NSUB + s, sum[bi][s]);
  }
  if (threadIdx.x == 0) counter_reset(&p.cnt[tile_lin]);
}

// ---------------------------------------------------------------------------------------
// Kind 1 ("ksplit"): one work-group = BTT*16 batch rows x NSUB*16 columns; its WPG waves split
// the work-group's share of the block list into contiguous slices and are reduced through LDS
// in wave order.  Each wave loads its own X fragments.  Best when bt is small (the X fragments
// are few) and many narrow column tiles are needed to fill the chip.
template <typename T, int BTT, int NSUB, int WPG, int DEPTH, bool N2D, bool SEL = false>
__global__ __launch_bounds__(64 * WPG) void bsg_gemm_kernel(GemmParams p) {
  constexpr int NT = 64 * WPG;
  constexpr int F = BTT * NSUB;
  constexpr int RED_BYTES = WPG > 1 ? (WPG - 1) * F * 64 * 16 : 0;  // waves 1..WPG-1
  constexpr int IDS_BYTES = BSG_MAX_NBLK * 4;
  // The block list (main loop) and the wave-reduction buffer (epilogue) share LDS.
  __shared__ __attribute__((aligned(16))) char s_mem[RED_BYTES > IDS_BYTES ? RED_BYTES : IDS_BYTES];
  __shared__ int s_misc[WPG + 2];
  int* const s_ids = (int*)s_mem;
  f32x4* const s_red = (f32x4*)s_mem;

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int tile, sk;
  tile_of_group(p.split_k, &tile, &sk);
  const int S = p.split_k;
  int n0, n0y;
  if (!tile_columns<N2D>(p, tile, 16 * NSUB, &n0, &n0y)) return;
  const int y0 = blockIdx.y * (16 * BTT);
  BSG_TL_DECL
  BSG_TL(0);

  const int na = stage_block_list<NT, !N2D, SEL, SEL && BTT == 1>(p, s_ids, s_misc);
  BSG_TL(1);

  // This wave's contiguous slice [pbeg, pend) of the list.
  const int G = S * WPG;
  const int g = sk * WPG + w;
  const int pbeg = (int)(((int64_t)na * g) / G);
  const int pend = (int)(((int64_t)na * (g + 1)) / G);
  const int cnt = pend - pbeg;

  const int blk_bytes = p.npad * 128;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(p.x, p.x_bytes);
  int xrow_off[BTT];
  bool xrow_ok[BTT];
#pragma unroll
  for (int bi = 0; bi < BTT; ++bi) {
    const int row = y0 + 16 * bi + (lane & 15);
    xrow_ok[bi] = row < p.bt;
    xrow_off[bi] = xrow_ok[bi] ? row * (int)p.ldx * 2 : 0;
  }
  const int xcol = 8 * (lane >> 4);
  const int wcol = lane * 16 + (n0 >> 4) * 2048;

  u32x4 wv[DEPTH][NSUB][2];
  u32x4 xv[DEPTH][BTT][2];
  f32x4 acc[BTT][NSUB];
#pragma unroll
  for (int bi = 0; bi < BTT; ++bi)
#pragma unroll
    for (int s = 0; s < NSUB; ++s) acc[bi][s] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto issue = [&](u32x4 (&wd)[NSUB][2], u32x4 (&xd)[BTT][2], int t) {
    const bool in = (unsigned)t < (unsigned)cnt;
    const int q = in ? pbeg + t : 0;
    int blk = s_ids[q];
    blk = __builtin_amdgcn_readfirstlane(blk);
    const bool ok = in && blk >= 0 && blk < p.nblk;
    const char* wb = (const char*)p.wp + (size_t)(ok ? blk : 0) * (size_t)blk_bytes;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(wb, ok ? blk_bytes : 0);
#pragma unroll
    for (int s = 0; s < NSUB; ++s) {
      wd[s][0] = ld16_stream(wr, wcol + s * 2048);
      wd[s][1] = ld16_stream(wr, wcol + s * 2048 + 1024);
    }
    const int kb = (ok ? blk : 0) * 64 + xcol;
#pragma unroll
    for (int bi = 0; bi < BTT; ++bi) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int col = kb + 32 * h;
        const bool v = ok && xrow_ok[bi] && col < p.K;
        xd[bi][h] = ld16(xr, v ? xrow_off[bi] + col * 2 : kOOB);
      }
    }
  };

  auto compute = [&](const u32x4 (&wd)[NSUB][2], const u32x4 (&xd)[BTT][2]) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int bi = 0; bi < BTT; ++bi)
#pragma unroll
        for (int s = 0; s < NSUB; ++s) acc[bi][s] = Elem<T>::mfma(wd[s][h], xd[bi][h], acc[bi][s]);
  };

  // Rolling pipeline, DEPTH blocks in flight, over U = cnt rounded up to DEPTH slots: slot u
  // holds list entry u - pad, so the pad leading slots are out-of-range loads (zero, no memory
  // traffic) issued with the first real ones, the passes have no data-dependent branches, and
  // the last pass only drains (no load is in flight when the loop ends).
  if (cnt > 0) {
    const int pad = (DEPTH - cnt % DEPTH) % DEPTH;
    const int U = cnt + pad;
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) issue(wv[d], xv[d], d - pad);
    int u0 = 0;
    for (; u0 + DEPTH < U; u0 += DEPTH) {
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) {
        compute(wv[d], xv[d]);
        BSG_TL_IF(2, u0 + d == pad);
        issue(wv[d], xv[d], u0 + d + DEPTH - pad);
        // Keep slot d's loads between its MFMAs and slot d+1's: left free, the scheduler may
        // gather a pass's MFMAs above its loads (each pass then waits for every block in
        // flight: vmcnt(0)), and which kernels it does this to changes with unrelated code.
        __builtin_amdgcn_sched_barrier(0);
      }
    }
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      compute(wv[d], xv[d]);
      BSG_TL_IF(2, u0 + d == pad);
    }
  }
  BSG_TL_LOOP_END();

  const size_t tile_lin = (size_t)blockIdx.y * (size_t)p.n_tiles + (size_t)tile;
  auto emit = [&](int f, f32x4 v) {
    if (S == 1)
      store_y<T, NSUB>(p, y0, n0y, f, v);
    else
      part_emit<F>(p, tile_lin, sk, f, v);
  };

  if constexpr (WPG > 1) {
    // Waves 1..WPG-1 hand their accumulators to wave 0 through LDS; wave 0 sums in wave
    // order and emits every fragment.
    __syncthreads();  // every wave is done reading s_ids before s_red overwrites it
    if (w > 0) {
#pragma unroll
      for (int bi = 0; bi < BTT; ++bi)
#pragma unroll
        for (int s = 0; s < NSUB; ++s) s_red[((w - 1) * F + bi * NSUB + s) * 64 + lane] = acc[bi][s];
    }
    __syncthreads();
    if (w == 0) {
#pragma unroll
      for (int bi = 0; bi < BTT; ++bi)
#pragma unroll
        for (int s = 0; s < NSUB; ++s) {
          for (int ww = 1; ww < WPG; ++ww) acc[bi][s] += s_red[((ww - 1) * F + bi * NSUB + s) * 64 + lane];
          emit(bi * NSUB + s, acc[bi][s]);
        }
    }
  } else {
#pragma unroll
    for (int bi = 0; bi < BTT; ++bi)
#pragma unroll
      for (int s = 0; s < NSUB; ++s) emit(bi * NSUB + s, acc[bi][s]);
  }

  BSG_TL(4);
  if (S > 1) splitk_finish<T, BTT, NSUB, NSUB, F>(p, tile_lin, y0, n0y, sk, 0, w == 0, acc, &s_misc[WPG]);
  BSG_TL_END(p, S == 1 || s_misc[WPG] != 0);
}

// Kinds 2 and 4 ("xlds"): one work-group = BTT*16 batch rows x WC*NSUB*16 columns; its waves
// walk the same block list together.  Each block's X tile (BTT*16 rows x 64 channels) is loaded
// once per work-group, in MFMA B-fragment order, into a double-buffered LDS stage (one barrier
// per block) and shared by every wave, so X costs 1/WPG of the loads of kind 1 and the prefetch
// registers hold weights only.  Kind 2 (WK = 1): the WC waves split the columns.  Kind 4
// (WK = 2): 2*WC waves, column group x 32-channel half of every block, so each wave issues half
// the MFMAs and LDS reads of a block and two waves share each SIMD, overlapping one wave's
// barrier and LDS waits with the other's MFMAs; the halves are summed through LDS at the end.
template <typename T, int BTT, int NSUB, int WC, int WK, int DEPTH, bool N2D, bool SEL = false>
__global__ __launch_bounds__(64 * WC * WK) void bsg_gemm_xl_kernel(GemmParams p) {
  constexpr int WPG = WC * WK;
  constexpr int NT = 64 * WPG;
  constexpr int XF = 2 * BTT;                // X fragments (1 KiB each) per block
  constexpr int XPW = (XF + WPG - 1) / WPG;  // X fragments each wave loads per block
  constexpr int CS = WC * NSUB;              // 16-column subtiles per work-group
  constexpr int FT = BTT * CS;               // output fragments per work-group
  constexpr int HPW = 2 / WK;                // channel halves per wave
  __shared__ __attribute__((aligned(16))) int s_ids[BSG_MAX_NBLK];
  __shared__ __attribute__((aligned(16))) u32x4 s_x[2][XF][64];
  __shared__ __attribute__((aligned(16))) f32x4 s_red[WK > 1 ? WC * BTT * NSUB : 1][64];
  __shared__ int s_misc[WPG + 2];

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wc = w % WC;  // column group
  const int wk = w / WC;  // channel half (kind 4)
  int tile, sk;
  tile_of_group(p.split_k, &tile, &sk);
  const int S = p.split_k;
  int n0, n0y;
  if (!tile_columns<N2D>(p, tile, 16 * CS, &n0, &n0y)) return;
  const int y0 = blockIdx.y * (16 * BTT);
  BSG_TL_DECL
  BSG_TL(0);

  const int na = stage_block_list<NT, !N2D, SEL, SEL && BTT == 1>(p, s_ids, s_misc);
  BSG_TL(1);

  // The work-group's contiguous slice of the list (all its waves walk it together).
  const int pbeg = (int)(((int64_t)na * sk) / S);
  const int pend = (int)(((int64_t)na * (sk + 1)) / S);
  const int cnt = pend - pbeg;

  const int blk_bytes = p.npad * 128;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(p.x, p.x_bytes);
  // X fragments this wave brings in: f = w + j*WPG -> batch tile f/2, k-half f%2.
  int xrow_off[XPW];
  bool xrow_ok[XPW];
  int xcol[XPW];
#pragma unroll
  for (int j = 0; j < XPW; ++j) {
    const int f = w + j * WPG;
    const int row = y0 + 16 * (f >> 1) + (lane & 15);
    xrow_ok[j] = f < XF && row < p.bt;
    xrow_off[j] = xrow_ok[j] ? row * (int)p.ldx * 2 : 0;
    xcol[j] = 32 * (f & 1) + 8 * (lane >> 4);
  }
  const int wcol = lane * 16 + ((n0 >> 4) + wc * NSUB) * 2048;

  u32x4 wv[DEPTH][NSUB][HPW];
  u32x4 xs[DEPTH][XPW];
  f32x4 acc[BTT][NSUB];
#pragma unroll
  for (int bi = 0; bi < BTT; ++bi)
#pragma unroll
    for (int s = 0; s < NSUB; ++s) acc[bi][s] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto issue = [&](u32x4 (&wd)[NSUB][HPW], u32x4 (&xd)[XPW], int t) {
    const bool in = (unsigned)t < (unsigned)cnt;
    const int q = in ? pbeg + t : 0;
    int blk = s_ids[q];
    blk = __builtin_amdgcn_readfirstlane(blk);
    const bool ok = in && blk >= 0 && blk < p.nblk;
    const char* wb = (const char*)p.wp + (size_t)(ok ? blk : 0) * (size_t)blk_bytes;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(wb, ok ? blk_bytes : 0);
#pragma unroll
    for (int s = 0; s < NSUB; ++s)
#pragma unroll
      for (int hh = 0; hh < HPW; ++hh) wd[s][hh] = ld16_stream(wr, wcol + s * 2048 + (WK > 1 ? wk : hh) * 1024);
    const int kb = (ok ? blk : 0) * 64;
#pragma unroll
    for (int j = 0; j < XPW; ++j) {
      const int col = kb + xcol[j];
      const bool v = ok && xrow_ok[j] && col < p.K;
      xd[j] = ld16(xr, v ? xrow_off[j] + col * 2 : kOOB);
    }
  };

  // Slot u: publish its X (LDS stage u & 1); after the barrier every wave has also finished
  // reading the stage it will overwrite at slot u + 1.
  auto consume = [&](const u32x4 (&wd)[NSUB][HPW], const u32x4 (&xd)[XPW], int u) {
    const int stage = u & 1;
#pragma unroll
    for (int j = 0; j < XPW; ++j)
      if (w + j * WPG < XF) s_x[stage][w + j * WPG][lane] = xd[j];
    __syncthreads();
#pragma unroll
    for (int hh = 0; hh < HPW; ++hh) {
      const int h = WK > 1 ? wk : hh;
#pragma unroll
      for (int bi = 0; bi < BTT; ++bi) {
        const u32x4 xb = s_x[stage][2 * bi + h][lane];
#pragma unroll
        for (int s = 0; s < NSUB; ++s) acc[bi][s] = Elem<T>::mfma(wd[s][hh], xb, acc[bi][s]);
      }
    }
  };

  // Rolling pipeline as in kind 1 (leading out-of-range slots, branch-free passes, a drain).
  // Every wave walks the same slice, so all take the same passes and barriers.
  if (cnt > 0) {
    const int pad = (DEPTH - cnt % DEPTH) % DEPTH;
    const int U = cnt + pad;
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) issue(wv[d], xs[d], d - pad);
    int u0 = 0;
    for (; u0 + DEPTH < U; u0 += DEPTH) {
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) {
        consume(wv[d], xs[d], u0 + d);
        BSG_TL_IF(2, u0 + d == pad);
        issue(wv[d], xs[d], u0 + d + DEPTH - pad);
        // Keep slot d's loads between its MFMAs and slot d+1's: left free, the scheduler may
        // gather a pass's MFMAs above its loads (each pass then waits for every block in
        // flight: vmcnt(0)), and which kernels it does this to changes with unrelated code.
        __builtin_amdgcn_sched_barrier(0);
      }
    }
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      consume(wv[d], xs[d], u0 + d);
      BSG_TL_IF(2, u0 + d == pad);
    }
  }
  BSG_TL_LOOP_END();

  if constexpr (WK > 1) {
    // The second channel half hands its accumulators to the first through LDS.
    if (wk == 1) {
#pragma unroll
      for (int bi = 0; bi < BTT; ++bi)
#pragma unroll
        for (int s = 0; s < NSUB; ++s) s_red[(wc * BTT + bi) * NSUB + s][lane] = acc[bi][s];
    }
    __syncthreads();
    if (wk == 0) {
#pragma unroll
      for (int bi = 0; bi < BTT; ++bi)
#pragma unroll
        for (int s = 0; s < NSUB; ++s) acc[bi][s] += s_red[(wc * BTT + bi) * NSUB + s][lane];
    }
  }

  const size_t tile_lin = (size_t)blockIdx.y * (size_t)p.n_tiles + (size_t)tile;
  if (wk == 0) {
#pragma unroll
    for (int bi = 0; bi < BTT; ++bi)
#pragma unroll
      for (int s = 0; s < NSUB; ++s) {
        const int g = bi * CS + wc * NSUB + s;
        if (S == 1)
          store_y<T, CS>(p, y0, n0y, g, acc[bi][s]);
        else
          part_emit<FT>(p, tile_lin, sk, g, acc[bi][s]);
      }
  }
  BSG_TL(4);
  if (S > 1) splitk_finish<T, BTT, NSUB, CS, FT>(p, tile_lin, y0, n0y, sk, wc, wk == 0, acc, &s_misc[WPG]);
  BSG_TL_END(p, S == 1 || s_misc[WPG] != 0);
}

// Kind 3 ("fma", batch tiles of 1-8 rows): the contraction is too thin for MFMA, so each lane
// multiplies the 8 consecutive channels of one weight column that its 16-byte load of the packed
// tile holds (channels 32h + 8g .. +7 of column c, with the four channel groups of a column on
// the four lanes of a quad: g = lane % 4, c = lane / 4; each load still covers one contiguous
// KiB) with the same channels of every batch row, in fp32 with packed fp16/bf16 dot products,
// and the quad is summed once at the end by two DPP quad permutes.  The waves split the work-group's block
// list (as kind 1); each wave stages the activations of its own slice (BT rows x 64 channels per
// block) in LDS once at the start, in [list position][row][half h][group g] 16-byte order, so
// each of its later reads is a broadcast and the loop streams weights only.  A wave reads only
// what it wrote, and one wave's LDS accesses complete in order, so the staging needs no
// barrier.  The waves are reduced through LDS in wave order.
template <typename T, int BT, int NSUB, int WPG, int DEPTH, bool N2D>
__global__ __launch_bounds__(64 * WPG) void bsg_gemm_fma_kernel(GemmParams p) {
  constexpr int NT = 64 * WPG;
  constexpr int XI = BSG_FMA_X_LOADS;  // staging loads per wave (host guarantees enough)
  __shared__ __attribute__((aligned(16))) int s_ids[BSG_MAX_NBLK];
  __shared__ float s_red[WPG > 1 ? WPG - 1 : 1][NSUB * BT][16];
  __shared__ int s_misc[WPG + 2];
  extern __shared__ __attribute__((aligned(16))) u32x4 s_xs[];  // [na][BT][2][4]

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tile = blockIdx.x;
  int n0, n0y;
  if (!tile_columns<N2D>(p, tile, 16 * NSUB, &n0, &n0y)) return;
  const int y0 = blockIdx.y * BT;
  BSG_TL_DECL
  BSG_TL(0);

  const int na = stage_block_list<NT, !N2D>(p, s_ids, s_misc);
  BSG_TL(1);
  const int pbeg = (int)(((int64_t)na * w) / WPG);
  const int pend = (int)(((int64_t)na * (w + 1)) / WPG);
  const int cnt = pend - pbeg;

  // Stage this wave's slice of X: 16-byte piece e = (q*BT + b)*8 + (4h + g) holds
  // x[y0+b][64 ids[q] + 32h + 8g ..] for list positions q in [pbeg, pend); the wave loads its
  // pieces pbeg*BT*8 + i*64 + lane, i < nxi.
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(p.x, p.x_bytes);
  const int e0 = pbeg * BT * 8;
  const int pieces = cnt * BT * 8;
  const int nxi = (pieces + 63) / 64;
  int qid[XI];  // block id of each staged piece, read as one batch
#pragma unroll
  for (int i = 0; i < XI; ++i) {
    const int q = pbeg + (i * 64 + lane) / (BT * 8);
    qid[i] = s_ids[q < pend ? q : 0];
  }
  const int blk_bytes = p.npad * 128;
  const int wcol = (lane & 3) * 256 + (lane >> 2) * 16 + (n0 >> 4) * 2048;  // quad layout
  u32x4 wv[DEPTH][NSUB][2];
  float acc[NSUB][BT];
#pragma unroll
  for (int s = 0; s < NSUB; ++s)
#pragma unroll
    for (int b = 0; b < BT; ++b) acc[s][b] = 0.f;

  auto issue = [&](u32x4 (&wd)[NSUB][2], int t) {
    const bool in = (unsigned)t < (unsigned)cnt;
    const int qq = in ? pbeg + t : 0;
    int blk = s_ids[qq];
    blk = __builtin_amdgcn_readfirstlane(blk);
    const bool ok = in && blk >= 0 && blk < p.nblk;
    const char* wb = (const char*)p.wp + (size_t)(ok ? blk : 0) * (size_t)blk_bytes;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(wb, ok ? blk_bytes : 0);
#pragma unroll
    for (int s = 0; s < NSUB; ++s) {
      wd[s][0] = ld16_stream(wr, wcol + s * 2048);
      wd[s][1] = ld16_stream(wr, wcol + s * 2048 + 1024);
    }
  };

  // The staging loads go out first and the first weight loads right behind them: loads complete
  // in issue order, so waiting for the staging leaves the weight loads in flight.
  u32x4 xs[XI];
#pragma unroll
  for (int i = 0; i < XI; ++i) {
    if (i < nxi) {
      const int e = i * 64 + lane;
      const int blk = e < pieces ? qid[i] : -1;
      const int row = y0 + (e / 8) % BT;
      const int col = blk * 64 + (e & 7) * 8;
      const bool v = blk >= 0 && blk < p.nblk && row < p.bt && col < p.K;
      xs[i] = ld16(xr, v ? row * (int)p.ldx * 2 + col * 2 : kOOB);
    }
  }
  // Rolling pipeline as in kind 1: slot u holds list entry u - pad (leading out-of-range
  // slots), branch-free passes, a drain.
  const int pad = (DEPTH - cnt % DEPTH) % DEPTH;
  const int U = cnt + pad;
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) issue(wv[d], d - pad);
#pragma unroll
  for (int i = 0; i < XI; ++i) {
    const int e = i * 64 + lane;
    if (i < nxi && e < pieces) s_xs[e0 + e] = xs[i];
  }
  // The wave's staging writes have completed before any of its reads of them is issued.
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt unconstrained

  // The X pieces of a block are read from LDS XD blocks ahead of its dot products (LDS latency
  // off the per-block path); XD shrinks as the batch tile grows to bound the registers.
  constexpr int XD = BT >= 8 ? 1 : (BT >= 4 ? 2 : DEPTH);
  static_assert(DEPTH % XD == 0, "X prefetch distance");
  const int g = lane & 3;
  u32x4 xv[XD][2][BT];
  auto xread = [&](u32x4 (&xd)[2][BT], int t) {
    // Positions outside the slice carry zero weights; read a valid X piece for them.
    const int q = pbeg + (t < 0 ? 0 : (t < cnt ? t : cnt - 1));
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int b = 0; b < BT; ++b) xd[h][b] = s_xs[((q * BT + b) * 2 + h) * 4 + g];
  };
  auto compute = [&](const u32x4 (&wd)[NSUB][2], const u32x4 (&xd)[2][BT]) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int b = 0; b < BT; ++b)
#pragma unroll
        for (int s = 0; s < NSUB; ++s) {
          float a = acc[s][b];
          a = Elem<T>::dot2(wd[s][h].x, xd[h][b].x, a);
          a = Elem<T>::dot2(wd[s][h].y, xd[h][b].y, a);
          a = Elem<T>::dot2(wd[s][h].z, xd[h][b].z, a);
          acc[s][b] = Elem<T>::dot2(wd[s][h].w, xd[h][b].w, a);
        }
  };

  if (cnt > 0) {
#pragma unroll
    for (int k = 0; k < XD; ++k) xread(xv[k], k - pad);
    int u0 = 0;
    for (; u0 + DEPTH < U; u0 += DEPTH) {
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) {
        compute(wv[d], xv[d % XD]);
        BSG_TL_IF(2, u0 + d == pad);
        xread(xv[d % XD], u0 + d + XD - pad);
        issue(wv[d], u0 + d + DEPTH - pad);
        // Keep block d's loads between its dot products and block d+1's: left free, the
        // scheduler gathers every dot product of the pass above every load, so each pass
        // starts by waiting for all DEPTH blocks in flight and the pipeline drains.
        __builtin_amdgcn_sched_barrier(0);
      }
    }
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      compute(wv[d], xv[d % XD]);
      BSG_TL_IF(2, u0 + d == pad);
      if (d + XD < DEPTH) xread(xv[d % XD], u0 + d + XD - pad);
    }
  }

  BSG_TL_LOOP_END();
  // Column c of subtile s: the quad of lanes 4c .. 4c+3 holds its four channel groups; two DPP
  // quad permutes (swap neighbours, then swap pairs) leave the column's sum on every lane of the
  // quad, (g0 + g1) + (g2 + g3) in a fixed order.
#pragma unroll
  for (int s = 0; s < NSUB; ++s)
#pragma unroll
    for (int b = 0; b < BT; ++b) {
      float v = acc[s][b];
      v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xf, 0xf, false));
      v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xf, 0xf, false));
      acc[s][b] = v;
    }
  const int qc = lane >> 2;  // the quad's column
  if constexpr (WPG > 1) {
    if (w > 0 && (lane & 3) == 0) {
#pragma unroll
      for (int s = 0; s < NSUB; ++s)
#pragma unroll
        for (int b = 0; b < BT; ++b) s_red[w - 1][s * BT + b][qc] = acc[s][b];
    }
    __syncthreads();
  }
  if (w == 0 && (lane & 3) == 0) {
#pragma unroll
    for (int s = 0; s < NSUB; ++s) {
      const int n = n0y + 16 * s + qc;
#pragma unroll
      for (int b = 0; b < BT; ++b) {
        float v = acc[s][b];
        for (int ww = 1; ww < WPG; ++ww) v += s_red[ww - 1][s * BT + b][qc];
        const int row = y0 + b;
        if (row < p.bt && n < p.ny) ((uint16_t*)p.y)[(size_t)row * (size_t)p.ldy + n] = Elem<T>::bits(v);
      }
    }
  }
  BSG_TL(4);
  BSG_TL_END(p, true);
}


// Column group t of G (kind 5): the N/16 subtiles are dealt out as evenly as possible, the
// first T mod G groups taking one more, so any G (the compute-unit count) is filled whatever N is.
__device__ __forceinline__ void vt_columns(int t, int G, int T, int* first, int* count) {
  const int base = T / G;
  const int extra = T - base * G;
  *first = t * base + (t < extra ? t : extra);
  *count = base + (t < extra ? 1 : 0);
}

// Kind 5 ("vt", variable-width tiles): one work-group = BTT*16 batch rows x nv <= NSUB 16-column
// subtiles, nv from vt_columns.  Its 2*WB waves are (32-channel half h) x (block slice b): wave
// (h, b) walks slice b of the list and, per block, loads the h-half of the weights of every
// subtile (NSUB x 1 KiB) and the h-half activation fragment of every row tile (BTT x 1 KiB)
// straight into registers.  Every weight and activation byte of the work-group is loaded by
// exactly one wave; the loop has no LDS traffic and no barrier.  At the end the 2*WB partial
// accumulators meet in LDS and wave w sums fragments w, w + 2*WB, ... in wave order and stores
// them.  Activation bytes per weight byte: 16*BTT / (16*nv); 256 groups of 2-3 subtiles fill
// 256 compute units at N = 11008 without split-K.
// KH = 1 (kind 6): no channel-half split; each of the WB waves loads both halves of every
// weight subtile and activation row tile of its blocks (the two halves of an activation row are
// one 128-byte line, requested back to back by one wave).
template <typename T, int BTT, int NSUB, int WB, int DEPTH, int KH = 2, bool SEL = false>
__global__ __launch_bounds__(64 * KH * WB) void bsg_gemm_vt_kernel(GemmParams p) {
  constexpr int NW = KH * WB;
  constexpr int NT = 64 * NW;
  constexpr int F = BTT * NSUB;
  constexpr int HP = 3 - KH;  // halves per wave
  __shared__ __attribute__((aligned(16))) int s_ids[BSG_MAX_NBLK];
  __shared__ __attribute__((aligned(16))) f32x4 s_red[NW][F][64];
  __shared__ int s_misc[NW + 2];

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = KH == 2 ? (w & 1) : 0;  // first channel half of this wave
  const int b = KH == 2 ? (w >> 1) : w;  // block slice
  int tile, sk;
  tile_of_group(1, &tile, &sk);
  int st, nv;
  vt_columns(tile, p.n_tiles, p.npad >> 4, &st, &nv);
  const int y0 = blockIdx.y * (16 * BTT);
  BSG_TL_DECL
  BSG_TL(0);

  const int na = stage_block_list<NT, true, SEL, SEL && BTT == 1>(p, s_ids, s_misc);
  BSG_TL(1);
  const int pbeg = (int)(((int64_t)na * b) / WB);
  const int pend = (int)(((int64_t)na * (b + 1)) / WB);
  const int cnt = pend - pbeg;

  const int blk_bytes = p.npad * 128;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(p.x, p.x_bytes);
  int xrow_off[BTT];
  bool xrow_ok[BTT];
#pragma unroll
  for (int bi = 0; bi < BTT; ++bi) {
    const int row = y0 + 16 * bi + (lane & 15);
    xrow_ok[bi] = row < p.bt;
    xrow_off[bi] = xrow_ok[bi] ? row * (int)p.ldx * 2 : 0;
  }
  const int xcol = 32 * h + 8 * (lane >> 4);
  int woff[NSUB];
#pragma unroll
  for (int s = 0; s < NSUB; ++s) woff[s] = s < nv ? lane * 16 + (st + s) * 2048 + h * 1024 : kOOB;

  u32x4 wv[DEPTH][NSUB][HP];
  u32x4 xv[DEPTH][BTT][HP];
  f32x4 acc[BTT][NSUB];
#pragma unroll
  for (int bi = 0; bi < BTT; ++bi)
#pragma unroll
    for (int s = 0; s < NSUB; ++s) acc[bi][s] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto issue = [&](u32x4 (&wd)[NSUB][HP], u32x4 (&xd)[BTT][HP], int t) {
    const bool in = (unsigned)t < (unsigned)cnt;
    const int q = in ? pbeg + t : 0;
    int blk = s_ids[q];
    blk = __builtin_amdgcn_readfirstlane(blk);
    const bool ok = in && blk >= 0 && blk < p.nblk;
    const char* wb = (const char*)p.wp + (size_t)(ok ? blk : 0) * (size_t)blk_bytes;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(wb, ok ? blk_bytes : 0);
#pragma unroll
    for (int s = 0; s < NSUB; ++s)
#pragma unroll
      for (int hh = 0; hh < HP; ++hh) wd[s][hh] = ld16_stream(wr, woff[s] + hh * 1024);
    // A skipped slot reads zeros through an empty resource (as its weights do), so the lanes'
    // selects below do not depend on `ok`: a uniform branch there let the register allocator
    // reuse an in-flight load's register and drain the pipeline (vmcnt(0)) every block.
    const __amdgpu_buffer_rsrc_t xb = make_rsrc(p.x, ok ? p.x_bytes : 0);
    const int col = (ok ? blk : 0) * 64 + xcol;
#pragma unroll
    for (int bi = 0; bi < BTT; ++bi)
#pragma unroll
      for (int hh = 0; hh < HP; ++hh) {
        const bool v = xrow_ok[bi] && col + 32 * hh < p.K;
        xd[bi][hh] = ld16(xb, v ? xrow_off[bi] + (col + 32 * hh) * 2 : kOOB);
      }
  };

  auto compute = [&](const u32x4 (&wd)[NSUB][HP], const u32x4 (&xd)[BTT][HP]) {
#pragma unroll
    for (int hh = 0; hh < HP; ++hh)
#pragma unroll
      for (int bi = 0; bi < BTT; ++bi)
#pragma unroll
        for (int s = 0; s < NSUB; ++s) acc[bi][s] = Elem<T>::mfma(wd[s][hh], xd[bi][hh], acc[bi][s]);
  };

  // Rolling pipeline as in kind 1: leading out-of-range slots, branch-free passes, a drain.
  if (cnt > 0) {
    const int pad = (DEPTH - cnt % DEPTH) % DEPTH;
    const int U = cnt + pad;
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) issue(wv[d], xv[d], d - pad);
    int u0 = 0;
    for (; u0 + DEPTH < U; u0 += DEPTH) {
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) {
        compute(wv[d], xv[d]);
        BSG_TL_IF(2, u0 + d == pad);
        issue(wv[d], xv[d], u0 + d + DEPTH - pad);
        // Keep slot d's loads between its MFMAs and slot d+1's: left free, the scheduler may
        // gather a pass's MFMAs above its loads (each pass then waits for every block in
        // flight: vmcnt(0)), and which kernels it does this to changes with unrelated code.
        __builtin_amdgcn_sched_barrier(0);
      }
    }
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      compute(wv[d], xv[d]);
      BSG_TL_IF(2, u0 + d == pad);
    }
  }
  BSG_TL_LOOP_END();

  // The 2*WB accumulator sets meet in LDS (the list buffer is no longer read: s_red is separate).
#pragma unroll
  for (int bi = 0; bi < BTT; ++bi)
#pragma unroll
    for (int s = 0; s < NSUB; ++s) s_red[w][bi * NSUB + s][lane] = acc[bi][s];
  __syncthreads();
  for (int f = w; f < F; f += NW) {
    f32x4 v = s_red[0][f][lane];
#pragma unroll
    for (int ww = 1; ww < NW; ++ww) v += s_red[ww][f][lane];
    if (f % NSUB < nv) store_y<T, NSUB>(p, y0, st * 16, f, v);
  }
  BSG_TL(4);
  BSG_TL_END(p, true);
}

// Kind 7 ("vtx"): the groups, waves and pipeline of kind 6, with each block's activations
// loaded into the wave's own LDS slot instead of into registers: BTT*16 rows x 64 channels
// arrive by 16-byte-per-lane loads, 16 rows x 64 contiguous bytes per load (a quad of lanes
// covers one half row, where kind 6 requests 16 rows x 16 bytes per quad), and are read back in
// MFMA order.  The quad's 16-byte chunks are rotated per row so that those reads hit distinct
// bank groups in every 8 and every 16 consecutive lanes.  The registers the activations no longer hold leave room
// for four block-slice waves at 64 rows; the wave reduction reuses each wave's own slots.  A
// separate kernel from kind 6 so that kind 6's generated code stays as it is (its schedules
// change with unrelated code in the same function).
template <typename T, int BTT, int NSUB, int WB, int DEPTH, bool SEL = false>
__global__ __launch_bounds__(64 * WB) void bsg_gemm_vtx_kernel(GemmParams p) {
  constexpr int NT = 64 * WB;
  constexpr int F = BTT * NSUB;
  constexpr int SLOT = BTT * 2;  // 1 KiB activation pieces per block: row tile x channel half
  static_assert(F <= DEPTH * SLOT, "the wave reduction reuses the wave's own activation slots");
  __shared__ __attribute__((aligned(16))) int s_ids[BSG_MAX_NBLK];
  __shared__ __attribute__((aligned(16))) u32x4 s_x[WB * DEPTH * SLOT][64];
  __shared__ int s_misc[WB + 2];

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // the wave's block slice
  int tile, sk;
  tile_of_group(1, &tile, &sk);
  int st, nv;
  vt_columns(tile, p.n_tiles, p.npad >> 4, &st, &nv);
  const int y0 = blockIdx.y * (16 * BTT);
  BSG_TL_DECL
  BSG_TL(0);

  const int na = stage_block_list<NT, true, SEL, SEL && BTT == 1>(p, s_ids, s_misc);
  BSG_TL(1);
  const int pbeg = (int)(((int64_t)na * w) / WB);
  const int pend = (int)(((int64_t)na * (w + 1)) / WB);
  const int cnt = pend - pbeg;

  const int blk_bytes = p.npad * 128;
  // lane 4q + c loads row q, 16-byte chunk (c - f(q)) % 4 of a 32-channel half, and MFMA lane m
  // reads its (row r = m % 16, chunk m / 16) back at 4r + (chunk + f(r)) % 4, with
  // f(r) = r/2 + r/8: any 8 consecutive lanes then read 8 distinct 16-byte bank groups of 128
  // bytes, and any 16 lanes 16 distinct groups of 256 bytes
  const int xq = lane >> 2;
  auto rot = [](int r) { return ((r >> 1) + (r >> 3)) & 3; };
  int xrow_off[BTT];
  bool xrow_ok[BTT];
#pragma unroll
  for (int bi = 0; bi < BTT; ++bi) {
    const int row = y0 + 16 * bi + xq;
    xrow_ok[bi] = row < p.bt;
    xrow_off[bi] = xrow_ok[bi] ? row * (int)p.ldx * 2 : 0;
  }
  const int xcol = 8 * (((lane & 3) - rot(xq)) & 3);
  const int rd_pos = 4 * (lane & 15) + (((lane >> 4) + rot(lane & 15)) & 3);
  int woff[NSUB];
#pragma unroll
  for (int s = 0; s < NSUB; ++s) woff[s] = s < nv ? lane * 16 + (st + s) * 2048 : kOOB;
  auto slot = [&](int d, int bi, int hh) -> u32x4* { return &s_x[(w * DEPTH + d) * SLOT + bi * 2 + hh][0]; };

  u32x4 wv[DEPTH][NSUB][2];
  f32x4 acc[BTT][NSUB];
#pragma unroll
  for (int bi = 0; bi < BTT; ++bi)
#pragma unroll
    for (int s = 0; s < NSUB; ++s) acc[bi][s] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Slot d's loads for list entry t: the activations (into LDS slot d) first, then the weights,
  // so that a wait for the weights covers the activations too.  A skipped entry loads through
  // empty resources: zeros for the weights, and zeros written to the slot.
  auto issue = [&](u32x4 (&wd)[NSUB][2], int d, int t) {
    const bool in = (unsigned)t < (unsigned)cnt;
    const int q = in ? pbeg + t : 0;
    int blk = s_ids[q];
    blk = __builtin_amdgcn_readfirstlane(blk);
    const bool ok = in && blk >= 0 && blk < p.nblk;
    const char* wb = (const char*)p.wp + (size_t)(ok ? blk : 0) * (size_t)blk_bytes;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(wb, ok ? blk_bytes : 0);
    const __amdgpu_buffer_rsrc_t xb = make_rsrc(p.x, ok ? p.x_bytes : 0);
    const int col = (ok ? blk : 0) * 64 + xcol;
#pragma unroll
    for (int bi = 0; bi < BTT; ++bi)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const bool v = xrow_ok[bi] && col + 32 * hh < p.K;
        ld16_lds(xb, slot(d, bi, hh), v ? xrow_off[bi] + (col + 32 * hh) * 2 : kOOB);
      }
    // The waits by count (read below) rely on this order: every activation load of the slot
    // before its weight loads, and the slot's loads before the next slot's.
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < NSUB; ++s)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) wd[s][hh] = ld16_stream(wr, woff[s] + hh * 1024);
    __builtin_amdgcn_sched_barrier(0);
  };

  // Slot d's activations, read from LDS into registers once every load up to its weights is
  // done (`later` slots' loads, SLOT activation + 2 NSUB weight loads each, and slot d's own
  // weights may still be in flight).  Each read comes right after an explicit wait inside the
  // loop body, so no read follows the loop's back edge, where the compiler's own wait for the
  // LDS loads would be for all of them (vmcnt(0)).
  constexpr int LX = SLOT, LW = NSUB * 2;
  u32x4 xl[BTT][2];
  auto read = [&](int d, auto later) {
    vmem_wait<LW + decltype(later)::value * (LX + LW)>();
#pragma unroll
    for (int bi = 0; bi < BTT; ++bi)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) xl[bi][hh] = slot(d, bi, hh)[rd_pos];
  };
  auto compute = [&](const u32x4 (&wd)[NSUB][2]) {
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int bi = 0; bi < BTT; ++bi)
#pragma unroll
        for (int s = 0; s < NSUB; ++s) acc[bi][s] = Elem<T>::mfma(wd[s][hh], xl[bi][hh], acc[bi][s]);
  };

  // Rolling pipeline as in kind 1 (leading out-of-range slots, branch-free passes, a drain), with
  // slot d+1's activations read before slot d's refill is waited on: compute slot d, refill it,
  // read slot d+1.
  if (cnt > 0) {
    const int pad = (DEPTH - cnt % DEPTH) % DEPTH;
    const int U = cnt + pad;
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) issue(wv[d], d, d - pad);
    read(0, std::integral_constant<int, DEPTH - 1>{});
    int u0 = 0;
    for (; u0 + DEPTH < U; u0 += DEPTH) {
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) {
        compute(wv[d]);
        BSG_TL_IF(2, u0 + d == pad);
        issue(wv[d], d, u0 + d + DEPTH - pad);
        // as in kinds 1 and 5/6: keep slot d's loads between its MFMAs and slot d+1's
        __builtin_amdgcn_sched_barrier(0);
        read((d + 1) % DEPTH, std::integral_constant<int, DEPTH - 1>{});
      }
    }
    static_for<DEPTH>([&](auto dd) {
      constexpr int d = decltype(dd)::value;
      compute(wv[d]);
      BSG_TL_IF(2, u0 + d == pad);
      if constexpr (d + 1 < DEPTH) read(d + 1, std::integral_constant<int, DEPTH - 2 - d>{});
    });
  }
  BSG_TL_LOOP_END();

  // The WB accumulator sets meet in LDS, each wave writing into its own slots (every load into
  // them has been waited for and read).
  auto red = [&](int ww, int f) -> f32x4* { return (f32x4*)&s_x[ww * DEPTH * SLOT + f][0]; };
#pragma unroll
  for (int bi = 0; bi < BTT; ++bi)
#pragma unroll
    for (int s = 0; s < NSUB; ++s) red(w, bi * NSUB + s)[lane] = acc[bi][s];
  __syncthreads();
  for (int f = w; f < F; f += WB) {
    f32x4 v = red(0, f)[lane];
#pragma unroll
    for (int ww = 1; ww < WB; ++ww) v += red(ww, f)[lane];
    if (f % NSUB < nv) store_y<T, NSUB>(p, y0, st * 16, f, v);
  }
  BSG_TL(4);
  BSG_TL_END(p, true);
}

// The 2-D instantiation of a tile, or null when its work-group covers more than one 64-column
// output block (the discarded branch is never instantiated).
template <int KIND, typename T, int B, int S, int W, int D>
constexpr GemmFn kernel_2d() {
  constexpr int gc = KIND == KIND_XLDS ? 16 * S * W : (KIND == KIND_XLDS_KH ? 16 * S * (W / 2) : 16 * S);
  if constexpr (gc > 64) {
    return nullptr;
  } else if constexpr (KIND == KIND_KSPLIT) {
    return bsg_gemm_kernel<T, B, S, W, D, true>;
  } else if constexpr (KIND == KIND_XLDS) {
    return bsg_gemm_xl_kernel<T, B, S, W, 1, D, true>;
  } else if constexpr (KIND == KIND_XLDS_KH) {
    return bsg_gemm_xl_kernel<T, B, S, W / 2, 2, D, true>;
  } else {
    return bsg_gemm_fma_kernel<T, B, S, W, D, true>;
  }
}

// The selection form (fp16, 1-D, in-GEMM top-k) of a tile of the MFMA kinds.
template <int KIND, int B, int S, int W, int D>
constexpr GemmFn kernel_sel() {
  if constexpr (KIND == KIND_KSPLIT) {
    return bsg_gemm_kernel<_Float16, B, S, W, D, false, true>;
  } else if constexpr (KIND == KIND_XLDS) {
    return bsg_gemm_xl_kernel<_Float16, B, S, W, 1, D, false, true>;
  } else if constexpr (KIND == KIND_XLDS_KH) {
    return bsg_gemm_xl_kernel<_Float16, B, S, W / 2, 2, D, false, true>;
  } else if constexpr (KIND == KIND_VT) {
    return bsg_gemm_vt_kernel<_Float16, B, S, W / 2, D, 2, true>;
  } else if constexpr (KIND == KIND_VT1) {
    return bsg_gemm_vt_kernel<_Float16, B, S, W, D, 1, true>;
  } else {
    return bsg_gemm_vtx_kernel<_Float16, B, S, W, D, true>;
  }
}

#define BSG_K(B, S, W, D)                                                                                          \
  {KIND_KSPLIT, 16 * B, S, W, D, bsg_gemm_kernel<_Float16, B, S, W, D, false>, bsg_gemm_kernel<__bf16, B, S, W, D, false>, \
   kernel_2d<KIND_KSPLIT, _Float16, B, S, W, D>(), kernel_2d<KIND_KSPLIT, __bf16, B, S, W, D>(),                   \
   kernel_sel<KIND_KSPLIT, B, S, W, D>()}
#define BSG_X(B, S, W, D)                                                                     \
  {KIND_XLDS, 16 * B, S, W, D, bsg_gemm_xl_kernel<_Float16, B, S, W, 1, D, false>,           \
   bsg_gemm_xl_kernel<__bf16, B, S, W, 1, D, false>, kernel_2d<KIND_XLDS, _Float16, B, S, W, D>(), \
   kernel_2d<KIND_XLDS, __bf16, B, S, W, D>(), kernel_sel<KIND_XLDS, B, S, W, D>()}
#define BSG_Y(B, S, W, D)                                                                        \
  {KIND_XLDS_KH, 16 * B, S, W, D, bsg_gemm_xl_kernel<_Float16, B, S, W / 2, 2, D, false>,        \
   bsg_gemm_xl_kernel<__bf16, B, S, W / 2, 2, D, false>, kernel_2d<KIND_XLDS_KH, _Float16, B, S, W, D>(), \
   kernel_2d<KIND_XLDS_KH, __bf16, B, S, W, D>(), kernel_sel<KIND_XLDS_KH, B, S, W, D>()}
#define BSG_V(B, S, W, D)                                                                               \
  {KIND_VT, 16 * B, S, W, D, bsg_gemm_vt_kernel<_Float16, B, S, W / 2, D>, bsg_gemm_vt_kernel<__bf16, B, S, W / 2, D>, \
   nullptr, nullptr, kernel_sel<KIND_VT, B, S, W, D>()}
#define BSG_V1(B, S, W, D)                                                                                \
  {KIND_VT1, 16 * B, S, W, D, bsg_gemm_vt_kernel<_Float16, B, S, W, D, 1>, bsg_gemm_vt_kernel<__bf16, B, S, W, D, 1>, \
   nullptr, nullptr, kernel_sel<KIND_VT1, B, S, W, D>()}
#define BSG_V1X(B, S, W, D)                                                                                    \
  {KIND_VT1X, 16 * B, S, W, D, bsg_gemm_vtx_kernel<_Float16, B, S, W, D>, bsg_gemm_vtx_kernel<__bf16, B, S, W, D>, \
   nullptr, nullptr, kernel_sel<KIND_VT1X, B, S, W, D>()}
#define BSG_F(R, S, W, D)                                                                                 \
  {KIND_FMA, R, S, W, D, bsg_gemm_fma_kernel<_Float16, R, S, W, D, false>, bsg_gemm_fma_kernel<__bf16, R, S, W, D, false>, \
   kernel_2d<KIND_FMA, _Float16, R, S, W, D>(), kernel_2d<KIND_FMA, __bf16, R, S, W, D>(), nullptr}

}  // namespace
