// bsgemm.hip — gfx950 (MI355X / CDNA4) C ABI, plan resolution, launches and the selector,
// packing and helper kernels for the batch-shared 64-channel block-sparse GEMM
//   Y[bt,N] = sum_{j active} X[bt,64j:64j+64] · W[64j:64j+64,N].
// The GEMM kernel templates are in bsg_device.hpp; their instantiated tiles are split over
// tiles_*.hip (one table per translation unit, compiled in parallel).
//
// Reference semantics: kernels/shared_mask_batched_triton_min_runtime.py
//   naive list kernel 684-733, bitmap kernel 814-874, split-K write/reduce 1898-1988,
//   packing 3133-3163, host wrappers 1064-1454 and 3166-3344.
//
// Design (MI355X-first, not a translation of the Triton kernels):
//   * The weight is packed once into a tiled K-major layout (see include/bsgemm.h): each
//     K-block is a contiguous slab and each 16-column tile of it is a 2 KiB run that a single
//     64-lane dwordx4 buffer load per k-half delivers straight into the A operand of
//     v_mfma_f32_16x16x32_{f16,bf16}.  No LDS staging of W, no transposes.
//   * The batch tile (16/32/64 rows) is the MFMA B operand, read with 16-byte loads from X
//     (tiny, L2-resident).  Rows >= bt, blocks past the list and k >= K are turned into
//     out-of-range buffer offsets, which return zeros without touching memory.
//   * Each work-group owns cols_per_wave output columns.  Its waves split the active-block
//     list into contiguous slices (in-group split-K, reduced through LDS in wave order), and
//     split_k work-groups share one column tile (fp32 partials + arrival counter; the last
//     work-group to arrive sums the partials in split order, so results are run-to-run
//     deterministic and a single launch suffices — no second reduce kernel).
//   * Every wave keeps `depth` K-blocks of loads in flight (a rolling register pipeline);
//     block ids come from LDS and are made wave-uniform, so buffer descriptors are scalar.
//   * The work-group -> tile map is XCD-aware: consecutive logical work-groups land on the
//     same XCD, so the split_k partners of a tile share one L2.

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>

#include "bsg_device.hpp"
#include "bsgemm.h"

// The GEMM ranks the block scores itself (MODE_TOPK) when each of its waves has at most this many
// rank items (64 blocks x 16 scores each); otherwise a separate rank launch runs first.
// The GEMM scores the blocks itself as well (one launch for the whole selection + GEMM) when
// the activations every work-group reads for that, bt x K x 2 bytes, are at most this many bytes
// (and bt <= BSG_SELF_MAX_ROWS).  Measured (selection + GEMM per call, graph of rotated launches,
// s=0.5): one launch saves 1.5 / 1.0 us at q/k/v/o B=1 / 2, 1.6 / 0.8 us at gate/up and 1.0 us at
// down B=1 (22 KiB); at 32 KiB (B=4, K=4096) it loses 0.3-0.4 us, since the wait for x grows
// with the bytes while the two-launch cost (a score launch and a cold load of its scores) stays.
#ifndef BSG_SELF_SCORE_MAX_X_BYTES
#define BSG_SELF_SCORE_MAX_X_BYTES 24576
#endif

#ifndef BSG_TOPK_ITEMS_PER_WAVE
#define BSG_TOPK_ITEMS_PER_WAVE 12
#endif

#define BSG_VERSION_STR "bsgemm 0.1 (gfx950, mfma_f32_16x16x32)"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(BSG_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

// Reference scoring rules (scripts/bench_roundrobin_e2e_decode.py:90-176) on the device, in
// fp64: per block j over its 64 channels, with b over the bt rows,
//   L2 mean       e2_j = mean_b sqrt(sum_c x^2)                       (RRD:100)
//   energy        e_j  = mean_b sum_c x^2 [* scale_c]                 (RRD:103-105, 131)
// optionally times max(prior_j + eps, 1e-6)^alpha (RRD:106-112).  Blocks are floor(K/64), as
// there.  Ranking is (score desc, id asc); with an energy budget the kept count grows from k to
// the first rank whose cumulative (unscaled) energy reaches budget * total (RRD:155-176).
// Scores are stored as order keys (score_order_key): unsigned 64-bit values in the order of the
// fp64 scores, so the rank kernel and a GEMM's in-kernel top-k compare them as integers.
struct SelScoreParams {
  const void* x;
  int64_t ldx;
  const float* prior;
  const float* scale;
  uint64_t* keys;   // ceil(K/64): floor(K/64) scored blocks, a partial last block at key 0
  double* energy;
  int32_t* idx_out;
  int32_t* na_out;
  float* ratio_out;
  float alpha, eps, energy_keep;
  int32_t bt, K, nb, k, mode;
};

template <typename T>
__device__ __forceinline__ float elem_to_float(uint32_t bits16);
template <>
__device__ __forceinline__ float elem_to_float<_Float16>(uint32_t b) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)b);
}
template <>
__device__ __forceinline__ float elem_to_float<__bf16>(uint32_t b) {
  return __builtin_bit_cast(float, b << 16);
}

// An fp64 score as an unsigned key in the same order: non-negative values keep their bits
// with the sign bit set, negative ones are complemented; -0 counts as +0 (they compare equal)
// and every NaN takes the largest key (a NaN score ranks first, as torch.topk ranks NaN above
// every number).  Every key of a real score is above 0, the key of padding and of a partial
// last block.
__device__ __forceinline__ uint64_t score_order_key(double s) {
  if (s != s) return ~0ull;
  const uint64_t b = __builtin_bit_cast(uint64_t, s + 0.0);
  return (b >> 63) ? ~b : (b | (1ull << 63));
}

// x plus lane i - n's x within the same 16-lane row (0 outside it), in fp64.
template <int CTRL>
__device__ __forceinline__ double f64_row_shr(double x) {
  return x + __builtin_bit_cast(double, u64_row_shr<CTRL>(__builtin_bit_cast(uint64_t, x)));
}

// Sum of lanes 15, 31, 47 and 63 (each row's last lane), the same value in every lane.
__device__ __forceinline__ double f64_rows_total(double x) {
  const uint64_t b = __builtin_bit_cast(uint64_t, x);
  const int lo = (int)(uint32_t)b, hi = (int)(uint32_t)(b >> 32);
  double r[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    r[i] = __builtin_bit_cast(double, ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(hi, 16 * i + 15) << 32) |
                                          (uint32_t)__builtin_amdgcn_readlane(lo, 16 * i + 15));
  return ((r[0] + r[1]) + r[2]) + r[3];
}

template <typename T>
__global__ __launch_bounds__(256) void bsg_score_rule_kernel(SelScoreParams p) {
  __shared__ double s_part[3][4];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int j = blockIdx.x;
  if (j >= p.nb) {
    // the partial last block (K % 64 != 0) is never scored (RRD:97-99): lowest key, no energy
    if (tid == 0) {
      p.keys[j] = 0;
      p.energy[j] = 0.0;
    }
    return;
  }

  // Thread gi: row gi / 8, channels 64j + 8(gi % 8) .. +7; the 8 threads of a row are
  // adjacent lanes, so a row's sum of squares is a 3-step butterfly.  The channel scales are
  // read once, and the 16-byte loads of up to U 32-row groups are in flight before any is
  // summed, so up to 32 * U rows cost one memory round trip (rows are still summed in order).
  constexpr int U = 4;
  double a_l2 = 0.0, a_e = 0.0, a_es = 0.0;
  const int rows = p.bt;
  const int c0 = 64 * j + 8 * (tid & 7);
  double scv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) scv[e] = p.scale ? (double)p.scale[c0 + e] : 0.0;
  for (int r0 = 0; r0 < rows; r0 += 32 * U) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int row = r0 + 32 * u + (tid >> 3);
      v[u] = u32x4{0u, 0u, 0u, 0u};
      if (row < rows) v[u] = *(const u32x4*)((const uint16_t*)p.x + (size_t)row * (size_t)p.ldx + c0);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int row = r0 + 32 * u + (tid >> 3);
      double sq = 0.0, sqs = 0.0;
      if (row < rows) {
        const uint32_t h[8] = {v[u].x & 0xffffu, v[u].x >> 16, v[u].y & 0xffffu, v[u].y >> 16,
                               v[u].z & 0xffffu, v[u].z >> 16, v[u].w & 0xffffu, v[u].w >> 16};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const double f = (double)elem_to_float<T>(h[e]);
          sq += f * f;
          if (p.scale) sqs += f * f * scv[e];
        }
      }
      // inclusive scans within 16-lane rows (DPP, no LDS round trip): the last lane of each
      // 8-lane group ends with its row's sum
      sq = f64_row_shr<0x111>(sq);
      sq = f64_row_shr<0x112>(sq);
      sq = f64_row_shr<0x114>(sq);
      sqs = f64_row_shr<0x111>(sqs);
      sqs = f64_row_shr<0x112>(sqs);
      sqs = f64_row_shr<0x114>(sqs);
      if ((tid & 7) == 7 && row < rows) {
        a_l2 += sqrt(sq);
        a_e += sq;
        a_es += sqs;
      }
    }
  }
  // lanes 7 and 15 of each row hold the partials: lane 15 takes their sum, and the wave's total
  // is the four rows' lanes 15, 31, 47 and 63
  a_l2 = f64_row_shr<0x118>(a_l2);
  a_e = f64_row_shr<0x118>(a_e);
  a_es = f64_row_shr<0x118>(a_es);
  a_l2 = f64_rows_total(a_l2);
  a_e = f64_rows_total(a_e);
  a_es = f64_rows_total(a_es);
  if (lane == 0) {
    s_part[0][w] = a_l2;
    s_part[1][w] = a_e;
    s_part[2][w] = a_es;
  }
  __syncthreads();
  if (tid == 0) {
    const double inv = 1.0 / (double)rows;
    const double l2 = (((s_part[0][0] + s_part[0][1]) + s_part[0][2]) + s_part[0][3]) * inv;
    const double en = (((s_part[1][0] + s_part[1][1]) + s_part[1][2]) + s_part[1][3]) * inv;
    const double es = (((s_part[2][0] + s_part[2][1]) + s_part[2][2]) + s_part[2][3]) * inv;
    double sc = p.mode == BSG_SCORE_L2_MEAN ? l2 : (p.scale ? es : en);
    if (p.prior) {
      const double pr = (double)p.prior[j] + (double)p.eps;
      sc *= pow(pr > 1e-6 ? pr : 1e-6, (double)p.alpha);
    }
    p.keys[j] = score_order_key(sc);
    p.energy[j] = en;
  }
}

// One work-group after bsg_score_rule_kernel on the same stream (the launch boundary orders
// the scores before these loads): ranks, applies the energy budget, writes the kept ids.
__global__ __launch_bounds__(256) void bsg_rank_rule_kernel(SelScoreParams p) {
  __shared__ double s_sc[BSG_MAX_NBLK];
  __shared__ double s_en[BSG_MAX_NBLK];
  __shared__ int s_order[BSG_MAX_NBLK];
  __shared__ uint8_t s_sel[BSG_MAX_NBLK];
  __shared__ double s_csum[256];
  __shared__ double s_total;
  __shared__ int s_scan[4];
  __shared__ int s_keep, s_first;
  const int tid = threadIdx.x;
  const int nb = p.nb;
  // the order keys first (in s_sc's storage), the cumulative energy by rank after the ranking
  uint64_t* s_key = (uint64_t*)s_sc;
  for (int i = tid; i < nb; i += 256) {
    s_key[i] = p.keys[i];
    s_en[i] = p.energy[i];
  }
  pad_scores(s_key, nb);
  __syncthreads();
  // rank of every block; order[rank] = block (keys of real scores are above the pads' 0)
  for (int j = tid; j < nb; j += 256) s_order[rank_of<false>(s_key, nb, j, s_key[j])] = j;
  const int k0 = p.k < nb ? p.k : nb;
  if (tid == 0) {
    s_keep = k0;
    s_first = nb;
  }
  for (int i = tid; i < nb; i += 256) s_sel[i] = 0;
  __syncthreads();  // s_sc is free again: it holds the cumulative energy by rank from here on
  if (p.energy_keep > 0.f || p.ratio_out) {
    // Cumulative energy in rank order: each thread sums a contiguous run of ranks, the run
    // totals are scanned in thread order, then each run is walked again.
    const int per = (nb + 255) / 256;
    const int beg = tid * per < nb ? tid * per : nb;
    const int end = beg + per < nb ? beg + per : nb;
    double run = 0.0;
    for (int r = beg; r < end; ++r) run += s_en[s_order[r]];
    s_csum[tid] = run;
    __syncthreads();
    if (tid == 0) {
      double acc = 0.0;
      for (int t = 0; t < 256; ++t) {
        const double v = s_csum[t];
        s_csum[t] = acc;
        acc += v;
      }
      s_total = acc;
    }
    __syncthreads();
    const double thr = (double)p.energy_keep * (s_total > 1e-12 ? s_total : 1e-12);
    double cum = s_csum[tid];
    int first = nb;
    for (int r = beg; r < end; ++r) {
      cum += s_en[s_order[r]];
      s_sc[r] = cum;
      if (first == nb && cum >= thr) first = r;
    }
    if (first < nb) atomicMin(&s_first, first);
    __syncthreads();
    if (tid == 0) {
      const double total = s_total > 1e-12 ? s_total : 1e-12;
      int keep = k0;
      if (p.energy_keep > 0.f && k0 > 0 && s_sc[k0 - 1] / total < (double)p.energy_keep) {
        keep = s_first + 1;
        keep = keep < k0 ? k0 : (keep > nb ? nb : keep);
      }
      s_keep = keep;
      if (p.ratio_out) *p.ratio_out = keep > 0 ? (float)(s_sc[keep - 1] / total) : 0.f;
    }
    __syncthreads();
  }
  const int keep = s_keep;
  for (int r = tid; r < keep; r += 256) s_sel[s_order[r]] = 1;
  __syncthreads();
  const int per = (nb + 255) / 256;
  const int beg = tid * per < nb ? tid * per : nb;
  const int end = beg + per < nb ? beg + per : nb;
  int c = 0;
  for (int jj = beg; jj < end; ++jj) c += s_sel[jj];
  int total = 0;
  int o = wg_exclusive_scan<256>(c, s_scan, &total);
  for (int jj = beg; jj < end; ++jj)
    if (s_sel[jj]) p.idx_out[o++] = jj;
  if (tid == 0) *p.na_out = keep;
}
// Read-rate calibration (no counterpart in the reference): streams `bytes` from src with the
// access pattern of the GEMM's weight stream (one 1 KiB wave-load per 16-byte lane slice,
// non-temporal, DEPTH = 4 in flight, each wave walking its own contiguous run), and writes only
// if the data XOR-folds to a value the caller names, so the loads cannot be dropped.  It gives
// the practical HBM read time of a launch of the same size on this device.
__global__ __launch_bounds__(256) void bsg_read_kernel(const char* __restrict__ src, int64_t n1k, uint32_t magic,
                                                       uint32_t* __restrict__ sink) {
  constexpr int DEPTH = 4;
  const int lane = threadIdx.x & 63;
  const int64_t nw = (int64_t)gridDim.x * 4;
  const int64_t wv = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t per = (n1k + nw - 1) / nw;
  const int64_t beg = wv * per;
  u32x4 acc = {0u, 0u, 0u, 0u};
  u32x4 v[DEPTH];
  auto load = [&](int64_t i) -> u32x4 {
    const int64_t b = beg + i;
    const bool ok = i < per && b < n1k;
    return ld16_stream(make_rsrc(src + (ok ? b : 0) * 1024, ok ? 1024 : 0), lane * 16);
  };
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) v[d] = load(d);
  for (int64_t i0 = 0; i0 < per; i0 += DEPTH) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      acc ^= v[d];
      v[d] = load(i0 + d + DEPTH);
    }
  }
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == magic) sink[0] = 1u;
}

// Pack W (logical [N,K], element strides sn/sk) into the tiled K-major layout.
// One thread per 8-element (16-byte) group of the packed slab.
__global__ __launch_bounds__(256) void bsg_pack_kernel(const uint16_t* __restrict__ w, int64_t N,
                                                       int64_t K, int64_t sn, int64_t skk,
                                                       int64_t ntile, int64_t groups,
                                                       uint16_t* __restrict__ wp) {
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (gid >= groups) return;
  const int64_t blk = gid / (ntile * 128);
  const int64_t rem = gid - blk * ntile * 128;
  const int64_t t = rem >> 7;
  const int r = (int)(rem & 127);
  const int h = r >> 6, g = (r >> 4) & 3, c = r & 15;
  const int64_t n = 16 * t + c;
  const int64_t k0 = 64 * blk + 32 * h + 8 * g;
  uint16_t v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = (n < N && k0 + e < K) ? w[n * sn + (k0 + e) * skk] : (uint16_t)0;
  u32x4 o;
  o.x = v[0] | ((uint32_t)v[1] << 16);
  o.y = v[2] | ((uint32_t)v[3] << 16);
  o.z = v[4] | ((uint32_t)v[5] << 16);
  o.w = v[6] | ((uint32_t)v[7] << 16);
  *(u32x4*)(wp + gid * 8) = o;
}

__global__ __launch_bounds__(256) void bsg_zero_kernel(uint32_t* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = 0u;
}

struct SelParams {
  const uint16_t* x;
  int64_t ldx;
  uint64_t* scores;
  int32_t* idx_out;
  int32_t* na_out;
  int32_t bt, K, nblk, k;
};

// Exact-L1 selector, first launch: work-group j sums |x| over block j and every row, in exact
// integer units, and stores it.  The ranking (bsg_rank_l1_kernel, or a GEMM in top-k mode) is a
// separate launch: a last-arriver hand-off would put every work-group's increment on one
// device-scope counter, and those serialize (4-7 us at 64-172 blocks, measured).

__global__ __launch_bounds__(256) void bsg_score_l1_kernel(SelParams p) {
  __shared__ uint64_t s_part[16];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int j = blockIdx.x;

  // Up to U 16-byte groups per thread are loaded before any is summed, so a batch of up to
  // 32 * U rows costs one memory round trip rather than one per 32 rows.
  constexpr int U = 4;
  uint64_t acc = 0;
  const int groups = p.bt * 8;
  for (int g0 = 0; g0 < groups; g0 += 256 * U) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int gi = g0 + 256 * u + tid;
      const int row = gi >> 3;
      const int col = 64 * j + 8 * (gi & 7);
      v[u] = u32x4{0u, 0u, 0u, 0u};
      if (gi < groups && col < p.K) v[u] = *(const u32x4*)(p.x + (size_t)row * (size_t)p.ldx + col);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc += f16x8_units(v[u]);
  }
  // Inclusive scan within each 16-lane row (a few cycles per step, no LDS round trip): lane 15
  // of every row ends with the row's sum; the 16 row sums of the work-group meet in LDS.
  acc += u64_row_shr<0x111>(acc);
  acc += u64_row_shr<0x112>(acc);
  acc += u64_row_shr<0x114>(acc);
  acc += u64_row_shr<0x118>(acc);
  if ((lane & 15) == 15) s_part[4 * w + (lane >> 4)] = acc;
  __syncthreads();
  if (tid == 0) {
    uint64_t t = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) t += s_part[i];
    p.scores[j] = t;
  }
}

// One work-group after bsg_score_l1_kernel on the same stream (the launch boundary orders the
// scores before these loads): the top-k, written ascending with its count.
__global__ __launch_bounds__(1024) void bsg_rank_l1_kernel(SelParams p) {
  __shared__ __attribute__((aligned(16))) uint64_t s_key[BSG_MAX_NBLK];
  __shared__ int s_rank[BSG_MAX_NBLK];
  const int k = topk_l1_list<1024>(p.scores, p.nblk, p.k, p.bt <= 64, s_key, s_rank,
                                  [&](int pos, int id) { p.idx_out[pos] = id; });
  if (threadIdx.x == 0) *p.na_out = k;
}

// ----------------------------------------------------------------------------------------
// Host side: kernel table, plan resolution, validation, launches.

// Compact 2-D output back to the dense N axis: work-group i copies active block i (64 columns,
// 256 threads = 4 rows x 64 columns per step) to columns 64 * n_blocks[i] .. (below N).
__global__ __launch_bounds__(256) void bsg_scatter_kernel(const uint16_t* __restrict__ c, int64_t ldc, int32_t bt,
                                                          const int32_t* __restrict__ nb, int32_t nn,
                                                          const int32_t* __restrict__ nn_dev, int32_t N,
                                                          uint16_t* __restrict__ out, int64_t ldo) {
  const int i = blockIdx.x;
  int cnt = nn;
  if (nn_dev != nullptr) {
    const int d = *nn_dev;
    cnt = d < 0 ? 0 : (d < nn ? d : nn);
  }
  if (i >= cnt) return;
  const int b = nb[i];
  if (b < 0 || b >= (N + 63) / 64) return;
  const int col = threadIdx.x & 63;
  const int dst = 64 * b + col;
  if (dst >= N) return;
  for (int r = blockIdx.y * 4 + (threadIdx.x >> 6); r < bt; r += gridDim.y * 4)
    out[(size_t)r * (size_t)ldo + dst] = c[(size_t)r * (size_t)ldc + 64 * i + col];
}

// Active 64-column blocks of an element mask (any byte != 0), ascending, with their count: one
// work-group walks the blocks 1024 at a time, each thread testing one block, and compacts the
// flags with a work-group scan.
__global__ __launch_bounds__(1024) void bsg_nmask_kernel(const uint8_t* __restrict__ mask, int64_t N,
                                                         int32_t* __restrict__ out, int32_t* __restrict__ count) {
  __shared__ int s_scan[16];
  const int tid = threadIdx.x;
  const int64_t nb = (N + 63) / 64;
  int base = 0;
  for (int64_t b0 = 0; b0 < nb; b0 += 1024) {
    const int64_t b = b0 + tid;
    int any = 0;
    if (b < nb) {
      const int64_t e = 64 * b + 64 < N ? 64 * b + 64 : N;
      for (int64_t c = 64 * b; c < e; ++c) any |= mask[c];
    }
    int total = 0;
    const int o = wg_exclusive_scan<1024>(any != 0, s_scan, &total);
    if (any != 0) out[base + o] = (int32_t)b;
    base += total;
  }
  if (tid == 0) *count = base;
}

// The whole instantiated tile set, one table per translation unit.
const TileTable* const kTables[] = {&kTilesK1R16, &kTilesK1R32, &kTilesK1R64, &kTilesK2, &kTilesK4, &kTilesK3,
                                    &kTilesK5, &kTilesK7};

const KernelEntry* find_kernel_scan(int kind, int rows, int nsub, int wpg, int depth) {
  for (const TileTable* t : kTables)
    for (int i = 0; i < t->n; ++i) {
      const KernelEntry& e = t->e[i];
      if (e.kind == kind && e.rows == rows && e.nsub == nsub && e.wpg == wpg && e.depth == depth) return &e;
    }
  return nullptr;
}

// A launch looks its tile up two to four times (plan validation, then the launch itself), and
// eager callers repeat the same few tiles: the last hits of this thread are kept.
const KernelEntry* find_kernel(int kind, int rows, int nsub, int wpg, int depth) {
  struct Hit {
    int kind, rows, nsub, wpg, depth;
    const KernelEntry* e;
  };
  static thread_local Hit hits[4] = {{-1, 0, 0, 0, 0, nullptr}, {-1, 0, 0, 0, 0, nullptr},
                                     {-1, 0, 0, 0, 0, nullptr}, {-1, 0, 0, 0, 0, nullptr}};
  static thread_local int next = 0;
  for (const Hit& h : hits)
    if (h.kind == kind && h.rows == rows && h.nsub == nsub && h.wpg == wpg && h.depth == depth) return h.e;
  const KernelEntry* e = find_kernel_scan(kind, rows, nsub, wpg, depth);
  if (e != nullptr) {
    hits[next] = Hit{kind, rows, nsub, wpg, depth, e};
    next = (next + 1) & 3;
  }
  return e;
}

// Kind 3: each wave stages its slice of the list's activation blocks (at most ceil(na / wpg)
// blocks x rows pieces of 128 B) in LDS with at most BSG_FMA_X_LOADS 1 KiB loads, and the
// work-group's list takes na x rows x 128 B of LDS.
bool fma_fits(int64_t na, int rows, int wpg) {
  return (na + wpg - 1) / wpg * rows <= (int64_t)BSG_FMA_X_LOADS * 8 && na * rows * 128 <= BSG_FMA_LDS_MAX;
}

int pow2_ceil(int64_t v) {
  int r = 1;
  while (r < v) r <<= 1;
  return r;
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

bool pow2_in(int v, int lo, int hi) { return v >= lo && v <= hi && (v & (v - 1)) == 0; }

// Columns covered by one work-group of a resolved plan (kind 5: at most; its groups take the
// floor or ceiling of an even share).
int64_t group_cols(const bsg_plan* pl) {
  if (pl->kind == KIND_XLDS) return (int64_t)pl->cols_per_wave * pl->waves_per_group;
  if (pl->kind == KIND_XLDS_KH) return (int64_t)pl->cols_per_wave * (pl->waves_per_group / 2);
  return pl->cols_per_wave;
}

int resolve_fma(int64_t bt, int32_t na, bsg_plan* pl) {
  if (pl->rows_per_group != 1 && pl->rows_per_group != 2 && pl->rows_per_group != 4 && pl->rows_per_group != 8)
    return fail(BSG_ERR_UNSUPPORTED, "plan: kind 3 rows_per_group=%d (1, 2, 4 or 8)", pl->rows_per_group);
  if (pl->split_k == 0) pl->split_k = 1;
  if (pl->split_k != 1) return fail(BSG_ERR_UNSUPPORTED, "plan: kind 3 needs split_k=1 (got %d)", pl->split_k);
  if (pl->cols_per_wave == 0) pl->cols_per_wave = 16;
  if (pl->depth == 0) pl->depth = 4;
  if (pl->waves_per_group == 0) {
    pl->waves_per_group = 4;
    while (pl->waves_per_group < 8 && !fma_fits(na, pl->rows_per_group, pl->waves_per_group))
      pl->waves_per_group *= 2;
  }
  if (!fma_fits(na, pl->rows_per_group, pl->waves_per_group))
    return fail(BSG_ERR_UNSUPPORTED, "plan: kind 3 stages %d blocks x %d rows, more than %d waves can (use kind 1)",
                na, pl->rows_per_group, pl->waves_per_group);
  if (!find_kernel(KIND_FMA, pl->rows_per_group, pl->cols_per_wave / 16, pl->waves_per_group, pl->depth))
    return fail(BSG_ERR_UNSUPPORTED, "plan: no kind 3 kernel for rows_per_group=%d cols_per_wave=%d "
                "waves_per_group=%d depth=%d", pl->rows_per_group, pl->cols_per_wave, pl->waves_per_group,
                pl->depth);
  return BSG_OK;
}

// Kind 5, 6 and 7 plans: explicit or tuned only; no split-K (their groups already fill the chip).
int resolve_vt(bsg_plan* pl) {
  const int rpg = pl->rows_per_group;
  if (rpg != 16 && rpg != 32 && rpg != 64)
    return fail(BSG_ERR_UNSUPPORTED, "plan: kind %d rows_per_group=%d (16, 32 or 64)", pl->kind, rpg);
  if (pl->split_k == 0) pl->split_k = 1;
  if (pl->split_k != 1)
    return fail(BSG_ERR_UNSUPPORTED, "plan: kind %d needs split_k=1 (got %d)", pl->kind, pl->split_k);
  if (pl->cols_per_wave == 0) pl->cols_per_wave = 48;
  if (pl->waves_per_group == 0) pl->waves_per_group = 4;
  if (pl->depth == 0) pl->depth = 4;
  if (pl->cols_per_wave % 16 != 0 ||
      !find_kernel(pl->kind, rpg, pl->cols_per_wave / 16, pl->waves_per_group, pl->depth))
    return fail(BSG_ERR_UNSUPPORTED, "plan: no kind %d kernel for rows_per_group=%d cols_per_wave=%d "
                "waves_per_group=%d depth=%d", pl->kind, rpg, pl->cols_per_wave, pl->waves_per_group, pl->depth);
  return BSG_OK;
}

// Kind 5 column groups: every compute unit (per row group) gets one, unless that would leave a
// group more than the plan's subtiles; never more groups than subtiles.
int64_t vt_groups(int64_t N, int64_t ygroups, int32_t cu, const bsg_plan* pl) {
  const int64_t T = cdiv(N, 16);
  const int64_t nsub = pl->cols_per_wave / 16;
  int64_t g = cu / ygroups;
  if (g < cdiv(T, nsub)) g = cdiv(T, nsub);
  if (g > T) g = T;
  return g < 1 ? 1 : g;
}

int resolve(int64_t bt, int64_t N, int32_t nblk, int32_t na, int32_t cu, bsg_plan* pl) {
  if (bt <= 0 || N <= 0 || nblk <= 0 || na < 0 || cu <= 0)
    return fail(BSG_ERR_ARG, "plan: bt=%lld N=%lld nblk=%d na=%d cu=%d", (long long)bt, (long long)N,
                nblk, na, cu);
  if (pl->kind < 0 || pl->kind > KIND_VT1X)
    return fail(BSG_ERR_UNSUPPORTED, "plan: kind=%d (1 = waves split the block list, 2 = X tile in LDS, "
                "3 = fp32 dot products for 1-8 rows, 4 = as 2 with channel-half waves, 5 = variable-width "
                "column groups, 6 = as 5 with waves splitting blocks only, 7 = as 6 with the activations "
                "loaded into LDS)", pl->kind);
  if (pl->kind == KIND_VT || pl->kind == KIND_VT1 || pl->kind == KIND_VT1X) {
    if (pl->rows_per_group == 0) pl->rows_per_group = bt <= 16 ? 16 : (bt <= 32 ? 32 : 64);
    return resolve_vt(pl);
  }
  // The dot-product kernel (kind 3) runs when a plan names it; automatic plans use the MFMA
  // kinds, which measure faster at every batch size on gfx950.
  if (pl->rows_per_group == 0 && pl->kind == KIND_FMA) pl->rows_per_group = bt <= 8 ? pow2_ceil(bt) : 8;
  if (pl->rows_per_group == 0) pl->rows_per_group = bt <= 16 ? 16 : (bt <= 32 ? 32 : 64);
  const int rpg = pl->rows_per_group;
  if (pl->kind == 0) pl->kind = rpg <= 8 ? KIND_FMA : (rpg == 16 ? KIND_KSPLIT : KIND_XLDS);
  if (pl->kind == KIND_FMA) return resolve_fma(bt, na, pl);
  if (rpg != 16 && rpg != 32 && rpg != 64)
    return fail(BSG_ERR_UNSUPPORTED, "plan: rows_per_group=%d (16, 32 or 64 for kinds 1-2)", rpg);
  const int auto_fields = (pl->cols_per_wave == 0 ? 1 : 0) | (pl->waves_per_group == 0 ? 2 : 0) |
                          (pl->depth == 0 ? 4 : 0);
  if (pl->kind == KIND_KSPLIT) {
    if (pl->cols_per_wave == 0) pl->cols_per_wave = rpg == 16 ? 16 : 32;
    if (pl->waves_per_group == 0) pl->waves_per_group = rpg == 16 ? 2 : 4;
    if (pl->depth == 0) pl->depth = rpg == 64 ? 2 : 4;
  } else {
    if (pl->cols_per_wave == 0) pl->cols_per_wave = 16;
    if (pl->waves_per_group == 0) pl->waves_per_group = pl->kind == KIND_XLDS_KH ? 8 : 4;
    if (pl->depth == 0) pl->depth = 4;
  }
  if (!pow2_in(pl->cols_per_wave, 16, 128) || !pow2_in(pl->waves_per_group, 1, 8) ||
      !pow2_in(pl->depth, 1, 8))
    return fail(BSG_ERR_UNSUPPORTED, "plan: cols_per_wave=%d waves_per_group=%d depth=%d",
                pl->cols_per_wave, pl->waves_per_group, pl->depth);
  if (!find_kernel(pl->kind, rpg, pl->cols_per_wave / 16, pl->waves_per_group, pl->depth) &&
      auto_fields) {
    // An automatic field led to a tile that is not compiled: take the instantiated kernel
    // that keeps every explicit field and is closest in the automatic ones.
    const KernelEntry* best = nullptr;
    int best_d = 1 << 30;
    for (const TileTable* t : kTables)
      for (int i = 0; i < t->n; ++i) {
        const KernelEntry& e = t->e[i];
        if (e.kind != pl->kind || e.rows != rpg) continue;
        if (!(auto_fields & 1) && e.nsub * 16 != pl->cols_per_wave) continue;
        if (!(auto_fields & 2) && e.wpg != pl->waves_per_group) continue;
        if (!(auto_fields & 4) && e.depth != pl->depth) continue;
        const int d = abs(e.nsub * 16 - pl->cols_per_wave) * 64 + abs(e.wpg - pl->waves_per_group) * 8 +
                      abs(e.depth - pl->depth);
        if (d < best_d) {
          best_d = d;
          best = &e;
        }
      }
    if (best) {
      pl->cols_per_wave = best->nsub * 16;
      pl->waves_per_group = best->wpg;
      pl->depth = best->depth;
    }
  }
  if (!find_kernel(pl->kind, rpg, pl->cols_per_wave / 16, pl->waves_per_group, pl->depth))
    return fail(BSG_ERR_UNSUPPORTED,
                "plan: no kernel instantiated for kind=%d rows_per_group=%d cols_per_wave=%d "
                "waves_per_group=%d depth=%d",
                pl->kind, rpg, pl->cols_per_wave, pl->waves_per_group, pl->depth);
  if (pl->split_k == 0) {
    // Enough work-groups to cover every compute unit once, without giving a wave fewer than
    // two blocks; kind 1 also counts its waves as list splitters.
    const int64_t n_tiles = cdiv(cdiv(N, 16) * 16, group_cols(pl));
    const int64_t groups = n_tiles * cdiv(bt, rpg);
    int64_t s = cdiv(cu, groups);
    const int64_t splitters = pl->kind == KIND_KSPLIT ? pl->waves_per_group : 1;
    const int64_t by_work = (int64_t)na / (2 * splitters);
    if (s > by_work) s = by_work;
    if (s > 32) s = 32;
    if (s < 1) s = 1;
    pl->split_k = (int32_t)s;
  }
  if (pl->split_k < 1 || pl->split_k > 256)
    return fail(BSG_ERR_UNSUPPORTED, "plan: split_k=%d (1..256)", pl->split_k);
  return BSG_OK;
}

// Output tiles a split-K workspace is sized for: the 1-D tiling, or a 2-D launch over every
// 64-column block, whichever is larger.  Every launch of a plan on (bt, N) keeps its arrival
// counters in the first ws_counter_bytes and its partials right after, whatever its own tile
// count (a 2-D launch over few output blocks uses a prefix of both), so calls that share a
// workspace always agree on where the counters end.
int64_t ws_max_tiles(int64_t bt, int64_t N, const bsg_plan* pl) {
  const int64_t gc = group_cols(pl);
  int64_t n_tiles = cdiv(cdiv(N, 16) * 16, gc);
  if (gc <= 64 && cdiv(N, 64) * (64 / gc) > n_tiles) n_tiles = cdiv(N, 64) * (64 / gc);
  return n_tiles * cdiv(bt, pl->rows_per_group);
}

int64_t ws_counter_bytes(int64_t bt, int64_t N, const bsg_plan* pl) {
  return cdiv(ws_max_tiles(bt, N, pl) * 4, 256) * 256;
}

int64_t gemm_ws_bytes(int64_t bt, int64_t N, const bsg_plan* pl) {
  if (pl->split_k <= 1) return 0;
  const int64_t frag = (int64_t)(pl->rows_per_group / 16) * (group_cols(pl) / 16);
  const int64_t part = ws_max_tiles(bt, N, pl) * pl->split_k * frag * 64 * 16;
  return ws_counter_bytes(bt, N, pl) + part;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Compute units of the current device, cached per device ordinal.
int device_cu_count() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    cache[dev] = v;
  }
  return cache[dev];
}

// y_cols: the columns Y must hold (N, or the compact width of a 2-D launch).
int check_common(const void* x, int64_t ldx, int64_t bt, int64_t K, const void* wp, int64_t N,
                 void* y, int64_t ldy, int dtype, int64_t y_cols) {
  if (dtype != BSG_F16 && dtype != BSG_BF16) return fail(BSG_ERR_DTYPE, "dtype=%d (0=fp16, 1=bf16)", dtype);
  if (bt < 0 || K <= 0 || N <= 0) return fail(BSG_ERR_ARG, "sizes bt=%lld K=%lld N=%lld", (long long)bt, (long long)K, (long long)N);
  if (cdiv(K, BSG_BLOCK_K) > BSG_MAX_NBLK)
    return fail(BSG_ERR_UNSUPPORTED, "K=%lld exceeds %d blocks of 64", (long long)K, BSG_MAX_NBLK);
  if (bt == 0) return BSG_OK;
  if (!x || !wp || !y) return fail(BSG_ERR_ARG, "null pointer (x=%p wp=%p y=%p)", x, wp, y);
  if (K % 8 != 0) return fail(BSG_ERR_ALIGN, "K=%lld must be a multiple of 8", (long long)K);
  if (ldx < K || ldx % 8 != 0 || !aligned16(x))
    return fail(BSG_ERR_ALIGN, "x must be 16-byte aligned with ldx >= K and ldx %% 8 == 0 (ldx=%lld)", (long long)ldx);
  if (!aligned16(wp)) return fail(BSG_ERR_ALIGN, "packed weight must be 16-byte aligned");
  if (ldy < y_cols) return fail(BSG_ERR_ARG, "ldy=%lld < %lld output columns", (long long)ldy, (long long)y_cols);
  if (((uintptr_t)y & 1u) != 0) return fail(BSG_ERR_ALIGN, "y must be 2-byte aligned");
  if ((bt - 1) * ldx * 2 + ldx * 2 >= (int64_t)0x7fffffff)
    return fail(BSG_ERR_UNSUPPORTED, "x spans >= 2 GiB");
  if (cdiv(N, 16) * 16 * 128 >= (int64_t)0x7fffffff) return fail(BSG_ERR_UNSUPPORTED, "N too large");
  return BSG_OK;
}

#ifdef BSG_TIMELINE
// Profiling build: launches write their work-groups' phase stamps to consecutive slots of a
// caller buffer (bsg_timeline_attach), slot = launch count modulo the slot count, so the R
// launches of a captured graph each keep their own slot across replays.
uint64_t* g_tl_base = nullptr;
int64_t g_tl_slots = 0, g_tl_slot_groups = 0, g_tl_next = 0;

uint64_t* timeline_slot(int64_t groups) {
  if (g_tl_base == nullptr || groups > g_tl_slot_groups) return nullptr;
  uint64_t* t = g_tl_base + (g_tl_next % g_tl_slots) * g_tl_slot_groups * 8;
  ++g_tl_next;
  return t;
}
#else
uint64_t* timeline_slot(int64_t) { return nullptr; }
#endif

// Optional parts of a launch.  MODE_TOPK: the exact-L1 block scores (na is then k), and where
// work-group (0, 0) publishes the kept list and its count (null: not published).  2-D
// sparsity: the active 64-column output blocks nidx[nn] (device; nn_dev, when set, a device
// count <= nn), and whether Y is compact ([bt, nn * 64], the blocks side by side).
struct LaunchExtras {
  const uint64_t* scores = nullptr;
  // the scores are exact-L1 integers below 2^53 (so (score << 11) | id is a unique key); 0 for
  // any other order key, e.g. the reference rules' (two compares per pair)
  int score_keyed = 1;
  int32_t* idx_out = nullptr;
  int32_t* na_out = nullptr;
  const int32_t* nidx = nullptr;
  int32_t nn = 0;
  const int32_t* nn_dev = nullptr;
  int ncompact = 0;
  // Fixed split-K storage (the allocation-free entry point): counters and partials at these
  // addresses, with room for cnt_cap_tiles counters and part_cap_bytes of partials, instead of
  // being carved from ws.
  uint32_t* cnt_fixed = nullptr;
  float* part_fixed = nullptr;
  int64_t cnt_cap_tiles = 0;
  int64_t part_cap_bytes = 0;
  // MODE_LIST: the kernel sorts the list ascending while staging it
  int sort_list = 0;
};

int launch_gemm(int mode, const void* x, int64_t ldx, int64_t bt, int64_t K, const void* wp,
                int64_t N, const int32_t* idx, int32_t na, const int32_t* na_dev,
                const uint8_t* bitmap, int32_t nbm, void* y, int64_t ldy, int dtype, void* ws, int64_t ws_bytes,
                const bsg_plan* plan_in, void* stream, const LaunchExtras& ex = LaunchExtras{}) {
  const int64_t n_blocks = cdiv(N, 64);
  if (ex.nidx != nullptr && (ex.nn < 0 || ex.nn > n_blocks))
    return fail(BSG_ERR_ARG, "2-D: %d active output blocks (0..%lld)", ex.nn, (long long)n_blocks);
  const int64_t y_cols = ex.nidx != nullptr && ex.ncompact ? (int64_t)ex.nn * 64 : N;
  int rc = check_common(x, ldx, bt, K, wp, N, y, ldy, dtype, y_cols);
  if (rc != BSG_OK || bt == 0) return rc;
  if (ex.nidx != nullptr && ex.nn == 0) return BSG_OK;  // no output block: nothing to write
  const int32_t nblk = (int32_t)cdiv(K, BSG_BLOCK_K);
  if (mode == MODE_LIST) {
    if (na < 0 || na > BSG_MAX_NBLK) return fail(BSG_ERR_ARG, "num_active=%d (0..%d)", na, BSG_MAX_NBLK);
    if (na > 0 && !idx) return fail(BSG_ERR_ARG, "active_blocks is null");
    if (ex.sort_list && na > BSG_MAX_NBLK / 2)
      return fail(BSG_ERR_UNSUPPORTED, "in-kernel sort: num_active=%d (at most %d)", na, BSG_MAX_NBLK / 2);
  } else if (mode == MODE_TOPK || mode == MODE_TOPK_SELF) {
    if (mode == MODE_TOPK && !ex.scores)
      return fail(BSG_ERR_ARG, "top-k: scores=%p k=%d", (const void*)ex.scores, na);
    if (na < 0) return fail(BSG_ERR_ARG, "top-k: k=%d", na);
    if (mode == MODE_TOPK_SELF && (bt > BSG_SELF_MAX_ROWS || dtype != BSG_F16 || ex.nidx != nullptr))
      return fail(BSG_ERR_UNSUPPORTED, "self-scored top-k: bt=%lld dtype=%d (fp16, at most %d rows, 1-D)",
                  (long long)bt, dtype, BSG_SELF_MAX_ROWS);
    if (nblk > BSG_TOPK_MAX_NBLK)
      return fail(BSG_ERR_UNSUPPORTED, "top-k in the GEMM: %d blocks (at most %d)", nblk, BSG_TOPK_MAX_NBLK);
    if (na > nblk) na = nblk;
  } else if (mode == MODE_BITMAP) {
    if (!bitmap) return fail(BSG_ERR_ARG, "bitmap is null");
    if (nbm < 1 || nbm > nblk)
      return fail(BSG_ERR_ARG, "total_k_blocks=%d outside [1, ceil(K/64)=%d]", nbm, nblk);
    na = nbm;
  } else {
    na = nblk;
  }
  bsg_plan pl = plan_in ? *plan_in : bsg_plan{0, 0, 0, 0, 0, 0};
  int cu = 256;
  if (pl.split_k == 0) cu = device_cu_count();  // only feeds the automatic split-K choice
  // a 2-D launch fills the chip with its active blocks only
  rc = resolve(bt, ex.nidx != nullptr ? (int64_t)ex.nn * 64 : N, nblk, na, cu, &pl);
  if (rc != BSG_OK) return rc;
  const int64_t need = gemm_ws_bytes(bt, N, &pl);
  const bool fixed_ws = ex.part_fixed != nullptr;
  if (fixed_ws) {
    const int64_t part_need = need > 0 ? need - ws_counter_bytes(bt, N, &pl) : 0;
    if (need > 0 && (ws_max_tiles(bt, N, &pl) > ex.cnt_cap_tiles || part_need > ex.part_cap_bytes))
      return fail(BSG_ERR_WORKSPACE,
                  "split-K %d needs %lld tile counters and %lld bytes of partials; the static scratch holds "
                  "%lld counters and %lld bytes (use the workspace entry point)",
                  pl.split_k, (long long)ws_max_tiles(bt, N, &pl), (long long)part_need,
                  (long long)ex.cnt_cap_tiles, (long long)ex.part_cap_bytes);
  } else {
    if (need > 0 && !aligned16(ws)) return fail(BSG_ERR_ALIGN, "workspace must be 16-byte aligned");
    if (need > 0 && (!ws || ws_bytes < need))
      return fail(BSG_ERR_WORKSPACE, "workspace %lld bytes < %lld needed (split_k=%d)", (long long)ws_bytes,
                  (long long)need, pl.split_k);
  }
  const KernelEntry* ke =
      find_kernel(pl.kind, pl.rows_per_group, pl.cols_per_wave / 16, pl.waves_per_group, pl.depth);
  const int64_t npad = cdiv(N, 16) * 16;
  const int64_t gc = group_cols(&pl);
  if (ex.nidx != nullptr && gc > 64)
    return fail(BSG_ERR_UNSUPPORTED, "2-D: the plan covers %lld columns per work-group (at most 64: "
                "cols_per_wave x column waves)", (long long)gc);
  // 2-D: 64 / gc tiles per active output block (a device-side count leaves tiles idle)
  const int64_t ygroups = cdiv(bt, pl.rows_per_group);
  const bool vt = pl.kind == KIND_VT || pl.kind == KIND_VT1 || pl.kind == KIND_VT1X;
  if (vt && ex.nidx != nullptr)
    return fail(BSG_ERR_UNSUPPORTED, "2-D: kinds 5-7 (variable-width column groups) have no 2-D form");
  const int64_t n_tiles = vt ? vt_groups(N, ygroups, device_cu_count(), &pl)
                          : ex.nidx != nullptr ? (int64_t)ex.nn * (64 / gc) : cdiv(npad, gc);
  if (n_tiles * pl.split_k > 0x7fffffff || ygroups > 65535) return fail(BSG_ERR_UNSUPPORTED, "grid too large");

  GemmParams p;
  p.x = x;
  p.wp = wp;
  p.y = y;
  p.idx = idx;
  p.na_dev = na_dev;
  p.bitmap = bitmap;
  if (need > 0 && n_tiles * ygroups > ws_max_tiles(bt, N, &pl))
    return fail(BSG_ERR_UNSUPPORTED, "%lld output tiles exceed the workspace layout", (long long)(n_tiles * ygroups));
  p.cnt = need > 0 ? (fixed_ws ? ex.cnt_fixed : (uint32_t*)ws) : nullptr;
  p.part = need > 0 ? (fixed_ws ? ex.part_fixed : (float*)((char*)ws + ws_counter_bytes(bt, N, &pl))) : nullptr;
  p.ldx = ldx;
  p.ldy = ldy;
  p.bt = (int32_t)bt;
  p.K = (int32_t)K;
  p.N = (int32_t)N;
  p.npad = (int32_t)npad;
  p.nblk = nblk;
  p.nbm = nbm;
  p.na = na;
  p.mode = mode;
  p.split_k = pl.split_k;
  p.n_tiles = (int32_t)n_tiles;
  p.x_bytes = (int32_t)(((bt - 1) * ldx + K) * 2);
  p.ny = (int32_t)y_cols;
  p.y_fast = (y_cols % 4 == 0) && (ldy % 4 == 0) && (((uintptr_t)y & 7u) == 0);
  p.scores = ex.scores;
  p.idx_out = ex.idx_out;
  p.na_out = ex.na_out;
  p.keyed = ex.score_keyed && bt <= 64;
  p.sort_list = mode == MODE_LIST && ex.sort_list && ex.nidx == nullptr;
  p.nidx = ex.nidx;
  p.nn_dev = ex.nn_dev;
  p.nn = ex.nn;
  p.ncompact = ex.ncompact;
  p.tl = timeline_slot((int64_t)n_tiles * pl.split_k * ygroups);

  dim3 grid((unsigned)(n_tiles * pl.split_k), (unsigned)ygroups, 1);
  dim3 block((unsigned)(64 * pl.waves_per_group), 1, 1);
  const bool topk = mode == MODE_TOPK || mode == MODE_TOPK_SELF;
  GemmFn fn = topk ? (dtype == BSG_F16 ? ke->f16_sel : nullptr)
              : ex.nidx != nullptr ? (dtype == BSG_F16 ? ke->f16_2d : ke->bf16_2d)
                                   : (dtype == BSG_F16 ? ke->f16 : ke->bf16);
  if (topk && (fn == nullptr || (mode == MODE_TOPK_SELF && pl.rows_per_group != 16)))
    return fail(BSG_ERR_UNSUPPORTED, "top-k in the GEMM: no selection instantiation for this tile (fp16, MFMA kinds; "
                "self-scored: 16-row tiles)");
  if (fn == nullptr) return fail(BSG_ERR_UNSUPPORTED, "2-D: no instantiation for this tile");
  // Kind 3: LDS for the staged activations of the whole list (na is the list capacity; a
  // device-side count or a bitmap only shortens it).
  const size_t dyn_lds = pl.kind == KIND_FMA ? (size_t)na * (size_t)pl.rows_per_group * 128 : 0;
  hipLaunchKernelGGL(fn, grid, block, dyn_lds, (hipStream_t)stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "bsg_gemm launch");
  return BSG_OK;
}

// The allocation-free entry point's storage: one static device array per GPU, laid out as
// [tile arrival counters | exact-L1 block scores | split-K partials].  The counters start at
// zero (the array is zero-filled when the code object loads, and cleared again on the first call
// on each device) and every GEMM leaves them at zero; scores and partials are written before
// they are read.  Host code never passes the array's name: it is a host-side stand-in, and a
// kernel given it would fault.  Its device address comes from hipGetSymbolAddress, once per
// device, and that address is what the kernels receive.
constexpr int64_t kScratchCntBytes = 64 * 1024;                      // 16384 tile counters
constexpr int64_t kScratchScoreBytes = BSG_MAX_NBLK * 8;             // uint64 scores, 16 KiB
constexpr int64_t kScratchPartOff = kScratchCntBytes + kScratchScoreBytes;
static_assert(kScratchPartOff % 256 == 0 && kScratchPartOff < BSG_NOALLOC_SCRATCH_BYTES, "scratch layout");

static __device__ __attribute__((aligned(256))) unsigned char scratch[BSG_NOALLOC_SCRATCH_BYTES];

std::mutex g_scratch_mu;
char* g_scratch_ptr[64] = {};

// The scratch array's device address on the current device (looked up, and its counters
// cleared on `stream`, on the first call there).
int noalloc_scratch(char** out, void* stream) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= 64) return fail(BSG_ERR_UNSUPPORTED, "device ordinal %d (at most 63)", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    // The first call may come while this thread's stream is being captured: the symbol lookup is
    // not a stream operation, so it runs under the relaxed capture mode (the global mode may
    // refuse it), and the counter clear below then becomes a node of the graph (run on every
    // replay, before the call's own kernels).
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    e = hipThreadExchangeStreamCaptureMode(&mode);
    if (e != hipSuccess) return hip_fail(e, "hipThreadExchangeStreamCaptureMode");
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    const hipError_t restore = hipThreadExchangeStreamCaptureMode(&mode);
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (restore != hipSuccess) return hip_fail(restore, "hipThreadExchangeStreamCaptureMode (restore)");
    if (ptr == nullptr || ((uintptr_t)ptr & 255u) != 0) return fail(BSG_ERR_HIP, "scratch address %p", ptr);
    const int64_t n = kScratchCntBytes / 4;
    hipLaunchKernelGGL(bsg_zero_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, (hipStream_t)stream,
                       (uint32_t*)ptr, n);
    e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "scratch counter clear");
    g_scratch_ptr[dev] = (char*)ptr;
  }
  *out = g_scratch_ptr[dev];
  return BSG_OK;
}

}  // namespace

extern "C" {

const char* bsg_version(void) { return BSG_VERSION_STR; }

const char* bsg_last_error(void) { return g_err; }

int64_t bsg_packed_bytes(int64_t N, int64_t K, int dtype) {
  if (N <= 0 || K <= 0 || (dtype != BSG_F16 && dtype != BSG_BF16)) return -1;
  return cdiv(K, BSG_BLOCK_K) * 64 * cdiv(N, 16) * 16 * 2;
}

int bsg_pack_weight(const void* w, int64_t N, int64_t K, int64_t stride_n, int64_t stride_k, int dtype,
                    void* wp, int64_t wp_bytes, void* stream) {
  if (dtype != BSG_F16 && dtype != BSG_BF16) return fail(BSG_ERR_DTYPE, "dtype=%d", dtype);
  if (N <= 0 || K <= 0 || stride_n <= 0 || stride_k <= 0)
    return fail(BSG_ERR_ARG, "pack: N=%lld K=%lld stride_n=%lld stride_k=%lld", (long long)N, (long long)K,
                (long long)stride_n, (long long)stride_k);
  if (!w || !wp) return fail(BSG_ERR_ARG, "pack: null pointer");
  if (!aligned16(wp)) return fail(BSG_ERR_ALIGN, "pack: destination must be 16-byte aligned");
  if (cdiv(K, BSG_BLOCK_K) > BSG_MAX_NBLK) return fail(BSG_ERR_UNSUPPORTED, "pack: K=%lld too large", (long long)K);
  const int64_t need = bsg_packed_bytes(N, K, dtype);
  if (wp_bytes < need) return fail(BSG_ERR_ARG, "pack: destination %lld bytes < %lld", (long long)wp_bytes, (long long)need);
  const int64_t ntile = cdiv(N, 16);
  const int64_t groups = cdiv(K, BSG_BLOCK_K) * ntile * 128;
  const int64_t nb = cdiv(groups, 256);
  if (nb > 0x7fffffff) return fail(BSG_ERR_UNSUPPORTED, "pack: too large");
  hipLaunchKernelGGL(bsg_pack_kernel, dim3((unsigned)nb), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)w, N, K, stride_n, stride_k, ntile, groups, (uint16_t*)wp);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "bsg_pack_weight launch");
  return BSG_OK;
}

int bsg_plan_resolve(int64_t bt, int64_t N, int32_t nblk, int32_t na, int32_t cu_count, bsg_plan* plan) {
  if (!plan) return fail(BSG_ERR_ARG, "plan is null");
  return resolve(bt, N, nblk, na, cu_count, plan);
}

int64_t bsg_gemm_workspace_bytes(int64_t bt, int64_t N, const bsg_plan* plan) {
  if (!plan || bt <= 0 || N <= 0) return -1;
  return gemm_ws_bytes(bt, N, plan);
}

int bsg_workspace_init(void* ws, int64_t ws_bytes, void* stream) {
  if (ws_bytes < 0 || (ws_bytes > 0 && !ws)) return fail(BSG_ERR_ARG, "workspace_init: bad arguments");
  if (ws_bytes == 0) return BSG_OK;
  if (((uintptr_t)ws & 3u) != 0) return fail(BSG_ERR_ALIGN, "workspace must be 4-byte aligned");
  const int64_t n = ws_bytes / 4;
  int64_t nb = cdiv(n, 256);
  if (nb > 4096) nb = 4096;
  hipLaunchKernelGGL(bsg_zero_kernel, dim3((unsigned)nb), dim3(256), 0, (hipStream_t)stream, (uint32_t*)ws, n);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "bsg_workspace_init launch");
  return BSG_OK;
}

int bsg_gemm(const void* x, int64_t ldx, int64_t bt, int64_t K, const void* wp, int64_t N,
             const int32_t* active_blocks, int32_t num_active, const int32_t* num_active_dev, void* y,
             int64_t ldy, int dtype, void* ws, int64_t ws_bytes, const bsg_plan* plan, void* stream) {
  return launch_gemm(MODE_LIST, x, ldx, bt, K, wp, N, active_blocks, num_active, num_active_dev, nullptr, 0, y,
                     ldy, dtype, ws, ws_bytes, plan, stream);
}

int bsg_gemm_sorted(const void* x, int64_t ldx, int64_t bt, int64_t K, const void* wp, int64_t N,
                    const int32_t* active_blocks, int32_t num_active, const int32_t* num_active_dev, void* y,
                    int64_t ldy, int dtype, void* ws, int64_t ws_bytes, const bsg_plan* plan, void* stream) {
  LaunchExtras ex;
  ex.sort_list = 1;
  return launch_gemm(MODE_LIST, x, ldx, bt, K, wp, N, active_blocks, num_active, num_active_dev, nullptr, 0, y,
                     ldy, dtype, ws, ws_bytes, plan, stream, ex);
}

int bsg_gemm_bitmap(const void* x, int64_t ldx, int64_t bt, int64_t K, const void* wp, int64_t N,
                    const uint8_t* bitmap, int32_t total_k_blocks, void* y, int64_t ldy, int dtype, void* ws,
                    int64_t ws_bytes, const bsg_plan* plan, void* stream) {
  return launch_gemm(MODE_BITMAP, x, ldx, bt, K, wp, N, nullptr, 0, nullptr, bitmap, total_k_blocks, y, ldy, dtype,
                     ws, ws_bytes, plan, stream);
}

int bsg_gemm_dense(const void* x, int64_t ldx, int64_t bt, int64_t K, const void* wp, int64_t N, void* y,
                   int64_t ldy, int dtype, void* ws, int64_t ws_bytes, const bsg_plan* plan, void* stream) {
  return launch_gemm(MODE_DENSE, x, ldx, bt, K, wp, N, nullptr, 0, nullptr, nullptr, 0, y, ldy, dtype, ws,
                     ws_bytes, plan, stream);
}

int bsg_gemm_2d(const void* x, int64_t ldx, int64_t bt, int64_t K, const void* wp, int64_t N,
                const int32_t* active_blocks, int32_t num_active, const int32_t* num_active_dev,
                const int32_t* n_blocks, int32_t num_n, const int32_t* num_n_dev, int compact, void* y,
                int64_t ldy, int dtype, void* ws, int64_t ws_bytes, const bsg_plan* plan, void* stream) {
  if (num_n < 0 || num_n > cdiv(N, 64))
    return fail(BSG_ERR_ARG, "2-D: num_n=%d outside [0, ceil(N/64)] (N=%lld)", num_n, (long long)N);
  if (num_n == 0)  // no output block: only the checks run, nothing is written
    return check_common(x, ldx, bt, K, wp, N, y, ldy, dtype, compact ? 0 : N);
  if (!n_blocks) return fail(BSG_ERR_ARG, "2-D: n_blocks is null");
  LaunchExtras ex;
  ex.nidx = n_blocks;
  ex.nn = num_n;
  ex.nn_dev = num_n_dev;
  ex.ncompact = compact != 0;
  if (active_blocks == nullptr && num_active_dev == nullptr)
    return launch_gemm(MODE_DENSE, x, ldx, bt, K, wp, N, nullptr, 0, nullptr, nullptr, 0, y, ldy, dtype, ws,
                       ws_bytes, plan, stream, ex);
  return launch_gemm(MODE_LIST, x, ldx, bt, K, wp, N, active_blocks, num_active, num_active_dev, nullptr, 0, y,
                     ldy, dtype, ws, ws_bytes, plan, stream, ex);
}

int bsg_scatter_nblocks(const void* compact, int64_t ldc, int64_t bt, const int32_t* n_blocks, int32_t num_n,
                        const int32_t* num_n_dev, int64_t N, void* out, int64_t ldo, void* stream) {
  if (bt < 0 || N <= 0 || num_n < 0 || num_n > cdiv(N, 64) || N > 0x7fffffff)
    return fail(BSG_ERR_ARG, "scatter: bt=%lld N=%lld num_n=%d", (long long)bt, (long long)N, num_n);
  if (bt == 0 || num_n == 0) return BSG_OK;
  if (!compact || !n_blocks || !out) return fail(BSG_ERR_ARG, "scatter: null pointer");
  if (ldc < (int64_t)num_n * 64 || ldo < N)
    return fail(BSG_ERR_ARG, "scatter: ldc=%lld (>= %d) ldo=%lld (>= N)", (long long)ldc, num_n * 64, (long long)ldo);
  if (((uintptr_t)compact & 1u) || ((uintptr_t)out & 1u)) return fail(BSG_ERR_ALIGN, "scatter: 2-byte alignment");
  const int64_t gy = cdiv(bt, 4) < 64 ? cdiv(bt, 4) : 64;
  hipLaunchKernelGGL(bsg_scatter_kernel, dim3((unsigned)num_n, (unsigned)gy), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)compact, ldc, (int32_t)bt, n_blocks, num_n, num_n_dev, (int32_t)N,
                     (uint16_t*)out, ldo);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "bsg_scatter_nblocks launch");
  return BSG_OK;
}

int bsg_nmask_blocks(const uint8_t* mask, int64_t N, int32_t* n_blocks_out, int32_t* num_out, void* stream) {
  if (N <= 0 || N > 0x7fffffff) return fail(BSG_ERR_ARG, "nmask: N=%lld", (long long)N);
  if (!mask || !n_blocks_out || !num_out) return fail(BSG_ERR_ARG, "nmask: null pointer");
  hipLaunchKernelGGL(bsg_nmask_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, mask, N, n_blocks_out, num_out);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "bsg_nmask_blocks launch");
  return BSG_OK;
}

int64_t bsg_select_workspace_bytes(int64_t K) {
  if (K <= 0) return -1;
  return cdiv(256 + cdiv(K, BSG_BLOCK_K) * 16, 256) * 256;
}

// Checks, then the score launch (into scores[ceil(K/64)], 8-byte aligned) and (rank) the top-k
// launch of the exact-L1 selector.
static int select_l1_check(const void* x, int64_t ldx, int64_t bt, int64_t K, int32_t k, const int32_t* idx_out,
                           const int32_t* na_out, int dtype) {
  if (dtype != BSG_F16)
    return fail(BSG_ERR_DTYPE, "select: exact L1 scoring is defined for fp16 inputs (dtype=%d)", dtype);
  if (bt <= 0 || K <= 0) return fail(BSG_ERR_ARG, "select: bt=%lld K=%lld", (long long)bt, (long long)K);
  const int64_t nblk = cdiv(K, BSG_BLOCK_K);
  if (nblk > BSG_MAX_NBLK) return fail(BSG_ERR_UNSUPPORTED, "select: K=%lld too large", (long long)K);
  if (k < 0) return fail(BSG_ERR_ARG, "select: k=%d", k);
  if (!x || !idx_out || !na_out) return fail(BSG_ERR_ARG, "select: null pointer");
  if (K % 8 != 0 || ldx < K || ldx % 8 != 0 || !aligned16(x))
    return fail(BSG_ERR_ALIGN, "select: x must be 16-byte aligned, K %% 8 == 0, ldx %% 8 == 0");
  if (bt * 8 > 0x7fffffff) return fail(BSG_ERR_UNSUPPORTED, "select: bt too large");
  return BSG_OK;
}

static int select_l1_run(const void* x, int64_t ldx, int64_t bt, int64_t K, int32_t k, int32_t* idx_out,
                         int32_t* na_out, int dtype, uint64_t* scores, void* stream, bool rank) {
  const int rc = select_l1_check(x, ldx, bt, K, k, idx_out, na_out, dtype);
  if (rc != BSG_OK) return rc;
  const int64_t nblk = cdiv(K, BSG_BLOCK_K);
  SelParams p;
  p.x = (const uint16_t*)x;
  p.ldx = ldx;
  p.scores = scores;
  p.idx_out = idx_out;
  p.na_out = na_out;
  p.bt = (int32_t)bt;
  p.K = (int32_t)K;
  p.nblk = (int32_t)nblk;
  p.k = k;
  hipLaunchKernelGGL(bsg_score_l1_kernel, dim3((unsigned)nblk), dim3(256), 0, (hipStream_t)stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "bsg_select_topk_l1 score launch");
  if (!rank) return BSG_OK;
  hipLaunchKernelGGL(bsg_rank_l1_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, p);
  e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "bsg_select_topk_l1 rank launch");
  return BSG_OK;
}

// The exact-L1 selector with its scores in a caller workspace (after a 256-byte header).
static int select_l1_launch(const void* x, int64_t ldx, int64_t bt, int64_t K, int32_t k, int32_t* idx_out,
                            int32_t* na_out, int dtype, void* ws, int64_t ws_bytes, void* stream, bool rank) {
  const int rc = select_l1_check(x, ldx, bt, K, k, idx_out, na_out, dtype);
  if (rc != BSG_OK) return rc;
  const int64_t need = bsg_select_workspace_bytes(K);
  if (!ws || ws_bytes < need || ((uintptr_t)ws & 7u) != 0)
    return fail(BSG_ERR_WORKSPACE, "select: workspace %lld bytes < %lld (8-byte aligned)", (long long)ws_bytes,
                (long long)need);
  return select_l1_run(x, ldx, bt, K, k, idx_out, na_out, dtype, (uint64_t*)((char*)ws + 256), stream, rank);
}

int bsg_select_topk_l1(const void* x, int64_t ldx, int64_t bt, int64_t K, int32_t k, int32_t* idx_out,
                       int32_t* na_out, int dtype, void* ws, int64_t ws_bytes, void* stream) {
  return select_l1_launch(x, ldx, bt, K, k, idx_out, na_out, dtype, ws, ws_bytes, stream, true);
}

}  // extern "C"

namespace {

const bsg_select_opts kSelectDefaults = {BSG_SCORE_L1, 0.f, nullptr, 1.f, 0.1f, nullptr, nullptr};

// Checks of a reference-rule selection (bsg_select_topk's arguments, score L2 mean or energy).
int select_rule_check(const void* x, int64_t ldx, int64_t bt, int64_t K, int32_t k, const bsg_select_opts& o,
                      int32_t* idx_out, int32_t* na_out, int dtype) {
  if (o.score != BSG_SCORE_L2_MEAN && o.score != BSG_SCORE_ENERGY)
    return fail(BSG_ERR_UNSUPPORTED, "select: score=%d (0 = L1, 1 = L2 mean, 2 = energy)", o.score);
  if (dtype != BSG_F16 && dtype != BSG_BF16) return fail(BSG_ERR_DTYPE, "select: dtype=%d", dtype);
  if (bt <= 0 || K < BSG_BLOCK_K)
    return fail(BSG_ERR_ARG, "select: bt=%lld K=%lld (scored blocks are floor(K/64) >= 1)", (long long)bt,
                (long long)K);
  if (cdiv(K, BSG_BLOCK_K) > BSG_MAX_NBLK) return fail(BSG_ERR_UNSUPPORTED, "select: K=%lld too large", (long long)K);
  if (k < 0) return fail(BSG_ERR_ARG, "select: k=%d", k);
  if (!(o.energy_keep >= 0.f && o.energy_keep <= 1.f))
    return fail(BSG_ERR_ARG, "select: energy_keep=%g outside [0, 1]", (double)o.energy_keep);
  if (o.channel_scale && o.score != BSG_SCORE_ENERGY)
    return fail(BSG_ERR_ARG, "select: channel_scale applies to the energy score only");
  if (!x || !idx_out || !na_out) return fail(BSG_ERR_ARG, "select: null pointer");
  if (K % 8 != 0 || ldx < K || ldx % 8 != 0 || !aligned16(x))
    return fail(BSG_ERR_ALIGN, "select: x must be 16-byte aligned, K %% 8 == 0, ldx %% 8 == 0");
  if (bt > (1 << 24)) return fail(BSG_ERR_UNSUPPORTED, "select: bt too large");
  return BSG_OK;
}

// Launches of a checked reference-rule selection: the score launch (order keys and energies of
// the ceil(K/64) blocks into the selector workspace sel_ws), then, when `rank`, the one-work-group
// rank launch (ids, count and ratio on the device).
int select_rule_run(const void* x, int64_t ldx, int64_t bt, int64_t K, int32_t k, const bsg_select_opts& o,
                    int32_t* idx_out, int32_t* na_out, int dtype, void* sel_ws, void* stream, bool rank) {
  SelScoreParams p;
  p.x = x;
  p.ldx = ldx;
  p.prior = o.block_prior;
  p.scale = o.channel_scale;
  p.keys = (uint64_t*)((char*)sel_ws + 256);
  p.energy = (double*)(p.keys + cdiv(K, BSG_BLOCK_K));
  p.idx_out = idx_out;
  p.na_out = na_out;
  p.ratio_out = o.ratio_out;
  p.alpha = o.prior_alpha;
  p.eps = o.prior_eps;
  p.energy_keep = o.energy_keep;
  p.bt = (int32_t)bt;
  p.K = (int32_t)K;
  p.nb = (int32_t)(K / BSG_BLOCK_K);
  p.k = k;
  p.mode = o.score;
  const dim3 grid((unsigned)cdiv(K, BSG_BLOCK_K));
  if (dtype == BSG_F16)
    hipLaunchKernelGGL(bsg_score_rule_kernel<_Float16>, grid, dim3(256), 0, (hipStream_t)stream, p);
  else
    hipLaunchKernelGGL(bsg_score_rule_kernel<__bf16>, grid, dim3(256), 0, (hipStream_t)stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "reference-rule score launch");
  if (!rank) return BSG_OK;
  hipLaunchKernelGGL(bsg_rank_rule_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, p);
  e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "reference-rule rank launch");
  return BSG_OK;
}

}  // namespace

extern "C" {

int bsg_select_topk(const void* x, int64_t ldx, int64_t bt, int64_t K, int32_t k, const bsg_select_opts* opts,
                    int32_t* idx_out, int32_t* na_out, int dtype, void* ws, int64_t ws_bytes, void* stream) {
  const bsg_select_opts o = opts ? *opts : kSelectDefaults;
  if (o.score == BSG_SCORE_L1) {
    if (o.energy_keep != 0.f || o.block_prior || o.channel_scale || o.ratio_out)
      return fail(BSG_ERR_UNSUPPORTED, "select: the exact L1 score takes no prior, scale or energy budget");
    return bsg_select_topk_l1(x, ldx, bt, K, k, idx_out, na_out, dtype, ws, ws_bytes, stream);
  }
  int rc = select_rule_check(x, ldx, bt, K, k, o, idx_out, na_out, dtype);
  if (rc != BSG_OK) return rc;
  const int64_t need = bsg_select_workspace_bytes(K);
  if (!ws || ws_bytes < need || ((uintptr_t)ws & 7u) != 0)
    return fail(BSG_ERR_WORKSPACE, "select: workspace %lld bytes < %lld (8-byte aligned)", (long long)ws_bytes,
                (long long)need);
  return select_rule_run(x, ldx, bt, K, k, o, idx_out, na_out, dtype, ws, stream, true);
}

int bsg_read_calibrate(const void* src, int64_t bytes, void* sink, void* stream) {
  if (!src || !sink || bytes < 1024 || bytes % 1024 != 0)
    return fail(BSG_ERR_ARG, "read_calibrate: bytes=%lld (a positive multiple of 1024) and non-null pointers",
                (long long)bytes);
  if (!aligned16(src)) return fail(BSG_ERR_ALIGN, "read_calibrate: src must be 16-byte aligned");
  const int64_t n1k = bytes / 1024;
  const int cu = device_cu_count();
  int64_t groups = 2 * (int64_t)cu;  // 8 waves per compute unit
  if (groups * 4 > n1k) groups = (n1k + 3) / 4;
  hipLaunchKernelGGL(bsg_read_kernel, dim3((unsigned)groups), dim3(256), 0, (hipStream_t)stream, (const char*)src,
                     n1k, 0x9E3779B9u, (uint32_t*)sink);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "bsg_read_calibrate launch");
  return BSG_OK;
}

// The body of bsg_select_gemm and of its allocation-free variant: exact-L1 scores into
// scores[ceil(K/64)], then the GEMM on the kept list, its split-K storage carved from
// gws/gws_bytes or, when fx.part_fixed is set, taken from fx.  Every argument and the GEMM's
// storage are checked before the first launch.
static int select_gemm_run(const void* x, int64_t ldx, int64_t bt, int64_t K, int32_t k, const void* wp,
                           int64_t N, int32_t* idx_out, int32_t* na_out, void* y, int64_t ldy, int dtype,
                           uint64_t* scores, void* gws, int64_t gws_bytes, const LaunchExtras& fx,
                           const bsg_plan* plan, void* stream) {
  const int64_t nblk = K > 0 ? cdiv(K, BSG_BLOCK_K) : 0;
  if (k < 0) return fail(BSG_ERR_ARG, "select_gemm: k=%d", k);
  if (bt <= 0 || N <= 0 || K <= 0 || nblk > BSG_MAX_NBLK)
    return fail(BSG_ERR_ARG, "select_gemm: bt=%lld N=%lld K=%lld", (long long)bt, (long long)N, (long long)K);
  int rc = check_common(x, ldx, bt, K, wp, N, y, ldy, dtype, N);
  if (rc != BSG_OK) return rc;
  if (!idx_out || !na_out) return fail(BSG_ERR_ARG, "select_gemm: null idx_out or na_out");
  bsg_plan pl = plan ? *plan : bsg_plan{0, 0, 0, 0, 0, 0};
  const int32_t kk = k < nblk ? k : (int32_t)nblk;
  rc = resolve(bt, N, (int32_t)nblk, kk, pl.split_k == 0 ? device_cu_count() : 256, &pl);
  if (rc != BSG_OK) return rc;
  const int64_t need = gemm_ws_bytes(bt, N, &pl);
  if (fx.part_fixed != nullptr) {
    if (need > 0 && (ws_max_tiles(bt, N, &pl) > fx.cnt_cap_tiles ||
                     need - ws_counter_bytes(bt, N, &pl) > fx.part_cap_bytes))
      return fail(BSG_ERR_WORKSPACE,
                  "select_gemm: split-K %d needs %lld tile counters and %lld bytes of partials; the static "
                  "scratch holds %lld counters and %lld bytes",
                  pl.split_k, (long long)ws_max_tiles(bt, N, &pl), (long long)(need - ws_counter_bytes(bt, N, &pl)),
                  (long long)fx.cnt_cap_tiles, (long long)fx.part_cap_bytes);
  } else if (need > 0 && (!gws || gws_bytes < need || !aligned16(gws))) {
    return fail(BSG_ERR_WORKSPACE, "select_gemm: GEMM workspace %lld bytes < %lld needed (split_k=%d)",
                (long long)gws_bytes, (long long)need, pl.split_k);
  }
  // The GEMM ranks the scores itself when every work-group can do it quickly: the nblk^2
  // compares, in items of 64 blocks x 16 scores, come to at most BSG_TOPK_ITEMS_PER_WAVE items per
  // wave (12: down's 172 blocks on a four-wave plan take 9, 2.49 vs 2.51 ms per decode step with
  // the rank launch that 8 forced).  Otherwise a
  // one-work-group rank launch (about 3 us) is cheaper than ranking in each work-group.
  const int64_t items = cdiv(nblk, 64) * cdiv(nblk, 16);
  const KernelEntry* ke = find_kernel(pl.kind, pl.rows_per_group, pl.cols_per_wave / 16, pl.waves_per_group, pl.depth);
  const bool rank_in_gemm = nblk <= BSG_TOPK_MAX_NBLK && ke != nullptr && ke->f16_sel != nullptr &&
                            items <= BSG_TOPK_ITEMS_PER_WAVE * (int64_t)pl.waves_per_group;
  if (rank_in_gemm && bt <= BSG_SELF_MAX_ROWS && bt * K * 2 <= BSG_SELF_SCORE_MAX_X_BYTES &&
      pl.rows_per_group == 16) {
    // One launch: every GEMM work-group scores the blocks from x itself, ranks them and walks
    // the kept list; no score buffer is written.
    rc = select_l1_check(x, ldx, bt, K, k, idx_out, na_out, dtype);
    if (rc != BSG_OK) return rc;
    LaunchExtras ex = fx;
    ex.idx_out = idx_out;
    ex.na_out = na_out;
    return launch_gemm(MODE_TOPK_SELF, x, ldx, bt, K, wp, N, nullptr, k, nullptr, nullptr, 0, y, ldy, dtype, gws,
                       gws_bytes, &pl, stream, ex);
  }
  if (rank_in_gemm) {
    // Two launches: the block scores, then the GEMM, whose work-groups each rank them and walk
    // the kept list (work-group (0, 0) also publishes it).
    rc = select_l1_run(x, ldx, bt, K, k, idx_out, na_out, dtype, scores, stream, false);
    if (rc != BSG_OK) return rc;
    LaunchExtras ex = fx;
    ex.scores = scores;
    ex.idx_out = idx_out;
    ex.na_out = na_out;
    return launch_gemm(MODE_TOPK, x, ldx, bt, K, wp, N, nullptr, k, nullptr, nullptr, 0, y, ldy, dtype, gws,
                       gws_bytes, &pl, stream, ex);
  }
  rc = select_l1_run(x, ldx, bt, K, k, idx_out, na_out, dtype, scores, stream, true);
  if (rc != BSG_OK) return rc;
  return launch_gemm(MODE_LIST, x, ldx, bt, K, wp, N, idx_out, kk, nullptr, nullptr, 0, y, ldy, dtype, gws,
                     gws_bytes, &pl, stream, fx);
}

int bsg_select_gemm(const void* x, int64_t ldx, int64_t bt, int64_t K, int32_t k, const void* wp, int64_t N,
                    int32_t* idx_out, int32_t* na_out, void* y, int64_t ldy, int dtype, void* ws, int64_t ws_bytes,
                    const bsg_plan* plan, void* stream) {
  const int64_t sel = bsg_select_workspace_bytes(K);
  if (sel < 0) return fail(BSG_ERR_ARG, "select_gemm: K=%lld", (long long)K);
  if (!ws || ws_bytes < sel || ((uintptr_t)ws & 15u) != 0)
    return fail(BSG_ERR_WORKSPACE, "select_gemm: workspace %lld bytes < the selector's %lld (16-byte aligned)",
                (long long)ws_bytes, (long long)sel);
  return select_gemm_run(x, ldx, bt, K, k, wp, N, idx_out, na_out, y, ldy, dtype, (uint64_t*)((char*)ws + 256),
                         (char*)ws + sel, ws_bytes - sel, LaunchExtras{}, plan, stream);
}

int bsg_select_gemm_rule(const void* x, int64_t ldx, int64_t bt, int64_t K, int32_t k, const bsg_select_opts* opts,
                         const void* wp, int64_t N, int32_t* idx_out, int32_t* na_out, void* y, int64_t ldy,
                         int dtype, void* ws, int64_t ws_bytes, const bsg_plan* plan, void* stream) {
  const bsg_select_opts o = opts ? *opts : kSelectDefaults;
  if (o.score == BSG_SCORE_L1) {
    if (o.energy_keep != 0.f || o.block_prior || o.channel_scale || o.ratio_out)
      return fail(BSG_ERR_UNSUPPORTED, "select_gemm: the exact L1 score takes no prior, scale or energy budget");
    return bsg_select_gemm(x, ldx, bt, K, k, wp, N, idx_out, na_out, y, ldy, dtype, ws, ws_bytes, plan, stream);
  }
  const int64_t sel = bsg_select_workspace_bytes(K);
  if (sel < 0) return fail(BSG_ERR_ARG, "select_gemm: K=%lld", (long long)K);
  if (!ws || ws_bytes < sel || ((uintptr_t)ws & 15u) != 0)
    return fail(BSG_ERR_WORKSPACE, "select_gemm: workspace %lld bytes < the selector's %lld (16-byte aligned)",
                (long long)ws_bytes, (long long)sel);
  int rc = select_rule_check(x, ldx, bt, K, k, o, idx_out, na_out, dtype);
  if (rc != BSG_OK) return rc;
  if (N <= 0) return fail(BSG_ERR_ARG, "select_gemm: N=%lld", (long long)N);
  rc = check_common(x, ldx, bt, K, wp, N, y, ldy, dtype, N);
  if (rc != BSG_OK) return rc;
  const int64_t nblk = cdiv(K, BSG_BLOCK_K);
  const int32_t nb = (int32_t)(K / BSG_BLOCK_K);
  // GEMM list capacity: every scored block may be kept under an energy budget, else min(k, nb)
  const int32_t cap = o.energy_keep > 0.f ? nb : (k < nb ? k : nb);
  bsg_plan pl = plan ? *plan : bsg_plan{0, 0, 0, 0, 0, 0};
  rc = resolve(bt, N, (int32_t)nblk, cap, pl.split_k == 0 ? device_cu_count() : 256, &pl);
  if (rc != BSG_OK) return rc;
  void* gws = (char*)ws + sel;
  const int64_t gws_bytes = ws_bytes - sel;
  const int64_t need = gemm_ws_bytes(bt, N, &pl);
  if (need > 0 && (gws_bytes < need || !aligned16(gws)))
    return fail(BSG_ERR_WORKSPACE, "select_gemm: GEMM workspace %lld bytes < %lld needed (split_k=%d)",
                (long long)gws_bytes, (long long)need, pl.split_k);
  // Without an energy budget or a ratio the kept set is the top min(k, nb) by key, which the GEMM's
  // work-groups rank themselves (as for the L1 rule, same limits); the budget's cumulative-energy
  // scan runs in the one-work-group rank launch.
  const int64_t items = cdiv(nblk, 64) * cdiv(nblk, 16);
  const KernelEntry* ke = find_kernel(pl.kind, pl.rows_per_group, pl.cols_per_wave / 16, pl.waves_per_group, pl.depth);
  const bool rank_in_gemm = o.energy_keep == 0.f && o.ratio_out == nullptr && dtype == BSG_F16 &&
                            nblk <= BSG_TOPK_MAX_NBLK && ke != nullptr && ke->f16_sel != nullptr &&
                            items <= BSG_TOPK_ITEMS_PER_WAVE * (int64_t)pl.waves_per_group;
  rc = select_rule_run(x, ldx, bt, K, k, o, idx_out, na_out, dtype, ws, stream, !rank_in_gemm);
  if (rc != BSG_OK) return rc;
  if (rank_in_gemm) {
    LaunchExtras ex;
    ex.scores = (const uint64_t*)((char*)ws + 256);
    ex.score_keyed = 0;
    ex.idx_out = idx_out;
    ex.na_out = na_out;
    return launch_gemm(MODE_TOPK, x, ldx, bt, K, wp, N, nullptr, cap, nullptr, nullptr, 0, y, ldy, dtype, gws,
                       gws_bytes, &pl, stream, ex);
  }
  return launch_gemm(MODE_LIST, x, ldx, bt, K, wp, N, idx_out, cap, na_out, nullptr, 0, y, ldy, dtype, gws,
                     gws_bytes, &pl, stream);
}

int bsg_select_gemm_noalloc(const void* x, int64_t ldx, int64_t bt, int64_t K, int32_t k, const void* wp,
                            int64_t N, int32_t* idx_out, int32_t* na_out, void* y, int64_t ldy, int dtype,
                            const bsg_plan* plan, void* stream) {
  char* base = nullptr;
  int rc = noalloc_scratch(&base, stream);
  if (rc != BSG_OK) return rc;
  LaunchExtras fx;
  fx.cnt_fixed = (uint32_t*)base;
  fx.cnt_cap_tiles = kScratchCntBytes / 4;
  fx.part_fixed = (float*)(base + kScratchPartOff);
  fx.part_cap_bytes = BSG_NOALLOC_SCRATCH_BYTES - kScratchPartOff;
  return select_gemm_run(x, ldx, bt, K, k, wp, N, idx_out, na_out, y, ldy, dtype,
                         (uint64_t*)(base + kScratchCntBytes), nullptr, 0, fx, plan, stream);
}

#ifdef BSG_TIMELINE
// Profiling build only (include/bsgemm_timeline.h): later GEMM launches record phase stamps into
// buf, `slots` launches of up to `slot_groups` work-groups each (8 uint64 per work-group), cycling.
// buf = NULL detaches.  Returns BSG_OK or BSG_ERR_ARG.
int bsg_timeline_attach(void* buf, int64_t slots, int64_t slot_groups) {
  if (buf != nullptr && (slots <= 0 || slot_groups <= 0 || ((uintptr_t)buf & 7u) != 0))
    return fail(BSG_ERR_ARG, "timeline: slots=%lld slot_groups=%lld", (long long)slots, (long long)slot_groups);
  g_tl_base = (uint64_t*)buf;
  g_tl_slots = buf ? slots : 0;
  g_tl_slot_groups = buf ? slot_groups : 0;
  g_tl_next = 0;
  return BSG_OK;
}
#else
int bsg_timeline_attach(void* buf, int64_t, int64_t) {
  if (buf == nullptr) return BSG_OK;
  return fail(BSG_ERR_UNSUPPORTED, "timeline: this is not the profiling build (libbsgemm_timeline.so)");
}
#endif

int64_t bsg_timeline_clock_khz(void) {
  int dev = 0, khz = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess) return -1;
  return khz;
}

}  // extern "C"
