/*
 * bsgemm.h — C ABI of the MI355X (gfx950) batch-shared 64-channel block-sparse GEMM.
 *
 *   Y[bt, N] = sum over active K-blocks j of  X[bt, 64j:64j+64] · W[64j:64j+64, N]
 *
 * One block mask (a list of active 64-channel K-blocks) is shared by every row of the
 * decode batch.  Inputs and output are fp16 or bf16, accumulation is fp32, indices int32.
 *
 * Conventions (all entry points):
 *   - Pointers are device pointers; `stream` is a hipStream_t passed as void* (0 = null stream).
 *   - Nothing here allocates device memory or synchronises the host: every call only enqueues
 *     kernels on `stream`, so every call is safe inside hipStreamBeginCapture/EndCapture.
 *   - Return value: BSG_OK (0) or a negative BSG_ERR_* code; bsg_last_error() gives a
 *     thread-local message for the last failing call on the calling thread.
 *   - Argument validation happens on the host before any HIP call, so an invalid call
 *     never launches a kernel.
 *
 * Packed weight layout ("tiled K-major"): for K-block j (64 rows of K), column tile t
 * (16 columns of N), k-half h, 8-row group g, column c, row e (k = 32h + 8g + e,
 * n = 16t + c) the element lives at
 *     j*64*Np + t*1024 + h*512 + g*128 + c*8 + e            (Np = N rounded up to 16)
 * so each K-block is one contiguous 128*Np-byte slab and each 16-column tile of it is a
 * contiguous 2 KiB run that one 64-lane dwordx4 load per k-half brings straight into
 * the A operand of v_mfma_f32_16x16x32_{f16,bf16}.  Rows k >= K and columns n >= N are 0.
 */
#ifndef BSGEMM_H
#define BSGEMM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BSG_BLOCK_K 64           /* channels per K-block (reference INDEX_BLOCK_META_SIZE) */
#define BSG_MAX_NBLK 2048        /* K <= 131072 */

enum bsg_dtype { BSG_F16 = 0, BSG_BF16 = 1 };

enum bsg_status {
  BSG_OK = 0,
  BSG_ERR_ARG = -1,         /* bad size, null pointer, inconsistent arguments */
  BSG_ERR_DTYPE = -2,       /* dtype not fp16/bf16 */
  BSG_ERR_WORKSPACE = -3,   /* workspace missing or smaller than *_workspace_bytes() */
  BSG_ERR_ALIGN = -4,       /* pointer or leading dimension not 16-byte aligned */
  BSG_ERR_UNSUPPORTED = -5, /* plan or shape outside what the kernels implement */
  BSG_ERR_HIP = -100        /* a HIP runtime call failed; see bsg_last_error() */
};

/* Launch plan of the GEMM.  A zero field means "choose automatically".
 *   split_k         : work-groups that share one output tile and split the active-block
 *                     list (fp32 partials + in-kernel deterministic reduction), >= 1
 *   cols_per_wave   : output columns per wavefront (kinds 1-4: 16, 32, 64 or 128); kinds 5-7:
 *                     the most columns one work-group may take (16 x its most subtiles)
 *   waves_per_group : wavefronts per work-group: 1, 2, 4 or 8
 *   depth           : K-blocks whose loads each wave keeps in flight: 1, 2, 4 or 8
 *   rows_per_group  : batch rows per work-group (16, 32 or 64; 1, 2, 4 or 8 for kind 3); bt
 *                     above it adds grid rows
 *   kind            : the kernel family.
 *     1  the waves of a work-group split its block list, each loading its own activation
 *        fragments; work-group columns = cols_per_wave.  Any split_k.
 *     2  the waves split the work-group's columns and share each block's activation tile
 *        through LDS; work-group columns = cols_per_wave * waves_per_group.  Any split_k.
 *     3  fp32 dot products instead of MFMA, for 1-8 rows; each wave stages the activations of
 *        its slice of the list in LDS once and the quads of lanes meet through DPP; work-group
 *        columns = cols_per_wave; split_k must be 1; runs only when a plan names it.
 *     4  as 2, with the waves split over columns and over the two 32-channel halves of every
 *        block (two waves per SIMD); work-group columns = cols_per_wave * waves_per_group / 2;
 *        waves_per_group 4 or 8.  Any split_k.
 *     5  variable-width column groups: the ceil(N/16) 16-column subtiles are dealt as evenly as
 *        possible over G = min(ceil(N/16), max(CUs / row groups, ceil(N / cols_per_wave)))
 *        work-groups per row group, so a group takes at most cols_per_wave columns and any N
 *        fills every compute unit without split-K.  Waves = 32-channel half x block slice
 *        (waves_per_group even: waves_per_group / 2 slices of the list); every weight and
 *        activation byte of a group is loaded by one wave, straight into registers, and the
 *        waves meet in LDS once at the end.  split_k must be 1 (0 resolves to 1).
 *     6  as 5, with the waves splitting the block list only (waves_per_group slices), each
 *        loading both channel halves of its blocks.  split_k must be 1.
 *     7  as 6, with each block's activations loaded into the wave's own LDS slot (16 rows x 64
 *        contiguous bytes per load) and read back in MFMA order instead of loaded into
 *        registers; the registers this frees allow four block-slice waves at 64 rows.
 *        split_k must be 1.
 *   Kinds 5-7 run 1-D lists only (bsg_gemm_2d rejects them), and only the tiles compiled
 *   into the library resolve (BSG_ERR_UNSUPPORTED names any other); a zero field of a kind 5-7
 *   plan takes rows 16/32/64 from bt, cols_per_wave 48, waves_per_group 4, depth 4.
 * kind 0 here resolves by heuristic to kind 1 (bt <= 16) or kind 2 (larger bt).  The Python
 * layer does not rely on it: its plans come from a table tuned on the MI355X
 * (bsa_mi355x/tuned_plans.json) whose entries name kinds 1, 2, 4, 5, 6 and 7, or from
 * first-call tuning of problems the table does not hold.
 * Maps onto the reference's Triton tile (BLOCK_B, BLOCK_N, num_warps, num_stages) and
 * split-K factor (shared_mask_batched_triton_min_runtime.py:1296-1299, 1350-1361). */
typedef struct bsg_plan {
  int32_t split_k;
  int32_t cols_per_wave;
  int32_t waves_per_group;
  int32_t depth;
  int32_t rows_per_group;
  int32_t kind;
} bsg_plan;

/* Library identification and thread-local error message. */
const char* bsg_version(void);
const char* bsg_last_error(void);

/* Bytes of the packed weight for a logical W[N,K]. */
int64_t bsg_packed_bytes(int64_t N, int64_t K, int dtype);

/* Pack W into the tiled K-major layout.  W is addressed as W[n][k] = w[n*stride_n + k*stride_k]
 * (nn.Linear [N,K]: stride_n=K, stride_k=1; a [K,N] matrix: stride_n=1, stride_k=N).
 * Replaces _get_prepacked_weight_block_major
 * (kernels/shared_mask_batched_triton_min_runtime.py:3133-3163), which builds
 * pad(W^T).view(nblk, 64, N); the cache around it stays in the host layer. */
int bsg_pack_weight(const void* w, int64_t N, int64_t K, int64_t stride_n, int64_t stride_k,
                    int dtype, void* wp, int64_t wp_bytes, void* stream);

/* Resolve a plan: fills every zero field of *plan for this problem (bt rows, N columns,
 * nblk = ceil(K/64) blocks, na active blocks) on a device with cu_count compute units.
 * Validates non-zero fields.  Host-only; no HIP call. */
int bsg_plan_resolve(int64_t bt, int64_t N, int32_t nblk, int32_t na, int32_t cu_count,
                     bsg_plan* plan);

/* Workspace bytes the GEMM needs for this resolved plan (0 when split_k == 1).
 * The workspace holds fp32 partials and per-tile arrival counters; the counter region
 * must be zero before first use (bsg_workspace_init) and every GEMM leaves it zero. */
int64_t bsg_gemm_workspace_bytes(int64_t bt, int64_t N, const bsg_plan* plan);
int bsg_workspace_init(void* ws, int64_t ws_bytes, void* stream);

/* Block-sparse GEMM from an active-block index list.
 *   x            : [bt, K] activations, row stride ldx (elements); K % 8 == 0, ldx % 8 == 0,
 *                  16-byte aligned base
 *   wp           : packed weight from bsg_pack_weight(N, K)
 *   active_blocks: int32 list of K-block ids, length num_active (host count) — or, when
 *                  num_active_dev != NULL, length *num_active_dev read on the device
 *                  (capacity num_active, which bounds the device count)
 *                  ids outside [0, ceil(K/64)) contribute nothing
 *   y            : [bt, N] output, row stride ldy (elements); written, never read
 * num_active == 0 (host count) writes zeros, like the reference's out.zero_().
 * Replaces, with one kernel family:
 *   _prepacked_block_sparse_gemm_from_active_blocks      (…min_runtime.py:3166-3344)
 *   _prepacked_block_sparse_gemm_from_active_blocks_splitk (…min_runtime.py:1350-1454)
 *   prepacked_block_sparse_gemm_batched_kernel / _splitk_write_kernel / _splitk_reduce_kernel
 *                                                          (…min_runtime.py:684-733, 1898-1988) */
int bsg_gemm(const void* x, int64_t ldx, int64_t bt, int64_t K,
             const void* wp, int64_t N,
             const int32_t* active_blocks, int32_t num_active, const int32_t* num_active_dev,
             void* y, int64_t ldy, int dtype,
             void* ws, int64_t ws_bytes, const bsg_plan* plan, void* stream);

/* bsg_gemm with the list sorted ascending inside the GEMM's own list staging (no separate sort
 * launch): the same arguments, the same result as an ascending sort of the list followed by
 * bsg_gemm, bit for bit.  With num_active_dev the count is applied first: only the first
 * min(*num_active_dev, num_active) entries are sorted and used, so the result is bsg_gemm on
 * sort(active_blocks[0 .. count)), not on the count smallest ids of the whole list.
 * num_active <= BSG_MAX_NBLK / 2 (else BSG_ERR_UNSUPPORTED).
 * Replaces the sort + GEMM pair of _prepacked_block_sparse_gemm_from_active_blocks with
 * sort_active_blocks=True: _sort_active_blocks_asc (…min_runtime.py:140-163, called at
 * :3193-3194) followed by prepacked_block_sparse_gemm_batched_kernel (…min_runtime.py:684-733). */
int bsg_gemm_sorted(const void* x, int64_t ldx, int64_t bt, int64_t K,
                    const void* wp, int64_t N,
                    const int32_t* active_blocks, int32_t num_active, const int32_t* num_active_dev,
                    void* y, int64_t ldy, int dtype,
                    void* ws, int64_t ws_bytes, const bsg_plan* plan, void* stream);

/* Same GEMM driven by a u8 bitmap[total_k_blocks] (non-zero = active; 1 <= total_k_blocks <=
 * ceil(K/64), later blocks count as inactive), compacted on the
 * device into ascending block order; the block list never leaves the GPU.
 * Replaces _prepacked_block_sparse_gemm_from_active_blocks_bitmap_preload(_splitk) and
 * prepacked_block_sparse_gemm_bitmap_preload_batched_kernel / _splitk_kernel
 * (…min_runtime.py:814-874, 1064-1147, 1150-1216, 1235-1347). */
int bsg_gemm_bitmap(const void* x, int64_t ldx, int64_t bt, int64_t K,
                    const void* wp, int64_t N,
                    const uint8_t* bitmap, int32_t total_k_blocks,
                    void* y, int64_t ldy, int dtype,
                    void* ws, int64_t ws_bytes, const bsg_plan* plan, void* stream);

/* The same kernel with every K-block active: the in-run dense baseline.  Stands in for the
 * reference's dense torch.mm(x, W^T) (scripts/bench_perstep_actual_kernel_speedup.py:162,
 * scripts/profile_kernel_configs.py:229). */
int bsg_gemm_dense(const void* x, int64_t ldx, int64_t bt, int64_t K,
                   const void* wp, int64_t N,
                   void* y, int64_t ldy, int dtype,
                   void* ws, int64_t ws_bytes, const bsg_plan* plan, void* stream);

/* 2-D sparsity: only the active 64-column output blocks n_blocks[num_n] (device, ascending
 * expected, block b = columns 64b .. 64b+63) are computed.  K-blocks as bsg_gemm
 * (active_blocks[num_active], num_active_dev), or every K-block when both are NULL.
 *   compact = 0 : Y [bt, N]; only the active blocks' columns are written, the rest untouched
 *   compact = 1 : Y [bt, num_n * 64] (ldy >= num_n * 64); list entry i at columns 64i .. 64i+63,
 *                 columns past N inside a block hold zeros
 * num_n_dev (device, nullable) shortens the list below num_n with no host round trip; the
 * tiles past it write nothing.  A block id outside [0, ceil(N/64)) reads no weights and writes
 * nothing in place (zeros when compact).  num_n = 0 writes nothing.  The plan must cover at
 * most 64 columns per work-group (cols_per_wave x column waves).  Workspace as bsg_gemm.
 * Replaces _prepacked_block_sparse_gemm_2d_from_active_blocks (KRN:3498-3850) with its
 * in-place (KRN:2289-2384) and compact (KRN:2473-2557) kernels. */
int bsg_gemm_2d(const void* x, int64_t ldx, int64_t bt, int64_t K, const void* wp, int64_t N,
                const int32_t* active_blocks, int32_t num_active, const int32_t* num_active_dev,
                const int32_t* n_blocks, int32_t num_n, const int32_t* num_n_dev, int compact,
                void* y, int64_t ldy, int dtype,
                void* ws, int64_t ws_bytes, const bsg_plan* plan, void* stream);

/* Scatter a compact 2-D output back to the dense N axis:
 * out[r, 64 n_blocks[i] + c] = compact[r, 64 i + c] for c < 64 and 64 n_blocks[i] + c < N,
 * i < num_n (or *num_n_dev when set); other columns of out are untouched.  16-bit elements.
 * Replaces _scatter_compact_to_dense_output (KRN:3470-3495), which loops on the host. */
int bsg_scatter_nblocks(const void* compact, int64_t ldc, int64_t bt, const int32_t* n_blocks, int32_t num_n,
                        const int32_t* num_n_dev, int64_t N, void* out, int64_t ldo, void* stream);

/* Active 64-column output blocks of an element mask over N: the blocks b < ceil(N/64) with any
 * mask[64b .. 64b+63] != 0, ascending, into n_blocks_out (room for ceil(N/64)), and their count
 * into *num_out, both on the device.  Replaces the block-count state of
 * _get_cached_active_n_blocks_delta (KRN:453-495); recomputed per call, so there is no delta
 * state to keep. */
int bsg_nmask_blocks(const uint8_t* mask, int64_t N, int32_t* n_blocks_out, int32_t* num_out, void* stream);

/* Online block selector: score_j = sum_b sum_{c in block j} |x[b, 64j+c]| computed exactly
 * (integer units of 2^-24), top-k by (score desc, block id asc), compacted to an ascending
 * int32 list idx_out[min(k, nblk)] with the count written to *na_out (device).  Two launches
 * on `stream` (block scores, then a one-work-group top-k); the mask never round-trips to the
 * host.  The workspace needs no initialisation.  Replaces the torch op chain of
 * _select_active_blocks (scripts/bench_roundrobin_e2e_decode.py:90-113) with the L1 rule. */
int64_t bsg_select_workspace_bytes(int64_t K);
int bsg_select_topk_l1(const void* x, int64_t ldx, int64_t bt, int64_t K, int32_t k,
                       int32_t* idx_out, int32_t* na_out, int dtype,
                       void* ws, int64_t ws_bytes, void* stream);

/* Selector with the reference's own scoring rules (scripts/bench_roundrobin_e2e_decode.py,
 * RRD:90-176), computed in fp64.  Scored blocks are floor(K/64), as there.
 *   score         : BSG_SCORE_L2_MEAN  mean over rows of the block's L2 norm   (RRD:100)
 *                   BSG_SCORE_ENERGY   mean over rows of sum x^2 [* channel_scale]  (RRD:103-105)
 *                   BSG_SCORE_L1       the exact L1 rule of bsg_select_topk_l1 (no other option)
 *   block_prior   : score *= max(prior + prior_eps, 1e-6)^prior_alpha            (RRD:106-112)
 *   energy_keep   : > 0 keeps more than k blocks, up to the first rank whose cumulative
 *                   energy (unscaled, in score order) reaches energy_keep of the total; idx_out
 *                   then needs room for floor(K/64) entries                     (RRD:155-176)
 *   ratio_out     : kept energy fraction (float, device), as RRD:141 / RRD:176 return it
 * Ranking is (score desc, block id asc), on the fp64 scores: -0 ties with +0, and a NaN score
 * ranks above every number (as torch.topk ranks NaN).  idx_out holds the kept ids ascending and
 * *na_out their count, both on the device.  Workspace as bsg_select_topk_l1.  Replaces
 * _select_active_blocks (RRD:90-113), _topk_energy_ratio (RRD:116-141) and
 * _energy_expanded_active_blocks (RRD:144-176). */
enum bsg_score { BSG_SCORE_L1 = 0, BSG_SCORE_L2_MEAN = 1, BSG_SCORE_ENERGY = 2 };
typedef struct bsg_select_opts {
  int32_t score;
  float energy_keep;
  const float* block_prior;
  float prior_alpha;
  float prior_eps;
  const float* channel_scale;
  float* ratio_out;
} bsg_select_opts;
int bsg_select_topk(const void* x, int64_t ldx, int64_t bt, int64_t K, int32_t k, const bsg_select_opts* opts,
                    int32_t* idx_out, int32_t* na_out, int dtype, void* ws, int64_t ws_bytes, void* stream);

/* Selector followed by the GEMM on its device-side list, both on `stream`; idx_out and
 * *na_out receive the kept list and count as from bsg_select_topk_l1.  Where the plan's waves
 * can rank the scores quickly (an MFMA kind, nblk <= 512 and at most 12 items of 64 blocks x 16
 * scores per wave) every GEMM work-group ranks them itself and the call is two launches (scores, GEMM);
 * at small batches (bt <= 8 and bt x K x 2 <= 24 KiB, MFMA kinds) every GEMM work-group also
 * computes the scores from x itself and the call is one launch; otherwise three (scores,
 * top-k, GEMM).  The selection is the same in every form.  ws is split: the first bsg_select_workspace_bytes(K)
 * bytes for the selector, the rest (bsg_gemm_workspace_bytes) for the GEMM.  Replaces the
 * select -> bitmap -> GEMM sequence of _sparse_linear
 * (scripts/bench_roundrobin_e2e_decode.py:179-284). */
int bsg_select_gemm(const void* x, int64_t ldx, int64_t bt, int64_t K, int32_t k,
                    const void* wp, int64_t N, int32_t* idx_out, int32_t* na_out,
                    void* y, int64_t ldy, int dtype,
                    void* ws, int64_t ws_bytes, const bsg_plan* plan, void* stream);

/* Selection by the reference's own rules (bsg_select_opts, as bsg_select_topk) followed by the
 * GEMM on the kept blocks, both on `stream`, with no host round trip: the decode linear of
 * _sparse_linear (scripts/bench_roundrobin_e2e_decode.py:179-284), whose selection is
 * _select_active_blocks (RRD:90-113), or _energy_expanded_active_blocks (RRD:144-176) with an
 * energy budget.  idx_out, *na_out and ratio_out receive exactly what bsg_select_topk gives for
 * the same x and opts (idx_out needs room for floor(K/64) ids under an energy budget, min(k,
 * floor(K/64)) otherwise).  Two launches (fp64 order keys of the block scores, then the GEMM,
 * whose work-groups rank the keys themselves) when there is no energy budget, no ratio_out, the
 * dtype is fp16 and the plan's waves can rank the blocks (as bsg_select_gemm); otherwise three
 * (scores, one-work-group rank, GEMM on the device count).  opts->score == BSG_SCORE_L1 is
 * bsg_select_gemm.  Workspace as bsg_select_gemm: bsg_select_workspace_bytes(K) bytes for the
 * selector, then the GEMM's. */
int bsg_select_gemm_rule(const void* x, int64_t ldx, int64_t bt, int64_t K, int32_t k, const bsg_select_opts* opts,
                         const void* wp, int64_t N, int32_t* idx_out, int32_t* na_out, void* y, int64_t ldy,
                         int dtype, void* ws, int64_t ws_bytes, const bsg_plan* plan, void* stream);

/* Allocation-free variant of bsg_select_gemm.  It has no counterpart in the reference: it is for
 * callers that cannot allocate or hand over device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  Same arguments, selection, kernels and results
 * as bsg_select_gemm, without the workspace: the selector's block scores and the GEMM's split-K
 * counters and partials live in a library-owned static device array of
 * BSG_NOALLOC_SCRATCH_BYTES on each GPU it runs on (held until the process ends).  Layout: 64 KiB
 * of tile arrival counters, 16 KiB of block scores, the rest for partials.  A call whose plan
 * needs more partials or counters than that returns BSG_ERR_WORKSPACE before any launch.  The
 * first call on a device looks the array up and clears its counters (a kernel on `stream`; when
 * that first call is made under stream capture, the lookup runs in the relaxed capture mode and
 * the clear is recorded into the graph, so it runs at the start of every replay).
 * Nothing is allocated and no allocating library routine is called.  Every call on one GPU shares
 * that GPU's array, so calls that overlap on one GPU (concurrent streams, or host threads) race
 * and must be serialised by the caller. */
#define BSG_NOALLOC_SCRATCH_BYTES (16 * 1024 * 1024)
int bsg_select_gemm_noalloc(const void* x, int64_t ldx, int64_t bt, int64_t K, int32_t k,
                            const void* wp, int64_t N, int32_t* idx_out, int32_t* na_out,
                            void* y, int64_t ldy, int dtype, const bsg_plan* plan, void* stream);

/* Read-rate calibration; no counterpart in the reference.  Streams `bytes` (a multiple of
 * 1024) from src with the GEMM's weight-load pattern (non-temporal 1 KiB wave loads, 8 waves
 * per compute unit) and writes sink[0] only if the data folds to a fixed constant.  Its
 * duration is the practical HBM read time of a launch of that size, the context for a
 * GEMM's fraction of the 8 TB/s peak. */
int bsg_read_calibrate(const void* src, int64_t bytes, void* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* BSGEMM_H */
