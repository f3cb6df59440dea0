/*
 * cce_mi355x.h — C ABI of the MI355X (gfx950) Cut Cross-Entropy library.
 *
 * loss_r = lse(E_r . C^T + b) - (E_r . C_{t_r} + b_{t_r}), computed without ever
 * materialising the [N, V] logits.  Every entry point is asynchronous on the
 * caller's HIP stream, never allocates, never synchronises, and returns 0 on
 * success or a negative CCE_ERR_* code (message via cce_last_error()).
 * No exception crosses this boundary.
 *
 * Layouts (all row-major, contiguous, 16-byte aligned base pointers):
 *   e        [N, D]   dtype                 hidden states (the reference's "e")
 *   c        [V, D]   dtype                 classifier rows (the reference's "c")
 *   bias     [V]      dtype, nullable
 *   targets  [N]      int64; rows equal to ignore_index (when has_ignore != 0) are masked
 *   tile_max, tile_sum_exp  [num_vocab_tiles, N] fp32, vocab-tile major, tile width
 *                      CCE_STAT_TILE (128) columns; num_vocab_tiles = ceil(V / 128)
 *   neg_target_logit, lse, nll   [N] fp32
 *
 * Reference boundary replaced (sb1992/mlx-cross-entropy):
 *   csrc/bindings.cpp:12-87 (nanobind module mlx_cce._ext) and the MLX primitives
 *   CutCrossEntropy / CutCrossEntropyBwd in csrc/cce/cce.h:37-101, cce.cpp:31-454.
 */
#ifndef CCE_MI355X_H
#define CCE_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes (reference accepts float32 / float16 / bfloat16: csrc/cce/cce.cpp:222-227) */
#define CCE_DTYPE_F32 0
#define CCE_DTYPE_F16 1
#define CCE_DTYPE_BF16 2

/* error codes */
#define CCE_OK 0
#define CCE_ERR_INVALID_ARGUMENT (-1) /* reference: std::invalid_argument, cce.cpp:41-73 */
#define CCE_ERR_UNSUPPORTED_DTYPE (-2) /* reference: runtime_error "unsupported dtype", cce.cpp:226 */
#define CCE_ERR_WORKSPACE (-3)        /* workspace missing or smaller than cce_backward_workspace_size() */
#define CCE_ERR_LAUNCH (-4)           /* a HIP launch failed */
#define CCE_ERR_NO_DEVICE (-5)        /* no HIP device (reference: eval_cpu throws, cce.cpp:185-199) */

/* Width (vocabulary columns) of one tile_max / tile_sum_exp statistic and of
 * the backward filter tile.  Reference uses 32 (cce.metal:34, cce.cpp:76). */
#define CCE_STAT_TILE 128
/* Token rows per backward tile (reference: 32, cce.metal:168). */
#define CCE_BWD_ROWS 128

/* ln(2^-12): the reference's gradient-filter threshold FILTER_LOG_EPS
 * (csrc/cce/cce.metal:143, reference/_fused_backward.py:17). */
#define CCE_FILTER_LOG_EPS (-8.3177661667f)

/* Message describing the last error returned on this thread ("" if none). */
const char* cce_last_error(void);

/* Library version string. */
const char* cce_version(void);

/* Tile geometry compiled into the library: forward workgroup tile (tokens x vocab),
 * statistic tile width, backward tile (tokens x vocab). Any pointer may be NULL. */
void cce_tile_config(int* fwd_tokens, int* fwd_vocab, int* stat_tile, int* bwd_tokens, int* bwd_vocab);

/* Number of vocabulary statistic tiles: ceil(V / CCE_STAT_TILE). */
int64_t cce_num_vocab_tiles(int64_t V);

/* The reference's statistic tile (32 columns) and the number of them: ceil(V / 32). */
#define CCE_REF_STAT_TILE 32
int64_t cce_num_ref_tiles(int64_t V);

/*
 * Forward pass.  Replaces cce_forward_raw (csrc/bindings.cpp:58-69, cce.cpp:123-145)
 * and CutCrossEntropy::eval_gpu (cce.cpp:207-277): one fused tiled-MFMA kernel that
 * writes per-(vocab tile, row) max and sum-exp plus the target logit, then one
 * combine kernel (reference reduce_tile_to_lse, cce.metal:332-355) that writes
 *   lse[r] = logsumexp_v(E_r . C_v + b_v)
 *   nll[r] = lse[r] + neg_target_logit[r]     for rows kept by the ignore mask,
 *            0                                for masked rows (mlx_cce/__init__.py:59-70),
 *            NaN                              for kept rows whose target is outside [0, V).
 * tile_sum_exp is required (it is the combine kernel's input).  neg_target_logit[r] is
 * written only for rows whose target lies in [0, V); other entries keep what the buffer
 * held, as the reference's kernel leaves them (cce.metal:108-114 writes it only where
 * the target falls in the tile).
 */
int cce_forward(int dtype, const void* e, const void* c, const void* bias,
                const int64_t* targets, int64_t ignore_index, int has_ignore,
                int64_t N, int64_t D, int64_t V,
                float* tile_max, float* tile_sum_exp, float* neg_target_logit,
                float* lse, float* nll, void* hip_stream);

/*
 * As cce_forward, and also fills zero_bytes bytes at zero_buf with zeros, spread over
 * the tile kernel's work (that kernel is MFMA-bound and leaves HBM write bandwidth
 * idle).  For the dC buffer a later cce_backward_ex(..., CCE_BWD_DC_ZEROED) writes:
 * that backward then writes only the dC rows of vocabulary tiles with kept tiles.
 * zero_buf must be 16-byte aligned and zero_bytes a multiple of 16 (NULL / 0: none).
 * Replaces the same reference interfaces as cce_forward; the zero fill stands in for
 * the zero fill of the outputs the reference's backward accumulates into
 * (csrc/cce/cce.cpp:315-327 fill_zero_f32; reference/_fused_backward.py:1649 init_value=0.0).
 */
int cce_forward_ex(int dtype, const void* e, const void* c, const void* bias,
                   const int64_t* targets, int64_t ignore_index, int has_ignore,
                   int64_t N, int64_t D, int64_t V,
                   float* tile_max, float* tile_sum_exp, float* neg_target_logit,
                   float* lse, float* nll, void* zero_buf, int64_t zero_bytes, void* hip_stream);

/*
 * As cce_forward, with tile_max and tile_sum_exp in the reference's layout: per 32
 * vocabulary columns, flat [N * ceil(V/32)], row major per row of e -- what
 * cce_forward_raw returns in the reference (csrc/bindings.cpp:58-69, cce.cpp:123-145)
 * and its glue reshapes to (B, (V + 31) // 32) (mlx_cce/__init__.py:25-30).  lse and
 * nll are merged from those tiles (reference reduce_tile_to_lse, cce.metal:332-355).
 * A later cce_backward_ex(..., CCE_BWD_REF_STATS) takes this tile_max as it is.
 */
int cce_forward_ref(int dtype, const void* e, const void* c, const void* bias,
                    const int64_t* targets, int64_t ignore_index, int has_ignore,
                    int64_t N, int64_t D, int64_t V,
                    float* tile_max, float* tile_sum_exp, float* neg_target_logit,
                    float* lse, float* nll, void* hip_stream);

/*
 * Bytes of the default device workspace of cce_backward for these sizes and outputs.
 * The backward holds the G tiles of the kept (128-row, 128-column) pairs in passes of
 * a bounded size (8192 tiles by default, at least 2 tiles per 128-row block; a tile
 * takes 64 KiB, 512 MiB in all): the workspace is O(budget + N*D + V), never O(N*V).
 * The size is enough for every filter and flag; cce_backward_workspace_size_flags
 * gives the smaller one of a 16-bit backward with the filter on.  Reference interface
 * replaced: the output-sized accumulators of cce.cpp:315-340 (zero_alloc dE / dC).
 */
size_t cce_backward_workspace_size(int dtype, int64_t N, int64_t D, int64_t V,
                                   int want_dE, int want_dC, int want_dBias);

/*
 * As cce_backward_workspace_size, for passes of at most max_g_tiles G tiles (0: the
 * default budget; values below 2 tiles per 128-row block are raised to that, values
 * above the default are lowered to it) and vocabulary chunks of at most
 * max_chunk_tiles 128-column tiles (0: the library's choice; else a multiple of 32).
 * A cce_backward_ex given a workspace of this size and the same max_chunk_tiles runs
 * exactly these passes when its G tiles take 64 KiB (fp32, or the filter off), larger
 * ones when they take 32 KiB.  Same reference interface as above.
 */
size_t cce_backward_workspace_size_ex(int dtype, int64_t N, int64_t D, int64_t V,
                                      int want_dE, int want_dC, int want_dBias, int64_t max_g_tiles,
                                      int64_t max_chunk_tiles);

/*
 * As cce_backward_workspace_size_ex, for a cce_backward_ex with this filter_log_eps
 * and these flags.  They fix the G tiles' layout: 16-bit G rounded once (the filter
 * on, or CCE_BWD_G_SINGLE) takes 32 KiB a tile instead of the hi / lo pair's 64 KiB,
 * so the same passes need half the G bytes (256 MiB by default).  A cce_backward_ex
 * given a workspace of this size and the same filter_log_eps, flags and
 * max_chunk_tiles runs exactly these passes.  0 for a NaN filter_log_eps or invalid
 * flags.  Same reference interface as above.
 */
size_t cce_backward_workspace_size_flags(int dtype, int64_t N, int64_t D, int64_t V,
                                         int want_dE, int want_dC, int want_dBias, int64_t max_g_tiles,
                                         int64_t max_chunk_tiles, float filter_log_eps, int flags);

/*
 * Backward pass.  Replaces cce_backward_raw (csrc/bindings.cpp:71-86, cce.cpp:152-179),
 * CutCrossEntropyBwd::eval_gpu (cce.cpp:283-375) and the full-gradient research
 * kernel (reference/_fused_backward.py:1406-1655), whose dC/dBias semantics it follows.
 *   G[r,v] = d_nll[r] * (softmax(E_r . C^T + b)[v] - [v == t_r])
 *   dE = G . C,  dC = G^T . E,  dBias = sum_r G[r, :]
 * A (128-row, 128-column) tile is skipped when no row in it with d_nll != 0 has its
 * target inside the tile and every row's tile_max - lse < filter_log_eps
 * (reference predicate: cce.metal:191-204).  filter_log_eps = -INFINITY keeps all tiles.
 * dE/dC/dBias are written in `dtype`; pass NULL for any gradient not wanted.
 * No atomics: kept tiles' G blocks are staged (bf16/fp16/fp32, the input dtype) in
 * the workspace, one pass of a bounded number of them at a time, then every output
 * row block is summed in fp32 registers by the one workgroup that owns it and written
 * once (dE through an fp32 carry in the workspace when the kept tiles take more than
 * one pass).  Every output element is written, so the outputs need no zero-fill.
 * Rows of dE/dC/dBias that no kept tile touches are 0.
 * The plan depends only on the sizes, the outputs asked for, the G tiles' layout
 * (filter_log_eps and the G flags) and workspace_bytes: the default plan when the
 * workspace holds cce_backward_workspace_size_flags() bytes (which
 * cce_backward_workspace_size() always covers), else smaller passes
 * (CCE_ERR_WORKSPACE below the least size).
 * The workspace must stay untouched until the backward's work on the stream ends.
 * tile_stats (nullable, device int64[3]) receives {kept tiles, total tiles, kept tiles
 * of the input-order token blocks}.  The backward may form its 128-row token blocks
 * from the rows sorted by the vocabulary tile of their target (when that keeps at
 * least 10% fewer tiles); the first entry counts the blocks it used.
 */
int cce_backward(int dtype, const void* e, const void* c, const void* bias,
                 const int64_t* targets, int64_t ignore_index, int has_ignore,
                 int64_t N, int64_t D, int64_t V,
                 const float* lse, const float* tile_max, const float* d_nll,
                 float filter_log_eps,
                 void* dE, void* dC, void* dBias,
                 void* workspace, size_t workspace_bytes,
                 int64_t* tile_stats, void* hip_stream);

/* Flags of cce_backward_ex. */
#define CCE_BWD_DC_ZEROED 1       /* dC already holds zeros (e.g. from cce_forward_ex) */
/* Overrides of choices the backward otherwise makes itself (for tests and tuning;
 * results agree to rounding either way): */
#define CCE_BWD_TOKENS_INPUT 2    /* token blocks of 128 rows in input order */
#define CCE_BWD_TOKENS_SORTED 4   /* token blocks of the rows grouped by target tile, when available */
#define CCE_BWD_DE_SUMS_WIDE 8    /* dE sums in 512-column tasks */
#define CCE_BWD_DE_SUMS_NARROW 16 /* dE sums in 256-column tasks */
#define CCE_BWD_DC_SUMS_WIDE 32   /* dC sums in 512-column tasks */
#define CCE_BWD_DC_SUMS_NARROW 64 /* dC sums in 256-column tasks */
/* tile_max is in the reference's layout (cce_forward_ref: per 32 columns, [N][ceil(V/32)]);
 * the filter takes each 128-column tile's max as the max of its four 32-column maxima. */
#define CCE_BWD_REF_STATS 128
/* Launch the passes of the dense worst case and let the device skip the ones the data
 * does not need, instead of waiting on the host, once per vocabulary chunk, for the
 * compaction's pass count (which then launches exactly the passes needed).  The wait
 * is skipped anyway while the stream is being captured into a graph, and by
 * cce_backward_noalloc. */
#define CCE_BWD_DEVICE_PASSES 256
/* Precision of the softmax gradient G between the backward's two products (16-bit
 * inputs; fp32 inputs keep G in fp32).  By default G is carried as a pair of 16-bit
 * values (hi + lo, fp32-accurate: the reference keeps it in fp32 through both
 * products) when the filter is disabled, and rounded once to the input dtype when it
 * is on (the filter's own tolerance is 2e-2; the rounding adds about 2e-3).  These
 * force one or the other. */
#define CCE_BWD_G_PAIR 512
#define CCE_BWD_G_SINGLE 1024
/* The narrow dC sums (16-bit inputs, G rounded once) run the owners with one kept
 * tile as tasks per (token block, D slice): the block's E slice is loaded once and
 * the G tiles of its one-tile owners are streamed through it.  This runs every owner
 * as its own task instead (the results are the same bit for bit). */
#define CCE_BWD_DC_OWNER_TASKS 2048
/* With the filter on and the kept tiles shared by three or more token blocks on
 * average, the G kernel's tasks are a vocabulary tile with up to 4 of its kept blocks
 * (the tile's C rows read once for them), not a token block with up to 4 of its kept
 * tiles.  This keeps the token-block tasks (the G values can differ in the last bits:
 * the contraction's slices are summed in another order). */
#define CCE_BWD_G_TASKS_BY_BLOCK 4096
/* When a pass has at most half as many (128-row block, 256-column D slice) dE tasks
 * as workgroups (small N and D), each task is cut along its kept tiles into pieces
 * summed by different workgroups and added in a fixed order by a finishing kernel;
 * when the tasks overflow the grid by at most half of it, the tasks past the grid are cut
 * (after a launch of one whole task per workgroup).
 * This keeps whole tasks (dE can differ in the last bits: the tiles' fp32 sums are
 * added in another order). */
#define CCE_BWD_DE_WHOLE_TASKS 8192

/* As cce_backward, with flags (CCE_BWD_*) and vocabulary chunks of at most
 * max_chunk_tiles tiles (0: the library's choice; else a multiple of 32; the workspace
 * size is then cce_backward_workspace_size_ex's with the same value).  Same reference
 * interfaces as cce_backward. */
int cce_backward_ex(int dtype, const void* e, const void* c, const void* bias,
                    const int64_t* targets, int64_t ignore_index, int has_ignore,
                    int64_t N, int64_t D, int64_t V,
                    const float* lse, const float* tile_max, const float* d_nll,
                    float filter_log_eps,
                    void* dE, void* dC, void* dBias,
                    void* workspace, size_t workspace_bytes,
                    int64_t* tile_stats, int flags, int64_t max_chunk_tiles, void* hip_stream);

/*
 * Backward without any allocation -- no counterpart in the reference.  For callers
 * that cannot call hipMalloc or take a caller-owned workspace: code under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation.  As cce_backward_ex
 * (max_chunk_tiles 0), with the workspace taken from a static device array of
 * CCE_NOALLOC_SCRATCH_BYTES (64 MiB) that every GPU the library runs on holds from
 * its first call until the process ends.  The backward then runs in passes that fit
 * the array; a problem whose least workspace (cce_backward_workspace_size_ex with
 * max_g_tiles = 1) exceeds it is refused with CCE_ERR_WORKSPACE before any device
 * work.  The caller still passes the inputs and the outputs.  Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (other streams, other
 * threads) race and give wrong results; calls ordered on one stream are safe.
 */
#define CCE_NOALLOC_SCRATCH_BYTES (64ull << 20)

/* Bytes of the static scratch cce_backward_noalloc uses (CCE_NOALLOC_SCRATCH_BYTES). */
size_t cce_backward_noalloc_scratch_size(void);

int cce_backward_noalloc(int dtype, const void* e, const void* c, const void* bias,
                         const int64_t* targets, int64_t ignore_index, int has_ignore,
                         int64_t N, int64_t D, int64_t V,
                         const float* lse, const float* tile_max, const float* d_nll,
                         float filter_log_eps,
                         void* dE, void* dC, void* dBias,
                         int64_t* tile_stats, int flags, void* hip_stream);

/*
 * Quantized classifier rows.  The reference's callers pass an lm_head / tied
 * embedding stored with MLX's affine group quantization through mx.dequantize
 * before the loss (README.md:84-95,136; examples/mlx_lm_lora_test.py:16-21),
 * materialising the [V, D] rows.  These entry points take the quantized rows
 * instead and dequantize chunk_rows of them at a time into a caller-provided
 * scratch (0 selects 32768 rows; otherwise a multiple of 4096).
 *   weight   [V, D * bits / 32] uint32: code j of a word in bits [j * bits, (j + 1) * bits)
 *   scales, qbiases  [V, D / group_size] dtype;  w = scale * q + bias
 *   bits 2, 4 or 8; group_size 32, 64 or 128; D % group_size == 0
 * Dequantized values: fp32 product scale * q, fp32 add of the bias, rounded to
 * dtype to nearest-even; the quantized passes equal the plain passes over
 * cce_dequantize's output bit for bit.  The rows carry no gradient (no dC).
 */
/* rows x D dequantized into out [rows, D] dtype (16-byte aligned); mx.dequantize's
 * affine mode, which the reference's callers run before the loss. */
int cce_dequantize(int dtype, const uint32_t* weight, const void* scales, const void* qbiases, int group_size,
                   int bits, int64_t rows, int64_t D, void* out, void* hip_stream);

/* Bytes of scratch cce_forward_q needs: min(chunk_rows, V) rows of D dtype elements. */
size_t cce_forward_q_scratch_size(int dtype, int64_t V, int64_t D, int64_t chunk_rows);

/* As cce_forward with quantized classifier rows (reference: the same interfaces
 * as cce_forward, fed by mx.dequantize's output). */
int cce_forward_q(int dtype, const void* e, const uint32_t* weight, const void* scales, const void* qbiases,
                  int group_size, int bits, const void* bias, const int64_t* targets, int64_t ignore_index,
                  int has_ignore, int64_t N, int64_t D, int64_t V, float* tile_max, float* tile_sum_exp,
                  float* neg_target_logit, float* lse, float* nll, void* scratch, size_t scratch_bytes,
                  int64_t chunk_rows, void* hip_stream);

/* Workspace bytes of cce_backward_q (includes one chunk of dequantized rows). */
size_t cce_backward_q_workspace_size(int dtype, int64_t N, int64_t D, int64_t V, int want_dE, int want_dBias,
                                     int64_t chunk_rows);

/* As cce_backward with quantized classifier rows: dE and dBias only (reference:
 * the same interfaces as cce_backward; the frozen-head mode compute_all_grads=False
 * of csrc/bindings.cpp:15-56 returns no dC either). */
int cce_backward_q(int dtype, const void* e, const uint32_t* weight, const void* scales, const void* qbiases,
                   int group_size, int bits, const void* bias, const int64_t* targets, int64_t ignore_index,
                   int has_ignore, int64_t N, int64_t D, int64_t V, const float* lse, const float* tile_max,
                   const float* d_nll, float filter_log_eps, void* dE, void* dBias, void* workspace,
                   size_t workspace_bytes, int64_t chunk_rows, int64_t* tile_stats, void* hip_stream);

/* Reduction modes of cce_reduce_loss. */
#define CCE_REDUCE_SUM 1
#define CCE_REDUCE_MEAN 2

/*
 * Reduced loss of cce_loss (reference mlx_cce/__init__.py:72-76, where MLX ops do
 * it; no native counterpart there).  One workgroup sums nll[0..N) in a fixed order
 * (deterministic) and counts the rows kept by the ignore mask (all N when
 * has_ignore == 0):
 *   CCE_REDUCE_SUM:  loss_out[0] = sum
 *   CCE_REDUCE_MEAN: loss_out[0] = sum / max(count, 1)
 * scale_out (nullable, fp32[1]) receives max(count, 1).  nll is cce_forward's.
 */
int cce_reduce_loss(const float* nll, const int64_t* targets, int64_t ignore_index, int has_ignore,
                    int64_t N, int mode, float* loss_out, float* scale_out, void* hip_stream);

/*
 * Cotangent of every per-token loss under a reduced loss (the VJP of
 * mlx_cce/__init__.py:72-76): d_nll[r] = grad[0] / scale[0], or grad[0] when scale
 * is NULL.  grad and scale are device fp32[1]; d_nll is device fp32[N].
 */
int cce_broadcast_grad(const float* grad, const float* scale, int64_t N, float* d_nll, void* hip_stream);

#ifdef __cplusplus
}
#endif

#endif /* CCE_MI355X_H */
