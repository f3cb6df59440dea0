// cce_launch.h — host-side launch wrappers shared between the kernel
// translation units and the C-ABI layer.  Internal; not installed.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

#include <cstdlib>

namespace cce {

// Forward workgroup tile: 256 tokens x 256 vocabulary rows.
constexpr int kFwdTokens = 256;
constexpr int kFwdVocab = 256;
// Statistic / filter tile: 128 vocabulary columns (one wave's share of a forward tile).
constexpr int kStatTile = 128;
// Backward tile: 128 tokens x 128 vocabulary rows.
constexpr int kBwdTokens = 128;
constexpr int kBwdVocab = 128;

struct FwdArgs {
  const void* e;
  const void* c;
  const void* bias;
  const int64_t* targets;
  int64_t ignore_index;
  int has_ignore;
  int64_t N, D, V;
  float* tile_max;
  float* tile_sum_exp;
  float* neg_target_logit;
  float* lse;
  float* nll;
  int num_cus;  // compute units of the device (the persistent forward runs one workgroup per CU)
  void* zero_buf;       // filled with zeros alongside the tiles (null: none)
  int64_t zero_units;   // 16-byte units of zero_buf
  void* e_frag;         // E in MFMA fragment order (e_frag_bytes(); null: E staged through LDS)
};

// Bytes of the fragment-order copy of E that the forward's register-operand main
// loop reads: every 32-row token block of the whole 256-token tiles, the row
// bytes rounded up to the 128-byte slice.
inline size_t e_frag_bytes(int64_t N, int64_t row_bytes) {
  const int64_t blocks = (N + 255) / 256 * 8;
  const int64_t slices = (row_bytes + 127) / 128;
  return (size_t)(blocks * slices * 4096);
}

// Classifier rows stored with affine group quantization (the layout of MLX's
// mx.quantize / mx.dequantize, mlx >= 0.22, which the reference's callers apply
// before the loss: README.md:90-95, examples/mlx_lm_lora_test.py:16-21): row r of
// the [rows, D] weight is D * bits / 32 uint32 words, element j of a word in bits
// [j * bits, (j + 1) * bits); scales and biases are [rows, D / group_size] in the
// compute dtype; w = scale * q + bias.  The passes dequantize chunk_rows rows at a
// time into `scratch` ([chunk_rows, D], compute dtype) and run on that chunk.
struct QuantRows {
  const uint32_t* wq;  // null: the classifier rows are plain
  const void* scales;
  const void* biases;
  int group_size;      // 32, 64 or 128
  int bits;            // 2, 4 or 8
  void* scratch;
  int64_t chunk_rows;  // a multiple of kQuantChunkAlign
};
constexpr int64_t kQuantChunkAlign = 4096;         // rows: whole 32-tile chunks of the backward
constexpr int64_t kQuantDefaultChunkRows = 32768;  // 256 MiB of bf16 scratch at D = 4096

// Backward work plan.  Kept (token block, vocabulary tile) pairs are found by the
// filter as a bitmap, one bit per pair, rows by token block.  The vocabulary is
// cut into chunks of `chunk_nvt` tiles (one chunk unless the problem is large);
// per chunk the kept pairs get consecutive "slots" in (token block, vocab tile)
// order, and every slot's 128 x 128 G tile lives in a scratch of `cap` slots.
// A chunk holds every token block of its vocabulary tiles, so dC and dBias of a
// chunk are final when its sums end; dE is carried between chunks in fp32.
// G-tile scratch per chunk.  A chunk holds every pair it may keep, so the budget sets
// the chunk width: 16 GiB keeps a 70B-class head (N = 32768, V = 128256: 8.4 GB) in one
// chunk, which saves the fp32 dE carry between chunks (at that size 1.5 of 4.5 ms).
#ifndef CCE_G_SCRATCH_GIB
#define CCE_G_SCRATCH_GIB 16
#endif
constexpr size_t kWScratchBudget = size_t(CCE_G_SCRATCH_GIB) << 30;
constexpr int kCompactMaxWords = 8192;                 // bitmap words one compaction holds in LDS
constexpr int kCompactMaxVt = 4096;                    // vocabulary tiles per chunk (LDS counts)
constexpr int kMaxDcBins = 256;                        // workgroup bins of the dC sums' schedule
// Token order of the backward.  The token blocks of the tile filter can be formed
// from the rows grouped by the vocabulary tile of their target: with a peaked
// softmax a block then keeps a few tiles instead of one per distinct target.  The
// grouping (a stable sort, then the rows of rare targets spread evenly over the
// blocks) runs in one workgroup on 16-bit (tile, row) keys.
constexpr int64_t kPermMaxN = 65536;   // rows the sort handles
constexpr int64_t kPermMaxKey = 16384; // tiles + 1 (the key of rows without gradient)
constexpr int kPermFlag = 15;          // counts[kPermFlag]: 1 when the backward runs on sorted rows

struct BwdPlan {
  int64_t nvt, nrb, total;  // vocab tiles, token blocks, pairs
  int64_t nwords;           // 32-bit bitmap words per token block: ceil(nvt / 32)
  int64_t chunk_nvt;        // vocab tiles per chunk (a multiple of 32 unless it is nvt)
  int64_t n_chunks;
  int64_t cap;              // slots per chunk: nrb * chunk_nvt
  size_t g_bytes;           // bytes of one G tile (128 x 128 x sizeof(T))
  bool perm_ok;             // the sorted token order is available (N and tile count in range)
  // workspace byte offsets
  size_t bits, counts, rb_start, slot_vt, slot_rb, vt_start, vt_slot, g_task, g_task_rb, own_rb, own_vt, dc_bin_start,
      dc_bin_owner, gtile, colsum, de_acc;
  size_t perm, sort_buf, rowbits, bits_p, t_perm, lse_perm, dnll_perm, e_perm;  // sorted order (perm_ok)
  size_t qrows;  // dequantized classifier rows of one chunk (quantized classifier only)
  size_t total_bytes;
};

inline size_t plan_align(size_t x) { return (x + 255) & ~size_t(255); }

// max_chunk_nvt > 0 caps the chunk width (a multiple of 32 tiles); quant reserves the
// scratch of one chunk's dequantized classifier rows.
inline BwdPlan make_bwd_plan(size_t esize, int64_t N, int64_t D, int64_t V, bool want_de, bool want_dc,
                             bool want_db, int64_t max_chunk_nvt = 0, bool quant = false) {
  BwdPlan P{};
  P.nvt = (V + kBwdVocab - 1) / kBwdVocab;
  P.nrb = (N + kBwdTokens - 1) / kBwdTokens;
  P.total = P.nvt * P.nrb;
  P.nwords = (P.nvt + 31) / 32;
  P.g_bytes = (size_t)kBwdTokens * kBwdVocab * esize;
  const bool want_g = want_de || want_dc;
  // Chunk width: bounded by the G scratch budget (a chunk may keep every pair),
  // the compaction's LDS bitmap, and its per-tile counts; at least 32 tiles.
  int64_t cw = P.nvt;
  if (want_g) {
    const int64_t by_budget = (int64_t)(kWScratchBudget / P.g_bytes) / P.nrb;
    cw = cw < by_budget ? cw : by_budget;
  }
  const int64_t by_lds = 32 * (kCompactMaxWords / P.nrb);
  cw = cw < by_lds ? cw : by_lds;
  cw = cw < kCompactMaxVt ? cw : kCompactMaxVt;
  if (max_chunk_nvt > 0 && max_chunk_nvt < cw) cw = max_chunk_nvt;
  // Test hook: CCE_TEST_CHUNK_VT narrows the chunks (rounded down to a multiple of 32)
  // so that the multi-chunk path runs at small sizes.
  if (const char* env = std::getenv("CCE_TEST_CHUNK_VT")) {
    const long long t = std::atoll(env);
    if (t > 0 && t < cw) cw = t;
  }
  if (cw < P.nvt) cw = cw / 32 * 32;
  if (cw < 32) cw = P.nvt < 32 ? P.nvt : 32;
  P.chunk_nvt = cw;
  P.n_chunks = (P.nvt + cw - 1) / cw;
  P.cap = P.nrb * cw;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off += plan_align(bytes);
    return o;
  };
  P.bits = take((size_t)P.nrb * P.nwords * 4);
  P.counts = take(16 * 4);
  P.rb_start = take((size_t)(P.nrb + 1) * 4);
  P.slot_vt = take((size_t)P.cap * 4);
  P.slot_rb = take((size_t)P.cap * 4);
  P.vt_start = take((size_t)(cw + 1) * 4);
  P.vt_slot = take((size_t)P.cap * 4);
  P.g_task = take((size_t)P.cap * 4);
  P.g_task_rb = take((size_t)P.cap * 4);
  P.own_rb = take((size_t)P.nrb * 4);
  P.own_vt = take((size_t)cw * 4);
  P.dc_bin_start = take((size_t)(kMaxDcBins + 1) * 4);
  P.dc_bin_owner = take((size_t)cw * 4);
  P.gtile = want_g ? take((size_t)P.cap * P.g_bytes) : 0;
  P.colsum = want_db ? take((size_t)P.cap * kBwdVocab * sizeof(float)) : 0;
  P.de_acc = (want_de && P.n_chunks > 1) ? take((size_t)N * (size_t)D * sizeof(float)) : 0;
  // (dE rows are then written through the map with one buffer over all of dE: < 2^31 bytes)
  P.perm_ok = N <= kPermMaxN && P.nvt + 1 <= kPermMaxKey && (want_g || want_db) &&
              (double)N * (double)D * (double)esize < 2147483648.0;
  if (P.perm_ok) {
    P.perm = take((size_t)N * 4);
    P.sort_buf = take((size_t)N * 8);
    P.rowbits = take((size_t)N * P.nwords * 4);
    P.bits_p = take((size_t)P.nrb * P.nwords * 4);
    P.t_perm = take((size_t)N * 8);
    P.lse_perm = take((size_t)N * 4);
    P.dnll_perm = take((size_t)N * 4);
    P.e_perm = take((size_t)N * (size_t)D * esize);
  }
  P.qrows = quant ? take((size_t)P.chunk_nvt * kBwdVocab * (size_t)D * esize) : 0;
  P.total_bytes = off;
  return P;
}

struct BwdArgs {
  const void* e;
  const void* c;
  const void* bias;
  const int64_t* targets;
  int64_t ignore_index;
  int has_ignore;
  int64_t N, D, V;
  const float* lse;
  const float* tile_max;
  const float* d_nll;
  float filter_log_eps;
  void* dE;     // output, dtype, or null
  void* dC;     // output, dtype, or null
  void* dBias;  // output, dtype, or null
  // workspace (see BwdPlan); the lists are rebuilt for every chunk
  uint32_t* bits;     // [nrb][nwords] keep bitmap, bit b of word w = vocab tile 32 w + b
  int* counts;        // [0] kept pairs, [1] G tasks, [2] tail item counter, [4] / [5] entries of own_rb / own_vt
  int* rb_start;      // [nrb + 1] first slot of each token block
  int* slot_vt;       // [cap] chunk-local vocab tile of each slot
  int* slot_rb;       // [cap] token block of each slot
  int* vt_start;      // [chunk_nvt + 1] first entry of each vocab tile in vt_slot
  int* vt_slot;       // [cap] slots grouped by vocab tile, token blocks ascending
  int* g_task;        // [cap] first slot of each G task (up to 4 slots of one token block)
  int* g_task_rb;     // [cap] token block of each G task
  int* own_rb;        // [nrb] token blocks with kept tiles, most tiles first (dE owners)
  int* own_vt;        // [chunk_nvt] chunk vocab tiles with kept tiles, most first (dC owners)
  int* dc_bin_start;  // [kMaxDcBins + 1] dC schedule: owners of bin m are dc_bin_owner[start[m] .. start[m + 1])
  int* dc_bin_owner;  // [chunk_nvt]
  char* gtile;        // [cap][128 tokens][128 vocab] G tiles, token-major, dtype
  float* colsum;      // [cap][128] per-slot column sums of G (dBias)
  float* de_acc;      // [N, D] fp32, only when n_chunks > 1
  int64_t* tile_stats;  // [3] or null: kept pairs, all pairs, kept pairs of the input-order token blocks
  BwdPlan plan;
  int num_cus;
  // sorted token order (plan.perm_ok; null otherwise).  Row p of the sorted order is
  // row perm[p] of the input; when counts[kPermFlag] is set the G kernel and the
  // sums read e_perm / t_perm / lse_perm / dnll_perm and write dE row perm[p] for p.
  int* perm;            // [N]
  uint32_t* sort_buf;   // [2 N] radix-sort ping-pong of (key << 16 | row)
  uint32_t* rowbits;    // [N][nwords] keep bits of every row (input order)
  uint32_t* bits_p;     // [nrb][nwords] keep bitmap of the sorted token blocks
  int64_t* t_perm;      // [N]
  float* lse_perm;      // [N]
  float* dnll_perm;     // [N]
  void* e_perm;         // [N, D] dtype
  int perm_mode;        // 0: sorted order when it keeps >= 10% fewer tiles, 1: never, 2: always
  int dc_zeroed;        // dC already holds zeros: only rows of vocab tiles with kept tiles are written
  QuantRows q;          // q.wq set: c is unused; every chunk first dequantizes its rows into q.scratch
};

// dtype: 0 f32, 1 f16, 2 bf16.  Return hipError_t of the launches.
hipError_t launch_forward(int dtype, const FwdArgs& a, hipStream_t s);
// As launch_forward with the classifier rows in q (a.c unused).
hipError_t launch_forward_q(int dtype, const FwdArgs& a, const QuantRows& q, hipStream_t s);
// Rows [row0, row0 + rows) of q dequantized into out ([rows, D], dtype).
hipError_t launch_dequantize(int dtype, const QuantRows& q, int64_t row0, int64_t rows, int64_t D, void* out,
                             hipStream_t s);
hipError_t launch_backward(int dtype, const BwdArgs& a, hipStream_t s);
hipError_t launch_reduce_loss(const float* nll, const int64_t* targets, int64_t ignore_index, int has_ignore,
                              int64_t N, int mode, float* loss, float* scale, hipStream_t s);
hipError_t launch_broadcast_grad(const float* grad, const float* scale, int64_t N, float* d_nll, hipStream_t s);

}  // namespace cce
