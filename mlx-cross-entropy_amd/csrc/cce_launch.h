// cce_launch.h — host-side launch wrappers shared between the kernel
// translation units and the C-ABI layer.  Internal; not installed.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

namespace cce {

// Forward workgroup tile: 256 tokens x 256 vocabulary rows.
constexpr int kFwdTokens = 256;
constexpr int kFwdVocab = 256;
// Statistic / filter tile: 128 vocabulary columns (one wave's share of a forward tile).
constexpr int kStatTile = 128;
// The reference's statistic tile (cce.metal: 32 columns), for its layout of the raw
// statistics: [N][ceil(V / 32)], row major per token (mlx_cce/__init__.py:25-30).
constexpr int kRefStatTile = 32;
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
  int stats32;          // tile_max / tile_sum_exp per 32 columns in the reference's layout [N][ceil(V/32)]
                        // (else per 128 columns, [ceil(V/128)][N])
};

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
// filter as a bitmap, one bit per pair, rows by token block.  Two levels cut the
// work so that every scratch buffer has a bounded size:
//   * chunks: the vocabulary in runs of `chunk_nvt` tiles, fixed on the host by the
//     compaction's LDS limits only (one chunk unless N and V are large);
//   * passes: a chunk's tiles in runs chosen on the device by kept-pair count, so
//     that one pass keeps at most `cap` pairs.  Pass p holds the tiles v whose
//     exclusive prefix of kept pairs P[v] lies in [p (cap - nrb), (p + 1)(cap - nrb)):
//     a tile keeps at most nrb pairs, so a pass keeps fewer than cap.  The host
//     launches `max_passes` passes per chunk (the dense worst case); passes past
//     the last one the data needs find nothing to do and return at once.
// Per chunk the kept pairs get "slots" ordered by (pass, token block, vocab tile);
// a pass's G tiles live in a scratch of `cap` tiles (slot s at s - first slot of
// the pass).  A pass holds every token block of its tiles, so dC and dBias of a
// pass are final when its sums end; dE is carried between passes and chunks in
// fp32 when the backward takes more than one pass.
// G tiles: fp32 inputs store G in fp32.  16-bit inputs store it either rounded once
// to the input dtype (rows of 128 columns), or (g_split) as a pair of 16-bit values,
// hi = round(G) and lo = round(G - hi) (hi + lo = G to about 2^-17 relative), with
// the sums issuing one MFMA per half against the same E / C fragment: the reference
// keeps the softmax weight in fp32 through both products.  A tile row of the pair is
// 256 16-bit values: columns 32 q + i go to elements 64 q + i (hi) and 64 q + 32 + i
// (lo), so that a 128-byte slice of a row holds 32 columns' hi and lo (the dE sums'
// contraction slice).  A tile slot is 64 KiB for fp32 and for the pair, 32 KiB for a
// 16-bit G rounded once.
constexpr size_t g_tile_bytes(size_t esize, bool split) {
  return (size_t)kBwdTokens * kBwdVocab * (esize == 2 && split ? 2 * esize : esize);
}
// G-tile budget of one pass, in MiB of 64 KiB slots (the default workspace; a smaller
// workspace gives smaller passes, down to 2 tiles per token block).  512 MiB holds 8192
// tiles, an eighth of the Llama-3 8B head's (N = 8192, V = 128256: 4.2 GB of G when
// nothing is skipped), so a dense backward takes 8 passes there; a filtered one keeps a
// few hundred tiles and takes one.  A 16-bit G rounded once holds the same tiles in
// half the bytes.
#ifndef CCE_G_SCRATCH_MIB
#define CCE_G_SCRATCH_MIB 512
#endif
constexpr size_t kGScratchBudget = size_t(CCE_G_SCRATCH_MIB) << 20;
constexpr int kCompactMaxWords = 8192;                 // bitmap words one compaction holds in LDS
constexpr int kCompactMaxVt = 4096;                    // vocabulary tiles per chunk (LDS counts)
constexpr int kMaxDcBins = 256;                        // workgroup bins of the dC sums' schedule
constexpr int kDcBlkMaxRb = 4096;                      // token blocks the dC block tasks group by (LDS counts)
constexpr int kDcBlkChunk = 4;                         // one-tile owners per dC block task at most
// Token order of the backward.  The token blocks of the tile filter can be formed
// from the rows grouped by the vocabulary tile of their target: with a peaked
// softmax a block then keeps a few tiles instead of one per distinct target.  The
// grouping (a stable sort, then the rows of rare targets spread evenly over the
// blocks) runs in one workgroup on 16-bit (tile, row) keys.
constexpr int64_t kPermMaxN = 65536;   // rows the sort handles
constexpr int64_t kPermMaxKey = 16384; // tiles + 1 (the key of rows without gradient)
constexpr int kPermFlag = 15;          // counts[kPermFlag]: 1 when the backward runs on sorted rows
// counts[kGScaleExp]: fp16 G tiles hold G * 2^s with s = counts[kGScaleExp] (written by
// the compaction from max |d_nll|, so that G's largest values sit near 2^14 and its
// small ones stay clear of fp16's subnormal range); the sums scale back by 2^-s.
constexpr int kGScaleExp = 14;

// Pass table: kPassInts ints per pass of the current chunk, written by the compaction.
constexpr int kPassInts = 16;
enum PassField {
  kPiVt0 = 0,      // chunk-local vocabulary tiles [vt0, vt1) of the pass
  kPiVt1 = 1,
  kPiS0 = 2,       // slots [s0, s1); the G scratch holds slot s at index s - s0
  kPiS1 = 3,
  kPiTask0 = 4,    // G tasks [task0, task1) in g_task / g_task_rb
  kPiTask1 = 5,
  kPiOwnRb = 6,    // dE owners: own_rb[p * nrb + i], i < this count
  kPiOwnVt = 7,    // dC owners: own_vt[vt0 + i], i < this count
  kPiTail = 8,     // item counter of the G kernel's tail (zeroed by the compaction)
  kPiDeMode = 9,   // -1: no work (past the passes the data needs); else a dE write mode (WriteMode)
  kPiRun = 10,     // G tasks are runs of at most this many slots of one token block
  kPiDcWide = 11,  // filter on: 1 if the dC sums of the pass run in the wide geometry, 0 narrow
  kPiDcBlk = 12,   // dC block tasks per D slice: dc_blk_task[vt0 + i], i < this count
  kPiDcQueue = 13, // dC block tasks: counter of the tasks taken (zeroed by the compaction)
  kPiDcDeal = 14,  // dC owners dealt to the schedule's bins: own_vt[vt0 + i], i < this count (the rest: block tasks)
  kPiGVt = 15,     // 1: G tasks are runs of a vocabulary tile's vt_slot entries (g_task: the first, g_task_rb: the tile)
};
// dE write mode of a pass: one pass over everything writes dE directly; with more
// passes (or chunks) dE is summed in an fp32 carry: the first pass stores it, the
// middle ones add to it, the last one adds and writes dE.
enum WriteMode { kWriteT = 0, kStoreF32 = 1, kAddF32 = 2, kFinishT = 3, kPartF32 = 4 };
// dE pieces: when a pass has at most half as many (token block, D slice) tasks as
// workgroups (or kDePartSlots), the narrow dE sums cut each task along its kept tiles
// into P pieces; a piece's fp32 sums go to its own slot of the de_part scratch (mode
// kPartF32) and bwd_de_pieces_kernel adds a task's pieces in order and writes dE in the
// pass's mode.  When the tasks overflow the grid by at most half of it, the first
// launch (de_stage 0) runs one whole task per workgroup and a second (de_stage 1) the
// pieces of the tasks past the grid.
constexpr int kDePartSlots = 256;  // pieces at most (fp32 slots of 128 x 256 sums)
constexpr int kDePartCols = 256;   // the narrow sums' D slice

struct BwdPlan {
  int64_t nvt, nrb, total;  // vocab tiles, token blocks, pairs
  int64_t nwords;           // 32-bit bitmap words per token block: ceil(nvt / 32)
  int64_t chunk_nvt;        // vocab tiles per chunk (a multiple of 32 unless it is nvt)
  int64_t n_chunks;
  int64_t chunk_pairs;      // nrb * chunk_nvt: the most pairs one chunk may keep
  int64_t cap;              // G tiles per pass: chunk_pairs, or at least 2 nrb
  int64_t max_passes;       // passes launched per chunk
  size_t g_bytes;           // bytes of one G tile slot (g_tile_bytes of the layout)
  bool g_split;             // 16-bit G slots hold the hi / lo pair (else G rounded once)
  int esize;                // bytes of one input element
  bool perm_ok;             // the sorted token order is available (N and tile count in range)
  bool carry;               // the fp32 dE carry is reserved (more than one pass or chunk may run)
  bool de_pieces;           // the dE pieces' slots are reserved (few dE tasks possible)
  // workspace byte offsets
  size_t bits, counts, pinfo, rb_start, slot_vt, slot_rb, vt_start, vt_slot, g_task, g_task_rb, own_rb, own_vt,
      dc_bin_start, dc_bin_owner, dc_blk_task, dc_blk_own, gtile, colsum, de_acc, de_part;
  size_t perm, sort_buf, rowbits, bits_p, t_perm, lse_perm, dnll_perm, e_perm;  // sorted order (perm_ok)
  size_t qrows;  // dequantized classifier rows of one chunk (quantized classifier only)
  size_t total_bytes;
};

inline size_t plan_align(size_t x) { return (x + 255) & ~size_t(255); }

// Chunks of the vocabulary: the compaction's LDS limits; max_chunk_nvt > 0 caps the
// width further (a multiple of 32 tiles: the quantized rows' chunks).
inline int64_t plan_chunk_nvt(int64_t nvt, int64_t nrb, int64_t max_chunk_nvt) {
  int64_t cw = nvt;
  const int64_t by_lds = 32 * (kCompactMaxWords / nrb);
  cw = cw < by_lds ? cw : by_lds;
  cw = cw < kCompactMaxVt ? cw : kCompactMaxVt;
  if (max_chunk_nvt > 0 && max_chunk_nvt < cw) cw = max_chunk_nvt;
  if (cw < nvt) cw = cw / 32 * 32;
  if (cw < 32) cw = nvt < 32 ? nvt : 32;
  return cw;
}

// The plan for passes of at most `cap` G tiles (clamped to [min(2 nrb, chunk_pairs),
// chunk_pairs]); perm: reserve the sorted token order when it is available; quant
// reserves the scratch of one chunk's dequantized classifier rows; g_split: the G
// tiles' layout (the hi / lo pair of 16-bit types, else G rounded once).
inline BwdPlan make_bwd_plan_cap(size_t esize, int64_t N, int64_t D, int64_t V, bool want_de, bool want_dc,
                                 bool want_db, int64_t cap, bool perm, int64_t max_chunk_nvt, bool quant,
                                 bool g_split) {
  BwdPlan P{};
  P.nvt = (V + kBwdVocab - 1) / kBwdVocab;
  P.nrb = (N + kBwdTokens - 1) / kBwdTokens;
  P.total = P.nvt * P.nrb;
  P.nwords = (P.nvt + 31) / 32;
  P.g_split = esize == 2 && g_split;
  P.g_bytes = g_tile_bytes(esize, P.g_split);
  P.esize = (int)esize;
  const bool want_g = want_de || want_dc;
  const int64_t cw = plan_chunk_nvt(P.nvt, P.nrb, max_chunk_nvt);
  P.chunk_nvt = cw;
  P.n_chunks = (P.nvt + cw - 1) / cw;
  P.chunk_pairs = P.nrb * cw;
  const int64_t cap_min = 2 * P.nrb < P.chunk_pairs ? 2 * P.nrb : P.chunk_pairs;
  cap = cap < cap_min ? cap_min : cap;
  cap = cap > P.chunk_pairs ? P.chunk_pairs : cap;
  P.cap = cap;
  // a chunk's tile v lies in pass floor(P[v] / (cap - nrb)), P[v] <= nrb (cw - 1)
  P.max_passes = cap >= P.chunk_pairs ? 1 : (P.nrb * (cw - 1)) / (cap - P.nrb) + 1;
  P.carry = want_de && (P.n_chunks > 1 || P.max_passes > 1);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off += plan_align(bytes);
    return o;
  };
  P.bits = take((size_t)P.nrb * P.nwords * 4);
  P.counts = take(16 * 4);
  P.pinfo = take((size_t)P.max_passes * kPassInts * 4);
  P.rb_start = take((size_t)(P.max_passes * P.nrb + 1) * 4);
  P.slot_vt = take((size_t)P.chunk_pairs * 4);
  P.slot_rb = take((size_t)P.chunk_pairs * 4);
  P.vt_start = take((size_t)(cw + 1) * 4);
  P.vt_slot = take((size_t)P.chunk_pairs * 4);
  P.g_task = take((size_t)P.chunk_pairs * 4);
  P.g_task_rb = take((size_t)P.chunk_pairs * 4);
  P.own_rb = take((size_t)P.max_passes * P.nrb * 4);
  P.own_vt = take((size_t)cw * 4);
  P.dc_bin_start = take((size_t)(kMaxDcBins + 1) * 4);
  P.dc_bin_owner = take((size_t)cw * 4);
  P.dc_blk_task = take((size_t)cw * 16);
  P.dc_blk_own = take((size_t)cw * 8);
  P.gtile = want_g ? take((size_t)P.cap * P.g_bytes) : 0;
  P.colsum = want_db ? take((size_t)P.cap * kBwdVocab * sizeof(float)) : 0;
  P.de_acc = P.carry ? take((size_t)N * (size_t)D * sizeof(float)) : 0;
  // the most dE tasks a pass can have (every token block x the narrow D slices) leave
  // two workgroups per task or more on a 256-CU part, or overflow a 256-workgroup grid
  // by at most half of it (the tasks past the grid are then cut)
  const int64_t de_tasks = P.nrb * ((D + kDePartCols - 1) / kDePartCols);
  P.de_pieces = want_de && (de_tasks * 2 <= kDePartSlots || (de_tasks > kDePartSlots && de_tasks * 2 <= 3 * kDePartSlots));
  P.de_part = P.de_pieces ? take((size_t)kDePartSlots * kBwdTokens * kDePartCols * sizeof(float)) : 0;
  // (dE rows are then written through the map with one buffer over all of dE: < 2^31 bytes)
  P.perm_ok = perm && N <= kPermMaxN && P.nvt + 1 <= kPermMaxKey && (want_g || want_db) &&
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

// G tiles of a pass in the default workspace: the budget's 64 KiB slots (whatever
// the layout), at least 2 per token block.
inline int64_t default_cap(int64_t N) {
  const int64_t nrb = (N + kBwdTokens - 1) / kBwdTokens;
  const int64_t by_budget = (int64_t)(kGScratchBudget / g_tile_bytes(4, true));
  return by_budget > 2 * nrb ? by_budget : 2 * nrb;
}

// The plan of the default workspace (max_g_tiles <= 0), or of passes of at most
// max_g_tiles G tiles.
inline BwdPlan make_bwd_plan(size_t esize, int64_t N, int64_t D, int64_t V, bool want_de, bool want_dc,
                             bool want_db, int64_t max_chunk_nvt, bool quant, int64_t max_g_tiles, bool g_split) {
  const int64_t dcap = default_cap(N);
  const int64_t cap = max_g_tiles > 0 && max_g_tiles < dcap ? max_g_tiles : dcap;
  return make_bwd_plan_cap(esize, N, D, V, want_de, want_dc, want_db, cap, true, max_chunk_nvt, quant, g_split);
}

// The plan a workspace of ws_bytes runs: the default plan when it fits, else the
// largest pass capacity that fits (the sorted token order is dropped when even the
// smallest passes do not fit with it).  ok = false when nothing fits.
inline BwdPlan plan_for_workspace(size_t esize, int64_t N, int64_t D, int64_t V, bool want_de, bool want_dc,
                                  bool want_db, int64_t max_chunk_nvt, bool quant, bool g_split, size_t ws_bytes,
                                  bool& ok) {
  BwdPlan P = make_bwd_plan(esize, N, D, V, want_de, want_dc, want_db, max_chunk_nvt, quant, 0, g_split);
  ok = P.total_bytes <= ws_bytes;
  if (ok) return P;
  const int64_t dcap = P.cap;
  for (int perm = 1; perm >= 0; --perm) {
    // Below one pass per chunk (cap < chunk_pairs) the size grows with cap: bisect.
    int64_t lo = 1, hi = dcap < P.chunk_pairs ? dcap : P.chunk_pairs - 1;
    BwdPlan best{};
    bool found = false;
    if (hi >= 1) {
      BwdPlan m =
          make_bwd_plan_cap(esize, N, D, V, want_de, want_dc, want_db, lo, perm != 0, max_chunk_nvt, quant, g_split);
      if (m.total_bytes <= ws_bytes) {
        best = m;
        found = true;
        lo = m.cap;  // the clamped minimum
        while (lo < hi) {
          const int64_t mid = lo + (hi - lo + 1) / 2;
          BwdPlan t = make_bwd_plan_cap(esize, N, D, V, want_de, want_dc, want_db, mid, perm != 0, max_chunk_nvt,
                                        quant, g_split);
          if (t.total_bytes <= ws_bytes) {
            best = t;
            lo = mid;
          } else {
            hi = mid - 1;
          }
        }
      }
    }
    if (found) {
      ok = true;
      return best;
    }
  }
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
  int* counts;        // [kPermFlag]: the sorted token order is in use
  int* pinfo;         // [max_passes][kPassInts] pass table of the current chunk
  int* rb_start;      // [max_passes * nrb + 1] first slot of (pass, token block), flattened
  int* slot_vt;       // [chunk_pairs] chunk-local vocab tile of each slot
  int* slot_rb;       // [chunk_pairs] token block of each slot
  int* vt_start;      // [chunk_nvt + 1] first entry of each vocab tile in vt_slot
  int* vt_slot;       // [chunk_pairs] slots grouped by vocab tile, token blocks ascending
  int* g_task;        // [chunk_pairs] first slot of each G task (up to 4 slots of one token block)
  int* g_task_rb;     // [chunk_pairs] token block of each G task
  int* own_rb;        // [max_passes][nrb] token blocks with kept tiles in the pass, most tiles first (dE owners)
  int* own_vt;        // [chunk_nvt] vocab tiles with kept tiles, by pass, most first (dC owners)
  int* dc_bin_start;  // [kMaxDcBins + 1] dC schedule: owners of bin m are dc_bin_owner[start[m] .. start[m + 1])
  int* dc_bin_owner;  // [chunk_nvt]
  // dC block tasks (dc_blk): the owners with one kept tile of a pass, grouped by the
  // token block of that tile, at most kDcBlkChunk per task.  Task i of the pass (per D
  // slice) is dc_blk_task[vt0 + i] = (token block, e0, e1, 0): its owners are the
  // (owner, slot) pairs dc_blk_own[vt0 + e], e0 <= e < e1 (vt0: the pass's first tile).
  int* dc_blk_task;   // [chunk_nvt][4]
  int* dc_blk_own;    // [chunk_nvt][2]
  char* gtile;        // [cap] G tiles of one pass, token-major (g_tile_bytes each)
  float* colsum;      // [cap][128] per-slot column sums of G (dBias)
  float* de_acc;      // [N, D] fp32, only when the plan reserves the carry
  float* de_part;     // [kDePartSlots][128][kDePartCols] fp32 sums of the dE pieces, or null (whole tasks)
  int de_stage;       // narrow dE sums launch: 0 the tasks (overflow: the first grid's worth), 1 the overflow's pieces
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
  int de_geo;           // dE sums geometry: 0 the backward's choice (filter off: by size; on: narrow), 1 wide, 2 narrow
  int dc_geo;           // dC sums geometry: 0 the backward's choice (filter off: wide; on: per pass), 1 wide, 2 narrow
  int dc_zeroed;        // dC already holds zeros: only rows of vocab tiles with kept tiles are written
  int stats32;          // tile_max per 32 columns in the reference's layout [N][ceil(V/32)] (else [nvt][N])
  int g_scaled;         // fp16: G tiles hold G * 2^counts[kGScaleExp] (else unscaled)
  int g_split;          // 16-bit: G tiles hold the hi / lo pair (else G rounded once)
  int dc_blk;           // the narrow dC sums run owners with one kept tile as tasks per (token block, D slice)
  int g_tiles_ok;       // the compaction may list G tasks by vocabulary tile
  // Pinned host memory of 1 + max_passes ints, or null.  The compaction writes the
  // chunk's pass count to [0] and each pass's kPiDcWide to [1 + p]; the host then
  // launches only those passes and only the dC geometry picked (launch_backward's
  // event), instead of max_passes passes with both geometries.
  int* host_pass;
  QuantRows q;          // q.wq set: c is unused; every chunk first dequantizes its rows into q.scratch
};

// dtype: 0 f32, 1 f16, 2 bf16.  Return hipError_t of the launches.
hipError_t launch_forward(int dtype, const FwdArgs& a, hipStream_t s);
// As launch_forward with the classifier rows in q (a.c unused).
hipError_t launch_forward_q(int dtype, const FwdArgs& a, const QuantRows& q, hipStream_t s);
// Rows [row0, row0 + rows) of q dequantized into out ([rows, D], dtype); with keep (a
// per-128-row-tile table, entries t and t + 1 equal = tile t not needed) only the
// rows of the tiles needed.
hipError_t launch_dequantize(int dtype, const QuantRows& q, int64_t row0, int64_t rows, int64_t D, void* out,
                             hipStream_t s, const int* keep = nullptr);
// With a.host_pass set, pass_ev (an event of the current device) is recorded after
// each chunk's compaction and waited for on the host before the chunk's passes past
// the first G kernel are launched.
hipError_t launch_backward(int dtype, const BwdArgs& a, hipStream_t s, hipEvent_t pass_ev = nullptr);
hipError_t launch_reduce_loss(const float* nll, const int64_t* targets, int64_t ignore_index, int has_ignore,
                              int64_t N, int mode, float* loss, float* scale, hipStream_t s);
hipError_t launch_broadcast_grad(const float* grad, const float* scale, int64_t N, float* d_nll, hipStream_t s);

}  // namespace cce
