// cce_launch.h — host-side launch wrappers shared between the kernel
// translation units and the C-ABI layer.  Internal; not installed.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cce {

// Forward workgroup tile: 256 tokens x 256 vocabulary rows (4 waves, each 128 x 128).
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
};

// Backward work plan: kept (vocab tile, token block) pairs get consecutive
// "slots" in vocab-major order; the slots are processed in chunks of at most
// `cap` whose boundaries fall between vocabulary tiles, so that every vocab tile
// (and its dC rows) belongs to exactly one chunk.  Each chunk's G tiles live in
// a bounded scratch of `cap` slots.
constexpr size_t kWScratchBudget = size_t(2) << 30;  // bytes of G-tile scratch per chunk

struct BwdPlan {
  int64_t nvt, nrb, total;  // vocab tiles, token blocks, pairs
  int64_t cap;              // slots per chunk
  int64_t max_chunks;       // upper bound on chunks (host launches this many)
  int64_t n_dslices;        // 256-byte slices of a row of E / C
  size_t w_bytes;           // bytes of one G tile in one layout (128 x 128 x sizeof(T))
  // workspace byte offsets
  size_t flags, slot_map, list, vt_start, rb_list, rb_vt, rb_start, chunk_vt, chunk_slot, w_tok, w_voc, colsum, de_acc;
  size_t total_bytes;
};

inline size_t plan_align(size_t x) { return (x + 255) & ~size_t(255); }

inline BwdPlan make_bwd_plan(size_t esize, int64_t N, int64_t D, int64_t V, bool want_de, bool want_dc,
                             bool want_db) {
  BwdPlan P{};
  P.nvt = (V + kBwdVocab - 1) / kBwdVocab;
  P.nrb = (N + kBwdTokens - 1) / kBwdTokens;
  P.total = P.nvt * P.nrb;
  P.w_bytes = (size_t)kBwdTokens * kBwdVocab * esize;
  const size_t per_slot = (want_de ? P.w_bytes : 0) + (want_dc ? P.w_bytes : 0) +
                          (want_db ? 2 * kBwdVocab * sizeof(float) : 0);
  int64_t cap = per_slot ? (int64_t)(kWScratchBudget / per_slot) : P.total;
  if (cap < 2 * P.nrb) cap = 2 * P.nrb;  // a chunk must hold any one vocab tile's token blocks
  if (cap > P.total) cap = P.total;
  P.cap = cap;
  // Vocab tile vt goes to chunk vt_start[vt] / step (computed on the device); a chunk then
  // spans fewer than step + nrb slots, i.e. at most cap, and there are at most
  // total / step + 1 chunks.  With cap == total everything fits one chunk.
  const int64_t step = cap - P.nrb + 1;
  P.max_chunks = (cap == P.total) ? 1 : P.total / step + 1;
  P.n_dslices = (D * (int64_t)esize + 255) / 256;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off += plan_align(bytes);
    return o;
  };
  P.flags = take((size_t)P.total);
  P.slot_map = take((size_t)P.total * 4);
  P.list = take((size_t)P.total * 4);
  P.vt_start = take((size_t)(P.nvt + 1) * 4);
  P.rb_list = take((size_t)P.total * 4);
  P.rb_vt = take((size_t)P.total * 4);
  P.rb_start = take((size_t)(P.nrb + 1) * 4);
  P.chunk_vt = take((size_t)(P.max_chunks + 1) * 4);
  P.chunk_slot = take((size_t)(P.max_chunks + 1) * 4);
  P.w_tok = want_de ? take((size_t)cap * P.w_bytes) : 0;
  P.w_voc = want_dc ? take((size_t)cap * P.w_bytes) : 0;
  P.colsum = want_db ? take((size_t)cap * 2 * kBwdVocab * sizeof(float)) : 0;
  P.de_acc = (want_de && P.max_chunks > 1) ? take((size_t)N * (size_t)D * sizeof(float)) : 0;
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
  // workspace (see BwdPlan)
  uint8_t* flags;     // [nvt * nrb], index vt * nrb + rb
  int* slot_map;      // [nvt * nrb] slot of a kept pair, -1 otherwise
  int* list;          // [nvt * nrb] slot -> pair, vocab-major
  int* vt_start;      // [nvt + 1] first slot of each vocab tile
  int* rb_list;       // [nvt * nrb] slots ordered by token block, then vocab tile
  int* rb_vt;         // [nvt * nrb] vocab tile of each rb_list entry
  int* rb_start;      // [nrb + 1]
  int* chunk_vt;      // [max_chunks + 1] first vocab tile of each chunk
  int* chunk_slot;    // [max_chunks + 1] first slot of each chunk
  char* w_tok;        // [cap][128 tokens][128 vocab] G tiles, token-major
  char* w_voc;        // [cap][128 vocab][128 tokens] G tiles, vocab-major
  float* colsum;      // [cap][2][128] per-tile column sums of G (two token halves)
  float* de_acc;      // [N, D] fp32, only when max_chunks > 1
  int64_t* tile_stats;  // [2] or null
  BwdPlan plan;
  int num_cus;
};

// dtype: 0 f32, 1 f16, 2 bf16.  Return hipError_t of the launches.
hipError_t launch_forward(int dtype, const FwdArgs& a, hipStream_t s);
hipError_t launch_backward(int dtype, const BwdArgs& a, hipStream_t s);

}  // namespace cce
