// cce_bwd.hip — backward pass of Cut Cross-Entropy on CDNA4 (gfx950).
//
//   G[r, v] = d_nll[r] * (softmax_v(E_r . C^T + b) - [v == t_r])
//   dE = G . C      dC = G^T . E      dBias = sum_r G[r, :]
//
// Reference: csrc/cce/cce.metal:146-326 (cce_backward: filter :191-204, weight
// w = d_nll exp(S + b - lse) - d_nll [v == t] :279-280) and the full-gradient
// research kernel reference/_fused_backward.py:1406-1587 (dC :1535-1545,
// dBias :1546-1553), which accumulate per-tile partials with fp32 atomics.
//
// On MI355X fp32 global atomics retire at ~2.9e11 per second — 2.5e9 of them
// (the per-tile partial flushes at the Llama-3.1-8B head) cost ~8 ms — so this
// backward gives every output element exactly one writer instead, and never
// materialises a [N, tiles, D] scratch:
//
//   1. bwd_filter_kernel   keep bit per (token block, vocabulary tile) of 128 x 128:
//                          some row with d_nll != 0 has its target in the tile or
//                          tile_max - lse >= filter_log_eps; also each row's own
//                          keep bits.  When the token order below is available the
//                          same launch (bwd_filter_sort_kernel) sorts the rows by
//                          the vocabulary tile of their target in one extra
//                          workgroup, and bwd_filter_sorted_kernel ORs the row bits
//                          over the blocks of the sorted order.
//   per chunk of vocabulary tiles (one chunk unless the problem is large):
//   2. bwd_compact_kernel  one workgroup picks the token order (the first chunk: the
//                          sorted blocks when they keep >= 10% fewer tiles), turns
//                          the chunk's bitmap (held in LDS) into slots in (token
//                          block, vocab tile) order, the same slots grouped by vocab
//                          tile, the G task list and the sums' owner orders; the
//                          launch's other workgroups copy E rows (and per-row data)
//                          into the sorted order meanwhile.
//   3. empty_owner         owners (row blocks of dE / dC) without kept tiles get
//                          zeros (and the fp32 dE carry is started / finished);
//                          done by the G kernel's workgroups once out of tasks,
//                          after the first of them deals the dC schedule.
//   4. bwd_g_kernel        per task (one token block with up to 4 of its kept vocab
//                          tiles, or one vocab tile with up to 4 of its kept blocks):
//                          recompute the 512 x 128 logits on MFMA, form G, store
//                          each 128 x 128 G tile token-major in the input dtype, plus
//                          fp32 column sums for dBias.
//   5. bwd_sum_kernel<0>   dE = sum over a token block's kept tiles of G_j . C_j;
//      (or the narrow      written to the dE rows of the block (through the sorted
//      geometry)           order's permutation when it is used);
//      bwd_sum_narrow<1>   dC = sum over a vocab tile's kept blocks of G_j^T . E_j.
//                          Persistent, software-pipelined GEMMs over the gathered
//                          tile lists: E / C rows stream into LDS by DMA in their
//                          natural [k][d] layout and are read as MFMA fragments
//                          with ds_read_b64_tr_b16 (dC reads G transposed the same
//                          way), output rows written once in the output dtype.
//   6. bwd_dbias_kernel    dBias = sum of the column sums of a vocab tile's slots.
#include <type_traits>

#include "cce_device.h"
#include "cce_launch.h"

namespace cce {

static_assert(kStatTile == kBwdVocab, "filter statistics are kept per backward vocabulary tile");
static_assert(kBwdTokens == 128 && kBwdVocab == 128, "the G-tile kernels assume 128 x 128 tiles");

// Two floats rounded to a 16-bit type, packed low-first into one dword.
template <typename T>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (T)lo) | ((uint32_t)__builtin_bit_cast(uint16_t, (T)hi) << 16);
}

// ---------------------------------------------------------------- 1. filter
// One wave per (token block rb, bitmap word w): bits b = 0..31 for vocab tiles 32 w + b.
// Lanes hold two rows each; eight tiles' statistics are fetched before they are tested.
__device__ __forceinline__ void filter_item(const BwdArgs& a, int item) {
  const int nrb = (int)a.plan.nrb, nw = (int)a.plan.nwords, nvt = (int)a.plan.nvt;
  const int lane = threadIdx.x & 63;
  if (item >= nrb * nw) return;  // uniform per wave
  const int rb = item / nw;
  const int w = item - rb * nw;
  int64_t row[2], tg[2];
  float lz[2];
  bool act[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    row[k] = (int64_t)rb * kBwdTokens + k * 64 + lane;
    act[k] = false;
    lz[k] = 0.f;
    tg[k] = -1;
    if (row[k] < a.N) {
      const int64_t t = a.targets[row[k]];
      act[k] = a.d_nll[row[k]] != 0.f && !(a.has_ignore && t == a.ignore_index);
      lz[k] = a.lse[row[k]];
      tg[k] = t;
    }
  }
  uint32_t word = 0, rw[2] = {0u, 0u};  // the block's word and each row's own bits
  const int vt0 = w * 32;
  for (int b0 = 0; b0 < 32; b0 += 8) {
    if (vt0 + b0 >= nvt) break;
    float tm[8][2];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int vt = vt0 + b0 + u;
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        tm[u][k] = -INFINITY;
        if (vt < nvt && act[k]) {
          if (a.stats32) {  // the reference's layout: the max of the tile's four 32-column maxima
            const int64_t nt = (a.V + kRefStatTile - 1) / kRefStatTile;
            const float* p = a.tile_max + row[k] * nt;
#pragma unroll
            for (int q = 0; q < kStatTile / kRefStatTile; ++q)
              if (vt * (kStatTile / kRefStatTile) + q < nt) tm[u][k] = fmaxf(tm[u][k], p[vt * (kStatTile / kRefStatTile) + q]);
          } else {
            tm[u][k] = a.tile_max[(size_t)vt * a.N + row[k]];
          }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int vt = vt0 + b0 + u;
      const int64_t v0 = (int64_t)vt * kBwdVocab;
      bool keep = false;
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const bool kk = vt < nvt && act[k] && ((tg[k] >= v0 && tg[k] < v0 + kBwdVocab) || (tm[u][k] - lz[k] >= a.filter_log_eps));
        rw[k] |= kk ? 1u << (b0 + u) : 0u;
        keep = keep || kk;
      }
      if (__any(keep)) word |= 1u << (b0 + u);
    }
  }
  if (lane == 0) a.bits[(size_t)rb * nw + w] = word;
  if (a.rowbits) {
#pragma unroll
    for (int k = 0; k < 2; ++k)
      if (row[k] < a.N) a.rowbits[(size_t)row[k] * nw + w] = rw[k];
  }
}

__global__ __launch_bounds__(256) void bwd_filter_kernel(BwdArgs a) {
  filter_item(a, blockIdx.x * 4 + (threadIdx.x >> 6));
}

// Keep bitmap of the sorted token blocks: block rb of the sorted order holds rows
// perm[128 rb ..], and keeps a tile when one of them does (their per-row bits).
__global__ __launch_bounds__(256) void bwd_filter_sorted_kernel(BwdArgs a) {
  const int nrb = (int)a.plan.nrb, nw = (int)a.plan.nwords;
  const int lane = threadIdx.x & 63;
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= nrb * nw) return;  // uniform per wave
  const int rb = item / nw;
  const int w = item - rb * nw;
  uint32_t x = 0;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int64_t p = (int64_t)rb * kBwdTokens + k * 64 + lane;
    if (p < a.N) x |= a.rowbits[(size_t)min((int64_t)a.perm[p], a.N - 1) * nw + w];
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x |= (uint32_t)__shfl_xor((int)x, o);
  if (lane == 0) a.bits_p[(size_t)rb * nw + w] = x;
}

// Inclusive prefix sum across the 64 lanes of a wave.
__device__ __forceinline__ int wave_incl_scan(int v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int u = __shfl_up(v, o);
    if (lane >= o) v += u;
  }
  return v;
}

// Sum across the 64 lanes of a wave (every lane gets it).  Counters in LDS take one
// atomic per wave of such a sum: an atomic from many lanes to one address becomes a
// loop over the active lanes, ~35 ns per lane here.
__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Exclusive prefix sum over the NW waves of a workgroup (all threads call it);
// `total` gets the sum.
template <int NW = 16>
__device__ __forceinline__ int block_excl_scan(int v, int* wsum, int& total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int incl = wave_incl_scan(v);
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  int wbase = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const int x = wsum[w];
    wbase += w < wave ? x : 0;
    tot += x;
  }
  __syncthreads();  // wsum may be rewritten by the next scan
  total = tot;
  return wbase + incl - v;
}

// ---------------------------------------------------------------- token order
// The backward's token order: rows grouped by key = the vocab tile of the target,
// or nvt for rows that get no gradient (ignored, target out of range, d_nll == 0).
//   1. A stable LSD radix sort of (key << 16 | row), 4 key bits per pass.  Element
//      i of a pass is held by thread i % 1024 in round i / 1024, so rounds, then
//      waves, then lanes run in element order; a lane's place among the elements
//      with its digit is the digit's start + the count in earlier (round, wave)
//      pairs + the count in lower lanes of its wave (a ballot).
//   2. Rows whose key has fewer than kSortHeadRun rows ("tail" rows: rare targets;
//      run lengths are read off the sorted keys)
//      are spread evenly over the token blocks, in sorted order: block b takes the
//      tail rows [tb(b), tb(b + 1)), tb(b) = floor(min(128 b, N) nT / N), then the
//      next head rows in sorted order.  Every block then holds a slice of the long
//      runs (one or two keys) and a few rare keys, instead of the last blocks
//      holding one key per row.
// One workgroup of 1024 threads; perm[p] = input row at position p.
constexpr int kSortMaxRounds = (int)(kPermMaxN / 1024);
constexpr int kSortHeadRun = 16;
// Lanes of the wave whose 5-bit value d (a 4-bit digit, or 16 for no element) equals
// v: five ballots, one per bit, intersected with the bit or its complement as v has it.
// Every lane must call this (the ballots span the wave).
__device__ __forceinline__ uint64_t digit_lanes(int d, int v) {
  uint64_t m = ~0ull;
#pragma unroll
  for (int k = 0; k < 5; ++k) {
    const uint64_t b = __ballot((d >> k) & 1);
    m &= ((v >> k) & 1) ? b : ~b;
  }
  return m;
}

template <int MAXR>  // rounds the elements of one thread can span: N <= 1024 MAXR
__device__ void sort_rows(const BwdArgs& a) {
  // the ping-pong buffers sit in LDS for up to 8 rounds (8192 rows), else in the workspace
  constexpr int kLdsRows = MAXR <= 8 ? 8 * 1024 : 1;
  __shared__ int hist[kPermMaxKey];                // first sorted position of each key, then its rows
  __shared__ int cnt[MAXR * 16 * 16];              // [round][wave][digit], then exclusive prefixes
  __shared__ int dstart[17];
  __shared__ int tbl[kPermMaxN / kBwdTokens + 1];  // tail rows before each block
  __shared__ uint32_t lbuf[2][kLdsRows];
  static_assert(MAXR % 8 == 0 && MAXR <= kSortMaxRounds, "rounds in groups of 8");
  const int N = (int)a.N, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nvt = (int)a.plan.nvt;
  const int rounds = (N + 1023) >> 10;
  const uint64_t lt = (1ull << lane) - 1ull;
  uint32_t* buf0 = MAXR <= 8 ? lbuf[0] : a.sort_buf;
  uint32_t* buf1 = MAXR <= 8 ? lbuf[1] : a.sort_buf + N;
  // Exclusive prefix of cnt[stride * e + off] over e < n by wave `wave_id` (n <= 64 * 16);
  // returns the total on every lane of that wave.
  auto wave_prefix = [&](int n, int stride, int off) {
    const int per = (n + 63) >> 6;
    const int e0 = min(n, lane * per), e1 = min(n, e0 + per);
    int sum = 0;
    for (int e = e0; e < e1; ++e) sum += cnt[e * stride + off];
    const int incl = wave_incl_scan(sum);
    int run = incl - sum;
    for (int e = e0; e < e1; ++e) {
      const int c = cnt[e * stride + off];
      cnt[e * stride + off] = run;
      run += c;
    }
    return __shfl(incl, 63);
  };
  // This thread's elements, one per round (element r * 1024 + tid), kept in registers;
  // global loads are issued in batches so that their latencies overlap.
  uint32_t x[MAXR];
  auto valid = [&](int r) { return r < rounds && r * 1024 + tid < N; };
#pragma unroll
  for (int r0 = 0; r0 < MAXR; r0 += 8) {
    int64_t t[8];
    float g[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      t[k] = valid(r0 + k) ? a.targets[(r0 + k) * 1024 + tid] : -1;
      g[k] = valid(r0 + k) ? a.d_nll[(r0 + k) * 1024 + tid] : 0.f;
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const bool act = g[k] != 0.f && !(a.has_ignore && t[k] == a.ignore_index) && t[k] >= 0 && t[k] < a.V;
      const uint32_t key = act ? (uint32_t)(t[k] >> 7) : (uint32_t)nvt;  // t / kBwdVocab
      x[r0 + k] = (key << 16) | (uint32_t)((r0 + k) * 1024 + tid);
    }
  }
  static_assert(kBwdVocab == 128, "key = target >> 7");
  int bits = 1;
  while ((1 << bits) <= nvt) ++bits;
  const int passes = (bits + 3) >> 2;
  for (int ps = 0; ps < passes; ++ps) {
    uint32_t* dst = (ps & 1) ? buf0 : buf1;
    const int sh = 16 + 4 * ps;
#pragma unroll
    for (int r = 0; r < MAXR; ++r) {
      if (r >= rounds) break;
      const int d = valid(r) ? (int)((x[r] >> sh) & 15u) : 16;
      // lane dd < 16 stores the wave's count of digit dd (lanes of digit dd: digit_lanes(dd))
      const uint64_t m = digit_lanes(d, lane);
      if (lane < 16) cnt[(r * 16 + wave) * 16 + lane] = __popcll(m);
    }
    __syncthreads();
    {  // wave dd: exclusive prefix of digit dd over the (round, wave) pairs, in order
      const int tot = wave_prefix(rounds * 16, 16, wave);
      if (lane == 0) dstart[wave] = tot;  // digit total, turned into starts below
    }
    __syncthreads();
    if (tid == 0) {
      int acc = 0;
      for (int dd = 0; dd < 16; ++dd) {
        const int c = dstart[dd];
        dstart[dd] = acc;
        acc += c;
      }
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < MAXR; ++r) {
      if (r >= rounds) break;
      const int d = valid(r) ? (int)((x[r] >> sh) & 15u) : 16;
      const uint64_t mine = digit_lanes(d, d);  // the lanes holding this lane's digit
      if (valid(r)) dst[dstart[d] + cnt[(r * 16 + wave) * 16 + d] + __popcll(mine & lt)] = x[r];
    }
    __syncthreads();  // this pass's stores are visible to the workgroup (and cnt free)
#pragma unroll
    for (int r = 0; r < MAXR; ++r) x[r] = valid(r) ? dst[r * 1024 + tid] : 0u;
  }
  const uint32_t* fin = (passes & 1) ? buf1 : buf0;
  // Rows per key from the runs of the sorted keys: the first element of a run records
  // where it starts, the last one the run's length.
  uint32_t nb[MAXR];
#pragma unroll
  for (int r = 0; r < MAXR; ++r) {
    const int s = r * 1024 + tid;
    nb[r] = (valid(r) && s > 0) ? fin[s - 1] : 0xFFFFFFFFu;
  }
#pragma unroll
  for (int r = 0; r < MAXR; ++r)
    if (valid(r) && (nb[r] >> 16) != (x[r] >> 16)) hist[x[r] >> 16] = r * 1024 + tid;
#pragma unroll
  for (int r = 0; r < MAXR; ++r) {
    const int s = r * 1024 + tid;
    nb[r] = (valid(r) && s + 1 < N) ? fin[s + 1] : 0xFFFFFFFFu;
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < MAXR; ++r)
    if (valid(r) && (nb[r] >> 16) != (x[r] >> 16)) hist[x[r] >> 16] = r * 1024 + tid + 1 - hist[x[r] >> 16];
  __syncthreads();
  // Head / tail ranks in sorted order (rounds, waves, lanes in order).
#pragma unroll
  for (int r = 0; r < MAXR; ++r) {
    if (r >= rounds) break;
    const bool head = valid(r) && hist[x[r] >> 16] >= kSortHeadRun;
    const uint64_t m = __ballot(head);
    if (lane == 0) cnt[r * 16 + wave] = __popcll(m);
  }
  __syncthreads();
  if (wave == 0) {
    const int tot = wave_prefix(rounds * 16, 1, 0);
    if (lane == 0) dstart[16] = tot;  // head rows
  }
  __syncthreads();
  const int nH = dstart[16], nT = N - nH;
  const int nrb = (N + kBwdTokens - 1) / kBwdTokens;
  for (int b = tid; b <= nrb; b += 1024) tbl[b] = (int)((int64_t)min(b * kBwdTokens, N) * nT / N);
  __syncthreads();
  auto tb = [&](int b) { return tbl[b]; };                              // tail rows before block b
  auto hb = [&](int b) { return min(b * kBwdTokens, N) - tbl[b]; };   // head rows before block b
#pragma unroll
  for (int r = 0; r < MAXR; ++r) {
    if (r >= rounds) break;
    const int s = r * 1024 + tid;
    const bool head = valid(r) && hist[x[r] >> 16] >= kSortHeadRun;
    const uint64_t m = __ballot(head);
    if (valid(r)) {
      const int hr = cnt[r * 16 + wave] + __popcll(m & lt);  // head rank
      int pos;
      if (head) {  // last block b with hb(b) <= hr
        int lo = 0, hi = nrb - 1;
        while (lo < hi) {
          const int mid = (lo + hi + 1) >> 1;
          if (hb(mid) <= hr) lo = mid; else hi = mid - 1;
        }
        pos = lo * kBwdTokens + (tb(lo + 1) - tb(lo)) + (hr - hb(lo));
      } else {  // last block b with tb(b) <= tail rank
        const int tr = s - hr;
        int lo = 0, hi = nrb - 1;
        while (lo < hi) {
          const int mid = (lo + hi + 1) >> 1;
          if (tb(mid) <= tr) lo = mid; else hi = mid - 1;
        }
        pos = lo * kBwdTokens + (tr - tb(lo));
      }
      a.perm[pos] = (int)(x[r] & 0xFFFFu);
    }
  }
}

// The sort and the filter in one launch: workgroup 0 sorts (one CU) while the
// others run the filter items, 16 per workgroup (one per wave).
template <int MAXR>
__global__ __launch_bounds__(1024) void bwd_filter_sort_kernel(BwdArgs a) {
  if (blockIdx.x == 0) {
    sort_rows<MAXR>(a);
    return;
  }
  filter_item(a, (blockIdx.x - 1) * 16 + (threadIdx.x >> 6));
}

// The same token order by a counting sort, for up to kCsKeys keys and 16 rounds
// (N <= 16384), in far fewer workgroup-wide steps than the radix passes.  Wave w
// holds rows [w S, (w + 1) S), S = ceil(N / 16), 64 per round in row order.
//   1. Per round, the lanes holding the same key find each other (a ballot per key
//      bit); a lane's place among the wave's earlier rows of its key is the wave's
//      running count of that key (an LDS counter per wave and key) plus the lower
//      lanes with its key; the highest such lane advances the counter.
//   2. Per key, the counters become an exclusive prefix over the waves and give the
//      key's total; scans over the keys (two per thread, in key order) give every
//      key's first place among the head rows (keys with kSortHeadRun or more rows)
//      or among the tail rows.
//   3. A row's head or tail rank is its key's start plus its place among the key's
//      rows; the block placement is the radix path's.  The order is assembled in
//      LDS and written out in row order.
constexpr int kCsKeys = 2048;
template <int MAXR>
__device__ void csort_rows(const BwdArgs& a) {
  static_assert(MAXR <= 16, "per-wave counts fit 16 bits: N <= 16384");
  __shared__ uint16_t cnt[16 * kCsKeys];          // [wave][key]
  __shared__ int kinfo[kCsKeys];                  // 2 (first head or tail rank of the key) + is-head
  __shared__ int tbl[MAXR * 1024 / kBwdTokens + 1];  // tail rows before each block
  __shared__ int wsum[16];
  __shared__ int pl[MAXR * 1024];  // the order, written out in one coalesced pass (stores
                                   // from one workgroup to scattered places run ~1 ns each)
  const int N = (int)a.N, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nvt = (int)a.plan.nvt;
  const int S = (N + 15) >> 4;
  const uint64_t lt = (1ull << lane) - 1ull;
  for (int i = tid; i < 16 * kCsKeys / 2; i += 1024) reinterpret_cast<uint32_t*>(cnt)[i] = 0u;
  uint32_t key[MAXR];
  bool val[MAXR];
#pragma unroll
  for (int r0 = 0; r0 < MAXR; r0 += 8) {
    int64_t t[8];
    float g[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int j = (r0 + k) * 64 + lane, row = wave * S + j;
      val[r0 + k] = j < S && row < N;
      t[k] = val[r0 + k] ? a.targets[row] : -1;
      g[k] = val[r0 + k] ? a.d_nll[row] : 0.f;
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const bool act = g[k] != 0.f && !(a.has_ignore && t[k] == a.ignore_index) && t[k] >= 0 && t[k] < a.V;
      key[r0 + k] = act ? (uint32_t)(t[k] >> 7) : (uint32_t)nvt;  // t / kBwdVocab
    }
  }
  static_assert(kBwdVocab == 128, "key = target >> 7");
  __syncthreads();
  uint16_t* mine = cnt + wave * kCsKeys;
  int rk[MAXR];  // place among the wave's earlier rows of the key
#pragma unroll
  for (int j = 0; j < MAXR; ++j) {
    rk[j] = 0;
    if (j * 64 >= S) continue;  // uniform
    uint64_t m = __ballot(val[j]);
#pragma unroll
    for (int b = 0; b < 11; ++b) {
      const uint64_t q = __ballot((key[j] >> b) & 1u);
      m &= ((key[j] >> b) & 1u) ? q : ~q;
    }
    const int base = val[j] ? (int)mine[key[j]] : 0;
    rk[j] = base + __popcll(m & lt);
    if (val[j] && (m >> lane) == 1ull) mine[key[j]] = (uint16_t)(base + __popcll(m));
  }
  __syncthreads();
  // keys 2 tid and 2 tid + 1: prefix over the waves, totals, head / tail starts
  int tot[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int k = 2 * tid + u;
    int run = 0;
    if (k <= nvt) {
#pragma unroll
      for (int w = 0; w < 16; ++w) {
        const int c = cnt[w * kCsKeys + k];
        cnt[w * kCsKeys + k] = (uint16_t)run;
        run += c;
      }
    }
    tot[u] = run;
  }
  const int h0 = tot[0] >= kSortHeadRun ? tot[0] : 0, h1 = tot[1] >= kSortHeadRun ? tot[1] : 0;
  int nH, nall;
  const int hs = block_excl_scan(h0 + h1, wsum, nH);
  const int as = block_excl_scan(tot[0] + tot[1], wsum, nall);
  if (2 * tid <= nvt) kinfo[2 * tid] = h0 ? (hs << 1) | 1 : (as - hs) << 1;
  if (2 * tid + 1 <= nvt) kinfo[2 * tid + 1] = h1 ? ((hs + h0) << 1) | 1 : (as + tot[0] - hs - h0) << 1;
  const int nT = N - nH;
  const int nrb = (N + kBwdTokens - 1) / kBwdTokens;
  for (int b = tid; b <= nrb; b += 1024) tbl[b] = (int)((int64_t)min(b * kBwdTokens, N) * nT / N);
  __syncthreads();
  // A head rank r goes to the last block b with hb(b) <= r, a tail rank to the last
  // with tb(b) <= r (tb(b) = tbl[b] tail rows and hb(b) = min(128 b, N) - tbl[b] head
  // rows before block b, both non-decreasing from 0).  The search is binary lifting
  // over fixed steps (nrb <= 8 MAXR) without branches, so that the rows' chains of
  // LDS reads interleave; rows past N compute a place and store nothing.
  static_assert(MAXR * 1024 / kBwdTokens <= 8 * MAXR, "the steps reach every block");
#pragma unroll
  for (int j = 0; j < MAXR; ++j) {
    const int info = kinfo[key[j]];
    const int r = (info >> 1) + (int)cnt[wave * kCsKeys + key[j]] + rk[j];
    const bool head = (info & 1) != 0;
    int lo = 0;
#pragma unroll
    for (int step = 4 * MAXR; step >= 1; step >>= 1) {
      const int c = lo + step;  // <= 8 MAXR - 1: inside tbl
      const int t = tbl[min(c, nrb)];
      const int f = head ? min(c * kBwdTokens, N) - t : t;
      lo = c < nrb && f <= r ? c : lo;
    }
    const int t0 = tbl[lo], t1 = tbl[lo + 1];
    const int pos = lo * kBwdTokens + (head ? (t1 - t0) + r - (min(lo * kBwdTokens, N) - t0) : r - t0);
    if (val[j]) pl[pos] = wave * S + j * 64 + lane;
  }
  __syncthreads();
  for (int i = tid; i < N; i += 1024) a.perm[i] = pl[i];
}

template <int MAXR>
__global__ __launch_bounds__(1024) void bwd_filter_csort_kernel(BwdArgs a) {
  if (blockIdx.x == 0) {
    csort_rows<MAXR>(a);
    return;
  }
  filter_item(a, (blockIdx.x - 1) * 16 + (threadIdx.x >> 6));
}

// Pointers of the per-row data the G kernel and the sums read -- the sorted copies
// when the compaction chose the sorted token order -- and the map from the row
// order they work in to the rows of dE (perm; null for the input order).
struct RowData {
  const char* e;
  const int64_t* targets;
  const float* lse;
  const float* d_nll;
  const int* map;
};
__device__ __forceinline__ RowData row_data(const BwdArgs& a) {
  if (a.perm && ldu(a.counts, kPermFlag) != 0)
    return RowData{reinterpret_cast<const char*>(a.e_perm), a.t_perm, a.lse_perm, a.dnll_perm, a.perm};
  return RowData{reinterpret_cast<const char*>(a.e), a.targets, a.lse, a.d_nll, nullptr};
}

// Row copy into the sorted order, when the compaction chose it: one wave per row,
// 8 loads of 16 bytes in flight per lane.
__device__ __forceinline__ void copy_row(const char* __restrict__ src, char* __restrict__ dst, int64_t nb) {
  const int lane = threadIdx.x & 63;
  int64_t o = (int64_t)lane * 16;
  for (; o + 7 * 1024 < nb; o += 8 * 1024) {
    u32x4 v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = *reinterpret_cast<const u32x4*>(src + o + k * 1024);
#pragma unroll
    for (int k = 0; k < 8; ++k) *reinterpret_cast<u32x4*>(dst + o + k * 1024) = v[k];
  }
  for (; o < nb; o += 1024) *reinterpret_cast<u32x4*>(dst + o) = *reinterpret_cast<const u32x4*>(src + o);
}

// Row p of the sorted order gathered from row perm[p], with its target, lse and d_nll
// (by one wave; rows of nb bytes).
__device__ __forceinline__ void permute_row(const BwdArgs& a, int64_t p, int64_t nb) {
  if (p >= a.N) return;  // uniform per wave
  const int64_t r = min((int64_t)a.perm[p], a.N - 1);  // a permutation of [0, N); the clamp only guards the reads
  copy_row(reinterpret_cast<const char*>(a.e) + r * nb, reinterpret_cast<char*>(a.e_perm) + p * nb, nb);
  if ((threadIdx.x & 63) == 0) {
    a.t_perm[p] = a.targets[r];
    a.lse_perm[p] = a.lse[r];
    a.dnll_perm[p] = a.d_nll[r];
  }
}

// Writes to out[] the owners base + o (o < n) with size(o) > 0, largest size first (a
// counting sort over LDS buckets; sizes past the last bucket share it, and the order
// among equal sizes is not fixed), and returns how many there are.  All 1024 threads
// call it.
constexpr int kOrderBuckets = 4096;
template <typename F>
__device__ __forceinline__ int order_by_size(int n, F size, int* out, int base, int* hist, int* wsum) {
  const int tid = threadIdx.x;
  auto bucket = [](int sz) { return kOrderBuckets - 1 - min(sz, kOrderBuckets - 1); };
  for (int i = tid; i < kOrderBuckets; i += 1024) hist[i] = 0;
  __syncthreads();
  for (int o = tid; o < n; o += 1024) {
    const int sz = size(o);
    if (sz > 0) atomicAdd(&hist[bucket(sz)], 1);
  }
  __syncthreads();
  constexpr int PER = kOrderBuckets / 1024;
  int loc[PER], sum = 0;
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    loc[k] = hist[tid * PER + k];
    sum += loc[k];
  }
  int total;
  int pos = block_excl_scan(sum, wsum, total);  // its barriers order the reads above before the writes below
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    hist[tid * PER + k] = pos;
    pos += loc[k];
  }
  __syncthreads();
  for (int o = tid; o < n; o += 1024) {
    const int sz = size(o);
    if (sz > 0) out[atomicAdd(&hist[bucket(sz)], 1)] = base + o;
  }
  __syncthreads();  // hist free for the next call
  return total;
}

// ---------------------------------------------------------------- 2. compaction
// One workgroup of 1024 threads per chunk.  The chunk's bitmap (token block rb,
// word wl) sits in LDS as bm[rb * cwd + wl], with each row's kept count before every
// word (pre).  The chunk's tiles are cut into passes by the exclusive prefix P[v] of
// their kept counts: tile v belongs to pass floor(P[v] / (cap - nrb)) (one pass when
// the chunk fits the G scratch), so every pass keeps fewer than cap pairs.  Slots run
// by pass, then token block, then vocab tile: slot(rb, v) = first slot of (pass,
// rb) + the kept tiles of row rb in the pass before v.  Per vocab tile the kept token
// blocks are listed in vt_slot (ascending), the G tasks cut every (pass, token block)
// run of slots, or every tile's vt_slot run, into runs of at most 4, and per pass the
// owners of the dE and dC sums
// (token blocks, vocab tiles) that hold kept tiles are listed by descending tile
// count.  The pass table gets every pass's ranges, counts and dE write mode; passes
// past the last one the data needs are marked empty.  The token blocks are those of
// the input order or of the sorted order (the first chunk picks one for all chunks).
constexpr int kRbsLds = 8192;  // (pass, token block) slot starts held in LDS when they fit

__global__ __launch_bounds__(1024) void bwd_compact_kernel(BwdArgs a, int chunk) {
  // Workgroups past the first copy the rows into the sorted order (16 rows each, one
  // per wave) while the first compacts: the copy does not wait for the choice of
  // order, and is only read if the sorted order is chosen.
  if (blockIdx.x > 0) {
    permute_row(a, (int64_t)(blockIdx.x - 1) * 16 + (threadIdx.x >> 6), a.D * (int64_t)a.plan.esize);
    return;
  }
  __shared__ uint32_t bm[kCompactMaxWords];
  __shared__ int pre[kCompactMaxWords];     // kept tiles of row rb before word wl
  __shared__ int vpre[kCompactMaxVt + 1];   // kept pairs of the chunk's tiles before tile v
  __shared__ int pvt[kCompactMaxVt + 1];    // first tile of each pass (nv from the pass after the last on)
  __shared__ int rbs_l[kRbsLds + 1];        // rb_start, when the chunk's (pass, block) pairs fit
  __shared__ int hist[kCompactMaxVt + 1];   // the G-task run indices before each pass (kbp), then order_by_size's
  __shared__ uint16_t vt1_rb[kCompactMaxVt];  // the token block of each tile that keeps exactly one
  __shared__ int wsum[16];
  static_assert(kOrderBuckets <= kCompactMaxVt, "order_by_size's buckets fit hist");
  int* kbp = hist;  // G-task run indices of the passes before pass p (free again once the tasks are written)
  const int tid = threadIdx.x;
  const int nrb = (int)a.plan.nrb, nw = (int)a.plan.nwords, nvt = (int)a.plan.nvt;
  const int maxp = (int)a.plan.max_passes;
  const int vlo = chunk * (int)a.plan.chunk_nvt;
  const int nv = min(nvt, vlo + (int)a.plan.chunk_nvt) - vlo;
  const int wlo = vlo >> 5;  // chunks start on a word boundary
  const int cwd = (nv + 31) >> 5;
  const int E = nrb * cwd;

  // Token order (decided by the first chunk for all of them): the sorted blocks'
  // bitmap when it keeps at least 10% fewer pairs than the input blocks' (or as the
  // caller forces with perm_mode).
  __shared__ int sorted;
  if (chunk == 0) {
    int flag = 0;
    if (a.perm) {
      int cn = 0, cs = 0;
      for (int e = tid; e < nrb * nw; e += 1024) {
        const int w = e % nw;
        const int inside = nvt - w * 32;
        const uint32_t m = inside < 32 ? (1u << inside) - 1u : ~0u;
        cn += __builtin_popcount(a.bits[e] & m);
        cs += __builtin_popcount(a.bits_p[e] & m);
      }
      int tn, ts;
      block_excl_scan(cn, wsum, tn);
      block_excl_scan(cs, wsum, ts);
      flag = a.perm_mode == 1 ? 0 : a.perm_mode == 2 ? 1 : ((int64_t)ts * 10 <= (int64_t)tn * 9 ? 1 : 0);
      if (tid == 0 && a.tile_stats) a.tile_stats[2] = tn;  // kept pairs of the input-order blocks
    }
    if (tid == 0) {
      sorted = flag;
      a.counts[kPermFlag] = flag;
    }
  } else if (tid == 0) {
    sorted = a.counts[kPermFlag];
  }
  __syncthreads();
  const uint32_t* bsrc = sorted ? a.bits_p : a.bits;
  if (chunk == 0 && a.g_scaled) {
    // fp16 G tiles: s with max |d_nll| 2^s in [2^13, 2^14) (|G| <= |d_nll|), so G * 2^s
    // neither overflows fp16 nor meets its subnormals above 2^-10 of the largest
    // value; 0 when every d_nll is 0 or one is not finite.
    uint32_t mb = 0u;
    for (int64_t r = tid; r < a.N; r += 1024) mb = max(mb, __float_as_uint(a.d_nll[r]) & 0x7fffffffu);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) mb = max(mb, (uint32_t)__shfl_xor((int)mb, o));
    if ((tid & 63) == 0) wsum[tid >> 6] = (int)mb;
    __syncthreads();
    if (tid == 0) {
      for (int w = 1; w < 16; ++w) mb = max(mb, (uint32_t)wsum[w]);
      int se = 0;
      if (mb >= 0x7f800000u || mb == 0u) se = 0;
      else if (mb < 0x00800000u) se = 120;  // subnormal
      else se = min(120, 14 - ((int)(mb >> 23) - 126));
      a.counts[kGScaleExp] = se;
    }
    __syncthreads();
  }

  for (int e = tid; e < E; e += 1024) {
    const int rb = e / cwd, wl = e - rb * cwd;
    uint32_t x = bsrc[(size_t)rb * nw + wlo + wl];
    const int inside = nv - wl * 32;
    if (inside < 32) x &= (1u << inside) - 1u;
    bm[e] = x;
  }
  __syncthreads();
  for (int rb = tid; rb < nrb; rb += 1024) {
    int acc = 0;
#pragma unroll 8
    for (int wl = 0; wl < cwd; ++wl) {
      pre[rb * cwd + wl] = acc;
      acc += __builtin_popcount(bm[rb * cwd + wl]);
    }
  }
  // kept pairs per tile, then their exclusive prefix (each thread a contiguous run of tiles)
  int kept;
  {
    const int pv = (nv + 1023) >> 10;
    const int v0 = min(nv, tid * pv), v1 = min(nv, v0 + pv);
    int vs = 0;
    for (int v = v0; v < v1; ++v) {
      const int wl = v >> 5, bit = v & 31;
      int c = 0;
#pragma unroll 16
      for (int rb = 0; rb < nrb; ++rb) c += (bm[rb * cwd + wl] >> bit) & 1u;
      vpre[v] = c;
      vs += c;
    }
    int vp = block_excl_scan(vs, wsum, kept);
    for (int v = v0; v < v1; ++v) {
      const int c = vpre[v];
      vpre[v] = vp;
      vp += c;
    }
    if (tid == 0) vpre[nv] = kept;
  }
  __syncthreads();

  // Passes.  With max_passes > 1 the plan has cap >= 2 nrb, so consecutive tiles
  // (at most nrb pairs each) never skip a pass, and every pass holds a tile.
  const int cp = maxp > 1 ? (int)(a.plan.cap - nrb) : 0x7fffffff;
  auto pass_of = [&](int v) { return vpre[v] / cp; };
  for (int v = tid; v < nv; v += 1024) {
    const int p = pass_of(v);
    if (v == 0 || pass_of(v - 1) != p) pvt[p] = v;
  }
  const int npass = pass_of(nv - 1) + 1;  // <= maxp
  for (int p = npass + tid; p <= maxp; p += 1024) pvt[p] = nv;
  __syncthreads();
  // kept tiles of row rb before tile x (0 <= x <= nv), and of row rb in pass p
  auto rowpre = [&](int rb, int x) -> int {
    const int wl = x >> 5;
    if (wl >= cwd) return pre[rb * cwd + cwd - 1] + __builtin_popcount(bm[rb * cwd + cwd - 1]);
    return pre[rb * cwd + wl] + __builtin_popcount(bm[rb * cwd + wl] & ((1u << (x & 31)) - 1u));
  };
  auto pcnt = [&](int p, int rb) { return rowpre(rb, pvt[p + 1]) - rowpre(rb, pvt[p]); };

  // First slot of every (pass, token block): an exclusive scan in that order; and
  // the most kept tiles of one block in each pass (hist, before it holds kbp).
  const int I = npass * nrb;
  for (int p = tid; p < npass; p += 1024) hist[p] = 0;
  __shared__ int ntr[4];  // G tasks with runs of at most 1, 2, 3, 4 slots
  if (tid < 4) ntr[tid] = 0;
  {
    const int per = (I + 1023) >> 10;
    const int i0 = min(I, tid * per), i1 = min(I, i0 + per);
    int sum = 0;
    for (int i = i0; i < i1; ++i) sum += pcnt(i / nrb, i % nrb);
    int tot;
    int pos = block_excl_scan(sum, wsum, tot);  // its barriers order the zeroing of hist before the maxima
    int tr[4] = {0, 0, 0, 0};
    for (int i = i0; i < i1; ++i) {
      const int c = pcnt(i / nrb, i % nrb);
      a.rb_start[i] = pos;
      if (I <= kRbsLds) rbs_l[i] = pos;
      atomicMax(&hist[i / nrb], c);
      pos += c;
#pragma unroll
      for (int r = 0; r < 4; ++r) tr[r] += (c + r) / (r + 1);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tw = wave_sum(tr[r]);
      if ((tid & 63) == 0 && tw > 0) atomicAdd(&ntr[r], tw);
    }
  }
  for (int i = I + tid; i <= maxp * nrb; i += 1024) a.rb_start[i] = kept;
  if (tid == 0 && I <= kRbsLds) rbs_l[I] = kept;
  __syncthreads();
  auto rbs = [&](int i) { return I <= kRbsLds ? rbs_l[i] : a.rb_start[i]; };  // i <= I
  auto slot_of = [&](int p, int rb, int v) { return rbs(p * nrb + rb) + rowpre(rb, v) - rowpre(rb, pvt[p]); };

  // slot lists.  Dense bitmaps (16+ kept tiles per word on average): a wave takes two
  // words at a time, a lane per bit, so the lanes of a row's kept tiles store
  // consecutive slots (the table reads are the same word per half-wave: broadcasts).
  // Sparse ones: a thread per word; a row's kept tiles of one pass hold consecutive
  // slots, so it looks its first slot up and counts on, again after a pass boundary.
  typedef __attribute__((address_space(1))) int gint;
  gint* slot_vt = (gint*)a.slot_vt;
  gint* slot_rb = (gint*)a.slot_rb;
  if (kept >= 16 * E) {
    const int half = (tid >> 5) & 1, bitl = tid & 31;
    for (int e = 2 * (tid >> 6) + half; e < E; e += 32) {
      if (!((bm[e] >> bitl) & 1u)) continue;
      const int rb = e / cwd;
      const int v = (e - rb * cwd) * 32 + bitl;
      const int sl = slot_of(pass_of(v), rb, v);
      slot_vt[sl] = v;
      slot_rb[sl] = rb;
    }
  } else {
    for (int e = tid; e < E; e += 1024) {
      uint32_t x = bm[e];
      if (!x) continue;
      const int rb = e / cwd;
      const int vb = (e - rb * cwd) * 32;
      int v = vb + __builtin_ctz(x);
      int p = pass_of(v);
      int pend = pvt[p + 1];
      int sl = slot_of(p, rb, v);
      for (;;) {
        slot_vt[sl] = v;
        slot_rb[sl] = rb;
        x &= x - 1u;
        if (!x) break;
        v = vb + __builtin_ctz(x);
        if (v >= pend) {
          p = pass_of(v);
          pend = pvt[p + 1];
          sl = slot_of(p, rb, v);
        } else {
          ++sl;
        }
      }
    }
  }
  __shared__ int ntiles;  // the chunk's tiles that keep a pair
  // per vocab tile: its kept token blocks, ascending, as slots.  A tile with few kept
  // blocks takes one thread; when only a few tiles keep many (the tiles of popular
  // targets), each of those takes a wave, a lane per token block, so that no thread
  // walks a long list alone.  (With many such tiles -- the filter off -- threads keep
  // them all: a wave's lanes would read the bitmap a row apart, in one LDS bank.)
  {
    // the lists in global memory, through global-space pointers: the compiler then
    // knows that their stores do not alias the LDS tables it reads next
    gint* vt_slot = (gint*)a.vt_slot;
    gint* vt_start = (gint*)a.vt_start;
    constexpr int kVtWave = 8, kVtWaveTiles = 64;
    const int lane = tid & 63, wv = tid >> 6;
    const uint64_t below = (1ull << lane) - 1ull;
    // the heavy tiles (more than kVtWave kept blocks), listed when they are few
    __shared__ int nheavy;
    __shared__ int heavy[kVtWaveTiles];
    if (tid == 0) {
      nheavy = 0;
      ntiles = 0;
    }
    __syncthreads();
    for (int vb = 0; vb < nv; vb += 1024) {
      const int v = vb + tid;
      const bool hv = v < nv && vpre[v + 1] - vpre[v] > kVtWave;
      const uint64_t m = __ballot(hv);
      const uint64_t mt = __ballot(v < nv && vpre[v + 1] > vpre[v]);
      if (lane == 0 && mt != 0ull) atomicAdd(&ntiles, __builtin_popcountll(mt));
      int base = 0;
      if (lane == 0 && m != 0ull) base = atomicAdd(&nheavy, __builtin_popcountll(m));
      base = __shfl(base, 0);
      const int k = base + __builtin_popcountll(m & below);
      if (hv && k < kVtWaveTiles) heavy[k] = v;
    }
    __syncthreads();
    const int nh = nheavy;
    const int wave_min = nh <= kVtWaveTiles ? kVtWave : 0x7fffffff;  // kept blocks that make a wave's tile
    for (int v = tid; v < nv; v += 1024) {
      vt_start[v] = vpre[v];
      if (vpre[v + 1] - vpre[v] > wave_min) continue;
      const int p = pass_of(v);
      const int wl = v >> 5, bit = v & 31;
      int q = vpre[v];
      for (int r0 = 0; r0 < nrb; r0 += 64) {  // the tile's column of the bitmap, 64 blocks at a time
        const int nr = min(64, nrb - r0);
        uint64_t col = 0;
#pragma unroll 16
        for (int r = 0; r < nr; ++r) col |= (uint64_t)((bm[(r0 + r) * cwd + wl] >> bit) & 1u) << r;
        while (col) {
          const int rb = r0 + __builtin_ctzll(col);
          col &= col - 1ull;
          vt_slot[q++] = slot_of(p, rb, v);
          vt1_rb[v] = (uint16_t)rb;  // (read only for tiles that keep one block)
        }
      }
    }
    for (int i = wv; i < (nh <= kVtWaveTiles ? nh : 0); i += 16) {
      const int v = heavy[i];
      const int p = pass_of(v);
      const int wl = v >> 5, bit = v & 31;
      int q = vpre[v];
      for (int r0 = 0; r0 < nrb; r0 += 64) {
        const int rb = r0 + lane;
        const bool k = rb < nrb && ((bm[rb * cwd + wl] >> bit) & 1u);
        const uint64_t m = __ballot(k);
        if (k) vt_slot[q + __builtin_popcountll(m & below)] = slot_of(p, rb, v);
        q += __builtin_popcountll(m);
      }
    }
  }
  if (tid == 0) a.vt_start[nv] = kept;

  // G tasks.  With the filter on and the tiles keeping three or more blocks each on
  // average: runs of up to 4 of one vocabulary tile's vt_slot entries, tiles in order
  // (the G kernel then reads the tile's C rows once for its blocks; below).  Otherwise
  // runs of at most R consecutive slots of one (pass, token block).  When the
  // tiles keep more than two blocks each on average, they are ordered by pass, then run
  // index, then token block: tasks that run at the same time then read the same
  // vocabulary tiles, and every block's first run (its lowest, most shared tiles) is
  // taken early.  Otherwise (each tile read by few tasks) by pass, then token block,
  // then run index: the tasks an XCD takes at once (a contiguous range) then share few
  // token blocks, whose rows its L2 fetches once.  R is the shortest run (1 to 4) whose
  // tasks all fit one round of the G kernel's persistent grid, else 4: a task streams
  // only its own tiles' rows, and the task's time is the kernel's.  In the first order,
  // item (p, k) -- run index k of pass p, k < ceil(most kept tiles of a block in the
  // pass / R), at least one item per pass -- counts the blocks with more than k runs;
  // the counts are scanned and every item writes its column.
  const int gwg = (a.num_cus > 0 ? a.num_cus + 7 : 256 + 7) / 8 * 8;  // the G kernel's grid
  const int R = ntr[0] <= gwg ? 1 : ntr[1] <= gwg ? 2 : ntr[2] <= gwg ? 3 : 4;
  {
    const int pp = (npass + 1023) >> 10;
    const int p0 = min(npass, tid * pp), p1 = min(npass, p0 + pp);
    int kb[4];  // this thread's passes' item counts (pp <= 4: npass <= 4096)
    int sum = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      kb[q] = p0 + q < p1 ? max(1, (hist[p0 + q] + R - 1) / R) : 0;
      sum += kb[q];
    }
    int J;
    int pos = block_excl_scan(sum, wsum, J);  // its barriers order the reads of hist before the writes of kbp
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (p0 + q < p1) kbp[p0 + q] = pos;
      pos += kb[q];
    }
    if (tid == 0) kbp[npass] = J;
  }
  __syncthreads();
  const int J = kbp[npass];
  auto item_pass = [&](int j) {  // the pass p < npass with kbp[p] <= j < kbp[p + 1]
    int lo = 0, hi = npass - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (kbp[mid] <= j) lo = mid; else hi = mid - 1;
    }
    return lo;
  };
  int ntask;
  // vocabulary-tile tasks: filtered, each tile kept by three or more blocks on average
  const bool gvt = a.g_tiles_ok && a.filter_log_eps > -INFINITY && kept >= 3 * ntiles;
  if (gvt) {
    // per tile of the chunk (a contiguous run of tiles per thread), runs of up to 4 of
    // its vt_slot entries (its kept blocks, ascending)
    const int pv = (nv + 1023) >> 10;
    const int v0 = min(nv, tid * pv), v1 = min(nv, v0 + pv);
    int cnt = 0;
    for (int v = v0; v < v1; ++v) cnt += (vpre[v + 1] - vpre[v] + 3) >> 2;
    int tb = block_excl_scan(cnt, wsum, ntask);
    for (int v = v0; v < v1; ++v) {
      const int p = pass_of(v);
      if (v == pvt[p]) {  // the pass's first tile: its tasks start here
        a.pinfo[p * kPassInts + kPiTask0] = tb;
        a.pinfo[p * kPassInts + kPiRun] = 4;
        if (p > 0) a.pinfo[(p - 1) * kPassInts + kPiTask1] = tb;
      }
      for (int q = vpre[v]; q < vpre[v + 1]; q += 4, ++tb) {
        a.g_task[tb] = q;
        a.g_task_rb[tb] = v;
      }
    }
  } else if (kept <= 2 * ntiles) {
    // (pass, token block) pairs in order, a contiguous run of them per thread, each
    // listing its runs
    const int per = (I + 1023) >> 10;
    const int i0 = min(I, tid * per), i1 = min(I, i0 + per);
    int cnt = 0;
    for (int i = i0; i < i1; ++i) cnt += (rbs(i + 1) - rbs(i) + R - 1) / R;
    int tb = block_excl_scan(cnt, wsum, ntask);
    for (int i = i0; i < i1; ++i) {
      const int p = i / nrb, rb = i - p * nrb;
      if (rb == 0) {  // the pass's first pair: its tasks start here
        a.pinfo[p * kPassInts + kPiTask0] = tb;
        a.pinfo[p * kPassInts + kPiRun] = R;
        if (p > 0) a.pinfo[(p - 1) * kPassInts + kPiTask1] = tb;
      }
      const int b0 = rbs(i), c = rbs(i + 1) - b0;
      for (int k4 = 0; k4 < c; k4 += R, ++tb) {
        a.g_task[tb] = b0 + k4;
        a.g_task_rb[tb] = rb;
      }
    }
  } else {
    // (item, token block) pairs in task order, a contiguous run of them per thread:
    // pair f = j nrb + rb holds a task when block rb keeps more than R k tiles in the
    // item's pass (k its run index).
    const int P = J * nrb;
    const int per = (P + 1023) >> 10;
    const int f0 = min(P, tid * per), f1 = min(P, f0 + per);
    int cnt = 0;
    {
      int jc = -1, p = 0, k4 = 0;
      for (int f = f0; f < f1; ++f) {
        const int j = f / nrb, rb = f - j * nrb;
        if (j != jc) {
          jc = j;
          p = item_pass(j);
          k4 = R * (j - kbp[p]);
        }
        cnt += rbs(p * nrb + rb + 1) - rbs(p * nrb + rb) > k4 ? 1 : 0;
      }
    }
    int tb = block_excl_scan(cnt, wsum, ntask);
    int jc = -1, p = 0, k4 = 0;
    for (int f = f0; f < f1; ++f) {
      const int j = f / nrb, rb = f - j * nrb;
      if (j != jc) {
        jc = j;
        p = item_pass(j);
        k4 = R * (j - kbp[p]);
      }
      if (k4 == 0 && rb == 0) {  // the pass's first pair: its tasks start here
        a.pinfo[p * kPassInts + kPiTask0] = tb;
        a.pinfo[p * kPassInts + kPiRun] = R;
        if (p > 0) a.pinfo[(p - 1) * kPassInts + kPiTask1] = tb;
      }
      const int b0 = rbs(p * nrb + rb);
      if (rbs(p * nrb + rb + 1) - b0 > k4) {
        a.g_task[tb] = b0 + k4;
        a.g_task_rb[tb] = rb;
        ++tb;
      }
    }
  }
  if (tid == 0) a.pinfo[(npass - 1) * kPassInts + kPiTask1] = ntask;
  // kbp lives in hist, which order_by_size clears first thing: every thread must be
  // done with the task lists before any thread starts on the owners.
  __syncthreads();

  // the owners of every pass's sums, most kept tiles first
  __shared__ int pblk;  // the pass's dC sums run block tasks
  for (int p = 0; p < npass; ++p) {
    const int n_rb = order_by_size(nrb, [&](int rb) { return rbs(p * nrb + rb + 1) - rbs(p * nrb + rb); },
                                   a.own_rb + (size_t)p * nrb, 0, hist, wsum);
    const int vt0 = pvt[p];
    const int n_vt = order_by_size(pvt[p + 1] - vt0, [&](int i) { return vpre[vt0 + i + 1] - vpre[vt0 + i]; },
                                   a.own_vt + vt0, vt0, hist, wsum);
    // dC geometry of the pass: the wide one (512 columns, 8 waves) unless its largest
    // owner's tasks alone outlast a workgroup's average share (a popular target's tile
    // keeping many blocks), which the narrow one spreads over twice as many workgroups
    int mk = 0;
    for (int i = tid; i < pvt[p + 1] - vt0; i += 1024) mk = max(mk, vpre[vt0 + i + 1] - vpre[vt0 + i]);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) mk = max(mk, __shfl_xor(mk, o));
    if ((tid & 63) == 0) wsum[tid >> 6] = mk;
    __syncthreads();
    if (tid == 0) {
      for (int w = 1; w < 16; ++w) mk = max(mk, wsum[w]);
      const int64_t kept_p = rbs((p + 1) * nrb) - rbs(p * nrb);
      const int64_t nds_w = (a.D + 511) / 512;
      a.pinfo[p * kPassInts + kPiOwnRb] = n_rb;
      a.pinfo[p * kPassInts + kPiOwnVt] = n_vt;
      const int wide = (int64_t)mk * gwg <= kept_p * nds_w ? 1 : 0;
      a.pinfo[p * kPassInts + kPiDcWide] = wide;
      if (a.host_pass) a.host_pass[1 + p] = wide;
      // block tasks when the pass's dC sums run in the narrow geometry
      pblk = a.dc_blk && nrb <= kDcBlkMaxRb &&
             (a.dc_geo == 2 || (a.dc_geo == 0 && a.filter_log_eps > -INFINITY && wide == 0));
      a.pinfo[p * kPassInts + kPiDcBlk] = 0;
      a.pinfo[p * kPassInts + kPiDcDeal] = n_vt;
    }
    __syncthreads();  // wsum is the next scan's
    if (pblk) {
      // The pass's tiles that keep one token block (its last owners in own_vt), grouped
      // by that block: counts per block (hist, free until the next pass's ordering) and
      // each tile's place among its block's tiles, in the order the LDS atomics hand
      // out (the sums do not depend on it); tasks listed in token-block order.
      int* cntb = hist;
      for (int r = tid; r < nrb; r += 1024) cntb[r] = 0;
      __syncthreads();
      constexpr int kTq = kCompactMaxVt / 1024;
      int rk[kTq];
#pragma unroll
      for (int q = 0; q < kTq; ++q) {
        const int v = vt0 + tid + 1024 * q;
        rk[q] = v < pvt[p + 1] && vpre[v + 1] - vpre[v] == 1 ? atomicAdd(&cntb[vt1_rb[v]], 1) : -1;
      }
      __syncthreads();
      // tasks of at most kDcBlkChunk owners of one block
      const int perb = (nrb + 1023) >> 10;
      const int r0 = min(nrb, tid * perb), r1 = min(nrb, r0 + perb);
      int fb = 0, cb = 0;
      for (int r = r0; r < r1; ++r) {
        fb += (cntb[r] + kDcBlkChunk - 1) / kDcBlkChunk;
        cb += cntb[r];
      }
      int ntk, ones;
      int kb = block_excl_scan(fb, wsum, ntk);
      int ob = block_excl_scan(cb, wsum, ones);
      int* task = a.dc_blk_task + 4 * vt0;
      for (int r = r0; r < r1; ++r) {
        const int c = cntb[r];
        for (int e = 0; e < c; e += kDcBlkChunk, ++kb) {
          task[4 * kb] = r;
          task[4 * kb + 1] = ob + e;
          task[4 * kb + 2] = ob + min(c, e + kDcBlkChunk);
          task[4 * kb + 3] = 0;
        }
        cntb[r] = ob;  // the block's first entry
        ob += c;
      }
      if (tid == 0) {
        a.pinfo[p * kPassInts + kPiDcBlk] = ntk;
        a.pinfo[p * kPassInts + kPiDcDeal] = n_vt - ones;
      }
      __syncthreads();
#pragma unroll
      for (int q = 0; q < kTq; ++q) {
        if (rk[q] < 0) continue;
        const int v = vt0 + tid + 1024 * q, rb = vt1_rb[v];
        const int e = vt0 + cntb[rb] + rk[q];
        a.dc_blk_own[2 * e] = v;
        a.dc_blk_own[2 * e + 1] = slot_of(p, rb, v);
      }
      __syncthreads();  // hist is the next pass's
    }
  }
  // the rest of the pass table
  const bool multi = a.plan.n_chunks > 1 || npass > 1;
  const int last_chunk = (int)a.plan.n_chunks - 1;
  for (int p = tid; p < maxp; p += 1024) {
    int* pi = a.pinfo + p * kPassInts;
    pi[kPiTail] = 0;
    pi[kPiDcQueue] = 0;
    pi[kPiGVt] = gvt ? 1 : 0;
    if (p < npass) {
      pi[kPiVt0] = pvt[p];
      pi[kPiVt1] = pvt[p + 1];
      pi[kPiS0] = rbs(p * nrb);
      pi[kPiS1] = rbs((p + 1) * nrb);
      pi[kPiDeMode] = !multi ? kWriteT
                             : (chunk == 0 && p == 0) ? kStoreF32
                                                      : (chunk == last_chunk && p == npass - 1) ? kFinishT : kAddF32;
    } else {
      pi[kPiVt0] = nv;
      pi[kPiVt1] = nv;
      pi[kPiS0] = kept;
      pi[kPiS1] = kept;
      pi[kPiTask0] = ntask;
      pi[kPiTask1] = ntask;
      pi[kPiOwnRb] = 0;
      pi[kPiOwnVt] = 0;
      pi[kPiDcBlk] = 0;
      pi[kPiDcDeal] = 0;
      pi[kPiDeMode] = -1;
    }
  }
  if (tid == 0 && a.host_pass) {  // the host launches exactly these passes
    a.host_pass[0] = npass;
    __threadfence_system();
  }
  if (tid == 0 && a.tile_stats) {  // [2]: already set from the whole bitmap when the sorted order was available
    if (chunk == 0) {
      a.tile_stats[0] = kept;
      a.tile_stats[1] = a.plan.total;
      if (!a.perm) a.tile_stats[2] = kept;
    } else {
      a.tile_stats[0] += kept;
      if (!a.perm) a.tile_stats[2] += kept;
    }
  }
}

// ---------------------------------------------------------------- 3. owners without kept tiles
// Item o of a pass: token block rb = o < nrb (dE rows), then the pass's vocab tiles
// (dC rows).  In the pass's dE write mode, a block without kept tiles in the pass
// gets zero dE rows (kWriteT: one pass over everything), zero carry rows (kStoreF32:
// the first pass), its carry converted to the output dtype (kFinishT: the last
// pass), or nothing (kAddF32); blocks with kept tiles are stored / added / finished by
// the dE sums themselves.  A vocab tile of the pass without kept blocks gets zero dC
// rows.  NT threads work on one item.  The G kernel's workgroups take these items
// once they run out of G tasks.
template <typename T, int NT>
__device__ __forceinline__ void empty_owner(const BwdArgs& a, int chunk, int pass, int o) {
  const int nrb = (int)a.plan.nrb;
  const int* pi = a.pinfo + pass * kPassInts;
  const int vlo = chunk * (int)a.plan.chunk_nvt;
  const int64_t D = a.D;
  if (o < nrb) {
    if (!a.dE || ldu(a.rb_start, pass * nrb + o + 1) != ldu(a.rb_start, pass * nrb + o)) return;
    const int mode = ldu(pi, kPiDeMode);
    if (mode == kAddF32) return;
    const int64_t row0 = (int64_t)o * kBwdTokens;
    const int64_t nrows = a.N - row0 < kBwdTokens ? a.N - row0 : kBwdTokens;
    const int* map = row_data(a).map;  // dE row of each row of the block (null: the same)
    T* dE = reinterpret_cast<T*>(a.dE);
    if (mode == kWriteT) {
      for (int64_t r = 0; r < nrows; ++r) {
        T* out = dE + (map ? (int64_t)map[row0 + r] : row0 + r) * D;
        for (int64_t i = (int64_t)threadIdx.x * (16 / sizeof(T)); i < D; i += NT * (16 / sizeof(T)))
          *reinterpret_cast<u32x4*>(out + i) = u32x4{0u, 0u, 0u, 0u};
      }
    } else if (mode == kStoreF32) {
      float* acc = a.de_acc + row0 * D;
      for (int64_t i = (int64_t)threadIdx.x * 4; i < nrows * D; i += NT * 4)
        *reinterpret_cast<f32x4*>(acc + i) = f32x4{0.f, 0.f, 0.f, 0.f};
    } else {
      for (int64_t r = 0; r < nrows; ++r) {
        const float* acc = a.de_acc + (row0 + r) * D;
        T* out = dE + (map ? (int64_t)map[row0 + r] : row0 + r) * D;
        for (int64_t i = (int64_t)threadIdx.x * 4; i < D; i += NT * 4) {
          const f32x4 x = *reinterpret_cast<const f32x4*>(acc + i);
#pragma unroll
          for (int k = 0; k < 4; ++k) out[i + k] = (T)x[k];
        }
      }
    }
    return;
  }
  const int v = ldu(pi, kPiVt0) + (o - nrb);
  if (v >= ldu(pi, kPiVt1) || !a.dC || ldu(a.vt_start, v + 1) != ldu(a.vt_start, v)) return;
  const int64_t row0 = (int64_t)(vlo + v) * kBwdVocab;
  const int64_t n = (a.V - row0 < kBwdVocab ? a.V - row0 : kBwdVocab) * D;
  T* out = reinterpret_cast<T*>(a.dC) + row0 * D;
  for (int64_t i = (int64_t)threadIdx.x * (16 / sizeof(T)); i < n; i += NT * (16 / sizeof(T)))
    *reinterpret_cast<u32x4*>(out + i) = u32x4{0u, 0u, 0u, 0u};
}

// ---------------------------------------------------------------- dC schedule
// The dC sums run one D slice of kDcSliceCols columns per workgroup and deal the
// chunk's dC owners (vocab tiles with kept blocks) to bins: workgroup v takes bin
// v / nds at slice v % nds, so every slice of an owner runs at the same time, in
// the same order, on one XCD.  With more slices than workgroups there is one bin
// and workgroup v takes slices v, v + nwg, ...
constexpr int kDcSliceCols = 256;
__host__ __device__ inline int dc_bins(int nwg, int nds) {
  return nds <= nwg ? (nwg / nds < kMaxDcBins ? nwg / nds : kMaxDcBins) : 0;
}

// Longest-processing-time-first dealing of the dC owners of a pass (own_vt: most kept
// blocks first) to nbins bins: each owner goes to the bin with the least work so far
// (ties: lowest bin).  An owner's work is its pipeline steps (spt per kept block) plus
// kDcOwnerCost for its epilogue and pipeline restart.  Owners of equal size form a
// batch, dealt at once by water-filling: bin b offers the work levels W_b, W_b + w,
// W_b + 2w, ... (w = the owners' work) and dealing one at a time takes the c lowest
// levels, ties to the lower bin; so the smallest level L at which c levels are
// available is found by bisection, every bin takes its levels below L, and the rest
// go to the bins with a level exactly at L in bin order.  A bin lists its owners in
// dealing order.  Run by one workgroup of NT threads (the bisection by wave 0);
// smem holds its tables.
constexpr int kDcOwnerCost = 3;  // a task's epilogue and restart, in pipeline steps (measured at c3)
// pipeline steps of the narrow dC sums per kept tile: one per 128-byte G row slice
template <typename T>
constexpr int dc_steps_per_tile(bool split) {
  return kBwdVocab / (split ? 32 : 128 / (int)sizeof(T));
}

__device__ __forceinline__ int wave_min(int v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = min(v, __shfl_xor(v, o));
  return v;
}

template <int NT>
__device__ void dc_schedule(const BwdArgs& a, int pass, int nbins, int spt, char* smem) {
  constexpr int NW = NT / 64;
  const int tid = threadIdx.x;
  const int* pi = a.pinfo + pass * kPassInts;
  const int n = ldu(pi, kPiDcDeal);  // owners dealt to bins: the rest are block tasks
  const int* own_vt = a.own_vt + ldu(pi, kPiVt0);
  int* sz = reinterpret_cast<int*>(smem);  // [n] kept blocks of owner i
  int* bst = sz + kCompactMaxVt;           // [batches + 1] first owner of each batch
  int* bin = bst + kCompactMaxVt + 1;      // [n] bin of owner i
  int* pos = bin + kCompactMaxVt;          // [n] place of owner i in its bin
  int* work = pos + kCompactMaxVt;         // [nbins] work dealt so far, then bin starts
  int* cnt = work + kMaxDcBins;            // [nbins] owners dealt so far
  int* take = cnt + kMaxDcBins;            // [nbins] owners of the current batch per bin
  int* pre = take + kMaxDcBins;            // [nbins] first owner of the batch per bin
  int* wsum = pre + kMaxDcBins;            // [NW]
  for (int i = tid; i < n; i += NT) {
    const int v = own_vt[i];
    sz[i] = a.vt_start[v + 1] - a.vt_start[v];
  }
  for (int b = tid; b < kMaxDcBins; b += NT) {
    work[b] = 0;
    cnt[b] = 0;
  }
  __syncthreads();
  const int per = (n + NT - 1) / NT;
  const int i0 = min(n, tid * per), i1 = min(n, i0 + per);
  int f = 0;
  for (int i = i0; i < i1; ++i) f += (i == 0 || sz[i] != sz[i - 1]) ? 1 : 0;
  int nb;
  int p = block_excl_scan<NW>(f, wsum, nb);
  for (int i = i0; i < i1; ++i)
    if (i == 0 || sz[i] != sz[i - 1]) bst[p++] = i;
  if (tid == 0) bst[nb] = n;
  __syncthreads();
  for (int bt = 0; bt < nb; ++bt) {
    const int b0 = bst[bt], c = bst[bt + 1] - b0;
    const int w = spt * sz[b0] + kDcOwnerCost;
    if (tid < 64) {
      const int lane = tid;
      int wmin = INT_MAX;
      for (int b = lane; b < nbins; b += 64) wmin = min(wmin, work[b]);
      wmin = wave_min(wmin);
      // levels at or below L over all bins
      auto levels = [&](int L) {
        int k = 0;
        for (int b = lane; b < nbins; b += 64) {
          const int wb = work[b];
          k += L >= wb ? (L - wb) / w + 1 : 0;
        }
        return wave_sum(k);
      };
      int lo = wmin, hi = wmin + (c - 1) * w;  // the least loaded bin alone has c levels up to hi
      while (lo < hi) {
        const int mid = lo + (hi - lo) / 2;
        if (levels(mid) >= c)
          hi = mid;
        else
          lo = mid + 1;
      }
      const int L = lo;
      int below = 0;
      for (int b = lane; b < nbins; b += 64) {
        const int wb = work[b];
        const int k = L > wb ? (L - 1 - wb) / w + 1 : 0;
        take[b] = k;
        below += k;
      }
      int rest = c - wave_sum(below);  // 1 .. the bins with a level at L
      int carry = 0;
      for (int base = 0; base < nbins; base += 64) {
        const int b = base + lane;
        const int at = (b < nbins && rest > 0 && L >= work[b] && (L - work[b]) % w == 0) ? 1 : 0;
        const int r = wave_incl_scan(at);
        if (at && r <= rest) take[b] += 1;
        rest -= min(rest, __shfl(r, 63));
        const int v = b < nbins ? take[b] : 0;
        const int incl = wave_incl_scan(v);
        if (b < nbins) pre[b] = carry + incl - v;
        carry += __shfl(incl, 63);
      }
    }
    __syncthreads();
    for (int t = tid; t < c; t += NT) {  // owner t goes to the last bin whose first owner is at or before it
      int lo = 0, hi = nbins - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (pre[mid] <= t)
          lo = mid;
        else
          hi = mid - 1;
      }
      bin[b0 + t] = lo;
      pos[b0 + t] = cnt[lo] + t - pre[lo];
    }
    __syncthreads();
    for (int b = tid; b < nbins; b += NT) {
      work[b] += take[b] * w;
      cnt[b] += take[b];
    }
    __syncthreads();
  }
  if (tid == 0) {
    int acc = 0;
    for (int b = 0; b < nbins; ++b) {
      work[b] = acc;
      a.dc_bin_start[b] = acc;
      acc += cnt[b];
    }
    a.dc_bin_start[nbins] = acc;
  }
  __syncthreads();
  for (int i = tid; i < n; i += NT) a.dc_bin_owner[work[bin[i]] + pos[i]] = own_vt[i];
}

// ---------------------------------------------------------------- 4. G tiles
// Task = up to 4 consecutive slots of one token block (its kept vocab tiles in this
// chunk).  The 128 x 128 logit tiles of the task's 4 vocab tiles are recomputed
// with the forward's main loop over the gathered 512 C rows and the block's 128 E
// rows; 8 waves, wave (wa, wb) = (w % 4, w / 4) owns vocab tile wa and tokens
// [64 wb, 64 wb + 64).  Waves whose vocab tile is beyond the task's count compute a
// duplicate and store nothing.  The kernel is persistent: a workgroup issues the
// next task's pipeline fill before it forms G of the current one.  Tasks are taken
// XCD-major (consecutive tasks on one XCD) so tasks that run together share C rows
// in that XCD's L2.
#ifndef CCE_G_SLICE
#define CCE_G_SLICE 128
#endif
#ifndef CCE_G_STAGES
#define CCE_G_STAGES 2
#endif
constexpr int kGSlice = CCE_G_SLICE, kGStages = CCE_G_STAGES;
template <typename T>
using GLoop = NTMainLoop<T, 4 * kBwdVocab, kBwdTokens, 4, 2, kGSlice, kGStages>;  // A = 4 x 128 C rows, B = 128 E rows
template <typename T>  // vocabulary-tile tasks: A = 4 x 128 E rows, B = 128 C rows, MFMAs swapped
using GTLoop = NTMainLoop<T, 4 * kBwdTokens, kBwdVocab, 8, 1, kGSlice, kGStages, true>;
constexpr int kGThreads = GLoop<__bf16>::NTHREADS;

// G of one wave's 128 x 64 block of a tile from its logits w: w[i][j][r] is the logit
// of vocabulary v0 + 32 i + 8 (r/4) + 4 h + r%4 and token tok0 + 32 j + n.  Stored
// token-major into the slot's G tile gtile at rows row0 + 32 j + n: fp32 as it is,
// 16-bit types rounded once (rows of 128 columns) or, with a.g_split, as the hi / lo
// pair of g_tile_bytes's layout (fp16 scaled by 2^gexp either way); with WANT_DB the
// block's (unscaled) column sums over its 64 tokens go to red[0, 128).  Per token: g (0 for masked / out-of-range rows), lz =
// lse log2(e), or +inf when g == 0 so that p = 0 and G = 0 without a select, and the
// target's place in the tile as tl - 4 h, which register (i, r) holds iff it equals
// 32 i + 8 (r/4) + r%4 (a compile-time constant).  Columns past V (last vocabulary
// tile) keep finite values: the dE sums read zeros for C rows past V, and dC / dBias
// are never written there.
// A G block's per-token inputs (target, cotangent, lse) for the lane's two token
// columns, loaded together (tokens past N read nothing).
struct GRows {
  int64_t tg[2];
  float dn[2], lse[2];
};
__device__ __forceinline__ GRows g_rows_load(const BwdArgs& a, const RowData& rd, int64_t tok0) {
  GRows r;
  const int n = threadIdx.x & 31;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t tok = tok0 + j * 32 + n;
    const bool ok = tok < a.N;
    r.tg[j] = ok ? rd.targets[tok] : 0;
    r.dn[j] = ok ? rd.d_nll[tok] : 0.f;
    r.lse[j] = ok ? rd.lse[tok] : 0.f;
  }
  return r;
}

// The exponent s of the fp16 G tiles' scale 2^s (0 unless a.g_scaled).
__device__ __forceinline__ int g_scale_exp(const BwdArgs& a) { return a.g_scaled ? ldu(a.counts, kGScaleExp) : 0; }

template <typename T, bool HAS_BIAS, bool WANT_G, bool WANT_DB>
__device__ __forceinline__ void g_block_epilogue(const BwdArgs& a, const RowData& rd, const f32x16 (&w)[4][2],
                                                 int64_t v0, int64_t tok0, int row0, char* gtile, float* red,
                                                 const GRows* pre = nullptr) {
  constexpr int TI = 4, TJ = 2, ES = sizeof(T);
  const int lane = threadIdx.x & 63;
  const int n = lane & 31, h = lane >> 5;
  const T* bias = reinterpret_cast<const T*>(a.bias);
  // fp16: G is formed as (d_nll 2^s) (p - onehot), exact scaling by a power of two;
  // the column sums take it back out
  const int gexp = ES == 2 ? g_scale_exp(a) : 0;
  const float gmul = __builtin_ldexpf(1.f, gexp), gdiv = __builtin_ldexpf(1.f, -gexp);
  float g[TJ], lz[TJ];
  int tl[TJ];
  GRows gr;
  if (pre != nullptr) gr = *pre; else gr = g_rows_load(a, rd, tok0);
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    const int64_t tok = tok0 + j * 32 + n;
    g[j] = 0.f;
    lz[j] = INFINITY;
    tl[j] = -4096;
    if (tok < a.N) {
      const int64_t tg = gr.tg[j];
      g[j] = (a.has_ignore && tg == a.ignore_index) ? 0.f : gr.dn[j] * gmul;
      if (g[j] != 0.f) lz[j] = gr.lse[j] * kLog2e;
      const int64_t loc = tg - v0;
      if (loc >= 0 && loc < kBwdVocab) tl[j] = (int)loc - 4 * h;
    }
  }
  // One 32-column block i at a time: form its 32 G values per lane, store them
  // token-major (4 consecutive vocab columns per store), add their column sums.
  const __amdgpu_buffer_rsrc_t grs =
      __builtin_amdgcn_make_buffer_rsrc(gtile, (short)0, (int)a.plan.g_bytes, 0x00020000);
#pragma unroll
  for (int i = 0; i < TI; ++i) {
    float gv[TJ][16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int c = i * 32 + (r >> 2) * 8 + (r & 3);
      float add = 0.f;
      if (HAS_BIAS) {
        const int64_t v = v0 + c + 4 * h;
        add = v < a.V ? to_f32(bias[v]) * kLog2e : 0.f;
      }
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        const float p = __builtin_amdgcn_exp2f(fmaf(w[i][j][r], kLog2e, add - lz[j]));
        gv[j][r] = g[j] * p - (tl[j] == c ? g[j] : 0.f);
      }
    }
    if constexpr (WANT_G) {
      // Buffer stores at 32-bit offsets within the 128 x 128 tile: row (token)
      // row0 + 32 j + n of 128 ES bytes.  Lane (n, h) holds columns 32 i + 8 q +
      // 4 h + 0..3; for 16-bit types one lane swap per q pair gives every lane the 8
      // consecutive columns 32 i + 16 p + 8 h + 0..7 of the pair (2 p, 2 p + 1).
      if constexpr (ES == 4) {
        const uint32_t lane_off = (uint32_t)((row0 + n) * kBwdVocab * ES + h * 4 * ES);
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const f32x4 v{gv[j][q * 4], gv[j][q * 4 + 1], gv[j][q * 4 + 2], gv[j][q * 4 + 3]};
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), grs,
                                                   lane_off + (uint32_t)((j * 32 * kBwdVocab + i * 32 + q * 8) * ES), 0, 0);
          }
      } else if (!a.g_split) {
        const uint32_t lane_off = (uint32_t)((row0 + n) * kBwdVocab * ES + h * 8 * ES);
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
          uint32_t pk[4][2];
#pragma unroll
          for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int k = 0; k < 2; ++k) pk[q][k] = pack2<T>(gv[j][4 * q + 2 * k], gv[j][4 * q + 2 * k + 1]);
#pragma unroll
          for (int pq = 0; pq < 2; ++pq) {
            u32x4 v;
#pragma unroll
            for (int k = 0; k < 2; ++k) {
              const auto sw = __builtin_amdgcn_permlane32_swap(pk[2 * pq][k], pk[2 * pq + 1][k], false, false);
              v[k] = sw[0];
              v[2 + k] = sw[1];
            }
            __builtin_amdgcn_raw_buffer_store_b128(v, grs,
                                                   lane_off + (uint32_t)((j * 32 * kBwdVocab + i * 32 + pq * 16) * ES), 0, 0);
          }
        }
      } else {
        // The hi / lo pair: rows of 256 elements, column 32 i + c of the tile at
        // element 64 i + c (hi) and 64 i + 32 + c (lo), hi = round(G), lo =
        // round(G - hi) (the difference is exact in fp32).
        constexpr int RP = 2 * kBwdVocab * ES;  // bytes of one G row
        const uint32_t lane_off = (uint32_t)((row0 + n) * RP + h * 8 * ES);
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
          uint32_t pk[2][4][2];
#pragma unroll
          for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int k = 0; k < 2; ++k) {
              const float x0 = gv[j][4 * q + 2 * k], x1 = gv[j][4 * q + 2 * k + 1];
              const T h0 = (T)x0, h1 = (T)x1;
              pk[0][q][k] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
              pk[1][q][k] = pack2<T>(x0 - (float)h0, x1 - (float)h1);
            }
#pragma unroll
          for (int hl = 0; hl < 2; ++hl)
#pragma unroll
            for (int pq = 0; pq < 2; ++pq) {
              u32x4 v;
#pragma unroll
              for (int k = 0; k < 2; ++k) {
                const auto sw = __builtin_amdgcn_permlane32_swap(pk[hl][2 * pq][k], pk[hl][2 * pq + 1][k], false, false);
                v[k] = sw[0];
                v[2 + k] = sw[1];
              }
              __builtin_amdgcn_raw_buffer_store_b128(
                  v, grs, lane_off + (uint32_t)(j * 32 * RP + (i * 64 + hl * 32 + pq * 16) * ES), 0, 0);
            }
        }
      }
    }
    if constexpr (WANT_DB) {
      // column sums over this wave's 64 tokens; lanes n == 0 of each half hold them
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float sm = gv[0][r] + gv[1][r];
        sm += __shfl_xor(sm, 1);
        sm += __shfl_xor(sm, 2);
        sm += __shfl_xor(sm, 4);
        sm += __shfl_xor(sm, 8);
        sm += __shfl_xor(sm, 16);
        if (n == 0) red[i * 32 + (r >> 2) * 8 + h * 4 + (r & 3)] = ES == 2 ? sm * gdiv : sm;
      }
    }
  }
}

// The G kernel's loop over its workgroup's tasks (t = its XCD-major number, then on
// by the grid size).  VT false: a task is a token block with up to 4 kept tiles
// (consecutive slots), A = the tiles' C rows, B = the block's E rows, and wave (wa,
// wb) forms G of tile wa for tokens 64 wb ..; VT true: a task is a vocabulary tile
// with up to 4 of its kept blocks (consecutive vt_slot entries), A = the blocks' E
// rows, B = the tile's C rows, the MFMAs swapped so the accumulators hold the same
// [vocabulary][token] block, and wave w forms G of block w / 2 for tokens 64 (w % 2)
// ..: the tile's C rows are read once for its blocks.  Either way a wave's G block is
// 128 columns x 64 tokens of one slot, formed by g_block_epilogue.
template <typename T, bool HAS_BIAS, bool WANT_G, bool WANT_DB, bool RAGGED, bool VT>
__device__ __forceinline__ void g_task_loop(const BwdArgs& a, int chunk, int pass, char* smem) {
  using Loop = typename std::conditional<VT, GTLoop<T>, GLoop<T>>::type;
  static_assert(Loop::NTHREADS == kGThreads, "one launch shape for every dtype and task kind");
  static_assert(Loop::SMEM_BYTES == GLoop<T>::SMEM_BYTES, "one LDS size for both task kinds");
  constexpr int ES = sizeof(T);
  const int* pi = a.pinfo + pass * kPassInts;
  const int task0 = ldu(pi, kPiTask0);
  const int ntask = ldu(pi, kPiTask1) - task0;
  const int s0 = ldu(pi, kPiS0);  // the scratch holds slot s at s - s0
  const int* rb_start = a.rb_start + pass * (int)a.plan.nrb;
  const int vlo = chunk * (int)a.plan.chunk_nvt;
  const int xcd = (int)(blockIdx.x & 7), lidx = (int)(blockIdx.x >> 3), nper = (int)(gridDim.x >> 3);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t pitch = a.D * (int64_t)ES;
  const RowData rd = row_data(a);
  const char* E = rd.e;
  const char* C = reinterpret_cast<const char*>(a.c);
  (void)lane;

  // VT false: s0 the first slot, rb the block, seg the tiles' first C rows; VT true:
  // s0 the first vt_slot entry, rb the chunk-local tile, seg the blocks' first E rows
  struct Task {
    int s0, rb, cnt;
    int64_t seg[4];
  };
  auto load_task = [&](int t, Task& k) {
    k.s0 = ldu(a.g_task, task0 + t);
    k.rb = ldu(a.g_task_rb, task0 + t);
    if constexpr (VT) {
      k.cnt = min(ldu(pi, kPiRun), ldu(a.vt_start, k.rb + 1) - k.s0);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        k.seg[i] = (int64_t)ldu(a.slot_rb, ldu(a.vt_slot, k.s0 + (i < k.cnt ? i : k.cnt - 1))) * kBwdTokens;
    } else {
      k.cnt = min(ldu(pi, kPiRun), ldu(rb_start, k.rb + 1) - k.s0);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        k.seg[i] = (int64_t)(vlo + ldu(a.slot_vt, k.s0 + (i < k.cnt ? i : k.cnt - 1))) * kBwdVocab;
    }
  };
  // the rows of A segments past the task's count are not loaded (their waves compute
  // on stale bytes and store nothing)
  static_assert(Loop::RPL * Loop::NW * 2 == kBwdVocab && kBwdVocab == kBwdTokens, "two load rounds per A segment");
  static_assert(kGStages == 2, "skipped loads rely on the vmcnt(0) stage waits of two stages");
  auto sources = [&](const Task& k) {
    auto src = VT ? Loop::template make_src<kBwdTokens>(E, a.N, k.seg, C, a.V, (int64_t)(vlo + k.rb) * kBwdVocab,
                                                         pitch, pitch, xcd)
                  : Loop::template make_src<kBwdVocab>(C, a.V, k.seg, E, a.N, (int64_t)k.rb * kBwdTokens, pitch,
                                                       pitch, xcd);
    src.skip = (0xffu << (2 * k.cnt)) & 0xffu;
    return src;
  };
  auto prefetch = [&](const typename Loop::template Src<4>& src) { Loop::template prefetch<RAGGED>(src, smem); };

  int t = xcd * nper + lidx;  // logical task of this workgroup; advances by the grid size
  if (t >= ntask) return;
  Task cur;
  load_task(t, cur);
  auto src = sources(cur);
  prefetch(src);

  for (;;) {
    f32x16 w[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) w[i][j] = zero16();
    Loop::template consume<RAGGED>(src, smem, w);

    const int tn = t + (int)gridDim.x;
    Task nxt;
    if (tn < ntask) {
      load_task(tn, nxt);
      src = sources(nxt);
      prefetch(src);  // all stages but the last; the epilogue below uses the last one's bytes
    }

    // This wave's G block: A segment (tile or block) ia of the task, token half ih.
    const int ia = VT ? wave >> 1 : wave & 3, ih = VT ? wave & 1 : wave >> 2;
    const bool active = ia < cur.cnt;  // uniform per wave
    int64_t sg = cur.seg[0];
#pragma unroll
    for (int k = 1; k < 4; ++k) sg = ia == k ? cur.seg[k] : sg;
    const int slot = VT ? (active ? ldu(a.vt_slot, cur.s0 + ia) : s0) : cur.s0 + ia;
    const int64_t v0 = VT ? (int64_t)(vlo + cur.rb) * kBwdVocab : sg;
    const int64_t t0 = VT ? sg : (int64_t)cur.rb * kBwdTokens;
    float* red = reinterpret_cast<float*>(smem + (Loop::SMEM_BYTES - Loop::STAGE_BYTES));  // [8 waves][128] column sums
    static_assert(8 * kBwdVocab * sizeof(float) <= Loop::STAGE_BYTES, "column sums fit one stage");
    // red: the two token halves of segment ia at red[(2 ia + ih) 128] (VT) or red[(4 ih + ia) 128]
    const int rw = VT ? 2 * ia + ih : 4 * ih + ia;
    if (active)
      g_block_epilogue<T, HAS_BIAS, WANT_G, WANT_DB>(a, rd, w, v0, t0 + 64 * ih, 64 * ih,
                                                     a.gtile + (size_t)(slot - s0) * a.plan.g_bytes,
                                                     red + rw * kBwdVocab);
    if constexpr (WANT_DB) {
      // the two token halves' column sums meet in LDS (the last stage, which no DMA
      // fills until the next task's main loop has passed its first barrier)
      __syncthreads();
      if (active && ih == 0) {
        float* cs = a.colsum + (size_t)(slot - s0) * kBwdVocab;
        const int r0 = VT ? 2 * ia : ia, r1 = VT ? 2 * ia + 1 : 4 + ia;
        for (int c = lane; c < kBwdVocab; c += 64) cs[c] = red[r0 * kBwdVocab + c] + red[r1 * kBwdVocab + c];
      }
      __syncthreads();
    }
    if (tn >= ntask) break;
    t = tn;
    cur = nxt;
  }
}

template <typename T, bool HAS_BIAS, bool WANT_G, bool WANT_DB, bool RAGGED>
__global__ __launch_bounds__(kGThreads, 1) void bwd_g_kernel(BwdArgs a, int chunk, int pass) {
  __shared__ __attribute__((aligned(16))) char smem[GLoop<T>::SMEM_BYTES];
  const int* pi = a.pinfo + pass * kPassInts;
  if (ldu(pi, kPiDeMode) < 0) return;  // past the passes the data needs
  if (ldu(pi, kPiGVt))
    g_task_loop<T, HAS_BIAS, WANT_G, WANT_DB, RAGGED, true>(a, chunk, pass, smem);
  else
    g_task_loop<T, HAS_BIAS, WANT_G, WANT_DB, RAGGED, false>(a, chunk, pass, smem);

  // Once out of tasks, the workgroup takes items from the pass's counter, which the
  // compaction kernel reset (only when dE or dC is wanted): first the dC schedule
  // (when dC is wanted), then the owners without kept tiles in the pass, whose rows it
  // zeroes or finishes (dC rows only when dC did not come zeroed).
  if constexpr (WANT_G) {
    const int sched = a.dC != nullptr ? 1 : 0;
    // dC rows of vocab tiles without kept tiles need zeros unless dC came zeroed
    const int nitems = sched + (int)a.plan.nrb + (a.dc_zeroed ? 0 : ldu(pi, kPiVt1) - ldu(pi, kPiVt0));
    int* box = reinterpret_cast<int*>(smem);
    for (;;) {
      __syncthreads();  // box (and smem) free
      if (threadIdx.x == 0) box[0] = atomicAdd(&a.pinfo[pass * kPassInts + kPiTail], 1);
      __syncthreads();
      const int o = box[0];
      if (o >= nitems) break;
      if (o < sched) {
        const int nds = (int)((a.D + kDcSliceCols - 1) / kDcSliceCols);
        const int nb = dc_bins((int)gridDim.x, nds);
        dc_schedule<kGThreads>(a, pass, nb > 0 ? nb : 1, dc_steps_per_tile<T>(a.g_split != 0),
                               smem + 256);  // its tables start past box
      } else {
        empty_owner<T, kGThreads>(a, chunk, pass, o - sched);
      }
    }
  }
}

// ---------------------------------------------------------------- 4b. G tiles, filter off
// With the filter off a token block keeps every tile of the pass or none, so the kept
// pairs form the pass's whole [token blocks x vocabulary tiles] block: one GEMM's
// worth of logits, computed here with the forward tile kernel's geometry (256 x 256
// workgroup tiles, 8 waves of 128 vocabulary x 64 tokens, rounds of gt token blocks x
// gv vocabulary blocks per XCD that share their rows in that XCD's L2) instead of the
// task list's runs of 512 x 128.  A wave's block is half of one (token block,
// vocabulary tile) G tile; its slot is the block's first slot of the pass plus the
// block's kept tiles before this one (a popcount over the filter's bitmap), and a tile
// the bitmap does not keep is not stored: the kernel is right for any kept set, and
// fast for the full one.  Owners without kept tiles take the tail, as in bwd_g_kernel
// (no dC schedule: the wide dC sums run with it).
template <typename T>
using GDLoop = NTMainLoop<T, 2 * kBwdVocab, 2 * kBwdTokens, 2, 4>;  // A = 256 C rows, B = 256 E rows
// Buffer stores one wave's G block epilogue issues (WANT_G, every one unconditional):
// 4 column blocks x 2 token blocks x (4 for fp32; 2 each for the hi and lo halves of
// the 16-bit pair).  The dense kernel's next first stage barrier lets exactly these
// stay in flight; the count must follow g_block_epilogue's store loops (fewer stores
// would let prefetch loads through), so after a single 16-bit G (16 stores) that
// barrier waits for all of them instead.
template <typename T>
constexpr int kGStoresPerWave = 32;
constexpr int kGDThreads = GDLoop<__bf16>::NTHREADS;

template <typename T, bool HAS_BIAS, bool WANT_G, bool WANT_DB, bool RAGGED>
__global__ __launch_bounds__(kGDThreads, 1) void bwd_g_dense_kernel(BwdArgs a, int chunk, int pass) {
  using Loop = GDLoop<T>;
  static_assert(Loop::NTHREADS == kGDThreads && Loop::TI == 4 && Loop::TJ == 2, "wave block: 128 vocabulary x 64 tokens");
  __shared__ __attribute__((aligned(16))) char smem[Loop::SMEM_BYTES];
  const int* pi = a.pinfo + pass * kPassInts;
  if (ldu(pi, kPiDeMode) < 0) return;  // past the passes the data needs
  const int nrb = (int)a.plan.nrb, nw = (int)a.plan.nwords;
  const int vt0 = ldu(pi, kPiVt0), vt1 = ldu(pi, kPiVt1);
  const int s0 = ldu(pi, kPiS0);  // the G scratch holds slot s at s - s0
  const int* rb_start = a.rb_start + pass * nrb;
  const int vlo = chunk * (int)a.plan.chunk_nvt;
  const RowData rd = row_data(a);
  const uint32_t* bits = rd.map ? a.bits_p : a.bits;  // the token blocks the compaction used
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int wv = wave & 1, wt = wave >> 1;  // NTMainLoop: wa = wave % 2 (vocabulary), wb = wave / 2 (tokens)

  // rounds of gt token blocks (256 rows) x gv vocabulary blocks (2 tiles) per XCD
  const int ntb = (nrb + 1) / 2, nvb = (vt1 - vt0 + 1) / 2;
  const int cpx = (int)(gridDim.x >> 3);
  const int gt = (ntb >= 4 && cpx % 4 == 0) ? 4 : (ntb >= 2 && cpx % 2 == 0) ? 2 : 1;
  const int gv = cpx / gt;
  const int ngv = (nvb + gv - 1) / gv;
  const int rounds = ((ntb + gt - 1) / gt) * ngv;
  const int xcd = (int)(blockIdx.x & 7), member = (int)(blockIdx.x >> 3);
  const int st = member % gt, sv = member / gt;
  const int r_end = (int)((int64_t)(xcd + 1) * rounds / 8);
  auto next_round = [&](int r, int& tb, int& vb) {
    for (; r < r_end; ++r) {
      tb = (r / ngv) * gt + st;
      vb = (r % ngv) * gv + sv;
      if (tb < ntb && vb < nvb) break;
    }
    return r;
  };
  const int64_t pitch = a.D * (int64_t)sizeof(T);
  const char* C = reinterpret_cast<const char*>(a.c);
  auto sources = [&](int tb, int vb) {
    const int64_t seg[1] = {(int64_t)(vlo + vt0 + 2 * vb) * kBwdVocab};
    return Loop::template make_src<2 * kBwdVocab>(C, a.V, seg, rd.e, a.N, (int64_t)tb * 2 * kBwdTokens, pitch, pitch,
                                                  xcd);
  };
  // slot of (token block rb, chunk-local tile vt) of the pass, or -1 when not kept
  auto slot_of = [&](int rb, int vt) {
    const uint32_t* row = bits + (size_t)rb * nw + (vlo >> 5);
    const int* rowi = reinterpret_cast<const int*>(row);
    if (!(((uint32_t)ldu(rowi, vt >> 5) >> (vt & 31)) & 1u)) return -1;
    int cnt = 0;
    for (int w = vt0 >> 5; w <= (vt >> 5); ++w) {
      uint32_t x = (uint32_t)ldu(rowi, w);
      if (w == (vt0 >> 5)) x &= ~((1u << (vt0 & 31)) - 1u);
      if (w == (vt >> 5)) x &= (1u << (vt & 31)) - 1u;
      cnt += __builtin_popcount(x);
    }
    return ldu(rb_start, rb) + cnt;
  };

  int tb = 0, vb = 0;
  int r = next_round((int)((int64_t)xcd * rounds / 8), tb, vb);
  if (r < r_end) {
    auto src = sources(tb, vb);
    Loop::template prefetch<RAGGED>(src, smem);
    float* red = reinterpret_cast<float*>(smem + (Loop::SMEM_BYTES - Loop::STAGE_BYTES));  // [8 waves][128] column sums
    bool stored = false;  // this wave's previous G block stores may still be in flight
    static_assert(8 * kBwdVocab * sizeof(float) <= Loop::STAGE_BYTES, "column sums fit one stage");
    for (;;) {
      f32x16 w[4][2];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) w[i][j] = zero16();
      Loop::template consume<RAGGED, 1, typename Loop::NoHook, kGStoresPerWave<T>>(src, smem, w, typename Loop::NoHook(),
                                                                                     stored);
      int tbn = tb, vbn = vb;
      const int rn = next_round(r + 1, tbn, vbn);
      const int vt = vt0 + 2 * vb + wv;  // this wave's chunk-local vocabulary tile
      const int rb = 2 * tb + (wt >> 1), half = wt & 1;
      const int slot = (vt < vt1 && rb < nrb) ? slot_of(rb, vt) : -1;  // uniform per wave
      // the block's row inputs before the next tile's loads: their wait then does not
      // include the DMA
      GRows gr;
      if (slot >= 0) {
        gr = g_rows_load(a, rd, (int64_t)rb * kBwdTokens + half * 64);
        wait_vmcnt<0>();
      }
      if (rn < r_end) {
        src = sources(tbn, vbn);
        Loop::template prefetch<RAGGED>(src, smem);  // all stages but the last; red uses the last one's bytes
      }
      if (slot >= 0)
        g_block_epilogue<T, HAS_BIAS, WANT_G, WANT_DB>(a, rd, w, (int64_t)(vlo + vt) * kBwdVocab,
                                                       (int64_t)rb * kBwdTokens + half * 64, half * 64,
                                                       a.gtile + (size_t)(slot - s0) * a.plan.g_bytes,
                                                       red + wave * kBwdVocab, &gr);
      stored = WANT_G && !WANT_DB && slot >= 0 && (sizeof(T) == 4 || a.g_split);
      if constexpr (WANT_DB) {
        // the two token halves of a tile are waves wave and wave + 2
        __syncthreads();
        if (slot >= 0 && half == 0) {
          float* cs = a.colsum + (size_t)(slot - s0) * kBwdVocab;
          for (int c = lane; c < kBwdVocab; c += 64) cs[c] = red[wave * kBwdVocab + c] + red[(wave + 2) * kBwdVocab + c];
        }
        __syncthreads();
      }
      if (rn >= r_end) break;
      r = rn;
      tb = tbn;
      vb = vbn;
    }
  }
  // owners without kept tiles in the pass: dE rows, and dC rows unless dC came zeroed
  if constexpr (WANT_G) {
    const int nitems = nrb + (a.dc_zeroed ? 0 : vt1 - vt0);
    int* box = reinterpret_cast<int*>(smem);
    for (;;) {
      __syncthreads();  // box (and smem) free
      if (threadIdx.x == 0) box[0] = atomicAdd(&a.pinfo[pass * kPassInts + kPiTail], 1);
      __syncthreads();
      const int o = box[0];
      if (o >= nitems) break;
      empty_owner<T, kGDThreads>(a, chunk, pass, o);
    }
  }
}

// ---------------------------------------------------------------- 5. sums of G_j . X_j
// Geometry of one sum task: output rows = the owner's 128 rows (tokens for dE,
// vocabulary for dC), output columns = one DN (512) slice of D; contraction over
// the owner's kept tiles, 128 deep each, in slices of KS contraction elements: a
// 128-byte G row slice (fp32 and single 16-bit G: 32 and 64 columns; the hi / lo
// pair of 16-bit G: 32 columns' hi then lo).  Eight waves (two per SIMD): wave
// (wm, wd) = (w % 2, w / 2) owns rows [64 wm, +64) and columns [128 wd, +128) of the
// slice.  A wide slice loads each G slice once for 512 output columns.
//   X region of a stage: KS contraction rows x DN columns of E / C, natural
//     [k][d] layout, 64-byte segments XOR-swizzled by tr_swz(row) so the
//     transposing fragment reads are free of bank conflicts.
//   G region (16 KiB): dE -- 128 G rows (tokens) x the 128-byte row slice, the main
//     loop's 16-byte-chunk swizzle; dC -- KS G rows (tokens = contraction) x the
//     whole G row (128 vocab columns; GTP bytes), read transposed like X.
// With the hi / lo pair (SPLIT) every 16-deep contraction step kp takes one MFMA per
// G half on the same X fragment: the hi fragment (chunks 2 kp + kg of the dE row
// slice, or element columns 64 q + 0..31 of a dC row) and the lo one (chunks
// 4 + 2 kp + kg, or columns 64 q + 32..63).
template <typename T, bool SPLIT>
struct SumGeo {
  static constexpr int ES = sizeof(T);
  static_assert(!SPLIT || ES == 2, "the hi / lo pair is a 16-bit layout");
  static constexpr int NW = 8;                     // waves: 2 (rows) x 4 (column quarters)
  static constexpr int NT = 64 * NW;
  static constexpr int DN = 512;
  static constexpr int KS = SPLIT ? 32 : 128 / ES;  // contraction elements per slice
  static constexpr int SPT = kBwdVocab / KS;       // slices per 128-deep tile
  static constexpr int XP = DN * ES;               // bytes of one X row in LDS
  static constexpr int X_BYTES = KS * XP;          // 32 KiB (hi / lo), 64 KiB (otherwise)
  static constexpr int GTP = (SPLIT ? 2 : 1) * kBwdVocab * ES;  // bytes of one G row
  static constexpr int G_BYTES = 16384;            // 128 x 128 B (dE) = KS x GTP (dC)
  static constexpr int STAGE = X_BYTES + G_BYTES;  // 48 KiB (hi / lo), 80 KiB (otherwise)
  static constexpr int STAGES = SPLIT ? 3 : 2;
  static constexpr int XLW = X_BYTES / 1024 / NW;  // X loads per wave per stage (4 / 8)
  static constexpr int GLW = G_BYTES / 1024 / NW;  // G loads per wave per stage (2)
  static constexpr int LPW = XLW + GLW;
  static constexpr int KE = 32 / ES;               // contraction elements per MFMA step
  static constexpr int NSTORE = 4 * 2 * (ES == 2 ? 2 : 4);  // output stores per wave per task
  static_assert(KS * GTP == G_BYTES && 128 * 128 == G_BYTES, "stage geometry");
  static_assert(STAGES * STAGE <= 163840, "the stages fit the 160 KiB of LDS");
  static_assert((STAGES - 2) * LPW + NSTORE < 64, "in-flight operations must fit vmcnt");
};

// The narrow geometry: 4 waves, 256 output columns, 3 stages of 48 KiB (or 4 of 32 KiB
// with the hi / lo pair) (the dC sums: many owners with one or two kept tiles, where
// a deeper pipeline and shorter epilogues pay more than the wide slice's halved G
// traffic).
// 16-bit output of a 64-row x 128-column wave block straight from the MFMA
// accumulators: lane (n, h) holds columns 8 q + 4 h + 0..3 of row n of each 32 x 32
// block (i, jj); one lane swap between the halves per q pair gives it columns 16 pq +
// 8 h + 0..7, stored as 16 bytes at rowoff[jj] + 2 (d0 + 32 i + 16 pq) (d0: the
// block's first column + 8 h; columns past D and rows with a dropped offset store
// nothing).
template <typename T>
__device__ __forceinline__ void store_direct16(const f32x16 (&acc)[4][2], const __amdgpu_buffer_rsrc_t rs,
                                               const uint32_t (&rowoff)[2], int64_t d0, int64_t D) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      uint32_t pk[4][2];
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int k = 0; k < 2; ++k) pk[q][k] = pack2<T>(acc[i][jj][4 * q + 2 * k], acc[i][jj][4 * q + 2 * k + 1]);
#pragma unroll
      for (int pq = 0; pq < 2; ++pq) {
        u32x4 v;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const auto sw = __builtin_amdgcn_permlane32_swap(pk[2 * pq][k], pk[2 * pq + 1][k], false, false);
          v[k] = sw[0];
          v[2 + k] = sw[1];
        }
        const int64_t d = d0 + 32 * i + 16 * pq;
        const uint32_t off = d < D ? rowoff[jj] + (uint32_t)(d * (int64_t)sizeof(T)) : 0x80000000u;
        __builtin_amdgcn_raw_buffer_store_b128(v, rs, off, 0, 0);
      }
    }
  }
}

template <typename T, bool SPLIT>
struct SumGeoNarrow {
  static constexpr int NT = 256;
  static constexpr int ES = sizeof(T);
  static_assert(!SPLIT || ES == 2, "the hi / lo pair is a 16-bit layout");
  static constexpr int DN = 256;
  static constexpr int KS = SPLIT ? 32 : 128 / ES;  // contraction elements per slice
  static constexpr int SPT = kBwdVocab / KS;       // slices per 128-deep tile
  static constexpr int XP = DN * ES;               // bytes of one X row in LDS
  static constexpr int X_BYTES = KS * XP;          // 16 KiB (hi / lo), 32 KiB (otherwise)
  static constexpr int GTP = (SPLIT ? 2 : 1) * kBwdVocab * ES;  // bytes of one G row
  static constexpr int G_BYTES = 16384;            // 128 x 128 B (dE) = KS x GTP (dC)
  static constexpr int STAGE = X_BYTES + G_BYTES;  // 32 KiB (hi / lo), 48 KiB (otherwise)
  static constexpr int STAGES = SPLIT ? 4 : 3;
  static constexpr int XLW = X_BYTES / 1024 / 4;   // X loads per wave per stage (4 / 8)
  static constexpr int GLW = G_BYTES / 1024 / 4;   // G loads per wave per stage (4)
  static constexpr int LPW = XLW + GLW;
  static constexpr int KE = 32 / ES;               // contraction elements per MFMA step
  static constexpr int NSTORE = 4 * 2 * (ES == 2 ? 2 : 4);  // output stores per wave per task
  static constexpr int TP_BYTES = ES == 2 ? 32 * 128 : 0;    // per wave: the epilogue's transpose unit
  static_assert(KS * GTP == G_BYTES && 128 * 128 == G_BYTES, "stage geometry");
  static_assert(STAGES * STAGE + 4 * TP_BYTES <= 163840, "the stages and transpose units fit the 160 KiB of LDS");
  static_assert((STAGES - 2) * LPW + NSTORE < 64, "in-flight operations must fit vmcnt");
};

// 64-byte segment swizzle of a row of P bytes read by transposing fragment loads.
// One ds_read_b64_tr_b16 touches rows k0..k0+3 and k0+8..k0+11 (k0 % 4 == 0) in
// one 64-byte segment: with 8+ segments per row those 8 rows land in 8 distinct
// segments, with 4 the two groups of 4 share each segment exactly twice.
template <int P>
__device__ __forceinline__ uint32_t tr_off(uint32_t row, uint32_t byte) {
  constexpr int NSEG = P / 64;
  const uint32_t sw = NSEG >= 8 ? ((row & 3u) | (((row >> 3) & 1u) << 2)) : (row & 3u);
  return row * P + ((((byte >> 6) ^ sw) << 6) | (byte & 63u));
}

typedef short s16x4 __attribute__((ext_vector_type(4)));

// Transposing fragment reads of a [k][col] tile with rows of P bytes (16-bit types).
// The MFMA fragment of column col0 + lane%32 holds the contraction elements
// k0 + 8 (lane/32) + 0..7: two ds_read_b64_tr_b16, where source lane s of each
// 16-lane group g addresses row k0 + 8 (g/2) + 4 t + s/4 and columns
// col0 + 16 (g%2) + 4 (s%4) .. +3.  For k0 a multiple of 16 the row's swizzle term
// does not depend on k0 or t, so the address is a per-lane constant (tr_lane_off)
// plus (k0 + 4 t) P.
template <int P>
__device__ __forceinline__ uint32_t tr_lane_off(int col0) {
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, s = lane & 15;
  const uint32_t row0 = (uint32_t)(8 * (g >> 1) + (s >> 2));
  const uint32_t byte = (uint32_t)(col0 * 2 + 32 * (g & 1) + 8 * (s & 3));
  return tr_off<P>(row0, byte);
}

__device__ __forceinline__ u32x4 frag_tr16(const char* p, uint32_t step_bytes) {
  u32x4 out;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4*)(p + t * step_bytes));
    const u32x2 w = __builtin_bit_cast(u32x2, v);
    out[2 * t] = w.x;
    out[2 * t + 1] = w.y;
  }
  return out;
}

// fp32: the fragment of column col0 + lane%32 holds k0 + 4 (lane/32) + 0..3, four
// 32-bit reads.
template <int P>
__device__ __forceinline__ u32x4 frag_tr32(const char* region, int k0, int col0) {
  const int lane = threadIdx.x & 63;
  const uint32_t byte = (uint32_t)(col0 + (lane & 31)) * 4u;
  const uint32_t row = (uint32_t)(k0 + 4 * (lane >> 5));
  u32x4 out;
#pragma unroll
  for (int q = 0; q < 4; ++q) out[q] = *reinterpret_cast<const uint32_t*>(region + tr_off<P>(row + q, byte));
  return out;
}

// As dma16, with a wave-uniform 64-bit base and a per-lane 32-bit offset (saddr form).
// The base is passed through readfirstlane so it is held in scalar registers.
__device__ __forceinline__ void dma16_s(const char* sbase, uint32_t voff, uint32_t lds) {
  const uint64_t v = reinterpret_cast<uint64_t>(sbase);
  const uint64_t u = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)v) |
                     ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32)) << 32);
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(u),
               "s"(__builtin_amdgcn_readfirstlane(lds))
               : "memory", "m0");
}

// Software pipeline of the sums for 16-bit types (the G hi / lo geometry): stage st
// holds two 16-deep contraction steps, and the loop runs them half a stage apart:
//   read step 1 of st | MFMAs of step 0 of st
//   barrier: stage st + 1 has landed and every wave is done reading st
//   DMA of the stage STAGES - 1 ahead into st
//   read step 0 of st + 1 | MFMAs of step 1 of st      (task end: epilogue)
// so the matrix pipe has queued work across every barrier.  The fragments of one step
// are in registers before the barrier that precedes their MFMAs.  The epilogue's
// stores are the newest vector memory operations at the next STAGES - 1 barriers,
// which then wait with vmcnt(NSTORE) on top of the STAGES - 2 stages left in flight.
// NK steps per stage (even), MF MFMAs and RS LDS reads per step; XF, GF: the fragment
// arrays of one step (the hi / lo pair: a 16-deep step with X per column block and G
// hi / lo per row block, 2 per 32-deep stage; a single G: a 16-deep step with X per
// column block and G per row block, 4 per 64-deep stage), read into one set while the
// MFMAs consume the other.
template <int STAGES, int LPW, int NSTORE, int SPT, int RS, int NK = 2, int MF = 16, typename XF = u32x4[4],
          typename GF = u32x4[2][2], typename Cur, typename IssueNext, typename AdvanceNext, typename FragStep,
          typename MmaStep, typename Epilogue, typename Seek>
__device__ __forceinline__ void sum_split_pipeline(Cur& cs, f32x16 (&acc)[4][2], int mode, IssueNext& issue_next,
                                                   AdvanceNext& advance_next, FragStep& frag_step,
                                                   MmaStep& mma_step, Epilogue& epilogue, Seek& seek) {
  static_assert(STAGES >= 3 && (STAGES - 2) * LPW + NSTORE < 64, "in-flight operations must fit vmcnt");
  static_assert(NK >= 2 && NK % 2 == 0, "the last step of a stage reads into the second fragment set");
#pragma unroll
  for (int p = 0; p < STAGES - 1; ++p) {
    issue_next(p);
    advance_next();
  }
  stage_barrier<(STAGES - 2) * LPW>();  // stage 0 has landed
  issue_next(STAGES - 1);
  advance_next();
  XF xa, xb;
  GF ga, gb;
  frag_step(0, 0, xa, ga);
  int st = 0;
  int since_store = STAGES;  // barriers since the last epilogue that left stores in flight
  for (;;) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) acc[i][jj] = zero16();
    for (;;) {
#pragma unroll
      for (int k = 1; k < NK; ++k) {  // steps 1 .. NK - 1 of stage st: read step k, MFMAs of step k - 1
        if (k & 1) {
          frag_step(st, k, xb, gb);
          mma_step(xa, ga);
        } else {
          frag_step(st, k, xa, ga);
          mma_step(xb, gb);
        }
        sched_interleave<0, MF, RS, 0, 0>();
        __builtin_amdgcn_sched_barrier(0);
      }
      if (++since_store < STAGES)
        stage_barrier<(STAGES - 2) * LPW + NSTORE>();
      else
        stage_barrier<(STAGES - 2) * LPW>();
      issue_next(st);
      advance_next();
      __builtin_amdgcn_sched_barrier(0);
      st = st + 1 == STAGES ? 0 : st + 1;
      frag_step(st, 0, xa, ga);
      mma_step(xb, gb);
      sched_interleave<0, MF, RS, 0, 0>();
      if (++cs.h < SPT) continue;
      cs.h = 0;
      if (++cs.j == cs.cnt) break;
    }
    epilogue(cs);
    if (mode == kWriteT) since_store = 0;
    if (!seek(cs.q + 1, cs)) break;
  }
  wait_vmcnt<0>();
}

// Output of a finished dE / dC task: kWriteT stores the output dtype (one pass over
// everything, and always for dC); the fp32 modes carry dE between passes (WriteMode).

// Persistent owner-computes sums.  PHASE 0 (dE): owner = token block rb, tiles =
// its slots rb_start[rb] .. rb_start[rb + 1]; A-side rows = C rows of each slot's
// vocab tile.  PHASE 1 (dC): owner = vocab tile v of the chunk, tiles = vt_slot
// entries; A-side rows = E rows of each slot's token block.
//
// Tasks are the (owner, D slice) pairs of the owners that hold kept tiles, listed
// largest owner first (own_rb / own_vt) with an owner's D slices consecutive, and
// dealt out in rounds of one task per workgroup, the workgroups numbered XCD-major
// and the direction reversed every round ("snake" order): every workgroup then gets
// a large and a small task in turn, so their totals stay close, and the tasks of
// one round that sit next to each other in the list -- the D slices of one owner,
// which share its G tiles -- run at the same time on one XCD.  A workgroup walks the (task, tile, slice) steps
// of its tasks as one pipeline: the next slice is in flight while one is consumed,
// across task boundaries.  The epilogue's stores are buffer stores (out-of-range
// lanes are dropped by the buffer's range check).  Every per-step address is a
// wave-uniform base plus a per-lane constant computed once: DMA sources in the
// saddr form, fragment reads as constant LDS offsets.
template <typename T, int PHASE, bool SPLIT>
__global__ __launch_bounds__((SumGeo<T, SPLIT>::NT), 1) void bwd_sum_kernel(BwdArgs a, int chunk, int pass) {
  using S = SumGeo<T, SPLIT>;
  __shared__ __attribute__((aligned(16))) char smem[S::STAGES * S::STAGE];
  constexpr int ES = S::ES;
  const int nrb = (int)a.plan.nrb, nds = (int)((a.D + S::DN - 1) / S::DN);
  const int vlo = chunk * (int)a.plan.chunk_nvt;
  const int xcd = (int)(blockIdx.x & 7), lidx = (int)(blockIdx.x >> 3), nper = (int)(gridDim.x >> 3);
  const int* pi = a.pinfo + pass * kPassInts;
  const int pmode = ldu(pi, kPiDeMode);
  if (pmode < 0) return;  // past the passes the data needs
  // the filtered backward launches both dC geometries; the compaction picked one per pass
  if (PHASE == 1 && a.dc_geo == 0 && a.filter_log_eps > -INFINITY && ldu(pi, kPiDcWide) != 1) return;
  const int s0 = ldu(pi, kPiS0);  // the G scratch holds slot s at s - s0
  const int ntasks = ldu(pi, PHASE == 0 ? kPiOwnRb : kPiOwnVt) * nds;
  const int* own = PHASE == 0 ? a.own_rb + pass * nrb : a.own_vt + ldu(pi, kPiVt0);
  const int* ostart = PHASE == 0 ? a.rb_start + pass * nrb : a.vt_start;  // an owner's slots / vt_slot entries
  const int vwg = xcd * nper + lidx, nwg = (int)gridDim.x;  // workgroups numbered XCD-major
  const int64_t D = a.D;
  const int64_t pitch = D * ES;
  const RowData rd = row_data(a);
  const char* X = PHASE == 0 ? reinterpret_cast<const char*>(a.c) : rd.e;
  const int64_t xrows = PHASE == 0 ? a.V : a.N;
  const int mode = PHASE == 0 ? pmode : kWriteT;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 31, h = lane >> 5, kg = lane >> 5;
  const int wm = wave & 1;   // output rows [64 wm, 64 wm + 64)
  const int wd = wave >> 1;  // output columns [128 wd, 128 wd + 128) of the slice (4 quarters)

  // This wave's DMA loads: XLW into the X region, GLW into the G region.  Per lane:
  // the region row it fills and the byte of the source row that belongs there.
  uint32_t xrow[S::XLW], xcol[S::XLW], xoff[S::XLW], goff[S::GLW];
#pragma unroll
  for (int j = 0; j < S::XLW; ++j) {
    const uint32_t o = (uint32_t)(wave * S::XLW + j) * 1024u + lane * 16u;
    const uint32_t row = o / S::XP, pb = o % S::XP;
    xrow[j] = row;
    xcol[j] = tr_off<S::XP>(row, pb) - row * S::XP;  // the swizzle is an involution on the segment index
    xoff[j] = (uint32_t)(row * pitch) + xcol[j];
  }
#pragma unroll
  for (int j = 0; j < S::GLW; ++j) {
    const uint32_t o = (uint32_t)(wave * S::GLW + j) * 1024u + lane * 16u;
    if (PHASE == 0) {
      const uint32_t row = o / 128u, ch = (o % 128u) / 16u;
      goff[j] = row * S::GTP + (ch ^ ((row ^ (row >> 3)) & 7u)) * 16u;
    } else {
      const uint32_t row = o / S::GTP, pb = o % S::GTP;
      goff[j] = tr_off<S::GTP>(row, pb);
    }
  }
  // Fragment read offsets within a stage (16-bit types): go_t[hl][jj] the dC
  // fragments (hl: the hi / lo halves of the pair; 0 only for a single G), go_n[jj][ks]
  // the dE row chunks 2 ks + kg.
  uint32_t xo[4], go_t[2][2], go_n[2][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) xo[i] = tr_lane_off<S::XP>(wd * 128 + 32 * i);
#pragma unroll
  for (int jj = 0; jj < 2; ++jj) {
#pragma unroll
    for (int hl = 0; hl < 2; ++hl)
      go_t[hl][jj] = S::X_BYTES + tr_lane_off<S::GTP>(SPLIT ? 2 * (wm * 64 + 32 * jj) + 32 * hl : wm * 64 + 32 * jj);
    const uint32_t row = (uint32_t)(wm * 64 + 32 * jj + n);
    const uint32_t c = (row ^ (row >> 3)) & 7u;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) go_n[jj][ks] = S::X_BYTES + row * 128u + ((((uint32_t)(2 * ks + kg)) ^ c) << 4);
  }

  // slot / xrow: the G slot and first X row of tile j, resolved by prep() from the
  // scalar lists; the loads are issued at the end of a step and land at the next
  // step's barrier, so no fragment read waits behind them.
  struct Cur {
    int q, owner, ds, b, cnt, j, h, slot;
    int64_t xrow;
  };
  auto seek = [&](int q, Cur& c) -> bool {
    const int p = q * nwg + ((q & 1) ? nwg - 1 - vwg : vwg);
    if (p >= ntasks) return false;
    const int owner = ldu(own, p / nds);
    const int b = ldu(ostart, owner);
    c.q = q;
    c.owner = owner;
    c.ds = p - (p / nds) * nds;
    c.b = b;
    c.cnt = ldu(ostart, owner + 1) - b;
    c.j = 0;
    c.h = 0;
    return true;
  };
  auto prep = [&](Cur& c) {
    if (PHASE == 0) {
      c.slot = c.b + c.j;
      c.xrow = (int64_t)(vlo + ldu(a.slot_vt, c.slot)) * kBwdVocab;
    } else {
      c.slot = ldu(a.vt_slot, c.b + c.j);
      c.xrow = (int64_t)ldu(a.slot_rb, c.slot) * kBwdTokens;
    }
  };
  auto advance = [&](Cur& c) -> bool {
    if (++c.h < S::SPT) return true;
    c.h = 0;
    if (++c.j < c.cnt) {
      prep(c);
      return true;
    }
    if (!seek(c.q + 1, c)) return false;
    prep(c);
    return true;
  };

  // LDS-DMA of tile c's slice into stage st.  The loads are inline assembly: the
  // compiler then adds no vmcnt wait for them in front of the fragment reads of
  // other stages (the stage barriers order them).
  const uint32_t smem_lds = lds_addr(smem);
  auto issue = [&](const Cur& c, int st) {
    const uint32_t sb = smem_lds + (uint32_t)(st * S::STAGE);
    const int64_t xr0 = c.xrow + c.h * S::KS;
    const int64_t dcol = (int64_t)c.ds * S::DN * ES;
    const char* xbase = X + xr0 * pitch + dcol;
    if (xr0 + S::KS <= xrows && dcol + S::DN * ES <= pitch) {
#pragma unroll
      for (int j = 0; j < S::XLW; ++j) dma16_s(xbase, xoff[j], sb + (wave * S::XLW + j) * 1024);
    } else {  // last row block or ragged D slice: zeros past the last row and the row end
#pragma unroll
      for (int j = 0; j < S::XLW; ++j) {
        const int64_t r = xr0 + xrow[j];
        const int64_t cb = dcol + xcol[j];
        const char* src = (r < xrows && cb < pitch) ? X + r * pitch + cb : reinterpret_cast<const char*>(g_zero16);
        dma16(src, sb + (wave * S::XLW + j) * 1024);
      }
    }
    const char* gbase =
        a.gtile + (size_t)(c.slot - s0) * a.plan.g_bytes + (PHASE == 0 ? c.h * 128 : c.h * S::KS * S::GTP);
#pragma unroll
    for (int j = 0; j < S::GLW; ++j) dma16_s(gbase, goff[j], sb + S::X_BYTES + (wave * S::GLW + j) * 1024);
  };

  f32x16 acc[4][2];
  // Fragments of one 32-byte contraction step ks of stage st, and its 8 MFMAs.
  auto frags = [&](int st, int ks, u32x4 (&xf)[4], u32x4 (&gf)[2]) {
    const char* sp = smem + st * S::STAGE;
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      if constexpr (PHASE == 0)
        gf[jj] = lds_ld16(sp, go_n[jj][ks]);
      else if constexpr (ES == 2)
        gf[jj] = frag_tr16(sp + go_t[0][jj] + 16 * ks * S::GTP, 4 * S::GTP);
      else
        gf[jj] = frag_tr32<S::GTP>(sp + S::X_BYTES, ks * S::KE, wm * 64 + 32 * jj);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (ES == 2)
        xf[i] = frag_tr16(sp + xo[i] + 16 * ks * S::XP, 4 * S::XP);
      else
        xf[i] = frag_tr32<S::XP>(sp, ks * S::KE, wd * 128 + 32 * i);
    }
  };
  auto mma = [&](const u32x4 (&xf)[4], const u32x4 (&gf)[2]) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) acc[i][jj] = Traits<T>::mfma(xf[i], gf[jj], acc[i][jj]);
  };
  // The hi / lo pair: the fragments of one 16-deep contraction step kp of a stage (an
  // X fragment per column block, a G hi and lo fragment per row block) and its 16
  // MFMAs, hi ones first: the 8 accumulators then separate each dependent pair.
  auto frag_step = [&](int st, int kp, u32x4 (&x)[4], u32x4 (&g)[2][2]) {
    const char* sp = smem + st * S::STAGE;
#pragma unroll
    for (int hl = 0; hl < 2; ++hl)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        if constexpr (PHASE == 0)
          g[hl][jj] = lds_ld16(sp, go_n[jj][2 * hl + kp]);
        else
          g[hl][jj] = frag_tr16(sp + go_t[hl][jj] + 16 * kp * S::GTP, 4 * S::GTP);
      }
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = frag_tr16(sp + xo[i] + 16 * kp * S::XP, 4 * S::XP);
  };
  auto mma_step = [&](const u32x4 (&x)[4], const u32x4 (&g)[2][2]) {
#pragma unroll
    for (int hl = 0; hl < 2; ++hl)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) acc[i][jj] = Traits<T>::mfma(x[i], g[hl][jj], acc[i][jj]);
  };
  // RK = LDS read instructions per contraction step, MK = MFMAs per contraction step.
  constexpr int RK = (ES == 2 ? 8 : 16) + (PHASE == 0 ? 2 : (ES == 2 ? 4 : 8));
  constexpr int MK = 8 * Traits<T>::kInstrPerStep;
  // fp16 G tiles hold G 2^gexp: the epilogue scales the sums back (exact)
  const float gdiv = __builtin_ldexpf(1.f, -(ES == 2 ? g_scale_exp(a) : 0));

  // acc[i][jj][r]: output column ds DN + 128 wd + 32 i + 8 (r/4) + 4 h + r%4 of row 64 wm + 32 jj + n.
  auto epilogue = [&](const Cur& c) {
    if (ES == 2 && gdiv != 1.f) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) acc[i][jj] *= gdiv;
    }
    const int64_t orow0 = (int64_t)(PHASE == 0 ? c.owner : vlo + c.owner) * 128;
    const int64_t orows = PHASE == 0 ? a.N : a.V;
    const int64_t nrows = orows - orow0 < 128 ? orows - orow0 : 128;
    // dE rows of the sorted order go to dE row map[row] (the whole of dE is then one
    // buffer, under 2^31 bytes when the sorted order is available); rows past the
    // owner's end get an out-of-range offset, so every lane issues every store.
    const int* map = PHASE == 0 ? rd.map : nullptr;
    T* out = reinterpret_cast<T*>(PHASE == 0 ? a.dE : a.dC) + (map ? 0 : orow0 * D);
    uint32_t rowoff[2];
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int64_t m = wm * 64 + 32 * jj + n;
      rowoff[jj] = m >= nrows ? 0x80000000u : (uint32_t)((map ? (int64_t)map[orow0 + m] : m) * D * ES);
    }
    const int64_t d00 = (int64_t)c.ds * S::DN + wd * 128 + h * 4;
    if (mode == kWriteT) {
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
          out, (short)0, (int)((map ? a.N : nrows) * D * ES), 0x00020000);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          const int64_t m = wm * 64 + 32 * jj + n;
          if constexpr (ES == 4) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int64_t d = d00 + 32 * i + 8 * q;
              const uint32_t off = d < D ? rowoff[jj] + (uint32_t)(d * ES) : 0x80000000u;
              const u32x4 v{__float_as_uint(acc[i][jj][4 * q]), __float_as_uint(acc[i][jj][4 * q + 1]),
                            __float_as_uint(acc[i][jj][4 * q + 2]), __float_as_uint(acc[i][jj][4 * q + 3])};
              __builtin_amdgcn_raw_buffer_store_b128(v, rs, off, 0, 0);
            }
          } else {
            // Lane (n, h) holds columns 8 q + 4 h + 0..3 of its row; one lane swap
            // between the halves per q pair gives every lane 8 consecutive columns:
            // 16 p + 8 h + 0..7 for the pair (2 p, 2 p + 1), stored as 16 bytes.
            uint32_t pk[4][2];
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
              for (int k = 0; k < 2; ++k) pk[q][k] = pack2<T>(acc[i][jj][4 * q + 2 * k], acc[i][jj][4 * q + 2 * k + 1]);
#pragma unroll
            for (int pq = 0; pq < 2; ++pq) {
              u32x4 v;
#pragma unroll
              for (int k = 0; k < 2; ++k) {
                const auto sw = __builtin_amdgcn_permlane32_swap(pk[2 * pq][k], pk[2 * pq + 1][k], false, false);
                v[k] = sw[0];
                v[2 + k] = sw[1];
              }
              const int64_t d = d00 - h * 4 + 32 * i + 16 * pq + 8 * h;
              const uint32_t off = d < D ? rowoff[jj] + (uint32_t)(d * ES) : 0x80000000u;
              __builtin_amdgcn_raw_buffer_store_b128(v, rs, off, 0, 0);
            }
          }
        }
      }
    } else {
      float* carry = a.de_acc + orow0 * D;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          const int64_t m = wm * 64 + 32 * jj + n;
          if (m >= nrows) continue;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int64_t d = d00 + 32 * i + 8 * q;
            if (d >= D) continue;
            f32x4 v{acc[i][jj][4 * q], acc[i][jj][4 * q + 1], acc[i][jj][4 * q + 2], acc[i][jj][4 * q + 3]};
            f32x4* cp = reinterpret_cast<f32x4*>(carry + m * D + d);
            if (mode == kStoreF32) {
              *cp = v;
            } else if (mode == kAddF32) {
              *cp = *cp + v;
            } else {
              v = *cp + v;
              T* orow = out + (map ? (int64_t)map[orow0 + m] : m) * D;
#pragma unroll
              for (int k = 0; k < 4; ++k) orow[d + k] = (T)v[k];
            }
          }
        }
      }
      wait_vmcnt<0>();  // the fp32 modes leave nothing in flight for the stage waits
    }
  };

  Cur cs;
  if (!seek(0, cs)) return;
  prep(cs);
  Cur nx = cs, last = cs;
  bool have = true;
  // issue_next: the loads of nx (or, past the end, a repeat of the last one, which
  // keeps the per-stage load count uniform and is never consumed); advance_next:
  // step nx on, issuing the scalar list loads of its next tile.
  auto issue_next = [&](int st) { issue(have ? nx : last, st); };
  auto advance_next = [&]() {
    if (have) {
      last = nx;
      have = advance(nx);
    }
  };
  // Software pipeline over the (task, tile, slice) steps, two stages: step s reads
  // stage s % 2 while slice s + 1 streams into the other one.
  //   read ks 1 | MFMAs ks 0;  read ks 2 | MFMAs ks 1;  read ks 3 | MFMAs ks 2
  //   barrier: slice s + 1 has landed and every wave is done with stage s % 2
  //   DMA of slice s + 2 into stage s % 2 | read ks 0 of slice s + 1 | MFMAs ks 3
  //   (task end: epilogue)
  // The epilogue's stores are the newest vector memory operations at the next
  // barrier, so it waits with vmcnt(NSTORE) and lets them drain in the background.
  constexpr int NSTORE = S::NSTORE;  // buffer stores per wave per kWriteT epilogue
  if constexpr (SPLIT) {
    // LDS reads of one 16-deep step: 8 for X, 4 (dE) or 8 (dC, transposing) for G
    sum_split_pipeline<S::STAGES, S::LPW, NSTORE, S::SPT, 8 + (PHASE == 0 ? 4 : 8)>(
        cs, acc, mode, issue_next, advance_next, frag_step, mma_step, epilogue, seek);
    return;
  }
  issue_next(0);
  advance_next();
  stage_barrier<0>();
  issue_next(1);
  advance_next();
  u32x4 xa[4], ga[2], xb[4], gb[2];
  frags(0, 0, xa, ga);
  int st = 0;
  bool stores = false;  // the last epilogue's stores may still be in flight
  for (;;) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) acc[i][jj] = zero16();
    for (;;) {
      frags(st, 1, xb, gb);
      mma(xa, ga);
      sched_interleave<0, MK, RK, 0, 0>();
      frags(st, 2, xa, ga);
      mma(xb, gb);
      sched_interleave<0, MK, RK, 0, 0>();
      frags(st, 3, xb, gb);
      mma(xa, ga);
      sched_interleave<0, MK, RK, 0, 0>();
      __builtin_amdgcn_sched_barrier(0);
      if (stores)
        stage_barrier<NSTORE>();
      else
        stage_barrier<0>();
      stores = false;
      issue_next(st);
      advance_next();
      __builtin_amdgcn_sched_barrier(0);
      st ^= 1;
      frags(st, 0, xa, ga);
      mma(xb, gb);
      sched_interleave<0, MK, RK, 0, 0>();
      if (++cs.h < S::SPT) continue;
      cs.h = 0;
      if (++cs.j == cs.cnt) break;
    }
    epilogue(cs);
    stores = mode == kWriteT;
    if (!seek(cs.q + 1, cs)) break;
  }
  wait_vmcnt<0>();
}

// Which dE tasks of a pass are cut into pieces, for a grid of nwg workgroups: npc
// pieces each of the ncut tasks [tbase, tbase + ncut), or none (npc 1).  With few
// tasks (2 ntasks <= cap) all of them, npc = cap / ntasks; with tasks overflowing the
// grid by at most half of it (2 (ntasks - nwg) <= cap) the ones past the grid, npc =
// cap / (ntasks - nwg), after a first launch of one whole task per workgroup.  cap =
// min(nwg, kDePartSlots): piece q of cut task tbase + t has slot t npc + q.
__device__ __forceinline__ void de_pieces_of(const BwdArgs& a, int ntasks, int nwg, int& tbase, int& ncut, int& npc) {
  tbase = 0;
  ncut = 0;
  npc = 1;
  if (a.de_part == nullptr || ntasks <= 0) return;
  const int cap = nwg < kDePartSlots ? nwg : kDePartSlots;
  if (2 * ntasks <= cap) {
    ncut = ntasks;
    npc = cap / ntasks;
  } else if (ntasks > nwg && 2 * (ntasks - nwg) <= cap) {
    tbase = nwg;
    ncut = ntasks - nwg;
    npc = cap / ncut;
  }
}

// As bwd_sum_kernel, in the narrow geometry (one 4-wave pipeline of 48 KiB stages).
template <typename T, int PHASE, bool SPLIT>
__global__ __launch_bounds__(kThreads, 1) void bwd_sum_narrow_kernel(BwdArgs a, int chunk, int pass) {
  using S = SumGeoNarrow<T, SPLIT>;
  __shared__ __attribute__((aligned(16))) char smem[S::STAGES * S::STAGE + 4 * S::TP_BYTES];
  constexpr int ES = S::ES;
  const int nrb = (int)a.plan.nrb, nds = (int)((a.D + S::DN - 1) / S::DN);
  const int vlo = chunk * (int)a.plan.chunk_nvt;
  const int xcd = (int)(blockIdx.x & 7), lidx = (int)(blockIdx.x >> 3), nper = (int)(gridDim.x >> 3);
  const int* pi = a.pinfo + pass * kPassInts;
  const int pmode = ldu(pi, kPiDeMode);
  if (pmode < 0) return;  // past the passes the data needs
  // the filtered backward launches both dC geometries; the compaction picked one per pass
  if (PHASE == 1 && a.dc_geo == 0 && a.filter_log_eps > -INFINITY && ldu(pi, kPiDcWide) != 0) return;
  const int s0 = ldu(pi, kPiS0);  // the G scratch holds slot s at s - s0
  const int ntasks = ldu(pi, PHASE == 0 ? kPiOwnRb : kPiOwnVt) * nds;
  // dE pieces (de_pieces_of): npc pieces per task of [tbase, tbase + ncut) (items ncut *
  // npc <= kDePartSlots), or whole tasks (npc 1)
  int tbase = 0, ncut = 0, npc = 1;
  if (PHASE == 0) de_pieces_of(a, ntasks, (int)gridDim.x, tbase, ncut, npc);
  if (PHASE == 0 && a.de_stage == 1 && (npc == 1 || tbase == 0)) return;  // no overflow to cut
  const int nitems = PHASE == 0 && a.de_stage == 1 ? ncut * npc
                     : PHASE == 0 && npc > 1 && tbase == 0 ? ntasks * npc
                     : PHASE == 0 && npc > 1 ? tbase : ntasks;
  const bool cut = PHASE == 0 && npc > 1 && (a.de_stage == 1 || tbase == 0);  // this launch sums pieces
  const int* own = PHASE == 0 ? a.own_rb + pass * nrb : a.own_vt + ldu(pi, kPiVt0);
  const int* ostart = PHASE == 0 ? a.rb_start + pass * nrb : a.vt_start;  // an owner's slots / vt_slot entries
  const int vwg = xcd * nper + lidx, nwg = (int)gridDim.x;  // workgroups numbered XCD-major
  // dC: this workgroup's bin of the schedule the G kernel dealt, and its first D slice
  static_assert(PHASE == 0 || S::DN == kDcSliceCols, "the dC schedule assumes this slice width");
  static_assert(S::SPT == dc_steps_per_tile<T>(SPLIT), "the dC schedule counts these steps per kept tile");
  const int dcb = dc_bins(nwg, nds);
  const int dcm = dcb > 0 ? vwg / nds : 0;
  const int ds0 = dcb > 0 ? vwg - dcm * nds : vwg;
  const bool dc_mine = PHASE == 1 && (dcb > 0 ? dcm < dcb : ds0 < nds);
  const int bstart = dc_mine ? ldu(a.dc_bin_start, dcm) : 0;
  const int bcnt = dc_mine ? ldu(a.dc_bin_start, dcm + 1) - bstart : 0;
  const int64_t D = a.D;
  const int64_t pitch = D * ES;
  const RowData rd = row_data(a);
  const char* X = PHASE == 0 ? reinterpret_cast<const char*>(a.c) : rd.e;
  const int64_t xrows = PHASE == 0 ? a.V : a.N;
  const int mode = PHASE == 0 ? (cut ? kPartF32 : pmode) : kWriteT;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 31, h = lane >> 5, kg = lane >> 5;
  const int wm = wave & 1;   // output rows [64 wm, 64 wm + 64)
  const int wd = wave >> 1;  // output columns [128 wd, 128 wd + 128) of the slice

  // This wave's DMA loads: XLW into the X region, GLW into the G region.  Per lane:
  // the region row it fills and the byte of the source row that belongs there.
  // (Recomputed where the ragged loads need them rather than held in registers.)
  auto xslot = [&](int j, uint32_t& row, uint32_t& col) {
    const uint32_t o = (uint32_t)(wave * S::XLW + j) * 1024u + lane * 16u;
    row = o / S::XP;
    col = tr_off<S::XP>(row, o % S::XP) - row * S::XP;  // the swizzle is an involution on the segment index
  };
  uint32_t xoff[S::XLW], goff[S::GLW];
#pragma unroll
  for (int j = 0; j < S::XLW; ++j) {
    uint32_t row, col;
    xslot(j, row, col);
    xoff[j] = (uint32_t)(row * pitch) + col;
  }
#pragma unroll
  for (int j = 0; j < S::GLW; ++j) {
    const uint32_t o = (uint32_t)(wave * S::GLW + j) * 1024u + lane * 16u;
    if (PHASE == 0) {
      const uint32_t row = o / 128u, ch = (o % 128u) / 16u;
      goff[j] = row * S::GTP + (ch ^ ((row ^ (row >> 3)) & 7u)) * 16u;
    } else {
      const uint32_t row = o / S::GTP, pb = o % S::GTP;
      goff[j] = tr_off<S::GTP>(row, pb);
    }
  }
  // Fragment read offsets within a stage (16-bit types): go_t[hl][jj] the dC
  // fragments (hl: the hi / lo halves of the pair; 0 only for a single G), go_n[jj][ks]
  // the dE row chunks 2 ks + kg.
  uint32_t xo[4], go_t[2][2], go_n[2][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) xo[i] = tr_lane_off<S::XP>(wd * 128 + 32 * i);
#pragma unroll
  for (int jj = 0; jj < 2; ++jj) {
#pragma unroll
    for (int hl = 0; hl < 2; ++hl)
      go_t[hl][jj] = S::X_BYTES + tr_lane_off<S::GTP>(SPLIT ? 2 * (wm * 64 + 32 * jj) + 32 * hl : wm * 64 + 32 * jj);
    const uint32_t row = (uint32_t)(wm * 64 + 32 * jj + n);
    const uint32_t c = (row ^ (row >> 3)) & 7u;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) go_n[jj][ks] = S::X_BYTES + row * 128u + ((((uint32_t)(2 * ks + kg)) ^ c) << 4);
  }

  // slot / xrow: the G slot and first X row of tile j, resolved by prep() from the
  // scalar lists; the loads are issued at the end of a step and land at the next
  // step's barrier, so no fragment read waits behind them.
  struct Cur {
    int q, owner, ds, b, cnt, j, h, slot;
    int64_t xrow;
  };
  // dE pieces (cut): items number at most the workgroups, so workgroup vwg has item vwg
  // alone, piece k = vwg % npc of task tbase + vwg / npc: its tiles [j0, j1) of the
  // task's (none when the task has fewer tiles than pieces)
  int pc_j0 = 0, pc_j1 = 0;
  if (cut && vwg < nitems) {
    const int task = tbase + vwg / npc, k = vwg - (vwg / npc) * npc;
    const int ow = ldu(own, task / nds);
    const int cnt = ldu(ostart, ow + 1) - ldu(ostart, ow);
    pc_j0 = k * cnt / npc;
    pc_j1 = (k + 1) * cnt / npc;
  }
  auto seek = [&](int q, Cur& c) -> bool {
    int owner, ds;
    if constexpr (PHASE == 0) {
      const int p = q * nwg + ((q & 1) ? nwg - 1 - vwg : vwg);
      if (p >= nitems || (cut && pc_j0 == pc_j1)) return false;
      const int task = cut ? tbase + p / npc : p;
      owner = ldu(own, task / nds);
      ds = task - (task / nds) * nds;
    } else {  // the q-th owner of this workgroup's bin (then the same again at slice ds0 + nwg, ...)
      if (bcnt == 0) return false;
      const int t = q / bcnt;
      ds = ds0 + t * nwg;
      if (ds >= nds) return false;
      owner = ldu(a.dc_bin_owner, bstart + (q - t * bcnt));
    }
    const int b = ldu(ostart, owner);
    c.q = q;
    c.owner = owner;
    c.ds = ds;
    c.b = b + pc_j0;
    c.cnt = cut ? pc_j1 - pc_j0 : ldu(ostart, owner + 1) - b;
    c.j = 0;
    c.h = 0;
    return true;
  };
  auto prep = [&](Cur& c) {
    if (PHASE == 0) {
      c.slot = c.b + c.j;
      c.xrow = (int64_t)(vlo + ldu(a.slot_vt, c.slot)) * kBwdVocab;
    } else {
      c.slot = ldu(a.vt_slot, c.b + c.j);
      c.xrow = (int64_t)ldu(a.slot_rb, c.slot) * kBwdTokens;
    }
  };
  auto advance = [&](Cur& c) -> bool {
    if (++c.h < S::SPT) return true;
    c.h = 0;
    if (++c.j < c.cnt) {
      prep(c);
      return true;
    }
    if (!seek(c.q + 1, c)) return false;
    prep(c);
    return true;
  };

  // LDS-DMA of tile c's slice into stage st.  The loads are inline assembly: the
  // compiler then adds no vmcnt wait for them in front of the fragment reads of
  // other stages (the stage barriers order them).
  const uint32_t smem_lds = lds_addr(smem);
  // X rows [xr0, xr0 + KS) of D slice ds into the X region at LDS address sb
  auto issue_x = [&](int64_t xr0, int ds, uint32_t sb) {
    const int64_t dcol = (int64_t)ds * S::DN * ES;
    const char* xbase = X + xr0 * pitch + dcol;
    if (xr0 + S::KS <= xrows && dcol + S::DN * ES <= pitch) {
#pragma unroll
      for (int j = 0; j < S::XLW; ++j) dma16_s(xbase, xoff[j], sb + (wave * S::XLW + j) * 1024);
    } else {  // last row block or ragged D slice: zeros past the last row and the row end
#pragma unroll
      for (int j = 0; j < S::XLW; ++j) {
        uint32_t xr, xc;
        xslot(j, xr, xc);
        const int64_t r = xr0 + xr;
        const int64_t cb = dcol + xc;
        const char* src = (r < xrows && cb < pitch) ? X + r * pitch + cb : reinterpret_cast<const char*>(g_zero16);
        dma16(src, sb + (wave * S::XLW + j) * 1024);
      }
    }
  };
  // slice h of slot's G tile into the G region of the stage at LDS address sb
  auto issue_g = [&](int slot, int h, uint32_t sb) {
    const char* gbase =
        a.gtile + (size_t)(slot - s0) * a.plan.g_bytes + (PHASE == 0 ? h * 128 : h * S::KS * S::GTP);
#pragma unroll
    for (int j = 0; j < S::GLW; ++j) dma16_s(gbase, goff[j], sb + S::X_BYTES + (wave * S::GLW + j) * 1024);
  };
  auto issue = [&](const Cur& c, int st) {
    const uint32_t sb = smem_lds + (uint32_t)(st * S::STAGE);
    issue_x(c.xrow + c.h * S::KS, c.ds, sb);
    issue_g(c.slot, c.h, sb);
  };

  f32x16 acc[4][2];
  // A step's fragments for its four 32-byte contraction steps (ks): the reads of
  // ks 0 and 1 go first, those of ks 2 and 3 among the MFMAs of ks 0 and 1.
  u32x4 xf[4][4], gf[4][2];
  auto frags = [&](int st) {
    const char* sp = smem + st * S::STAGE;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        if constexpr (PHASE == 0)
          gf[ks][jj] = lds_ld16(sp, go_n[jj][ks]);
        else if constexpr (ES == 2)
          gf[ks][jj] = frag_tr16(sp + go_t[0][jj] + 16 * ks * S::GTP, 4 * S::GTP);
        else
          gf[ks][jj] = frag_tr32<S::GTP>(sp + S::X_BYTES, ks * S::KE, wm * 64 + 32 * jj);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (ES == 2)
          xf[ks][i] = frag_tr16(sp + xo[i] + 16 * ks * S::XP, 4 * S::XP);
        else
          xf[ks][i] = frag_tr32<S::XP>(sp, ks * S::KE, wd * 128 + 32 * i);
      }
    }
  };
  auto mma = [&]() {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) acc[i][jj] = Traits<T>::mfma(xf[ks][i], gf[ks][jj], acc[i][jj]);
  };
  // RK = LDS read instructions per contraction step, MK = MFMAs per contraction step.
  constexpr int RK = (ES == 2 ? 8 : 16) + (PHASE == 0 ? 2 : (ES == 2 ? 4 : 8));
  constexpr int MK = 8 * Traits<T>::kInstrPerStep;
  auto schedule = [&]() {
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * RK, 0);
    sched_interleave<0, MK, RK, 0, 0>();
    sched_interleave<0, MK, RK, 0, 0>();
    sched_interleave<0, MK, 0, 0, 0>();
    sched_interleave<0, MK, 0, 0, 0>();
  };
  // The hi / lo pair: the fragments of one 16-deep contraction step kp of a stage (an
  // X fragment per column block, a G hi and lo fragment per row block) and its 16
  // MFMAs, hi ones first: the 8 accumulators then separate each dependent pair.
  auto frag_step = [&](int st, int kp, u32x4 (&x)[4], u32x4 (&g)[2][2]) {
    const char* sp = smem + st * S::STAGE;
#pragma unroll
    for (int hl = 0; hl < 2; ++hl)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        if constexpr (PHASE == 0)
          g[hl][jj] = lds_ld16(sp, go_n[jj][2 * hl + kp]);
        else
          g[hl][jj] = frag_tr16(sp + go_t[hl][jj] + 16 * kp * S::GTP, 4 * S::GTP);
      }
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = frag_tr16(sp + xo[i] + 16 * kp * S::XP, 4 * S::XP);
  };
  auto mma_step = [&](const u32x4 (&x)[4], const u32x4 (&g)[2][2]) {
#pragma unroll
    for (int hl = 0; hl < 2; ++hl)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) acc[i][jj] = Traits<T>::mfma(x[i], g[hl][jj], acc[i][jj]);
  };
  // fp16 G tiles hold G 2^gexp: the epilogue scales the sums back (exact)
  const float gdiv = __builtin_ldexpf(1.f, -(ES == 2 ? g_scale_exp(a) : 0));

  // acc[i][jj][r]: output column ds DN + 128 wd + 32 i + 8 (r/4) + 4 h + r%4 of row 64 wm + 32 jj + n.
  auto epilogue = [&](const Cur& c) {
    if (ES == 2 && gdiv != 1.f) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) acc[i][jj] *= gdiv;
    }

    const int64_t orow0 = (int64_t)(PHASE == 0 ? c.owner : vlo + c.owner) * 128;
    const int64_t orows = PHASE == 0 ? a.N : a.V;
    const int64_t nrows = orows - orow0 < 128 ? orows - orow0 : 128;
    // dE rows of the sorted order go to dE row map[row] (the whole of dE is then one
    // buffer, under 2^31 bytes when the sorted order is available); rows past the
    // owner's end get an out-of-range offset, so every lane issues every store.
    const int* map = PHASE == 0 ? rd.map : nullptr;
    T* out = reinterpret_cast<T*>(PHASE == 0 ? a.dE : a.dC) + (map ? 0 : orow0 * D);
    // the dE sums (a few tasks per workgroup) store straight from the accumulators: the
    // transpose's registers would spill there
    constexpr bool kDirect16 = PHASE == 0;
    uint32_t rowoff[2];
    if (ES == 4 || kDirect16 || mode != kWriteT) {
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const int64_t m = wm * 64 + 32 * jj + n;
        rowoff[jj] = m >= nrows ? 0x80000000u : (uint32_t)((map ? (int64_t)map[orow0 + m] : m) * D * ES);
      }
    }
    const int64_t d00 = (int64_t)c.ds * S::DN + wd * 128 + h * 4;
    if (mode == kWriteT) {
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
          out, (short)0, (int)((map ? a.N : nrows) * D * ES), 0x00020000);
      if constexpr (ES == 4) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
          for (int jj = 0; jj < 2; ++jj) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int64_t d = d00 + 32 * i + 8 * q;
              const uint32_t off = d < D ? rowoff[jj] + (uint32_t)(d * ES) : 0x80000000u;
              const u32x4 v{__float_as_uint(acc[i][jj][4 * q]), __float_as_uint(acc[i][jj][4 * q + 1]),
                            __float_as_uint(acc[i][jj][4 * q + 2]), __float_as_uint(acc[i][jj][4 * q + 3])};
              __builtin_amdgcn_raw_buffer_store_b128(v, rs, off, 0, 0);
            }
          }
        }
      } else if constexpr (kDirect16) {
        store_direct16<T>(acc, rs, rowoff, d00 - h * 4 + 8 * h, D);
      } else {
        // 16-bit output through the wave's 4 KiB of LDS past the stages, one 32-row x
        // 64-column unit (jj, ip) at a time: lane (n, h) holds 16 bytes (8 columns) of
        // row n per (i, pq); they go in as rows of 128 bytes (16-byte chunk
        // 4 il + 2 pq + h, swizzled by bits 1..3 of the row) and come out as 8 rows x
        // 128 bytes per read, so every store covers 8 whole 128-byte row pieces
        // instead of 32 pieces of 32 bytes (a quarter of the L2 write requests).  The
        // region is this wave's alone and no DMA writes it: no barrier is needed.
        char* const tp = smem + S::STAGES * S::STAGE + wave * S::TP_BYTES;
        const int rl = lane >> 3, cl = lane & 7;
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
#pragma unroll
          for (int ip = 0; ip < 2; ++ip) {
#pragma unroll
            for (int il = 0; il < 2; ++il) {
              const int i = 2 * ip + il;
              // lane (n, h) holds columns 8 q + 4 h + 0..3 of its row; one lane swap
              // between the halves per q pair gives it columns 16 pq + 8 h + 0..7
              uint32_t pk[4][2];
#pragma unroll
              for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int k = 0; k < 2; ++k) pk[q][k] = pack2<T>(acc[i][jj][4 * q + 2 * k], acc[i][jj][4 * q + 2 * k + 1]);
#pragma unroll
              for (int pq = 0; pq < 2; ++pq) {
                u32x4 v;
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                  const auto sw = __builtin_amdgcn_permlane32_swap(pk[2 * pq][k], pk[2 * pq + 1][k], false, false);
                  v[k] = sw[0];
                  v[2 + k] = sw[1];
                }
                const int ck = 4 * il + 2 * pq + h;
                *reinterpret_cast<u32x4*>(tp + n * 128 + ((ck ^ ((n >> 1) & 7)) << 4)) = v;
              }
            }
            // the buffer spans under 2^31 bytes: 32-bit offsets
            const int d = c.ds * S::DN + wd * 128 + 64 * ip + 8 * cl;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              const int r = 8 * t + rl;
              const u32x4 w = *reinterpret_cast<const u32x4*>(tp + r * 128 + ((cl ^ ((r >> 1) & 7)) << 4));
              const int m = wm * 64 + 32 * jj + r;  // row of the owner (past its end: a dropped offset)
              const uint32_t off = m < nrows && d < D
                                       ? (uint32_t)(map ? map[orow0 + m] : m) * (uint32_t)(D * ES) + (uint32_t)(d * ES)
                                       : 0x80000000u;
              __builtin_amdgcn_raw_buffer_store_b128(w, rs, off, 0, 0);
            }
          }
        }
      }
    } else {
      // the fp32 carry rows of the owner, or (kPartF32) the piece's slot: 128 rows of
      // the D slice's kDePartCols columns, stored like kStoreF32
      float* carry = mode == kPartF32 ? a.de_part + (size_t)vwg * (kBwdTokens * kDePartCols) - (int64_t)c.ds * kDePartCols
                                      : a.de_acc + orow0 * D;
      const int64_t cstride = mode == kPartF32 ? kDePartCols : D;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          const int64_t m = wm * 64 + 32 * jj + n;
          if (m >= nrows) continue;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int64_t d = d00 + 32 * i + 8 * q;
            if (d >= D) continue;
            f32x4 v{acc[i][jj][4 * q], acc[i][jj][4 * q + 1], acc[i][jj][4 * q + 2], acc[i][jj][4 * q + 3]};
            f32x4* cp = reinterpret_cast<f32x4*>(carry + m * cstride + d);
            if (mode == kStoreF32 || mode == kPartF32) {
              *cp = v;
            } else if (mode == kAddF32) {
              *cp = *cp + v;
            } else {
              v = *cp + v;
              T* orow = out + (map ? (int64_t)map[orow0 + m] : m) * D;
#pragma unroll
              for (int k = 0; k < 4; ++k) orow[d + k] = (T)v[k];
            }
          }
        }
      }
      wait_vmcnt<0>();  // the fp32 modes leave nothing in flight for the stage waits
    }
  };

  Cur cs;
  if (seek(0, cs)) {  // this workgroup's bin or tasks
  prep(cs);
  Cur nx = cs, last = cs;
  bool have = true;
  // issue_next: the loads of nx (or, past the end, a repeat of the last one, which
  // keeps the per-stage load count uniform and is never consumed); advance_next:
  // step nx on, issuing the scalar list loads of its next tile.
  auto issue_next = [&](int st) { issue(have ? nx : last, st); };
  auto advance_next = [&]() {
    if (have) {
      last = nx;
      have = advance(nx);
    }
  };
  if constexpr (SPLIT) {
    // LDS reads of one 16-deep step: 8 for X, 4 (dE) or 8 (dC, transposing) for G
    sum_split_pipeline<S::STAGES, S::LPW, S::NSTORE, S::SPT, 8 + (PHASE == 0 ? 4 : 8)>(
        cs, acc, mode, issue_next, advance_next, frag_step, mma_step, epilogue, seek);
  } else if constexpr (ES == 2) {
    // A single G: the same pipeline over the four 16-deep steps of each 64-deep stage,
    // so the MFMAs of a stage's last step run across the barrier while the next
    // stage's first fragments are read.  LDS reads per step: 8 for X, 2 (dE) or 4 (dC,
    // transposing) for G.
    auto frag_ks = [&](int st, int ks, u32x4 (&x)[4], u32x4 (&g)[2]) {
      const char* sp = smem + st * S::STAGE;
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        if constexpr (PHASE == 0)
          g[jj] = lds_ld16(sp, go_n[jj][ks]);
        else
          g[jj] = frag_tr16(sp + go_t[0][jj] + 16 * ks * S::GTP, 4 * S::GTP);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = frag_tr16(sp + xo[i] + 16 * ks * S::XP, 4 * S::XP);
    };
    auto mma_ks = [&](const u32x4 (&x)[4], const u32x4 (&g)[2]) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) acc[i][jj] = Traits<T>::mfma(x[i], g[jj], acc[i][jj]);
    };
    static_assert(S::KS == 4 * S::KE, "four 16-deep steps per stage");
    sum_split_pipeline<S::STAGES, S::LPW, S::NSTORE, S::SPT, 8 + (PHASE == 0 ? 2 : 4), 4, 8, u32x4[4], u32x4[2]>(
        cs, acc, mode, issue_next, advance_next, frag_ks, mma_ks, epilogue, seek);
  } else {
#pragma unroll
  for (int p = 0; p < S::STAGES - 1; ++p) {
    issue_next(p);
    advance_next();
  }

  // Tasks outside, their steps inside: the accumulators are zeroed once per task,
  // so the step loop carries them only through MFMAs (no register copies), while
  // issue_next keeps STAGES - 1 slices in flight across the task boundary.
  int st = 0;
  int since_store = S::STAGES;  // steps since the last epilogue that left stores in flight
  for (;;) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) acc[i][jj] = zero16();
    for (;;) {
      if (since_store < S::STAGES)
        stage_barrier<(S::STAGES - 2) * S::LPW + S::NSTORE>();
      else
        stage_barrier<(S::STAGES - 2) * S::LPW>();
      issue_next((st + S::STAGES - 1) % S::STAGES);
      frags(st);
      mma();
      schedule();
      advance_next();
      ++since_store;
      st = st + 1 == S::STAGES ? 0 : st + 1;
      if (++cs.h < S::SPT) continue;
      cs.h = 0;
      if (++cs.j == cs.cnt) break;
    }
    epilogue(cs);
    if (mode == kWriteT) since_store = 1;
    if (!seek(cs.q + 1, cs)) break;
  }
  wait_vmcnt<0>();
  }
  }
  if constexpr (PHASE == 1 && ES == 2 && !SPLIT) {
    // Block tasks: up to kDcBlkChunk owners with one kept tile in the same token block,
    // per D slice, taken from the pass's counter once the bins are done.  The block's E
    // slice (128 rows x 256 columns) is loaded once into the X regions of stages 0 and
    // 1; the owners' G
    // tiles stream through two buffers: buffer 0 in the G regions of stages 0 and 1,
    // buffer 1 in the G region of stage 2 and the first 16 KiB of its X region.  Each
    // owner's sums are the bin path's: the same MFMAs in the same order.
    const int nbt = ldu(pi, kPiDcBlk) * nds;
    if (nbt == 0) return;
    const int* blk_task = a.dc_blk_task + 4 * ldu(pi, kPiVt0);
    const int* blk_own = a.dc_blk_own + 2 * ldu(pi, kPiVt0);
    // stage base whose G region (base + X_BYTES) holds half hh of buffer buf
    auto gsb = [&](int buf, int hh) -> uint32_t {
      return buf == 0 ? (uint32_t)(hh * S::STAGE) : (uint32_t)(2 * S::STAGE - (hh ? S::X_BYTES : 0));
    };
    static_assert(2 * S::STAGE - S::X_BYTES + S::X_BYTES + S::G_BYTES <= 2 * S::STAGE + S::X_BYTES,
                  "buffer 1's second half ends inside stage 2's X region");
    auto blk_ks = [&](int buf, int st, u32x4 (&x)[4], u32x4 (&g)[2]) {  // step st = 4 hh + ks
      const char* spe = smem + (st >> 2) * S::STAGE;
      const char* spg = smem + gsb(buf, st >> 2);
      const int ks = st & 3;
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) g[jj] = frag_tr16(spg + go_t[0][jj] + 16 * ks * S::GTP, 4 * S::GTP);
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = frag_tr16(spe + xo[i] + 16 * ks * S::XP, 4 * S::XP);
    };
    auto blk_mma = [&](const u32x4 (&x)[4], const u32x4 (&g)[2]) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) acc[i][jj] = Traits<T>::mfma(x[i], g[jj], acc[i][jj]);
    };
    int* box = reinterpret_cast<int*>(smem);
    for (;;) {
      wait_vmcnt<0>();
      __syncthreads();  // every wave is done with the LDS of the last task
      if (threadIdx.x == 0) box[0] = atomicAdd(&a.pinfo[pass * kPassInts + kPiDcQueue], 1);
      __syncthreads();
      const int t = __builtin_amdgcn_readfirstlane(box[0]);
      if (t >= nbt) break;
      __syncthreads();  // box is read before the DMA below overwrites it
      const int bi = t / nds, ds = t - bi * nds;
      const int o0 = ldu(blk_task, 4 * bi + 1), o1 = ldu(blk_task, 4 * bi + 2);
      const int64_t xr = (int64_t)ldu(blk_task, 4 * bi) * kBwdTokens;
      issue_x(xr, ds, smem_lds);
      issue_x(xr + S::KS, ds, smem_lds + S::STAGE);
      const int slot0 = ldu(blk_own, 2 * o0 + 1);
      issue_g(slot0, 0, smem_lds + gsb(0, 0));
      issue_g(slot0, 1, smem_lds + gsb(0, 1));
      for (int o = o0; o < o1; ++o) {
        const int buf = (o - o0) & 1;
        // this owner's G tile (and, first, the E slice) has landed: only the last
        // owner's stores may still be in flight
        if (o == o0)
          wait_vmcnt<0>();
        else
          wait_vmcnt<S::NSTORE>();
        __syncthreads();  // ... for every wave, and every wave is done with the other buffer
        if (o + 1 < o1) {
          const int ns = ldu(blk_own, 2 * (o + 1) + 1);
          issue_g(ns, 0, smem_lds + gsb(buf ^ 1, 0));
          issue_g(ns, 1, smem_lds + gsb(buf ^ 1, 1));
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int jj = 0; jj < 2; ++jj) acc[i][jj] = zero16();
        u32x4 xa[4], ga[2], xb[4], gb[2];
        blk_ks(buf, 0, xa, ga);
#pragma unroll
        for (int st = 0; st < 8; st += 2) {  // read step st + 1 while the MFMAs of step st run
          blk_ks(buf, st + 1, xb, gb);
          blk_mma(xa, ga);
          sched_interleave<0, 8, 12, 0, 0>();
          __builtin_amdgcn_sched_barrier(0);
          if (st + 2 < 8) blk_ks(buf, st + 2, xa, ga);
          blk_mma(xb, gb);
          if (st + 2 < 8)
            sched_interleave<0, 8, 12, 0, 0>();
          else
            sched_interleave<0, 8, 0, 0, 0>();
          __builtin_amdgcn_sched_barrier(0);
        }
        Cur c;
        c.owner = ldu(blk_own, 2 * o);
        c.ds = ds;
        epilogue(c);
      }
    }
    wait_vmcnt<0>();
  }
}

// ---------------------------------------------------------------- 5b. dE pieces
// The narrow dE sums cut some of a pass's tasks (token block, D slice) into npc pieces
// along their kept tiles (kPartF32, de_pieces_of): here the pieces' fp32 sums are added
// in piece order and dE is written in the pass's mode, as the sums' epilogue writes a
// whole task.  32 workgroups per task, 4 of its rows each; a thread takes 4 columns of
// one row and adds the npc pieces' values with four sums in flight.  The grid covers
// the most tasks that are cut (kDePartSlots / 2: two pieces each at least).
constexpr int kDePiecesPerTask = kBwdTokens / 4;
constexpr int kDePiecesGrid = kDePiecesPerTask * (kDePartSlots / 2);
template <typename T>
__global__ __launch_bounds__(256) void bwd_de_pieces_kernel(BwdArgs a, int chunk, int pass, int nwg) {
  (void)chunk;
  const int* pi = a.pinfo + pass * kPassInts;
  const int mode = ldu(pi, kPiDeMode);
  if (mode < 0 || a.de_part == nullptr) return;
  const int nrb = (int)a.plan.nrb;
  const int nds = (int)((a.D + kDePartCols - 1) / kDePartCols);
  const int ntasks = ldu(pi, kPiOwnRb) * nds;
  int tbase, ncut, npc;
  de_pieces_of(a, ntasks, nwg, tbase, ncut, npc);
  const int ti = (int)(blockIdx.x / kDePiecesPerTask);  // the cut task's index
  if (npc == 1 || ti >= ncut) return;                    // the sums ran whole tasks
  const int task = tbase + ti;
  const int owner = ldu(a.own_rb + pass * nrb, task / nds);
  const int ds = task - (task / nds) * nds;
  const int* rbs = a.rb_start + pass * nrb;
  const int cnt = ldu(rbs, owner + 1) - ldu(rbs, owner);
  const RowData rd = row_data(a);
  const int64_t D = a.D;
  const int64_t orow0 = (int64_t)owner * kBwdTokens;
  const int64_t nrows = a.N - orow0 < kBwdTokens ? a.N - orow0 : kBwdTokens;
  const int col = (int)(threadIdx.x & 63) * 4;
  const int64_t d = (int64_t)ds * kDePartCols + col;
  if (d >= D) return;  // D is a multiple of 4: the 4 columns are inside
  T* dE = reinterpret_cast<T*>(a.dE);
  {
    const int m = (int)(blockIdx.x % kDePiecesPerTask) * 4 + (int)(threadIdx.x >> 6);
    if (m >= nrows) return;
    const float* src = a.de_part + ((size_t)ti * npc * kBwdTokens + m) * kDePartCols + col;
    constexpr size_t kSlot = (size_t)kBwdTokens * kDePartCols;
    // pieces k ascending; an empty piece (never written) adds nothing
    auto piece = [&](int k) -> f32x4 {
      return k * cnt / npc == (k + 1) * cnt / npc ? f32x4{0.f, 0.f, 0.f, 0.f}
                                                  : *reinterpret_cast<const f32x4*>(src + (size_t)k * kSlot);
    };
    f32x4 sum{0.f, 0.f, 0.f, 0.f};
    int k = 0;
    for (; k + 4 <= npc; k += 4) {
      const f32x4 p0 = piece(k), p1 = piece(k + 1), p2 = piece(k + 2), p3 = piece(k + 3);
      sum += p0;
      sum += p1;
      sum += p2;
      sum += p3;
    }
    for (; k < npc; ++k) sum += piece(k);
    const int64_t orow = rd.map ? (int64_t)rd.map[orow0 + m] : orow0 + m;
    if (mode != kWriteT) {
      f32x4* cp = reinterpret_cast<f32x4*>(a.de_acc + (orow0 + m) * D + d);
      if (mode == kStoreF32) {
        *cp = sum;
        return;
      }
      if (mode == kAddF32) {
        *cp = *cp + sum;
        return;
      }
      sum = *cp + sum;  // kFinishT
    }
    T* o = dE + orow * D + d;
#pragma unroll
    for (int k = 0; k < 4; ++k) o[k] = (T)sum[k];
  }
}

// ---------------------------------------------------------------- 6. dBias
// One workgroup per vocab tile of the pass: the sum of its slots' column sums.
template <typename T>
__global__ __launch_bounds__(kBwdVocab) void bwd_dbias_kernel(BwdArgs a, int chunk, int pass) {
  const int* pi = a.pinfo + pass * kPassInts;
  const int vlo = chunk * (int)a.plan.chunk_nvt;
  const int v = ldu(pi, kPiVt0) + (int)blockIdx.x;
  if (v >= ldu(pi, kPiVt1)) return;
  const int s0 = ldu(pi, kPiS0);
  const int b = ldu(a.vt_start, v), e = ldu(a.vt_start, v + 1);
  float sum = 0.f;
  for (int k = b; k < e; ++k) sum += a.colsum[(size_t)(ldu(a.vt_slot, k) - s0) * kBwdVocab + threadIdx.x];
  const int64_t col = (int64_t)(vlo + v) * kBwdVocab + threadIdx.x;
  if (col < a.V) reinterpret_cast<T*>(a.dBias)[col] = (T)sum;
}

// ---------------------------------------------------------------- launch
template <typename T, bool HB>
static void launch_g(const BwdArgs& a, int chunk, int pass, dim3 grid, hipStream_t s) {
  const bool g = a.dE != nullptr || a.dC != nullptr, db = a.dBias != nullptr;
  const bool rg = (a.D * (int64_t)sizeof(T)) % kGSlice != 0;
#define CCE_G(G, DB, RG)                                                                               \
  if (g == G && db == DB && rg == RG) {                                                                \
    hipLaunchKernelGGL((bwd_g_kernel<T, HB, G, DB, RG>), grid, dim3(kGThreads), 0, s, a, chunk, pass); \
    return;                                                                                            \
  }
  CCE_G(true, true, false)
  CCE_G(true, false, false)
  CCE_G(false, true, false)
  CCE_G(true, true, true)
  CCE_G(true, false, true)
  CCE_G(false, true, true)
#undef CCE_G
}

template <typename T, bool HB>
static void launch_g_dense(const BwdArgs& a, int chunk, int pass, dim3 grid, hipStream_t s) {
  const bool g = a.dE != nullptr || a.dC != nullptr, db = a.dBias != nullptr;
  const bool rg = (a.D * (int64_t)sizeof(T)) % kSliceBytes != 0;
#define CCE_GD(G, DB, RG)                                                                                          \
  if (g == G && db == DB && rg == RG) {                                                                            \
    hipLaunchKernelGGL((bwd_g_dense_kernel<T, HB, G, DB, RG>), grid, dim3(kGDThreads), 0, s, a, chunk, pass);      \
    return;                                                                                                        \
  }
  CCE_GD(true, true, false)
  CCE_GD(true, false, false)
  CCE_GD(false, true, false)
  CCE_GD(true, true, true)
  CCE_GD(true, false, true)
  CCE_GD(false, true, true)
#undef CCE_GD
}

// The sums of one phase (0 dE, 1 dC) in the wide or narrow geometry, over G tiles
// rounded once or (16-bit a.g_split) held as the hi / lo pair.
template <typename T, int PHASE>
static void launch_sum(const BwdArgs& a, bool wide, int chunk, int pass, int grid, hipStream_t s) {
  if constexpr (sizeof(T) == 2) {
    if (a.g_split) {
      if (wide)
        hipLaunchKernelGGL((bwd_sum_kernel<T, PHASE, true>), dim3(grid), dim3(SumGeo<T, true>::NT), 0, s, a, chunk,
                           pass);
      else
        hipLaunchKernelGGL((bwd_sum_narrow_kernel<T, PHASE, true>), dim3(grid), dim3(SumGeoNarrow<T, true>::NT), 0, s,
                           a, chunk, pass);
      return;
    }
  }
  if (wide)
    hipLaunchKernelGGL((bwd_sum_kernel<T, PHASE, false>), dim3(grid), dim3(SumGeo<T, false>::NT), 0, s, a, chunk, pass);
  else
    hipLaunchKernelGGL((bwd_sum_narrow_kernel<T, PHASE, false>), dim3(grid), dim3(SumGeoNarrow<T, false>::NT), 0, s, a,
                       chunk, pass);
}

// dE sums: the wide geometry (512 columns per task, measured 0.85x the time of two
// narrow tasks) unless it leaves so few tasks that the narrow one finishes in fewer
// rounds of equal tasks over the persistent grid.  With the filter on the owners' kept
// counts differ, and two or four wide tasks per workgroup balance worse than twice as
// many narrow ones (c3: the wide tasks' 18 to 28 kept tiles per workgroup; narrow
// measured 10-13 us faster at c3 and c4), so the filter on takes the narrow one.
// a.de_geo forces one (1 wide, 2 narrow).
static bool use_wide_de_sums(const BwdArgs& a, int grid) {
  if (a.de_geo != 0) return a.de_geo == 1;
  if (a.filter_log_eps > -INFINITY) return false;
  const BwdPlan& P = a.plan;
  const int64_t tw = P.nrb * ((a.D + 511) / 512), tn = P.nrb * ((a.D + 255) / 256);
  const int64_t rw = (tw + grid - 1) / grid, rn = (tn + grid - 1) / grid;
  return rw * 512 * 85 < rn * 256 * 100;
}

// dC sums: with the filter off every owner keeps all of its token blocks and the wide
// geometry runs ~35% faster.  With the filter on the compaction picks one per pass
// (kPiDcWide): narrow when one owner keeps so many blocks that its tasks outlast a
// workgroup's average share (skewed targets, c3), else wide (c2, c4: 50-55 us faster).
// The host then launches both kernels and the one not picked returns at once: one
// kernel holding both bodies spilled the narrow one's registers (measured 50-90 us
// slower).  This function decides the dense G kernel and the forced choices; a.dc_geo
// forces one (1 wide, 2 narrow).
static bool use_wide_dc_sums(const BwdArgs& a) {
  if (a.dc_geo != 0) return a.dc_geo == 1;
  return !(a.filter_log_eps > -INFINITY);
}

template <typename T>
static hipError_t backward_typed(const BwdArgs& a, hipStream_t s, hipEvent_t pass_ev) {
  const BwdPlan& P = a.plan;
  const int items = (int)(P.nrb * P.nwords);
  const bool sorted_ok = a.perm != nullptr;  // the workspace holds the sorted token order
  hipError_t err;
  if (sorted_ok) {
    const dim3 fg((unsigned)(1 + (items + 15) / 16));
    if (a.N <= 8 * 1024 && P.nvt < kCsKeys)
      hipLaunchKernelGGL(bwd_filter_csort_kernel<8>, fg, dim3(1024), 0, s, a);
    else if (a.N <= 16 * 1024 && P.nvt < kCsKeys)
      hipLaunchKernelGGL(bwd_filter_csort_kernel<16>, fg, dim3(1024), 0, s, a);
    else if (a.N <= 8 * 1024)
      hipLaunchKernelGGL(bwd_filter_sort_kernel<8>, fg, dim3(1024), 0, s, a);
    else if (a.N <= 16 * 1024)
      hipLaunchKernelGGL(bwd_filter_sort_kernel<16>, fg, dim3(1024), 0, s, a);
    else if (a.N <= 32 * 1024)
      hipLaunchKernelGGL(bwd_filter_sort_kernel<32>, fg, dim3(1024), 0, s, a);
    else
      hipLaunchKernelGGL(bwd_filter_sort_kernel<kSortMaxRounds>, fg, dim3(1024), 0, s, a);
  } else {
    hipLaunchKernelGGL(bwd_filter_kernel, dim3((unsigned)((items + 3) / 4)), dim3(256), 0, s, a);
  }
  if ((err = hipGetLastError()) != hipSuccess) return err;
  if (sorted_ok) {
    hipLaunchKernelGGL(bwd_filter_sorted_kernel, dim3((unsigned)((items + 3) / 4)), dim3(256), 0, s, a);
    if ((err = hipGetLastError()) != hipSuccess) return err;
  }
  const bool want_de = a.dE != nullptr, want_dc = a.dC != nullptr, want_db = a.dBias != nullptr;
  const int cus = a.num_cus > 0 ? a.num_cus : 256;
  const int gp = (cus + 7) / 8 * 8;  // persistent grids: a multiple of the 8 XCDs
  const int dtype = sizeof(T) == 4 ? 0 : (std::is_same<T, _Float16>::value ? 1 : 2);
  const bool wide_de = use_wide_de_sums(a, gp), wide_dc = use_wide_dc_sums(a);
  // With the filter off the G tiles are one dense block per pass: the forward's tiling
  // (the narrow dC sums need the G kernel's dC schedule, so they keep that kernel).
  const bool dense_g = !(a.filter_log_eps > -INFINITY) && (!want_dc || wide_dc);
  // the filtered backward's dC geometry: the compaction's choice per pass
  const bool auto_dc = a.dc_geo == 0 && a.filter_log_eps > -INFINITY;
  for (int chunk = 0; chunk < (int)P.n_chunks; ++chunk) {
    const int vlo = chunk * (int)P.chunk_nvt;
    const int nv = (int)(P.nvt - vlo < P.chunk_nvt ? P.nvt - vlo : P.chunk_nvt);
    // chunk 0 also copies the rows into the sorted order (extra workgroups)
    const unsigned cg = 1 + (chunk == 0 && sorted_ok ? (unsigned)((a.N + 15) / 16) : 0u);
    hipLaunchKernelGGL(bwd_compact_kernel, dim3(cg), dim3(1024), 0, s, a, chunk);
    if ((err = hipGetLastError()) != hipSuccess) return err;
    if (!(want_de || want_dc || want_db)) continue;
    if (a.host_pass != nullptr && (err = hipEventRecord(pass_ev, s)) != hipSuccess) return err;
    // Quantized classifier rows: dequantize the rows of this chunk's tiles that keep
    // pairs (the compaction's vt_start) into the scratch and let c address it at global
    // row numbers (only the G kernel and the dE sums read c, and only kept tiles' rows).
    BwdArgs ac = a;
    if (a.q.wq != nullptr) {
      const int64_t r0 = (int64_t)vlo * kBwdVocab;
      const int64_t r1 = (int64_t)(vlo + nv) * kBwdVocab < a.V ? (int64_t)(vlo + nv) * kBwdVocab : a.V;
      err = launch_dequantize(dtype, a.q, r0, r1 - r0, a.D, a.q.scratch, s, a.vt_start);
      if (err != hipSuccess) return err;
      ac.c = reinterpret_cast<const char*>(a.q.scratch) - r0 * a.D * (int64_t)sizeof(T);
    }
    auto launch_g_pass = [&](int pass) {
      if (dense_g && a.bias)
        launch_g_dense<T, true>(ac, chunk, pass, dim3(gp), s);
      else if (dense_g)
        launch_g_dense<T, false>(ac, chunk, pass, dim3(gp), s);
      else if (a.bias)
        launch_g<T, true>(ac, chunk, pass, dim3(gp), s);
      else
        launch_g<T, false>(ac, chunk, pass, dim3(gp), s);
      return hipGetLastError();
    };
    // The sums of one pass; dc_pick: the dC geometry the compaction chose for it (1
    // wide, 0 narrow), or -1 when unknown on the host (both are launched, and the one
    // not chosen returns at once).
    auto launch_sums = [&](int pass, int dc_pick) {
      hipError_t e2;
      if (want_de) {
        launch_sum<T, 0>(ac, wide_de, chunk, pass, gp, s);
        if ((e2 = hipGetLastError()) != hipSuccess) return e2;
        if (!wide_de && a.de_part != nullptr) {  // pieces of dE tasks (de_pieces_of)
          if (P.nrb * ((a.D + kDePartCols - 1) / kDePartCols) > gp) {  // tasks may overflow the grid
            BwdArgs a1 = ac;
            a1.de_stage = 1;
            launch_sum<T, 0>(a1, false, chunk, pass, gp, s);
            if ((e2 = hipGetLastError()) != hipSuccess) return e2;
          }
          hipLaunchKernelGGL((bwd_de_pieces_kernel<T>), dim3((unsigned)kDePiecesGrid), dim3(256), 0, s, a, chunk,
                             pass, gp);
          if ((e2 = hipGetLastError()) != hipSuccess) return e2;
        }
      }
      if (want_dc) {
        const bool narrow = auto_dc ? dc_pick != 1 : !wide_dc;
        const bool wide = auto_dc ? dc_pick != 0 : wide_dc;
        if (narrow) launch_sum<T, 1>(a, false, chunk, pass, gp, s);
        if (wide) launch_sum<T, 1>(a, true, chunk, pass, gp, s);
        if ((e2 = hipGetLastError()) != hipSuccess) return e2;
      }
      if (want_db) {
        hipLaunchKernelGGL((bwd_dbias_kernel<T>), dim3((unsigned)nv), dim3(kBwdVocab), 0, s, a, chunk, pass);
        if ((e2 = hipGetLastError()) != hipSuccess) return e2;
      }
      return hipSuccess;
    };
    if (a.host_pass != nullptr) {
      // The host reads the compaction's pass summary: the first G kernel is queued
      // before the wait (it runs while the host waits and launches the rest), then
      // exactly the passes the data needs, each with the dC geometry chosen for it.
      if ((err = launch_g_pass(0)) != hipSuccess) return err;
      if ((err = hipEventSynchronize(pass_ev)) != hipSuccess) return err;
      const int npass = a.host_pass[0];
      if (npass < 1 || npass > (int)P.max_passes) return hipErrorInvalidValue;
      for (int pass = 0; pass < npass; ++pass) {
        if (pass > 0 && (err = launch_g_pass(pass)) != hipSuccess) return err;
        if ((err = launch_sums(pass, a.host_pass[1 + pass])) != hipSuccess) return err;
      }
      continue;
    }
    // Every pass the chunk may need; passes past the data's last return at once.
    for (int pass = 0; pass < (int)P.max_passes; ++pass) {
      if ((err = launch_g_pass(pass)) != hipSuccess) return err;
      if ((err = launch_sums(pass, -1)) != hipSuccess) return err;
    }
  }
  return hipGetLastError();
}

hipError_t launch_backward(int dtype, const BwdArgs& a, hipStream_t s, hipEvent_t pass_ev) {
  if (a.host_pass != nullptr && pass_ev == nullptr) return hipErrorInvalidValue;
  switch (dtype) {
    case 0:
      return backward_typed<float>(a, s, pass_ev);
    case 1:
      return backward_typed<_Float16>(a, s, pass_ev);
    default:
      return backward_typed<__bf16>(a, s, pass_ev);
  }
}

}  // namespace cce
