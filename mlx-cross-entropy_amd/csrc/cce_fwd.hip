// cce_fwd.hip — forward pass of Cut Cross-Entropy on CDNA4 (gfx950).
//
// fwd_tile_kernel: one workgroup computes a 256-token x 256-vocabulary block of
// logits S^T = C_blk . E_blk^T on MFMA (contraction over D staged through LDS),
// adds the bias, and reduces it on the spot: for every (token, 128-column
// vocabulary tile) it writes the tile max and the sum of exp(logit - max), and
// the wave whose tile holds a token's target writes -(target logit).  The [N, V]
// logits never leave registers.
//   Reference: csrc/cce/cce.metal:19-135 (cce_forward: 32x32 simdgroup tile,
//   per-row max/sum-exp over 32 columns, target gather :108-115).
//
// lse_kernel: per token, merges the per-tile (max, sum-exp) pairs into
// lse = max + log(sum) and forms the masked per-token loss.
//   Reference: csrc/cce/cce.metal:332-355 (reduce_tile_to_lse) and the masking of
//   mlx_cce/__init__.py:59-70 (valid = targets != ignore_index, nll * valid).
#include <type_traits>

#include "cce_device.h"
#include "cce_launch.h"

namespace cce {

static_assert(kStatTile == 128, "one wave covers one statistic tile");

// Waves of the forward tile: 2 along the vocabulary (128 rows each, one statistic
// tile) x kFwdWB along the tokens.  With kFwdWB = 4 two waves share each SIMD, so
// one wave's LDS / barrier / epilogue stalls are covered by the other's MFMAs.
#ifndef CCE_FWD_WB
#define CCE_FWD_WB 4
#endif
constexpr int kFwdWB = CCE_FWD_WB;
template <typename T>
using FwdLoop = NTMainLoop<T, kFwdVocab, kFwdTokens, 2, kFwdWB>;  // A = C rows (vocab), B = E rows (tokens)

// Persistent schedule of the forward tiles.  The grid is 8 * cpx workgroups, one
// per CU: the hardware deals workgroups to the 8 XCDs round-robin, so workgroup b
// runs on XCD b % 8 as that XCD's member s = b / 8.  Tiles are grouped in rounds of
// gt token blocks x gv vocabulary blocks (gt * gv = cpx), numbered token-group
// major; XCD x takes rounds [x R / 8, (x + 1) R / 8).  In a round, member s
// computes tile (token block tg gt + s % gt, vocabulary block vg gv + s / gt).
// All members of an XCD do equal work per round, so they move through the rounds
// together and stream the same gt E blocks and gv C blocks through that XCD's L2
// at the same time; the XCDs sweep the vocabulary in step, so they share C blocks
// in the infinity cache.
struct FwdSched {
  int ntb, nvb;     // token / vocabulary blocks (the launch covers blocks vb0 .. vb0 + nvb - 1)
  int gt, gv, ngv;  // round shape, vocabulary groups
  int rounds;       // R
  int nvt;          // statistic tiles of the whole vocabulary
  int vb0;          // first vocabulary block (a chunk of dequantized rows; 0 otherwise)
};

// Epilogue of one tile (its bias already added), registers only: ragged-vocabulary mask, per token
// and 128-column tile the max and sum of exp(logit - max), and the target gather.
// acc[i][j][r] holds logit(vocab = vbase + 32i + 8(r/4) + 4h + r%4,
//                          token = tbase + 32j + n)   with n = lane%32, h = lane/32.
// S32: the statistics per 32 columns (the four 32-row blocks i of the wave's tile)
// in the reference's layout, [N][ceil(V/32)], instead of per 128 columns.
// The epilogue's stores of a tile (per token the statistics of its 128-column tile, and
// the target logit) go out right after the next tile's first stage barrier instead of
// just before it: every stage barrier waits for all of a wave's memory operations, so
// stores issued at the end of the epilogue held the next tile's first slice for their
// write latency (≈0.5% of the forward at c3).  The last tile stores at once.
template <int TJ>
struct FwdPending {
  float m[TJ], s[TJ], tv[TJ];
  uint32_t flags;  // bit j: statistics of column j; bit 8 + j: its target logit
};

// The stores fwd_epilogue deferred: tile (tb, vb)'s statistics and target logits.
template <int TJ>
__device__ __forceinline__ void fwd_store_pending(const FwdArgs& a, const FwdPending<TJ>& p, int tb, int vb) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wv = wave & 1, wt = wave >> 1;
  const int64_t vbase = (int64_t)vb * kFwdVocab + wv * 128;
  const int64_t tbase = (int64_t)tb * kFwdTokens + wt * (kFwdTokens / kFwdWB);
  const int tile = (int)(vbase / kStatTile);
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    const int64_t tok = tbase + j * 32 + (lane & 31);
    if (p.flags & (1u << j)) {
      a.tile_max[(size_t)tile * a.N + tok] = p.m[j];
      a.tile_sum_exp[(size_t)tile * a.N + tok] = p.s[j];
    }
    if (p.flags & (1u << (8 + j))) a.neg_target_logit[tok] = p.tv[j];
  }
}

// How a tile kernel adds the bias: none; from global memory after the contraction
// (fwd_add_bias); or as the accumulators' starting value, staged through LDS
// (fwd_stage_bias / fwd_init_bias_lds), when the bias is 16-byte aligned and
// V * sizeof(T) is a multiple of 16 (no 16-byte piece of the bias then straddles its
// end).  The two orders of the fp32 sums differ in the last bits.
enum FwdBias { kBiasNone = 0, kBiasGlobal = 1, kBiasLds = 2 };

// The bias of the wave's 128 vocabulary rows added to a tile's logits.  The tile
// kernel does this before it issues the next tile's pipeline fill: waiting for the
// bias loads after it would wait for the fill's DMA as well (vmcnt counts in order).
template <typename T, int TI, int TJ>
__device__ __forceinline__ void fwd_add_bias(const FwdArgs& a, f32x16 (&acc)[TI][TJ], int vb) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int h = lane >> 5;
  const int64_t vbase = (int64_t)vb * kFwdVocab + (wave & 1) * 128;
  const T* bias = reinterpret_cast<const T*>(a.bias);
#pragma unroll
  for (int i = 0; i < TI; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t v = vbase + i * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
      const float add = v < a.V ? to_f32(bias[v]) : 0.f;
#pragma unroll
      for (int j = 0; j < TJ; ++j) acc[i][j][r] += add;
    }
  }
}

// The bias through LDS (kBiasLds).  Per tile the block's kFwdVocab bias values (1
// KiB at most; zeros past V) are copied into an LDS buffer by one LDS-DMA load of
// wave 0, issued ahead of the tile's pipeline fill, so that the tile's first stage
// barrier, which waits for all of a wave's loads, covers it.  Right after that barrier
// the accumulators are set to the bias (fwd_init_bias_lds), and the MFMAs add the
// products to it: no bias work is left in the epilogue, where 64 global loads per
// lane cost 7% of the forward at N = 4096, D = 2304, V = 256000 (adding from LDS
// there still 4%: the added registers spilled).  The buffer is rewritten at the end
// of the tile that read it, after every wave has passed the tile's stage barriers.
constexpr int kBiasLdsBytes = 1024;
static_assert(kFwdVocab * 4 <= kBiasLdsBytes, "one LDS-DMA load holds a block's bias");
// The lane index, formed where it is used: a value the compiler cannot hoist out of the
// tile loop, where it would hold a register through every main loop.
__device__ __forceinline__ int lane_here() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}
template <typename T>
__device__ __forceinline__ void fwd_stage_bias(const FwdArgs& a, int vb, char* buf) {
  if (__builtin_amdgcn_readfirstlane(threadIdx.x >> 6) != 0) return;  // wave 0 (a uniform branch)
  constexpr int chunks = kFwdVocab * (int)sizeof(T) / 16;  // 16-byte pieces of a block's bias
  const int lane = lane_here();
  // lanes past the block's pieces load the first ones again (into bytes nobody reads)
  const int64_t off = ((int64_t)vb * kFwdVocab * (int64_t)sizeof(T)) + (lane % chunks) * 16;
  const char* g = off < a.V * (int64_t)sizeof(T) ? reinterpret_cast<const char*>(a.bias) + off
                                                  : reinterpret_cast<const char*>(g_zero16);
  dma16(g, __builtin_amdgcn_readfirstlane(lds_addr(buf)));
}
// acc[i][j][r] = the bias of the register's vocabulary column (see fwd_epilogue's layout).
template <typename T, int TI, int TJ>
__device__ __forceinline__ void fwd_init_bias_lds(const char* buf, f32x16 (&acc)[TI][TJ]) {
  const int lane = lane_here();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c0 = (wave & 1) * 128 + (lane >> 5) * 4;
#pragma unroll
  for (int i = 0; i < TI; ++i) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      // columns c0 + 32 i + 8 q + 0..3 of the block: registers r = 4 q + 0..3
      const int col = c0 + i * 32 + q * 8;
      float add[4];
      if constexpr (sizeof(T) == 4) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(buf + col * 4);
#pragma unroll
        for (int k = 0; k < 4; ++k) add[k] = v[k];
      } else {
        const uint2 w = *reinterpret_cast<const uint2*>(buf + col * 2);
        const uint32_t h[4] = {w.x & 0xffffu, w.x >> 16, w.y & 0xffffu, w.y >> 16};
#pragma unroll
        for (int k = 0; k < 4; ++k) add[k] = to_f32(__builtin_bit_cast(T, (uint16_t)h[k]));
      }
#pragma unroll
      for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j][4 * q + k] = add[k];
    }
  }
}

template <typename T, bool S32, int TI, int TJ>
__device__ __forceinline__ void fwd_epilogue(const FwdArgs& a, int nvt, f32x16 (&acc)[TI][TJ], int tb, int vb,
                                             const int64_t (&tg)[TJ], FwdPending<TJ>* pend = nullptr) {
  if (pend) pend->flags = 0;
  static_assert(TI == 4, "a wave covers one 128-column statistic tile");
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wv = wave & 1;   // vocab half (NTMainLoop: wa = wave % 2)
  const int wt = wave >> 1;  // token part of kFwdTokens / kFwdWB rows
  const int n = lane & 31;
  const int h = lane >> 5;
  const int64_t vbase = (int64_t)vb * kFwdVocab + wv * 128;
  const int64_t tbase = (int64_t)tb * kFwdTokens + wt * (kFwdTokens / kFwdWB);

  if (vbase + 128 > a.V) {  // last vocabulary block only (uniform per wave)
    const int lim = (int)(a.V - vbase) - 4 * h;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const bool ok = i * 32 + (r >> 2) * 8 + (r & 3) < lim;
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j][r] = ok ? acc[i][j][r] : -INFINITY;
      }
  }

  const int tile = (int)(vbase / kStatTile);
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    const int64_t tok = tbase + j * 32 + n;

    if constexpr (S32) {
      const int64_t nt = (a.V + kRefStatTile - 1) / kRefStatTile;
      const int64_t g0 = vbase / kRefStatTile;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float m = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) m = fmaxf(m, acc[i][j][r]);
        m = fmaxf(m, __shfl_xor(m, 32));
        const float mb = (m == -INFINITY) ? 0.f : m * kLog2e;
        float s = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) s += __builtin_amdgcn_exp2f(fmaf(acc[i][j][r], kLog2e, -mb));
        s += __shfl_xor(s, 32);
        if (h == 0 && tok < a.N && g0 + i < nt) {
          a.tile_max[tok * nt + g0 + i] = m;
          a.tile_sum_exp[tok * nt + g0 + i] = s;
        }
      }
    } else {
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) m = fmaxf(m, acc[i][j][r]);
    m = fmaxf(m, __shfl_xor(m, 32));
    const float mb = (m == -INFINITY) ? 0.f : m * kLog2e;
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) s += __builtin_amdgcn_exp2f(fmaf(acc[i][j][r], kLog2e, -mb));
    s += __shfl_xor(s, 32);

    if (pend) {
      pend->m[j] = m;
      pend->s[j] = s;
      if (h == 0 && tok < a.N && tile < nvt) pend->flags |= 1u << j;
    } else if (h == 0 && tok < a.N && tile < nvt) {
      a.tile_max[(size_t)tile * a.N + tok] = m;
      a.tile_sum_exp[(size_t)tile * a.N + tok] = s;
    }
    }

    // Target gather: the lane holding (target, token) writes -(logit + bias).
    const int64_t loc = tg[j] - vbase;
    const bool hit = tok < a.N && loc >= 0 && loc < 128 && tg[j] < a.V;
    if (__any(hit)) {
      const int li = hit ? (int)loc : 0;
      const int ti = li >> 5;
      const int vv = li & 31;
      const int ht = (vv >> 2) & 1;
      const int rt = ((vv >> 3) << 2) | (vv & 3);
      float val = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) val = (i == ti && r == rt) ? acc[i][j][r] : val;
      if (pend) {
        pend->tv[j] = -val;
        if (hit && h == ht) pend->flags |= 1u << (8 + j);
      } else if (hit && h == ht) {
        a.neg_target_logit[tok] = -val;
      }
    }
  }
}

template <typename T, int BIAS, bool RAGGED, bool S32>
__global__ __launch_bounds__(FwdLoop<T>::NTHREADS, 1) void fwd_tile_kernel(FwdArgs a, FwdSched sc) {
  using Loop = FwdLoop<T>;
  constexpr int TI = Loop::TI, TJ = Loop::TJ;
  __shared__ __attribute__((aligned(16))) char smem[Loop::SMEM_BYTES];
  __shared__ __attribute__((aligned(16))) char bias_lds[BIAS == kBiasLds ? kBiasLdsBytes : 16];

  const int xcd = blockIdx.x & 7;
  const int member = blockIdx.x >> 3;
  const int st = member % sc.gt, sv = member / sc.gt;
  const int r_end = (int)((int64_t)(xcd + 1) * sc.rounds / 8);
  // first round at or after r that holds a tile for this member (r_end if none)
  auto next_round = [&](int r, int& tb, int& vb) {
    for (; r < r_end; ++r) {
      tb = (r / sc.ngv) * sc.gt + st;
      vb = (r % sc.ngv) * sc.gv + sv;
      if (tb < sc.ntb && vb < sc.nvb) break;
    }
    vb += sc.vb0;
    return r;
  };
  const int64_t pitch = a.D * (int64_t)sizeof(T);
  const char* C = reinterpret_cast<const char*>(a.c);
  const char* E = reinterpret_cast<const char*>(a.e);
  auto sources = [&](int tb, int vb) {
    const int64_t seg[1] = {(int64_t)vb * kFwdVocab};
    return Loop::template make_src<kFwdVocab>(C, a.V, seg, E, a.N, (int64_t)tb * kFwdTokens, pitch, pitch, xcd);
  };
  // targets of this lane's tokens (clamped reads past N; the epilogue ignores them)
  auto targets = [&](int tb, int64_t (&tg)[TJ]) {
    const int64_t tbase = (int64_t)tb * kFwdTokens + (threadIdx.x >> 7) * (kFwdTokens / kFwdWB) + (threadIdx.x & 31);
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      const int64_t tok = tbase + j * 32;
      tg[j] = a.targets[tok < a.N ? tok : a.N - 1];
    }
  };

  // Zero fill riding along (zero_buf, if any): this workgroup's share [z0, z1) of the
  // 16-byte units, one piece after each tile's epilogue (the next tile's first DMA
  // stage is then in flight) and the rest after its last tile.
  const int r_begin = (int)((int64_t)xcd * sc.rounds / 8);
  const int64_t z0 = (int64_t)blockIdx.x * a.zero_units / gridDim.x;
  const int64_t z1 = ((int64_t)blockIdx.x + 1) * a.zero_units / gridDim.x;
  const int64_t zpiece = ((z1 - z0 + max(1, r_end - r_begin) - 1) / max(1, r_end - r_begin) + Loop::NTHREADS - 1) /
                         Loop::NTHREADS * Loop::NTHREADS;
  int64_t zc = z0;
  auto zero_upto = [&](int64_t lim) {
    u32x4* zb = reinterpret_cast<u32x4*>(a.zero_buf);
    for (int64_t u = zc + threadIdx.x; u < lim; u += Loop::NTHREADS) zb[u] = u32x4{0u, 0u, 0u, 0u};
    zc = lim;
  };

  int tb = 0, vb = 0;
  int r = next_round(r_begin, tb, vb);
  if (r >= r_end) {
    zero_upto(z1);
    return;
  }
  if constexpr (BIAS == kBiasLds) fwd_stage_bias<T>(a, vb, bias_lds);
  auto src = sources(tb, vb);
  Loop::template prefetch<RAGGED>(src, smem);
  int64_t tg[TJ];
  targets(tb, tg);

  FwdPending<TJ> pend;
  pend.flags = 0;
  int ptb = 0, pvb = 0;  // the tile whose stores are pending
  for (;;) {
    f32x16 acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int j = 0; j < TJ; ++j) acc[i][j] = zero16();
    // kBiasLds: the accumulators start from the tile's bias (in LDS after the first stage barrier)
    if constexpr (S32) {
      Loop::template consume<RAGGED>(src, smem, acc, [&]() {
        if constexpr (BIAS == kBiasLds) fwd_init_bias_lds<T>(bias_lds, acc);
      });
    } else {
      Loop::template consume<RAGGED>(src, smem, acc, [&]() {
        if constexpr (BIAS == kBiasLds) fwd_init_bias_lds<T>(bias_lds, acc);
        fwd_store_pending(a, pend, ptb, pvb);
      });
    }

    // Start the next tile's pipeline fill and target reads, then reduce this
    // tile from registers while they are in flight.
    int tbn = tb, vbn = vb;
    const int rn = next_round(r + 1, tbn, vbn);
    int64_t tgn[TJ];
    if constexpr (BIAS == kBiasGlobal) fwd_add_bias<T>(a, acc, vb);
    if (rn < r_end) {
      if constexpr (BIAS == kBiasLds) fwd_stage_bias<T>(a, vbn, bias_lds);
      src = sources(tbn, vbn);
      Loop::template prefetch<RAGGED>(src, smem);
      targets(tbn, tgn);
    }
    if constexpr (S32) {
      fwd_epilogue<T, S32>(a, sc.nvt, acc, tb, vb, tg);
    } else {
      fwd_epilogue<T, S32>(a, sc.nvt, acc, tb, vb, tg, &pend);
      ptb = tb;
      pvb = vb;
      if (rn >= r_end) fwd_store_pending(a, pend, ptb, pvb);  // no next tile to carry them
    }
    zero_upto(min(zc + zpiece, z1));
    if (rn >= r_end) break;
    r = rn;
    tb = tbn;
    vb = vbn;
#pragma unroll
    for (int j = 0; j < TJ; ++j) tg[j] = tgn[j];
  }
  zero_upto(z1);
}

__device__ __forceinline__ void lse_merge(float& M, float& S, float m, float s) {
  if (s == 0.f) return;  // tile entirely past V (max = -inf); NaN still propagates
  if (m > M) {
    S = S * __expf(M - m) + s;
    M = m;
  } else {
    S += s * __expf(m - M);
  }
}

// lse[tok] = l and the masked per-token loss (mlx_cce/__init__.py:59-70).
__device__ __forceinline__ void nll_of(const FwdArgs& a, int64_t tok, float l) {
  a.lse[tok] = l;
  const int64_t tg = a.targets[tok];
  float out;
  if (a.has_ignore && tg == a.ignore_index) {
    out = 0.f;
  } else if (tg < 0 || tg >= a.V) {
    out = __builtin_nanf("");
  } else {
    out = l + a.neg_target_logit[tok];
  }
  a.nll[tok] = out;
}

// 64 tokens per workgroup (one per lane, coalesced 256-byte rows); the 16 waves
// split the vocabulary tiles 16 ways and each lane keeps 8 loads in flight.
constexpr int kLseSplits = 16;
__global__ __launch_bounds__(64 * kLseSplits) void lse_kernel(FwdArgs a, int nvt) {
  __shared__ float sm[kLseSplits][64];
  __shared__ float ss[kLseSplits][64];
  const int lane = threadIdx.x & 63;
  const int split = threadIdx.x >> 6;
  const int64_t tok = (int64_t)blockIdx.x * 64 + lane;
  float M = -INFINITY, S = 0.f;
  if (tok < a.N) {
    const float* tm = a.tile_max + tok;
    const float* ts = a.tile_sum_exp + tok;
    int t = split;
    for (; t + 7 * kLseSplits < nvt; t += 8 * kLseSplits) {
      float m[8], x[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        m[u] = tm[(size_t)(t + u * kLseSplits) * a.N];
        x[u] = ts[(size_t)(t + u * kLseSplits) * a.N];
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) lse_merge(M, S, m[u], x[u]);
    }
    for (; t < nvt; t += kLseSplits) lse_merge(M, S, tm[(size_t)t * a.N], ts[(size_t)t * a.N]);
  }
  sm[split][lane] = M;
  ss[split][lane] = S;
  __syncthreads();
  if (split == 0 && tok < a.N) {
#pragma unroll
    for (int k = 1; k < kLseSplits; ++k) lse_merge(M, S, sm[k][lane], ss[k][lane]);
    nll_of(a, tok, M + __logf(S));
  }
}

// lse / nll from statistics in the reference's layout ([N][nt], a token's tiles
// contiguous): one wave per token, each lane merging a strided share of the row
// (coalesced), then the lanes' pairs in a fixed butterfly; lane 0's result is kept.
// Reference: reduce_tile_to_lse, csrc/cce/cce.metal:332-355.
__global__ __launch_bounds__(256) void lse_rows_kernel(FwdArgs a, int64_t nt) {
  const int lane = threadIdx.x & 63;
  const int64_t tok = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (tok >= a.N) return;  // uniform per wave
  const float* tm = a.tile_max + tok * nt;
  const float* ts = a.tile_sum_exp + tok * nt;
  float M = -INFINITY, S = 0.f;
  for (int64_t t = lane; t < nt; t += 64) lse_merge(M, S, tm[t], ts[t]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float m2 = __shfl_xor(M, off), s2 = __shfl_xor(S, off);
    lse_merge(M, S, m2, s2);
  }
  if (lane == 0) nll_of(a, tok, M + __logf(S));
}

template <typename T>
static void launch_tile_variant(const FwdArgs& a, const FwdSched& sc, int bias, bool ragged, dim3 grid, dim3 block,
                                hipStream_t s) {
#define CCE_T(B, R, S)                                                                   \
  if (bias == B && ragged == R && (a.stats32 != 0) == S) {                               \
    hipLaunchKernelGGL((fwd_tile_kernel<T, B, R, S>), grid, block, 0, s, a, sc);         \
    return;                                                                              \
  }
#define CCE_T2(B)         \
  CCE_T(B, false, false)  \
  CCE_T(B, true, false)   \
  CCE_T(B, false, true)   \
  CCE_T(B, true, true)
  CCE_T2(kBiasNone)
  CCE_T2(kBiasGlobal)
  CCE_T2(kBiasLds)
#undef CCE_T2
#undef CCE_T
}

// The tile kernel over vocabulary blocks [vb0, vb0 + nvb): a.c must address the
// rows of those blocks at their global row numbers.
template <typename T>
static hipError_t launch_tiles(const FwdArgs& a, int vb0, int nvb, hipStream_t s) {
  FwdSched sc{};
  sc.ntb = (int)((a.N + kFwdTokens - 1) / kFwdTokens);
  sc.nvb = nvb;
  sc.vb0 = vb0;
  sc.nvt = (int)((a.V + kStatTile - 1) / kStatTile);
  // members per XCD; a round is gt token blocks x gv vocabulary blocks
  const int cpx = a.num_cus / 8 > 0 ? a.num_cus / 8 : 1;
  sc.gt = (sc.ntb >= 4 && cpx % 4 == 0) ? 4 : (sc.ntb >= 2 && cpx % 2 == 0) ? 2 : 1;
  sc.gv = cpx / sc.gt;
  sc.ngv = (sc.nvb + sc.gv - 1) / sc.gv;
  const int64_t ngt = (sc.ntb + sc.gt - 1) / sc.gt;
  const int64_t rounds = ngt * sc.ngv;
  if (rounds > INT32_MAX / 8) return hipErrorInvalidValue;
  sc.rounds = (int)rounds;
  const dim3 grid(8 * cpx), block(FwdLoop<T>::NTHREADS);
  const bool ragged = (a.D * (int64_t)sizeof(T)) % kSliceBytes != 0;
  const int bias = a.bias == nullptr ? kBiasNone
                   : ((reinterpret_cast<uintptr_t>(a.bias) & 15) == 0 && (a.V * (int64_t)sizeof(T)) % 16 == 0)
                       ? kBiasLds
                       : kBiasGlobal;
  launch_tile_variant<T>(a, sc, bias, ragged, grid, block, s);
  return hipGetLastError();
}

template <typename T>
static hipError_t launch_lse(const FwdArgs& a, hipStream_t s) {
  if (a.stats32) {
    hipLaunchKernelGGL(lse_rows_kernel, dim3((unsigned)((a.N + 3) / 4)), dim3(256), 0, s, a,
                       (a.V + kRefStatTile - 1) / kRefStatTile);
    return hipGetLastError();
  }
  const int nvt = (int)((a.V + kStatTile - 1) / kStatTile);
  hipLaunchKernelGGL(lse_kernel, dim3((unsigned)((a.N + 63) / 64)), dim3(64 * kLseSplits), 0, s, a, nvt);
  return hipGetLastError();
}

template <typename T>
static hipError_t forward_typed(const FwdArgs& a, hipStream_t s) {
  hipError_t err = launch_tiles<T>(a, 0, (int)((a.V + kFwdVocab - 1) / kFwdVocab), s);
  if (err != hipSuccess) return err;
  return launch_lse<T>(a, s);
}

// Quantized classifier rows: per chunk of q.chunk_rows rows (whole vocabulary
// blocks), dequantize into q.scratch, then run the tile kernel on the chunk's blocks
// with c addressing the scratch at global row numbers; one lse merge at the end.
template <typename T>
static hipError_t forward_q_typed(int dtype, const FwdArgs& a, const QuantRows& q, hipStream_t s) {
  static_assert(kQuantChunkAlign % kFwdVocab == 0, "chunks hold whole vocabulary blocks");
  const int64_t row_bytes = a.D * (int64_t)sizeof(T);
  for (int64_t v0 = 0; v0 < a.V; v0 += q.chunk_rows) {
    const int64_t rows = a.V - v0 < q.chunk_rows ? a.V - v0 : q.chunk_rows;
    hipError_t err = launch_dequantize(dtype, q, v0, rows, a.D, q.scratch, s);
    if (err != hipSuccess) return err;
    FwdArgs ac = a;
    ac.c = reinterpret_cast<const char*>(q.scratch) - v0 * row_bytes;
    err = launch_tiles<T>(ac, (int)(v0 / kFwdVocab), (int)((rows + kFwdVocab - 1) / kFwdVocab), s);
    if (err != hipSuccess) return err;
  }
  return launch_lse<T>(a, s);
}

// Reduced loss of cce_loss (mlx_cce/__init__.py:72-76): one workgroup sums nll in a
// fixed order (fp64 per thread, then a tree over the threads) and counts the rows
// the ignore mask keeps.  mode 1: loss = sum; mode 2: loss = sum / max(count, 1),
// scale = max(count, 1).  Masked rows already hold nll = 0.
constexpr int kReduceThreads = 1024;
__global__ __launch_bounds__(kReduceThreads) void reduce_loss_kernel(const float* __restrict__ nll,
                                                                     const int64_t* __restrict__ targets,
                                                                     int64_t ignore_index, int has_ignore, int64_t N,
                                                                     int mode, float* loss, float* scale) {
  __shared__ double ssum[kReduceThreads];
  __shared__ long long scnt[kReduceThreads];
  double acc = 0.0;
  long long cnt = 0;
  for (int64_t i = threadIdx.x; i < N; i += kReduceThreads) {
    acc += (double)nll[i];
    cnt += (has_ignore && targets[i] == ignore_index) ? 0 : 1;
  }
  ssum[threadIdx.x] = acc;
  scnt[threadIdx.x] = cnt;
  __syncthreads();
  for (int w = kReduceThreads / 2; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) {
      ssum[threadIdx.x] += ssum[threadIdx.x + w];
      scnt[threadIdx.x] += scnt[threadIdx.x + w];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const double c = scnt[0] > 0 ? (double)scnt[0] : 1.0;
    loss[0] = mode == 2 ? (float)(ssum[0] / c) : (float)ssum[0];
    if (scale) scale[0] = (float)c;
  }
}

hipError_t launch_reduce_loss(const float* nll, const int64_t* targets, int64_t ignore_index, int has_ignore,
                              int64_t N, int mode, float* loss, float* scale, hipStream_t s) {
  hipLaunchKernelGGL(reduce_loss_kernel, dim3(1), dim3(kReduceThreads), 0, s, nll, targets, ignore_index,
                     has_ignore, N, mode, loss, scale);
  return hipGetLastError();
}

// d_nll[r] = grad[0] / scale[0] (scale null: grad[0]) — the cotangent of every
// per-token loss under a summed or averaged reduction.
__global__ __launch_bounds__(256) void broadcast_grad_kernel(const float* __restrict__ grad,
                                                             const float* __restrict__ scale, int64_t N,
                                                             float* __restrict__ d_nll) {
  const float g = scale ? grad[0] / scale[0] : grad[0];
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < N; i += (int64_t)gridDim.x * 256) d_nll[i] = g;
}

hipError_t launch_broadcast_grad(const float* grad, const float* scale, int64_t N, float* d_nll, hipStream_t s) {
  const int64_t blocks = (N + 255) / 256;
  hipLaunchKernelGGL(broadcast_grad_kernel, dim3((unsigned)(blocks < 1024 ? blocks : 1024)), dim3(256), 0, s, grad,
                     scale, N, d_nll);
  return hipGetLastError();
}

hipError_t launch_forward(int dtype, const FwdArgs& a, hipStream_t s) {
  switch (dtype) {
    case 0:
      return forward_typed<float>(a, s);
    case 1:
      return forward_typed<_Float16>(a, s);
    default:
      return forward_typed<__bf16>(a, s);
  }
}

hipError_t launch_forward_q(int dtype, const FwdArgs& a, const QuantRows& q, hipStream_t s) {
  switch (dtype) {
    case 0:
      return forward_q_typed<float>(dtype, a, q, s);
    case 1:
      return forward_q_typed<_Float16>(dtype, a, q, s);
    default:
      return forward_q_typed<__bf16>(dtype, a, q, s);
  }
}

}  // namespace cce
