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

template <typename T, bool HAS_BIAS>
__global__ __launch_bounds__(FwdLoop<T>::NTHREADS, 1) void fwd_tile_kernel(FwdArgs a, int n_tok_blocks,
                                                                           int n_voc_blocks, int grid_padded,
                                                                           int nvt) {
  using Loop = FwdLoop<T>;
  constexpr int TI = Loop::TI, TJ = Loop::TJ;
  __shared__ __attribute__((aligned(16))) char smem[Loop::SMEM_BYTES];

  // Tile order: workgroups are dealt round-robin to the 8 XCDs, so first make
  // each XCD walk a contiguous range of logical tiles, then walk that range in
  // groups of 4 token blocks so the 32 workgroups an XCD runs at once share
  // 4 E blocks and 8 C blocks in its L2.
  const int b = blockIdx.x;
  const int pid = (b & 7) * (grid_padded >> 3) + (b >> 3);
  const int total = n_tok_blocks * n_voc_blocks;
  if (pid >= total) return;
  constexpr int GROUP = 4;
  const int per_group = GROUP * n_voc_blocks;
  const int grp = pid / per_group;
  const int first = grp * GROUP;
  const int gsize = min(n_tok_blocks - first, GROUP);
  const int local = pid - grp * per_group;
  const int tb = first + local % gsize;
  const int vb = local / gsize;

  f32x16 acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j) acc[i][j] = zero16();

  const int64_t pitch = a.D * (int64_t)sizeof(T);
  Loop::run(reinterpret_cast<const char*>(a.c), a.V, (int64_t)vb * kFwdVocab, reinterpret_cast<const char*>(a.e),
            a.N, (int64_t)tb * kFwdTokens, pitch, pitch, smem, acc, b & 7);

  // ---------------------------------------------------------------- epilogue
  // acc[i][j][r] holds logit(vocab = vbase + 32i + 8(r/4) + 4h + r%4,
  //                           token = tbase + 32j + n)   with n = lane%32, h = lane/32.
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wv = wave & 1;   // vocab half (NTMainLoop: wa = wave % 2)
  const int wt = wave >> 1;  // token part of kFwdTokens / kFwdWB rows
  const int n = lane & 31;
  const int h = lane >> 5;
  const int64_t vbase = (int64_t)vb * kFwdVocab + wv * 128;
  const int64_t tbase = (int64_t)tb * kFwdTokens + wt * (kFwdTokens / kFwdWB);
  const T* bias = reinterpret_cast<const T*>(a.bias);

#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t v = vbase + i * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
      const bool ok = v < a.V;
      float add = 0.f;
      if (HAS_BIAS) add = ok ? to_f32(bias[v]) : 0.f;
#pragma unroll
      for (int j = 0; j < TJ; ++j) acc[i][j][r] = ok ? acc[i][j][r] + add : -INFINITY;
    }
  }

  const int tile = (int)(vbase / kStatTile);
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    const int64_t tok = tbase + j * 32 + n;

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

    if (h == 0 && tok < a.N && tile < nvt) {
      a.tile_max[(size_t)tile * a.N + tok] = m;
      a.tile_sum_exp[(size_t)tile * a.N + tok] = s;
    }

    // Target gather: the lane holding (target, token) writes -(logit + bias).
    const int64_t tg = tok < a.N ? a.targets[tok] : -1;
    const int64_t loc = tg - vbase;
    const bool hit = loc >= 0 && loc < 128 && tg < a.V;
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
      if (hit && h == ht) a.neg_target_logit[tok] = -val;
    }
  }
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
    const float l = M + __logf(S);
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
}

template <typename T>
static hipError_t forward_typed(const FwdArgs& a, hipStream_t s) {
  const int ntb = (int)((a.N + kFwdTokens - 1) / kFwdTokens);
  const int nvb = (int)((a.V + kFwdVocab - 1) / kFwdVocab);
  const int nvt = (int)((a.V + kStatTile - 1) / kStatTile);
  const int total = ntb * nvb;
  const int grid = (total + 7) / 8 * 8;
  if (a.bias) {
    hipLaunchKernelGGL((fwd_tile_kernel<T, true>), dim3(grid), dim3(FwdLoop<T>::NTHREADS), 0, s, a, ntb, nvb, grid, nvt);
  } else {
    hipLaunchKernelGGL((fwd_tile_kernel<T, false>), dim3(grid), dim3(FwdLoop<T>::NTHREADS), 0, s, a, ntb, nvb, grid, nvt);
  }
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(lse_kernel, dim3((unsigned)((a.N + 63) / 64)), dim3(64 * kLseSplits), 0, s, a, nvt);
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

}  // namespace cce
