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
// On MI355X fp32 global atomics retire at ~2.9e11 per second (one per memory
// channel per clock) — 2.5e9 of them (the per-tile partial flushes at the
// Llama-3.1-8B head) cost ~8 ms — so this backward gives every output element
// exactly one writer instead, and never materialises a [N, tiles, D] scratch:
//
//   1. bwd_filter_kernel     one wave per (vocab tile, token block): keep the
//                            128 x 128 tile iff a row with d_nll != 0 has its
//                            target in it or tile_max - lse >= filter_log_eps.
//   2. bwd_compact_vt_kernel kept pairs -> slots in vocab-major order; chunk plan.
//   3. bwd_compact_rb_kernel the same slots ordered by token block.
//   per chunk of at most `cap` slots (chunk boundaries between vocab tiles):
//   4. bwd_g_kernel          recompute the logit tile on MFMA, form G, store it in
//                            the chunk's scratch (bf16/fp16/fp32, token-major and
//                            vocab-major) plus its fp32 column sums.
//   5. bwd_sum_kernel<0>     dE: owner = (token block, 256-byte D slice);
//                            dE = sum over the block's kept tiles of G_j . C_j.
//   6. bwd_sum_kernel<1>     dC: owner = (vocab tile, D slice);
//                            dC = sum over the tile's kept blocks of G_j^T . E_j,
//                            dBias from the column sums; written in the output dtype.
//   Both are persistent workgroups walking (owner, tile) steps as one pipeline.
//   With more than one chunk, dE is carried between chunks in an fp32 buffer by
//   the owner itself (store / add / finish), still without atomics.
#include "cce_device.h"
#include "cce_launch.h"

namespace cce {

static_assert(kStatTile == kBwdVocab, "filter statistics are kept per backward vocabulary tile");
static_assert(kBwdTokens == 128 && kBwdVocab == 128, "the G-tile kernels assume 128 x 128 tiles");

// ---------------------------------------------------------------- 1. filter
__global__ __launch_bounds__(256) void bwd_filter_kernel(BwdArgs a) {
  const int nvt = (int)a.plan.nvt, nrb = (int)a.plan.nrb;
  const int lane = threadIdx.x & 63;
  const int pair = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (pair >= nvt * nrb) return;  // uniform per wave
  const int vt = pair / nrb;
  const int rb = pair - vt * nrb;
  const int64_t v0 = (int64_t)vt * kBwdVocab;
  bool keep = false;
#pragma unroll
  for (int k = 0; k < kBwdTokens / 64; ++k) {
    const int64_t r = (int64_t)rb * kBwdTokens + k * 64 + lane;
    if (r < a.N) {
      const float g = a.d_nll[r];
      const int64_t t = a.targets[r];
      const bool active = g != 0.f && !(a.has_ignore && t == a.ignore_index);
      if (active) {
        const bool tin = t >= v0 && t < v0 + kBwdVocab;
        const float tm = a.tile_max[(size_t)vt * a.N + r];
        keep = keep || tin || (tm - a.lse[r] >= a.filter_log_eps);
      }
    }
  }
  const bool any = __any(keep);
  if (lane == 0) a.flags[pair] = any ? 1 : 0;
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

// ---------------------------------------------------------------- 2. compaction, vocab-major
// One workgroup of 16 waves.  Pair indices (vt * nrb + rb) are taken in rounds of
// 65536; thread t of a round owns the 64 consecutive pairs [64 t, 64 t + 64),
// loaded as four 16-byte vectors.  Writes list / slot_map / vt_start, the tile
// statistics, and the chunk plan: vocab tile vt belongs to chunk
// vt_start[vt] / step, step = cap - nrb + 1.
__global__ __launch_bounds__(1024) void bwd_compact_vt_kernel(BwdArgs a) {
  __shared__ int wsum[16];
  const int total = (int)a.plan.total, nrb = (int)a.plan.nrb, nvt = (int)a.plan.nvt;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int carry = 0;
  for (int base = 0; base < total; base += 65536) {
    const int i0 = base + tid * 64;
    uint32_t f[16];
    if (i0 + 64 <= total) {
      const u32x4* src = reinterpret_cast<const u32x4*>(a.flags + i0);  // i0 % 64 == 0: 16-byte aligned
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const u32x4 v = src[q];
        f[4 * q] = v.x;
        f[4 * q + 1] = v.y;
        f[4 * q + 2] = v.z;
        f[4 * q + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int w = 0; w < 16; ++w) {
        uint32_t x = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const int i = i0 + 4 * w + b;
          if (i < total) x |= (uint32_t)a.flags[i] << (8 * b);
        }
        f[w] = x;
      }
    }
    int cnt = 0;
#pragma unroll
    for (int w = 0; w < 16; ++w) cnt += __builtin_popcount(f[w]);  // flags are 0 / 1 bytes
    const int incl = wave_incl_scan(cnt);
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    int wbase = 0, round_total = 0;
#pragma unroll
    for (int w = 0; w < 16; ++w) {
      const int x = wsum[w];
      wbase += w < wave ? x : 0;
      round_total += x;
    }
    int pos = carry + wbase + incl - cnt;
    if (i0 < total) {
      int vt = i0 / nrb;
      int rb = i0 - vt * nrb;
      int sm[64];
#pragma unroll
      for (int k = 0; k < 64; ++k) {
        const bool in = i0 + k < total;
        const bool kept = in && ((f[k >> 2] >> (8 * (k & 3))) & 1u);
        if (in && rb == 0) a.vt_start[vt] = pos;
        sm[k] = kept ? pos : -1;
        if (kept) a.list[pos++] = i0 + k;
        if (++rb == nrb) {
          rb = 0;
          ++vt;
        }
      }
      if (i0 + 64 <= total) {
        int* dst = a.slot_map + i0;
#pragma unroll
        for (int q = 0; q < 16; ++q)
          *reinterpret_cast<u32x4*>(dst + 4 * q) =
              u32x4{(uint32_t)sm[4 * q], (uint32_t)sm[4 * q + 1], (uint32_t)sm[4 * q + 2], (uint32_t)sm[4 * q + 3]};
      } else {
#pragma unroll
        for (int k = 0; k < 64; ++k)
          if (i0 + k < total) a.slot_map[i0 + k] = sm[k];
      }
    }
    carry += round_total;
    __syncthreads();  // wsum is rewritten by the next round
  }
  const int kept = carry;
  if (tid == 0) {
    a.vt_start[nvt] = kept;
    if (a.tile_stats) {
      a.tile_stats[0] = kept;
      a.tile_stats[1] = total;
    }
  }
  __threadfence_block();
  __syncthreads();
  const int step = (int)(a.plan.cap - a.plan.nrb + 1);
  const int maxc = (int)a.plan.max_chunks;
  for (int vt = tid; vt <= nvt; vt += 1024) {
    // chunk c starts at the first vocab tile whose first slot reaches c * step
    const int c = vt < nvt ? min(a.vt_start[vt] / step, maxc - 1) : maxc;
    const int prev = vt == 0 ? -1 : min(a.vt_start[vt - 1] / step, maxc - 1);
    const int first_slot = vt < nvt ? a.vt_start[vt] : kept;
    for (int cc = prev + 1; cc <= c; ++cc) {
      a.chunk_vt[cc] = vt;
      a.chunk_slot[cc] = first_slot;
    }
  }
}

// ---------------------------------------------------------------- 3. compaction, block-major
// One workgroup of 16 waves.  Token blocks are taken 64 at a time, one per lane;
// wave w walks the vocab tiles [w R, w R + R), R = ceil(nvt / 16), in order, so
// each load reads 64 consecutive flags of one vocab tile.  A first pass counts
// per (wave, block), a second writes rb_list / rb_vt in (block, vocab tile) order.
__global__ __launch_bounds__(1024) void bwd_compact_rb_kernel(BwdArgs a) {
  __shared__ int cnt_s[16][64];
  __shared__ int colbase[65];
  const int nrb = (int)a.plan.nrb, nvt = (int)a.plan.nvt;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int R = (nvt + 15) / 16;
  const int vt_lo = min(wave * R, nvt), vt_hi = min(vt_lo + R, nvt);
  int carry = 0;
  for (int rb0 = 0; rb0 < nrb; rb0 += 64) {
    const int rb = rb0 + lane;
    const bool ok = rb < nrb;
    int c = 0;
    if (ok) {
#pragma unroll 8
      for (int vt = vt_lo; vt < vt_hi; ++vt) c += a.flags[(size_t)vt * nrb + rb];
    }
    cnt_s[wave][lane] = c;
    __syncthreads();
    if (wave == 0) {
      int tot = 0;
#pragma unroll
      for (int w = 0; w < 16; ++w) tot += cnt_s[w][lane];
      const int incl = wave_incl_scan(tot);
      const int st = carry + incl - tot;
      if (ok) a.rb_start[rb] = st;
      colbase[lane] = st;
      if (lane == 63) colbase[64] = carry + incl;
    }
    __syncthreads();
    if (ok) {
      int pos = colbase[lane];
      for (int w = 0; w < wave; ++w) pos += cnt_s[w][lane];
      for (int vt = vt_lo; vt < vt_hi; ++vt) {
        const size_t pr = (size_t)vt * nrb + rb;
        if (a.flags[pr]) {
          a.rb_list[pos] = a.slot_map[pr];
          a.rb_vt[pos] = vt;
          ++pos;
        }
      }
    }
    carry = colbase[64];
    __syncthreads();  // cnt_s / colbase are rewritten by the next group
  }
  if (tid == 0) a.rb_start[nrb] = carry;
}

// ---------------------------------------------------------------- LDS tiles of G
// A G tile in LDS: 128 rows x 128 elements, row-major, 16-byte chunks swizzled by swz().
template <typename T>
struct GTile {
  static constexpr uint32_t ROW_BYTES = 128 * sizeof(T);
  static constexpr uint32_t BYTES = 128 * ROW_BYTES;
  static constexpr int CPR = ROW_BYTES / 16;           // chunks per row
  static constexpr int PER_THREAD = 128 * CPR / kThreads;  // 16-byte chunks per thread
};

// G (fp32 registers, pass-1 accumulator layout) -> LDS as [token][vocab].
// acc[i][j][r]: vocab 64 wv + 32 i + 8 (r/4) + 4 h + r%4, token 64 wt + 32 j + n.
template <typename T>
__device__ __forceinline__ void store_g_token_major(char* gsm, const f32x16 (&w)[2][2], int wv, int wt, int n,
                                                    int h) {
  constexpr uint32_t ROW_BYTES = GTile<T>::ROW_BYTES;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int row = wt * 64 + j * 32 + n;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int col = wv * 64 + i * 32 + rq * 8 + h * 4;  // 4 consecutive vocab columns
        if constexpr (sizeof(T) == 4) {
          u32x4 o{__float_as_uint(w[i][j][rq * 4 + 0]), __float_as_uint(w[i][j][rq * 4 + 1]),
                  __float_as_uint(w[i][j][rq * 4 + 2]), __float_as_uint(w[i][j][rq * 4 + 3])};
          lds_st16(gsm, swz(row, col >> 2, ROW_BYTES), o);
        } else {
          T v0 = (T)w[i][j][rq * 4 + 0], v1 = (T)w[i][j][rq * 4 + 1];
          T v2 = (T)w[i][j][rq * 4 + 2], v3 = (T)w[i][j][rq * 4 + 3];
          const uint32_t p0 = (uint32_t)__builtin_bit_cast(uint16_t, v0) |
                              ((uint32_t)__builtin_bit_cast(uint16_t, v1) << 16);
          const uint32_t p1 = (uint32_t)__builtin_bit_cast(uint16_t, v2) |
                              ((uint32_t)__builtin_bit_cast(uint16_t, v3) << 16);
          *reinterpret_cast<u32x2*>(gsm + swz(row, col >> 3, ROW_BYTES) + (col & 7) * 2) = u32x2{p0, p1};
        }
      }
    }
  }
}

// G -> LDS as [vocab][token].
template <typename T>
__device__ __forceinline__ void store_g_vocab_major(char* gsm, const f32x16 (&w)[2][2], int wv, int wt, int n,
                                                    int h) {
  constexpr uint32_t ROW_BYTES = GTile<T>::ROW_BYTES;
  constexpr int EPC = 16 / sizeof(T);
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int col = wt * 64 + j * 32 + n;  // token
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = wv * 64 + i * 32 + (r >> 2) * 8 + h * 4 + (r & 3);  // vocab
        *reinterpret_cast<T*>(gsm + swz(row, col / EPC, ROW_BYTES) + (col % EPC) * sizeof(T)) = (T)w[i][j][r];
      }
    }
  }
}

// Swizzled LDS tile <-> plain row-major tile in global memory (coalesced 16-byte accesses).
template <typename T>
__device__ __forceinline__ void copy_lds_to_global(const char* gsm, char* dst) {
#pragma unroll
  for (int k = 0; k < GTile<T>::PER_THREAD; ++k) {
    const int i = threadIdx.x + kThreads * k;
    const int row = i / GTile<T>::CPR, ch = i % GTile<T>::CPR;
    *reinterpret_cast<u32x4*>(dst + (size_t)i * 16) = lds_ld16(gsm, swz(row, ch, GTile<T>::ROW_BYTES));
  }
}

// ---------------------------------------------------------------- 4. G tiles
template <typename T, bool HAS_BIAS, bool WANT_TOK, bool WANT_VOC, bool WANT_DB>
__global__ __launch_bounds__(kThreads, 1) void bwd_g_kernel(BwdArgs a, int chunk) {
  using Loop = NTMainLoop<T, kBwdVocab, kBwdTokens, 2, 2>;  // A = C rows (vocab), B = E rows (tokens)
  __shared__ __attribute__((aligned(16))) char smem[Loop::SMEM_BYTES + GTile<T>::BYTES];
  char* gsm = smem + Loop::SMEM_BYTES;

  const int nrb = (int)a.plan.nrb;
  const int lo = a.chunk_slot[chunk], hi = a.chunk_slot[chunk + 1];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wv = wave & 1;
  const int wt = wave >> 1;
  const int n = lane & 31;
  const int h = lane >> 5;
  const int64_t pitch = a.D * (int64_t)sizeof(T);
  const T* bias = reinterpret_cast<const T*>(a.bias);
  const char* E = reinterpret_cast<const char*>(a.e);
  const char* C = reinterpret_cast<const char*>(a.c);

  for (int slot = lo + (int)blockIdx.x; slot < hi; slot += (int)gridDim.x) {
    const int pair = a.list[slot];
    const int vt = pair / nrb;
    const int rb = pair - vt * nrb;
    const int64_t v0 = (int64_t)vt * kBwdVocab;
    const int64_t t0 = (int64_t)rb * kBwdTokens;

    f32x16 w[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) w[i][j] = zero16();
    Loop::run(C, a.V, v0, E, a.N, t0, pitch, pitch, smem, w);

    // G = g (softmax - onehot), zero outside [0,N) x [0,V) and for rows with g == 0.
    float g[2], lz[2];
    int64_t tg[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t tok = t0 + wt * 64 + j * 32 + n;
      g[j] = 0.f;
      lz[j] = 0.f;
      tg[j] = -1;
      if (tok < a.N) {
        tg[j] = a.targets[tok];
        g[j] = (a.has_ignore && tg[j] == a.ignore_index) ? 0.f : a.d_nll[tok];
        lz[j] = a.lse[tok] * kLog2e;
      }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t v = v0 + wv * 64 + i * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
        const bool vok = v < a.V;
        float add = 0.f;
        if (HAS_BIAS) add = vok ? to_f32(bias[v]) : 0.f;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const float p = __builtin_amdgcn_exp2f(fmaf(w[i][j][r] + add, kLog2e, -lz[j]));
          const float val = g[j] * (p - (v == tg[j] ? 1.f : 0.f));
          w[i][j][r] = (vok && g[j] != 0.f) ? val : 0.f;
        }
      }
    }
    const size_t s_local = (size_t)(slot - lo);

    if constexpr (WANT_DB) {
      // column sums over this wave's 64 tokens; lanes n == 0 of each half hold them
      float* cs = a.colsum + s_local * 2 * kBwdVocab + wt * kBwdVocab;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float s = w[i][0][r] + w[i][1][r];
          s += __shfl_xor(s, 1);
          s += __shfl_xor(s, 2);
          s += __shfl_xor(s, 4);
          s += __shfl_xor(s, 8);
          s += __shfl_xor(s, 16);
          if (n == 0) cs[wv * 64 + i * 32 + (r >> 2) * 8 + h * 4 + (r & 3)] = s;
        }
      }
    }
    if constexpr (WANT_TOK) {
      store_g_token_major<T>(gsm, w, wv, wt, n, h);
      __syncthreads();
      copy_lds_to_global<T>(gsm, a.w_tok + s_local * a.plan.w_bytes);
      __syncthreads();
    }
    if constexpr (WANT_VOC) {
      store_g_vocab_major<T>(gsm, w, wv, wt, n, h);
      __syncthreads();
      copy_lds_to_global<T>(gsm, a.w_voc + s_local * a.plan.w_bytes);
      __syncthreads();
    }
  }
}

// ---------------------------------------------------------------- 5/6. sums of G_j . X_j
// acc[128 x DK] += G_j[128 x 128] . X_j[128 x DK] over a list of tiles j, where
// G_j is a stored G tile (rows = output rows, columns = contraction) and X_j is
// a 128-row block of E or C restricted to one 256-byte slice of D.  X_j is
// transposed into LDS ([d][k], k contiguous) on the way in so both MFMA operands
// are k-contiguous 16-byte fragments.
template <typename T>
struct GSum {
  static constexpr int EPC = 16 / sizeof(T);               // elements per 16-byte fragment
  static constexpr int DK = 256 / sizeof(T);               // D elements per slice
  static constexpr uint32_t XROW_BYTES = 128 * sizeof(T);  // transposed slice row (128 k)
  static constexpr uint32_t X_BYTES = DK * XROW_BYTES;     // 32 KiB for every dtype
  static constexpr uint32_t G_BYTES = GTile<T>::BYTES;
  static constexpr uint32_t BUF_BYTES = G_BYTES + X_BYTES;
  static constexpr int NBUF = (2 * BUF_BYTES <= 160 * 1024) ? 2 : 1;
  static constexpr int NB = (128 / EPC) * 16 / kThreads;  // EPC x EPC transpose blocks per thread
  static constexpr int GP = GTile<T>::PER_THREAD;          // G-tile chunks per thread
  static constexpr int TJ = DK / 2 / 32;                   // 32-col MFMA tiles per wave along D
  static constexpr int KS = (int)(XROW_BYTES / 32);        // 32-byte K steps over 128 elements
  static_assert(NB >= 1 && NB * kThreads == (128 / EPC) * 16, "transpose blocks must split evenly");

  struct Regs {
    u32x4 x[NB][EPC];
    u32x4 g[GP];
  };

  static __device__ __forceinline__ void load(Regs& R, const char* gtile, const char* src, int64_t src_rows,
                                              int64_t src_row0, int64_t pitch, int64_t kbytes, int ds) {
#pragma unroll
    for (int k = 0; k < GP; ++k) R.g[k] = gld16(gtile + (size_t)(threadIdx.x + kThreads * k) * 16);
#pragma unroll
    for (int s = 0; s < NB; ++s) {
      const int b = threadIdx.x + kThreads * s;
      const int dblk = b & 15;
      const int vblk = b >> 4;
      const int64_t col = (int64_t)ds * 256 + dblk * 16;
      const bool in = col < kbytes;
#pragma unroll
      for (int x = 0; x < EPC; ++x) {
        int64_t g = src_row0 + vblk * EPC + x;
        g = g < src_rows ? g : src_rows - 1;
        R.x[s][x] = in ? gld16(src + g * pitch + col) : u32x4{0u, 0u, 0u, 0u};
      }
    }
  }

  static __device__ __forceinline__ void store(const Regs& R, char* buf) {
    char* gsm = buf;
    char* xsm = buf + G_BYTES;
#pragma unroll
    for (int k = 0; k < GP; ++k) {
      const int i = threadIdx.x + kThreads * k;
      lds_st16(gsm, swz(i / GTile<T>::CPR, i % GTile<T>::CPR, GTile<T>::ROW_BYTES), R.g[k]);
    }
#pragma unroll
    for (int s = 0; s < NB; ++s) {
      const int b = threadIdx.x + kThreads * s;
      const int dblk = b & 15;
      const int vblk = b >> 4;
#pragma unroll
      for (int y = 0; y < EPC; ++y) {
        u32x4 o;
        if constexpr (sizeof(T) == 4) {
          o = u32x4{R.x[s][0][y], R.x[s][1][y], R.x[s][2][y], R.x[s][3][y]};
        } else {
          const int wd = y >> 1;
          const bool hi = y & 1;
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const uint32_t lo_src = R.x[s][2 * k][wd];
            const uint32_t hi_src = R.x[s][2 * k + 1][wd];
            o[k] = hi ? ((lo_src >> 16) | (hi_src & 0xffff0000u)) : ((lo_src & 0xffffu) | (hi_src << 16));
          }
        }
        lds_st16(xsm, swz(dblk * EPC + y, vblk, XROW_BYTES), o);
      }
    }
  }

  static __device__ __forceinline__ void mma(const char* buf, f32x16 (&acc)[2][TJ]) {
    const char* gsm = buf;
    const char* xsm = buf + G_BYTES;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave & 1, wn = wave >> 1;
    const int n = lane & 31, kg = lane >> 5;
    u32x4 af[2][2], bf[2][TJ];  // fragments double-buffered across K steps
    auto frags = [&](int ks, u32x4 (&a2)[2], u32x4 (&b2)[TJ]) {
#pragma unroll
      for (int ti = 0; ti < 2; ++ti)
        a2[ti] = lds_ld16(gsm, swz(wm * 64 + ti * 32 + n, ks * 2 + kg, GTile<T>::ROW_BYTES));
#pragma unroll
      for (int tj = 0; tj < TJ; ++tj) b2[tj] = lds_ld16(xsm, swz(wn * (DK / 2) + tj * 32 + n, ks * 2 + kg, XROW_BYTES));
    };
    frags(0, af[0], bf[0]);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if (ks + 1 < KS) frags(ks + 1, af[(ks + 1) & 1], bf[(ks + 1) & 1]);
      // X slice as the MFMA "A" operand and G as "B": the 32 x 32 result then holds
      // D along registers and output rows along lanes, so each lane owns runs of
      // 4 consecutive D elements of one output row (written as 8 or 16 bytes).
#pragma unroll
      for (int ti = 0; ti < 2; ++ti)
#pragma unroll
        for (int tj = 0; tj < TJ; ++tj) acc[ti][tj] = Traits<T>::mfma(bf[ks & 1][tj], af[ks & 1][ti], acc[ti][tj]);
    }
  }

  // Per-wave output staging tile: 64 output rows x 128 bytes (DK / 2 elements),
  // 16-byte chunks XOR-swizzled by the row so both the 8-byte / 16-byte register
  // writes and the 16-byte row reads are free of bank conflicts.
  static constexpr uint32_t STAGE_BYTES = 64 * 128;
  static __device__ __forceinline__ uint32_t stage_off(uint32_t row, uint32_t chunk) {
    return row * 128u + ((chunk ^ (row & 7u)) << 4);
  }
};

// Output write of one owner tile (128 rows x one D slice).
//   kWriteT: write the output dtype; kStoreF32 / kAddF32: fp32 accumulator;
//   kFinishT: write dtype of (fp32 accumulator + acc); kSkip: nothing.
// acc[ti][tj][r] holds output row (wm 64 + ti 32 + n) and D element
// (wn DK/2 + tj 32 + 8 (r/4) + 4 h + r%4) of the slice.
enum WriteMode { kWriteT = 0, kStoreF32 = 1, kAddF32 = 2, kFinishT = 3, kSkip = 4 };

// kWriteT through the wave's LDS staging tile: registers -> LDS (8 or 16-byte
// writes), then 16-byte row-contiguous global stores.
template <typename T>
__device__ __forceinline__ void write_owner_tile_staged(void* out_t, const f32x16 (&acc)[2][GSum<T>::TJ],
                                                        int64_t row0, int64_t rows, int64_t D, int ds, char* stage) {
  using S = GSum<T>;
  constexpr int TJ = S::TJ, DK = S::DK, EPC = S::EPC;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int n = lane & 31, h = lane >> 5;
#pragma unroll
  for (int ti = 0; ti < 2; ++ti) {
    const uint32_t rr = (uint32_t)(ti * 32 + n);
#pragma unroll
    for (int tj = 0; tj < TJ; ++tj) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int e0 = tj * 32 + q * 8 + h * 4;  // first of 4 consecutive elements
        const uint32_t byte = (uint32_t)e0 * sizeof(T);
        if constexpr (sizeof(T) == 4) {
          lds_st16(stage, S::stage_off(rr, byte >> 4),
                   u32x4{__float_as_uint(acc[ti][tj][q * 4]), __float_as_uint(acc[ti][tj][q * 4 + 1]),
                         __float_as_uint(acc[ti][tj][q * 4 + 2]), __float_as_uint(acc[ti][tj][q * 4 + 3])});
        } else {
          const T v0 = (T)acc[ti][tj][q * 4], v1 = (T)acc[ti][tj][q * 4 + 1];
          const T v2 = (T)acc[ti][tj][q * 4 + 2], v3 = (T)acc[ti][tj][q * 4 + 3];
          const uint32_t p0 = (uint32_t)__builtin_bit_cast(uint16_t, v0) |
                              ((uint32_t)__builtin_bit_cast(uint16_t, v1) << 16);
          const uint32_t p1 = (uint32_t)__builtin_bit_cast(uint16_t, v2) |
                              ((uint32_t)__builtin_bit_cast(uint16_t, v3) << 16);
          *reinterpret_cast<u32x2*>(stage + S::stage_off(rr, byte >> 4) + (byte & 15)) = u32x2{p0, p1};
        }
      }
    }
  }
  // The wave reads back only what it wrote; LDS operations of one wave complete in order.
  const int64_t dcol0 = (int64_t)ds * DK + wn * (DK / 2);
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    const uint32_t rr = (uint32_t)(it * 8 + (lane >> 3));
    const uint32_t ch = (uint32_t)(lane & 7);
    const u32x4 val = lds_ld16(stage, S::stage_off(rr, ch));
    const int64_t row = row0 + wm * 64 + rr;
    const int64_t d = dcol0 + ch * EPC;
    if (row < rows && d < D) *reinterpret_cast<u32x4*>(reinterpret_cast<T*>(out_t) + (size_t)row * D + d) = val;
  }
}

// An owner tile with no kept tiles: zeros, 16-byte stores.
template <typename T>
__device__ __forceinline__ void write_owner_tile_zero(void* out_t, int64_t row0, int64_t rows, int64_t D, int ds) {
  using S = GSum<T>;
  constexpr int DK = S::DK, EPC = S::EPC;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wm = wave & 1, wn = wave >> 1;
  const int64_t dcol0 = (int64_t)ds * DK + wn * (DK / 2);
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    const int64_t row = row0 + wm * 64 + it * 8 + (lane >> 3);
    const int64_t d = dcol0 + (lane & 7) * EPC;
    if (row < rows && d < D)
      *reinterpret_cast<u32x4*>(reinterpret_cast<T*>(out_t) + (size_t)row * D + d) = u32x4{0u, 0u, 0u, 0u};
  }
}

// fp32-accumulator modes (dE carried between chunks): element-wise.
template <typename T>
__device__ __forceinline__ void write_owner_tile_f32(void* out_t, float* out_f32, int mode,
                                                     const f32x16 (&acc)[2][GSum<T>::TJ], int64_t row0, int64_t rows,
                                                     int64_t D, int ds) {
  constexpr int TJ = GSum<T>::TJ, DK = GSum<T>::DK;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int n = lane & 31, h = lane >> 5;
#pragma unroll
  for (int ti = 0; ti < 2; ++ti) {
    const int64_t row = row0 + wm * 64 + ti * 32 + n;
    if (row >= rows) continue;
#pragma unroll
    for (int tj = 0; tj < TJ; ++tj) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t d = (int64_t)ds * DK + wn * (DK / 2) + tj * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
        if (d >= D) continue;
        const size_t idx = (size_t)row * D + d;
        const float v = acc[ti][tj][r];
        if (mode == kStoreF32) {
          out_f32[idx] = v;
        } else if (mode == kAddF32) {
          out_f32[idx] += v;
        } else {
          reinterpret_cast<T*>(out_t)[idx] = (T)(out_f32[idx] + v);
        }
      }
    }
  }
}

// Persistent owner-computes sums.  PHASE 0 (dE): owner = token block rb; group
// (rb, D slice) sums G_j . C_j over rb's kept tiles j of this chunk (G from the
// token-major scratch, C rows of tile j's vocab tile).  PHASE 1 (dC): owner =
// vocab tile vt of this chunk; group (vt, slice) sums G_j^T . E_j over vt's kept
// token blocks (G from the vocab-major scratch); the slice-0 group also writes
// dBias from the column sums.
//
// Owners are dealt to the 8 XCDs round-robin; the workgroups of an XCD take its
// groups in order, so all D slices of one owner run at the same time on one XCD
// and share its G tiles in L2.  Each workgroup walks its
// (group, tile) steps as one software pipeline: the next step's G tile and
// source slice are fetched while the current step's MFMAs run and while a
// finished group's output is written, so short groups cost no extra latency.
// A finished group's output goes through the wave's LDS staging tile and leaves
// as 16-byte row-contiguous stores (measured 19% faster dC than element stores).
template <typename T, int PHASE, bool WANT_DB>
__global__ __launch_bounds__(kThreads, 1) void bwd_sum_kernel(BwdArgs a, int chunk) {
  using S = GSum<T>;
  __shared__ __attribute__((aligned(16))) char smem[S::NBUF * S::BUF_BYTES + 4 * S::STAGE_BYTES];
  char* stage = smem + S::NBUF * S::BUF_BYTES + (threadIdx.x >> 6) * S::STAGE_BYTES;
  const int nrb = (int)a.plan.nrb, nds = (int)a.plan.n_dslices;
  const bool single = a.plan.max_chunks == 1;
  const int vt_lo = a.chunk_vt[chunk], vt_hi = a.chunk_vt[chunk + 1];
  const int slot_lo = a.chunk_slot[chunk];
  const int own_lo = PHASE == 0 ? 0 : vt_lo;
  const int own_hi = PHASE == 0 ? nrb : vt_hi;
  const int n_own = own_hi - own_lo;
  if (n_own <= 0) return;
  if (PHASE == 0 && !single && slot_lo == a.chunk_slot[chunk + 1] && chunk > 0) return;  // nothing to add
  // Owners are dealt to the XCDs round-robin (owner own_lo + xcd + 8k), which spreads
  // the heavy owners of skewed target distributions over all XCDs.
  const int xcd = (int)(blockIdx.x & 7), lidx = (int)(blockIdx.x >> 3), nper = (int)(gridDim.x >> 3);
  const int n_mine = n_own > xcd ? (n_own - xcd + 7) / 8 : 0;
  const int ngroups = n_mine * nds;
  const int64_t pitch = a.D * (int64_t)sizeof(T);
  const char* src = reinterpret_cast<const char*>(PHASE == 0 ? a.c : a.e);
  const int64_t src_rows = PHASE == 0 ? a.V : a.N;

  struct Step {
    int q, owner, ds, b, cnt, j, mode;
  };
  auto group = [&](int q, Step& st) -> bool {
    if (q >= ngroups) return false;
    st.q = q;
    st.owner = own_lo + xcd + 8 * (q / nds);
    st.ds = q - (q / nds) * nds;
    st.j = 0;
    if (PHASE == 0) {
      const int rs = a.rb_start[st.owner], re = a.rb_start[st.owner + 1];
      if (single) {
        st.b = rs;
        st.cnt = re - rs;
        st.mode = kWriteT;
      } else {
        int b = rs;
        while (b < re && a.rb_vt[b] < vt_lo) ++b;
        int cnt = 0;
        while (b + cnt < re && a.rb_vt[b + cnt] < vt_hi) ++cnt;
        st.b = b;
        st.cnt = cnt;
        const bool prev = b > rs, next = b + cnt < re;
        if (cnt == 0) st.mode = (rs == re && chunk == 0) ? kWriteT : kSkip;
        else st.mode = prev ? (next ? kAddF32 : kFinishT) : (next ? kStoreF32 : kWriteT);
      }
    } else {
      st.b = a.vt_start[st.owner];
      st.cnt = a.vt_start[st.owner + 1] - st.b;
      st.mode = kWriteT;
    }
    return true;
  };
  auto next = [&](const Step& cur, Step& nx) -> bool {
    if (cur.j + 1 < cur.cnt) {
      nx = cur;
      ++nx.j;
      return true;
    }
    return group(cur.q + nper, nx);
  };
  auto source = [&](const Step& st, const char*& gt, int64_t& row0) {
    if (PHASE == 0) {
      const int pos = st.b + st.j;
      gt = a.w_tok + (size_t)(a.rb_list[pos] - slot_lo) * a.plan.w_bytes;
      row0 = (int64_t)a.rb_vt[pos] * kBwdVocab;
    } else {
      const int slot = st.b + st.j;
      gt = a.w_voc + (size_t)(slot - slot_lo) * a.plan.w_bytes;
      row0 = (int64_t)(a.list[slot] % nrb) * kBwdTokens;
    }
  };
  auto finish = [&](const Step& st, const f32x16 (&acc)[2][S::TJ]) {
    const int64_t orow0 = (int64_t)st.owner * (PHASE == 0 ? kBwdTokens : kBwdVocab);
    const int64_t orows = PHASE == 0 ? a.N : a.V;
    void* out = PHASE == 0 ? a.dE : a.dC;
    if (st.mode == kWriteT) {
      if (st.cnt > 0)
        write_owner_tile_staged<T>(out, acc, orow0, orows, a.D, st.ds, stage);
      else
        write_owner_tile_zero<T>(out, orow0, orows, a.D, st.ds);
    } else if (st.mode != kSkip) {
      write_owner_tile_f32<T>(out, a.de_acc, st.mode, acc, orow0, orows, a.D, st.ds);
    }
    if constexpr (PHASE == 1 && WANT_DB) {
      if (st.ds == 0 && threadIdx.x < kBwdVocab) {
        const int64_t v = (int64_t)st.owner * kBwdVocab + threadIdx.x;
        float sum = 0.f;
        for (int j = 0; j < st.cnt; ++j) {
          const float* cs = a.colsum + (size_t)(st.b + j - slot_lo) * 2 * kBwdVocab;
          sum += cs[threadIdx.x] + cs[kBwdVocab + threadIdx.x];
        }
        if (v < a.V) reinterpret_cast<T*>(a.dBias)[v] = (T)sum;
      }
    }
  };

  Step cur;
  if (!group(lidx, cur)) return;
  f32x16 acc[2][S::TJ];
#pragma unroll
  for (int ti = 0; ti < 2; ++ti)
#pragma unroll
    for (int tj = 0; tj < S::TJ; ++tj) acc[ti][tj] = zero16();
  typename S::Regs R;
  const char* gt;
  int64_t row0;
  if (cur.cnt > 0) {
    source(cur, gt, row0);
    S::load(R, gt, src, src_rows, row0, pitch, pitch, cur.ds);
    S::store(R, smem);
  }
  __syncthreads();
  int bi = 0;
  for (;;) {
    Step nx;
    const bool has_next = next(cur, nx);
    const bool next_loads = has_next && nx.cnt > 0;
    if (next_loads) {
      source(nx, gt, row0);
      S::load(R, gt, src, src_rows, row0, pitch, pitch, nx.ds);
    }
    if (cur.cnt > 0) S::mma(smem + bi * S::BUF_BYTES, acc);
    if (cur.j + 1 >= (cur.cnt > 0 ? cur.cnt : 1)) {
      finish(cur, acc);
#pragma unroll
      for (int ti = 0; ti < 2; ++ti)
#pragma unroll
        for (int tj = 0; tj < S::TJ; ++tj) acc[ti][tj] = zero16();
    }
    if (!has_next) break;
    if constexpr (S::NBUF == 2) {
      if (next_loads) S::store(R, smem + (bi ^ 1) * S::BUF_BYTES);
      __syncthreads();
      bi ^= 1;
    } else {
      __syncthreads();  // every wave is done reading the single buffer
      if (next_loads) S::store(R, smem);
      __syncthreads();
    }
    cur = nx;
  }
}

// dBias only (c does not require a gradient): sum of the column sums per vocab tile.
template <typename T>
__global__ __launch_bounds__(kBwdVocab) void bwd_dbias_kernel(BwdArgs a, int chunk) {
  const int vt = a.chunk_vt[chunk] + (int)blockIdx.x;
  if (vt >= a.chunk_vt[chunk + 1]) return;
  const int slot_lo = a.chunk_slot[chunk];
  const int b = a.vt_start[vt], cnt = a.vt_start[vt + 1] - b;
  const int64_t v = (int64_t)vt * kBwdVocab + threadIdx.x;
  float sum = 0.f;
  for (int j = 0; j < cnt; ++j) {
    const float* cs = a.colsum + (size_t)(b + j - slot_lo) * 2 * kBwdVocab;
    sum += cs[threadIdx.x] + cs[kBwdVocab + threadIdx.x];
  }
  if (v < a.V) reinterpret_cast<T*>(a.dBias)[v] = (T)sum;
}

// ---------------------------------------------------------------- launch
template <typename T, bool HB>
static void launch_g(const BwdArgs& a, int chunk, dim3 grid, hipStream_t s) {
  const bool tok = a.dE != nullptr, voc = a.dC != nullptr, db = a.dBias != nullptr;
#define CCE_G(TOK, VOC, DB)                                                                               \
  if (tok == TOK && voc == VOC && db == DB) {                                                           \
    hipLaunchKernelGGL((bwd_g_kernel<T, HB, TOK, VOC, DB>), grid, dim3(kThreads), 0, s, a, chunk);       \
    return;                                                                                             \
  }
  CCE_G(true, true, true)
  CCE_G(true, true, false)
  CCE_G(true, false, true)
  CCE_G(true, false, false)
  CCE_G(false, true, true)
  CCE_G(false, true, false)
  CCE_G(false, false, true)
#undef CCE_G
}

template <typename T>
static hipError_t backward_typed(const BwdArgs& a, hipStream_t s) {
  const BwdPlan& P = a.plan;
  const int total = (int)P.total;
  hipLaunchKernelGGL(bwd_filter_kernel, dim3((unsigned)((total + 3) / 4)), dim3(256), 0, s, a);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(bwd_compact_vt_kernel, dim3(1), dim3(1024), 0, s, a);
  if ((err = hipGetLastError()) != hipSuccess) return err;
  const bool want_de = a.dE != nullptr, want_dc = a.dC != nullptr, want_db = a.dBias != nullptr;
  if (!(want_de || want_dc || want_db)) return hipSuccess;
  if (want_de) {
    hipLaunchKernelGGL(bwd_compact_rb_kernel, dim3(1), dim3(1024), 0, s, a);
    if ((err = hipGetLastError()) != hipSuccess) return err;
  }
  int g = a.num_cus > 0 ? a.num_cus : 256;
  if (g > P.cap) g = (int)P.cap;
  const int gp = ((a.num_cus > 0 ? a.num_cus : 256) + 7) / 8 * 8;  // persistent sum kernels
  const bool multi = P.max_chunks > 1;
  for (int chunk = 0; chunk < (int)P.max_chunks; ++chunk) {
    if (a.bias)
      launch_g<T, true>(a, chunk, dim3(g), s);
    else
      launch_g<T, false>(a, chunk, dim3(g), s);
    if ((err = hipGetLastError()) != hipSuccess) return err;
    if (want_de) {
      hipLaunchKernelGGL((bwd_sum_kernel<T, 0, false>), dim3(gp), dim3(kThreads), 0, s, a, chunk);
      if ((err = hipGetLastError()) != hipSuccess) return err;
    }
    if (want_dc) {
      if (want_db)
        hipLaunchKernelGGL((bwd_sum_kernel<T, 1, true>), dim3(gp), dim3(kThreads), 0, s, a, chunk);
      else
        hipLaunchKernelGGL((bwd_sum_kernel<T, 1, false>), dim3(gp), dim3(kThreads), 0, s, a, chunk);
      if ((err = hipGetLastError()) != hipSuccess) return err;
    } else if (want_db) {
      hipLaunchKernelGGL((bwd_dbias_kernel<T>), dim3((unsigned)P.nvt), dim3(kBwdVocab), 0, s, a, chunk);
      if ((err = hipGetLastError()) != hipSuccess) return err;
    }
  }
  (void)multi;
  return hipGetLastError();
}

hipError_t launch_backward(int dtype, const BwdArgs& a, hipStream_t s) {
  switch (dtype) {
    case 0:
      return backward_typed<float>(a, s);
    case 1:
      return backward_typed<_Float16>(a, s);
    default:
      return backward_typed<__bf16>(a, s);
  }
}

}  // namespace cce
