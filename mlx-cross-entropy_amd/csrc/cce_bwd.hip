// cce_bwd.hip — backward pass of Cut Cross-Entropy on CDNA4 (gfx950).
//
//   G[r, v] = d_nll[r] * (softmax_v(E_r . C^T + b) - [v == t_r])
//   dE = G . C      dC = G^T . E      dBias = sum_r G[r, :]
//
// Pipeline (all on the caller's stream):
//   1. bwd_filter_kernel  — one wave per (vocab tile, token block): keep the
//      128x128 tile iff some row with d_nll != 0 has its target in the tile or
//      tile_max - lse >= filter_log_eps.
//      Reference predicate: csrc/cce/cce.metal:191-204 (32x32 granularity there).
//   2. bwd_compact_kernel — ordered compaction of the kept tiles (vocab-tile
//      major, so consecutive work items share C rows).
//   3. bwd_tile_kernel    — persistent; per kept tile: recompute the logits on
//      MFMA, form W = G tile in fp32 registers, then stream D in 256-byte chunks
//      through LDS (transposed on the way in) for dE_tile = W . C_blk and
//      dC_tile = W^T . E_blk on MFMA, each flushed with fp32 atomics.  dBias is a
//      column sum of W.  No [N, tiles, D] scratch exists.
//      Reference: cce.metal:146-326 (cce_backward) and the full-gradient spec
//      reference/_fused_backward.py:1406-1587 (dC :1535-1545, dBias :1546-1553).
//   4. cast_kernel        — fp32 accumulators -> output dtype
//      (reference: astype in cce.cpp:178,442-446 / _fused_backward.py:1652-1654).
#include "cce_device.h"
#include "cce_launch.h"

namespace cce {

static_assert(kStatTile == kBwdVocab, "filter statistics are kept per backward vocabulary tile");

__global__ __launch_bounds__(256) void bwd_filter_kernel(BwdArgs a, int nvt, int nrb) {
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

__global__ __launch_bounds__(1024) void bwd_compact_kernel(BwdArgs a, int total) {
  __shared__ int scan[1024];
  const int tid = threadIdx.x;
  const int per = (total + 1023) / 1024;
  const int beg = min(tid * per, total);
  const int end = min(beg + per, total);
  int cnt = 0;
  for (int i = beg; i < end; ++i) cnt += a.flags[i];
  scan[tid] = cnt;
  __syncthreads();
  for (int o = 1; o < 1024; o <<= 1) {
    const int v = tid >= o ? scan[tid - o] : 0;
    __syncthreads();
    scan[tid] += v;
    __syncthreads();
  }
  int pos = scan[tid] - cnt;
  for (int i = beg; i < end; ++i)
    if (a.flags[i]) a.list[pos++] = i;
  if (tid == 1023) {
    *a.count = scan[1023];
    if (a.tile_stats) {
      a.tile_stats[0] = scan[1023];
      a.tile_stats[1] = total;
    }
  }
}

// ------------------------------------------------------------------ pass 2
// out[out_row0 + m, d] += sum_k W[m, k] * SRC[src_row0 + k, d]   for m, k in [0, 128)
// W sits in LDS (wsm) as 128 rows of 128 elements (row-major, k contiguous).
// SRC rows are streamed in chunks of 256 bytes of D, transposed into LDS
// ([d][k], k contiguous) so both MFMA operands are k-contiguous fragments.
template <typename T>
struct Pass2 {
  static constexpr int EPC = 16 / sizeof(T);           // elements per 16-byte fragment
  static constexpr int DK = 256 / sizeof(T);           // D elements per chunk
  static constexpr uint32_t ROW_BYTES = 128 * sizeof(T);  // one row of W or of the transposed chunk
  static constexpr uint32_t CHUNK_BYTES = DK * ROW_BYTES;  // 32 KiB for every dtype
  static constexpr int NB = (128 / EPC) * 16 / kThreads;   // EPC x EPC transpose blocks per thread
  static constexpr int TJ = DK / 2 / 32;                   // 32-col MFMA tiles per wave along D
  static constexpr int KS = (int)(ROW_BYTES / 32);         // 32-byte K steps over 128 elements
  static_assert(NB >= 1 && NB * kThreads == (128 / EPC) * 16, "transpose blocks must split evenly");

  static __device__ __forceinline__ void load(u32x4 (&reg)[NB][EPC], const char* src, int64_t src_rows,
                                              int64_t src_row0, int64_t pitch, int64_t kbytes, int c) {
#pragma unroll
    for (int s = 0; s < NB; ++s) {
      const int b = threadIdx.x + kThreads * s;
      const int dblk = b & 15;
      const int vblk = b >> 4;
      const int64_t col = (int64_t)c * 256 + dblk * 16;
      const bool in = col < kbytes;
#pragma unroll
      for (int x = 0; x < EPC; ++x) {
        int64_t g = src_row0 + vblk * EPC + x;
        g = g < src_rows ? g : src_rows - 1;
        reg[s][x] = in ? gld16(src + g * pitch + col) : u32x4{0u, 0u, 0u, 0u};
      }
    }
  }

  static __device__ __forceinline__ void store_transposed(const u32x4 (&reg)[NB][EPC], char* buf) {
#pragma unroll
    for (int s = 0; s < NB; ++s) {
      const int b = threadIdx.x + kThreads * s;
      const int dblk = b & 15;
      const int vblk = b >> 4;
#pragma unroll
      for (int y = 0; y < EPC; ++y) {
        u32x4 o;
        if constexpr (sizeof(T) == 4) {
          o = u32x4{reg[s][0][y], reg[s][1][y], reg[s][2][y], reg[s][3][y]};
        } else {
          const int wd = y >> 1;
          const bool hi = y & 1;
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const uint32_t lo_src = reg[s][2 * k][wd];
            const uint32_t hi_src = reg[s][2 * k + 1][wd];
            o[k] = hi ? ((lo_src >> 16) | (hi_src & 0xffff0000u)) : ((lo_src & 0xffffu) | (hi_src << 16));
          }
        }
        lds_st16(buf, swz(dblk * EPC + y, vblk, ROW_BYTES), o);
      }
    }
  }

  static __device__ __forceinline__ void run(const char* wsm, const char* src, int64_t src_rows, int64_t src_row0,
                                             int64_t pitch, int64_t D, float* out, int64_t out_rows,
                                             int64_t out_row0, char* smem) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave & 1;
    const int wn = wave >> 1;
    const int n = lane & 31;
    const int h = lane >> 5;
    const int kg = lane >> 5;
    const int64_t kbytes = D * (int64_t)sizeof(T);
    const int NC = (int)((kbytes + 255) / 256);

    u32x4 reg[NB][EPC];
    load(reg, src, src_rows, src_row0, pitch, kbytes, 0);
    store_transposed(reg, smem);
    __syncthreads();

    for (int c = 0; c < NC; ++c) {
      if (c + 1 < NC) load(reg, src, src_rows, src_row0, pitch, kbytes, c + 1);
      const char* buf = smem + (c & 1) * CHUNK_BYTES;
      f32x16 acc[2][TJ];
#pragma unroll
      for (int ti = 0; ti < 2; ++ti)
#pragma unroll
        for (int tj = 0; tj < TJ; ++tj) acc[ti][tj] = zero16();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        u32x4 af[2], bf[TJ];
#pragma unroll
        for (int ti = 0; ti < 2; ++ti) af[ti] = lds_ld16(wsm, swz(wm * 64 + ti * 32 + n, ks * 2 + kg, ROW_BYTES));
#pragma unroll
        for (int tj = 0; tj < TJ; ++tj)
          bf[tj] = lds_ld16(buf, swz(wn * (DK / 2) + tj * 32 + n, ks * 2 + kg, ROW_BYTES));
#pragma unroll
        for (int ti = 0; ti < 2; ++ti)
#pragma unroll
          for (int tj = 0; tj < TJ; ++tj) acc[ti][tj] = Traits<T>::mfma(af[ti], bf[tj], acc[ti][tj]);
      }
      if (c + 1 < NC) store_transposed(reg, smem + ((c + 1) & 1) * CHUNK_BYTES);
      // flush: lane holds column d = c*DK + wn*DK/2 + 32 tj + n, rows 8(r/4) + 4h + r%4
#pragma unroll
      for (int tj = 0; tj < TJ; ++tj) {
        const int64_t d = (int64_t)c * DK + wn * (DK / 2) + tj * 32 + n;
        if (d < D) {
#pragma unroll
          for (int ti = 0; ti < 2; ++ti) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int64_t row = out_row0 + wm * 64 + ti * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
              if (row < out_rows) atomicAdd(out + row * D + d, acc[ti][tj][r]);
            }
          }
        }
      }
      __syncthreads();
    }
  }
};

// W (fp32, in the pass-1 accumulator layout) -> LDS as [token][vocab].
// acc[i][j][r]: vocab 64 wv + 32 i + 8 (r/4) + 4 h + r%4, token 64 wt + 32 j + n.
template <typename T>
__device__ __forceinline__ void store_w_token_major(char* wsm, const f32x16 (&w)[2][2], int wv, int wt, int n,
                                                    int h) {
  constexpr uint32_t ROW_BYTES = 128 * sizeof(T);
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
          lds_st16(wsm, swz(row, col >> 2, ROW_BYTES), o);
        } else {
          T v0 = (T)w[i][j][rq * 4 + 0], v1 = (T)w[i][j][rq * 4 + 1];
          T v2 = (T)w[i][j][rq * 4 + 2], v3 = (T)w[i][j][rq * 4 + 3];
          const uint32_t p0 = (uint32_t)__builtin_bit_cast(uint16_t, v0) |
                              ((uint32_t)__builtin_bit_cast(uint16_t, v1) << 16);
          const uint32_t p1 = (uint32_t)__builtin_bit_cast(uint16_t, v2) |
                              ((uint32_t)__builtin_bit_cast(uint16_t, v3) << 16);
          *reinterpret_cast<u32x2*>(wsm + swz(row, col >> 3, ROW_BYTES) + (col & 7) * 2) = u32x2{p0, p1};
        }
      }
    }
  }
}

// W -> LDS as [vocab][token].
template <typename T>
__device__ __forceinline__ void store_w_vocab_major(char* wsm, const f32x16 (&w)[2][2], int wv, int wt, int n,
                                                    int h) {
  constexpr uint32_t ROW_BYTES = 128 * sizeof(T);
  constexpr int EPC = 16 / sizeof(T);
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int col = wt * 64 + j * 32 + n;  // token
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = wv * 64 + i * 32 + (r >> 2) * 8 + h * 4 + (r & 3);  // vocab
        *reinterpret_cast<T*>(wsm + swz(row, col / EPC, ROW_BYTES) + (col % EPC) * sizeof(T)) = (T)w[i][j][r];
      }
    }
  }
}

template <typename T, bool HAS_BIAS, bool WANT_DE, bool WANT_DC, bool WANT_DB>
__global__ __launch_bounds__(kThreads, 1) void bwd_tile_kernel(BwdArgs a, int nrb) {
  using Loop = NTMainLoop<T, kBwdVocab, kBwdTokens, 2, 2>;  // A = C rows (vocab), B = E rows (tokens)
  constexpr uint32_t STAGE = Loop::SMEM_BYTES;               // 64 KiB, reused by pass 2
  constexpr uint32_t W_BYTES = 128 * 128 * sizeof(T);
  static_assert(2 * Pass2<T>::CHUNK_BYTES <= STAGE, "pass-2 chunks alias the pass-1 stages");
  __shared__ __attribute__((aligned(16))) char smem[STAGE + W_BYTES];
  char* wsm = smem + STAGE;

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
  const int count = *a.count;

  for (int idx = blockIdx.x; idx < count; idx += gridDim.x) {
    const int pair = a.list[idx];
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

    // W = g (softmax - onehot), zero outside [0,N) x [0,V) and for rows with g == 0.
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

    if constexpr (WANT_DB) {
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
          const int64_t v = v0 + wv * 64 + i * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
          if (n == 0 && v < a.V) atomicAdd(a.dBias_acc + v, s);
        }
      }
    }

    if constexpr (WANT_DE) {
      store_w_token_major<T>(wsm, w, wv, wt, n, h);
      Pass2<T>::run(wsm, C, a.V, v0, pitch, a.D, a.dE_acc, a.N, t0, smem);
    }
    if constexpr (WANT_DC) {
      store_w_vocab_major<T>(wsm, w, wv, wt, n, h);
      Pass2<T>::run(wsm, E, a.N, t0, pitch, a.D, a.dC_acc, a.V, v0, smem);
    }
  }
}

__global__ __launch_bounds__(256) void fill_zero_kernel(u32x4* p, int64_t n16) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) p[i] = u32x4{0u, 0u, 0u, 0u};
}

template <typename T>
__global__ __launch_bounds__(256) void cast_kernel(const float* __restrict__ src, T* __restrict__ dst, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x * 4;
  for (int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4; i < n; i += stride) {
    if (i + 4 <= n) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(src + i);
      if constexpr (sizeof(T) == 4) {
        *reinterpret_cast<f32x4*>(dst + i) = v;
      } else {
        T o0 = (T)v.x, o1 = (T)v.y, o2 = (T)v.z, o3 = (T)v.w;
        const uint32_t p0 = (uint32_t)__builtin_bit_cast(uint16_t, o0) | ((uint32_t)__builtin_bit_cast(uint16_t, o1) << 16);
        const uint32_t p1 = (uint32_t)__builtin_bit_cast(uint16_t, o2) | ((uint32_t)__builtin_bit_cast(uint16_t, o3) << 16);
        *reinterpret_cast<u32x2*>(dst + i) = u32x2{p0, p1};
      }
    } else {
      for (int64_t k = i; k < n; ++k) dst[k] = (T)src[k];
    }
  }
}

static unsigned grid_for(int64_t items, int per_block) {
  int64_t g = (items + per_block - 1) / per_block;
  if (g < 1) g = 1;
  if (g > 65536) g = 65536;
  return (unsigned)g;
}

hipError_t launch_fill_zero(void* p, size_t bytes, hipStream_t s) {
  const int64_t n16 = (int64_t)(bytes / 16);
  if (n16 == 0) return hipSuccess;
  hipLaunchKernelGGL(fill_zero_kernel, dim3(grid_for(n16, 256)), dim3(256), 0, s, reinterpret_cast<u32x4*>(p), n16);
  return hipGetLastError();
}

hipError_t launch_cast(int dtype, const float* src, void* dst, int64_t n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  const dim3 grid(grid_for(n, 1024)), block(256);
  switch (dtype) {
    case 0:
      hipLaunchKernelGGL((cast_kernel<float>), grid, block, 0, s, src, reinterpret_cast<float*>(dst), n);
      break;
    case 1:
      hipLaunchKernelGGL((cast_kernel<_Float16>), grid, block, 0, s, src, reinterpret_cast<_Float16*>(dst), n);
      break;
    default:
      hipLaunchKernelGGL((cast_kernel<__bf16>), grid, block, 0, s, src, reinterpret_cast<__bf16*>(dst), n);
      break;
  }
  return hipGetLastError();
}

template <typename T, bool HB>
static void launch_tile(const BwdArgs& a, int nrb, dim3 grid, hipStream_t s) {
  const bool de = a.dE_acc != nullptr, dc = a.dC_acc != nullptr, db = a.dBias_acc != nullptr;
#define CCE_TILE(DE, DC, DB)                                                                              \
  if (de == DE && dc == DC && db == DB) {                                                               \
    hipLaunchKernelGGL((bwd_tile_kernel<T, HB, DE, DC, DB>), grid, dim3(kThreads), 0, s, a, nrb);        \
    return;                                                                                             \
  }
  CCE_TILE(true, true, true)
  CCE_TILE(true, true, false)
  CCE_TILE(true, false, true)
  CCE_TILE(true, false, false)
  CCE_TILE(false, true, true)
  CCE_TILE(false, true, false)
  CCE_TILE(false, false, true)
#undef CCE_TILE
}

template <typename T>
static hipError_t backward_typed(const BwdArgs& a, hipStream_t s) {
  const int nvt = (int)((a.V + kBwdVocab - 1) / kBwdVocab);
  const int nrb = (int)((a.N + kBwdTokens - 1) / kBwdTokens);
  const int total = nvt * nrb;
  hipLaunchKernelGGL(bwd_filter_kernel, dim3((unsigned)((total + 3) / 4)), dim3(256), 0, s, a, nvt, nrb);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(bwd_compact_kernel, dim3(1), dim3(1024), 0, s, a, total);
  if ((err = hipGetLastError()) != hipSuccess) return err;
  if (a.dE_acc || a.dC_acc || a.dBias_acc) {
    int g = a.num_cus > 0 ? a.num_cus : 256;
    if (g > total) g = total;
    if (a.bias)
      launch_tile<T, true>(a, nrb, dim3(g), s);
    else
      launch_tile<T, false>(a, nrb, dim3(g), s);
  }
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
