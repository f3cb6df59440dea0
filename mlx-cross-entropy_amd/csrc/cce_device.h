// cce_device.h — device-side building blocks shared by the forward and the
// backward kernels: dtype traits over the CDNA4 MFMA instructions, the
// XOR-swizzled LDS tile addressing, and the double-buffered "NT" MFMA main loop
// (both operands stored row-major with the contraction dimension contiguous,
// exactly how E [N, D] and C [V, D] sit in HBM).
//
// MFMA operand convention used everywhere (v_mfma_f32_32x32x16_{bf16,f16}):
//   lane l supplies 16 bytes of row (l % 32) of A and of B, taken from K-group
//   (l / 32) of a 32-byte K step.  The 32x32 fp32 result has, in lane l and
//   register r, row 8*(r/4) + 4*(l/32) + (r%4) and column l % 32.
// For fp32 inputs the same 16-byte fragment (4 floats) feeds four
// v_mfma_f32_32x32x2_f32 instructions; instruction q takes float q of each
// lane, so every K index is still paired with itself in A and B.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cce {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kThreads = 256;      // 4 waves of 64
constexpr int kStageRowBytes = 128; // bytes of the contraction dim staged per row per K tile
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ---------------------------------------------------------------- dtype traits
template <typename T>
struct Traits;

// Instruction scheduling hints: interleave the MF MFMA instructions of one step
// with NR LDS reads, NV global loads and NW LDS writes, front-loading the memory
// instructions into the first half of the MFMAs (masks: 0x008 MFMA, 0x100 DS
// read, 0x200 DS write, 0x020 VMEM read).
__host__ __device__ constexpr int sched_share(int i, int slots, int n) {
  const int use = slots / 2 > 0 ? slots / 2 : 1;
  return i < use ? (n * (i + 1) / use - n * i / use) : 0;
}

template <int I, int MF, int NR, int NV, int NW>
__device__ __forceinline__ void sched_interleave() {
  if constexpr (I < MF) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    constexpr int r = sched_share(I, MF, NR);
    constexpr int v = sched_share(I, MF, NV);
    constexpr int w = sched_share(I, MF, NW);
    if constexpr (r > 0) __builtin_amdgcn_sched_group_barrier(0x100, r, 0);
    if constexpr (v > 0) __builtin_amdgcn_sched_group_barrier(0x020, v, 0);
    if constexpr (w > 0) __builtin_amdgcn_sched_group_barrier(0x200, w, 0);
    sched_interleave<I + 1, MF, NR, NV, NW>();
  }
}

template <>
struct Traits<__bf16> {
  static constexpr int kInstrPerStep = 1;
  static __device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 acc) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
  }
};

template <>
struct Traits<_Float16> {
  static constexpr int kInstrPerStep = 1;
  static __device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 acc) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), acc, 0, 0, 0);
  }
};

template <>
struct Traits<float> {
  static constexpr int kInstrPerStep = 4;
  static __device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 acc) {
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.x), __uint_as_float(b.x), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.y), __uint_as_float(b.y), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.z), __uint_as_float(b.z), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.w), __uint_as_float(b.w), acc, 0, 0, 0);
    return acc;
  }
};

template <typename T>
__device__ __forceinline__ float to_f32(T x) {
  return static_cast<float>(x);
}

// ------------------------------------------------------------ LDS addressing
// Row-major tile of 16-byte chunks.  Chunk index is XOR-ed with a 3-bit hash of
// the row so that (a) 8 consecutive rows reading the same logical chunk (MFMA
// fragment reads) and (b) rows 8 apart writing the same chunk (transposed
// stores) land on distinct bank groups.
__device__ __forceinline__ uint32_t swz(uint32_t row, uint32_t chunk, uint32_t row_bytes) {
  return row * row_bytes + ((chunk ^ ((row ^ (row >> 3)) & 7u)) << 4);
}

__device__ __forceinline__ u32x4 lds_ld16(const char* smem, uint32_t off) {
  return *reinterpret_cast<const u32x4*>(smem + off);
}
__device__ __forceinline__ void lds_st16(char* smem, uint32_t off, u32x4 v) {
  *reinterpret_cast<u32x4*>(smem + off) = v;
}

__device__ __forceinline__ u32x4 gld16(const char* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// --------------------------------------------------------------- main loop
// acc[TI][TJ] = A_blk . B_blk^T over the full contraction length Kbytes, where
// A_blk = rows [a_row0, a_row0 + ROWS_A) of A (row pitch `pitch` bytes, rows past
// a_rows-1 clamped to the last row) and B_blk likewise.  Waves are arranged
// WA x WB; wave (wa, wb) owns A rows [wa*ROWS_A/WA, ...) and B rows
// [wb*ROWS_B/WB, ...).  smem holds two stages of (ROWS_A + ROWS_B) x 128 bytes.
// Ends with a barrier, so the caller may reuse smem immediately.
template <typename T, int ROWS_A, int ROWS_B, int WA, int WB>
struct NTMainLoop {
  static constexpr int TI = ROWS_A / WA / 32;
  static constexpr int TJ = ROWS_B / WB / 32;
  static constexpr int ROWS = ROWS_A + ROWS_B;
  static constexpr int LOADS = ROWS * (kStageRowBytes / 16) / kThreads;  // 16-byte loads per thread
  static constexpr int LA = ROWS_A / 32;
  static constexpr uint32_t STAGE_BYTES = ROWS * kStageRowBytes;
  static_assert(LOADS * kThreads == ROWS * 8, "stage must split evenly over the workgroup");
  static_assert(LA * 32 == ROWS_A && (ROWS_B % 32) == 0, "rows must be multiples of 32");

  static __device__ __forceinline__ void run(const char* __restrict__ A, int64_t a_rows, int64_t a_row0,
                                             const char* __restrict__ B, int64_t b_rows, int64_t b_row0,
                                             int64_t pitch, int64_t kbytes, char* smem,
                                             f32x16 (&acc)[TI][TJ]) {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wa = wave % WA;
    const int wb = wave / WA;
    const int q = tid & 7;    // 16-byte chunk within the 128-byte row slice
    const int rr = tid >> 3;  // 0..31

    // Per-load row byte offsets relative to the block base (rows clamped).
    const char* abase = A + a_row0 * pitch;
    const char* bbase = B + b_row0 * pitch;
    uint32_t off[LOADS];
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int row = rr + 32 * i;
      if (i < LA) {
        int64_t g = a_row0 + row;
        g = g < a_rows ? g : a_rows - 1;
        off[i] = (uint32_t)((g - a_row0) * pitch) + q * 16;
      } else {
        int64_t g = b_row0 + (row - ROWS_A);
        g = g < b_rows ? g : b_rows - 1;
        off[i] = (uint32_t)((g - b_row0) * pitch) + q * 16;
      }
    }

    const int KT = (int)((kbytes + kStageRowBytes - 1) / kStageRowBytes);
    const int arow = wa * (ROWS_A / WA) + (lane & 31);
    const int brow = ROWS_A + wb * (ROWS_B / WB) + (lane & 31);
    const int kg = lane >> 5;
    // A ragged contraction length (D*sizeof(T) not a multiple of 128) only changes
    // the loads of the last K tile; resolve it once, outside the pipelined loop.
    if (kbytes % kStageRowBytes == 0) {
      loop<false>(abase, bbase, off, kbytes, KT, smem, arow, brow, kg, q, rr, acc);
    } else {
      loop<true>(abase, bbase, off, kbytes, KT, smem, arow, brow, kg, q, rr, acc);
    }
  }

  // One K tile = 4 MFMA steps of 32 bytes.  Software pipeline (one barrier per tile):
  //   step 0: issue the global loads of tile kt+1, read fragments of step 1
  //   step 1: read fragments of step 2
  //   step 2: read fragments of step 3, write tile kt+1 (registers -> other stage)
  //   barrier
  //   step 3: read fragments of step 0 of tile kt+1
  // and every step's MFMAs are interleaved with those memory instructions so that
  // LDS and global latency hide behind the matrix cores.  The last iteration
  // reloads the last tile into the idle stage, which keeps the body branch-free.
  template <bool RAGGED>
  static __device__ __forceinline__ void loop(const char* abase, const char* bbase, const uint32_t (&off)[LOADS],
                                              int64_t kbytes, int KT, char* smem, int arow, int brow, int kg,
                                              int q, int rr, f32x16 (&acc)[TI][TJ]) {
    u32x4 pre[LOADS];
    auto gload = [&](int kt) {
      const int64_t k0 = (int64_t)kt * kStageRowBytes;
      if constexpr (RAGGED) {
        const bool kin = k0 + q * 16 < kbytes;
        const int64_t kk = kin ? k0 : 0;  // out-of-range chunks re-read column 0 and are zeroed
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
          const u32x4 v = gld16((i < LA ? abase : bbase) + kk + off[i]);
          pre[i] = kin ? v : u32x4{0u, 0u, 0u, 0u};
        }
      } else {
#pragma unroll
        for (int i = 0; i < LOADS; ++i) pre[i] = gld16((i < LA ? abase : bbase) + k0 + off[i]);
      }
    };
    auto sstore = [&](char* s) {
#pragma unroll
      for (int i = 0; i < LOADS; ++i) lds_st16(s, swz(rr + 32 * i, q, kStageRowBytes), pre[i]);
    };
    auto frags = [&](const char* s, int ks, u32x4 (&af)[TI], u32x4 (&bf)[TJ]) {
#pragma unroll
      for (int ti = 0; ti < TI; ++ti) af[ti] = lds_ld16(s, swz(arow + ti * 32, ks * 2 + kg, kStageRowBytes));
#pragma unroll
      for (int tj = 0; tj < TJ; ++tj) bf[tj] = lds_ld16(s, swz(brow + tj * 32, ks * 2 + kg, kStageRowBytes));
    };
    auto mma = [&](const u32x4 (&af)[TI], const u32x4 (&bf)[TJ]) {
#pragma unroll
      for (int ti = 0; ti < TI; ++ti)
#pragma unroll
        for (int tj = 0; tj < TJ; ++tj) acc[ti][tj] = Traits<T>::mfma(af[ti], bf[tj], acc[ti][tj]);
    };
    static_assert(kStageRowBytes / 32 == 4, "the pipeline below is written for 4 steps per K tile");
    constexpr int MF = TI * TJ * Traits<T>::kInstrPerStep;  // MFMA instructions per step
    constexpr int NR = TI + TJ;                             // fragment reads per step

    gload(0);
    sstore(smem);
    __syncthreads();
    u32x4 fa0[TI], fb0[TJ], fa1[TI], fb1[TJ];
    frags(smem, 0, fa0, fb0);
    for (int kt = 0; kt < KT; ++kt) {
      const char* s = smem + (kt & 1) * STAGE_BYTES;
      char* sn = smem + ((kt + 1) & 1) * STAGE_BYTES;
      gload(kt + 1 < KT ? kt + 1 : KT - 1);
      frags(s, 1, fa1, fb1);
      mma(fa0, fb0);
      sched_interleave<0, MF, NR, LOADS, 0>();
      frags(s, 2, fa0, fb0);
      mma(fa1, fb1);
      sched_interleave<0, MF, NR, 0, 0>();
      frags(s, 3, fa1, fb1);
      mma(fa0, fb0);
      sstore(sn);
      sched_interleave<0, MF, NR, 0, LOADS>();
      __builtin_amdgcn_sched_barrier(0);  // keep every step-2 MFMA ahead of the barrier
      __syncthreads();
      __builtin_amdgcn_sched_barrier(0);
      frags(sn, 0, fa0, fb0);
      mma(fa1, fb1);
      sched_interleave<0, MF, NR, 0, 0>();
    }
    __syncthreads();
  }
};

}  // namespace cce
