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

template <>
struct Traits<__bf16> {
  static __device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 acc) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
  }
};

template <>
struct Traits<_Float16> {
  static __device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 acc) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), acc, 0, 0, 0);
  }
};

template <>
struct Traits<float> {
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

    u32x4 pre[LOADS];
    const int KT = (int)((kbytes + kStageRowBytes - 1) / kStageRowBytes);

    // Global -> registers for K tile kt.  Full tiles take the branch-free path;
    // only a ragged last tile (D*sizeof(T) not a multiple of 128) predicates per lane.
    auto gload = [&](int kt) {
      const int64_t k0 = (int64_t)kt * kStageRowBytes;
      if (k0 + kStageRowBytes <= kbytes) {
#pragma unroll
        for (int i = 0; i < LOADS; ++i) pre[i] = gld16((i < LA ? abase : bbase) + k0 + off[i]);
      } else {
        const bool kin = k0 + q * 16 < kbytes;
#pragma unroll
        for (int i = 0; i < LOADS; ++i)
          pre[i] = kin ? gld16((i < LA ? abase : bbase) + k0 + off[i]) : u32x4{0u, 0u, 0u, 0u};
      }
    };
    auto sstore = [&](int stage) {
      char* s = smem + stage * STAGE_BYTES;
#pragma unroll
      for (int i = 0; i < LOADS; ++i) lds_st16(s, swz(rr + 32 * i, q, kStageRowBytes), pre[i]);
    };

    const int arow = wa * (ROWS_A / WA) + (lane & 31);
    const int brow = ROWS_A + wb * (ROWS_B / WB) + (lane & 31);
    const int kg = lane >> 5;
    auto frags = [&](const char* s, int ks, u32x4 (&af)[TI], u32x4 (&bf)[TJ]) {
#pragma unroll
      for (int ti = 0; ti < TI; ++ti) af[ti] = lds_ld16(s, swz(arow + ti * 32, ks * 2 + kg, kStageRowBytes));
#pragma unroll
      for (int tj = 0; tj < TJ; ++tj) bf[tj] = lds_ld16(s, swz(brow + tj * 32, ks * 2 + kg, kStageRowBytes));
    };

    gload(0);
    sstore(0);
    __syncthreads();

    constexpr int KS = kStageRowBytes / 32;  // 32-byte K steps per stage
    for (int kt = 0; kt < KT; ++kt) {
      if (kt + 1 < KT) gload(kt + 1);
      const char* s = smem + (kt & 1) * STAGE_BYTES;
      // Fragments of step ks+1 are read from LDS while the MFMAs of step ks run.
      u32x4 af[2][TI], bf[2][TJ];
      frags(s, 0, af[0], bf[0]);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        if (ks + 1 < KS) frags(s, ks + 1, af[(ks + 1) & 1], bf[(ks + 1) & 1]);
#pragma unroll
        for (int ti = 0; ti < TI; ++ti)
#pragma unroll
          for (int tj = 0; tj < TJ; ++tj) acc[ti][tj] = Traits<T>::mfma(af[ks & 1][ti], bf[ks & 1][tj], acc[ti][tj]);
      }
      if (kt + 1 < KT) sstore((kt + 1) & 1);
      __syncthreads();
    }
  }
};

}  // namespace cce
