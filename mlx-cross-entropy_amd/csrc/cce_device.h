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

// 16 bytes per lane from global memory into LDS (global_load_lds_dwordx4; the
// wave's 64 lanes fill 1 KiB at LDS byte address `lds`, lane l at lds + 16 l).
// Issued as inline assembly: the compiler then does not track the LDS write, so
// it adds no conservative vmcnt wait in front of later LDS reads it cannot prove
// disjoint (it would for the transposing reads).  The caller orders the DMA and
// the reads of its LDS bytes with explicit vmcnt waits and barriers.
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)(p);
}

// Wave-uniform read of an int list written by an earlier kernel: through the
// constant address space with a readfirstlane'd index the compiler emits a scalar
// load (counted by lgkmcnt), so it never waits on the vector-memory counter that
// tracks the LDS-DMA pipeline.
__device__ __forceinline__ int ldu(const int* p, int i) {
  return reinterpret_cast<const __attribute__((address_space(4))) int*>(reinterpret_cast<uintptr_t>(p))
      [__builtin_amdgcn_readfirstlane(i)];
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// --------------------------------------------------------------- main loop
// Stage geometry: every stage holds one SLICE-byte slice of the contraction
// dim for all ROWS_A + ROWS_B rows, as 16-byte chunks stored in the order
// chunk ^ f(row).  Measured on gfx950 with the MFMA fragment pattern (lane l
// reads row l%32, chunk 2s + l/32), both orders below are free of LDS bank
// conflicts (unswizzled 64-byte rows conflict 75% of the time).  One
// global_load_lds_dwordx4 (64 lanes x 16 bytes, written contiguously) fills
// 1024 / SLICE whole rows, each lane group covering one row's slice with a
// single SLICE-byte request.
#ifndef CCE_SLICE_BYTES
#define CCE_SLICE_BYTES 128
#endif
#ifndef CCE_STAGES
#define CCE_STAGES 2
#endif
constexpr int kSliceBytes = CCE_SLICE_BYTES;  // the forward's slice and stage count
constexpr int kStages = CCE_STAGES;

template <int SLICE>
__device__ __forceinline__ uint32_t slice_swz(uint32_t row) {
  static_assert(SLICE == 64 || SLICE == 128, "slice of 64 or 128 bytes");
  return SLICE == 128 ? ((row ^ (row >> 3)) & 7u) : ((row >> 2) & 3u);
}
template <int SLICE>
__device__ __forceinline__ uint32_t slice_off(uint32_t row, uint32_t chunk) {
  return row * SLICE + ((chunk ^ slice_swz<SLICE>(row)) << 4);
}

// Source of the zeros that pad a ragged last slice (contraction length not a
// multiple of the slice): lanes whose chunk lies past the row end read these 16 bytes.
__device__ __attribute__((aligned(16))) static const uint32_t g_zero16[4] = {0u, 0u, 0u, 0u};

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  // gfx9 s_waitcnt: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Workgroup barrier for the LDS pipeline: waits until at most N of this wave's
// LDS-DMA loads are in flight and all its LDS reads have returned, then
// s_barrier.  Unlike __syncthreads() it does not drain every outstanding load
// (the workgroup release fence would wait for vmcnt(0)), so later stages keep
// streaming in across the barrier.  The empty asm statements stop the compiler
// from moving memory operations across it.
template <int N>
__device__ __forceinline__ void stage_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (0 << 8) | ((N >> 4) << 14));
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// The "NT" main loop: acc[TI][TJ] = A_blk . B_blk^T for a ROWS_A x ROWS_B block,
// both operands row-major with the contraction contiguous, staged through LDS in
// STAGES stages of (ROWS_A + ROWS_B) x SLICE bytes by direct-to-LDS loads.
// make_src() computes one block pair's per-lane sources, prefetch() issues the
// pipeline fill and consume() runs the contraction; run() / run_gather() do all
// three.  The phase rotation of the slices (make_src) measured 5% faster in the
// forward than all XCDs streaming the same slice.
//
// SWAP: the MFMAs take the B fragment as their first operand, so acc holds the block
// transposed: acc[TJ][TI], rows of B by columns of A (same reads, same products).
template <typename T, int ROWS_A, int ROWS_B, int WA, int WB, int SLICE = kSliceBytes, int STAGES = kStages,
          bool SWAP = false>
struct NTMainLoop {
  static constexpr int kChunks = SLICE / 16;
  static constexpr int TI = ROWS_A / WA / 32;
  static constexpr int TJ = ROWS_B / WB / 32;
  static constexpr int ROWS = ROWS_A + ROWS_B;
  static constexpr int RPL = 1024 / SLICE;                 // rows filled by one LDS-DMA load
  static constexpr int NW = WA * WB;                             // waves (64 NW threads)
  static constexpr int NTHREADS = 64 * NW;
  static constexpr int LPW = ROWS / RPL / NW;                    // LDS-DMA loads per wave per stage
  static constexpr int KSTEPS = SLICE / 32;                // 32-byte MFMA steps per slice
  static constexpr uint32_t STAGE_BYTES = ROWS * SLICE;
  static constexpr uint32_t SMEM_BYTES = STAGES * STAGE_BYTES;
  using Acc = f32x16[SWAP ? TJ : TI][SWAP ? TI : TJ];
  static_assert(LPW * RPL * NW == ROWS, "stage must split evenly over the waves");
  static_assert(ROWS_A % 32 == 0 && ROWS_B % 32 == 0, "rows must be multiples of 32");
  static_assert((STAGES - 1) * LPW < 64, "in-flight loads must fit vmcnt");

  // Per-lane sources of one operand block pair.  Load j of wave w fills rows
  // [r0, r0 + RPL) of a stage, r0 = (j * NW + w) * RPL, so which operand (and which
  // segment of A) a load reads is known at compile time.  Lane l writes row
  // r0 + l/kChunks, stored chunk l%kChunks, i.e. logical chunk (l%kChunks) ^ f(row).
  // The source is the segment's wave-uniform base plus a per-lane 32-bit offset;
  // rows past the operand's end are clamped to its last row (a segment always
  // starts inside the operand).
  template <int NSEG>
  struct Src {
    const char* segb[NSEG + 1];
    uint32_t off[LPW];
    uint32_t qb[LPW];
    int64_t kbytes;
    int KT, kskew;
    uint32_t skip;  // wave-uniform: load j is not issued when bit j is set
  };

  // Sources for A_blk gathered from ROWS_A / A_SEG segments (rows [s * A_SEG,
  // (s + 1) * A_SEG) of A_blk are rows [a_seg0[s], a_seg0[s] + A_SEG) of A) and
  // B_blk = rows [b_row0, b_row0 + ROWS_B) of B.  The slices are visited starting
  // at slice phase8 * KT / 8 and wrapping around (phase8 in [0, 8)): workgroups on
  // different XCDs then stream different columns of the same rows at any moment,
  // which spreads their L2 misses over more memory channels; workgroups on one XCD
  // share a phase so that they keep sharing slices in that XCD's L2.
  template <int A_SEG>
  static __device__ __forceinline__ Src<ROWS_A / A_SEG> make_src(const char* __restrict__ A, int64_t a_rows,
                                                                 const int64_t (&a_seg0)[ROWS_A / A_SEG],
                                                                 const char* __restrict__ B, int64_t b_rows,
                                                                 int64_t b_row0, int64_t pitch, int64_t kbytes,
                                                                 int phase8) {
    constexpr int NSEG = ROWS_A / A_SEG;
    static_assert(ROWS_A % A_SEG == 0 && A_SEG % (NW * RPL) == 0, "a load round must not straddle two segments");
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    Src<NSEG> src;
#pragma unroll
    for (int k = 0; k < NSEG; ++k) src.segb[k] = A + a_seg0[k] * pitch;
    src.segb[NSEG] = B + b_row0 * pitch;
#pragma unroll
    for (int j = 0; j < LPW; ++j) {
      const int r0 = (j * NW + wave) * RPL;
      const int row = r0 + lane / kChunks;
      const uint32_t q = (uint32_t)(lane % kChunks) ^ slice_swz<SLICE>((uint32_t)row);
      src.qb[j] = q * 16;
      int64_t g;
      if (j * NW * RPL < ROWS_A) {
        const int sg = (j * NW * RPL) / A_SEG;
        g = a_seg0[sg] + (row - sg * A_SEG);
        g = g < a_rows ? g : a_rows - 1;
        src.off[j] = (uint32_t)((g - a_seg0[sg]) * pitch) + q * 16;
      } else {
        g = b_row0 + (row - ROWS_A);
        g = g < b_rows ? g : b_rows - 1;
        src.off[j] = (uint32_t)((g - b_row0) * pitch) + q * 16;
      }
    }
    src.kbytes = kbytes;
    src.skip = 0;
    src.KT = (int)((kbytes + SLICE - 1) / SLICE);
    src.kskew = (int)(((int64_t)(phase8 & 7) * src.KT) >> 3);
    return src;
  }

  // LDS-DMA loads of slice kt (clamped to the last slice: harmless reloads into
  // idle stages) into stage kt % STAGES.  Issued as inline assembly in the saddr
  // form (a scalar base plus the lane's 32-bit offset): the compiler then does not
  // count these loads, so it keeps exact lgkmcnt waits for the fragment reads (with
  // compiler-visible LDS-DMA in flight it waits for all of them), and the stage
  // barriers order the DMA against the reads of its stage.
  template <bool RAGGED, int NSEG>
  static __device__ __forceinline__ void issue(const Src<NSEG>& src, int kt, char* smem) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t lds_w = (uint32_t)(wave * RPL * SLICE);
    kt = kt < src.KT ? kt : src.KT - 1;
    char* st = smem + (kt % STAGES) * STAGE_BYTES;
    int kr = kt + src.kskew;  // slice actually loaded: rotated by the phase
    kr = kr < src.KT ? kr : kr - src.KT;
    const int64_t k0 = (int64_t)kr * SLICE;
#pragma unroll
    for (int j = 0; j < LPW; ++j) {
      if ((src.skip >> j) & 1u) continue;
      const int sg = j * NW * RPL < ROWS_A ? (j * NW * RPL) / (ROWS_A / NSEG) : NSEG;
      const uint32_t lds = __builtin_amdgcn_readfirstlane(lds_addr(st + lds_w + j * NW * RPL * SLICE));
      if constexpr (RAGGED) {
        const char* g = (src.segb[sg] + k0) + src.off[j];
        if (k0 + (int64_t)src.qb[j] >= src.kbytes) g = reinterpret_cast<const char*>(g_zero16);
        asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
      } else {
        asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(src.off[j]),
                     "s"(src.segb[sg] + k0), "s"(lds)
                     : "memory", "m0");
      }
    }
  }

  // Pipeline fill: the loads of the first STAGES - 1 slices.  smem must be free
  // (no wave still reads it); consume() then runs the contraction.  Issuing the
  // fill early lets its latency overlap other work (a persistent kernel's
  // epilogue of the previous tile).
  template <bool RAGGED, int NSEG>
  static __device__ __forceinline__ void prefetch(const Src<NSEG>& src, char* smem) {
#pragma unroll
    for (int p = 0; p < STAGES - 1; ++p) issue<RAGGED>(src, p, smem);
  }

  // acc[TI][TJ] += A_blk . B_blk^T over the full contraction, after prefetch() of
  // the same sources.  Waves are arranged WA x WB; wave (wa, wb) owns A rows
  // [wa*ROWS_A/WA, ...) and B rows [wb*ROWS_B/WB, ...).  Ends with a barrier, so
  // the caller may reuse smem immediately.
  //
  // Iteration it consumes slice it (stage it % STAGES, KSTEPS MFMA steps):
  //   read fragments of step 1 | issue the LDS-DMA loads of slice it + STAGES - 1
  //   (into the stage freed by the previous iteration) | MFMAs of step 0
  //   step s >= 1: read fragments of step s+1 | MFMAs of step s
  //   wait for slice it+1 (vmcnt), barrier
  //   read fragments of step 0 of slice it+1 | MFMAs of the last step
  // The step-1 fragment reads are placed before the DMA issue on purpose: the
  // compiler cannot tell the DMA's LDS writes from the reads, so reads that
  // follow the DMA in program order are held behind all of it, and the MFMAs of
  // step 1 would then wait on their own operands.
  // consume() calls hook() once, right after its first stage barrier (the caller's
  // deferred stores then drain while the first slice computes).
  struct NoHook {
    __device__ void operator()() const {}
  };
  template <bool RAGGED, int NSEG, typename Hook = NoHook, int FIRST_STORES = 0>
  static __device__ __forceinline__ void consume(const Src<NSEG>& src, char* smem, Acc& acc,
                                                 Hook hook = Hook(), bool stores_pending = false) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wa = wave % WA;
    const int wb = wave / WA;
    const int arow = wa * (ROWS_A / WA) + (lane & 31);
    const int brow = ROWS_A + wb * (ROWS_B / WB) + (lane & 31);
    const int kg = lane >> 5;
    const int KT = src.KT;
    auto frags = [&](const char* s, int ks, u32x4 (&af)[TI], u32x4 (&bf)[TJ]) {
#pragma unroll
      for (int ti = 0; ti < TI; ++ti) af[ti] = lds_ld16(s, slice_off<SLICE>(arow + ti * 32, ks * 2 + kg));
#pragma unroll
      for (int tj = 0; tj < TJ; ++tj) bf[tj] = lds_ld16(s, slice_off<SLICE>(brow + tj * 32, ks * 2 + kg));
    };
    auto mma = [&](const u32x4 (&af)[TI], const u32x4 (&bf)[TJ]) {
#pragma unroll
      for (int ti = 0; ti < TI; ++ti)
#pragma unroll
        for (int tj = 0; tj < TJ; ++tj) {
          if constexpr (SWAP)
            acc[tj][ti] = Traits<T>::mfma(bf[tj], af[ti], acc[tj][ti]);
          else
            acc[ti][tj] = Traits<T>::mfma(af[ti], bf[tj], acc[ti][tj]);
        }
    };
    static_assert(KSTEPS % 2 == 0, "fragments alternate between two register sets");
    constexpr int MF = TI * TJ * Traits<T>::kInstrPerStep;
    constexpr int NR = TI + TJ;
    constexpr int INFLIGHT = (STAGES - 2) * LPW;  // loads allowed in flight at the barrier

    // FIRST_STORES: the caller issued that many stores after this block pair's prefetch
    // (vmcnt counts in issue order, so waiting down to them leaves the loads landed)
    if (FIRST_STORES > 0 && stores_pending)
      stage_barrier<INFLIGHT + FIRST_STORES>();
    else
      stage_barrier<INFLIGHT>();
    hook();  // stores deferred from the caller's previous tile: they drain during this slice
    u32x4 fa0[TI], fb0[TJ], fa1[TI], fb1[TJ];
    frags(smem, 0, fa0, fb0);
    for (int it = 0; it < KT; ++it) {
      const char* s = smem + (it % STAGES) * STAGE_BYTES;
      const char* sn = smem + ((it + 1) % STAGES) * STAGE_BYTES;
      frags(s, 1, fa1, fb1);
      issue<RAGGED>(src, it + STAGES - 1, smem);
#pragma unroll
      for (int ks = 0; ks + 1 < KSTEPS; ks += 2) {
        if (ks > 0) frags(s, ks + 1, fa1, fb1);
        mma(fa0, fb0);
        if (ks == 0) {
          __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);
          sched_interleave<0, MF, 0, LPW, 0>();
        } else {
          sched_interleave<0, MF, NR, 0, 0>();
        }
        if (ks + 2 < KSTEPS) {
          frags(s, ks + 2, fa0, fb0);
          mma(fa1, fb1);
          sched_interleave<0, MF, NR, 0, 0>();
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      stage_barrier<INFLIGHT>();  // slice it+1 has landed in every wave's share of its stage
      __builtin_amdgcn_sched_barrier(0);
      frags(sn, 0, fa0, fb0);
      mma(fa1, fb1);
      sched_interleave<0, MF, NR, 0, 0>();
    }
    wait_vmcnt<0>();
    __syncthreads();
  }

  // acc[TI][TJ] = A_blk . B_blk^T over the full contraction length kbytes, where
  // A_blk = rows [a_row0, a_row0 + ROWS_A) of A (row pitch `pitch` bytes, rows past
  // a_rows-1 clamped to the last row) and B_blk likewise.  smem holds STAGES
  // stages of (ROWS_A + ROWS_B) x SLICE.
  static __device__ __forceinline__ void run(const char* __restrict__ A, int64_t a_rows, int64_t a_row0,
                                             const char* __restrict__ B, int64_t b_rows, int64_t b_row0,
                                             int64_t pitch, int64_t kbytes, char* smem,
                                             Acc& acc, int phase8 = 0) {
    const int64_t seg[1] = {a_row0};
    run_gather<ROWS_A>(A, a_rows, seg, B, b_rows, b_row0, pitch, kbytes, smem, acc, phase8);
  }

  // As run(), with A_blk gathered from segments (see make_src).
  template <int A_SEG>
  static __device__ __forceinline__ void run_gather(const char* __restrict__ A, int64_t a_rows,
                                                    const int64_t (&a_seg0)[ROWS_A / A_SEG],
                                                    const char* __restrict__ B, int64_t b_rows, int64_t b_row0,
                                                    int64_t pitch, int64_t kbytes, char* smem,
                                                    Acc& acc, int phase8 = 0) {
    const auto src = make_src<A_SEG>(A, a_rows, a_seg0, B, b_rows, b_row0, pitch, kbytes, phase8);
    if (kbytes % SLICE == 0) {
      prefetch<false>(src, smem);
      consume<false>(src, smem, acc);
    } else {
      prefetch<true>(src, smem);
      consume<true>(src, smem, acc);
    }
  }
};

}  // namespace cce
