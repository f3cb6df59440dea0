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
  float* dE_acc;     // fp32 [N, D] or null
  float* dC_acc;     // fp32 [V, D] or null
  float* dBias_acc;  // fp32 [V] or null
  uint8_t* flags;    // [nvt * nrb]
  int* list;         // [nvt * nrb]
  int* count;        // [1]
  int64_t* tile_stats;  // [2] or null
  int num_cus;
};

// dtype: 0 f32, 1 f16, 2 bf16.  Return hipError_t of the launches.
hipError_t launch_forward(int dtype, const FwdArgs& a, hipStream_t s);
hipError_t launch_backward(int dtype, const BwdArgs& a, hipStream_t s);
hipError_t launch_fill_zero(void* p, size_t bytes, hipStream_t s);
hipError_t launch_cast(int dtype, const float* src, void* dst, int64_t n, hipStream_t s);

}  // namespace cce
