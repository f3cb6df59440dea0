// cce_abi.hip — the extern "C" boundary declared in include/cce_mi355x.h.
//
// Host-side validation mirrors the reference's checks (csrc/cce/cce.cpp:41-73:
// ranks, D agreement, bias shape; :222-227 dtype) but reports them as negative
// return codes plus a thread-local message instead of C++ exceptions.  The
// reference's alignment precondition N%32 == 0, V%32 == 0 (cce.cpp:64-68) is
// lifted: ragged N and V are masked inside the kernels.  Rows must be 16-byte
// multiples (D % 8 == 0 for 16-bit dtypes, D % 4 == 0 for fp32); the reference
// requires D % 8 == 0 for every dtype.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "cce_launch.h"
#include "cce_mi355x.h"

// Workspace of cce_backward_noalloc: one static array per GPU, held from the first
// call on that GPU until the process ends.  Host code never uses this name as an
// address (on the host it is a stand-in symbol); it uses the device address that
// hipGetSymbolAddress returns for the current device.
static __device__ __align__(256) char scratch[CCE_NOALLOC_SCRATCH_BYTES];

namespace {

thread_local char g_err[512] = {0};

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

size_t elem_size(int dtype) { return dtype == CCE_DTYPE_F32 ? 4 : 2; }
size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Every CCE_BWD_* flag.
constexpr int kBwdFlags = CCE_BWD_DC_ZEROED | CCE_BWD_TOKENS_INPUT | CCE_BWD_TOKENS_SORTED | CCE_BWD_DE_SUMS_WIDE |
                          CCE_BWD_DE_SUMS_NARROW | CCE_BWD_DC_SUMS_WIDE | CCE_BWD_DC_SUMS_NARROW | CCE_BWD_REF_STATS |
                          CCE_BWD_DEVICE_PASSES | CCE_BWD_G_PAIR | CCE_BWD_G_SINGLE | CCE_BWD_DC_OWNER_TASKS |
                          CCE_BWD_G_TASKS_BY_BLOCK | CCE_BWD_DE_WHOLE_TASKS;
// Flags of which at most one may be set.
constexpr int kBwdFlagPairs[4][2] = {{CCE_BWD_TOKENS_INPUT, CCE_BWD_TOKENS_SORTED},
                                     {CCE_BWD_DE_SUMS_WIDE, CCE_BWD_DE_SUMS_NARROW},
                                     {CCE_BWD_DC_SUMS_WIDE, CCE_BWD_DC_SUMS_NARROW},
                                     {CCE_BWD_G_PAIR, CCE_BWD_G_SINGLE}};
bool bwd_flags_valid(int flags) {
  if (flags & ~kBwdFlags) return false;
  for (const auto& pr : kBwdFlagPairs)
    if ((flags & pr[0]) && (flags & pr[1])) return false;
  return true;
}
// The G tiles' layout: 16-bit G as the hi / lo pair with the filter off (the 1e-3
// bar), rounded once with it on, unless CCE_BWD_G_PAIR / CCE_BWD_G_SINGLE says.
bool g_split_for(size_t es, int flags, float filter_log_eps) {
  return es == 2 && !(flags & CCE_BWD_G_SINGLE) && ((flags & CCE_BWD_G_PAIR) || !(filter_log_eps > -INFINITY));
}
bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

const char* dtype_name(int dtype) {
  switch (dtype) {
    case CCE_DTYPE_F32:
      return "float32";
    case CCE_DTYPE_F16:
      return "float16";
    case CCE_DTYPE_BF16:
      return "bfloat16";
    default:
      return "?";
  }
}

int num_cus_current() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  static int cache[64] = {0};
  if (dev >= 0 && dev < 64 && cache[dev] > 0) return cache[dev];
  int cu = 0;
  if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return -1;
  if (dev >= 0 && dev < 64) cache[dev] = cu;
  return cu;
}

// Shape / pointer checks common to both passes.
int check_common(const char* fn, int dtype, const void* e, const void* c, const int64_t* targets, int64_t N,
                 int64_t D, int64_t V) {
  if (dtype != CCE_DTYPE_F32 && dtype != CCE_DTYPE_F16 && dtype != CCE_DTYPE_BF16)
    return fail(CCE_ERR_UNSUPPORTED_DTYPE, "[%s] unsupported dtype code %d (expected float32, float16 or bfloat16)",
                fn, dtype);
  if (N <= 0 || D <= 0 || V <= 0)
    return fail(CCE_ERR_INVALID_ARGUMENT, "[%s] N, D, V must be positive, got N=%lld D=%lld V=%lld", fn,
                (long long)N, (long long)D, (long long)V);
  const int64_t epc = 16 / (int64_t)elem_size(dtype);
  if (D % epc != 0)
    return fail(CCE_ERR_INVALID_ARGUMENT, "[%s] D must be a multiple of %lld for %s (16-byte rows), got D=%lld", fn,
                (long long)epc, dtype_name(dtype), (long long)D);
  if ((int64_t)elem_size(dtype) * D >= (int64_t)1 << 23)
    return fail(CCE_ERR_INVALID_ARGUMENT, "[%s] row of %lld bytes exceeds the 8 MiB limit", fn,
                (long long)(elem_size(dtype) * D));
  if (N > ((int64_t)cce::kCompactMaxWords * cce::kBwdTokens))
    return fail(CCE_ERR_INVALID_ARGUMENT, "[%s] N must be at most %lld tokens per call, got N=%lld", fn,
                (long long)cce::kCompactMaxWords * cce::kBwdTokens, (long long)N);
  if (V >= ((int64_t)1 << 31) - 256) return fail(CCE_ERR_INVALID_ARGUMENT, "[%s] V must be below 2^31", fn);
  const int64_t tiles = ((N + cce::kBwdTokens - 1) / cce::kBwdTokens) * ((V + cce::kBwdVocab - 1) / cce::kBwdVocab);
  if (tiles >= ((int64_t)1 << 31))
    return fail(CCE_ERR_INVALID_ARGUMENT, "[%s] N*V/16384 must be below 2^31", fn);
  if (!e || !c || !targets) return fail(CCE_ERR_INVALID_ARGUMENT, "[%s] e, c and targets must be non-null", fn);
  if (!aligned(e, 16) || !aligned(c, 16))
    return fail(CCE_ERR_INVALID_ARGUMENT, "[%s] e and c must be 16-byte aligned", fn);
  if (!aligned(targets, 8)) return fail(CCE_ERR_INVALID_ARGUMENT, "[%s] targets must be 8-byte aligned", fn);
  return CCE_OK;
}

// Checks of quantized classifier rows (the layout of MLX's affine quantization).
int check_quant(const char* fn, int dtype, const uint32_t* wq, const void* scales, const void* qbiases,
                int group_size, int bits, int64_t D) {
  if (!wq || !scales || !qbiases)
    return fail(CCE_ERR_INVALID_ARGUMENT, "[%s] weight, scales and biases must be non-null", fn);
  if (bits != 2 && bits != 4 && bits != 8)
    return fail(CCE_ERR_INVALID_ARGUMENT, "[%s] bits must be 2, 4 or 8, got %d", fn, bits);
  if (group_size != 32 && group_size != 64 && group_size != 128)
    return fail(CCE_ERR_INVALID_ARGUMENT, "[%s] group_size must be 32, 64 or 128, got %d", fn, group_size);
  if (D % group_size != 0)
    return fail(CCE_ERR_INVALID_ARGUMENT, "[%s] D must be a multiple of group_size (%d), got D=%lld", fn, group_size,
                (long long)D);
  if (!aligned(wq, 4) || !aligned(scales, elem_size(dtype)) || !aligned(qbiases, elem_size(dtype)))
    return fail(CCE_ERR_INVALID_ARGUMENT, "[%s] weight, scales or biases not aligned to their element size", fn);
  return CCE_OK;
}

int64_t quant_chunk_rows(int64_t chunk_rows) {
  return chunk_rows == 0 ? cce::kQuantDefaultChunkRows : chunk_rows;
}

int check_chunk_rows(const char* fn, int64_t chunk_rows) {
  if (chunk_rows < 0 || chunk_rows % cce::kQuantChunkAlign != 0 || chunk_rows > ((int64_t)1 << 30))
    return fail(CCE_ERR_INVALID_ARGUMENT, "[%s] chunk_rows must be a positive multiple of %lld (or 0), got %lld", fn,
                (long long)cce::kQuantChunkAlign, (long long)chunk_rows);
  return CCE_OK;
}

// cce_forward_ex / cce_forward_ref: stats32 selects the statistics' layout.
int forward_impl(const char* fn, int dtype, const void* e, const void* c, const void* bias, const int64_t* targets,
                 int64_t ignore_index, int has_ignore, int64_t N, int64_t D, int64_t V, float* tile_max,
                 float* tile_sum_exp, float* neg_target_logit, float* lse, float* nll, void* zero_buf,
                 int64_t zero_bytes, int stats32, void* hip_stream) {
  g_err[0] = 0;
  int rc = check_common(fn, dtype, e, c, targets, N, D, V);
  if (rc != CCE_OK) return rc;
  if (!tile_max || !tile_sum_exp || !neg_target_logit || !lse || !nll)
    return fail(CCE_ERR_INVALID_ARGUMENT, "[%s] tile_max, tile_sum_exp, neg_target_logit, lse and nll must be non-null",
                fn);
  if (bias && !aligned(bias, elem_size(dtype)))
    return fail(CCE_ERR_INVALID_ARGUMENT, "[%s] bias is not aligned to its element size", fn);
  if (zero_bytes < 0 || zero_bytes % 16 != 0 || (zero_bytes > 0 && (!zero_buf || !aligned(zero_buf, 16))))
    return fail(CCE_ERR_INVALID_ARGUMENT,
                "[%s] zero_buf must be 16-byte aligned and zero_bytes a non-negative multiple of 16", fn);
  const int cus = num_cus_current();
  if (cus <= 0) return fail(CCE_ERR_NO_DEVICE, "[%s] no HIP device is available", fn);
  cce::FwdArgs a{};
  a.e = e;
  a.c = c;
  a.bias = bias;
  a.targets = targets;
  a.ignore_index = ignore_index;
  a.has_ignore = has_ignore ? 1 : 0;
  a.N = N;
  a.D = D;
  a.V = V;
  a.tile_max = tile_max;
  a.tile_sum_exp = tile_sum_exp;
  a.neg_target_logit = neg_target_logit;
  a.lse = lse;
  a.nll = nll;
  a.num_cus = cus;
  a.zero_buf = zero_bytes > 0 ? zero_buf : nullptr;
  a.zero_units = zero_bytes / 16;
  a.stats32 = stats32;
  hipError_t err = cce::launch_forward(dtype, a, reinterpret_cast<hipStream_t>(hip_stream));
  if (err != hipSuccess)
    return fail(CCE_ERR_LAUNCH, "[%s] kernel launch failed: %s", fn, hipGetErrorString(err));
  return CCE_OK;
}

}  // namespace

extern "C" {

const char* cce_last_error(void) { return g_err; }

const char* cce_version(void) { return "cce-mi355x 0.1.0 (gfx950)"; }

void cce_tile_config(int* fwd_tokens, int* fwd_vocab, int* stat_tile, int* bwd_tokens, int* bwd_vocab) {
  if (fwd_tokens) *fwd_tokens = cce::kFwdTokens;
  if (fwd_vocab) *fwd_vocab = cce::kFwdVocab;
  if (stat_tile) *stat_tile = cce::kStatTile;
  if (bwd_tokens) *bwd_tokens = cce::kBwdTokens;
  if (bwd_vocab) *bwd_vocab = cce::kBwdVocab;
}

int64_t cce_num_vocab_tiles(int64_t V) { return V <= 0 ? 0 : (V + cce::kStatTile - 1) / cce::kStatTile; }

int cce_forward(int dtype, const void* e, const void* c, const void* bias, const int64_t* targets,
                int64_t ignore_index, int has_ignore, int64_t N, int64_t D, int64_t V, float* tile_max,
                float* tile_sum_exp, float* neg_target_logit, float* lse, float* nll, void* hip_stream) {
  return cce_forward_ex(dtype, e, c, bias, targets, ignore_index, has_ignore, N, D, V, tile_max, tile_sum_exp,
                        neg_target_logit, lse, nll, nullptr, 0, hip_stream);
}

int64_t cce_num_ref_tiles(int64_t V) { return V <= 0 ? 0 : (V + cce::kRefStatTile - 1) / cce::kRefStatTile; }

int cce_forward_ex(int dtype, const void* e, const void* c, const void* bias, const int64_t* targets,
                   int64_t ignore_index, int has_ignore, int64_t N, int64_t D, int64_t V, float* tile_max,
                   float* tile_sum_exp, float* neg_target_logit, float* lse, float* nll, void* zero_buf,
                   int64_t zero_bytes, void* hip_stream) {
  return forward_impl("cce_forward", dtype, e, c, bias, targets, ignore_index, has_ignore, N, D, V, tile_max,
                      tile_sum_exp, neg_target_logit, lse, nll, zero_buf, zero_bytes, 0, hip_stream);
}

int cce_forward_ref(int dtype, const void* e, const void* c, const void* bias, const int64_t* targets,
                    int64_t ignore_index, int has_ignore, int64_t N, int64_t D, int64_t V, float* tile_max,
                    float* tile_sum_exp, float* neg_target_logit, float* lse, float* nll, void* hip_stream) {
  return forward_impl("cce_forward_ref", dtype, e, c, bias, targets, ignore_index, has_ignore, N, D, V, tile_max,
                      tile_sum_exp, neg_target_logit, lse, nll, nullptr, 0, 1, hip_stream);
}

size_t cce_backward_workspace_size(int dtype, int64_t N, int64_t D, int64_t V, int want_dE, int want_dC,
                                   int want_dBias) {
  return cce_backward_workspace_size_ex(dtype, N, D, V, want_dE, want_dC, want_dBias, 0, 0);
}

size_t cce_backward_workspace_size_ex(int dtype, int64_t N, int64_t D, int64_t V, int want_dE, int want_dC,
                                      int want_dBias, int64_t max_g_tiles, int64_t max_chunk_tiles) {
  // the hi / lo pair's 64 KiB slots: enough for either layout
  return cce_backward_workspace_size_flags(dtype, N, D, V, want_dE, want_dC, want_dBias, max_g_tiles,
                                           max_chunk_tiles, -INFINITY, CCE_BWD_G_PAIR);
}

size_t cce_backward_workspace_size_flags(int dtype, int64_t N, int64_t D, int64_t V, int want_dE, int want_dC,
                                         int want_dBias, int64_t max_g_tiles, int64_t max_chunk_tiles,
                                         float filter_log_eps, int flags) {
  if (N <= 0 || D <= 0 || V <= 0 || max_g_tiles < 0 || max_chunk_tiles < 0 || max_chunk_tiles % 32 != 0) return 0;
  if (dtype != CCE_DTYPE_F32 && dtype != CCE_DTYPE_F16 && dtype != CCE_DTYPE_BF16) return 0;
  if (std::isnan(filter_log_eps) || !bwd_flags_valid(flags)) return 0;
  const size_t es = elem_size(dtype);
  return cce::make_bwd_plan(es, N, D, V, want_dE != 0, want_dC != 0, want_dBias != 0, max_chunk_tiles, false,
                            max_g_tiles, g_split_for(es, flags, filter_log_eps))
      .total_bytes;
}

int cce_backward(int dtype, const void* e, const void* c, const void* bias, const int64_t* targets,
                 int64_t ignore_index, int has_ignore, int64_t N, int64_t D, int64_t V, const float* lse,
                 const float* tile_max, const float* d_nll, float filter_log_eps, void* dE, void* dC, void* dBias,
                 void* workspace, size_t workspace_bytes, int64_t* tile_stats, void* hip_stream) {
  return cce_backward_ex(dtype, e, c, bias, targets, ignore_index, has_ignore, N, D, V, lse, tile_max, d_nll,
                         filter_log_eps, dE, dC, dBias, workspace, workspace_bytes, tile_stats, 0, 0, hip_stream);
}

}  // extern "C"

namespace {

// Pinned host ints the compaction writes the pass count into, and the event the host
// waits on for them: one set per host thread and device (a thread waits for its own
// call's count before it returns), grown as needed (a few KiB at most) and kept until
// the process ends.
hipError_t host_pass_buffer(size_t n, int** buf, hipEvent_t* ev) {
  struct Slot {
    int dev = -1;
    int* buf = nullptr;
    size_t n = 0;
    hipEvent_t ev = nullptr;
  };
  thread_local Slot slots[8];
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return err;
  Slot* sl = nullptr;
  for (Slot& x : slots)
    if (x.dev == dev || (sl == nullptr && x.dev < 0)) {
      sl = &x;
      if (x.dev == dev) break;
    }
  if (sl == nullptr) return hipErrorOutOfMemory;  // more devices than slots: the device-only schedule
  if (sl->ev == nullptr) {
    if ((err = hipEventCreateWithFlags(&sl->ev, hipEventDisableTiming)) != hipSuccess) return err;
    sl->dev = dev;
  }
  if (sl->n < n) {
    const size_t want = n < 256 ? 256 : n;
    int* p = nullptr;
    if ((err = hipHostMalloc(reinterpret_cast<void**>(&p), want * sizeof(int), hipHostMallocDefault)) != hipSuccess)
      return err;
    // the smaller buffer is not freed: a call that failed after queueing its compaction
    // may still have it written into
    sl->buf = p;
    sl->n = want;
  }
  *buf = sl->buf;
  *ev = sl->ev;
  return hipSuccess;
}

// The backward over plain (q == null) or quantized classifier rows.  Quantized rows
// reserve the scratch of one chunk in the workspace, and the chunks are capped at
// q->chunk_rows rows.
int backward_impl(int dtype, const void* e, const void* c, const void* bias, const int64_t* targets,
                  int64_t ignore_index, int has_ignore, int64_t N, int64_t D, int64_t V, const float* lse,
                  const float* tile_max, const float* d_nll, float filter_log_eps, void* dE, void* dC, void* dBias,
                  void* workspace, size_t workspace_bytes, int64_t* tile_stats, int flags, int64_t max_chunk_tiles,
                  const cce::QuantRows* q, void* hip_stream) {
  if (!lse || !tile_max || !d_nll)
    return fail(CCE_ERR_INVALID_ARGUMENT, "[cce_backward] lse, tile_max and d_nll must be non-null");
  if (dBias && !bias)
    return fail(CCE_ERR_INVALID_ARGUMENT, "[cce_backward] dBias requested but bias is null");
  if (bias && !aligned(bias, elem_size(dtype)))
    return fail(CCE_ERR_INVALID_ARGUMENT, "[cce_backward] bias is not aligned to its element size");
  if ((dE && !aligned(dE, 16)) || (dC && !aligned(dC, 16)) || (dBias && !aligned(dBias, 16)))
    return fail(CCE_ERR_INVALID_ARGUMENT, "[cce_backward] gradient outputs must be 16-byte aligned");
  if (std::isnan(filter_log_eps))
    return fail(CCE_ERR_INVALID_ARGUMENT, "[cce_backward] filter_log_eps must not be NaN");
  // The plan is a function of the sizes, the wanted outputs, the G tiles' layout (the
  // filter and the G flags) and the workspace size only: the default plan when the
  // workspace holds it, else smaller passes.
  const size_t es = elem_size(dtype);
  const bool g_split = g_split_for(es, flags, filter_log_eps);
  int64_t qcv = q ? q->chunk_rows / cce::kBwdVocab : 0;
  if (max_chunk_tiles > 0 && (qcv == 0 || max_chunk_tiles < qcv)) qcv = max_chunk_tiles;
  bool fits = false;
  const cce::BwdPlan P = cce::plan_for_workspace(es, N, D, V, dE != nullptr, dC != nullptr, dBias != nullptr, qcv,
                                                 q != nullptr, g_split, workspace ? workspace_bytes : 0, fits);
  if (!workspace || !fits) {
    const size_t least = cce::make_bwd_plan_cap(es, N, D, V, dE != nullptr, dC != nullptr, dBias != nullptr, 1, false,
                                                qcv, q != nullptr, g_split)
                             .total_bytes;
    return fail(CCE_ERR_WORKSPACE, "[cce_backward] workspace of %zu bytes required (at least %zu), %zu given",
                P.total_bytes, least, workspace ? workspace_bytes : (size_t)0);
  }
  if (!aligned(workspace, 256))
    return fail(CCE_ERR_WORKSPACE, "[cce_backward] workspace must be 256-byte aligned");
  const int cus = num_cus_current();
  if (cus <= 0) return fail(CCE_ERR_NO_DEVICE, "[cce_backward] no HIP device is available");

  hipStream_t s = reinterpret_cast<hipStream_t>(hip_stream);
  char* ws = reinterpret_cast<char*>(workspace);
  cce::BwdArgs a{};
  a.e = e;
  a.c = c;
  a.bias = bias;
  a.targets = targets;
  a.ignore_index = ignore_index;
  a.has_ignore = has_ignore ? 1 : 0;
  a.N = N;
  a.D = D;
  a.V = V;
  a.lse = lse;
  a.tile_max = tile_max;
  a.d_nll = d_nll;
  a.filter_log_eps = filter_log_eps;
  a.dE = dE;
  a.dC = dC;
  a.dBias = dBias;
  a.bits = reinterpret_cast<uint32_t*>(ws + P.bits);
  a.counts = reinterpret_cast<int*>(ws + P.counts);
  a.pinfo = reinterpret_cast<int*>(ws + P.pinfo);
  a.rb_start = reinterpret_cast<int*>(ws + P.rb_start);
  a.slot_vt = reinterpret_cast<int*>(ws + P.slot_vt);
  a.slot_rb = reinterpret_cast<int*>(ws + P.slot_rb);
  a.vt_start = reinterpret_cast<int*>(ws + P.vt_start);
  a.vt_slot = reinterpret_cast<int*>(ws + P.vt_slot);
  a.g_task = reinterpret_cast<int*>(ws + P.g_task);
  a.g_task_rb = reinterpret_cast<int*>(ws + P.g_task_rb);
  a.own_rb = reinterpret_cast<int*>(ws + P.own_rb);
  a.own_vt = reinterpret_cast<int*>(ws + P.own_vt);
  a.dc_bin_start = reinterpret_cast<int*>(ws + P.dc_bin_start);
  a.dc_bin_owner = reinterpret_cast<int*>(ws + P.dc_bin_owner);
  a.dc_blk_task = reinterpret_cast<int*>(ws + P.dc_blk_task);
  a.dc_blk_own = reinterpret_cast<int*>(ws + P.dc_blk_own);
  a.gtile = (dE || dC) ? ws + P.gtile : nullptr;
  a.colsum = dBias ? reinterpret_cast<float*>(ws + P.colsum) : nullptr;
  a.de_acc = P.carry ? reinterpret_cast<float*>(ws + P.de_acc) : nullptr;
  a.de_part = P.de_pieces && !(flags & CCE_BWD_DE_WHOLE_TASKS) ? reinterpret_cast<float*>(ws + P.de_part) : nullptr;
  if (P.perm_ok) {
    a.perm = reinterpret_cast<int*>(ws + P.perm);
    a.sort_buf = reinterpret_cast<uint32_t*>(ws + P.sort_buf);
    a.rowbits = reinterpret_cast<uint32_t*>(ws + P.rowbits);
    a.bits_p = reinterpret_cast<uint32_t*>(ws + P.bits_p);
    a.t_perm = reinterpret_cast<int64_t*>(ws + P.t_perm);
    a.lse_perm = reinterpret_cast<float*>(ws + P.lse_perm);
    a.dnll_perm = reinterpret_cast<float*>(ws + P.dnll_perm);
    a.e_perm = ws + P.e_perm;
  }
  a.perm_mode = (flags & CCE_BWD_TOKENS_INPUT) ? 1 : (flags & CCE_BWD_TOKENS_SORTED) ? 2 : 0;
  a.de_geo = (flags & CCE_BWD_DE_SUMS_WIDE) ? 1 : (flags & CCE_BWD_DE_SUMS_NARROW) ? 2 : 0;
  a.dc_geo = (flags & CCE_BWD_DC_SUMS_WIDE) ? 1 : (flags & CCE_BWD_DC_SUMS_NARROW) ? 2 : 0;
  a.tile_stats = tile_stats;
  a.dc_zeroed = (flags & CCE_BWD_DC_ZEROED) ? 1 : 0;
  a.stats32 = (flags & CCE_BWD_REF_STATS) ? 1 : 0;
  a.g_scaled = dtype == CCE_DTYPE_F16 ? 1 : 0;  // fp16 G tiles are scaled into fp16's normal range
  a.g_split = P.g_split ? 1 : 0;  // the layout the plan's slots are sized for
  // one-tile dC owners by token block: 16-bit inputs with G rounded once
  a.dc_blk = es == 2 && !a.g_split && dC != nullptr && P.nrb <= cce::kDcBlkMaxRb && !(flags & CCE_BWD_DC_OWNER_TASKS);
  a.g_tiles_ok = (flags & CCE_BWD_G_TASKS_BY_BLOCK) ? 0 : 1;
  a.plan = P;
  a.num_cus = cus;
  if (q) {
    a.q = *q;
    a.q.scratch = ws + P.qrows;
  }

  // The host waits for each chunk's pass count and launches exactly those passes,
  // unless told not to or the stream is being captured (a graph cannot wait).
  hipEvent_t pass_ev = nullptr;
  if (!(flags & CCE_BWD_DEVICE_PASSES)) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cap) == hipSuccess && cap == hipStreamCaptureStatusNone) {
      int* hp = nullptr;
      if (host_pass_buffer((size_t)P.max_passes + 1, &hp, &pass_ev) == hipSuccess) a.host_pass = hp;
    }
  }
  const hipError_t err = cce::launch_backward(dtype, a, s, a.host_pass ? pass_ev : nullptr);
  if (err != hipSuccess)
    return fail(CCE_ERR_LAUNCH, "[cce_backward] kernel launch failed: %s", hipGetErrorString(err));
  return CCE_OK;
}

}  // namespace

extern "C" {

int cce_backward_ex(int dtype, const void* e, const void* c, const void* bias, const int64_t* targets,
                    int64_t ignore_index, int has_ignore, int64_t N, int64_t D, int64_t V, const float* lse,
                    const float* tile_max, const float* d_nll, float filter_log_eps, void* dE, void* dC,
                    void* dBias, void* workspace, size_t workspace_bytes, int64_t* tile_stats, int flags,
                    int64_t max_chunk_tiles, void* hip_stream) {
  g_err[0] = 0;
  if (flags & ~kBwdFlags) return fail(CCE_ERR_INVALID_ARGUMENT, "[cce_backward] unknown flags 0x%x", flags);
  if ((flags & CCE_BWD_TOKENS_INPUT) && (flags & CCE_BWD_TOKENS_SORTED))
    return fail(CCE_ERR_INVALID_ARGUMENT, "[cce_backward] CCE_BWD_TOKENS_INPUT and CCE_BWD_TOKENS_SORTED exclude each other");
  if (((flags & CCE_BWD_DE_SUMS_WIDE) && (flags & CCE_BWD_DE_SUMS_NARROW)) ||
      ((flags & CCE_BWD_DC_SUMS_WIDE) && (flags & CCE_BWD_DC_SUMS_NARROW)))
    return fail(CCE_ERR_INVALID_ARGUMENT, "[cce_backward] a sums geometry flag pair excludes each other");
  if ((flags & CCE_BWD_G_PAIR) && (flags & CCE_BWD_G_SINGLE))
    return fail(CCE_ERR_INVALID_ARGUMENT, "[cce_backward] CCE_BWD_G_PAIR and CCE_BWD_G_SINGLE exclude each other");
  if (max_chunk_tiles < 0 || (max_chunk_tiles > 0 && max_chunk_tiles % 32 != 0))
    return fail(CCE_ERR_INVALID_ARGUMENT, "[cce_backward] max_chunk_tiles must be 0 or a positive multiple of 32, got %lld",
                (long long)max_chunk_tiles);
  const int rc = check_common("cce_backward", dtype, e, c, targets, N, D, V);
  if (rc != CCE_OK) return rc;
  return backward_impl(dtype, e, c, bias, targets, ignore_index, has_ignore, N, D, V, lse, tile_max, d_nll,
                       filter_log_eps, dE, dC, dBias, workspace, workspace_bytes, tile_stats, flags, max_chunk_tiles,
                       nullptr, hip_stream);
}

}  // extern "C"

namespace {

// Device address of `scratch` on each device, found once per device (with that
// device current) and kept: every GPU holds its own copy at its own address.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_of_current_device(const char* fn, void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0)
    return fail(CCE_ERR_NO_DEVICE, "[%s] no HIP device is available", fn);
  if (dev >= kMaxDevices) return fail(CCE_ERR_NO_DEVICE, "[%s] device %d is past the %d the library serves", fn, dev,
                                      kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || p == nullptr)
      return fail(CCE_ERR_NO_DEVICE, "[%s] hipGetSymbolAddress of the static scratch failed on device %d: %s", fn,
                  dev, hipGetErrorString(err));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return CCE_OK;
}

}  // namespace

extern "C" {

size_t cce_backward_noalloc_scratch_size(void) { return (size_t)CCE_NOALLOC_SCRATCH_BYTES; }

int cce_backward_noalloc(int dtype, const void* e, const void* c, const void* bias, const int64_t* targets,
                         int64_t ignore_index, int has_ignore, int64_t N, int64_t D, int64_t V, const float* lse,
                         const float* tile_max, const float* d_nll, float filter_log_eps, void* dE, void* dC,
                         void* dBias, int64_t* tile_stats, int flags, void* hip_stream) {
  g_err[0] = 0;
  if (flags & ~kBwdFlags)
    return fail(CCE_ERR_INVALID_ARGUMENT, "[cce_backward_noalloc] unknown flags 0x%x", flags);
  if (!bwd_flags_valid(flags))
    return fail(CCE_ERR_INVALID_ARGUMENT, "[cce_backward_noalloc] a pair of flags excludes each other");
  int rc = check_common("cce_backward_noalloc", dtype, e, c, targets, N, D, V);
  if (rc != CCE_OK) return rc;
  // Sizes beyond what the static scratch holds are refused before any device work.
  const size_t es = elem_size(dtype);
  const bool g_split = g_split_for(es, flags, filter_log_eps);
  bool fits = false;
  cce::plan_for_workspace(es, N, D, V, dE != nullptr, dC != nullptr, dBias != nullptr, 0, false, g_split,
                          (size_t)CCE_NOALLOC_SCRATCH_BYTES, fits);
  if (!fits) {
    const size_t least =
        cce::make_bwd_plan_cap(es, N, D, V, dE != nullptr, dC != nullptr, dBias != nullptr, 1, false, 0, false, g_split)
            .total_bytes;
    return fail(CCE_ERR_WORKSPACE,
                "[cce_backward_noalloc] N=%lld D=%lld V=%lld needs at least %zu bytes of workspace; the static scratch "
                "holds %zu (call cce_backward with a workspace instead)",
                (long long)N, (long long)D, (long long)V, least, (size_t)CCE_NOALLOC_SCRATCH_BYTES);
  }
  void* ws = nullptr;
  if ((rc = scratch_of_current_device("cce_backward_noalloc", &ws)) != CCE_OK) return rc;
  // no host wait for the pass count (its pinned buffer would be an allocation)
  return backward_impl(dtype, e, c, bias, targets, ignore_index, has_ignore, N, D, V, lse, tile_max, d_nll,
                       filter_log_eps, dE, dC, dBias, ws, (size_t)CCE_NOALLOC_SCRATCH_BYTES, tile_stats,
                       flags | CCE_BWD_DEVICE_PASSES, 0, nullptr, hip_stream);
}

int cce_dequantize(int dtype, const uint32_t* weight, const void* scales, const void* qbiases, int group_size,
                   int bits, int64_t rows, int64_t D, void* out, void* hip_stream) {
  g_err[0] = 0;
  if (dtype != CCE_DTYPE_F32 && dtype != CCE_DTYPE_F16 && dtype != CCE_DTYPE_BF16)
    return fail(CCE_ERR_UNSUPPORTED_DTYPE, "[cce_dequantize] unsupported dtype code %d", dtype);
  if (rows <= 0 || D <= 0 || rows >= ((int64_t)1 << 31))
    return fail(CCE_ERR_INVALID_ARGUMENT, "[cce_dequantize] rows and D must be positive (rows below 2^31), got %lld, %lld",
                (long long)rows, (long long)D);
  int rc = check_quant("cce_dequantize", dtype, weight, scales, qbiases, group_size, bits, D);
  if (rc != CCE_OK) return rc;
  if (!out || !aligned(out, 16)) return fail(CCE_ERR_INVALID_ARGUMENT, "[cce_dequantize] out must be 16-byte aligned");
  if (num_cus_current() <= 0) return fail(CCE_ERR_NO_DEVICE, "[cce_dequantize] no HIP device is available");
  cce::QuantRows q{weight, scales, qbiases, group_size, bits, nullptr, 0};
  const hipError_t err = cce::launch_dequantize(dtype, q, 0, rows, D, out, reinterpret_cast<hipStream_t>(hip_stream));
  if (err != hipSuccess)
    return fail(CCE_ERR_LAUNCH, "[cce_dequantize] kernel launch failed: %s", hipGetErrorString(err));
  return CCE_OK;
}

size_t cce_forward_q_scratch_size(int dtype, int64_t V, int64_t D, int64_t chunk_rows) {
  if (V <= 0 || D <= 0 || chunk_rows < 0 || chunk_rows % cce::kQuantChunkAlign != 0) return 0;
  if (dtype != CCE_DTYPE_F32 && dtype != CCE_DTYPE_F16 && dtype != CCE_DTYPE_BF16) return 0;
  const int64_t rows = quant_chunk_rows(chunk_rows) < V ? quant_chunk_rows(chunk_rows) : V;
  return (size_t)rows * (size_t)D * elem_size(dtype);
}

int cce_forward_q(int dtype, const void* e, const uint32_t* weight, const void* scales, const void* qbiases,
                  int group_size, int bits, const void* bias, const int64_t* targets, int64_t ignore_index,
                  int has_ignore, int64_t N, int64_t D, int64_t V, float* tile_max, float* tile_sum_exp,
                  float* neg_target_logit, float* lse, float* nll, void* scratch, size_t scratch_bytes,
                  int64_t chunk_rows, void* hip_stream) {
  g_err[0] = 0;
  // c is not read on this path: check the shapes with e standing in for it
  int rc = check_common("cce_forward_q", dtype, e, e, targets, N, D, V);
  if (rc != CCE_OK) return rc;
  if ((rc = check_quant("cce_forward_q", dtype, weight, scales, qbiases, group_size, bits, D)) != CCE_OK) return rc;
  if ((rc = check_chunk_rows("cce_forward_q", chunk_rows)) != CCE_OK) return rc;
  if (!tile_max || !tile_sum_exp || !neg_target_logit || !lse || !nll)
    return fail(CCE_ERR_INVALID_ARGUMENT,
                "[cce_forward_q] tile_max, tile_sum_exp, neg_target_logit, lse and nll must be non-null");
  if (bias && !aligned(bias, elem_size(dtype)))
    return fail(CCE_ERR_INVALID_ARGUMENT, "[cce_forward_q] bias is not aligned to its element size");
  const size_t need = cce_forward_q_scratch_size(dtype, V, D, chunk_rows);
  if (!scratch || scratch_bytes < need || !aligned(scratch, 256))
    return fail(CCE_ERR_WORKSPACE, "[cce_forward_q] scratch of %zu bytes (256-byte aligned) required, %zu given", need,
                scratch ? scratch_bytes : (size_t)0);
  const int cus = num_cus_current();
  if (cus <= 0) return fail(CCE_ERR_NO_DEVICE, "[cce_forward_q] no HIP device is available");

  cce::FwdArgs a{};
  a.e = e;
  a.c = nullptr;
  a.bias = bias;
  a.targets = targets;
  a.ignore_index = ignore_index;
  a.has_ignore = has_ignore ? 1 : 0;
  a.N = N;
  a.D = D;
  a.V = V;
  a.tile_max = tile_max;
  a.tile_sum_exp = tile_sum_exp;
  a.neg_target_logit = neg_target_logit;
  a.lse = lse;
  a.nll = nll;
  a.num_cus = cus;
  cce::QuantRows q{weight, scales, qbiases, group_size, bits, scratch, quant_chunk_rows(chunk_rows)};
  const hipError_t err = cce::launch_forward_q(dtype, a, q, reinterpret_cast<hipStream_t>(hip_stream));
  if (err != hipSuccess)
    return fail(CCE_ERR_LAUNCH, "[cce_forward_q] kernel launch failed: %s", hipGetErrorString(err));
  return CCE_OK;
}

size_t cce_backward_q_workspace_size(int dtype, int64_t N, int64_t D, int64_t V, int want_dE, int want_dBias,
                                     int64_t chunk_rows) {
  if (N <= 0 || D <= 0 || V <= 0 || chunk_rows < 0 || chunk_rows % cce::kQuantChunkAlign != 0) return 0;
  if (dtype != CCE_DTYPE_F32 && dtype != CCE_DTYPE_F16 && dtype != CCE_DTYPE_BF16) return 0;
  // the hi / lo pair's 64 KiB slots: enough for either layout
  return cce::make_bwd_plan(elem_size(dtype), N, D, V, want_dE != 0, false, want_dBias != 0,
                            quant_chunk_rows(chunk_rows) / cce::kBwdVocab, true, 0, true)
      .total_bytes;
}

int cce_backward_q(int dtype, const void* e, const uint32_t* weight, const void* scales, const void* qbiases,
                   int group_size, int bits, const void* bias, const int64_t* targets, int64_t ignore_index,
                   int has_ignore, int64_t N, int64_t D, int64_t V, const float* lse, const float* tile_max,
                   const float* d_nll, float filter_log_eps, void* dE, void* dBias, void* workspace,
                   size_t workspace_bytes, int64_t chunk_rows, int64_t* tile_stats, void* hip_stream) {
  g_err[0] = 0;
  int rc = check_common("cce_backward_q", dtype, e, e, targets, N, D, V);
  if (rc != CCE_OK) return rc;
  if ((rc = check_quant("cce_backward_q", dtype, weight, scales, qbiases, group_size, bits, D)) != CCE_OK) return rc;
  if ((rc = check_chunk_rows("cce_backward_q", chunk_rows)) != CCE_OK) return rc;
  cce::QuantRows q{weight, scales, qbiases, group_size, bits, nullptr, quant_chunk_rows(chunk_rows)};
  return backward_impl(dtype, e, nullptr, bias, targets, ignore_index, has_ignore, N, D, V, lse, tile_max, d_nll,
                       filter_log_eps, dE, nullptr, dBias, workspace, workspace_bytes, tile_stats, 0, 0, &q,
                       hip_stream);
}

int cce_reduce_loss(const float* nll, const int64_t* targets, int64_t ignore_index, int has_ignore, int64_t N,
                    int mode, float* loss_out, float* scale_out, void* hip_stream) {
  g_err[0] = 0;
  if (N <= 0) return fail(CCE_ERR_INVALID_ARGUMENT, "[cce_reduce_loss] N must be positive, got %lld", (long long)N);
  if (mode != CCE_REDUCE_SUM && mode != CCE_REDUCE_MEAN)
    return fail(CCE_ERR_INVALID_ARGUMENT, "[cce_reduce_loss] mode must be CCE_REDUCE_SUM or CCE_REDUCE_MEAN, got %d",
                mode);
  if (!nll || !loss_out || (has_ignore && !targets))
    return fail(CCE_ERR_INVALID_ARGUMENT, "[cce_reduce_loss] nll, loss_out (and targets with has_ignore) must be non-null");
  if (num_cus_current() <= 0) return fail(CCE_ERR_NO_DEVICE, "[cce_reduce_loss] no HIP device is available");
  const hipError_t err = cce::launch_reduce_loss(nll, targets, ignore_index, has_ignore, N, mode, loss_out, scale_out,
                                                 reinterpret_cast<hipStream_t>(hip_stream));
  if (err != hipSuccess)
    return fail(CCE_ERR_LAUNCH, "[cce_reduce_loss] kernel launch failed: %s", hipGetErrorString(err));
  return CCE_OK;
}

int cce_broadcast_grad(const float* grad, const float* scale, int64_t N, float* d_nll, void* hip_stream) {
  g_err[0] = 0;
  if (N <= 0) return fail(CCE_ERR_INVALID_ARGUMENT, "[cce_broadcast_grad] N must be positive, got %lld", (long long)N);
  if (!grad || !d_nll) return fail(CCE_ERR_INVALID_ARGUMENT, "[cce_broadcast_grad] grad and d_nll must be non-null");
  if (num_cus_current() <= 0) return fail(CCE_ERR_NO_DEVICE, "[cce_broadcast_grad] no HIP device is available");
  const hipError_t err = cce::launch_broadcast_grad(grad, scale, N, d_nll, reinterpret_cast<hipStream_t>(hip_stream));
  if (err != hipSuccess)
    return fail(CCE_ERR_LAUNCH, "[cce_broadcast_grad] kernel launch failed: %s", hipGetErrorString(err));
  return CCE_OK;
}

}  // extern "C"
