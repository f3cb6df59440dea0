// cce_quant.hip — dequantization of affine group-quantized classifier rows.
//
// Layout and formula follow MLX's affine quantization (mx.quantize / mx.dequantize,
// mlx >= 0.22; the reference's callers dequantize the lm_head / tied embedding
// with it before calling the loss: README.md:90-95, examples/mlx_lm_lora_test.py:
// 16-21): a row of D codes is D * bits / 32 uint32 words, code j of a word in bits
// [j * bits, (j + 1) * bits); every group_size consecutive codes share a scale and
// a bias, stored in the compute dtype; w = scale * q + bias.
//
// Rounding: the product scale * q is formed in fp32 (exact for 16-bit scales and
// codes below 256), the bias added in fp32 (one rounding), and the sum rounded to
// the output dtype to nearest-even.  The passes over quantized rows use these
// values, so they equal the passes over this kernel's output bit for bit.
//
// One thread per word: each thread writes 32 / bits consecutive elements of a row
// (16 bytes for 4-bit codes and 16-bit output).  HBM-bound: per element, bits / 8
// bytes of codes plus the shared scale and bias are read and sizeof(T) written.
#include "cce_device.h"
#include "cce_launch.h"

namespace cce {

template <typename T>
__device__ __forceinline__ T from_f32(float x) {
  return static_cast<T>(x);
}

// scale * q + bias with the product and the add rounded separately (no fma).
__device__ __forceinline__ float affine(float s, float q, float b) {
#pragma clang fp contract(off)
  return s * q + b;
}

// Rows are blockIdx.x (chunk-local); words of a row are split over blockIdx.y.  W
// (words per row) and G (groups per row) come from the host and group_size is a power
// of two, so the indexing needs no 64-bit division.  keep (or null: every row): the
// backward's per-tile table of the chunk (vt_start), rows of 128-row tiles without kept
// pairs are skipped -- nothing reads them.
template <typename T, int BITS>
__global__ __launch_bounds__(256) void dequant_kernel(const uint32_t* __restrict__ wq, const T* __restrict__ scales,
                                                      const T* __restrict__ biases, int W, int G, int gshift,
                                                      int64_t D, T* __restrict__ out, const int* __restrict__ keep) {
  constexpr int EPW = 32 / BITS;  // codes per word
  typedef T vec_t __attribute__((ext_vector_type(EPW)));
  const int w = (int)blockIdx.y * 256 + (int)threadIdx.x;
  if (w >= W) return;
  const int64_t r = blockIdx.x;
  if (keep != nullptr && ldu(keep, (int)(r >> 7) + 1) == ldu(keep, (int)(r >> 7))) return;
  const uint32_t word = wq[r * W + w];
  const int d0 = w * EPW;
  const float s = to_f32(scales[r * G + (d0 >> gshift)]);
  const float b = to_f32(biases[r * G + (d0 >> gshift)]);
  vec_t v;
#pragma unroll
  for (int j = 0; j < EPW; ++j) {
    const uint32_t q = (word >> (BITS * j)) & ((1u << BITS) - 1u);
    v[j] = from_f32<T>(affine(s, (float)q, b));
  }
  *reinterpret_cast<vec_t*>(out + r * D + d0) = v;
}

template <typename T>
static hipError_t dequantize_typed(const QuantRows& q, int64_t row0, int64_t rows, int64_t D, void* out,
                                   const int* keep, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  const int64_t words = D * q.bits / 32;  // D < 2^22 elements (8 MiB rows): fits int
  const dim3 grid((unsigned)rows, (unsigned)((words + 255) / 256));
  const uint32_t* wq = q.wq + row0 * words;
  const int64_t g = D / q.group_size;
  const int gshift = q.group_size == 32 ? 5 : q.group_size == 64 ? 6 : 7;
  const T* sc = reinterpret_cast<const T*>(q.scales) + row0 * g;
  const T* bi = reinterpret_cast<const T*>(q.biases) + row0 * g;
  T* o = reinterpret_cast<T*>(out);
  const int W = (int)words, G = (int)g;
  switch (q.bits) {
    case 2:
      hipLaunchKernelGGL((dequant_kernel<T, 2>), grid, dim3(256), 0, s, wq, sc, bi, W, G, gshift, D, o, keep);
      break;
    case 4:
      hipLaunchKernelGGL((dequant_kernel<T, 4>), grid, dim3(256), 0, s, wq, sc, bi, W, G, gshift, D, o, keep);
      break;
    case 8:
      hipLaunchKernelGGL((dequant_kernel<T, 8>), grid, dim3(256), 0, s, wq, sc, bi, W, G, gshift, D, o, keep);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_dequantize(int dtype, const QuantRows& q, int64_t row0, int64_t rows, int64_t D, void* out,
                             hipStream_t s, const int* keep) {
  switch (dtype) {
    case 0:
      return dequantize_typed<float>(q, row0, rows, D, out, keep, s);
    case 1:
      return dequantize_typed<_Float16>(q, row0, rows, D, out, keep, s);
    default:
      return dequantize_typed<__bf16>(q, row0, rows, D, out, keep, s);
  }
}

}  // namespace cce
