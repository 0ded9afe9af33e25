// Shared device types and helpers for the gfx950 (CDNA4) kernels of the causal
// pre-norm Transformer block.  Everything here is wave64 / MFMA specific.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace xb {

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));

constexpr int kWave = 64;

// v_mfma_f32_16x16x32_f16 (gfx950).  Lane layout, checked on the device:
//   A[16][32]: lane l holds A[l % 16][(l / 16) * 8 + m], m = 0..7
//   B[32][16]: lane l holds B[(l / 16) * 8 + m][l % 16]
//   D[16][16]: lane l holds D[(l / 16) * 4 + i][l % 16], i = 0..3
// Only the pairing of A's and B's k index matters for the product, so callers
// may permute k as long as both operands use the same permutation.
__device__ __forceinline__ float4_t mfma16x16x32(half8_t a, half8_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Wave-level butterfly reductions over groups of `width` consecutive lanes.
template <int width>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int off = width / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, width);
  return v;
}

template <int width>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int off = width / 2; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, width));
  return v;
}

// Exact-erf GELU, the formula nn.functional.gelu(approximate="none") uses.
__device__ __forceinline__ float gelu_erf(float x) {
  return 0.5f * x * (1.0f + erff(x * 0.70710678118654752440f));
}

}  // namespace xb
