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

// GELU with the exact-erf definition nn.functional.gelu(approximate="none")
// uses, gelu(x) = x * Phi(x) = x * (1 + erf(x / sqrt 2)) / 2, where erf comes
// from Abramowitz & Stegun, Handbook of Mathematical Functions, eq. 7.1.26:
//   erfc(z) ~= (a1 t + a2 t^2 + a3 t^3 + a4 t^4 + a5 t^5) exp(-z^2),
//   t = 1 / (1 + p z), z >= 0, |error| <= 1.5e-7,
// evaluated with one reciprocal and one exp2 (about 14 VALU instructions
// instead of a full-range erff).  The result feeds an FP16 store, whose
// rounding (2^-11 relative) is far above this approximation error.
__device__ __forceinline__ float gelu_erf(float x) {
  constexpr float kP = 0.3275911f * 0.70710678118654752440f;  // p / sqrt 2, z = |x| / sqrt 2
  constexpr float a1 = 0.254829592f, a2 = -0.284496736f, a3 = 1.421413741f;
  constexpr float a4 = -1.453152027f, a5 = 1.061405429f;
  const float t = __builtin_amdgcn_rcpf(fmaf(fabsf(x), kP, 1.0f));
  const float poly = t * fmaf(fmaf(fmaf(fmaf(a5, t, a4), t, a3), t, a2), t, a1);
  // exp(-z^2) = exp(-x^2 / 2) = 2^(-x^2 * log2(e) / 2)
  const float half_erfc = 0.5f * poly * __builtin_amdgcn_exp2f(x * x * -0.72134752044448170368f);
  const float phi = x >= 0.f ? 1.0f - half_erfc : half_erfc;
  return x * phi;
}

}  // namespace xb
