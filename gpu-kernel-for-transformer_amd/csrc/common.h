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
// evaluated with one reciprocal and one exp2 (about 13 VALU instructions
// instead of a full-range erff).  The result feeds an FP16 store, whose
// rounding (2^-11 relative) is far above this approximation error.
__device__ __forceinline__ float gelu_erf(float x) {
  constexpr float kP = 0.3275911f * 0.70710678118654752440f;  // p / sqrt 2, z = |x| / sqrt 2
  // A&S coefficients halved: h = 0.5 erfc(|x| / sqrt 2) = t (b1 + t (b2 + ...)) exp(-x^2 / 2)
  constexpr float b1 = 0.5f * 0.254829592f, b2 = 0.5f * -0.284496736f, b3 = 0.5f * 1.421413741f;
  constexpr float b4 = 0.5f * -1.453152027f, b5 = 0.5f * 1.061405429f;
  const float ax = fabsf(x);
  const float t = __builtin_amdgcn_rcpf(fmaf(ax, kP, 1.0f));
  const float poly = t * fmaf(fmaf(fmaf(fmaf(b5, t, b4), t, b3), t, b2), t, b1);
  // exp(-z^2) = exp(-x^2 / 2) = 2^(-x^2 * log2(e) / 2)
  const float h = poly * __builtin_amdgcn_exp2f(x * x * -0.72134752044448170368f);
  // x Phi(x) is x (1 - h) for x >= 0 and x h below: max(x, 0) - |x| h
  return fmaf(-ax, h, fmaxf(x, 0.f));
}

// Cross-lane reductions over lanes l, l^16, l^32, l^48 with the gfx950 lane
// swaps (VALU, no LDS round trip).  With both operands equal to v,
// v_permlane16_swap leaves {v, v[l^16]} and v_permlane32_swap {v, v[l^32]}
// in its two results, in some order per lane.
__device__ __forceinline__ float xor16_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor16_max(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// Sum / max over the four 16-lane groups (lanes with the same l % 16).
__device__ __forceinline__ float quad_group_sum(float v) { return xor32_sum(xor16_sum(v)); }
__device__ __forceinline__ float quad_group_max(float v) { return xor32_max(xor16_max(v)); }

}  // namespace xb
