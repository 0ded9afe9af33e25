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
// uses, gelu(x) = x * Phi(x).  Phi is approximated by a logistic function of
// an odd quintic,
//   Phi(x) ~= 1 / (1 + exp(-(c1 x + c3 x^3 + c5 x^5))),
// the structure of the well-known tanh form (Hendrycks & Gimpel 2016, which
// is the x, x^3 truncation with max |error| 3.8e-4) with one more term and
// the three coefficients fitted here for the smallest maximum of
// |x Phi~(x) - x Phi(x)| on a dense grid over [-5, 5].  The polynomial's
// argument is clamped to [-9, 9], where the logistic is within 2e-12 of 0
// or 1 and monotone, so large |x| stay exact.  Max abs error 2.6e-5 in FP32
// (a twentieth of the FP16 rounding of a stored activation near 1), for one
// clamp, four VALU operations, exp2 and a reciprocal.
__device__ __forceinline__ float gelu_erf(float x) {
  // -c * log2(e): the exponent is evaluated base 2.
  constexpr float k1 = -1.59501577f * 1.44269504088896340736f;
  constexpr float k3 = -0.0740112920f * 1.44269504088896340736f;
  constexpr float k5 = 7.03033577e-4f * 1.44269504088896340736f;
  const float xc = __builtin_amdgcn_fmed3f(x, -9.0f, 9.0f);
  const float x2 = xc * xc;
  const float u = xc * fmaf(x2, fmaf(x2, k5, k3), k1);
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(u));
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

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void global_void_t;

// One 16-byte-per-lane direct global -> LDS load (global_load_lds_dwordx4):
// lane i's bytes land at lds_wave_base + 16 i.  The LDS base must be
// wave-uniform; completion is counted by vmcnt.
__device__ __forceinline__ void dma16(const void* src_lane, void* lds_wave_base) {
  __builtin_amdgcn_global_load_lds((global_void_t*)src_lane, (lds_void_t*)lds_wave_base, 16, 0, 0);
}

}  // namespace xb
