// LayerNorm and fused residual-add + LayerNorm for gfx950.
//
// Math follows triton_fused_norm.py:37-121: FP32 sum of the row, mean = sum/D,
// biased variance of the centred row, y = (x - mean) * rsqrt(var + eps), with
// the optional affine transform.  The reference launches one program per row
// (triton_fused_norm.py:159-169); here a row belongs to a group of LPR lanes of
// one wave, each lane owning 4 (rows of 256 columns and more) or 8 consecutive
// columns per chunk, so every global access is an 8- to 32-byte vector, and
// both reductions are wave shuffles.
#include <type_traits>

#include "common.h"
#include "../../include/xblock.h"

namespace xb {

template <typename T>
struct Vec8;

template <>
struct Vec8<float> {
  __device__ static void load(const float* p, float v[8]) {
    float4_t a = *reinterpret_cast<const float4_t*>(p);
    float4_t b = *reinterpret_cast<const float4_t*>(p + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) { v[i] = a[i]; v[4 + i] = b[i]; }
  }
  __device__ static void store(float* p, const float v[8]) {
    float4_t a, b;
#pragma unroll
    for (int i = 0; i < 4; ++i) { a[i] = v[i]; b[i] = v[4 + i]; }
    *reinterpret_cast<float4_t*>(p) = a;
    *reinterpret_cast<float4_t*>(p + 4) = b;
  }
};

template <>
struct Vec8<half_t> {
  __device__ static void load(const half_t* p, float v[8]) {
    half8_t a = *reinterpret_cast<const half8_t*>(p);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (float)a[i];
  }
  __device__ static void store(half_t* p, const float v[8]) {
    half8_t a;
#pragma unroll
    for (int i = 0; i < 8; ++i) a[i] = (half_t)v[i];
    *reinterpret_cast<half8_t*>(p) = a;
  }
};

template <typename T>
struct Vec4;

template <>
struct Vec4<float> {
  __device__ static void load(const float* p, float v[4]) {
    const float4_t a = *reinterpret_cast<const float4_t*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = a[i];
  }
  __device__ static void store(float* p, const float v[4]) {
    *reinterpret_cast<float4_t*>(p) = float4_t{v[0], v[1], v[2], v[3]};
  }
};

template <>
struct Vec4<half_t> {
  __device__ static void load(const half_t* p, float v[4]) {
    const half4_t a = *reinterpret_cast<const half4_t*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = (float)a[i];
  }
  __device__ static void store(half_t* p, const float v[4]) {
    *reinterpret_cast<half4_t*>(p) = half4_t{(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3]};
  }
};

// A lane's VEC consecutive columns per chunk (VEC = 4 or 8).
template <int VEC, typename T>
using VecIO = typename std::conditional<VEC == 8, Vec8<T>, Vec4<T>>::type;

// D = CH * LPR * VEC columns (chunk c of lane l: columns VEC (c LPR + l) on);
// 256 / LPR rows per 256-thread block.
// RES: add `upd` to `x` first and (when res_out != nullptr) store the sum.
// row_valid (optional, one byte per row) with mask_mode bits
// XB_MASK_UPDATE / XB_MASK_SUM / XB_MASK_OUTPUT zeroes, for rows whose byte
// is 0, the update, the sum (stored residual and LayerNorm input), or the
// output (by selection, so NaN in a masked update does not leak).
template <int D, int LPR, int VEC, bool RES, typename TU, typename TY>
__global__ __launch_bounds__(256) void ln_rows_kernel(
    const float* x, const TU* __restrict__ upd,
    const float* __restrict__ gamma, const float* __restrict__ beta,
    float* res_out, TY* __restrict__ y, int64_t rows, float eps, int affine,
    const uint8_t* __restrict__ row_valid, int mask_mode) {
  constexpr int CH = D / (LPR * VEC);
  static_assert(CH * LPR * VEC == D, "row width must split into VEC-column lanes");
  constexpr int RPB = 256 / LPR;
  const int lr = threadIdx.x % LPR;
  const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / LPR;
  // Every lane of a row group takes the same branch, so the width-LPR
  // shuffles below only ever read lanes that are still active.
  if (row >= rows) return;
  const bool invalid = row_valid != nullptr && row_valid[row] == 0;
  const bool drop_update = invalid && (mask_mode & XB_MASK_UPDATE);
  const bool drop_sum = invalid && (mask_mode & XB_MASK_SUM);
  const bool drop_out = invalid && (mask_mode & XB_MASK_OUTPUT);

  float v[CH][VEC];
  const float* xr = x + row * D;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int col = (c * LPR + lr) * VEC;
    VecIO<VEC, float>::load(xr + col, v[c]);
    if constexpr (RES) {
      if (!drop_update) {
        float u[VEC];
        VecIO<VEC, TU>::load(upd + row * D + col, u);
#pragma unroll
        for (int i = 0; i < VEC; ++i) v[c][i] += u[i];
      }
    }
    if (drop_sum) {
#pragma unroll
      for (int i = 0; i < VEC; ++i) v[c][i] = 0.f;
    }
  }
  if constexpr (RES) {
    if (res_out != nullptr) {
#pragma unroll
      for (int c = 0; c < CH; ++c) VecIO<VEC, float>::store(res_out + row * D + (c * LPR + lr) * VEC, v[c]);
    }
  }

  float s = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c)
#pragma unroll
    for (int i = 0; i < VEC; ++i) s += v[c][i];
  const float mean = group_sum<LPR>(s) * (1.0f / D);
  float q = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c)
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      v[c][i] -= mean;
      q += v[c][i] * v[c][i];
    }
  const float rstd = rsqrtf(group_sum<LPR>(q) * (1.0f / D) + eps);

#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int col = (c * LPR + lr) * VEC;
    float o[VEC];
    if (affine) {
      float g[VEC], b[VEC];
      VecIO<VEC, float>::load(gamma + col, g);
      VecIO<VEC, float>::load(beta + col, b);
#pragma unroll
      for (int i = 0; i < VEC; ++i) o[i] = v[c][i] * rstd * g[i] + b[i];
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) o[i] = v[c][i] * rstd;
    }
    if (drop_out) {
#pragma unroll
      for (int i = 0; i < VEC; ++i) o[i] = 0.f;
    }
    VecIO<VEC, TY>::store(y + row * D + col, o);
  }
}

// Any width: one 256-thread block per row, block-level reductions in LDS.
template <bool RES, typename TU, typename TY>
__global__ __launch_bounds__(256) void ln_generic_kernel(
    const float* x, const TU* __restrict__ upd,
    const float* __restrict__ gamma, const float* __restrict__ beta,
    float* res_out, TY* __restrict__ y, int cols, float eps, int affine,
    const uint8_t* __restrict__ row_valid, int mask_mode) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const float* xr = x + row * cols;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const bool invalid = row_valid != nullptr && row_valid[row] == 0;
  const bool drop_update = invalid && (mask_mode & XB_MASK_UPDATE);
  const bool drop_sum = invalid && (mask_mode & XB_MASK_SUM);
  const bool drop_out = invalid && (mask_mode & XB_MASK_OUTPUT);

  float s = 0.f;
  for (int c = threadIdx.x; c < cols; c += 256) {
    float v = xr[c];
    if constexpr (RES) {
      if (!drop_update) v += (float)upd[row * cols + c];
      if (drop_sum) v = 0.f;
      if (res_out != nullptr) res_out[row * cols + c] = v;
    } else {
      if (drop_sum) v = 0.f;
    }
    s += v;
  }
  s = group_sum<kWave>(s);
  if (lane == 0) red[wave] = s;
  __syncthreads();
  const float mean = (red[0] + red[1] + red[2] + red[3]) / cols;
  __syncthreads();

  // Later passes re-read the summed row; when res_out is set (possibly
  // aliasing x) it already holds the sum this thread wrote in pass one.
  auto summed = [&](int c) -> float {
    if (drop_sum) return 0.f;
    if constexpr (RES) {
      if (res_out != nullptr) return res_out[row * cols + c];
      return drop_update ? xr[c] : xr[c] + (float)upd[row * cols + c];
    } else {
      return xr[c];
    }
  };
  float q = 0.f;
  for (int c = threadIdx.x; c < cols; c += 256) {
    float v = summed(c) - mean;
    q += v * v;
  }
  q = group_sum<kWave>(q);
  if (lane == 0) red[wave] = q;
  __syncthreads();
  const float rstd = rsqrtf((red[0] + red[1] + red[2] + red[3]) / cols + eps);

  for (int c = threadIdx.x; c < cols; c += 256) {
    float o = (summed(c) - mean) * rstd;
    if (affine) o = o * gamma[c] + beta[c];
    if (drop_out) o = 0.f;
    y[row * cols + c] = (TY)o;
  }
}

// Rows of 256 columns and more: 4-column lanes (FP32 rows 1 KB and up:
// 8192 x 1024 residual + LayerNorm 17.6 -> 16.5 us, 3.2M x 1024 7.5 -> 7.1 ms
// against 8-column lanes); shorter rows keep 8-column lanes (D = 128: 331
// against 337 us for 1.28M rows).
template <int D, int LPR, bool RES, typename TU, typename TY>
static hipError_t launch_rows(const float* x, const void* upd, const float* g,
                              const float* b, float* res_out, void* y,
                              int64_t rows, float eps, int affine,
                              const uint8_t* rv, int mm, hipStream_t s) {
  constexpr int RPB = 256 / LPR;
  const int64_t blocks = (rows + RPB - 1) / RPB;
  constexpr int VEC = D >= 256 ? 4 : 8;
  hipLaunchKernelGGL((ln_rows_kernel<D, LPR, VEC, RES, TU, TY>), dim3((unsigned)blocks),
                     dim3(256), 0, s, x, static_cast<const TU*>(upd), g, b,
                     res_out, static_cast<TY*>(y), rows, eps, affine, rv, mm);
  return hipGetLastError();
}

template <bool RES, typename TU, typename TY>
static hipError_t dispatch_width(const float* x, const void* upd, const float* g,
                                 const float* b, float* res_out, void* y,
                                 int64_t rows, int cols, float eps, int affine,
                                 hipStream_t s, const uint8_t* rv = nullptr, int mm = 0) {
  switch (cols) {
    case 64: return launch_rows<64, 8, RES, TU, TY>(x, upd, g, b, res_out, y, rows, eps, affine, rv, mm, s);
    case 128: return launch_rows<128, 16, RES, TU, TY>(x, upd, g, b, res_out, y, rows, eps, affine, rv, mm, s);
    case 256: return launch_rows<256, 32, RES, TU, TY>(x, upd, g, b, res_out, y, rows, eps, affine, rv, mm, s);
    case 512: return launch_rows<512, 64, RES, TU, TY>(x, upd, g, b, res_out, y, rows, eps, affine, rv, mm, s);
    case 1024: return launch_rows<1024, 64, RES, TU, TY>(x, upd, g, b, res_out, y, rows, eps, affine, rv, mm, s);
    case 2048: return launch_rows<2048, 64, RES, TU, TY>(x, upd, g, b, res_out, y, rows, eps, affine, rv, mm, s);
    default:
      hipLaunchKernelGGL((ln_generic_kernel<RES, TU, TY>), dim3((unsigned)rows), dim3(256), 0, s,
                         x, static_cast<const TU*>(upd), g, b, res_out, static_cast<TY*>(y),
                         cols, eps, affine, rv, mm);
      return hipGetLastError();
  }
}

static bool vector_width(int cols) {
  return cols == 64 || cols == 128 || cols == 256 || cols == 512 || cols == 1024 || cols == 2048;
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace xb

using namespace xb;

extern "C" int xb_layernorm(const float* x, const float* gamma, const float* beta, void* y,
                            int y_dtype, int64_t rows, int32_t cols, float eps,
                            int apply_affine, void* stream) {
  if (rows < 0 || cols <= 0 || rows > 0x7fffffffLL) return XB_ERR_BAD_SIZE;
  if (y_dtype != XB_F32 && y_dtype != XB_F16) return XB_ERR_BAD_DTYPE;
  if (rows == 0) return XB_OK;  // empty tensors may carry NULL data pointers
  if (!x || !y || (apply_affine && (!gamma || !beta))) return XB_ERR_NULL_POINTER;
  if (vector_width(cols) && (!aligned16(x) || !aligned16(y) ||
                             (apply_affine && (!aligned16(gamma) || !aligned16(beta)))))
    return XB_ERR_MISALIGNED;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e = y_dtype == XB_F16
      ? dispatch_width<false, half_t, half_t>(x, nullptr, gamma, beta, nullptr, y, rows, cols, eps, apply_affine, s)
      : dispatch_width<false, half_t, float>(x, nullptr, gamma, beta, nullptr, y, rows, cols, eps, apply_affine, s);
  return (int)e;
}

extern "C" int xb_residual_layernorm_masked(const float* residual, const void* update,
                                            int update_dtype, const float* gamma,
                                            const float* beta, float* residual_out, void* y,
                                            int y_dtype, int64_t rows, int32_t cols, float eps,
                                            int apply_affine, const uint8_t* row_valid,
                                            int mask_mode, void* stream) {
  if (rows < 0 || cols <= 0 || rows > 0x7fffffffLL) return XB_ERR_BAD_SIZE;
  if (y_dtype != XB_F32 && y_dtype != XB_F16) return XB_ERR_BAD_DTYPE;
  if (update_dtype != XB_F32 && update_dtype != XB_F16) return XB_ERR_BAD_DTYPE;
  if (mask_mode & ~(XB_MASK_UPDATE | XB_MASK_SUM | XB_MASK_OUTPUT)) return XB_ERR_BAD_EPILOGUE;
  if (rows == 0) return XB_OK;
  if (!residual || !update || !y || (apply_affine && (!gamma || !beta))) return XB_ERR_NULL_POINTER;
  if (mask_mode != 0 && !row_valid) return XB_ERR_NULL_POINTER;
  if (vector_width(cols) &&
      (!aligned16(residual) || !aligned16(update) || !aligned16(y) ||
       (residual_out && !aligned16(residual_out)) ||
       (apply_affine && (!aligned16(gamma) || !aligned16(beta)))))
    return XB_ERR_MISALIGNED;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint8_t* rv = mask_mode != 0 ? row_valid : nullptr;
  hipError_t e;
  if (update_dtype == XB_F16) {
    e = y_dtype == XB_F16
        ? dispatch_width<true, half_t, half_t>(residual, update, gamma, beta, residual_out, y, rows, cols, eps, apply_affine, s, rv, mask_mode)
        : dispatch_width<true, half_t, float>(residual, update, gamma, beta, residual_out, y, rows, cols, eps, apply_affine, s, rv, mask_mode);
  } else {
    e = y_dtype == XB_F16
        ? dispatch_width<true, float, half_t>(residual, update, gamma, beta, residual_out, y, rows, cols, eps, apply_affine, s, rv, mask_mode)
        : dispatch_width<true, float, float>(residual, update, gamma, beta, residual_out, y, rows, cols, eps, apply_affine, s, rv, mask_mode);
  }
  return (int)e;
}

extern "C" int xb_residual_layernorm(const float* residual, const void* update,
                                     int update_dtype, const float* gamma,
                                     const float* beta, float* residual_out, void* y,
                                     int y_dtype, int64_t rows, int32_t cols, float eps,
                                     int apply_affine, void* stream) {
  return xb_residual_layernorm_masked(residual, update, update_dtype, gamma, beta, residual_out, y, y_dtype,
                                      rows, cols, eps, apply_affine, nullptr, 0, stream);
}
