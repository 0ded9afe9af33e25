// FP16 MFMA GEMM with fused bias / exact-erf GELU epilogue for gfx950.
//
//   C[M, N] = epi(A[M, K] . W[N, K]^T + bias[N])
//
// W is nn.Linear's [out_features, in_features] layout, so both operands are
// K-contiguous: every lane feeds v_mfma_f32_16x16x32_f16 with one 16-byte
// LDS read per operand fragment.  The reference instead transposes weights to
// [K, N] for Triton's tl.dot (torch_transformer_benchmark.py:540-566) and
// computes GELU with tanh (triton_fused_ffn.py:198-213); the baseline it must
// match uses exact erf (torch_transformer_benchmark.py:286), as done here.
//
// Block = 4 waves in a 2 x 2 grid; each wave owns a (BM/2) x (BN/2) sub-tile.
// Tiles of A and W go global -> registers -> padded LDS, double buffered, so
// the next K-slab's global loads are in flight while MFMAs consume the
// current one.  The epilogue stages the FP16 tile through LDS so the stores
// to C are full 16-byte row segments.
#include "common.h"
#include "../../include/xblock.h"

namespace xb {

constexpr int kGemmBK = 64;
constexpr int kGemmLDK = kGemmBK + 8;  // padded LDS row (halves): 144 bytes

// Blocks are dispatched round-robin over the 8 XCDs (block b -> XCD b % 8).
// Renumber so that each XCD walks a contiguous range of tiles: neighbouring
// tiles share their A rows, which then stay in that XCD's L2.
__device__ __forceinline__ int xcd_contiguous_tile(int b, int nb) {
  const int q = nb / 8, r = nb % 8, x = b % 8;
  return x * q + (x < r ? x : r) + b / 8;
}

template <int BM, int BN, int EPI>
__global__ __launch_bounds__(256, 2) void gemm_nt_kernel(
    const half_t* __restrict__ A, const half_t* __restrict__ W,
    const float* __restrict__ bias, half_t* __restrict__ C, int M, int N,
    int K, int tiles_n) {
  constexpr int BK = kGemmBK, LDK = kGemmLDK;
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int FM = WM / 16, FN = WN / 16;
  constexpr int CPR = BK / 8;  // 16-byte chunks per tile row
  constexpr int A_CH = BM * CPR / 256, B_CH = BN * CPR / 256;
  static_assert(A_CH * 256 == BM * CPR && B_CH * 256 == BN * CPR, "tile/thread mismatch");
  constexpr int LDC = BN + 8;
  static_assert(BM * LDC <= 2 * (BM + BN) * LDK, "epilogue staging must fit");
  __shared__ __attribute__((aligned(16))) half_t smem[2 * (BM + BN) * LDK];

  const int tile = xcd_contiguous_tile(blockIdx.x, gridDim.x);
  const int m0 = (tile / tiles_n) * BM, n0 = (tile % tiles_n) * BN;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int wm = (wave / 2) * WM, wn = (wave % 2) * WN;

  half8_t ra[A_CH], rb[B_CH];
  const half8_t zero8 = {0, 0, 0, 0, 0, 0, 0, 0};
  auto gload = [&](int k0) {
#pragma unroll
    for (int j = 0; j < A_CH; ++j) {
      const int id = tid + 256 * j, r = id / CPR, c = id % CPR;
      const int gm = m0 + r, gk = k0 + c * 8;
      ra[j] = (gm < M && gk < K) ? *reinterpret_cast<const half8_t*>(A + (int64_t)gm * K + gk) : zero8;
    }
#pragma unroll
    for (int j = 0; j < B_CH; ++j) {
      const int id = tid + 256 * j, r = id / CPR, c = id % CPR;
      const int gn = n0 + r, gk = k0 + c * 8;
      rb[j] = (gn < N && gk < K) ? *reinterpret_cast<const half8_t*>(W + (int64_t)gn * K + gk) : zero8;
    }
  };
  auto sstore = [&](int buf) {
    half_t* as = smem + buf * (BM + BN) * LDK;
    half_t* bs = as + BM * LDK;
#pragma unroll
    for (int j = 0; j < A_CH; ++j) {
      const int id = tid + 256 * j;
      *reinterpret_cast<half8_t*>(as + (id / CPR) * LDK + (id % CPR) * 8) = ra[j];
    }
#pragma unroll
    for (int j = 0; j < B_CH; ++j) {
      const int id = tid + 256 * j;
      *reinterpret_cast<half8_t*>(bs + (id / CPR) * LDK + (id % CPR) * 8) = rb[j];
    }
  };

  float4_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};

  const int KT = (K + BK - 1) / BK;
  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) gload((kt + 1) * BK);
    const half_t* as = smem + cur * (BM + BN) * LDK;
    const half_t* bs = as + BM * LDK;
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      half8_t af[FM], bf[FN];
      const int koff = ks * 32 + (lane / 16) * 8;
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[i] = *reinterpret_cast<const half8_t*>(as + (wm + 16 * i + lane % 16) * LDK + koff);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bf[j] = *reinterpret_cast<const half8_t*>(bs + (wn + 16 * j + lane % 16) * LDK + koff);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = mfma16x16x32(af[i], bf[j], acc[i][j]);
    }
    if (kt + 1 < KT) sstore(cur ^ 1);
    __syncthreads();
  }

  // Epilogue: bias (+ GELU) in FP32, FP16 tile staged in LDS, 16-byte stores.
  half_t* cs = smem;
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int c = wn + 16 * j + lane % 16;
    const float bv = (bias != nullptr && n0 + c < N) ? bias[n0 + c] : 0.f;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float v = acc[i][j][e] + bv;
        if constexpr (EPI == XB_EPI_BIAS_GELU) v = gelu_erf(v);
        cs[(wm + 16 * i + (lane / 16) * 4 + e) * LDC + c] = (half_t)v;
      }
  }
  __syncthreads();
  constexpr int CCH = BM * (BN / 8) / 256;
#pragma unroll
  for (int j = 0; j < CCH; ++j) {
    const int id = tid + 256 * j, r = id / (BN / 8), c = (id % (BN / 8)) * 8;
    const int gm = m0 + r, gn = n0 + c;
    if (gm < M && gn < N)
      *reinterpret_cast<half8_t*>(C + (int64_t)gm * N + gn) = *reinterpret_cast<const half8_t*>(cs + r * LDC + c);
  }
}

template <int BM, int BN, int EPI>
static hipError_t launch_gemm(const half_t* a, const half_t* w, const float* bias, half_t* c,
                              int64_t m, int n, int k, hipStream_t s) {
  const int64_t tm = (m + BM - 1) / BM, tn = (n + BN - 1) / BN;
  if (tm * tn > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL((gemm_nt_kernel<BM, BN, EPI>), dim3((unsigned)(tm * tn)), dim3(256), 0, s,
                     a, w, bias, c, (int)m, n, k, (int)tn);
  return hipGetLastError();
}

template <int EPI>
static hipError_t dispatch_gemm(const half_t* a, const half_t* w, const float* bias, half_t* c,
                                int64_t m, int n, int k, hipStream_t s) {
  // Large tiles when they still give every CU a few tiles, else 64 x 64.
  const int64_t big_tiles = ((m + 127) / 128) * ((n + 127) / 128);
  if (big_tiles >= 512) return launch_gemm<128, 128, EPI>(a, w, bias, c, m, n, k, s);
  return launch_gemm<64, 64, EPI>(a, w, bias, c, m, n, k, s);
}

}  // namespace xb

using namespace xb;

extern "C" int xb_linear(const void* a, const void* w, const float* bias, void* c,
                         int64_t m, int32_t n, int32_t k, int epilogue, void* stream) {
  if (m < 0 || n <= 0 || k <= 0 || m > 0x7fffffffLL) return XB_ERR_BAD_SIZE;
  if (n % 8 != 0 || k % 8 != 0) return XB_ERR_UNSUPPORTED_SHAPE;
  if (epilogue != XB_EPI_BIAS && epilogue != XB_EPI_BIAS_GELU) return XB_ERR_BAD_EPILOGUE;
  if (m == 0) return XB_OK;  // empty tensors may carry NULL data pointers
  if (!a || !w || !c) return XB_ERR_NULL_POINTER;
  if (((uintptr_t)a | (uintptr_t)w | (uintptr_t)c) & 15u) return XB_ERR_MISALIGNED;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const half_t* A = static_cast<const half_t*>(a);
  const half_t* Wt = static_cast<const half_t*>(w);
  half_t* Cc = static_cast<half_t*>(c);
  hipError_t e = epilogue == XB_EPI_BIAS_GELU
      ? dispatch_gemm<XB_EPI_BIAS_GELU>(A, Wt, bias, Cc, m, n, k, s)
      : dispatch_gemm<XB_EPI_BIAS>(A, Wt, bias, Cc, m, n, k, s);
  return (int)e;
}
