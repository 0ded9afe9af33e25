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
// Two kernels:
//  * gemm_dma_kernel (K % 64 == 0, K >= 256): 8 waves, up to 256 x 256 tiles,
//    direct global -> LDS loads; used for the D >= 256 projections and FFN.
//  * gemm_nt_kernel (any K % 8 == 0): 4 waves in a 2 x 2 grid, tiles of A and
//    W go global -> registers -> padded LDS, double buffered; the epilogue
//    stages the FP16 tile through LDS so the stores to C are full 16-byte row
//    segments.
// Accumulators stay in VGPRs (the library builds this file with
// -amdgpu-mfma-vgpr-form): with AGPR accumulators the register allocator
// rotates accumulator tuples through copies on every loop iteration.
#include <cstdint>

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

// Tile coordinates of the direct-to-LDS kernel: tiles are ordered in bands of
// four row blocks, column by column inside a band, and each XCD takes a
// contiguous range of that order (xcd_contiguous_tile).  One round of 32
// tiles on an XCD then covers 4 row blocks x 8 column blocks instead of 2 x 16
// (row-major), which for the QKV projection (N = 3072) reads 5 MB of distinct
// operands per round instead of 7 MB through that XCD's 4 MB L2, and the next
// round keeps the same A rows.  Measured, outputs bitwise equal: 8192 x 3072
// x 1024 (256 x 192 tiles) 62.5 -> 60.3-61.6 us, 3.2M x 3072 x 1024 (256 x
// 256) 20.9 -> 19.6 ms, 3.2M x 1024 x 1024 7.23 -> 7.08 ms.
constexpr int kGemmBandRows = 4;
__device__ __forceinline__ void banded_tile(int tile, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int band = tile / (kGemmBandRows * tiles_n);
  const int l = tile - band * kGemmBandRows * tiles_n;
  const int rows = min(kGemmBandRows, tiles_m - band * kGemmBandRows);  // the last band may be shorter
  tm = band * kGemmBandRows + l % rows;
  tn = l / rows;
}

// FP32 -> FP16 of an epilogue value, rounded once from the FP32 value.  The
// empty asm pins the FP32 result: otherwise the backend may fold the last
// multiply or add into a singly-rounded v_fma_mix conversion in some tile
// instantiations and not others, and the FP16 output would then depend on
// the tile (hence on the batch size that selected it).
__device__ __forceinline__ half_t to_half_pinned(float v) {
  asm volatile("" : "+v"(v));
  return (half_t)v;
}

template <int BM, int BN, int WGM, int WGN, int EPI>
__global__ __launch_bounds__(64 * WGM * WGN, 1) void gemm_nt_kernel(
    const half_t* __restrict__ A, const half_t* __restrict__ W,
    const float* __restrict__ bias, half_t* __restrict__ C, int M, int N,
    int K, int tiles_n) {
  constexpr int NT = 64 * WGM * WGN;  // threads
  constexpr int BK = kGemmBK, LDK = kGemmLDK;
  constexpr int WM = BM / WGM, WN = BN / WGN;  // wave tile
  constexpr int FM = WM / 16, FN = WN / 16;
  constexpr int CPR = BK / 8;  // 16-byte chunks per tile row
  constexpr int A_CH = BM * CPR / NT, B_CH = BN * CPR / NT;
  static_assert(A_CH * NT == BM * CPR && B_CH * NT == BN * CPR, "tile/thread mismatch");
  constexpr int LDC = BN + 8;
  static_assert(BM * LDC <= 2 * (BM + BN) * LDK, "epilogue staging must fit");
  __shared__ __attribute__((aligned(16))) half_t smem[2 * (BM + BN) * LDK];

  const int tile = xcd_contiguous_tile(blockIdx.x, gridDim.x);
  const int m0 = (tile / tiles_n) * BM, n0 = (tile % tiles_n) * BN;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int wm = (wave / WGN) * WM, wn = (wave % WGN) * WN;

  half8_t ra[A_CH], rb[B_CH];
  const half8_t zero8 = {0, 0, 0, 0, 0, 0, 0, 0};
  auto gload = [&](int k0) {
#pragma unroll
    for (int j = 0; j < A_CH; ++j) {
      const int id = tid + NT * j, r = id / CPR, c = id % CPR;
      const int gm = m0 + r, gk = k0 + c * 8;
      ra[j] = (gm < M && gk < K) ? *reinterpret_cast<const half8_t*>(A + (int64_t)gm * K + gk) : zero8;
    }
#pragma unroll
    for (int j = 0; j < B_CH; ++j) {
      const int id = tid + NT * j, r = id / CPR, c = id % CPR;
      const int gn = n0 + r, gk = k0 + c * 8;
      rb[j] = (gn < N && gk < K) ? *reinterpret_cast<const half8_t*>(W + (int64_t)gn * K + gk) : zero8;
    }
  };
  auto sstore = [&](int buf) {
    half_t* as = smem + buf * (BM + BN) * LDK;
    half_t* bs = as + BM * LDK;
#pragma unroll
    for (int j = 0; j < A_CH; ++j) {
      const int id = tid + NT * j;
      *reinterpret_cast<half8_t*>(as + (id / CPR) * LDK + (id % CPR) * 8) = ra[j];
    }
#pragma unroll
    for (int j = 0; j < B_CH; ++j) {
      const int id = tid + NT * j;
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
        cs[(wm + 16 * i + (lane / 16) * 4 + e) * LDC + c] = to_half_pinned(v);
      }
  }
  __syncthreads();
  constexpr int CCH = BM * (BN / 8) / NT;
#pragma unroll
  for (int j = 0; j < CCH; ++j) {
    const int id = tid + NT * j, r = id / (BN / 8), c = (id % (BN / 8)) * 8;
    const int gm = m0 + r, gn = n0 + c;
    if (gm < M && gn < N)
      *reinterpret_cast<half8_t*>(C + (int64_t)gm * N + gn) = *reinterpret_cast<const half8_t*>(cs + r * LDC + c);
  }
}

// ---------------------------------------------------------------------------
// Large-tile kernel for K % 64 == 0.  8 waves (2 per SIMD) share a BM x BN
// tile; each wave owns a (BM/WGM) x (BN/WGN) sub-tile with its FP32
// accumulators in VGPRs.  Operands reach LDS by direct global -> LDS loads
// (global_load_lds_dwordx4), one 64-wide K slab at a time, in a ring of ST
// slab stages: slab kt+ST is requested as soon as every wave has read slab
// kt, so ST-1 slabs are in flight while one is consumed.  With one block per
// CU nothing else hides the memory latency, so the ring depth is what keeps
// the MFMAs fed when the grid is a single round of tiles.
//
// LDS slab layout: the A rows (BM) and then the W rows (BN), 128 bytes each
// (64 halves = eight 16-byte chunks).  Chunk c of row r lives at slot
// c ^ (r & 7), so the 8 rows one 8-lane phase of ds_read_b128 touches land in
// 8 distinct 16-byte bank groups.  A DMA load writes lane i's 16 bytes to
// consecutive LDS addresses, so the swizzle is applied on the global side:
// lane i of a 1 KB segment (8 rows) fetches the chunk that belongs in its slot.


// s_waitcnt with vmcnt <= N and lgkmcnt == 0 (gfx9 field layout:
// vmcnt[3:0], expcnt[6:4], lgkmcnt[11:8], vmcnt_hi[15:14]).
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (0 << 8) | ((N >> 4) << 14));
}

// Workgroup barrier that orders this wave's memory operations in the compiler
// without the vmcnt(0) a release fence would add.
__device__ __forceinline__ void slab_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ int row128_offset(int r, int c) { return r * 128 + ((c ^ (r & 7)) << 4); }

// V of a packed QKV projection written transposed per head for the long-
// sequence attention: vt[b][h][d][p] with rows of `row` = seq_len rounded up
// to 64 elements, the positions p of each 32-token group in the attention's
// key order (token 32t + 4g + i at 32t + 8g + i, token 32t + 16 + 4g + i at
// 32t + 8g + 4 + i), so one 16-byte LDS read there is one operand fragment.
// Positions seq_len .. row-1 hold zeros.  Columns from v_col0 on are V.
struct VtOut {
  half_t* vt;
  int64_t row;
  int seq_len, head_dim, heads, v_col0;
};

template <int BM, int BN, int WGM, int WGN, int EPI, int ST, bool VT = false>
__global__ __launch_bounds__(64 * WGM * WGN, 1) void gemm_dma_kernel(
    const half_t* __restrict__ A, const half_t* __restrict__ W,
    const float* __restrict__ bias, half_t* __restrict__ C, int M, int N,
    int K, int tiles_n, VtOut vo) {
  constexpr int NW = WGM * WGN;
  constexpr int WM = BM / WGM, WN = BN / WGN, FM = WM / 16, FN = WN / 16;
  constexpr int SLAB = (BM + BN) * 128;        // 64-wide K slab, 128-byte rows
  constexpr int SEGS = (BM + BN) / 8;          // 1 KB wave-loads per slab (8 rows)
  constexpr int SPW = SEGS / NW;
  static_assert(SEGS % NW == 0 && WM % 16 == 0 && WN % 16 == 0, "tile shape");
  static_assert(ST >= 2 && ST * SLAB <= 160 * 1024 && (ST - 1) * SPW < 64, "slab ring");
  __shared__ __attribute__((aligned(1024))) char smem[ST * SLAB];
  int tile_m, tile_n;
  banded_tile(xcd_contiguous_tile(blockIdx.x, gridDim.x), gridDim.x / tiles_n, tiles_n, tile_m, tile_n);
  const int m0 = tile_m * BM, n0 = tile_n * BN;
  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int wm = (wave / WGN) * WM, wn = (wave % WGN) * WN;
  const half_t* src[SPW];
#pragma unroll
  for (int j = 0; j < SPW; ++j) {
    const int r = (wave + NW * j) * 8 + lane / 8;
    const int c = (lane % 8) ^ (r & 7);
    src[j] = r < BM ? A + (int64_t)min(m0 + r, M - 1) * K + 8 * c
                    : W + (int64_t)min(n0 + r - BM, N - 1) * K + 8 * c;
  }
  auto issue = [&](int kt, int stage) {
#pragma unroll
    for (int j = 0; j < SPW; ++j)
      __builtin_amdgcn_global_load_lds((global_void_t*)(src[j] + kt * 64),
                                       (lds_void_t*)(smem + stage * SLAB + (wave + NW * j) * 1024), 16, 0, 0);
  };
  float4_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};
  const int KT = K / 64;
  auto read_frags = [&](int stage, int ks, half8_t (&af)[FM], half8_t (&bf)[FN]) {
    const char* st = smem + stage * SLAB;
    const int q = ks * 4 + lane / 16;
#pragma unroll
    for (int j = 0; j < FN; ++j)
      bf[j] = *reinterpret_cast<const half8_t*>(st + row128_offset(BM + wn + 16 * j + lane % 16, q));
#pragma unroll
    for (int i = 0; i < FM; ++i)
      af[i] = *reinterpret_cast<const half8_t*>(st + row128_offset(wm + 16 * i + lane % 16, q));
  };
  auto mma = [&](const half8_t (&af)[FM], const half8_t (&bf)[FN]) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = mfma16x16x32(bf[j], af[i], acc[i][j]);
  };
  // Slab kt: sub-step 0 reads sub-step 1's fragments of the same slab while
  // its own MFMAs run; sub-step 1 waits for slab kt+1 (leaving the ST-2 slabs
  // after it in flight), refills slab kt's stage with slab kt+ST and reads
  // slab kt+1's first fragments.  vmcnt retires loads in issue order, so
  // "at most (ST-2)*SPW outstanding" means slab kt+1 has landed.
  half8_t a0[FM], b0[FN], a1[FM], b1[FN];
#pragma unroll
  for (int s = 0; s < ST; ++s)
    if (s < KT) issue(s, s);
  if (KT >= ST) wait_vm_lgkm0<(ST - 1) * SPW>(); else wait_vm_lgkm0<0>();
  slab_barrier();
  read_frags(0, 0, a0, b0);
  int stage = 0;  // stage of slab kt
  for (int kt = 0; kt < KT; ++kt) {
    const int next = stage + 1 == ST ? 0 : stage + 1;
    __builtin_amdgcn_sched_barrier(0);
    read_frags(stage, 1, a1, b1);
    __builtin_amdgcn_sched_barrier(0);
    mma(a0, b0);
    __builtin_amdgcn_sched_barrier(0);
    if (kt + 1 < KT) {
      if (kt + ST - 1 < KT) wait_vm_lgkm0<(ST - 2) * SPW>(); else wait_vm_lgkm0<0>();
      slab_barrier();
      if (kt + ST < KT) issue(kt + ST, stage);
      read_frags(next, 0, a0, b0);
    } else {
      wait_vm_lgkm0<0>();
    }
    __builtin_amdgcn_sched_barrier(0);
    mma(a1, b1);
    stage = next;
  }

  // Epilogue: bias (+ GELU) in FP32, the FP16 tile staged in LDS (free once
  // every wave has read the last slab), then written out in 16-byte row
  // chunks, a wave covering whole rows: lane-sized row pieces of 8 bytes
  // scattered over 16 rows per store made the stores a fifth of the time.
  // Chunk k of tile row r sits at chunk k ^ (r & SW) of its LDS row, which
  // keeps both the 8-byte fragment writes and the 16-byte reads spread over
  // the banks.
  constexpr int CPR = BN / 8;                       // 16-byte chunks per tile row
  constexpr int SW = CPR % 16 == 0 ? 15 : 7;
  static_assert(BM * BN * 2 <= ST * SLAB, "the C tile fits in the slab stages");
  slab_barrier();
  if constexpr (VT) {
    if (n0 >= vo.v_col0) {  // a V tile (the host checked v_col0 % BN == 0, seq_len % 32 == 0)
      static_assert(BM % 32 == 0, "whole 32-token groups per tile");
      // Staged feature-major, [BN][BM], positions in key order, then written
      // as whole 16-byte chunks of the transposed rows.
      half_t* vs = reinterpret_cast<half_t*>(smem);
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int col = wn + 16 * j + (lane / 16) * 4;
        float b[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) b[e] = bias != nullptr ? bias[n0 + col + e] : 0.f;
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          const int r = wm + 16 * i + lane % 16;
          const int p = (r & ~31) | (((r & 15) >> 2) << 3) | (((r >> 4) & 1) << 2) | (r & 3);
#pragma unroll
          for (int e = 0; e < 4; ++e) vs[(col + e) * BM + p] = to_half_pinned(acc[i][j][e] + b[e]);
        }
      }
      slab_barrier();
      constexpr int NT = 64 * NW, CPF = BM / 8;  // 16-byte chunks per staged feature row
      static_assert((BN * CPF) % NT == 0, "whole rounds of chunks");
#pragma unroll
      for (int id0 = 0; id0 < BN * CPF; id0 += NT) {
        const int id = id0 + (int)threadIdx.x;
        const int f = id / CPF, c = id % CPF;
        const int m = m0 + 32 * (c / 4);  // first token of the chunk's 32-token group
        if (m < M) {
          const int bq = m / vo.seq_len, sq = m - bq * vo.seq_len;
          const int n = n0 + f - vo.v_col0;
          const int h = n / vo.head_dim, d = n - h * vo.head_dim;
          half_t* dst = vo.vt + ((int64_t)(bq * vo.heads + h) * vo.head_dim + d) * vo.row + sq + 8 * (c % 4);
          *reinterpret_cast<half8_t*>(dst) = *reinterpret_cast<const half8_t*>(vs + f * BM + 8 * c);
          if (sq + 32 == vo.seq_len && c % 4 == 0) {  // the sequence's last group: zero the row's padding
            for (int64_t z = vo.seq_len; z < vo.row; z += 8)
              *reinterpret_cast<half8_t*>(dst - sq + z) = half8_t{0, 0, 0, 0, 0, 0, 0, 0};
          }
        }
      }
      return;
    }
  }
  half_t* cs = reinterpret_cast<half_t*>(smem);
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int col = wn + 16 * j + (lane / 16) * 4;  // tile column of this lane's 4 values
    float b[4] = {0.f, 0.f, 0.f, 0.f};
    if (bias != nullptr && n0 + col < N) {
#pragma unroll
      for (int e = 0; e < 4; ++e) b[e] = bias[n0 + col + e];
    }
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int row = wm + 16 * i + lane % 16;
      half4_t h;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float v = acc[i][j][e] + b[e];
        if constexpr (EPI == XB_EPI_BIAS_GELU) v = gelu_erf(v);
        h[e] = to_half_pinned(v);
      }
      *reinterpret_cast<half4_t*>(cs + row * BN + 8 * ((col / 8) ^ (row & SW)) + (col & 7)) = h;
    }
  }
  slab_barrier();
  constexpr int NT = 64 * NW;
  static_assert((BM * CPR) % NT == 0, "whole rounds of 16-byte chunks");
#pragma unroll
  for (int id0 = 0; id0 < BM * CPR; id0 += NT) {
    const int id = id0 + (int)threadIdx.x;
    const int row = id / CPR, k = id % CPR;
    const int gm = m0 + row, gn = n0 + 8 * k;
    if (gm < M && gn < N)
      *reinterpret_cast<half8_t*>(C + (int64_t)gm * N + gn) =
          *reinterpret_cast<const half8_t*>(cs + row * BN + 8 * (k ^ (row & SW)));
  }
}

template <int BM, int BN, int WGM, int WGN, int EPI, int ST, bool VT = false>
static hipError_t launch_gemm_dma(const half_t* a, const half_t* w, const float* bias, half_t* c,
                                  int64_t m, int n, int k, hipStream_t s, VtOut vo = {}) {
  const int64_t tm = (m + BM - 1) / BM, tn = (n + BN - 1) / BN;
  if (tm * tn > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL((gemm_dma_kernel<BM, BN, WGM, WGN, EPI, ST, VT>), dim3((unsigned)(tm * tn)),
                     dim3(64 * WGM * WGN), 0, s, a, w, bias, c, (int)m, n, k, (int)tn, vo);
  return hipGetLastError();
}

template <int BM, int BN, int WGM, int WGN, int EPI>
static hipError_t launch_gemm(const half_t* a, const half_t* w, const float* bias, half_t* c,
                              int64_t m, int n, int k, hipStream_t s) {
  const int64_t tm = (m + BM - 1) / BM, tn = (n + BN - 1) / BN;
  if (tm * tn > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL((gemm_nt_kernel<BM, BN, WGM, WGN, EPI>), dim3((unsigned)(tm * tn)),
                     dim3(64 * WGM * WGN), 0, s, a, w, bias, c, (int)m, n, k, (int)tn);
  return hipGetLastError();
}

// Tile variants (XB_LINEAR_*): the gemm_dma_kernel tiles need K % 64 == 0
// and K >= 256 (256 x 192 also N % 192 == 0); the gemm_nt_kernel tiles take
// any K % 8 == 0.
static bool linear_variant_fits(int variant, int64_t m, int n, int k) {
  (void)m;
  const bool dma = k % 64 == 0 && k >= 256;
  switch (variant) {
    case XB_LINEAR_DMA_256x256: case XB_LINEAR_DMA_128x256: case XB_LINEAR_DMA_128x128: return dma;
    case XB_LINEAR_DMA_256x192: return dma && n % 192 == 0;
    case XB_LINEAR_NT_128x128: case XB_LINEAR_NT_64x64: return true;
    default: return false;
  }
}

// The library's choice for a shape.  With the DMA tiles one block runs per
// CU, so the cost is taken as rounds of 256 tiles x tile area, the 256 x 256
// tile ~15% cheaper per output (fewer LDS bytes per MFMA); 256 x 192 sits
// between them and fills whole rounds where 256 x 256 leaves half a round
// idle (M = 8192, N = 3072: 54 vs 60 us).  With the banded tile order a
// 128 x 128 round on an XCD reads about 3 MB of distinct operands at N =
// 1024, inside its 4 MB L2, and costs ~5% less per output than 128 x 256:
// a sweep (us, 256x256 / 128x256 / 128x128) of 8192 x 1024 x 1024 gave
// 31.4 / 22.5 / 21.2, 16384 x 1024 35.4 / 40.9 / 39.6, 3.2M x 1024
// 7311 / 8542 / 8052, and the factors below reproduce every best choice of
// that sweep (also 4096 x 1024, 4096 / 8192 / 3.2M x 3072).
static int select_linear(int64_t m, int n, int k) {
  auto tiles = [&](int64_t bm, int64_t bn) { return ((m + bm - 1) / bm) * ((n + bn - 1) / bn); };
  if (k % 64 == 0 && k >= 256) {
    const int64_t big = (tiles(256, 256) + 255) / 256 * 65536 * 85 / 100;
    const int64_t wide = n % 192 == 0 ? (tiles(256, 192) + 255) / 256 * 49152 * 90 / 100 : INT64_MAX;
    const int64_t mid = (tiles(128, 256) + 255) / 256 * 32768;
    const int64_t small = (tiles(128, 128) + 255) / 256 * 16384 * 95 / 100;
    if (big <= wide && big <= mid && big <= small) return XB_LINEAR_DMA_256x256;
    if (wide <= mid && wide <= small) return XB_LINEAR_DMA_256x192;
    if (mid <= small) return XB_LINEAR_DMA_128x256;
    return XB_LINEAR_DMA_128x128;
  }
  return tiles(128, 128) >= 512 ? XB_LINEAR_NT_128x128 : XB_LINEAR_NT_64x64;
}

template <int EPI>
static hipError_t run_gemm(int variant, const half_t* a, const half_t* w, const float* bias, half_t* c,
                           int64_t m, int n, int k, hipStream_t s) {
  switch (variant) {
    case XB_LINEAR_DMA_256x256: return launch_gemm_dma<256, 256, 4, 2, EPI, 2>(a, w, bias, c, m, n, k, s);
    case XB_LINEAR_DMA_256x192: return launch_gemm_dma<256, 192, 4, 2, EPI, 2>(a, w, bias, c, m, n, k, s);
    case XB_LINEAR_DMA_128x256: return launch_gemm_dma<128, 256, 2, 4, EPI, 2>(a, w, bias, c, m, n, k, s);
    case XB_LINEAR_DMA_128x128: return launch_gemm_dma<128, 128, 2, 2, EPI, 2>(a, w, bias, c, m, n, k, s);
    case XB_LINEAR_NT_128x128: return launch_gemm<128, 128, 2, 2, EPI>(a, w, bias, c, m, n, k, s);
    default: return launch_gemm<64, 64, 2, 2, EPI>(a, w, bias, c, m, n, k, s);
  }
}

}  // namespace xb

using namespace xb;

static int check_linear(int64_t m, int32_t n, int32_t k, int epilogue) {
  if (m < 0 || n <= 0 || k <= 0 || m > 0x7fffffffLL) return XB_ERR_BAD_SIZE;
  if (n % 8 != 0 || k % 8 != 0) return XB_ERR_UNSUPPORTED_SHAPE;
  if (epilogue != XB_EPI_BIAS && epilogue != XB_EPI_BIAS_GELU) return XB_ERR_BAD_EPILOGUE;
  return XB_OK;
}

extern "C" int xb_select_linear(int64_t m, int32_t n, int32_t k, int epilogue) {
  const int bad = check_linear(m, n, k, epilogue);
  return bad ? bad : select_linear(m, n, k);
}

extern "C" int xb_linear_v(const void* a, const void* w, const float* bias, void* c, int64_t m, int32_t n,
                           int32_t k, int epilogue, int variant, void* stream) {
  const int bad = check_linear(m, n, k, epilogue);
  if (bad) return bad;
  if (variant == XB_VARIANT_AUTO) variant = select_linear(m, n, k);
  if (!linear_variant_fits(variant, m, n, k)) return XB_ERR_BAD_VARIANT;
  if (m == 0) return XB_OK;  // empty tensors may carry NULL data pointers
  if (!a || !w || !c) return XB_ERR_NULL_POINTER;
  if (((uintptr_t)a | (uintptr_t)w | (uintptr_t)c) & 15u) return XB_ERR_MISALIGNED;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const half_t* A = static_cast<const half_t*>(a);
  const half_t* Wt = static_cast<const half_t*>(w);
  half_t* Cc = static_cast<half_t*>(c);
  hipError_t e = epilogue == XB_EPI_BIAS_GELU
      ? run_gemm<XB_EPI_BIAS_GELU>(variant, A, Wt, bias, Cc, m, n, k, s)
      : run_gemm<XB_EPI_BIAS>(variant, A, Wt, bias, Cc, m, n, k, s);
  return (int)e;
}

extern "C" int xb_linear(const void* a, const void* w, const float* bias, void* c,
                         int64_t m, int32_t n, int32_t k, int epilogue, void* stream) {
  return xb_linear_v(a, w, bias, c, m, n, k, epilogue, XB_VARIANT_AUTO, stream);
}

extern "C" int64_t xb_vt_row_stride(int64_t seq_len) { return seq_len <= 0 ? 0 : (seq_len + 63) / 64 * 64; }

extern "C" int xb_linear_qkv_vt(const void* a, const void* w, const float* bias, void* qkv, void* vt,
                                int32_t batch, int64_t seq_len, int32_t heads, int32_t head_dim, int32_t k,
                                int variant, void* stream) {
  if (batch < 0 || seq_len < 0 || heads <= 0 || head_dim <= 0 || k <= 0) return XB_ERR_BAD_SIZE;
  const int64_t m = (int64_t)batch * seq_len;
  const int64_t d = (int64_t)heads * head_dim;
  if (m > 0x7fffffffLL || 3 * d > 0x7fffffffLL) return XB_ERR_BAD_SIZE;
  const int n = (int)(3 * d);
  if (seq_len % 32 != 0 || head_dim % 8 != 0 || k % 64 != 0 || k < 256) return XB_ERR_UNSUPPORTED_SHAPE;
  if (variant == XB_VARIANT_AUTO) {
    variant = select_linear(m, n, k);
    if (variant == XB_LINEAR_DMA_256x192 || d % 256 != 0) variant = d % 256 == 0 ? XB_LINEAR_DMA_256x256 : XB_LINEAR_DMA_128x128;
  }
  int bn = 0;
  switch (variant) {
    case XB_LINEAR_DMA_256x256: case XB_LINEAR_DMA_128x256: bn = 256; break;
    case XB_LINEAR_DMA_128x128: bn = 128; break;
    default: return XB_ERR_BAD_VARIANT;  // the V boundary must fall between DMA tiles
  }
  if (d % bn != 0) return XB_ERR_BAD_VARIANT;  // every tile is all Q/K or all V
  if (m == 0) return XB_OK;
  if (!a || !w || !qkv || !vt) return XB_ERR_NULL_POINTER;
  if (((uintptr_t)a | (uintptr_t)w | (uintptr_t)qkv | (uintptr_t)vt) & 15u) return XB_ERR_MISALIGNED;
  const VtOut vo{static_cast<half_t*>(vt), xb_vt_row_stride(seq_len), (int)seq_len, head_dim, heads, (int)(2 * d)};
  const half_t* A = static_cast<const half_t*>(a);
  const half_t* Wt = static_cast<const half_t*>(w);
  half_t* Cc = static_cast<half_t*>(qkv);
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  switch (variant) {
    case XB_LINEAR_DMA_256x256:
      e = launch_gemm_dma<256, 256, 4, 2, XB_EPI_BIAS, 2, true>(A, Wt, bias, Cc, m, n, k, s, vo); break;
    case XB_LINEAR_DMA_128x256:
      e = launch_gemm_dma<128, 256, 2, 4, XB_EPI_BIAS, 2, true>(A, Wt, bias, Cc, m, n, k, s, vo); break;
    default:
      e = launch_gemm_dma<128, 128, 2, 2, XB_EPI_BIAS, 2, true>(A, Wt, bias, Cc, m, n, k, s, vo); break;
  }
  return (int)e;
}
