// Causal flash attention over the packed QKV projection, gfx950 MFMA.
//
// Computes, per (batch, head), softmax(q k^T * scale with the top-left causal
// mask) v -- the semantics of F.scaled_dot_product_attention(is_causal=True)
// used by the reference (torch_transformer_benchmark.py:767-808) and of the
// explicit baseline (torch_transformer_benchmark.py:242-257) -- without ever
// materialising the [S, S] scores.  Reads q/k/v straight out of the packed
// [B, S, 3, H, hd] projection and writes the context as [B, S, H, hd], which
// is the [B, S, D] row layout the output projection consumes (this removes
// the reference's transpose + reshape copy, torch_transformer_benchmark.py:809).
//
// Work decomposition: one 256-thread block = 4 waves handles BQ = 64*NQ
// consecutive queries of one head; wave w owns queries [16*NQ*w, 16*NQ*(w+1)).
// Keys are streamed in tiles of BKEYS through LDS.
//
// Scores are formed transposed, S^T = K . Q^T (MFMA M = keys, N = queries), so
// that each lane's accumulator holds scores of ONE query (column l % 16) for
// keys 16*jb + 4*(l/16) + i.  That is exactly the B-operand layout of the
// second product O^T = V^T . P^T once the MFMA k index (l/16)*8 + m is mapped
// to key 32*t + 4*(l/16) + (m & 3) + 16*(m >> 2): probabilities never leave
// registers.  The matching A operand reads V transposed, so V tiles are stored
// in LDS as Vt[hd][key].
//
// Softmax is online in FP32 and base 2 (scale * log2(e) folded into the
// scores); the running max is shared by the 4 lanes that own one query via two
// cross-lane max steps per tile, and the running sum stays per lane until the
// end.  Only tiles that straddle the diagonal pay for the mask.
#include "common.h"
#include "../../include/xblock.h"

namespace xb {

template <int HD>
struct AttnCfg {
  static constexpr int NQ = HD >= 256 ? 1 : 2;        // 16-query blocks per wave
  static constexpr int BKEYS = HD >= 256 ? 32 : 64;   // keys per LDS tile
  static constexpr int HDP = HD < 32 ? 32 : HD;       // reduction dim of S^T, padded
  static constexpr int HDO = HD < 16 ? 16 : HD;       // rows of O^T, padded
  static constexpr int QPW = 16 * NQ;                 // queries per wave
  static constexpr int BQ = 4 * QPW;                  // queries per block
  static constexpr int LDK = HDP + 8;                 // K tile row stride (halves)
  static constexpr int LDV = BKEYS + 4;               // Vt tile row stride (halves)
};

template <int HD>
__global__ __launch_bounds__(256) void attn_causal_kernel(
    const half_t* __restrict__ qkv, half_t* __restrict__ out, int H, int S,
    int q_tiles, float scale_log2) {
  using Cfg = AttnCfg<HD>;
  constexpr int NQ = Cfg::NQ, BKEYS = Cfg::BKEYS, HDP = Cfg::HDP, HDO = Cfg::HDO;
  constexpr int QPW = Cfg::QPW, BQ = Cfg::BQ, LDK = Cfg::LDK, LDV = Cfg::LDV;
  constexpr int KSTEPS = HDP / 32, KB = BKEYS / 16, HB = HDO / 16;
  constexpr int CPK = HD / 8;  // 16-byte chunks per key row

  __shared__ __attribute__((aligned(16))) half_t k_lds[BKEYS * LDK];
  __shared__ __attribute__((aligned(16))) half_t v_lds[HDO * LDV];

  // Heaviest query tiles (most keys under the causal mask) are issued first.
  const int bh = blockIdx.x / q_tiles;
  const int qt = q_tiles - 1 - (blockIdx.x % q_tiles);
  const int b = bh / H, h = bh % H;
  const int D = H * HD;
  const int64_t row_stride = 3 * (int64_t)D;  // halves between consecutive tokens
  const half_t* base = qkv + (int64_t)b * S * row_stride + (int64_t)h * HD;
  const half_t* kbase = base + D;
  const half_t* vbase = base + 2 * D;

  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int q0 = qt * BQ;
  const int qw0 = q0 + wave * QPW;

  // Zero the padding columns/rows once; tile loads never touch them.
  if constexpr (HDP > HD) {
    for (int i = tid; i < BKEYS * (HDP - HD); i += 256)
      k_lds[(i / (HDP - HD)) * LDK + HD + i % (HDP - HD)] = (half_t)0.f;
  }
  if constexpr (HDO > HD) {
    for (int i = tid; i < (HDO - HD) * LDV; i += 256) v_lds[HD * LDV + i] = (half_t)0.f;
  }

  // Q fragments (B operand of S^T): lane holds q[query][32*ks + 8*(l/16) .. +7].
  half8_t qf[NQ][KSTEPS];
  const half8_t zero8 = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int qb = 0; qb < NQ; ++qb) {
    const int q = qw0 + 16 * qb + lane % 16;
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      const int d = 32 * ks + 8 * (lane / 16);
      qf[qb][ks] = (q < S && d < HD) ? *reinterpret_cast<const half8_t*>(base + q * row_stride + d) : zero8;
    }
  }

  float4_t o[HB][NQ];
#pragma unroll
  for (int i = 0; i < HB; ++i)
#pragma unroll
    for (int j = 0; j < NQ; ++j) o[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};
  float m_run[NQ], l_run[NQ];
#pragma unroll
  for (int j = 0; j < NQ; ++j) { m_run[j] = -INFINITY; l_run[j] = 0.f; }

  const int key_end = min(S, q0 + BQ);
  const int n_tiles = (key_end + BKEYS - 1) / BKEYS;
  for (int t = 0; t < n_tiles; ++t) {
    const int k0 = t * BKEYS;
    __syncthreads();  // previous tile fully consumed
    for (int id = tid; id < BKEYS * CPK; id += 256) {
      const int r = id / CPK, c = (id % CPK) * 8;
      const int key = k0 + r;
      half8_t kv = zero8, vv = zero8;
      if (key < S) {
        kv = *reinterpret_cast<const half8_t*>(kbase + key * row_stride + c);
        vv = *reinterpret_cast<const half8_t*>(vbase + key * row_stride + c);
      }
      *reinterpret_cast<half8_t*>(k_lds + r * LDK + c) = kv;
#pragma unroll
      for (int e = 0; e < 8; ++e) v_lds[(c + e) * LDV + r] = vv[e];
    }
    __syncthreads();

    // Wave-uniform skip: every key of this tile lies above this wave's diagonal.
    if (k0 > qw0 + QPW - 1) continue;
    const bool diag = (k0 + BKEYS - 1 > qw0);

    // S^T tile = K . Q^T  ->  s[jb][qb][i]: key k0+16jb+4(l/16)+i, query qw0+16qb+l%16
    float4_t s[KB][NQ];
#pragma unroll
    for (int jb = 0; jb < KB; ++jb) {
#pragma unroll
      for (int qb = 0; qb < NQ; ++qb) s[jb][qb] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks) {
        const half8_t kf = *reinterpret_cast<const half8_t*>(
            k_lds + (16 * jb + lane % 16) * LDK + 32 * ks + 8 * (lane / 16));
#pragma unroll
        for (int qb = 0; qb < NQ; ++qb) s[jb][qb] = mfma16x16x32(kf, qf[qb][ks], s[jb][qb]);
      }
    }

#pragma unroll
    for (int qb = 0; qb < NQ; ++qb) {
      const int q = qw0 + 16 * qb + lane % 16;
      float mx = -INFINITY;
#pragma unroll
      for (int jb = 0; jb < KB; ++jb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float v = s[jb][qb][i] * scale_log2;
          if (diag && (k0 + 16 * jb + 4 * (lane / 16) + i > q)) v = -INFINITY;
          s[jb][qb][i] = v;
          mx = fmaxf(mx, v);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m_run[qb], mx);
      const float corr = __builtin_amdgcn_exp2f(m_run[qb] - m_new);
      m_run[qb] = m_new;
      float rs = 0.f;
#pragma unroll
      for (int jb = 0; jb < KB; ++jb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = __builtin_amdgcn_exp2f(s[jb][qb][i] - m_new);
          s[jb][qb][i] = p;
          rs += p;
        }
      l_run[qb] = l_run[qb] * corr + rs;
#pragma unroll
      for (int hb = 0; hb < HB; ++hb)
#pragma unroll
        for (int i = 0; i < 4; ++i) o[hb][qb][i] *= corr;
    }

    // O^T += V^T . P^T over 32-key steps.
#pragma unroll
    for (int ks = 0; ks < BKEYS / 32; ++ks) {
      half8_t pf[NQ];
#pragma unroll
      for (int qb = 0; qb < NQ; ++qb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pf[qb][i] = (half_t)s[2 * ks][qb][i];
          pf[qb][4 + i] = (half_t)s[2 * ks + 1][qb][i];
        }
#pragma unroll
      for (int hb = 0; hb < HB; ++hb) {
        const half_t* vr = v_lds + (16 * hb + lane % 16) * LDV + 32 * ks + 4 * (lane / 16);
        const half4_t lo = *reinterpret_cast<const half4_t*>(vr);
        const half4_t hi = *reinterpret_cast<const half4_t*>(vr + 16);
        const half8_t vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
        for (int qb = 0; qb < NQ; ++qb) o[hb][qb] = mfma16x16x32(vf, pf[qb], o[hb][qb]);
      }
    }
  }

  // Normalise and store: lane holds O^T[16hb + 4(l/16) + i][query l%16].
  half_t* obase = out + (int64_t)b * S * D + (int64_t)h * HD;
#pragma unroll
  for (int qb = 0; qb < NQ; ++qb) {
    float l = l_run[qb];
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    const float inv = 1.0f / l;
    const int q = qw0 + 16 * qb + lane % 16;
    if (q >= S) continue;
#pragma unroll
    for (int hb = 0; hb < HB; ++hb) {
      const int d = 16 * hb + 4 * (lane / 16);
      if (d < HD) {
        half4_t r;
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = (half_t)(o[hb][qb][i] * inv);
        *reinterpret_cast<half4_t*>(obase + (int64_t)q * D + d) = r;
      }
    }
  }
}

template <int HD>
static hipError_t launch_attn(const half_t* qkv, half_t* out, int B, int S, int H, float scale,
                              hipStream_t s) {
  constexpr int BQ = AttnCfg<HD>::BQ;
  const int q_tiles = (S + BQ - 1) / BQ;
  const int64_t blocks = (int64_t)q_tiles * B * H;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  const float scale_log2 = scale * 1.44269504088896340736f;
  hipLaunchKernelGGL((attn_causal_kernel<HD>), dim3((unsigned)blocks), dim3(256), 0, s, qkv, out,
                     H, S, q_tiles, scale_log2);
  return hipGetLastError();
}

}  // namespace xb

using namespace xb;

extern "C" int xb_attention_causal(const void* qkv, void* out, int32_t batch, int64_t seq_len,
                                   int32_t heads, int32_t head_dim, float scale, void* stream) {
  if (batch < 0 || seq_len < 0 || heads <= 0 || head_dim <= 0) return XB_ERR_BAD_SIZE;
  if (seq_len > 0x7fffffffLL / 4) return XB_ERR_BAD_SIZE;
  if (head_dim != 8 && head_dim != 16 && head_dim != 32 && head_dim != 64 && head_dim != 128 &&
      head_dim != 256)
    return XB_ERR_UNSUPPORTED_SHAPE;
  if (batch == 0 || seq_len == 0) return XB_OK;  // empty tensors may carry NULL data pointers
  if (!qkv || !out) return XB_ERR_NULL_POINTER;
  if (((uintptr_t)qkv | (uintptr_t)out) & 15u) return XB_ERR_MISALIGNED;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const half_t* q = static_cast<const half_t*>(qkv);
  half_t* o = static_cast<half_t*>(out);
  const int S = (int)seq_len;
  hipError_t e;
  switch (head_dim) {
    case 8: e = launch_attn<8>(q, o, batch, S, heads, scale, s); break;
    case 16: e = launch_attn<16>(q, o, batch, S, heads, scale, s); break;
    case 32: e = launch_attn<32>(q, o, batch, S, heads, scale, s); break;
    case 64: e = launch_attn<64>(q, o, batch, S, heads, scale, s); break;
    case 128: e = launch_attn<128>(q, o, batch, S, heads, scale, s); break;
    case 256: e = launch_attn<256>(q, o, batch, S, heads, scale, s); break;
    default: return XB_ERR_UNSUPPORTED_SHAPE;
  }
  return (int)e;
}
