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
// K and V tiles of BKEYS keys are double buffered in LDS, both row-major: the
// next tile's global loads are in flight while the current tile is consumed,
// one barrier per tile.
//
// Scores are formed transposed, S^T = K . Q^T (MFMA M = keys, N = queries), so
// that each lane's accumulator holds scores of ONE query (column l % 16) for
// keys 16*jb + 4*(l/16) + i.  That is exactly the B-operand layout of the
// second product O^T = V^T . P^T once the MFMA k index (l/16)*8 + m is mapped
// to key 32*t + 4*(l/16) + (m & 3) + 16*(m >> 2): probabilities never leave
// registers.  The matching A operand (V^T rows, that key order) is read from
// the row-major V tile with gfx950's transposing LDS read ds_read_b64_tr_b16:
// within a 16-lane group, lane j's element i is element j%4 of the 8 bytes
// lane 4i + j/4 addresses, so lane (g, j) addresses
// V[32t + 4g + j/4][16hb + 4(j%4)].
//
// Softmax is online in FP32, base 2, with Q pre-multiplied by scale*log2(e).
// The score MFMAs accumulate onto -m_run (the running exponent offset), so
// the probabilities are a bare exp2 of the accumulator.  The row sum comes out
// of the MFMA as one extra O^T block whose V^T rows are all ones, and m_run is
// only moved (and O rescaled) on the first tile and when a tile's maximum
// exceeds it by more than 8 (probabilities then stay <= 2^8, exact enough in
// FP16); the decision is wave-uniform.  Only tiles that straddle the diagonal
// pay for the mask.
#include "common.h"
#include "../../include/xblock.h"

namespace xb {

template <int HD, int NQ>
struct AttnCfg {
  static constexpr int BKEYS = HD >= 256 ? 32 : 64;   // keys per LDS tile
  static constexpr int HDP = HD < 32 ? 32 : HD;       // K columns incl. zero pad (S^T reduction)
  static constexpr int HDV = HD < 16 ? 16 : HD;       // V columns incl. zero pad (O^T rows)
  static constexpr int QPW = 16 * NQ;                 // queries per wave
  static constexpr int BQ = 4 * QPW;                  // queries per block
  static constexpr int LDK = HDP + 8;                 // K tile row stride (halves)
  // V tile row stride (halves): a multiple of 16 halves with an odd quotient
  // (row stride an odd multiple of 32 bytes), which spreads the 32 rows x 8
  // bytes one half-wave of ds_read_b64_tr_b16 touches over all 64 banks.
  static constexpr int LDV = (HDV / 16) % 2 ? HDV : HDV + 16;
  static constexpr int KSTEPS = HDP / 32, KB = BKEYS / 16, HB = HDV / 16, KT = BKEYS / 32;
  static constexpr int CPK = HD / 8;                  // 16-byte chunks per key row
  static constexpr int CH = (BKEYS * CPK + 255) / 256;  // chunks per thread per tile
};

typedef short short4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ half4_t lds_read_tr16(const half_t* p) {
  const short4_t v =
      __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4_t*)(p));
  return __builtin_bit_cast(half4_t, v);
}

// CAUSAL: apply the top-left causal mask.  KEYMASK: key_valid ([B, S] bytes,
// nonzero = the key may be attended to -- the reference's valid_token_mask,
// TTB:250-253) is staged per tile and masks keys; a query may then see no key
// in a tile, or at all.  Without KEYMASK every query sees key 0 in the first
// tile, which keeps the offset bookkeeping to a tile-index test.
template <int HD, int NQ, bool CAUSAL, bool KEYMASK>
__global__ __launch_bounds__(256, 2) void attn_kernel(
    const half_t* __restrict__ qkv, half_t* __restrict__ out, const uint8_t* __restrict__ key_valid,
    int H, int S, int q_tiles, float scale_log2) {
  using C = AttnCfg<HD, NQ>;
  constexpr int BKEYS = C::BKEYS, HDP = C::HDP, HDV = C::HDV, QPW = C::QPW, BQ = C::BQ;
  constexpr int LDK = C::LDK, LDV = C::LDV, KSTEPS = C::KSTEPS, KB = C::KB, HB = C::HB;
  constexpr int KT = C::KT, CPK = C::CPK, CH = C::CH;

  __shared__ __attribute__((aligned(16))) half_t k_lds[2][BKEYS * LDK];
  __shared__ __attribute__((aligned(16))) half_t v_lds[2][BKEYS * LDV];
  __shared__ __attribute__((aligned(16))) uint8_t kv_lds[2][BKEYS];  // key validity of the tile

  // Heaviest query tiles (most keys under the causal mask) are issued first.
  const int bh = blockIdx.x / q_tiles;
  const int qt = CAUSAL ? q_tiles - 1 - (blockIdx.x % q_tiles) : blockIdx.x % q_tiles;
  const int b = bh / H, h = bh % H;
  const int D = H * HD;
  const int64_t row_stride = 3 * (int64_t)D;  // halves between consecutive tokens
  const half_t* base = qkv + (int64_t)b * S * row_stride + (int64_t)h * HD;
  const half_t* kbase = base + D;
  const half_t* vbase = base + 2 * D;

  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int g = lane / 16, r16 = lane % 16;
  const int q0 = qt * BQ;
  const int qw0 = q0 + wave * QPW;

  // Zero the padding columns of both buffers once; tile stores never touch them.
  if constexpr (HDP > HD) {
    for (int i = tid; i < 2 * BKEYS * (HDP - HD); i += 256) {
      const int buf = i / (BKEYS * (HDP - HD)), j = i % (BKEYS * (HDP - HD));
      k_lds[buf][(j / (HDP - HD)) * LDK + HD + j % (HDP - HD)] = (half_t)0.f;
    }
  }
  if constexpr (HDV > HD) {
    for (int i = tid; i < 2 * BKEYS * (HDV - HD); i += 256) {
      const int buf = i / (BKEYS * (HDV - HD)), j = i % (BKEYS * (HDV - HD));
      v_lds[buf][(j / (HDV - HD)) * LDV + HD + j % (HDV - HD)] = (half_t)0.f;
    }
  }

  // Q fragments (B operand of S^T), pre-multiplied by scale * log2(e):
  // lane holds q[query][32*ks + 8*(l/16) .. +7].
  half8_t qf[NQ][KSTEPS];
  const half8_t zero8 = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int qb = 0; qb < NQ; ++qb) {
    const int q = qw0 + 16 * qb + r16;
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      const int d = 32 * ks + 8 * g;
      half8_t v = zero8;
      if (q < S && d < HD) {
        v = *reinterpret_cast<const half8_t*>(base + q * row_stride + d);
#pragma unroll
        for (int m = 0; m < 8; ++m) v[m] = (half_t)((float)v[m] * scale_log2);
      }
      qf[qb][ks] = v;
    }
  }

  // m_run: the base-2 exponent offset of query (l % 16) of block qb.  The score
  // MFMAs start from -m_run, so a tile's scores arrive already shifted; the
  // first tile with a visible key for a query moves m_run onto that tile's
  // exact maximum (m_set records that it happened; without KEYMASK that is
  // always tile 0).
  float4_t o[HB][NQ], lacc[NQ];
  float m_run[NQ];
  bool m_set[NQ];
#pragma unroll
  for (int qb = 0; qb < NQ; ++qb) {
#pragma unroll
    for (int hb = 0; hb < HB; ++hb) o[hb][qb] = float4_t{0.f, 0.f, 0.f, 0.f};
    lacc[qb] = float4_t{0.f, 0.f, 0.f, 0.f};
    m_run[qb] = 0.f;
    m_set[qb] = false;
  }
  const half8_t ones8 = {1, 1, 1, 1, 1, 1, 1, 1};

  // Key validity travels with the tile (0 past S as well).
  const uint8_t* kvb = KEYMASK ? key_valid + (int64_t)b * S : nullptr;
  uint8_t kvreg = 0;
  half8_t kreg[CH], vreg[CH];
  auto gload = [&](int k0) {
    if (KEYMASK && tid < BKEYS) {
      const int key = k0 + tid;
      kvreg = key < S ? kvb[key] : (uint8_t)0;
    }
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int id = tid + 256 * j;
      kreg[j] = zero8;
      vreg[j] = zero8;
      if (id < BKEYS * CPK) {
        const int key = k0 + id / CPK, c = (id % CPK) * 8;
        if (key < S) {
          kreg[j] = *reinterpret_cast<const half8_t*>(kbase + key * row_stride + c);
          vreg[j] = *reinterpret_cast<const half8_t*>(vbase + key * row_stride + c);
        }
      }
    }
  };
  auto sstore = [&](int buf) {
    if (KEYMASK && tid < BKEYS) kv_lds[buf][tid] = kvreg;
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int id = tid + 256 * j;
      if (id < BKEYS * CPK) {
        const int r = id / CPK, c = (id % CPK) * 8;
        *reinterpret_cast<half8_t*>(&k_lds[buf][r * LDK + c]) = kreg[j];
        *reinterpret_cast<half8_t*>(&v_lds[buf][r * LDV + c]) = vreg[j];
      }
    }
  };

  const int key_end = CAUSAL ? min(S, q0 + BQ) : S;
  const int n_tiles = (key_end + BKEYS - 1) / BKEYS;
  gload(0);
  sstore(0);
  __syncthreads();
  for (int t = 0; t < n_tiles; ++t) {
    const int cur = t & 1;
    const int k0 = t * BKEYS;
    if (t + 1 < n_tiles) gload(k0 + BKEYS);

    // Wave-uniform skip: every key of this tile lies above this wave's diagonal.
    if (!CAUSAL || k0 <= qw0 + QPW - 1) {
      const bool diag = CAUSAL && (k0 + BKEYS - 1 > qw0);
      // Non-causal tiles that run past S mask those keys (causal ones already do).
      const half_t* kt_lds = k_lds[cur];
      const half_t* vt_lds = v_lds[cur];

      // S^T tile = K . Q^T - m_run  ->  s[jb][qb][i]: key k0+16jb+4g+i, query qw0+16qb+r16
      float4_t s[KB][NQ];
      // Wave priority: raised over the MFMA-heavy stretches (the score MFMAs,
      // then the exp + PV MFMA interleave), normal over the max / rescale and
      // the tile store, so the co-resident wave's VALU work fills the gaps.
      __builtin_amdgcn_s_setprio(3);
#pragma unroll
      for (int jb = 0; jb < KB; ++jb) {
#pragma unroll
        for (int qb = 0; qb < NQ; ++qb) s[jb][qb] = float4_t{-m_run[qb], -m_run[qb], -m_run[qb], -m_run[qb]};
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
          const half8_t kf = *reinterpret_cast<const half8_t*>(kt_lds + (16 * jb + r16) * LDK + 32 * ks + 8 * g);
#pragma unroll
          for (int qb = 0; qb < NQ; ++qb) s[jb][qb] = mfma16x16x32(kf, qf[qb][ks], s[jb][qb]);
        }
      }
      __builtin_amdgcn_s_setprio(0);
      if (diag) {
#pragma unroll
        for (int jb = 0; jb < KB; ++jb)
#pragma unroll
          for (int qb = 0; qb < NQ; ++qb)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (k0 + 16 * jb + 4 * g + i > qw0 + 16 * qb + r16) s[jb][qb][i] = -INFINITY;
      }
      if constexpr (KEYMASK) {
#pragma unroll
        for (int jb = 0; jb < KB; ++jb) {
          const uint32_t v4 = *reinterpret_cast<const uint32_t*>(&kv_lds[cur][16 * jb + 4 * g]);
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (((v4 >> (8 * i)) & 0xffu) == 0u)
#pragma unroll
              for (int qb = 0; qb < NQ; ++qb) s[jb][qb][i] = -INFINITY;
        }
      } else if (!CAUSAL && k0 + BKEYS > S) {
#pragma unroll
        for (int jb = 0; jb < KB; ++jb)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (k0 + 16 * jb + 4 * g + i >= S)
#pragma unroll
              for (int qb = 0; qb < NQ; ++qb) s[jb][qb][i] = -INFINITY;
      }

      // The offset moves onto the exact per-query maximum on the first tile
      // that shows the query a key, and afterwards only when some score
      // exceeds it by more than 8 (probabilities then stay <= 2^8, exact
      // enough in FP16).  Whether any does is a lane-local max and one wave
      // vote; the per-query maxima are only formed on that rare path.
      float lm = -INFINITY;
      bool unset = t == 0;
#pragma unroll
      for (int qb = 0; qb < NQ; ++qb) {
        if constexpr (KEYMASK) unset |= !m_set[qb];
#pragma unroll
        for (int jb = 0; jb < KB; ++jb)
          lm = fmaxf(lm, fmaxf(fmaxf(s[jb][qb][0], s[jb][qb][1]), fmaxf(s[jb][qb][2], s[jb][qb][3])));
      }
      if (__any(unset || lm > 8.0f)) {
#pragma unroll
        for (int qb = 0; qb < NQ; ++qb) {
          float m = -INFINITY;
#pragma unroll
          for (int jb = 0; jb < KB; ++jb)
            m = fmaxf(m, fmaxf(fmaxf(s[jb][qb][0], s[jb][qb][1]), fmaxf(s[jb][qb][2], s[jb][qb][3])));
          const float mx = quad_group_max(m);
          // Until a query has seen a key its o and lacc are exactly zero: the
          // offset jumps to the first finite maximum and nothing is rescaled
          // (exp2(-sh) could overflow there).  Afterwards sh >= 0, corr <= 1.
          const bool was_set = KEYMASK ? m_set[qb] : t != 0;
          const float sh = was_set ? fmaxf(mx, 0.f) : (KEYMASK && mx == -INFINITY ? 0.f : mx);
          if constexpr (KEYMASK) m_set[qb] = was_set || mx != -INFINITY;
          const float corr = was_set ? __builtin_amdgcn_exp2f(-sh) : 1.f;
          m_run[qb] += sh;
#pragma unroll
          for (int hb = 0; hb < HB; ++hb) o[hb][qb] *= corr;
          lacc[qb] *= corr;
#pragma unroll
          for (int jb = 0; jb < KB; ++jb) s[jb][qb] -= sh;
        }
      }

      __builtin_amdgcn_s_setprio(3);
      // O^T += V^T . P^T (and the row sums via an all-ones V^T block), 32 keys per step.
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
        half8_t pf[NQ];
#pragma unroll
        for (int qb = 0; qb < NQ; ++qb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            pf[qb][i] = (half_t)__builtin_amdgcn_exp2f(s[2 * kt][qb][i]);
            pf[qb][4 + i] = (half_t)__builtin_amdgcn_exp2f(s[2 * kt + 1][qb][i]);
          }
#pragma unroll
        for (int qb = 0; qb < NQ; ++qb) lacc[qb] = mfma16x16x32(ones8, pf[qb], lacc[qb]);
        const half_t* vrow = vt_lds + (32 * kt + 4 * g + r16 / 4) * LDV + 4 * (r16 % 4);
#pragma unroll
        for (int hb = 0; hb < HB; ++hb) {
          const half4_t lo = lds_read_tr16(vrow + 16 * hb);
          const half4_t hi = lds_read_tr16(vrow + 16 * LDV + 16 * hb);
          const half8_t vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
          for (int qb = 0; qb < NQ; ++qb) o[hb][qb] = mfma16x16x32(vf, pf[qb], o[hb][qb]);
        }
      }
    }

    __builtin_amdgcn_s_setprio(0);
    if (t + 1 < n_tiles) sstore(cur ^ 1);
    __syncthreads();
  }

  // Normalise and store: lane holds O^T[16hb + 4g + i][query r16]; every row of
  // the all-ones block holds that query's probability sum.
  half_t* obase = out + (int64_t)b * S * D + (int64_t)h * HD;
#pragma unroll
  for (int qb = 0; qb < NQ; ++qb) {
    // A query that saw no key at all (every key masked) writes zeros.
    const float inv = lacc[qb][0] > 0.f ? __builtin_amdgcn_rcpf(lacc[qb][0]) : 0.f;
    const int q = qw0 + 16 * qb + r16;
    if (q >= S) continue;
#pragma unroll
    for (int hb = 0; hb < HB; ++hb) {
      const int d = 16 * hb + 4 * g;
      if (d < HD) {
        half4_t r;
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = (half_t)(o[hb][qb][i] * inv);
        *reinterpret_cast<half4_t*>(obase + (int64_t)q * D + d) = r;
      }
    }
  }
}

template <int HD, int NQ>
static hipError_t launch_attn(const half_t* qkv, half_t* out, const uint8_t* kv, int B, int S, int H,
                              float scale, int causal, hipStream_t s) {
  constexpr int BQ = AttnCfg<HD, NQ>::BQ;
  const int q_tiles = (S + BQ - 1) / BQ;
  const int64_t blocks = (int64_t)q_tiles * B * H;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  const float scale_log2 = scale * 1.44269504088896340736f;
  const dim3 grid((unsigned)blocks);
  if (kv != nullptr) {
    if (causal)
      hipLaunchKernelGGL((attn_kernel<HD, NQ, true, true>), grid, dim3(256), 0, s, qkv, out, kv, H, S, q_tiles, scale_log2);
    else
      hipLaunchKernelGGL((attn_kernel<HD, NQ, false, true>), grid, dim3(256), 0, s, qkv, out, kv, H, S, q_tiles, scale_log2);
  } else {
    if (causal)
      hipLaunchKernelGGL((attn_kernel<HD, NQ, true, false>), grid, dim3(256), 0, s, qkv, out, kv, H, S, q_tiles, scale_log2);
    else
      hipLaunchKernelGGL((attn_kernel<HD, NQ, false, false>), grid, dim3(256), 0, s, qkv, out, kv, H, S, q_tiles, scale_log2);
  }
  return hipGetLastError();
}

// Long sequences take 64 queries per wave (each K/V fragment read from LDS
// then feeds 4 MFMAs); short ones keep 32 so a block does not outgrow S.
template <int HD>
static hipError_t dispatch_attn(const half_t* qkv, half_t* out, const uint8_t* kv, int B, int S, int H,
                                float scale, int causal, hipStream_t s) {
  if constexpr (HD >= 256) {
    return launch_attn<HD, 1>(qkv, out, kv, B, S, H, scale, causal, s);
  } else if constexpr (HD >= 128) {
    return launch_attn<HD, 2>(qkv, out, kv, B, S, H, scale, causal, s);
  } else {
    if (S >= 1024) return launch_attn<HD, 4>(qkv, out, kv, B, S, H, scale, causal, s);
    return launch_attn<HD, 2>(qkv, out, kv, B, S, H, scale, causal, s);
  }
}

}  // namespace xb

using namespace xb;

extern "C" int xb_attention(const void* qkv, void* out, const uint8_t* key_valid, int32_t batch,
                            int64_t seq_len, int32_t heads, int32_t head_dim, float scale, int32_t causal,
                            void* stream) {
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
  const int c = causal ? 1 : 0;
  hipError_t e;
  switch (head_dim) {
    case 8: e = dispatch_attn<8>(q, o, key_valid, batch, S, heads, scale, c, s); break;
    case 16: e = dispatch_attn<16>(q, o, key_valid, batch, S, heads, scale, c, s); break;
    case 32: e = dispatch_attn<32>(q, o, key_valid, batch, S, heads, scale, c, s); break;
    case 64: e = dispatch_attn<64>(q, o, key_valid, batch, S, heads, scale, c, s); break;
    case 128: e = dispatch_attn<128>(q, o, key_valid, batch, S, heads, scale, c, s); break;
    default: e = dispatch_attn<256>(q, o, key_valid, batch, S, heads, scale, c, s); break;
  }
  return (int)e;
}

extern "C" int xb_attention_causal(const void* qkv, void* out, int32_t batch, int64_t seq_len,
                                   int32_t heads, int32_t head_dim, float scale, void* stream) {
  return xb_attention(qkv, out, nullptr, batch, seq_len, heads, head_dim, scale, 1, stream);
}
