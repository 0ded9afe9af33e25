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
#include <algorithm>
#include <atomic>
#include <mutex>
#include <type_traits>

#include "common.h"
#include "../../include/xblock.h"

namespace xb {

template <int HD, int NQ, int NW = 4>
struct AttnCfg {
  static constexpr int NT = 64 * NW;                  // threads per block
  static constexpr int BKEYS = HD >= 256 ? 32 : 64;   // keys per LDS tile
  static constexpr int HDP = HD < 32 ? 32 : HD;       // K columns incl. zero pad (S^T reduction)
  static constexpr int HDV = HD < 16 ? 16 : HD;       // V columns incl. zero pad (O^T rows)
  static constexpr int QPW = 16 * NQ;                 // queries per wave
  static constexpr int BQ = NW * QPW;                 // queries per block
  static constexpr int LDK = HDP + 8;                 // K tile row stride (halves)
  // V tile row stride (halves): a multiple of 16 halves with an odd quotient
  // (row stride an odd multiple of 32 bytes), which spreads the 32 rows x 8
  // bytes one half-wave of ds_read_b64_tr_b16 touches over all 64 banks.
  static constexpr int LDV = (HDV / 16) % 2 ? HDV : HDV + 16;
  static constexpr int KSTEPS = HDP / 32, KB = BKEYS / 16, HB = HDV / 16, KT = BKEYS / 32;
  static constexpr int CPK = HD / 8;                  // 16-byte chunks per key row
  static constexpr int CH = (BKEYS * CPK + NT - 1) / NT;  // chunks per thread per tile
};

// Where the operands live.  Query, key and value rows of token t of batch b,
// head h start at q + b*q_bstride + h*HD + t*q_rstride (likewise k, v with
// k_bstride, k_hstride, k_rstride; the context at out + b*o_bstride + h*HD +
// t*o_rstride).  The packed [B, S, 3, H, hd] projection and the [B, H, cap, hd]
// KV cache are both such strided views.  Query i has position q_offset + i;
// under the causal mask it sees keys j <= q_offset + i.
struct AttnArgs {
  const half_t* q;
  const half_t* k;
  const half_t* v;
  half_t* out;
  const uint8_t* key_valid;  // [B, S_k] bytes (KEYMASK only)
  float* ws_o;               // split partials: [B*H][splits][BQ][HD] (SPLIT only)
  float2* ws_ml;             // split partials: [B*H][splits][BQ] (offset, row sum)
  int64_t q_bstride, k_bstride, k_hstride, o_bstride;
  int q_rstride, k_rstride, o_rstride;
  int H, S_q, S_k, q_offset, q_tiles, n_splits, split_keys;
  float scale_log2;
  // Ping-pong kernel only: V transposed per head by the QKV GEMM,
  // vt[b][h][d][p] (rows of vt_row elements, key order inside each 32-key
  // group as that GEMM writes it), used instead of v when not NULL.
  const half_t* vt;
  int64_t vt_row;
};

typedef short short4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ half4_t lds_read_tr16(const half_t* p) {
  const short4_t v =
      __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4_t*)(p));
  return __builtin_bit_cast(half4_t, v);
}

// CAUSAL: apply the causal mask (with the query offset).  KEYMASK: key_valid
// ([B, S_k] bytes, nonzero = the key may be attended to -- the reference's
// valid_token_mask, TTB:250-253) is staged per tile and masks keys; a query
// may then see no key in a tile, or at all.  SPLIT: the block covers all
// S_q <= BQ queries of one (batch, head) but only keys [split*split_keys,
// +split_keys), and writes its unnormalised partial (o, offset, row sum) for
// attn_split_combine; that is the decode path, which needs the whole GPU on
// the key axis.  Without KEYMASK or SPLIT every query sees key 0 in the first
// tile, which keeps the offset bookkeeping to a tile-index test.
template <int HD, int NQ, int NW, bool CAUSAL, bool KEYMASK, bool SPLIT>
__global__ __launch_bounds__(64 * NW, 8 / NW) void attn_kernel(const AttnArgs a) {
  using C = AttnCfg<HD, NQ, NW>;
  constexpr int NT = C::NT, BKEYS = C::BKEYS, HDP = C::HDP, HDV = C::HDV, QPW = C::QPW, BQ = C::BQ;
  constexpr int LDK = C::LDK, LDV = C::LDV, KSTEPS = C::KSTEPS, KB = C::KB, HB = C::HB;
  constexpr int KT = C::KT, CPK = C::CPK, CH = C::CH;
  constexpr bool TRACK = KEYMASK || SPLIT;  // a query may see no key in its first tile
  // One-wave split blocks keep a single LDS tile (the next one waits in
  // registers), so more of them fit on a CU.
  constexpr int NBUF = SPLIT ? 1 : 2;
  static_assert(NT >= BKEYS, "one thread per key stages the validity bytes");

  __shared__ __attribute__((aligned(16))) half_t k_lds[NBUF][BKEYS * LDK];
  __shared__ __attribute__((aligned(16))) half_t v_lds[NBUF][BKEYS * LDV];
  __shared__ __attribute__((aligned(16))) uint8_t kv_lds[NBUF][BKEYS];  // key validity of the tile

  // Heaviest query tiles (most keys under the causal mask) are issued first.
  const int per_bh = SPLIT ? a.n_splits : a.q_tiles;
  const int bh = blockIdx.x / per_bh;
  const int sub = blockIdx.x % per_bh;
  const int qt = SPLIT ? 0 : (CAUSAL ? a.q_tiles - 1 - sub : sub);
  const int b = bh / a.H, h = bh % a.H;
  const int S_q = a.S_q, S_k = a.S_k, q_offset = a.q_offset;
  const half_t* base = a.q + (int64_t)b * a.q_bstride + (int64_t)h * HD;
  const int64_t q_rstride = a.q_rstride, k_rstride = a.k_rstride;
  const half_t* kbase = a.k + (int64_t)b * a.k_bstride + (int64_t)h * a.k_hstride;
  const half_t* vbase = a.v + (int64_t)b * a.k_bstride + (int64_t)h * a.k_hstride;
  const float scale_log2 = a.scale_log2;

  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int g = lane / 16, r16 = lane % 16;
  const int q0 = qt * BQ;
  const int qw0 = q0 + wave * QPW;

  // Zero the padding columns of both buffers once; tile stores never touch them.
  if constexpr (HDP > HD) {
    for (int i = tid; i < NBUF * BKEYS * (HDP - HD); i += NT) {
      const int buf = i / (BKEYS * (HDP - HD)), j = i % (BKEYS * (HDP - HD));
      k_lds[buf][(j / (HDP - HD)) * LDK + HD + j % (HDP - HD)] = (half_t)0.f;
    }
  }
  if constexpr (HDV > HD) {
    for (int i = tid; i < NBUF * BKEYS * (HDV - HD); i += NT) {
      const int buf = i / (BKEYS * (HDV - HD)), j = i % (BKEYS * (HDV - HD));
      v_lds[buf][(j / (HDV - HD)) * LDV + HD + j % (HDV - HD)] = (half_t)0.f;
    }
  }

  // Q fragments (B operand of S^T), pre-multiplied by scale * log2(e):
  // lane holds q[query][32*ks + 8*(l/16) .. +7].
  // Loaded unconditionally (outside the query range or past HD the lane
  // reads row 0, column 0 and zeroes the fragment afterwards), so every load
  // is in flight at once instead of one conditional load and wait per
  // fragment; scaled after the first K/V tile has been requested.
  half8_t qf[NQ][KSTEPS];
  const half8_t zero8 = {0, 0, 0, 0, 0, 0, 0, 0};
  auto q_ok = [&](int qb, int ks) { return qw0 + 16 * qb + r16 < S_q && 32 * ks + 8 * g < HD; };
#pragma unroll
  for (int qb = 0; qb < NQ; ++qb)
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      const bool ok = q_ok(qb, ks);
      const int q = ok ? qw0 + 16 * qb + r16 : 0, d = ok ? 32 * ks + 8 * g : 0;
      qf[qb][ks] = *reinterpret_cast<const half8_t*>(base + q * q_rstride + d);
    }

  // m_run: the base-2 exponent offset of query (l % 16) of block qb.  The score
  // MFMAs start from -m_run, so a tile's scores arrive already shifted; the
  // first tile with a visible key for a query moves m_run onto that tile's
  // exact maximum (m_set records that it happened; without TRACK that is
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
  const uint8_t* kvb = KEYMASK ? a.key_valid + (int64_t)b * S_k : nullptr;
  uint8_t kvreg = 0;
  half8_t kreg[CH], vreg[CH];
  auto gload = [&](int k0) {
    if (KEYMASK && tid < BKEYS) {
      const int key = k0 + tid;
      kvreg = key < S_k ? kvb[key] : (uint8_t)0;
    }
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int id = tid + NT * j;
      kreg[j] = zero8;
      vreg[j] = zero8;
      if (id < BKEYS * CPK) {
        const int key = k0 + id / CPK, c = (id % CPK) * 8;
        if (key < S_k) {
          const half8_t* kp = reinterpret_cast<const half8_t*>(kbase + key * k_rstride + c);
          const half8_t* vp = reinterpret_cast<const half8_t*>(vbase + key * k_rstride + c);
          if constexpr (SPLIT) {
            // Decode streams each cached row exactly once: non-temporal loads
            // keep it from displacing reusable lines (87% vs 77% of HBM peak
            // on a 100k-token cache).
            kreg[j] = __builtin_nontemporal_load(kp);
            vreg[j] = __builtin_nontemporal_load(vp);
          } else {
            kreg[j] = *kp;
            vreg[j] = *vp;
          }
        }
      }
    }
  };
  auto sstore = [&](int buf) {
    if (KEYMASK && tid < BKEYS) kv_lds[buf][tid] = kvreg;
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int id = tid + NT * j;
      if (id < BKEYS * CPK) {
        const int r = id / CPK, c = (id % CPK) * 8;
        *reinterpret_cast<half8_t*>(&k_lds[buf][r * LDK + c]) = kreg[j];
        *reinterpret_cast<half8_t*>(&v_lds[buf][r * LDV + c]) = vreg[j];
      }
    }
  };

  const int k_begin = SPLIT ? sub * a.split_keys : 0;
  int key_end = CAUSAL ? min(S_k, q_offset + q0 + BQ) : S_k;
  if constexpr (SPLIT) key_end = min(key_end, k_begin + a.split_keys);
  const int n_tiles = key_end > k_begin ? (key_end - k_begin + BKEYS - 1) / BKEYS : 0;
  if (n_tiles > 0) {
    gload(k_begin);
    sstore(0);
  }
#pragma unroll
  for (int qb = 0; qb < NQ; ++qb)
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      half8_t v = qf[qb][ks];
#pragma unroll
      for (int m = 0; m < 8; ++m) v[m] = (half_t)((float)v[m] * scale_log2);
      qf[qb][ks] = q_ok(qb, ks) ? v : zero8;
    }
  __syncthreads();
  for (int t = 0; t < n_tiles; ++t) {
    const int cur = NBUF == 1 ? 0 : t & 1;
    const int k0 = k_begin + t * BKEYS;
    if (t + 1 < n_tiles) gload(k0 + BKEYS);

    // Wave-uniform skip: every key of this tile lies above this wave's diagonal.
    if (!CAUSAL || k0 <= q_offset + qw0 + QPW - 1) {
      const bool diag = CAUSAL && (k0 + BKEYS - 1 > q_offset + qw0);
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
              if (k0 + 16 * jb + 4 * g + i > q_offset + qw0 + 16 * qb + r16) s[jb][qb][i] = -INFINITY;
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
      } else if (!CAUSAL && k0 + BKEYS > S_k) {
#pragma unroll
        for (int jb = 0; jb < KB; ++jb)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (k0 + 16 * jb + 4 * g + i >= S_k)
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
        if constexpr (TRACK) unset |= !m_set[qb];
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
          const bool was_set = TRACK ? m_set[qb] : t != 0;
          const float sh = was_set ? fmaxf(mx, 0.f) : (TRACK && mx == -INFINITY ? 0.f : mx);
          if constexpr (TRACK) m_set[qb] = was_set || mx != -INFINITY;
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
    if constexpr (NBUF == 1) __syncthreads();  // the tile is read completely before it is replaced
    if (t + 1 < n_tiles) sstore(NBUF == 1 ? 0 : cur ^ 1);
    __syncthreads();
  }

  if constexpr (SPLIT) {
    // Unnormalised partial of this key range: o, the offset m_run (-inf when
    // the range showed the query no key) and the row sum.
    const int64_t slot = (int64_t)bh * a.n_splits + sub;
#pragma unroll
    for (int qb = 0; qb < NQ; ++qb) {
      const int q = qw0 + 16 * qb + r16;
      if (q >= S_q) continue;
      float* wo = a.ws_o + (slot * BQ + q) * HD;
#pragma unroll
      for (int hb = 0; hb < HB; ++hb) {
        const int d = 16 * hb + 4 * g;
        if (d < HD) *reinterpret_cast<float4_t*>(wo + d) = o[hb][qb];
      }
      if (g == 0) a.ws_ml[slot * BQ + q] = make_float2(m_set[qb] ? m_run[qb] : -INFINITY, lacc[qb][0]);
    }
    return;
  }

  // Normalise: lane holds O^T[16hb + 4g + i][query r16]; every row of the
  // all-ones block holds that query's probability sum.  The wave's rows go
  // through LDS (its own rows of the freed K or V^T tiles) and leave as
  // whole-row 16-byte chunks: stored straight from the accumulators, one
  // store touched 16 rows with 8-byte pieces, and the stores took 30% of
  // the head_dim-256 kernel's time.
  static_assert(NBUF * BKEYS >= (NW - NW / 2) * QPW, "each wave's rows fit in the K or V^T tiles");
  __syncthreads();  // every wave is done with the K/V tiles
  half_t* const stg = wave < NW / 2 ? &k_lds[0][0] + wave * QPW * LDK : &v_lds[0][0] + (wave - NW / 2) * QPW * LDV;
  const int rs = wave < NW / 2 ? LDK : LDV;
#pragma unroll
  for (int qb = 0; qb < NQ; ++qb) {
    // A query that saw no key at all (every key masked) writes zeros.
    const float inv = lacc[qb][0] > 0.f ? __builtin_amdgcn_rcpf(lacc[qb][0]) : 0.f;
#pragma unroll
    for (int hb = 0; hb < HB; ++hb) {
      const int d = 16 * hb + 4 * g;
      if (d < HD) {
        half4_t r;
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = (half_t)(o[hb][qb][i] * inv);
        *reinterpret_cast<half4_t*>(stg + (16 * qb + r16) * rs + d) = r;
      }
    }
  }
  constexpr int CPR = HD / 8;  // 16-byte chunks per context row
  half_t* obase = a.out + (int64_t)b * a.o_bstride + (int64_t)h * HD;
#pragma unroll
  for (int c0 = 0; c0 < QPW * CPR; c0 += kWave) {
    const int c = c0 + lane;
    const int row = c / CPR, k = c % CPR;
    const int q = qw0 + row;
    if (c < QPW * CPR && q < S_q)
      *reinterpret_cast<half8_t*>(obase + (int64_t)q * a.o_rstride + 8 * k) =
          *reinterpret_cast<const half8_t*>(stg + row * rs + 8 * k);
  }
}

// dma16 issued from inline assembly: the compiler does not see this LDS
// write, so it adds no wait for it before later LDS reads (it cannot tell the
// ring buffer being filled from the one being read, and would wait before
// every read).  The caller waits itself (vmcnt) before the barrier that
// publishes the tile.  Any wait the compiler does emit for its own loads only
// waits longer, since it counts fewer operations in flight than there are.
__device__ __forceinline__ void dma16_untracked(const void* src_lane, void* lds_wave_base) {
  const uint32_t lds = (uint32_t)(uintptr_t)(lds_void_t*)lds_wave_base;
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src_lane), "s"(lds) : "memory", "m0");
}

// Ping-pong variant for long sequences (head_dim 64, no key mask): 8 waves in
// two groups of four, A = waves 0-3 and B = waves 4-7, one wave of each per
// SIMD.  Per 64-key tile a wave runs an MFMA phase (PV of the previous tile,
// then QK of this one) and a VALU phase (mask, offset check, exp2 and FP16
// packing of the probabilities).  Barriers split time into half-steps, and
// the groups take opposite phases in each: in half-step 2t group A does
// PV(t-1) + QK(t) while group B does the VALU work of tile t-1; in 2t+1 A does
// the VALU work of tile t while B does PV(t-1) + QK(t).  So on every SIMD one
// wave keeps the matrix core busy while the other issues the exponentials,
// instead of both waves reaching the same phase at once.
//
// K/V tiles sit in a ring of four LDS buffers (tile t in buffer t % 4) and
// arrive by direct global -> LDS loads (no VGPRs in between).  Tile t is read
// from half-step 2t (A's QK) to 2t+3 (B's PV); the loads of tile t+2 are
// issued in half-step 2t (into the buffer of tile t-2, last read in 2t-1) and
// waited for at the end of 2t+3.  Rows are 128 bytes, unpadded
// (a load fills 1 KB = 8 rows contiguously); chunk c of row r sits in slot
// c ^ (r & 7), applied on the global side, which keeps the K fragment reads
// and the transposing V reads free of bank conflicts.  Same arithmetic as
// attn_kernel (offset in the score accumulator, lazy rescale, MFMA row sums).
template <int HD, bool CAUSAL, bool VT = false>
__global__ __launch_bounds__(512, 1) void attn_pp_kernel(const AttnArgs a) {
  constexpr int NQ = 4, NW = 8;
  using C = AttnCfg<HD, NQ, NW>;
  constexpr int NT = C::NT, BKEYS = C::BKEYS, QPW = C::QPW, BQ = C::BQ;
  constexpr int LDK = C::LDK, LDV = C::LDV, KSTEPS = C::KSTEPS, KB = C::KB, HB = C::HB;
  constexpr int KT = C::KT, CPK = C::CPK, CH = C::CH;
  static_assert(HD == 64 && C::HDP == 64 && C::HDV == 64, "128-byte rows");
  static_assert(BKEYS == 8 * NW, "one 8-row load per wave per tile");
  constexpr int NBUF = 4;
  constexpr int ROW = HD;  // halves per LDS row

  __shared__ __attribute__((aligned(1024))) half_t k_lds[NBUF][BKEYS * ROW];
  __shared__ __attribute__((aligned(1024))) half_t v_lds[NBUF][BKEYS * ROW];
  // Q operands, fragment-major (wave, qb, ks, lane): re-read per tile rather
  // than held in 32 VGPRs, which two waves per SIMD cannot spare.
  __shared__ __attribute__((aligned(16))) half8_t q_lds[NW][NQ][KSTEPS][kWave];

  const int per_bh = a.q_tiles;
  const int bh = blockIdx.x / per_bh;
  const int sub = blockIdx.x % per_bh;
  const int qt = CAUSAL ? a.q_tiles - 1 - sub : sub;  // heaviest query tiles first
  const int b = bh / a.H, h = bh % a.H;
  const int S_q = a.S_q, S_k = a.S_k, q_offset = a.q_offset;
  const half_t* base = a.q + (int64_t)b * a.q_bstride + (int64_t)h * HD;
  const int64_t q_rstride = a.q_rstride, k_rstride = a.k_rstride;
  const half_t* kbase = a.k + (int64_t)b * a.k_bstride + (int64_t)h * a.k_hstride;
  const half_t* vbase = a.v + (int64_t)b * a.k_bstride + (int64_t)h * a.k_hstride;
  // VT: row d of head (b, h) of the transposed V; tile t is its 128 bytes from key 64t.
  const half_t* vtbase = VT ? a.vt + ((int64_t)b * a.H + h) * HD * a.vt_row : nullptr;
  const float scale_log2 = a.scale_log2;

  const int tid = threadIdx.x, lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int g = lane / 16, r16 = lane % 16;
  const int q0 = qt * BQ;
  const int qw0 = q0 + wave * QPW;
  // Waves w and w + 4 share a SIMD (measured: pairing them by the SIMD id in
  // HW_ID gives the same time; pairing w and w + 1 runs 1.6x slower).  Only
  // the schedule depends on it, not the result.
  const bool group_a = wave < NW / 2;

  const half8_t zero8 = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int qb = 0; qb < NQ; ++qb) {
    const int q = qw0 + 16 * qb + r16;
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      half8_t v = zero8;
      if (q < S_q) {
        v = *reinterpret_cast<const half8_t*>(base + q * q_rstride + 32 * ks + 8 * g);
#pragma unroll
        for (int m = 0; m < 8; ++m) v[m] = (half_t)((float)v[m] * scale_log2);
      }
      q_lds[wave][qb][ks][lane] = v;  // read back only by this wave, after the first barrier
    }
  }
  float4_t o[HB][NQ], lacc[NQ];
  float4_t minit[NQ];  // -m_run broadcast: the score accumulators' start value
#pragma unroll
  for (int qb = 0; qb < NQ; ++qb) {
#pragma unroll
    for (int hb = 0; hb < HB; ++hb) o[hb][qb] = float4_t{0.f, 0.f, 0.f, 0.f};
    lacc[qb] = float4_t{0.f, 0.f, 0.f, 0.f};
    minit[qb] = float4_t{0.f, 0.f, 0.f, 0.f};
  }
  const half8_t ones8 = {1, 1, 1, 1, 1, 1, 1, 1};

  // Tile loads: wave w fills rows 8w .. 8w+7 of the K and V buffers; lane i
  // fetches the chunk that belongs in slot i % 8 of row i / 8.  Rows past S_k
  // repeat row S_k - 1: those keys are masked (causal: they follow every
  // query; otherwise explicitly), so their probabilities are exactly 0, and a
  // real row is finite.
  const int ld_row = 8 * wave + lane / 8, ld_chunk = (lane % 8) ^ (lane / 8);
  auto dma_tile = [&](int t) {  // tile t into buffer t % NBUF
    const int64_t off = (int64_t)min(t * BKEYS + ld_row, S_k - 1) * k_rstride + 8 * ld_chunk;
    const int buf = t & (NBUF - 1);
    dma16_untracked(kbase + off, &k_lds[buf][8 * wave * ROW]);
    if constexpr (VT)  // rows are head dims here; keys past S_k are the GEMM's zeros
      dma16_untracked(vtbase + (int64_t)ld_row * a.vt_row + t * BKEYS + 8 * ld_chunk, &v_lds[buf][8 * wave * ROW]);
    else
      dma16_untracked(vbase + off, &v_lds[buf][8 * wave * ROW]);
  };
  // Barrier over LDS traffic only: the next tile's loads stay in flight ...
  auto half_step_barrier = [] {
    __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));  // vmcnt(63) expcnt(7) lgkmcnt(0)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  // ... except at the end of odd half-steps, where they must have landed.
  auto tile_barrier = [] {
    __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (0 << 8) | (0 << 14));  // vmcnt(0) expcnt(7) lgkmcnt(0)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  // With the tile after next in flight (its two loads are this wave's newest).
  auto tile_barrier_ahead = [](bool ahead) {
    if (ahead)
      __builtin_amdgcn_s_waitcnt(2 | (7 << 4) | (0 << 8) | (0 << 14));  // vmcnt(2) expcnt(7) lgkmcnt(0)
    else
      __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (0 << 8) | (0 << 14));
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

  int key_end = CAUSAL ? min(S_k, q_offset + q0 + BQ) : S_k;
  const int n_tiles = (key_end + BKEYS - 1) / BKEYS;
  // Tiles past this wave's last query (causal) are skipped by the wave, not by
  // the workgroup: every wave passes every barrier.
  auto active = [&](int t) { return t >= 0 && t < n_tiles && (!CAUSAL || t * BKEYS <= q_offset + qw0 + QPW - 1); };

  float4_t s[KB][NQ];
  half8_t pf[KT][NQ];

  // QK of tile t into s (offset already subtracted).
  // Lane parts of the LDS addresses come from opaque copies inside each call,
  // so they stay one base register plus instruction offsets instead of being
  // hoisted out of the tile loop as one register per fragment (and spilled).
  auto mma_qk = [&](int t) {
    // Row 16 jb + r16, chunk 4 ks + g, in slot (4 ks + g) ^ (r16 & 7).
    int ql = lane, kc = g ^ (r16 & 7), kr = r16 * ROW;
    asm volatile("" : "+v"(ql), "+v"(kc), "+v"(kr));
    const half_t* kt_lds = k_lds[t & (NBUF - 1)];
    const half_t* kp[KSTEPS] = {kt_lds + kr + 8 * kc, kt_lds + kr + 8 * (kc ^ 4)};
    // K fragments run two key blocks ahead of their products, in two slots
    // (a slot is refilled right after the products that read it issue).
    half8_t kf[2][KSTEPS];
    auto read_k = [&](int jb) {
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks) kf[jb % 2][ks] = *reinterpret_cast<const half8_t*>(kp[ks] + 16 * jb * ROW);
    };
    read_k(0);
    half8_t qf[NQ][KSTEPS];
#pragma unroll
    for (int qb = 0; qb < NQ; ++qb)
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks) qf[qb][ks] = q_lds[wave][qb][ks][ql];
    read_k(1);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int jb = 0; jb < KB; ++jb) {
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks)
#pragma unroll
        for (int qb = 0; qb < NQ; ++qb)
          s[jb][qb] = mfma16x16x32(kf[jb % 2][ks], qf[qb][ks], ks == 0 ? minit[qb] : s[jb][qb]);
      if (jb + 2 < KB) read_k(jb + 2);
    }
  };
  // O^T += V^T . P^T of tile t (and the row sums).
  auto mma_pv = [&](int t) {
    // Lane (g, j) reads 8 bytes of row 32 kt + 4 g + j / 4 (+16 for the high
    // half) at half 4 (j % 4) + 16 hb: chunk 2 hb + (j % 4) / 2, which sits in
    // slot chunk ^ (row & 7) = cb ^ 2 hb.
    int vr = (4 * g + r16 / 4) * ROW + 4 * (r16 % 2), cb = ((r16 % 4) / 2) ^ ((4 * g + r16 / 4) & 7);
    asm volatile("" : "+v"(vr), "+v"(cb));
    const half_t* vt_lds = v_lds[t % NBUF] + vr;
    // V fragments run two steps (4 kt + hb) ahead of their products in a
    // ring of three; the row-sum products, which read no LDS, go first and
    // cover the first two reads.  The sched_barriers keep that order.
    half8_t vf[3];
    // VT: the tile holds V^T (row = head dim, chunk 4kt + g = keys of the
    // P operand's lane group g in step kt), one 16-byte read per fragment.
    int tr = r16 * ROW, tg = g, ts = r16 & 7;
    if constexpr (VT) asm volatile("" : "+v"(tr), "+v"(tg), "+v"(ts));
    auto read_v = [&](int step) {
      const int kt = step / HB, hb = step % HB;
      if constexpr (VT) {
        vf[step % 3] = *reinterpret_cast<const half8_t*>(v_lds[t % NBUF] + 16 * hb * ROW + tr + 8 * ((4 * kt + tg) ^ ts));
      } else {
        const half_t* vrow = vt_lds + 32 * kt * ROW;
        const int slot = 8 * (cb ^ (2 * hb));
        const half4_t lo = lds_read_tr16(vrow + slot);
        const half4_t hi = lds_read_tr16(vrow + 16 * ROW + slot);
        vf[step % 3] = half8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      }
    };
    read_v(0);
    read_v(1);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int qb = 0; qb < NQ; ++qb) lacc[qb] = mfma16x16x32(ones8, pf[kt][qb], lacc[qb]);
#pragma unroll
    for (int step = 0; step < KT * HB; ++step) {
      __builtin_amdgcn_sched_barrier(0);
      if (step + 2 < KT * HB) read_v(step + 2);
      const int kt = step / HB, hb = step % HB;
#pragma unroll
      for (int qb = 0; qb < NQ; ++qb) o[hb][qb] = mfma16x16x32(vf[step % 3], pf[kt][qb], o[hb][qb]);
    }
  };
  // Mask, offset check / rescale, probabilities of tile t.
  auto softmax = [&](int t) {
    const int k0 = t * BKEYS;
    // The mask thresholds below come from opaque copies of the lane
    // coordinates: otherwise the compiler hoists all 64 lane constants out of
    // the tile loop and spills them.
    int g = lane / 16, r16 = lane % 16;
    asm volatile("" : "+v"(g), "+v"(r16));
    // One key block at a time: formed all at once, the 64 compare masks would
    // need 128 SGPRs.
    if (CAUSAL && k0 + BKEYS - 1 > q_offset + qw0) {
      const int d = 4 * g - r16 + k0 - q_offset - qw0;  // key - query of element (0, 0, 0)
#pragma unroll
      for (int jb = 0; jb < KB; ++jb) {
#pragma unroll
        for (int qb = 0; qb < NQ; ++qb)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (d + 16 * jb + i > 16 * qb) s[jb][qb][i] = -INFINITY;
        __builtin_amdgcn_sched_barrier(0);
      }
    } else if (!CAUSAL && k0 + BKEYS > S_k) {
#pragma unroll
      for (int jb = 0; jb < KB; ++jb) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (k0 + 16 * jb + 4 * g + i >= S_k)
#pragma unroll
            for (int qb = 0; qb < NQ; ++qb) s[jb][qb][i] = -INFINITY;
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    float lm = -INFINITY;
#pragma unroll
    for (int qb = 0; qb < NQ; ++qb)
#pragma unroll
      for (int jb = 0; jb < KB; ++jb)
        lm = fmaxf(lm, fmaxf(fmaxf(s[jb][qb][0], s[jb][qb][1]), fmaxf(s[jb][qb][2], s[jb][qb][3])));
    if (__any(t == 0 || lm > 8.0f)) {
#pragma unroll
      for (int qb = 0; qb < NQ; ++qb) {
        float m = -INFINITY;
#pragma unroll
        for (int jb = 0; jb < KB; ++jb)
          m = fmaxf(m, fmaxf(fmaxf(s[jb][qb][0], s[jb][qb][1]), fmaxf(s[jb][qb][2], s[jb][qb][3])));
        const float mx = quad_group_max(m);
        // Tile 0 shows every query key 0, so its maximum is finite: the offset
        // jumps there with nothing to rescale; later sh >= 0 and corr <= 1.
        const float sh = t != 0 ? fmaxf(mx, 0.f) : mx;
        const float corr = t != 0 ? __builtin_amdgcn_exp2f(-sh) : 1.f;
        minit[qb] -= sh;
#pragma unroll
        for (int hb = 0; hb < HB; ++hb) o[hb][qb] *= corr;
        lacc[qb] *= corr;
#pragma unroll
        for (int jb = 0; jb < KB; ++jb) s[jb][qb] -= sh;
      }
    }
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int qb = 0; qb < NQ; ++qb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pf[kt][qb][i] = (half_t)__builtin_amdgcn_exp2f(s[2 * kt][qb][i]);
          pf[kt][qb][4 + i] = (half_t)__builtin_amdgcn_exp2f(s[2 * kt + 1][qb][i]);
        }
  };
  auto mfma_phase = [&](int t) {
    __builtin_amdgcn_s_setprio(1);
    if (active(t - 1)) mma_pv(t - 1);
    // The probabilities die before the scores are born: no interleaving of
    // the two products, which would need both live (96 more VGPRs).
    __builtin_amdgcn_sched_barrier(0);
    if (active(t)) mma_qk(t);
    __builtin_amdgcn_s_setprio(0);
  };

  if (n_tiles > 0) dma_tile(0);
  if (1 < n_tiles) dma_tile(1);
  tile_barrier_ahead(1 < n_tiles);  // tile 0 and the Q operands have landed
  // The two groups run separate copies of the loop, each passing the same
  // 2 (n_tiles + 1) barriers, rotated so that only the probabilities (not the
  // scores) cross the back edge.  Every wave issues its share of tile t+2's
  // loads at the start of half-step 2t (into the buffer of tile t-2, which
  // every wave left at the end of 2t-1) and waits for tile t+1's at the end
  // of 2t+1, with tile t+2's still in flight (four buffers: one tile more of
  // latency hidden than with three, 1% faster on cfg5).
  if (group_a) {
    for (int t = 0; t <= n_tiles; ++t) {
      if (t + 2 < n_tiles) dma_tile(t + 2);
      mfma_phase(t);  // half-step 2t: PV(t-1) + QK(t)
      half_step_barrier();
      if (active(t)) softmax(t);  // half-step 2t+1
      tile_barrier_ahead(t + 2 < n_tiles);
    }
  } else {
    if (2 < n_tiles) dma_tile(2);
    half_step_barrier();  // half-step 0: nothing to exponentiate yet
    for (int t = 0; t < n_tiles; ++t) {
      mfma_phase(t);  // half-step 2t+1: PV(t-1) + QK(t)
      tile_barrier_ahead(t + 2 < n_tiles);
      if (t + 3 < n_tiles) dma_tile(t + 3);
      if (active(t)) softmax(t);  // half-step 2t+2
      half_step_barrier();
    }
    mfma_phase(n_tiles);  // half-step 2 n_tiles + 1: PV of the last tile
    tile_barrier();
  }

  half_t* obase = a.out + (int64_t)b * a.o_bstride + (int64_t)h * HD;
#pragma unroll
  for (int qb = 0; qb < NQ; ++qb) {
    const float inv = lacc[qb][0] > 0.f ? __builtin_amdgcn_rcpf(lacc[qb][0]) : 0.f;
    const int q = qw0 + 16 * qb + r16;
    if (q >= S_q) continue;
#pragma unroll
    for (int hb = 0; hb < HB; ++hb) {
      half4_t r;
#pragma unroll
      for (int i = 0; i < 4; ++i) r[i] = (half_t)(o[hb][qb][i] * inv);
      *reinterpret_cast<half4_t*>(obase + (int64_t)q * a.o_rstride + 16 * hb + 4 * g) = r;
    }
  }
}

// Merges the key-range partials of attn_kernel<..., SPLIT>: per (batch, head,
// query) M = max_s m_s, out = sum_s 2^(m_s - M) o_s / sum_s 2^(m_s - M) l_s.
// One thread per 8 context columns.
template <int HD>
__global__ __launch_bounds__(256) void attn_split_combine(const AttnArgs a, int BQ, int64_t total) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= total) return;
  constexpr int C8 = HD / 8;
  const int c = (int)(idx % C8);
  const int64_t rest = idx / C8;
  const int q = (int)(rest % a.S_q);
  const int64_t bh = rest / a.S_q;
  const int b = (int)(bh / a.H), h = (int)(bh % a.H);
  const float2* ml = a.ws_ml + bh * a.n_splits * BQ + q;
  float m = -INFINITY;
  for (int s = 0; s < a.n_splits; ++s) m = fmaxf(m, ml[(int64_t)s * BQ].x);
  float l = 0.f, acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < a.n_splits; ++s) {
    const float2 p = ml[(int64_t)s * BQ];
    if (p.x == -INFINITY) continue;
    const float w = __builtin_amdgcn_exp2f(p.x - m);
    l = fmaf(w, p.y, l);
    const float* wo = a.ws_o + ((bh * a.n_splits + s) * BQ + q) * HD + 8 * c;
    const float4_t lo = *reinterpret_cast<const float4_t*>(wo);
    const float4_t hi = *reinterpret_cast<const float4_t*>(wo + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[i] = fmaf(w, lo[i], acc[i]);
      acc[4 + i] = fmaf(w, hi[i], acc[4 + i]);
    }
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  half8_t r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (half_t)(acc[i] * inv);
  *reinterpret_cast<half8_t*>(a.out + (int64_t)b * a.o_bstride + (int64_t)q * a.o_rstride +
                              (int64_t)h * HD + 8 * c) = r;
}

template <int HD, int NQ, int NW = 4>
static hipError_t launch_attn(AttnArgs a, int B, int causal, hipStream_t s) {
  constexpr int BQ = AttnCfg<HD, NQ, NW>::BQ;
  a.q_tiles = (a.S_q + BQ - 1) / BQ;
  const int64_t blocks = (int64_t)a.q_tiles * B * a.H;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  const dim3 grid((unsigned)blocks), block(AttnCfg<HD, NQ, NW>::NT);
  if (a.key_valid != nullptr) {
    if (causal)
      hipLaunchKernelGGL((attn_kernel<HD, NQ, NW, true, true, false>), grid, block, 0, s, a);
    else
      hipLaunchKernelGGL((attn_kernel<HD, NQ, NW, false, true, false>), grid, block, 0, s, a);
  } else {
    if (causal)
      hipLaunchKernelGGL((attn_kernel<HD, NQ, NW, true, false, false>), grid, block, 0, s, a);
    else
      hipLaunchKernelGGL((attn_kernel<HD, NQ, NW, false, false, false>), grid, block, 0, s, a);
  }
  return hipGetLastError();
}

template <int HD>
static hipError_t launch_attn_pp(AttnArgs a, int B, int causal, hipStream_t s) {
  constexpr int BQ = AttnCfg<HD, 4, 8>::BQ;
  a.q_tiles = (a.S_q + BQ - 1) / BQ;
  const int64_t blocks = (int64_t)a.q_tiles * B * a.H;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  if (a.vt != nullptr) {  // causal only (the caller checked)
    hipLaunchKernelGGL((attn_pp_kernel<HD, true, true>), dim3((unsigned)blocks), dim3(512), 0, s, a);
    return hipGetLastError();
  }
  if (causal)
    hipLaunchKernelGGL((attn_pp_kernel<HD, true>), dim3((unsigned)blocks), dim3(512), 0, s, a);
  else
    hipLaunchKernelGGL((attn_pp_kernel<HD, false>), dim3((unsigned)blocks), dim3(512), 0, s, a);
  return hipGetLastError();
}

constexpr int kPingPongMinQueries = 4096;  // query ranges from here on take the ping-pong kernel
constexpr int kCUs = 256;  // MI355X compute units

// Kernel variants (XB_ATTN_*) and the head widths each is built for.
static bool attention_variant_fits(int variant, int hd, bool masked) {
  switch (variant) {
    case XB_ATTN_W4_Q16: case XB_ATTN_W8_Q16: return hd == 256;
    case XB_ATTN_W4_Q32: return hd <= 128;
    case XB_ATTN_W4_Q64: return hd <= 64;
    case XB_ATTN_PINGPONG: return hd == 64 && !masked;
    default: return false;
  }
}

// The library's choice.  head_dim 256 up to 128 queries: one 8-wave block
// takes all of them, so each K/V row is fetched once per (batch, head)
// instead of by two 64-query blocks (cfg3's geometry: 16.7 vs 18.6 us) -- when
// the B*H blocks still fill the GPU.  head_dim 64 without a key mask from
// kPingPongMinQueries on: the ping-pong kernel.  Other long ranges take 64
// queries per wave (each K/V fragment read from LDS then feeds 4 MFMAs);
// short ones keep 32 so a block does not outgrow S_q.
static int select_attention(int64_t B, int S_q, int H, int hd, bool masked) {
  if (hd >= 256) return S_q <= 128 && B * H >= kCUs ? XB_ATTN_W8_Q16 : XB_ATTN_W4_Q16;
  if (hd >= 128) return XB_ATTN_W4_Q32;
  if (hd == 64 && !masked && S_q >= kPingPongMinQueries) return XB_ATTN_PINGPONG;
  return S_q >= 1024 ? XB_ATTN_W4_Q64 : XB_ATTN_W4_Q32;
}

template <int HD>
static hipError_t run_attn(int variant, const AttnArgs& a, int B, int causal, hipStream_t s) {
  if constexpr (HD >= 256) {
    if (variant == XB_ATTN_W8_Q16) return launch_attn<HD, 1, 8>(a, B, causal, s);
    return launch_attn<HD, 1>(a, B, causal, s);
  } else if constexpr (HD >= 128) {
    return launch_attn<HD, 2>(a, B, causal, s);
  } else {
    if constexpr (HD == 64) {
      if (variant == XB_ATTN_PINGPONG) return launch_attn_pp<HD>(a, B, causal, s);
    }
    if (variant == XB_ATTN_W4_Q64) return launch_attn<HD, 4>(a, B, causal, s);
    return launch_attn<HD, 2>(a, B, causal, s);
  }
}

template <int HD>
static hipError_t dispatch_attn(const AttnArgs& a, int B, int causal, hipStream_t s) {
  return run_attn<HD>(select_attention(B, a.S_q, a.H, HD, a.key_valid != nullptr), a, B, causal, s);
}

// Decode (at most kDecodeQueries new tokens per sequence): one-wave blocks,
// each over a range of whole key tiles, sized so B*H*splits comes to about
// eight waves per CU when the cache is long enough.
constexpr int kDecodeQueries = 16;
constexpr int64_t kDecodeTargetBlocks = 2048;

struct DecodeGeometry {
  int n_splits, split_keys;
  int64_t o_bytes, bytes;  // partial o, then (offset, sum) pairs
};

// Bytes of one split's partials for one (batch, head): kDecodeQueries rows of
// HD FP32 outputs plus an (offset, sum) pair each.
static int64_t decode_split_bytes(int HD) {
  return (int64_t)kDecodeQueries * (HD * (int64_t)sizeof(float) + (int64_t)sizeof(float2));
}

// The split count is also capped so that the partials fit the no-allocation
// entry point's static scratch whenever one split per (batch, head) does:
// both entry points then run the same geometry and give the same bits.
static DecodeGeometry decode_geometry(int B, int H, int S_k, int HD) {
  const int bk = HD >= 256 ? 32 : 64;
  const int tiles = (S_k + bk - 1) / bk;
  const int64_t bh = (int64_t)B * H;
  const int64_t fit = std::max<int64_t>(1, XB_DECODE_SCRATCH_BYTES / (bh * decode_split_bytes(HD)));
  const int64_t want = std::min<int64_t>(std::min<int64_t>(tiles, fit),
                                         std::max<int64_t>(1, (kDecodeTargetBlocks + bh - 1) / bh));
  const int tiles_per = (int)((tiles + want - 1) / want);
  DecodeGeometry g;
  g.split_keys = tiles_per * bk;
  g.n_splits = (S_k + g.split_keys - 1) / g.split_keys;
  const int64_t slots = bh * g.n_splits * kDecodeQueries;
  g.o_bytes = slots * HD * (int64_t)sizeof(float);
  g.bytes = g.o_bytes + slots * (int64_t)sizeof(float2);
  return g;
}

template <int HD>
static hipError_t launch_decode(AttnArgs a, int B, const DecodeGeometry& geo, void* workspace, hipStream_t s) {
  static_assert(AttnCfg<HD, 1, 1>::BQ == kDecodeQueries, "one wave of 16 queries");
  a.n_splits = geo.n_splits;
  a.split_keys = geo.split_keys;
  a.ws_o = static_cast<float*>(workspace);
  a.ws_ml = reinterpret_cast<float2*>(static_cast<char*>(workspace) + geo.o_bytes);
  const int64_t blocks = (int64_t)B * a.H * geo.n_splits;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL((attn_kernel<HD, 1, 1, true, false, true>), dim3((unsigned)blocks), dim3(64), 0, s, a);
  const int64_t total = (int64_t)B * a.H * a.S_q * (HD / 8);
  const int64_t cblocks = (total + 255) / 256;
  if (cblocks > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL((attn_split_combine<HD>), dim3((unsigned)cblocks), dim3(256), 0, s, a, kDecodeQueries, total);
  return hipGetLastError();
}

// Copies the new tokens' keys and values out of the packed projection into
// the [B, H, capacity, hd] caches at positions start .. start + chunk - 1.
// One thread per 16 bytes of K (and the same 16 bytes of V).
__global__ __launch_bounds__(256) void kv_append_kernel(const half_t* __restrict__ qkv, half_t* __restrict__ kc,
                                                       half_t* __restrict__ vc, int H, int HD, int chunk,
                                                       int64_t start, int64_t cap, int64_t total) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= total) return;
  const int c8 = HD / 8;
  const int c = (int)(idx % c8);
  int64_t rest = idx / c8;
  const int h = (int)(rest % H);
  rest /= H;
  const int t = (int)(rest % chunk);
  const int64_t b = rest / chunk;
  const int64_t D = (int64_t)H * HD;
  const half_t* src = qkv + (b * chunk + t) * 3 * D + D + (int64_t)h * HD + 8 * c;
  const int64_t dst = ((b * H + h) * cap + start + t) * HD + 8 * c;
  *reinterpret_cast<half8_t*>(kc + dst) = *reinterpret_cast<const half8_t*>(src);
  *reinterpret_cast<half8_t*>(vc + dst) = *reinterpret_cast<const half8_t*>(src + D);
}

static bool supported_head_dim(int hd) {
  return hd == 8 || hd == 16 || hd == 32 || hd == 64 || hd == 128 || hd == 256;
}

template <typename F>
static hipError_t by_head_dim(int hd, F&& f) {
  switch (hd) {
    case 8: return f(std::integral_constant<int, 8>());
    case 16: return f(std::integral_constant<int, 16>());
    case 32: return f(std::integral_constant<int, 32>());
    case 64: return f(std::integral_constant<int, 64>());
    case 128: return f(std::integral_constant<int, 128>());
    default: return f(std::integral_constant<int, 256>());
  }
}

}  // namespace xb

using namespace xb;

static int check_attention(int32_t batch, int64_t seq_len, int32_t heads, int32_t head_dim) {
  if (batch < 0 || seq_len < 0 || heads <= 0 || head_dim <= 0) return XB_ERR_BAD_SIZE;
  if (seq_len > 0x7fffffffLL / 4) return XB_ERR_BAD_SIZE;
  if (3LL * heads * head_dim > 0x7fffffffLL) return XB_ERR_BAD_SIZE;
  if (!supported_head_dim(head_dim)) return XB_ERR_UNSUPPORTED_SHAPE;
  return XB_OK;
}

extern "C" int xb_select_attention(int32_t batch, int64_t seq_len, int32_t heads, int32_t head_dim,
                                   int32_t masked) {
  const int bad = check_attention(batch, seq_len, heads, head_dim);
  return bad ? bad : select_attention(batch, (int)seq_len, heads, head_dim, masked != 0);
}

extern "C" int xb_attention_v(const void* qkv, void* out, const uint8_t* key_valid, int32_t batch,
                              int64_t seq_len, int32_t heads, int32_t head_dim, float scale, int32_t causal,
                              int variant, void* stream) {
  const int bad = check_attention(batch, seq_len, heads, head_dim);
  if (bad) return bad;
  const bool masked = key_valid != nullptr;
  if (variant == XB_VARIANT_AUTO) variant = select_attention(batch, (int)seq_len, heads, head_dim, masked);
  if (!attention_variant_fits(variant, head_dim, masked)) return XB_ERR_BAD_VARIANT;
  if (batch == 0 || seq_len == 0) return XB_OK;  // empty tensors may carry NULL data pointers
  if (!qkv || !out) return XB_ERR_NULL_POINTER;
  if (((uintptr_t)qkv | (uintptr_t)out) & 15u) return XB_ERR_MISALIGNED;
  const int S = (int)seq_len;
  const int64_t D = (int64_t)heads * head_dim;
  AttnArgs a = {};
  a.q = static_cast<const half_t*>(qkv);
  a.k = a.q + D;
  a.v = a.q + 2 * D;
  a.out = static_cast<half_t*>(out);
  a.key_valid = key_valid;
  a.q_bstride = a.k_bstride = (int64_t)S * 3 * D;
  a.k_hstride = head_dim;
  a.o_bstride = (int64_t)S * D;
  a.q_rstride = a.k_rstride = (int)(3 * D);
  a.o_rstride = (int)D;
  a.H = heads;
  a.S_q = a.S_k = S;
  a.scale_log2 = scale * 1.44269504088896340736f;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int c = causal ? 1 : 0;
  return (int)by_head_dim(head_dim, [&](auto hd) { return run_attn<decltype(hd)::value>(variant, a, batch, c, s); });
}

extern "C" int xb_attention_causal_vt(const void* qkv, const void* vt, void* out, int32_t batch, int64_t seq_len,
                                      int32_t heads, int32_t head_dim, float scale, void* stream) {
  const int bad = check_attention(batch, seq_len, heads, head_dim);
  if (bad) return bad;
  if (head_dim != 64 || seq_len % 32 != 0) return XB_ERR_UNSUPPORTED_SHAPE;
  if (batch == 0 || seq_len == 0) return XB_OK;
  if (!qkv || !vt || !out) return XB_ERR_NULL_POINTER;
  if (((uintptr_t)qkv | (uintptr_t)vt | (uintptr_t)out) & 15u) return XB_ERR_MISALIGNED;
  const int S = (int)seq_len;
  const int64_t D = (int64_t)heads * head_dim;
  AttnArgs a = {};
  a.q = static_cast<const half_t*>(qkv);
  a.k = a.q + D;
  a.v = nullptr;
  a.vt = static_cast<const half_t*>(vt);
  a.vt_row = (seq_len + 63) / 64 * 64;
  a.out = static_cast<half_t*>(out);
  a.q_bstride = a.k_bstride = (int64_t)S * 3 * D;
  a.k_hstride = head_dim;
  a.o_bstride = (int64_t)S * D;
  a.q_rstride = a.k_rstride = (int)(3 * D);
  a.o_rstride = (int)D;
  a.H = heads;
  a.S_q = a.S_k = S;
  a.scale_log2 = scale * 1.44269504088896340736f;
  return (int)launch_attn_pp<64>(a, batch, 1, static_cast<hipStream_t>(stream));
}

extern "C" int xb_attention(const void* qkv, void* out, const uint8_t* key_valid, int32_t batch,
                            int64_t seq_len, int32_t heads, int32_t head_dim, float scale, int32_t causal,
                            void* stream) {
  return xb_attention_v(qkv, out, key_valid, batch, seq_len, heads, head_dim, scale, causal, XB_VARIANT_AUTO,
                        stream);
}

extern "C" int xb_attention_causal(const void* qkv, void* out, int32_t batch, int64_t seq_len,
                                   int32_t heads, int32_t head_dim, float scale, void* stream) {
  return xb_attention(qkv, out, nullptr, batch, seq_len, heads, head_dim, scale, 1, stream);
}

static int check_cache_args(int32_t batch, int64_t chunk, int32_t heads, int32_t head_dim, int64_t start,
                            int64_t capacity) {
  if (batch < 0 || chunk < 0 || heads <= 0 || head_dim <= 0 || start < 0 || capacity < 0) return XB_ERR_BAD_SIZE;
  if (capacity > 0x7fffffffLL / 4 || start + chunk > capacity) return XB_ERR_BAD_SIZE;
  if (3LL * heads * head_dim > 0x7fffffffLL) return XB_ERR_BAD_SIZE;
  if (!supported_head_dim(head_dim)) return XB_ERR_UNSUPPORTED_SHAPE;
  return XB_OK;
}

extern "C" int xb_kv_cache_append(const void* qkv, void* k_cache, void* v_cache, int32_t batch, int64_t chunk,
                                  int32_t heads, int32_t head_dim, int64_t start, int64_t capacity, void* stream) {
  const int bad = check_cache_args(batch, chunk, heads, head_dim, start, capacity);
  if (bad) return bad;
  if (batch == 0 || chunk == 0) return XB_OK;
  if (!qkv || !k_cache || !v_cache) return XB_ERR_NULL_POINTER;
  if (((uintptr_t)qkv | (uintptr_t)k_cache | (uintptr_t)v_cache) & 15u) return XB_ERR_MISALIGNED;
  const int64_t total = (int64_t)batch * chunk * heads * (head_dim / 8);
  const int64_t blocks = (total + 255) / 256;
  if (blocks > 0x7fffffffLL) return XB_ERR_BAD_SIZE;
  hipLaunchKernelGGL(kv_append_kernel, dim3((unsigned)blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const half_t*>(qkv), static_cast<half_t*>(k_cache), static_cast<half_t*>(v_cache),
                     heads, head_dim, (int)chunk, start, capacity, total);
  return (int)hipGetLastError();
}

extern "C" int64_t xb_attention_kv_cache_workspace_bytes(int32_t batch, int64_t chunk, int32_t heads,
                                                         int32_t head_dim, int64_t start) {
  const int bad = check_cache_args(batch, chunk, heads, head_dim, start, start + chunk);
  if (bad) return bad;
  if (batch == 0 || chunk == 0 || chunk > kDecodeQueries) return 0;
  return decode_geometry(batch, heads, (int)(start + chunk), head_dim).bytes;
}

// The cached-attention call behind xb_attention_kv_cache and its no-allocation
// variant.  `workspace_of(bytes, &ptr)` supplies the decode partials' memory
// (or an error code) once the call has been validated and sized.
template <typename WorkspaceOf>
static int attention_kv_cache(const void* qkv, const void* k_cache, const void* v_cache, void* out, int32_t batch,
                              int64_t chunk, int32_t heads, int32_t head_dim, int64_t start, int64_t capacity,
                              float scale, void* stream, WorkspaceOf&& workspace_of) {
  const int bad = check_cache_args(batch, chunk, heads, head_dim, start, capacity);
  if (bad) return bad;
  if (batch == 0 || chunk == 0) return XB_OK;
  if (!qkv || !k_cache || !v_cache || !out) return XB_ERR_NULL_POINTER;
  if (((uintptr_t)qkv | (uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)out) & 15u) return XB_ERR_MISALIGNED;
  const int64_t D = (int64_t)heads * head_dim;
  AttnArgs a = {};
  a.q = static_cast<const half_t*>(qkv);
  a.k = static_cast<const half_t*>(k_cache);
  a.v = static_cast<const half_t*>(v_cache);
  a.out = static_cast<half_t*>(out);
  a.q_bstride = chunk * 3 * D;
  a.q_rstride = (int)(3 * D);
  a.k_bstride = heads * capacity * head_dim;
  a.k_hstride = capacity * head_dim;
  a.k_rstride = head_dim;
  a.o_bstride = chunk * D;
  a.o_rstride = (int)D;
  a.H = heads;
  a.S_q = (int)chunk;
  a.S_k = (int)(start + chunk);
  a.q_offset = (int)start;
  a.scale_log2 = scale * 1.44269504088896340736f;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (chunk > kDecodeQueries)
    return (int)by_head_dim(head_dim, [&](auto hd) { return dispatch_attn<decltype(hd)::value>(a, batch, 1, s); });
  const DecodeGeometry geo = decode_geometry(batch, heads, a.S_k, head_dim);
  void* workspace = nullptr;
  const int got = workspace_of(geo.bytes, &workspace);
  if (got != XB_OK) return got;
  return (int)by_head_dim(head_dim, [&](auto hd) { return launch_decode<decltype(hd)::value>(a, batch, geo, workspace, s); });
}

extern "C" int xb_attention_kv_cache(const void* qkv, const void* k_cache, const void* v_cache, void* out,
                                     int32_t batch, int64_t chunk, int32_t heads, int32_t head_dim, int64_t start,
                                     int64_t capacity, float scale, void* workspace, int64_t workspace_bytes,
                                     void* stream) {
  return attention_kv_cache(qkv, k_cache, v_cache, out, batch, chunk, heads, head_dim, start, capacity, scale, stream,
                            [&](int64_t need, void** ptr) {
                              if (!workspace) return XB_ERR_NULL_POINTER;
                              if (workspace_bytes < need) return XB_ERR_WORKSPACE;
                              if ((uintptr_t)workspace & 15u) return XB_ERR_MISALIGNED;
                              *ptr = workspace;
                              return XB_OK;
                            });
}

// ---------------------------------------------------------------------------
// No-allocation decode: the split partials live in `scratch`, a file-scope
// device array (every GPU the library runs on holds its own copy, for the
// life of the process).  Host code never passes `scratch` itself to a kernel
// -- on the host that name is only a stand-in for the symbol -- but the
// address hipGetSymbolAddress returns for it, looked up once per device with
// that device current and kept in `g_scratch_ptr`.  The partials need no
// clearing: every split writes its (o, offset, sum) slots before the combine
// kernel, ordered after it on the same stream, reads them.
static __device__ __align__(256) char scratch[XB_DECODE_SCRATCH_BYTES];

constexpr int kMaxScratchDevices = 64;
static std::atomic<void*> g_scratch_ptr[kMaxScratchDevices];
static std::mutex g_scratch_mutex;

// The current device's scratch address; the stream (NULL = the current
// device's default stream) must belong to the current device.
static int scratch_address(hipStream_t stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxScratchDevices) return XB_ERR_WRONG_DEVICE;
  if (stream != nullptr) {
    hipDevice_t stream_dev = -1;
    e = hipStreamGetDevice(stream, &stream_dev);
    if (e != hipSuccess) return (int)e;
    if ((int)stream_dev != dev) return XB_ERR_WRONG_DEVICE;
  }
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return (int)e;
      if (p == nullptr) return (int)hipErrorInvalidSymbol;
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return XB_OK;
}

extern "C" int xb_attention_kv_cache_noalloc(const void* qkv, const void* k_cache, const void* v_cache, void* out,
                                             int32_t batch, int64_t chunk, int32_t heads, int32_t head_dim,
                                             int64_t start, int64_t capacity, float scale, void* stream) {
  return attention_kv_cache(qkv, k_cache, v_cache, out, batch, chunk, heads, head_dim, start, capacity, scale, stream,
                            [&](int64_t need, void** ptr) {
                              if (need > XB_DECODE_SCRATCH_BYTES) return XB_ERR_SCRATCH_TOO_SMALL;
                              return scratch_address(static_cast<hipStream_t>(stream), ptr);
                            });
}
