// Whole-stack forward for d_model = 128, seq_len <= 128: one workgroup per
// sequence runs every layer and the final LayerNorm, reading x and writing y
// exactly once (8 * D bytes per token instead of the pipeline's
// 4D + L * (48D + 4F)).  This is the per-sequence fusion the reference lists
// as future work (README.md:611-614) applied to its kernel sequence
// torch_transformer_benchmark.py:1092-1148; the math is that sequence's:
//   n1 = LN1(x); q,k,v = n1 Wqkv^T + b; ctx = causal_softmax(q k^T * scale) v;
//   x += ctx Wo^T + bo; n2 = LN2(x); x += gelu_erf(n2 W1^T + b1) W2^T + b2;
//   ... ; y = LN_final(x)
// with FP16 MFMA operands, FP32 accumulation, FP32 residual and softmax.
//
// Layout.  Eight waves (two per SIMD) each own one 16-token block: wave w
// holds block w for w < 4 and block 11-w otherwise, so the two waves sharing
// a SIMD (w and w+4) hold blocks b and 7-b and every SIMD gets the same causal
// attention work.  (FUSED_WAVES=4 builds the one-wave-per-SIMD variant: wave w
// owns blocks w and 7-w.)  The residual stream stays in
// registers in the C layout of a "swapped" MFMA product out^T = W . act^T:
// lane l holds token l%16 and features 16*fb + 4*(l/16) + i.  Read back as an
// MFMA operand, that layout gives a k-step ks the reduction indices
// 32ks + 4*(l/16) + (m & 3) + 16*(m >> 2) (m = 0..7); only the pairing of A's
// and B's k index matters, so the weights multiplied by register-resident
// activations are pre-packed in exactly that order ("permuted" packing, see
// xb_pack_linear_fragments), fragment-major, one coalesced 16-byte load per
// lane and MFMA operand.  Q, K and V^T are written to LDS by the QKV loop
// (K and V^T are needed by every wave); the attention context overwrites the
// wave's own Q rows and feeds the output projection from LDS in natural k
// order (so Wo uses the "natural" packing).  LN outputs and the FFN hidden
// activation never leave registers.
#include "common.h"
#include "../../include/xblock.h"

namespace xb {
namespace fused {

constexpr int D = 128;
constexpr int KS = D / 32;      // k-steps over the model width
constexpr int FB = D / 16;      // 16-wide feature blocks
constexpr int SMAX = 128;
constexpr int LD = D + 8;       // LDS row stride (halves) of Q/ctx, K and V^T (SMAX == D)

__device__ __forceinline__ half8_t frag(const half_t* __restrict__ w, int idx, int lane) {
  return *reinterpret_cast<const half8_t*>(w + ((size_t)idx * 64 + lane) * 8);
}

__device__ __forceinline__ float4_t ld4(const float* p) { return *reinterpret_cast<const float4_t*>(p); }

__device__ __forceinline__ half4_t to_half4(const float4_t& v) {
  return half4_t{(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3]};
}

// Two 16-wide feature blocks (lo = 2ks, hi = 2ks+1) of C layout -> one operand.
__device__ __forceinline__ half8_t to_operand(const float4_t& lo, const float4_t& hi) {
  half8_t r;
#pragma unroll
  for (int i = 0; i < 4; ++i) { r[i] = (half_t)lo[i]; r[4 + i] = (half_t)hi[i]; }
  return r;
}

__device__ __forceinline__ half8_t cat4(const half4_t& lo, const half4_t& hi) {
  return half8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// Mean and rstd of the row held by this lane and the three lanes l^16, l^32, l^48.
__device__ __forceinline__ void row_stats(const float4_t (&r)[FB], float& mean, float& rstd) {
  float s = 0.f;
#pragma unroll
  for (int fb = 0; fb < FB; ++fb) s += (r[fb][0] + r[fb][1]) + (r[fb][2] + r[fb][3]);
  s += __shfl_xor(s, 16);
  s += __shfl_xor(s, 32);
  mean = s * (1.0f / D);
  float q = 0.f;
#pragma unroll
  for (int fb = 0; fb < FB; ++fb)
#pragma unroll
    for (int i = 0; i < 4; ++i) { const float c = r[fb][i] - mean; q += c * c; }
  q += __shfl_xor(q, 16);
  q += __shfl_xor(q, 32);
  rstd = rsqrtf(q * (1.0f / D) + 1e-5f);
}

// LayerNorm of the wave's register-resident token blocks -> MFMA operands.
template <int T>
__device__ __forceinline__ void layer_norm(const float4_t (&res)[T][FB], const float* __restrict__ gamma,
                                           const float* __restrict__ beta, half8_t (&xn)[T][KS], int g) {
#pragma unroll
  for (int t = 0; t < T; ++t) {
    float mean, rstd;
    row_stats(res[t], mean, rstd);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      float4_t lo, hi;
      const float4_t g0 = ld4(gamma + 32 * ks + 4 * g), g1 = ld4(gamma + 32 * ks + 16 + 4 * g);
      const float4_t b0 = ld4(beta + 32 * ks + 4 * g), b1 = ld4(beta + 32 * ks + 16 + 4 * g);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        lo[i] = (res[t][2 * ks][i] - mean) * rstd * g0[i] + b0[i];
        hi[i] = (res[t][2 * ks + 1][i] - mean) * rstd * g1[i] + b1[i];
      }
      xn[t][ks] = to_operand(lo, hi);
    }
  }
}

// Waves per workgroup: 8 (two per SIMD, one 16-token block each) or 4 (one
// per SIMD, two token blocks each).
#ifndef FUSED_WAVES
#define FUSED_WAVES 8
#endif

// Weight fragments stream from L2 with PF output blocks in flight: the loads
// for block ob + PF are issued before block ob's MFMAs.  With one wave per
// SIMD nothing else hides their latency, so that layout prefetches deeper.
#ifndef FUSED_PF
#define FUSED_PF (FUSED_WAVES == 8 ? 2 : 4)
#endif
constexpr int PF = FUSED_PF;

// Fragments of output blocks [0, PF) of a weight with KIN k-steps.
template <int KIN>
__device__ __forceinline__ void prefetch_head(const half_t* __restrict__ w, half8_t (&buf)[PF][KIN], int lane) {
#pragma unroll
  for (int j = 0; j < PF; ++j)
#pragma unroll
    for (int ks = 0; ks < KIN; ++ks) buf[j][ks] = frag(w, j * KIN + ks, lane);
}

// res[t][ob] += (W . act^T)[ob] + bias over all FB output blocks; `buf` holds
// the fragments of blocks 0..PF-1 on entry (prefetch_head).
template <int KIN, int T>
__device__ __forceinline__ void gemm_accumulate(const half_t* __restrict__ w, const float* __restrict__ bias,
                                                const half8_t (&act)[T][KIN], float4_t (&res)[T][FB],
                                                half8_t (&buf)[PF][KIN], int lane, int g) {
#pragma unroll
  for (int ob = 0; ob < FB; ++ob) {
    half8_t cur[KIN];
#pragma unroll
    for (int ks = 0; ks < KIN; ++ks) cur[ks] = buf[ob % PF][ks];
    if (ob + PF < FB) {
#pragma unroll
      for (int ks = 0; ks < KIN; ++ks) buf[ob % PF][ks] = frag(w, (ob + PF) * KIN + ks, lane);
    }
    float4_t a[T];
#pragma unroll
    for (int t = 0; t < T; ++t) a[t] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KIN; ++ks)
#pragma unroll
      for (int t = 0; t < T; ++t) a[t] = mfma16x16x32(cur[ks], act[t][ks], a[t]);
    const float4_t b = ld4(bias + 16 * ob + 4 * g);
#pragma unroll
    for (int t = 0; t < T; ++t) res[t][ob] += a[t] + b;
  }
}

template <int HD, int NW>
__global__ __launch_bounds__(64 * NW, 1) void fused_stack_kernel(
    const float* __restrict__ x, float* __restrict__ y, const half_t* __restrict__ wpack,
    const float* __restrict__ ppack, int S, int layers) {
  constexpr int F = 128;  // ffn_dim (the packed-layer strides below assume it)
  constexpr int T = 8 / NW;  // 16-token blocks per wave
  constexpr int H = D / HD;
  constexpr int FKS = F / 32;
  constexpr int HDB = HD < 16 ? 1 : HD / 16;   // 16-row blocks of one head in V^T / ctx
  constexpr int KSH = HD >= 32 ? HD / 32 : 1;  // k-steps of one head's q.k
  constexpr int64_t W_LAYER = 4 * D * D + 2 * (int64_t)F * D;
  constexpr int P_LAYER = 9 * D + F;
  __shared__ __attribute__((aligned(16))) half_t q_lds[SMAX * LD];   // Q (pre-scaled), then ctx
  __shared__ __attribute__((aligned(16))) half_t k_lds[SMAX * LD];   // K, row-major
  __shared__ __attribute__((aligned(16))) half_t vt_lds[D * LD];     // V^T [feature][token]

  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int g = lane / 16, r16 = lane % 16;
  // Token block of the wave's t-th block.  Four waves: w and 7-w.  Eight waves
  // (two per SIMD, waves w and w+4 sharing one): w for w < 4, else 11-w, so
  // every SIMD again holds blocks b and 7-b.
  auto tblock = [&](int t) { return NW == 4 ? (t ? 7 - wave : wave) : (wave < 4 ? wave : 11 - wave); };
  // Additive causal mask of a diagonal 16x16 block: key 4g + i vs query r16.
  float4_t diag_mask;
#pragma unroll
  for (int i = 0; i < 4; ++i) diag_mask[i] = (4 * g + i > r16) ? -INFINITY : 0.f;
  const int64_t seq = blockIdx.x;
  const float* xs = x + seq * S * D;
  float* ys = y + seq * S * D;

  // Residual stream, C layout: res[t][fb][i] = x[16 tb_t + r16][16 fb + 4 g + i].
  float4_t res[T][FB];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int tok = 16 * tblock(t) + r16;
#pragma unroll
    for (int fb = 0; fb < FB; ++fb)
      res[t][fb] = tok < S ? ld4(xs + (int64_t)tok * D + 16 * fb + 4 * g) : float4_t{0.f, 0.f, 0.f, 0.f};
  }

  for (int layer = 0; layer < layers; ++layer) {
    const half_t* wqkv = wpack + layer * W_LAYER;  // Wq, Wk, Wv: 24 blocks of 16 output features
    const half_t* wo = wqkv + 3 * D * D;
    const half_t* w1 = wo + D * D;
    const half_t* w2 = w1 + F * D;
    const float* pp = ppack + layer * P_LAYER;
    const float* bqkv = pp;  // bq, bk, bv back to back
    const float* bo = pp + 3 * D;
    const float* b1 = pp + 4 * D;
    const float* b2 = pp + 4 * D + F;
    const float* g1 = pp + 5 * D + F;
    const float* be1 = pp + 6 * D + F;
    const float* g2 = pp + 7 * D + F;
    const float* be2 = pp + 8 * D + F;

    // ---- LN1 and the QKV projection into LDS ------------------------------
    half8_t xn[T][KS];
    layer_norm(res, g1, be1, xn, g);
    __syncthreads();  // the previous layer's attention has finished reading K / V^T
    {
      // 24 output blocks (Q, K, V) in groups of PF: group G+1's fragments load
      // while group G's MFMAs run.
      half8_t wbuf[PF][KS];
      prefetch_head<KS>(wqkv, wbuf, lane);
#pragma unroll 1
      for (int ob0 = 0; ob0 < 3 * FB; ob0 += PF) {
       half8_t wcur[PF][KS];
#pragma unroll
       for (int j = 0; j < PF; ++j)
#pragma unroll
         for (int ks = 0; ks < KS; ++ks) wcur[j][ks] = wbuf[j][ks];
       if (ob0 + PF < 3 * FB) {
#pragma unroll
         for (int j = 0; j < PF; ++j)
#pragma unroll
           for (int ks = 0; ks < KS; ++ks) wbuf[j][ks] = frag(wqkv, (ob0 + PF + j) * KS + ks, lane);
       }
#pragma unroll
       for (int j = 0; j < PF; ++j) {
        const int ob = ob0 + j;
        const half8_t (&cur)[KS] = wcur[j];
        if (ob < 2 * FB) {
          // Q / K: swapped product, lane = (token r16, features 16fb + 4g + i).
          // Q's weights and bias arrive pre-multiplied by scale * log2(e).
          const float4_t b = ld4(bqkv + 16 * ob + 4 * g);
          float4_t a[T];
#pragma unroll
          for (int t = 0; t < T; ++t) a[t] = b;
#pragma unroll
          for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int t = 0; t < T; ++t) a[t] = mfma16x16x32(cur[ks], xn[t][ks], a[t]);
          const int fb = ob % FB;
          half_t* dst = ob < FB ? q_lds : k_lds;
#pragma unroll
          for (int t = 0; t < T; ++t)
            *reinterpret_cast<half4_t*>(dst + (16 * tblock(t) + r16) * LD + 16 * fb + 4 * g) = to_half4(a[t]);
        } else {
          // V: unswapped product, lane = (tokens 16tb + 4g + i, feature 16fb + r16),
          // i.e. four consecutive entries of one V^T row.
          const float bv = bqkv[16 * ob + r16];
          float4_t a[T];
#pragma unroll
          for (int t = 0; t < T; ++t) a[t] = float4_t{bv, bv, bv, bv};
#pragma unroll
          for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int t = 0; t < T; ++t) a[t] = mfma16x16x32(xn[t][ks], cur[ks], a[t]);
          const int fb = ob - 2 * FB;
#pragma unroll
          for (int t = 0; t < T; ++t)
            *reinterpret_cast<half4_t*>(vt_lds + (16 * fb + r16) * LD + 16 * tblock(t) + 4 * g) = to_half4(a[t]);
        }
       }
      }
    }
    // The output projection's first fragments load during attention.
    half8_t wbuf_o[PF][KS];
    prefetch_head<KS>(wo, wbuf_o, lane);
    __syncthreads();

    // ---- causal attention of the wave's query blocks, every head ------------
    // S^T = K . Q^T (M = keys, N = queries): lane holds keys 16kb + 4g + i of
    // query r16, which with the key order 32kt + 4g + (m&3) + 16(m>>2) is the
    // B operand of O^T = V^T . P^T directly.  S <= 128 keys, so all scores of a
    // query block fit in registers and the softmax needs no running rescale.
#pragma unroll 1
    for (int t = 0; t < T; ++t) {
      const int qb = tblock(t);
      const int query = 16 * qb + r16;
#pragma unroll 1
      for (int h = 0; h < H; ++h) {
        const int ks0 = (h * HD) / 32;
        half8_t qh[KSH];
#pragma unroll
        for (int j = 0; j < KSH; ++j) {
          qh[j] = *reinterpret_cast<const half8_t*>(q_lds + query * LD + 32 * (ks0 + j) + 8 * g);
          if constexpr (HD < 32) {  // keep only this head's features of the shared k-step
#pragma unroll
            for (int m = 0; m < 8; ++m)
              if ((32 * ks0 + 8 * g + m) / HD != h) qh[j][m] = (half_t)0.f;
          }
        }
        float4_t s[8];
        float mx = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 8; ++kb) {
          s[kb] = float4_t{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
          if (kb <= qb) {
            float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < KSH; ++j) {
              const half8_t kf =
                  *reinterpret_cast<const half8_t*>(k_lds + (16 * kb + r16) * LD + 32 * (ks0 + j) + 8 * g);
              acc = mfma16x16x32(kf, qh[j], acc);
            }
            if (kb == qb) acc += diag_mask;  // -inf above the diagonal
            s[kb] = acc;
            mx = fmaxf(mx, fmaxf(fmaxf(acc[0], acc[1]), fmaxf(acc[2], acc[3])));
          }
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        float lsum = 0.f;
        const int vrow0 = HD < 16 ? 16 * (h / 2) : h * HD;
        float4_t o[HDB];
#pragma unroll
        for (int hb = 0; hb < HDB; ++hb) o[hb] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
          if (2 * kt <= qb) {
            float4_t p0, p1;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              p0[i] = __builtin_amdgcn_exp2f(s[2 * kt][i] - mx);
              p1[i] = __builtin_amdgcn_exp2f(s[2 * kt + 1][i] - mx);  // exp2(-inf) = 0 past qb
            }
            lsum += ((p0[0] + p0[1]) + (p0[2] + p0[3])) + ((p1[0] + p1[1]) + (p1[2] + p1[3]));
            const half8_t pf = to_operand(p0, p1);
#pragma unroll
            for (int hb = 0; hb < HDB; ++hb) {
              const half_t* vr = vt_lds + (vrow0 + 16 * hb + r16) * LD + 32 * kt + 4 * g;
              const half8_t vf = cat4(*reinterpret_cast<const half4_t*>(vr), *reinterpret_cast<const half4_t*>(vr + 16));
              o[hb] = mfma16x16x32(vf, pf, o[hb]);
            }
          }
        }
        lsum += __shfl_xor(lsum, 16);
        lsum += __shfl_xor(lsum, 32);
        const float inv = 1.0f / lsum;
        // O^T C layout: rows 4g + i of block (vrow0 + 16hb) for query r16. The
        // wave's own Q rows of this head are consumed, so ctx overwrites them.
        if constexpr (HD >= 16) {
#pragma unroll
          for (int hb = 0; hb < HDB; ++hb)
            *reinterpret_cast<half4_t*>(q_lds + query * LD + vrow0 + 16 * hb + 4 * g) = to_half4(o[hb] * inv);
        } else {
          // Two 8-wide heads share one 16-row block: rows 0-7 (g < 2) are the even head's.
          if ((g / 2) == (h & 1))
            *reinterpret_cast<half4_t*>(q_lds + query * LD + vrow0 + 4 * g) = to_half4(o[0] * inv);
        }
      }
    }

    // ---- output projection + residual (ctx from the wave's own LDS rows) -----
    {
      half8_t cf[T][KS];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int t = 0; t < T; ++t)
          cf[t][ks] = *reinterpret_cast<const half8_t*>(q_lds + (16 * tblock(t) + r16) * LD + 32 * ks + 8 * g);
      gemm_accumulate<KS>(wo, bo, cf, res, wbuf_o, lane, g);
    }

    // ---- LN2, FFN: gelu(n2 W1^T + b1) W2^T + b2 + residual ----------------
    half8_t wbuf1[PF][KS];
    prefetch_head<KS>(w1, wbuf1, lane);
    layer_norm(res, g2, be2, xn, g);
    half8_t hf[T][FKS];
    half8_t wbuf2[PF][FKS];
    {
#pragma unroll
      for (int ob = 0; ob < 2 * FKS; ++ob) {
        half8_t cur[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) cur[ks] = wbuf1[ob % PF][ks];
        if (ob + PF < 2 * FKS) {
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) wbuf1[ob % PF][ks] = frag(w1, (ob + PF) * KS + ks, lane);
        }
        const float4_t b = ld4(b1 + 16 * ob + 4 * g);
        float4_t a[T];
#pragma unroll
        for (int t = 0; t < T; ++t) a[t] = b;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
          for (int t = 0; t < T; ++t) a[t] = mfma16x16x32(cur[ks], xn[t][ks], a[t]);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int t = 0; t < T; ++t) hf[t][ob / 2][(ob & 1) * 4 + i] = (half_t)gelu_erf(a[t][i]);
        if (ob == 2 * FKS - PF - 1) prefetch_head<FKS>(w2, wbuf2, lane);
      }
    }
    gemm_accumulate<FKS>(w2, b2, hf, res, wbuf2, lane, g);
  }

  // ---- final LayerNorm, FP32 output -----------------------------------------
  const float* gf = ppack + layers * P_LAYER;
  const float* bf = gf + D;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    float mean, rstd;
    row_stats(res[t], mean, rstd);
    const int tok = 16 * tblock(t) + r16;
    if (tok < S) {
#pragma unroll
      for (int fb = 0; fb < FB; ++fb) {
        const float4_t gg = ld4(gf + 16 * fb + 4 * g), bb = ld4(bf + 16 * fb + 4 * g);
        float4_t o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = (res[t][fb][i] - mean) * rstd * gg[i] + bb[i];
        *reinterpret_cast<float4_t*>(ys + (int64_t)tok * D + 16 * fb + 4 * g) = o;
      }
    }
  }
}

// Fragment-major FP16 packing of an nn.Linear weight [n, k] (FP32 source).
// permuted: k index 32ks + 4(l/16) + (m&3) + 16(m>>2); natural: 32ks + 8(l/16) + m.
__global__ void pack_fragments_kernel(const float* __restrict__ w, half_t* __restrict__ out, int n, int k,
                                      int permuted, float scale) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)n * k;
  if (idx >= total) return;
  const int m = idx % 8;
  const int l = (idx / 8) % 64;
  const int64_t frag_id = idx / 512;
  const int kss = k / 32;
  const int ks = frag_id % kss;
  const int ob = frag_id / kss;
  const int row = 16 * ob + l % 16;
  const int col = permuted ? 32 * ks + 4 * (l / 16) + (m & 3) + 16 * (m >> 2) : 32 * ks + 8 * (l / 16) + m;
  // Round the FP32 product to FP16 (two roundings, as the host computes it).
  // The empty asm pins the FP32 value so the backend cannot fold multiply and
  // convert into one singly-rounded v_fma_mix.
  float v = w[(int64_t)row * k + col] * scale;
  asm volatile("" : "+v"(v));
  out[idx] = (half_t)v;
}

template <int HD>
static hipError_t launch(const float* x, float* y, const half_t* w, const float* p, int64_t batch, int S,
                         int layers, hipStream_t s) {
  hipLaunchKernelGGL((fused_stack_kernel<HD, FUSED_WAVES>), dim3((unsigned)batch), dim3(64 * FUSED_WAVES), 0, s,
                     x, y, w, p, S, layers);
  return hipGetLastError();
}

}  // namespace fused
}  // namespace xb

using namespace xb;

extern "C" int xb_pack_linear_fragments(const float* w, void* out, int32_t n, int32_t k, int32_t order,
                                        float scale, void* stream) {
  if (n <= 0 || k <= 0) return XB_ERR_BAD_SIZE;
  if (n % 16 != 0 || k % 32 != 0) return XB_ERR_UNSUPPORTED_SHAPE;
  if (order != XB_PACK_PERMUTED && order != XB_PACK_NATURAL) return XB_ERR_BAD_EPILOGUE;
  if (!w || !out) return XB_ERR_NULL_POINTER;
  if (((uintptr_t)out) & 15u) return XB_ERR_MISALIGNED;
  const int64_t total = (int64_t)n * k;
  hipLaunchKernelGGL(fused::pack_fragments_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), w, static_cast<half_t*>(out), n, k,
                     order == XB_PACK_PERMUTED ? 1 : 0, scale);
  return (int)hipGetLastError();
}

extern "C" int xb_fused_forward_d128(const float* x, float* y, const void* wpack, const float* ppack,
                                     int64_t batch, int32_t seq_len, int32_t heads, int32_t ffn_dim,
                                     int32_t layers, void* stream) {
  if (batch < 0 || seq_len <= 0 || heads <= 0 || ffn_dim <= 0 || layers <= 0) return XB_ERR_BAD_SIZE;
  if (batch > 0x7fffffffLL) return XB_ERR_BAD_SIZE;
  if (seq_len > fused::SMAX || fused::D % heads != 0) return XB_ERR_UNSUPPORTED_SHAPE;
  const int hd = fused::D / heads;
  if (hd != 8 && hd != 16 && hd != 32 && hd != 64 && hd != 128) return XB_ERR_UNSUPPORTED_SHAPE;
  if (ffn_dim != 128) return XB_ERR_UNSUPPORTED_SHAPE;
  if (batch == 0) return XB_OK;
  if (!x || !y || !wpack || !ppack) return XB_ERR_NULL_POINTER;
  if (((uintptr_t)x | (uintptr_t)y | (uintptr_t)wpack | (uintptr_t)ppack) & 15u) return XB_ERR_MISALIGNED;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const half_t* w = static_cast<const half_t*>(wpack);
  hipError_t e;
  switch (hd) {
    case 8: e = fused::launch<8>(x, y, w, ppack, batch, seq_len, layers, s); break;
    case 16: e = fused::launch<16>(x, y, w, ppack, batch, seq_len, layers, s); break;
    case 32: e = fused::launch<32>(x, y, w, ppack, batch, seq_len, layers, s); break;
    case 64: e = fused::launch<64>(x, y, w, ppack, batch, seq_len, layers, s); break;
    default: e = fused::launch<128>(x, y, w, ppack, batch, seq_len, layers, s); break;
  }
  return (int)e;
}
