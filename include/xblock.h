/*
 * xblock: C-ABI of the MI355X (gfx950) kernels behind the causal pre-norm
 * Transformer block inference path (UserOptimizedTransformer.forward).
 *
 * Conventions shared by every entry point:
 *   - plain device pointers to caller-owned memory, element counts in int64/int32;
 *   - `stream` is a hipStream_t passed as void* (NULL = the default stream);
 *   - work is only enqueued: no allocation, no host synchronisation, so every
 *     call is safe inside hipGraph stream capture;
 *   - return 0 on success, a negative XB_ERR_* for a rejected argument (nothing
 *     is launched), or a positive hipError_t from the launch.
 * Reference citations are file:line inside gwenlim89/GPU-kernel-for-transformer.
 */
#ifndef XBLOCK_H
#define XBLOCK_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define XB_ABI_VERSION 3

/* Argument errors (negative); positive values are hipError_t codes. */
#define XB_OK 0
#define XB_ERR_NULL_POINTER (-1)
#define XB_ERR_BAD_SIZE (-2)
#define XB_ERR_BAD_DTYPE (-3)
#define XB_ERR_UNSUPPORTED_SHAPE (-4)
#define XB_ERR_MISALIGNED (-5)
#define XB_ERR_BAD_EPILOGUE (-6)
#define XB_ERR_WORKSPACE (-7)   /* workspace_bytes below what the call needs */
#define XB_ERR_WRONG_DEVICE (-8) /* the stream is not on the current device   */
#define XB_ERR_SCRATCH_TOO_SMALL (-9) /* more than the static scratch holds  */
#define XB_ERR_BAD_VARIANT (-10) /* kernel variant not built for the shape  */

/* Element types of activations. */
#define XB_F32 0
#define XB_F16 1

/* GEMM epilogues applied to (A . W^T + bias) before the FP16 store. */
#define XB_EPI_BIAS 0       /* y = acc + bias                                  */
#define XB_EPI_BIAS_GELU 1  /* y = gelu(acc + bias), erf form to 3e-5 (not tanh) */

/* Row masks of xb_residual_layernorm_masked (bits; rows whose valid byte is 0). */
#define XB_MASK_UPDATE 1    /* the update is dropped: s = residual             */
#define XB_MASK_SUM 2       /* s = 0 (stored residual and LayerNorm input)    */
#define XB_MASK_OUTPUT 4    /* y = 0                                           */

int xb_abi_version(void);
const char* xb_strerror(int code);

/*
 * Execution plan.  Each op family has kernel variants; xb_select_* returns
 * the variant the library picks for a shape (>= 0) or a negative XB_ERR_*,
 * without touching a GPU, and the *_v entry points run a given variant
 * (XB_VARIANT_AUTO = the selection; a variant not built for the shape gives
 * XB_ERR_BAD_VARIANT).  The Python side turns the selections into the
 * model's ShapeExecutionPlan and passes them back, so the plan it describes
 * is what runs (the reference's per-shape plan, torch_transformer_benchmark.py:
 * 98-157).  xb_variant_name(op, variant) names a variant (NULL if unknown).
 */
#define XB_VARIANT_AUTO (-1)
#define XB_OP_LINEAR 0
#define XB_OP_ATTENTION 1
#define XB_OP_FUSED_D128 2
/* xb_linear_v: gemm_dma_kernel tiles (K % 64 == 0, K >= 256) and gemm_nt_kernel tiles (any K % 8 == 0). */
#define XB_LINEAR_DMA_256x256 0
#define XB_LINEAR_DMA_256x192 1   /* also N % 192 == 0 */
#define XB_LINEAR_DMA_128x256 2
#define XB_LINEAR_DMA_128x128 3
#define XB_LINEAR_NT_128x128 4
#define XB_LINEAR_NT_64x64 5
/* xb_attention_v: waves per block x queries per block. */
#define XB_ATTN_W4_Q16 0     /* head_dim 256                              */
#define XB_ATTN_W4_Q32 1     /* head_dim <= 128                           */
#define XB_ATTN_W4_Q64 2     /* head_dim <= 64                            */
#define XB_ATTN_W8_Q16 3     /* head_dim 256                              */
#define XB_ATTN_PINGPONG 4   /* head_dim 64, no key mask: 512 queries      */
#define XB_ATTN_PINGPONG_VT 5 /* XB_ATTN_PINGPONG reading V transposed by xb_linear_qkv_vt:
                                 runs through xb_attention_causal_vt only  */
/* xb_fused_forward_d128[_ws]: which form runs (the split needs a workspace). */
#define XB_FUSED_PAIRS 0     /* one workgroup per sequence, 8 waves x 2 token blocks (head_dim <= 64) */
#define XB_FUSED_SPLIT 1     /* two workgroups per sequence (xb_fused_forward_d128_ws)                */
#define XB_FUSED_HD128 2     /* one workgroup per sequence, head_dim 128                             */
const char* xb_variant_name(int op, int variant);
int xb_select_linear(int64_t m, int32_t n, int32_t k, int epilogue);
int xb_select_attention(int32_t batch, int64_t seq_len, int32_t heads,
                        int32_t head_dim, int32_t masked);
int xb_select_fused_d128(int64_t batch, int32_t seq_len, int32_t heads,
                         int32_t ffn_dim, int32_t causal, int32_t masked);

/*
 * y[r, :] = LayerNorm(x[r, :]) (* gamma + beta when apply_affine), FP32 math,
 * biased variance, y stored as y_dtype.  x: [rows, cols] FP32, contiguous.
 * Replaces layer_norm / _layer_norm_kernel (triton_fused_norm.py:140-170,
 * triton_fused_norm.py:84-121), called for layer 0's norm1
 * (torch_transformer_benchmark.py:1103-1111).
 */
int xb_layernorm(const float* x, const float* gamma, const float* beta, void* y,
                 int y_dtype, int64_t rows, int32_t cols, float eps,
                 int apply_affine, void* stream);

/*
 * s = residual + update (FP32); residual_out = s unless residual_out is NULL;
 * y = LayerNorm(s) (* gamma + beta) stored as y_dtype.  residual_out may alias
 * residual (in-place update of the residual stream).
 * Replaces fused_residual_layer_norm / _residual_layer_norm_kernel
 * (triton_fused_norm.py:173-215, triton_fused_norm.py:37-81); NULL
 * residual_out is the reference's store_residual=False.
 */
int xb_residual_layernorm(const float* residual, const void* update,
                          int update_dtype, const float* gamma,
                          const float* beta, float* residual_out, void* y,
                          int y_dtype, int64_t rows, int32_t cols, float eps,
                          int apply_affine, void* stream);

/*
 * xb_residual_layernorm with the reference's padding semantics: for rows whose
 * row_valid byte is 0, mask_mode selects (by selection, not multiplication, so
 * NaN in a dropped update does not leak) XB_MASK_UPDATE (attention output
 * zeroed before the residual add, torch_transformer_benchmark.py:263-264),
 * XB_MASK_SUM (block output zeroed, :290-291) and XB_MASK_OUTPUT (final
 * LayerNorm output zeroed, :314-315).  row_valid may be NULL only with
 * mask_mode 0.
 */
int xb_residual_layernorm_masked(const float* residual, const void* update,
                                 int update_dtype, const float* gamma,
                                 const float* beta, float* residual_out, void* y,
                                 int y_dtype, int64_t rows, int32_t cols, float eps,
                                 int apply_affine, const uint8_t* row_valid,
                                 int mask_mode, void* stream);

/*
 * c[M, N] = epilogue(a[M, K] . w[N, K]^T + bias[N]) with FP16 operands, FP32
 * MFMA accumulation and an FP16 store.  w is nn.Linear's own [out, in] layout;
 * bias is FP32 (may be NULL for no bias).  K and N must be multiples of 8.
 * Replaces F.linear under FP16 autocast (torch_transformer_benchmark.py:685,
 * :741), triton_ffn_gelu (triton_fused_ffn.py:224-261) and the grouped
 * accumulation kernels (triton_fused_ffn.py:264-411).
 */
int xb_linear(const void* a, const void* w, const float* bias, void* c,
              int64_t m, int32_t n, int32_t k, int epilogue, void* stream);
/* xb_linear running a given tile variant (XB_LINEAR_*, or XB_VARIANT_AUTO). */
int xb_linear_v(const void* a, const void* w, const float* bias, void* c,
                int64_t m, int32_t n, int32_t k, int epilogue, int variant,
                void* stream);

/*
 * Causal multi-head attention over a packed projection.
 * qkv: [batch, seq_len, 3, heads, head_dim] FP16 (the packed QKV GEMM output);
 * out: [batch, seq_len, heads, head_dim] FP16 (= [B, S, D], ready for the
 * output projection).  softmax(q k^T * scale, top-left causal) v with FP32
 * online softmax.  head_dim in {8, 16, 32, 64, 128, 256}.
 * Replaces F.scaled_dot_product_attention(is_causal=True) and the following
 * transpose/reshape (torch_transformer_benchmark.py:742-809).
 */
int xb_attention_causal(const void* qkv, void* out, int32_t batch,
                        int64_t seq_len, int32_t heads, int32_t head_dim,
                        float scale, void* stream);

/*
 * xb_attention_causal generalised: causal = 0 drops the causal mask, and
 * key_valid ([batch, seq_len] bytes, NULL = all valid) masks keys whose byte
 * is 0 -- the baseline's key padding mask (torch_transformer_benchmark.py:
 * 250-253; the reference's optimized path builds the same mask densely in
 * _prepare_attention_args, :464-522).  A query that sees no key at all writes
 * zeros.
 */
int xb_attention(const void* qkv, void* out, const uint8_t* key_valid,
                 int32_t batch, int64_t seq_len, int32_t heads,
                 int32_t head_dim, float scale, int32_t causal, void* stream);
/* xb_attention running a given kernel variant (XB_ATTN_*, or XB_VARIANT_AUTO). */
int xb_attention_v(const void* qkv, void* out, const uint8_t* key_valid,
                   int32_t batch, int64_t seq_len, int32_t heads,
                   int32_t head_dim, float scale, int32_t causal, int variant,
                   void* stream);

/*
 * The QKV projection and causal attention of long sequences with V handed
 * over transposed.  No reference counterpart: together they replace the
 * packed QKV F.linear and F.scaled_dot_product_attention(is_causal=True) of
 * torch_transformer_benchmark.py:741-809 (as xb_linear + xb_attention_causal
 * do) for head_dim 64 and seq_len % 32 == 0, the shapes that take the
 * ping-pong attention kernel (long sequences, no key mask).
 *
 * xb_linear_qkv_vt: qkv[M, 3D] = a[M, K] . w[3D, K]^T + bias as xb_linear
 * (M = batch * seq_len, D = heads * head_dim) for the Q and K columns only;
 * V goes to vt, [batch, heads, head_dim, xb_vt_row_stride(seq_len)] FP16,
 * each row holding one head dimension over the sequence with every 32-token
 * group in the attention's key order (token 32t + 4g + i at position
 * 32t + 8g + i, token 32t + 16 + 4g + i at 32t + 8g + 4 + i, g, i < 4) and
 * zeros past seq_len.  qkv's V columns are left unwritten.  variant: a
 * gemm_dma_kernel tile whose width divides D (XB_LINEAR_DMA_256x256,
 * _128x256, _128x128) or XB_VARIANT_AUTO; K % 64 == 0 and K >= 256.
 *
 * xb_attention_causal_vt: out = xb_attention_causal(qkv) with V read from vt;
 * bit for bit the same result.
 */
int64_t xb_vt_row_stride(int64_t seq_len);
int xb_linear_qkv_vt(const void* a, const void* w, const float* bias,
                     void* qkv, void* vt, int32_t batch, int64_t seq_len,
                     int32_t heads, int32_t head_dim, int32_t k, int variant,
                     void* stream);
int xb_attention_causal_vt(const void* qkv, const void* vt, void* out,
                           int32_t batch, int64_t seq_len, int32_t heads,
                           int32_t head_dim, float scale, void* stream);

/*
 * KV cache for incremental causal decoding (replaces _append_kv_cache and the
 * cached branch of _fast_attention_impl, torch_transformer_benchmark.py:
 * 426-462, :747-765).  Per layer the cache is two FP16 tensors k_cache,
 * v_cache of shape [batch, heads, capacity, head_dim] (the reference's
 * layout); a forward over `chunk` new tokens whose packed projection is qkv
 * ([batch, chunk, 3, heads, head_dim]) first appends, then attends:
 *
 *   xb_kv_cache_append: k/v_cache[:, :, start:start+chunk] = the chunk's k, v.
 *   xb_attention_kv_cache: out ([batch, chunk, heads*head_dim] FP16) = causal
 *     attention of the chunk's queries, at positions start .. start+chunk-1,
 *     over cached keys 0 .. start+chunk-1 (call it after the append).
 *
 * start + chunk <= capacity, else XB_ERR_BAD_SIZE (the reference raises
 * ValueError, TTB:434-438).  A chunk of at most 16 tokens (decode) splits
 * the keys over the GPU and needs a caller-provided workspace of
 * xb_attention_kv_cache_workspace_bytes(...) bytes (16-byte aligned; 0 for
 * longer chunks, which need none); a smaller one gives XB_ERR_WORKSPACE.
 */
int xb_kv_cache_append(const void* qkv, void* k_cache, void* v_cache,
                       int32_t batch, int64_t chunk, int32_t heads,
                       int32_t head_dim, int64_t start, int64_t capacity,
                       void* stream);
int64_t xb_attention_kv_cache_workspace_bytes(int32_t batch, int64_t chunk,
                                              int32_t heads, int32_t head_dim,
                                              int64_t start);
int xb_attention_kv_cache(const void* qkv, const void* k_cache,
                          const void* v_cache, void* out, int32_t batch,
                          int64_t chunk, int32_t heads, int32_t head_dim,
                          int64_t start, int64_t capacity, float scale,
                          void* workspace, int64_t workspace_bytes,
                          void* stream);

/*
 * xb_attention_kv_cache without a workspace argument, for callers that cannot
 * allocate (code under hipGraph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  No counterpart in the reference.  A decode chunk's
 * split partials go to a static device buffer of XB_DECODE_SCRATCH_BYTES
 * that the library holds on each GPU it runs on until the process ends; the
 * call allocates nothing.  The partials take
 *   batch * heads * n_splits * 16 * (4 * head_dim + 8) bytes,
 * and the split count n_splits (>= 1; the same in both entry points, which
 * is what keeps their results equal) is capped so that this stays within
 * XB_DECODE_SCRATCH_BYTES whenever n_splits = 1 does.  So a decode chunk
 * (at most 16 new tokens) fails only when batch * heads * 16 *
 * (4 * head_dim + 8) > XB_DECODE_SCRATCH_BYTES, whatever the cache length:
 * batch * heads above 52,428 / 29,127 / 15,420 / 7,943 / 4,032 / 2,032 at
 * head_dim 8 / 16 / 32 / 64 / 128 / 256.  Such a call returns
 * XB_ERR_SCRATCH_TOO_SMALL without launching; use xb_attention_kv_cache with
 * a workspace then (xb_attention_kv_cache_workspace_bytes gives the bytes
 * either call needs).  The stream must belong to the current device
 * (XB_ERR_WRONG_DEVICE otherwise).  All calls on one GPU share its buffer:
 * calls that overlap in time on one GPU (different streams, or concurrent
 * graph replays) race and must not be issued.  Results equal
 * xb_attention_kv_cache's bit for bit.
 */
#define XB_DECODE_SCRATCH_BYTES (32LL << 20)
int xb_attention_kv_cache_noalloc(const void* qkv, const void* k_cache,
                                  const void* v_cache, void* out,
                                  int32_t batch, int64_t chunk, int32_t heads,
                                  int32_t head_dim, int64_t start,
                                  int64_t capacity, float scale, void* stream);

/* Fragment orders of xb_pack_linear_fragments. */
#define XB_PACK_PERMUTED 0  /* k = 32*ks + 4*(l/16) + (m & 3) + 16*(m >> 2) */
#define XB_PACK_NATURAL 1   /* k = 32*ks + 8*(l/16) + m                      */

/*
 * Packs an FP32 nn.Linear weight w[n, k] (n % 16 == 0, k % 32 == 0) into the
 * FP16 fragment-major order xb_fused_forward_d128 streams its weights in:
 *   out[((ob * (k/32) + ks) * 64 + l) * 8 + m] = scale * w[16*ob + l%16][k(ks, l, m)]
 * with k(ks, l, m) given by `order` (one 16-byte MFMA operand per lane, 1 KiB
 * per 16x32 block); `scale` multiplies in FP32 before the FP16 rounding.
 * Replaces the reference's cached weight conversions
 * (_cached_linear_parameters / _packed_qkv, torch_transformer_benchmark.py:540-641).
 */
int xb_pack_linear_fragments(const float* w, void* out, int32_t n, int32_t k,
                             int32_t order, float scale, void* stream);

/*
 * The whole forward (every layer and the final LayerNorm) for d_model == 128,
 * seq_len <= 128, ffn_dim == 128, head_dim in {8, 16, 32, 64, 128}, LayerNorm
 * eps 1e-5: one workgroup per sequence keeps the residual stream in registers,
 * so x [batch, seq_len, 128] FP32 is read once and y (same shape, FP32) is
 * written once.  Same math as the per-op sequence above (FP16 MFMA operands,
 * FP32 accumulation / residual / softmax, exact-erf GELU).
 *   wpack: per layer, fragment-packed (xb_pack_linear_fragments) Wq, Wk, Wv,
 *          Wo [128,128], W1 [ffn,128], W2 [128,ffn], layers back to back, all
 *          in XB_PACK_PERMUTED order; Wq packed with
 *          scale = softmax_scale * log2(e);
 *   ppack: FP32, per layer bq * softmax_scale * log2(e), bk, bv, bo [128],
 *          b1 [ffn], b2 [128], norm1 gamma, beta, norm2 gamma, beta [128
 *          each]; then final_norm gamma, beta.
 * (softmax_scale is head_dim ** -0.5, torch_transformer_benchmark.py:215.)
 *   affine_mask: bit 2l set = apply norm1 gamma/beta of layer l, bit 2l+1 =
 *          norm2's; a clear bit skips an identity affine (gamma == 1,
 *          beta == 0 exactly), as the reference does (TTB:568-596).  Pass -1
 *          to always apply; layers beyond 31 always apply; the final norm
 *          always applies.
 *   token_valid ([batch, seq_len] bytes, NULL = all valid) and causal: the
 *          padding and non-causal semantics of xb_attention (padded tokens
 *          are masked as keys in every layer and leave as zero rows, a query
 *          that sees no key gets a zero context).  head_dim 128 takes only
 *          causal = 1 with token_valid = NULL.
 * Replaces _forward_cuda_fused_norm (torch_transformer_benchmark.py:1092-1148)
 * for the official d_model = 128 shapes.
 */
int xb_fused_forward_d128(const float* x, float* y, const void* wpack,
                          const float* ppack, int64_t batch, int32_t seq_len,
                          int32_t heads, int32_t ffn_dim, int32_t layers,
                          int64_t affine_mask, const uint8_t* token_valid,
                          int32_t causal, void* stream);

/* spin_limit / fault_flags of xb_fused_forward_d128_ws. */
#define XB_SPLIT_SPINS_DEFAULT (-1)    /* the library's bound, about 30-40 ms      */
#define XB_SPLIT_FAULT_NO_PUBLISH 1    /* test only: the first workgroup of each
                                          sequence never signals its K/V, so every
                                          wait of the second runs out             */
#define XB_SPLIT_FAULT_FOREIGN_XCD 2   /* test only: the first workgroup signals
                                          with an XCD id no XCD has, so every
                                          hand-off fails the second's XCD check   */

/*
 * xb_fused_forward_d128 with a caller workspace that lets small batches use
 * two workgroups per sequence (tokens 0..63 and 64..127; the first hands each
 * layer's K and V of its tokens to the second through the workspace), which
 * doubles the CUs a small batch occupies (at most 128 sequences).  Same
 * results, bit for bit, as xb_fused_forward_d128.
 *   xb_fused_forward_d128_workspace_bytes: bytes the split needs (0 = this
 *     shape runs one workgroup per sequence: head_dim above 64, causal = 0,
 *     seq_len <= 64 or a batch above those limits).
 *   workspace: 16-byte aligned, zero-filled before its first use, then
 *     reused as it is (hipGraph replays included): each launch signals with
 *     its own epoch (the workspace's launch generation plus one, advanced by
 *     the launch's last workgroup), so nothing left by an earlier launch can
 *     satisfy a later one.  Launches that overlap in time must not share a
 *     workspace.  NULL, or a shape that needs none, runs
 *     xb_fused_forward_d128; fewer than the needed bytes give
 *     XB_ERR_WORKSPACE.  Its layout depends only on `layers`, so a workspace
 *     sized for a larger batch serves a smaller one (the size for the
 *     largest split batch serves every batch).  Its first 4 bytes (int32)
 *     count hand-offs that failed (0 when every call was correct); bytes
 *     8..15 (uint64) count completed split launches.
 *   spin_limit: sleeps (s_sleep 1 each) the second workgroup waits for a
 *     layer's K/V before it gives up; XB_SPLIT_SPINS_DEFAULT for the
 *     library's bound.  The two workgroups of a sequence run on one XCD with
 *     the first dispatched first, and the first never waits, so a wait only
 *     runs out when something else is broken.  The K/V pass through that
 *     XCD's L2 alone; the second workgroup checks that the first ran on its
 *     XCD.  A wait that runs out, or a hand-off from another XCD, adds 1 to
 *     the failure counter and makes that workgroup's output rows NaN (the
 *     kernel still completes), so a failed hand-off can never pass for a
 *     result.
 *   fault_flags: 0, or XB_SPLIT_FAULT_NO_PUBLISH / XB_SPLIT_FAULT_FOREIGN_XCD
 *     to exercise those paths.
 * Replaces the same reference path as xb_fused_forward_d128.
 */
int64_t xb_fused_forward_d128_workspace_bytes(int64_t batch, int32_t seq_len,
                                              int32_t heads, int32_t layers,
                                              int32_t causal);
int xb_fused_forward_d128_ws(const float* x, float* y, const void* wpack,
                             const float* ppack, int64_t batch,
                             int32_t seq_len, int32_t heads, int32_t ffn_dim,
                             int32_t layers, int64_t affine_mask,
                             const uint8_t* token_valid, int32_t causal,
                             void* workspace, int64_t workspace_bytes,
                             int32_t spin_limit, int32_t fault_flags,
                             void* stream);

#ifdef __cplusplus
}
#endif

#endif /* XBLOCK_H */
