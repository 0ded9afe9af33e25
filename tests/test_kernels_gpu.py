"""Per-kernel parity of the HIP kernels against plain PyTorch FP32 references.

Every reference is computed on the CPU in FP32 from the same (FP16-rounded,
where the kernel takes FP16) inputs.  Tolerances, stated per test, allow for
the kernels' FP16 output rounding (2^-11 relative) and FP32 summation order.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu

F16, F32 = torch.float16, torch.float32


def _gen(seed):
    return torch.Generator().manual_seed(seed)


# ----------------------------------------------------------------------------- LayerNorm
@pytest.mark.parametrize("rows,cols", [(0, 128), (1, 128), (7, 128), (8192, 128), (33, 1024), (5, 64), (3, 96), (2, 2048), (4, 768), (3, 256), (9, 512), (2, 1000)])
@pytest.mark.parametrize("out_dtype", [F16, F32])
@pytest.mark.parametrize("affine", [False, True])
def test_layer_norm(pkg, cuda, rows, cols, out_dtype, affine):
    x = torch.randn(rows, cols, generator=_gen(rows * 7 + cols)) * 2.0 + 0.5
    g = torch.randn(cols, generator=_gen(1)) * 0.3 + 1.0
    b = torch.randn(cols, generator=_gen(2)) * 0.1
    y = pkg.layer_norm(x.to(cuda), g.to(cuda), b.to(cuda), 1e-5, out_dtype, apply_affine=affine)
    ref = F.layer_norm(x, (cols,), g if affine else None, b if affine else None, 1e-5)
    assert y.dtype == out_dtype and y.shape == x.shape
    if out_dtype == F32:
        torch.testing.assert_close(y.cpu(), ref, atol=2e-5, rtol=2e-5)
    else:  # within one FP16 ulp of the rounded reference
        torch.testing.assert_close(y.cpu().float(), ref.half().float(), atol=2e-3, rtol=1e-3)


@pytest.mark.parametrize("cols", [64, 128, 256, 512, 1024, 2048, 96])  # 8- and 4-column lanes, generic
@pytest.mark.parametrize("upd_dtype", [F16, F32])
@pytest.mark.parametrize("mode", ["store", "inplace", "nostore_f32"])
def test_fused_residual_layer_norm(pkg, cuda, cols, upd_dtype, mode):
    rows = 517
    r = torch.randn(rows, cols, generator=_gen(3)) * 1.5
    u = (torch.randn(rows, cols, generator=_gen(4)) * 0.7).to(upd_dtype)
    g = torch.randn(cols, generator=_gen(5)) * 0.3 + 1.0
    b = torch.randn(cols, generator=_gen(6)) * 0.1
    s = r + u.float()
    ref = F.layer_norm(s, (cols,), g, b, 1e-5)
    rg, ug = r.to(cuda), u.to(cuda)
    if mode == "store":
        res, norm = pkg.fused_residual_layer_norm(rg, ug, g.to(cuda), b.to(cuda), 1e-5, F16)
        torch.testing.assert_close(res.cpu(), s, atol=0, rtol=0)
        torch.testing.assert_close(rg.cpu(), r, atol=0, rtol=0)  # input untouched
        torch.testing.assert_close(norm.cpu().float(), ref.half().float(), atol=2e-3, rtol=1e-3)
    elif mode == "inplace":
        res, norm = pkg.fused_residual_layer_norm(rg, ug, g.to(cuda), b.to(cuda), 1e-5, F16, residual_out=rg)
        assert res.data_ptr() == rg.data_ptr()
        torch.testing.assert_close(rg.cpu(), s, atol=0, rtol=0)
        torch.testing.assert_close(norm.cpu().float(), ref.half().float(), atol=2e-3, rtol=1e-3)
    else:
        res, norm = pkg.fused_residual_layer_norm(rg, ug, g.to(cuda), b.to(cuda), 1e-5, F32, store_residual=False)
        assert res is rg
        torch.testing.assert_close(rg.cpu(), r, atol=0, rtol=0)
        torch.testing.assert_close(norm.cpu(), ref, atol=2e-5, rtol=2e-5)


def test_stream_handle_is_the_current_stream(pkg, cuda):
    """Launches go to torch's current stream: the raw handle equals current_stream().cuda_stream
    on the default stream, on a side stream and under graph capture."""
    capi = pkg._capi
    assert capi.stream_handle(cuda) == torch.cuda.current_stream(cuda).cuda_stream
    side = torch.cuda.Stream(device=cuda)
    with torch.cuda.stream(side):
        assert capi.stream_handle(cuda) == side.cuda_stream != torch.cuda.default_stream(cuda).cuda_stream
        assert capi.stream_handle(None) == side.cuda_stream
    graph = torch.cuda.CUDAGraph()
    x = torch.zeros(4, device=cuda)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=side):
        handle = capi.stream_handle(cuda)
        x += 1  # something to capture
    assert handle == side.cuda_stream
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(x, torch.ones(4, device=cuda))


def test_layer_norm_errors(pkg, cuda):
    x = torch.randn(4, 128, device=cuda)
    with pytest.raises(ValueError):
        pkg.layer_norm(x, torch.ones(64, device=cuda), torch.zeros(64, device=cuda), 1e-5, F16)
    with pytest.raises(ValueError):
        pkg.fused_residual_layer_norm(x, torch.zeros(4, 64, device=cuda), torch.ones(128, device=cuda), torch.zeros(128, device=cuda), 1e-5, F16)
    with pytest.raises(ValueError):
        pkg.layer_norm(x.cpu(), torch.ones(128), torch.zeros(128), 1e-5, F16)


# ----------------------------------------------------------------------------- GEMM
@pytest.mark.parametrize(
    "m,n,k",
    [(1, 128, 128), (7, 384, 128), (8192, 384, 128), (8192, 128, 128), (1000, 1024, 1024),
     (8192, 3072, 1024), (257, 136, 72), (64, 8, 8), (300, 1024, 128), (131072, 384, 128),
     (8192, 4096, 256), (16000, 2056, 200), (33000, 1024, 136), (3000, 1032, 512),
     (70000, 264, 1024)],
)
@pytest.mark.parametrize("gelu", [False, True])
def test_linear(pkg, cuda, m, n, k, gelu):
    a = torch.randn(m, k, generator=_gen(m + n)).half()
    w = (torch.randn(n, k, generator=_gen(k)) * k**-0.5).half()
    bias = torch.randn(n, generator=_gen(n)) * 0.1
    ref = a.float() @ w.float().T + bias
    if gelu:
        ref = F.gelu(ref, approximate="none")
    out = pkg.linear(a.to(cuda), w.to(cuda), bias.to(cuda), gelu=gelu)
    assert out.dtype == F16 and out.shape == (m, n)
    # FP16 store (2^-11 relative) plus FP32 accumulation-order noise.
    torch.testing.assert_close(out.cpu().float(), ref, atol=2e-3, rtol=2e-3)


@pytest.mark.parametrize("m,n,k", [(1000, 1152, 1024), (300, 384, 256), (8192, 768, 512)])
@pytest.mark.parametrize("gelu", [False, True])
def test_linear_every_variant(pkg, cuda, m, n, k, gelu):
    """Every tile variant the plan can name (xb_linear_v), forced on shapes all
    of them accept, against the FP32 reference; a variant not built for the
    shape is refused.  The plan picks the tile from the row count, so a
    batch's rows must not depend on it: every direct-to-LDS tile gives the
    same output bit for bit, and so does every register-staged tile (same
    K order; each epilogue rounds the FP32 result to FP16 once)."""
    capi = pkg._capi
    a = torch.randn(m, k, generator=_gen(m + k)).half()
    w = (torch.randn(n, k, generator=_gen(n)) * k**-0.5).half()
    bias = torch.randn(n, generator=_gen(k)) * 0.1
    ref = a.float() @ w.float().T + bias
    if gelu:
        ref = F.gelu(ref, approximate="none")
    ag, wg, bg = a.to(cuda), w.to(cuda), bias.to(cuda)
    outs = {}
    for variant in (capi.XB_LINEAR_DMA_256x256, capi.XB_LINEAR_DMA_256x192, capi.XB_LINEAR_DMA_128x256,
                    capi.XB_LINEAR_DMA_128x128, capi.XB_LINEAR_NT_128x128, capi.XB_LINEAR_NT_64x64):
        out = pkg.linear(ag, wg, bg, gelu=gelu, variant=variant)
        torch.testing.assert_close(out.cpu().float(), ref, atol=2e-3, rtol=2e-3,
                                   msg=lambda e, v=variant: f"variant {v}: {e}")
        outs[variant] = out
    dma = [capi.XB_LINEAR_DMA_256x256, capi.XB_LINEAR_DMA_256x192, capi.XB_LINEAR_DMA_128x256, capi.XB_LINEAR_DMA_128x128]
    for v in dma[1:]:
        assert torch.equal(outs[v], outs[dma[0]]), f"variant {v} differs from {dma[0]}"
    assert torch.equal(outs[capi.XB_LINEAR_NT_64x64], outs[capi.XB_LINEAR_NT_128x128])
    with pytest.raises(RuntimeError, match="code -10"):  # 256x192 needs N % 192 == 0
        pkg.linear(ag[:, :k], wg[:n - 128], None, variant=capi.XB_LINEAR_DMA_256x192)


def test_linear_without_bias_and_batched_shape(pkg, cuda):
    a = torch.randn(3, 5, 64, generator=_gen(1)).half()
    w = (torch.randn(32, 64, generator=_gen(2)) * 0.125).half()
    out = pkg.linear(a.to(cuda), w.to(cuda), None)
    assert out.shape == (3, 5, 32)
    torch.testing.assert_close(out.cpu().float(), a.float() @ w.float().T, atol=2e-3, rtol=2e-3)


def test_linear_errors(pkg, cuda):
    a = torch.randn(4, 64, device=cuda).half()
    with pytest.raises(ValueError):
        pkg.linear(a, torch.randn(32, 48, device=cuda).half(), None)
    with pytest.raises(ValueError):
        pkg.linear(a.float(), torch.randn(32, 64, device=cuda).half(), None)
    with pytest.raises(RuntimeError, match="code -4"):
        pkg.linear(torch.randn(4, 60, device=cuda).half(), torch.randn(32, 60, device=cuda).half(), None)


# ----------------------------------------------------------------------------- attention
def _attention_reference(qkv: torch.Tensor, heads: int, key_valid=None, causal: bool = True) -> torch.Tensor:
    """FP32 softmax attention; a query with no visible key gets a zero row."""
    b, s, width = qkv.shape
    d = width // 3
    hd = d // heads
    t = qkv.float().view(b, s, 3, heads, hd).permute(2, 0, 3, 1, 4)
    q, k, v = t[0], t[1], t[2]
    scores = (q @ k.transpose(-2, -1)) * hd**-0.5
    if causal:
        scores = scores.masked_fill(torch.ones(s, s, dtype=torch.bool).triu(1), float("-inf"))
    if key_valid is not None:
        scores = scores.masked_fill(~key_valid[:, None, None, :], float("-inf"))
    probs = torch.nan_to_num(torch.softmax(scores, -1), nan=0.0)
    return (probs @ v).transpose(1, 2).reshape(b, s, d)


@pytest.mark.parametrize("hd", [8, 16, 32, 64, 128, 256])
@pytest.mark.parametrize("b,s,h", [(2, 1, 2), (1, 17, 2), (2, 128, 4), (1, 200, 2), (1, 333, 1)])
def test_causal_attention(pkg, cuda, hd, b, s, h):
    qkv = torch.randn(b, s, 3 * h * hd, generator=_gen(hd * 1000 + s)).half()
    ref = _attention_reference(qkv, h)
    out = pkg.causal_attention(qkv.to(cuda), h)
    assert out.dtype == F16 and out.shape == (b, s, h * hd)
    # FP16 probabilities and FP16 output rounding.
    torch.testing.assert_close(out.cpu().float(), ref, atol=2e-3, rtol=1e-2)


@pytest.mark.parametrize("hd,s", [(64, 4096), (8, 1500), (256, 700)])
def test_causal_attention_long(pkg, cuda, hd, s):
    h = 2 if hd < 256 else 1
    qkv = torch.randn(1, s, 3 * h * hd, generator=_gen(s)).half()
    ref = _attention_reference(qkv, h)
    out = pkg.causal_attention(qkv.to(cuda), h)
    torch.testing.assert_close(out.cpu().float(), ref, atol=2e-3, rtol=1e-2)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("b,s,h", [(2, 4096, 2), (1, 4133, 3), (1, 8703, 1)])
def test_attention_long_hd64_ping_pong(pkg, cuda, b, s, h, causal):
    """head_dim 64, S >= 4096, no mask: the ping-pong kernel (two wave groups, K/V
    ring loaded straight into LDS).  FP32 reference, and bitwise equal to the
    four-wave kernel, which an all-valid key mask selects: same 64-query waves,
    same tile order and the same wave-uniform rescale decisions."""
    hd = 64
    qkv = torch.randn(b, s, 3 * h * hd, generator=_gen(s + h)).half()
    ref = _attention_reference(qkv, h, causal=causal)
    qg = qkv.to(cuda)
    out = pkg.attention(qg, h, causal=causal)
    torch.testing.assert_close(out.cpu().float(), ref, atol=2e-3, rtol=1e-2)
    ones = torch.ones(b, s, dtype=torch.bool, device=cuda)
    assert torch.equal(out, pkg.attention(qg, h, key_valid=ones, causal=causal))


def _rows_reference(qkv: torch.Tensor, heads: int, rows) -> torch.Tensor:
    """FP32 causal attention of the given query rows of one sequence ([1, S, 3D] FP16):
    O(S * head_dim) per row, so any row of a 100,000-token sequence is cheap."""
    _, s, width = qkv.shape
    d = width // 3
    hd = d // heads
    t = qkv[0].float().view(s, 3, heads, hd)
    q, k, v = t[:, 0].transpose(0, 1), t[:, 1].transpose(0, 1), t[:, 2].transpose(0, 1)   # [H, S, hd]
    idx = torch.tensor(rows)
    scores = (q[:, idx] @ k.transpose(1, 2)) * hd**-0.5                                    # [H, R, S]
    scores = scores.masked_fill(torch.arange(s)[None, None, :] > idx[None, :, None], float("-inf"))
    return (torch.softmax(scores, -1) @ v).transpose(0, 1).reshape(len(rows), d)


def test_attention_full_length_cfg5_sampled_rows(pkg, cuda):
    """cfg5's attention at its real length (S = 100,000, head_dim 64) beyond
    the 4096-token prefix the model tests check: the ping-pong kernel over
    the packed projection, the V-transposed form the cfg5 model runs (fed by
    xb_linear_qkv_vt through an identity projection, so its input is exactly
    the same projection), and the four-wave kernel under an all-valid key
    mask are bitwise equal over the whole output, and sampled query rows
    match an FP32 reference computed on the CPU from the same FP16 values.

    The rows sampled: the first and last ones, rows on 64-key tile and
    512-query block edges through the sequence, and the rows at and after two
    planted keys whose scores with every later query (about 16 and 26)
    exceed everything before them by about 10 (natural log), so the online
    softmax must move its running offset and rescale the partial output at
    positions 60,001 and 99,000 (offsets move lazily, only past a margin)."""
    capi = pkg._capi
    b, s, h, hd = 1, 100000, 2, 64
    d = h * hd
    g = _gen(100000)
    qkv = torch.randn(b, s, 3 * d, generator=g)
    q = qkv[..., :d].view(s, h, hd)
    q += 1.0                                       # every query leans on the all-ones direction
    planted = {60001: 2.0, 99000: 3.25}            # key position -> multiple of the all-ones vector
    k = qkv[..., d:2 * d].view(s, h, hd)
    for pos, alpha in planted.items():
        k[pos] = alpha                             # score ~ alpha * 64 / 8 with every later query
    qkv = qkv.half()
    rows = sorted({0, 1, 63, 64, 511, 512, 513, 4095, 4096, 4097, 50175, 50176, 60000, 60001, 60002, 60063,
                   60064, 60543, 60544, 61000, 98999, 99000, 99001, 99455, 99456, 99967, 99968, 99998, 99999}
                  | set(torch.randint(0, s, (16,), generator=g).tolist()))
    ref = _rows_reference(qkv, h, rows)
    qg = qkv.to(cuda)
    print(f"attention S={s} hd={hd} heads={h}: {len(rows)} sampled rows", flush=True)
    out = pkg.attention(qg, h, causal=True, variant=capi.XB_ATTN_PINGPONG)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all())
    got = out[0, rows].cpu().float()
    torch.testing.assert_close(got, ref, atol=2e-3, rtol=1e-2)
    # the planted keys dominate the rows after them: the offset did have to move
    late = torch.tensor([r >= 60001 for r in rows])
    v_planted = qkv[0, 60001, 2 * d:].float()
    assert float((ref[late & torch.tensor([r < 99000 for r in rows])] - v_planted).abs().mean()) < 0.1
    ones = torch.ones(b, s, dtype=torch.bool, device=cuda)
    assert torch.equal(out, pkg.attention(qg, h, key_valid=ones, causal=True)), "four-wave kernel differs"
    # The V-transposed form: an identity projection (K = 3D = 384) reproduces qkv exactly.
    eye = torch.eye(3 * d, dtype=torch.float16, device=cuda)
    zero = torch.zeros(3 * d, device=cuda)
    assert torch.equal(pkg.linear(qg, eye, zero), qg)
    qkv_vt, vt = pkg.linear_qkv_vt(qg, eye, zero, h)
    out_vt = pkg.attention_vt(qkv_vt, vt, h)
    torch.cuda.synchronize()
    assert torch.equal(out_vt, out), "V-transposed form differs from the ping-pong kernel"


def _key_order(s):
    """Position of each token of a row of the transposed V: inside every
    32-token group, token 32t + 4g + i sits at 32t + 8g + i and token
    32t + 16 + 4g + i at 32t + 8g + 4 + i (the attention's key order)."""
    t = torch.arange(s)
    r = t % 32
    return t - r + 8 * ((r % 16) // 4) + 4 * (r // 16) + r % 4


@pytest.mark.parametrize("b,s,h,k", [(2, 96, 4, 256), (3, 160, 8, 512), (1, 4160, 16, 1024)])
def test_linear_qkv_vt_layout(pkg, cuda, b, s, h, k):
    """The QKV GEMM with V written transposed: Q and K columns bitwise those of
    xb_linear, vt[b, h, d, position(s)] bitwise V[b, s, h, d], zeros past S
    (row stride S rounded up to 64), for every tile variant it accepts."""
    capi = pkg._capi
    hd, d = 64, h * 64
    x = torch.randn(b, s, k, generator=_gen(s + k)).half().to(cuda)
    w = (torch.randn(3 * d, k, generator=_gen(k)) / k ** 0.5).half().to(cuda)
    bias = torch.randn(3 * d, generator=_gen(d)).to(cuda)
    full = pkg.linear(x, w, bias)
    v = full[..., 2 * d:].reshape(b, s, h, hd).permute(0, 2, 3, 1)  # [b, h, hd, s]
    row = pkg.vt_row_stride(s)
    assert row == (s + 63) // 64 * 64
    pos = _key_order(s).to(cuda)
    variants = [capi.XB_VARIANT_AUTO, capi.XB_LINEAR_DMA_256x256, capi.XB_LINEAR_DMA_128x256,
                capi.XB_LINEAR_DMA_128x128]
    for variant in variants:
        if variant in (capi.XB_LINEAR_DMA_256x256, capi.XB_LINEAR_DMA_128x256) and d % 256:
            with pytest.raises(RuntimeError):
                pkg.linear_qkv_vt(x, w, bias, h, variant=variant)
            continue
        vt = torch.full((b, h, hd, row), float("nan"), device=cuda, dtype=torch.float16)
        qkv, vt = pkg.linear_qkv_vt(x, w, bias, h, vt=vt, variant=variant)
        assert torch.equal(qkv[..., :2 * d], full[..., :2 * d]), variant
        assert torch.equal(vt[..., :s][..., pos], v), variant
        assert torch.equal(vt[..., s:], torch.zeros_like(vt[..., s:])), variant


@pytest.mark.parametrize("b,s,h", [(3, 32, 2), (2, 96, 2), (1, 4160, 4), (1, 8224, 2)])
def test_attention_vt_matches_ping_pong(pkg, cuda, b, s, h):
    """Causal attention reading V transposed by the QKV GEMM: bitwise the
    ping-pong kernel over the full projection (same scores, probabilities and
    products; only the V fragment reads differ), and the FP32 reference."""
    capi = pkg._capi
    hd, d, k = 64, h * 64, 256
    x = torch.randn(b, s, k, generator=_gen(3 * s + h)).half().to(cuda)
    w = (torch.randn(3 * d, k, generator=_gen(s)) / k ** 0.5).half().to(cuda)
    bias = (0.1 * torch.randn(3 * d, generator=_gen(h))).to(cuda)
    full = pkg.linear(x, w, bias)
    expected = pkg.attention(full, h, causal=True, variant=capi.XB_ATTN_PINGPONG)
    qkv, vt = pkg.linear_qkv_vt(x, w, bias, h)
    out = pkg.attention_vt(qkv, vt, h)
    assert torch.equal(out, expected)
    if s <= 4160:
        ref = _attention_reference(full.cpu(), h, causal=True)
        torch.testing.assert_close(out.cpu().float(), ref, atol=2e-3, rtol=1e-2)


def test_wrong_destination_buffers_are_refused(pkg, cuda):
    """Caller-supplied destinations are checked against what the kernel writes
    (shape, dtype, device, contiguity) before anything is launched."""
    kernels = __import__(pkg.__name__ + ".kernels", fromlist=["linear"])
    x = torch.randn(2, 64, 256, device=cuda).half()
    w = torch.randn(3 * 256, 256, device=cuda).half()
    with pytest.raises(ValueError):
        pkg.linear(x, w, None, out=torch.empty(2, 64, 3 * 256 - 8, device=cuda, dtype=torch.float16))
    with pytest.raises(ValueError):
        pkg.linear(x, w, None, out=torch.empty(2, 64, 3 * 256, device=cuda, dtype=torch.float32))
    qkv = pkg.linear(x, w, None)
    with pytest.raises(ValueError):
        pkg.attention(qkv, 4, out=torch.empty(2, 63, 256, device=cuda, dtype=torch.float16))
    with pytest.raises(ValueError):
        pkg.attention(qkv, 4, out=torch.empty(2, 256, 64, device=cuda, dtype=torch.float16).transpose(1, 2))
    with pytest.raises(ValueError):
        pkg.linear_qkv_vt(x, w, None, 4, vt=torch.empty(2, 4, 64, 32, device=cuda, dtype=torch.float16))
    r = torch.randn(2, 64, 256, device=cuda)
    g, b = torch.ones(256, device=cuda), torch.zeros(256, device=cuda)
    with pytest.raises(ValueError):
        pkg.fused_residual_layer_norm(r, x, g, b, 1e-5, torch.float16,
                                      norm_out=torch.empty(2, 64, 256, device=cuda, dtype=torch.float32))
    xs = torch.randn(1, 16, 128, device=cuda)
    with pytest.raises(ValueError):  # the packed weights of one layer passed for two
        kernels.fused_forward_d128(xs, torch.empty(6 * 128 * 128, device=cuda, dtype=torch.float16),
                                   torch.empty(9 * 128 + 128 + 256, device=cuda), 4, 128, 2)


def test_qkv_vt_argument_errors(pkg, cuda):
    """Shapes the transposed-V path does not take are refused before any launch."""
    lib = pkg._capi.lib()
    unsupported, bad_variant = -4, -10  # XB_ERR_UNSUPPORTED_SHAPE, XB_ERR_BAD_VARIANT
    # seq_len not a multiple of 32, K % 64 != 0, head_dim other than 64 for the attention
    assert lib.xb_linear_qkv_vt(None, None, None, None, None, 1, 100, 2, 64, 256, -1, None) == unsupported
    assert lib.xb_linear_qkv_vt(None, None, None, None, None, 1, 96, 2, 64, 200, -1, None) == unsupported
    assert lib.xb_attention_causal_vt(None, None, None, 1, 96, 2, 32, 0.1, None) == unsupported
    assert lib.xb_attention_causal_vt(None, None, None, 1, 100, 2, 64, 0.1, None) == unsupported
    # an NT tile, or a tile width that does not divide D
    assert lib.xb_linear_qkv_vt(None, None, None, None, None, 1, 96, 2, 64, 256, 4, None) == bad_variant
    assert lib.xb_linear_qkv_vt(None, None, None, None, None, 1, 96, 3, 64, 256, 0, None) == bad_variant


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("hd,b,s,h,variants", [
    (256, 2, 300, 2, ("XB_ATTN_W4_Q16", "XB_ATTN_W8_Q16")),
    (128, 1, 333, 2, ("XB_ATTN_W4_Q32",)),
    (64, 2, 4100, 1, ("XB_ATTN_W4_Q32", "XB_ATTN_W4_Q64", "XB_ATTN_PINGPONG")),
    (32, 1, 1100, 3, ("XB_ATTN_W4_Q32", "XB_ATTN_W4_Q64")),
])
def test_attention_every_variant(pkg, cuda, causal, hd, b, s, h, variants):
    """Every attention kernel the plan can name (xb_attention_v), forced on a
    shape it is built for, against the FP32 reference; the ping-pong kernel is
    refused under a key mask."""
    capi = pkg._capi
    qkv = torch.randn(b, s, 3 * h * hd, generator=_gen(hd + s)).half()
    ref = _attention_reference(qkv, h, causal=causal)
    qg = qkv.to(cuda)
    for name in variants:
        out = pkg.attention(qg, h, causal=causal, variant=getattr(capi, name))
        torch.testing.assert_close(out.cpu().float(), ref, atol=2e-3, rtol=1e-2, msg=lambda e, n=name: f"{n}: {e}")
    if hd == 64:
        ones = torch.ones(b, s, dtype=torch.bool, device=cuda)
        with pytest.raises(RuntimeError, match="code -10"):
            pkg.attention(qg, h, key_valid=ones, causal=causal, variant=capi.XB_ATTN_PINGPONG)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("masked", [False, True])
def test_attention_hd256_short_one_block_per_head(pkg, cuda, causal, masked):
    """cfg3's geometry (B*H = 256 heads of S = 128, head_dim 256) takes one 8-wave
    block per head; slices of two sequences (8 heads) take the 4-wave blocks.
    Same per-wave work, so the two must agree bitwise; FP32 reference too."""
    b, s, h, hd = 64, 128, 4, 256
    qkv = torch.randn(b, s, 3 * h * hd, generator=_gen(256 + causal)).half()
    valid = _padding_mask(b, s, "random_with_empty", 3) if masked else None
    qg = qkv.to(cuda)
    vg = None if valid is None else valid.to(cuda)
    whole = pkg.attention(qg, h, key_valid=vg, causal=causal)
    for i in range(0, b, 2):
        part = pkg.attention(qg[i:i + 2].contiguous(), h, causal=causal,
                             key_valid=None if vg is None else vg[i:i + 2].contiguous())
        assert torch.equal(whole[i:i + 2], part), i
    ref = _attention_reference(qkv[:8], h, key_valid=None if valid is None else valid[:8], causal=causal)
    torch.testing.assert_close(whole[:8].cpu().float(), ref, atol=2e-3, rtol=1e-2)


def test_causal_attention_first_token_is_value(pkg, cuda):
    """Query 0 sees only key 0, so its context equals v[0] exactly (up to FP16)."""
    qkv = torch.randn(3, 50, 3 * 4 * 32, generator=_gen(9)).half()
    out = pkg.causal_attention(qkv.to(cuda), 4).cpu()
    v0 = qkv[:, 0, 2 * 128:].float()
    torch.testing.assert_close(out[:, 0].float(), v0, atol=1e-3, rtol=1e-3)


def _padding_mask(b: int, s: int, kind: str, seed: int) -> torch.Tensor:
    gen = _gen(seed)
    pos = torch.arange(s)[None, :]
    lengths = torch.randint(1, s + 1, (b,), generator=gen)
    if kind == "right":
        return pos < lengths[:, None]
    if kind == "left":
        return pos >= (s - lengths)[:, None]
    mask = torch.rand(b, s, generator=gen) > 0.3
    if kind == "random_with_empty" and b > 1:
        mask[1] = False  # a sequence with no valid key at all
    return mask


@pytest.mark.parametrize("hd", [8, 32, 64, 128, 256])
@pytest.mark.parametrize("b,s,h", [(3, 1, 2), (3, 77, 2), (2, 300, 2), (2, 1100, 1)])
@pytest.mark.parametrize("kind", ["right", "left", "random_with_empty"])
@pytest.mark.parametrize("causal", [True, False])
def test_attention_key_padding(pkg, cuda, hd, b, s, h, kind, causal):
    qkv = torch.randn(b, s, 3 * h * hd, generator=_gen(hd * 31 + s)).half()
    mask = _padding_mask(b, s, kind, seed=s + hd)
    ref = _attention_reference(qkv, h, key_valid=mask, causal=causal)
    out = pkg.attention(qkv.to(cuda), h, key_valid=mask.to(cuda), causal=causal)
    assert out.shape == (b, s, h * hd)
    # FP16 probabilities and FP16 output rounding; fully masked queries are exactly zero.
    torch.testing.assert_close(out.cpu().float(), ref, atol=2e-3, rtol=1e-2)


@pytest.mark.parametrize("hd", [16, 64, 128])
@pytest.mark.parametrize("s", [1, 100, 1500])
def test_attention_non_causal(pkg, cuda, hd, s):
    h = 2
    qkv = torch.randn(2, s, 3 * h * hd, generator=_gen(hd + 7 * s)).half()
    ref = _attention_reference(qkv, h, causal=False)
    out = pkg.attention(qkv.to(cuda), h, causal=False)
    torch.testing.assert_close(out.cpu().float(), ref, atol=2e-3, rtol=1e-2)


def test_attention_all_valid_mask_equals_unmasked(pkg, cuda):
    qkv = torch.randn(2, 257, 3 * 2 * 64, generator=_gen(5)).half().to(cuda)
    ones = torch.ones(2, 257, dtype=torch.bool, device=cuda)
    a = pkg.causal_attention(qkv, 2)
    m = pkg.attention(qkv, 2, key_valid=ones, causal=True)
    assert torch.equal(a, m)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("long_s", [False, True])  # True: the ping-pong kernel
def test_attention_large_negative_first_scores(pkg, cuda, causal, long_s):
    """First key tile scores far below zero (2^-185 probabilities before the shift).

    The running offset must jump onto them without rescaling the still-empty
    accumulators by exp2(185) (= inf, and 0 * inf = NaN).
    """
    b, s, h, hd = 1, 192 if long_s is False else 4160, 1, 64
    q = torch.full((s, hd), 4.0)
    k = torch.full((s, hd), 0.05)
    k[:64] = -4.0                      # q.k * scale * log2(e) = -184.7 for keys 0..63
    v = torch.randn(s, hd, generator=_gen(11))
    qkv = torch.cat((q, k, v), 1).reshape(b, s, 3 * hd).half()
    ref = _attention_reference(qkv, h, causal=causal)
    out = pkg.attention(qkv.to(cuda), h, causal=causal).cpu().float()
    assert torch.isfinite(out).all()
    torch.testing.assert_close(out, ref, atol=2e-3, rtol=1e-2)


@pytest.mark.parametrize("cols", [128, 1024, 96])
@pytest.mark.parametrize("mode", [1, 2, 4, 3, 6, 7])
def test_residual_layer_norm_row_masks(pkg, cuda, cols, mode):
    """XB_MASK_UPDATE (1) / XB_MASK_SUM (2) / XB_MASK_OUTPUT (4) on the rows whose flag is 0."""
    rows = 301
    r = torch.randn(rows, cols, generator=_gen(13)) * 1.5
    u = (torch.randn(rows, cols, generator=_gen(14)) * 0.7).half()
    valid = torch.rand(rows, generator=_gen(15)) > 0.4
    u[~valid] = float("nan")           # a masked update must not leak (selection, not multiply)
    g = torch.randn(cols, generator=_gen(16)) * 0.3 + 1.0
    b = torch.randn(cols, generator=_gen(17)) * 0.1
    inv = ~valid[:, None]
    s = r + u.float()
    if mode & 1:
        s = torch.where(inv, r, s)
    if mode & 2:
        s = torch.where(inv, torch.zeros_like(s), s)
    ref = F.layer_norm(s, (cols,), g, b, 1e-5)
    if mode & 4:
        ref = torch.where(inv, torch.zeros_like(ref), ref)
    res, norm = pkg.fused_residual_layer_norm(
        r.to(cuda), u.to(cuda), g.to(cuda), b.to(cuda), 1e-5, F32, row_valid=valid.to(cuda), mask_mode=mode)
    # Without UPDATE/SUM the masked rows keep the NaN sum, exactly as the reference would.
    torch.testing.assert_close(res.cpu(), s, atol=0, rtol=0, equal_nan=True)
    torch.testing.assert_close(norm.cpu(), ref, atol=2e-5, rtol=2e-5, equal_nan=True)


# ----------------------------------------------------------------------------- KV cache
def _fill_cache(pkg, qkv_full, heads, capacity, pieces, cuda):
    """Append qkv_full's tokens to fresh caches in the given chunk sizes."""
    b, length, width = qkv_full.shape
    hd = width // 3 // heads
    kc = torch.full((b, heads, capacity, hd), 7.0, dtype=F16, device=cuda)   # sentinel
    vc = torch.full_like(kc, -7.0)
    start = 0
    for n in pieces:
        pkg.kv_cache_append(qkv_full[:, start:start + n].contiguous().to(cuda), kc, vc, heads, start)
        start += n
    assert start == length
    return kc, vc


def test_kv_cache_append_layout(pkg, cuda):
    b, heads, hd, capacity = 2, 3, 32, 40
    qkv = torch.randn(b, 23, 3 * heads * hd, generator=_gen(31)).half()
    kc, vc = _fill_cache(pkg, qkv, heads, capacity, [1, 16, 6], cuda)
    t = qkv.view(b, 23, 3, heads, hd).permute(2, 0, 3, 1, 4)   # which, b, h, s, hd
    assert torch.equal(kc[:, :, :23].cpu(), t[1])
    assert torch.equal(vc[:, :, :23].cpu(), t[2])
    assert (kc[:, :, 23:] == 7.0).all() and (vc[:, :, 23:] == -7.0).all()   # nothing past the chunk
    with pytest.raises(ValueError, match="capacity exceeded"):
        pkg.kv_cache_append(qkv[:, :18].contiguous().to(cuda), kc, vc, heads, 23)


@pytest.mark.parametrize("hd", [8, 16, 32, 64, 128, 256])
@pytest.mark.parametrize("start,chunk", [(0, 1), (1, 1), (63, 1), (64, 5), (200, 16), (37, 17), (130, 100), (0, 70)])
def test_attention_kv_cache(pkg, cuda, hd, start, chunk):
    """Queries at positions start.. over the cached prefix == rows of full causal attention."""
    b, heads = 2, 2 if hd < 256 else 1
    length = start + chunk
    qkv_full = torch.randn(b, length, 3 * heads * hd, generator=_gen(hd * 7 + length)).half()
    kc, vc = _fill_cache(pkg, qkv_full, heads, length + 9, [start, chunk] if start else [chunk], cuda)
    ref = _attention_reference(qkv_full, heads)[:, start:]
    out = pkg.attention_kv_cache(qkv_full[:, start:].contiguous().to(cuda), kc, vc, heads, start)
    assert out.shape == (b, chunk, heads * hd)
    # FP16 probabilities and FP16 output rounding (as for the causal kernel).
    torch.testing.assert_close(out.cpu().float(), ref, atol=2e-3, rtol=1e-2)


@pytest.mark.parametrize("b,heads,hd,start", [(1, 16, 64, 20000), (3, 2, 128, 5000), (1, 1, 256, 3000), (64, 4, 32, 127)])
def test_decode_long_cache(pkg, cuda, b, heads, hd, start):
    """One new token over a long cache: many key splits merged by the combine kernel."""
    length = start + 1
    qkv_full = torch.randn(b, length, 3 * heads * hd, generator=_gen(start)).half()
    kc, vc = _fill_cache(pkg, qkv_full, heads, length, [start, 1], cuda)
    q_last = qkv_full[:, start:].contiguous()
    t = qkv_full.float().view(b, length, 3, heads, hd)
    scores = torch.einsum("bhd,bkhd->bhk", t[:, start, 0], t[:, :, 1]) * hd**-0.5
    ref = torch.einsum("bhk,bkhd->bhd", torch.softmax(scores, -1), t[:, :, 2]).reshape(b, 1, heads * hd)
    need = pkg.kernels.kv_cache_workspace_bytes(b, 1, heads, hd, start)
    assert need > 0
    out = pkg.attention_kv_cache(q_last.to(cuda), kc, vc, heads, start)
    torch.testing.assert_close(out.cpu().float(), ref, atol=2e-3, rtol=1e-2)


def test_decode_workspace_too_small(pkg, cuda):
    b, heads, hd, start = 1, 2, 64, 300
    qkv_full = torch.randn(b, start + 1, 3 * heads * hd, generator=_gen(3)).half()
    kc, vc = _fill_cache(pkg, qkv_full, heads, start + 1, [start, 1], cuda)
    lib = pkg._capi.lib()
    out = torch.empty(b, 1, heads * hd, device=cuda, dtype=F16)
    q = qkv_full[:, start:].contiguous().to(cuda)
    need = pkg.kernels.kv_cache_workspace_bytes(b, 1, heads, hd, start)
    ws = torch.empty(need, device=cuda, dtype=torch.uint8)
    code = lib.xb_attention_kv_cache(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), out.data_ptr(), b, 1, heads, hd,
                                     start, start + 1, 0.125, ws.data_ptr(), need - 16, None)
    assert code == -7
    code = lib.xb_attention_kv_cache(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), out.data_ptr(), b, 1, heads, hd,
                                     start, start + 1, 0.125, None, 0, None)
    assert code == -1
