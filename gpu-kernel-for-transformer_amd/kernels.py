"""Tensor-level wrappers over the C-ABI, mirroring the reference's kernel API.

`layer_norm` and `fused_residual_layer_norm` keep the names, argument meaning
and error behaviour of triton_fused_norm.py:140-215 (ValueError for device or
shape mismatches, RuntimeError when the kernels are unavailable).  `linear`,
`ffn_gelu` and `causal_attention` replace F.linear (torch_transformer_benchmark.py:685,
:741), triton_ffn_gelu (triton_fused_ffn.py:224-261) and the SDPA dispatch
(torch_transformer_benchmark.py:767-809).  The GEMM wrappers take weights in
nn.Linear's own [out, in] layout: both MFMA operands are then K-contiguous,
so the reference's cached [in, out] transposes have no counterpart here.

All wrappers allocate their outputs with torch (the caller owns them), enqueue
on torch's current stream, and never synchronise: they are capture-safe.
"""

from __future__ import annotations

import threading
import weakref
from functools import lru_cache
from typing import Callable, Dict, List, Optional, Tuple

import torch

from . import _capi
from ._capi import XB_EPI_BIAS, XB_EPI_BIAS_GELU, XB_F16, XB_F32, check, lib, stream_handle

_DTYPE_CODES = {torch.float32: XB_F32, torch.float16: XB_F16}


class LaunchRecorder:
    """Opt-in per-launch timing: brackets every kernel launch with HIP events.

    Used by bench.py to measure each kernel's average duration inside the timed
    region, on the stream the kernel is launched on.  While no recorder is
    active a launch costs one `is None` check.

        with LaunchRecorder() as rec:
            model(x)
        torch.cuda.synchronize(); rec.durations_ms() -> {name: [ms, ...]}
    """

    _active: Optional["LaunchRecorder"] = None

    def __init__(self) -> None:
        self.events: Dict[str, List[Tuple[torch.cuda.Event, torch.cuda.Event]]] = {}

    def __enter__(self) -> "LaunchRecorder":
        LaunchRecorder._active = self
        return self

    def __exit__(self, *exc) -> None:
        LaunchRecorder._active = None

    def durations_ms(self) -> Dict[str, List[float]]:
        return {name: [a.elapsed_time(b) for a, b in pairs] for name, pairs in self.events.items()}


def _launch(name: str, fn: Callable[[], int]) -> int:
    recorder = LaunchRecorder._active
    if recorder is None:
        return fn()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    code = fn()
    end.record()
    recorder.events.setdefault(name, []).append((start, end))
    return code


@lru_cache(maxsize=None)
def _device_is_gfx950(index: int) -> bool:
    return _capi.gfx_arch(torch.device("cuda", index)) == "gfx950"


def _require_device(tensor: torch.Tensor, what: str) -> None:
    lib()
    if tensor.device.type != "cuda":
        raise ValueError(f"{what} requires GPU tensors")
    if not _device_is_gfx950(tensor.device.index if tensor.device.index is not None else torch.cuda.current_device()):
        raise RuntimeError(f"{what}: the xblock kernels are built for gfx950 only")


def _dtype_code(dtype: torch.dtype, what: str) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise ValueError(f"{what}: unsupported dtype {dtype}") from None


def _check_buffer(t: torch.Tensor, shape, dtype: torch.dtype, device: torch.device, what: str) -> None:
    """A caller-supplied destination must be exactly what the kernel writes:
    the kernels index it from the sizes of the other arguments."""
    if tuple(t.shape) != tuple(shape) or t.dtype != dtype or t.device != device or not t.is_contiguous():
        raise ValueError(f"{what} must be a contiguous {dtype} tensor of shape {tuple(shape)} on {device}")


def _ptr(tensor: Optional[torch.Tensor]) -> Optional[int]:
    return None if tensor is None else tensor.data_ptr()


def layer_norm(
    inputs: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor,
    eps: float,
    output_dtype: torch.dtype,
    apply_affine: bool = True,
) -> torch.Tensor:
    """LayerNorm whose output is stored directly in the next GEMM's dtype (FN:140-170)."""
    _require_device(inputs, "layer_norm")
    n_cols = inputs.shape[-1]
    if n_cols != weight.numel() or weight.shape != bias.shape:
        raise ValueError("LayerNorm parameters do not match the input width")
    if inputs.dtype != torch.float32:
        raise ValueError("layer_norm expects float32 inputs")
    inputs = inputs.contiguous()
    output = torch.empty_like(inputs, dtype=output_dtype)
    rows = inputs.numel() // n_cols
    code = _dtype_code(output_dtype, "layer_norm")
    check(
        _launch(f"layernorm_{n_cols}", lambda: lib().xb_layernorm(
            inputs.data_ptr(), _ptr(weight), _ptr(bias), output.data_ptr(), code, rows, n_cols,
            float(eps), int(bool(apply_affine)), stream_handle(inputs.device),
        )),
        "xb_layernorm",
    )
    return output


def fused_residual_layer_norm(
    residual: torch.Tensor,
    update: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor,
    eps: float,
    norm_dtype: torch.dtype,
    store_residual: bool = True,
    apply_affine: bool = True,
    residual_out: Optional[torch.Tensor] = None,
    norm_out: Optional[torch.Tensor] = None,
    row_valid: Optional[torch.Tensor] = None,
    mask_mode: int = 0,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Return (residual + update in FP32, LayerNorm of it in `norm_dtype`) (FN:173-215).

    With store_residual=False the sum is not written and the input `residual`
    object is returned, as in the reference.  `residual_out` / `norm_out` let
    a caller supply destinations (residual_out may be `residual` itself).

    `row_valid` (bool or uint8, one entry per row) with `mask_mode` (a mask of
    XB_MASK_UPDATE / XB_MASK_SUM / XB_MASK_OUTPUT) applies the baseline's
    padding rules to the rows whose entry is false: drop the update, zero the
    sum, zero the normalised output (torch_transformer_benchmark.py:263-264,
    :290-291, :314-315).
    """
    _require_device(residual, "fused_residual_layer_norm")
    if residual.shape != update.shape:
        raise ValueError("residual and update must have identical shapes")
    if residual.shape[-1] != weight.numel() or weight.shape != bias.shape:
        raise ValueError("LayerNorm parameters do not match the input width")
    if residual.dtype != torch.float32:
        raise ValueError("the residual stream must be float32")
    if not residual.is_contiguous() or not update.is_contiguous():
        raise ValueError("residual and update must be contiguous")
    n_cols = residual.shape[-1]
    if store_residual:
        if residual_out is None:
            residual_out = torch.empty_like(residual)
        else:
            _check_buffer(residual_out, residual.shape, torch.float32, residual.device, "residual_out")
    else:
        residual_out = None
    if norm_out is None:
        norm_out = torch.empty_like(residual, dtype=norm_dtype)
    else:
        _check_buffer(norm_out, residual.shape, norm_dtype, residual.device, "norm_out")
    rows = residual.numel() // n_cols
    upd_code, norm_code = _dtype_code(update.dtype, "update"), _dtype_code(norm_out.dtype, "norm")
    name = f"residual_layernorm_{n_cols}{'' if store_residual else '_final'}"
    if row_valid is None:
        if mask_mode:
            raise ValueError("mask_mode needs row_valid")
        check(
            _launch(name, lambda: lib().xb_residual_layernorm(
                residual.data_ptr(), update.data_ptr(), upd_code, _ptr(weight), _ptr(bias),
                _ptr(residual_out), norm_out.data_ptr(), norm_code, rows, n_cols, float(eps),
                int(bool(apply_affine)), stream_handle(residual.device),
            )),
            "xb_residual_layernorm",
        )
    else:
        valid = _byte_mask(row_valid, rows, residual.device, "row_valid")
        check(
            _launch(name + "_masked", lambda: lib().xb_residual_layernorm_masked(
                residual.data_ptr(), update.data_ptr(), upd_code, _ptr(weight), _ptr(bias),
                _ptr(residual_out), norm_out.data_ptr(), norm_code, rows, n_cols, float(eps),
                int(bool(apply_affine)), valid.data_ptr(), int(mask_mode),
                stream_handle(residual.device),
            )),
            "xb_residual_layernorm_masked",
        )
    return (residual_out if store_residual else residual), norm_out


def _byte_mask(mask: torch.Tensor, count: int, device: torch.device, what: str) -> torch.Tensor:
    """`mask` as a contiguous uint8 tensor of `count` entries on `device`."""
    if mask.numel() != count:
        raise ValueError(f"{what} must have {count} entries, got {mask.numel()}")
    if mask.device != device:
        raise ValueError(f"{what} must be on {device}")
    if mask.dtype not in (torch.bool, torch.uint8):
        raise ValueError(f"{what} must be bool or uint8")
    if mask.dtype == torch.bool:
        mask = mask.view(torch.uint8) if mask.is_contiguous() else mask.contiguous().view(torch.uint8)
    return mask.contiguous()


def linear(
    inputs: torch.Tensor,
    weight: torch.Tensor,
    bias: Optional[torch.Tensor],
    gelu: bool = False,
    out: Optional[torch.Tensor] = None,
    variant: int = _capi.XB_VARIANT_AUTO,
) -> torch.Tensor:
    """FP16 `inputs @ weight.T + bias` (optionally exact-erf GELU), FP32 accumulation.

    inputs: [..., K] float16 contiguous; weight: [N, K] float16 (nn.Linear
    layout); bias: [N] float32 or None.  Returns [..., N] float16.  `variant`
    is a tile variant (XB_LINEAR_*) from the execution plan, or auto.
    """
    _require_device(inputs, "linear")
    if weight.ndim != 2 or (bias is not None and bias.ndim != 1):
        raise ValueError("weight must be 2-D and bias must be 1-D")
    k = inputs.shape[-1]
    n = weight.shape[0]
    if weight.shape[1] != k:
        raise ValueError("weight does not match the input width")
    if bias is not None and (bias.numel() != n or bias.dtype != torch.float32):
        raise ValueError("bias must be float32 with one entry per output feature")
    if inputs.dtype != torch.float16 or weight.dtype != torch.float16:
        raise ValueError("linear expects float16 inputs and weights")
    if not inputs.is_contiguous() or not weight.is_contiguous():
        raise ValueError("linear expects contiguous inputs and weights")
    m = inputs.numel() // k
    if out is None:
        out = torch.empty((*inputs.shape[:-1], n), device=inputs.device, dtype=torch.float16)
    else:
        _check_buffer(out, (*inputs.shape[:-1], n), torch.float16, inputs.device, "out")
    epi = XB_EPI_BIAS_GELU if gelu else XB_EPI_BIAS
    check(
        _launch(f"gemm_n{n}_k{k}{'_gelu' if gelu else ''}", lambda: lib().xb_linear_v(
            inputs.data_ptr(), weight.data_ptr(), _ptr(bias), out.data_ptr(), m, n, k, epi, int(variant),
            stream_handle(inputs.device),
        )),
        "xb_linear_v",
    )
    return out


def ffn_gelu(inputs: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    """GELU(inputs @ weight.T + bias) with FP32 accumulation (triton_fused_ffn.py:224-261).

    Unlike the reference's tanh epilogue (triton_fused_ffn.py:205-213) this is
    the exact-erf GELU of the baseline (torch_transformer_benchmark.py:286).
    """
    return linear(inputs, weight, bias, gelu=True)


def causal_attention(
    qkv: torch.Tensor,
    num_heads: int,
    scale: Optional[float] = None,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Causal attention over a packed [B, S, 3*D] FP16 projection -> [B, S, D] FP16.

    Column j of the packed projection is (which, head, dim) with
    which in (q, k, v), exactly the [B, S, 3, H, hd] view the reference takes
    (torch_transformer_benchmark.py:742-745).  `scale` defaults to
    head_dim ** -0.5, SDPA's default and the baseline's (TTB:215).
    """
    return attention(qkv, num_heads, key_valid=None, causal=True, scale=scale, out=out)


def attention(
    qkv: torch.Tensor,
    num_heads: int,
    key_valid: Optional[torch.Tensor] = None,
    causal: bool = True,
    scale: Optional[float] = None,
    out: Optional[torch.Tensor] = None,
    variant: int = _capi.XB_VARIANT_AUTO,
) -> torch.Tensor:
    """Attention over a packed [B, S, 3*D] FP16 projection with optional key padding.

    key_valid ([B, S] bool/uint8, None = all valid) excludes the keys whose
    entry is false, the baseline's key padding mask (torch_transformer_benchmark.py:
    250-253); causal=False drops the causal mask.  A query that sees no key
    gets a zero row (the baseline's softmax would give NaN there, which its
    block then overwrites by zeroing the padded rows, TTB:263-264).
    `variant` is a kernel variant (XB_ATTN_*) from the execution plan, or auto.
    """
    _require_device(qkv, "attention")
    if qkv.ndim != 3 or qkv.shape[-1] % (3 * num_heads) != 0:
        raise ValueError("qkv must be [B, S, 3 * num_heads * head_dim]")
    if qkv.dtype != torch.float16 or not qkv.is_contiguous():
        raise ValueError("qkv must be contiguous float16")
    batch, seq_len, width = qkv.shape
    d_model = width // 3
    head_dim = d_model // num_heads
    if scale is None:
        scale = head_dim ** -0.5
    if out is None:
        out = torch.empty((batch, seq_len, d_model), device=qkv.device, dtype=torch.float16)
    else:
        _check_buffer(out, (batch, seq_len, d_model), torch.float16, qkv.device, "out")
    valid = None if key_valid is None else _byte_mask(key_valid, batch * seq_len, qkv.device, "key_valid")
    name = f"attention_hd{head_dim}{'' if causal else '_full'}{'' if valid is None else '_masked'}"
    check(
        _launch(name, lambda: lib().xb_attention_v(
            qkv.data_ptr(), out.data_ptr(), _ptr(valid), batch, seq_len, num_heads, head_dim,
            float(scale), int(bool(causal)), int(variant), stream_handle(qkv.device),
        )),
        "xb_attention_v",
    )
    return out


def vt_row_stride(seq_len: int) -> int:
    """Row length (elements) of the transposed-V buffer: seq_len rounded up to 64."""
    return int(lib().xb_vt_row_stride(int(seq_len)))


def linear_qkv_vt(
    inputs: torch.Tensor,
    weight: torch.Tensor,
    bias: Optional[torch.Tensor],
    num_heads: int,
    out: Optional[torch.Tensor] = None,
    vt: Optional[torch.Tensor] = None,
    variant: int = _capi.XB_VARIANT_AUTO,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """The packed QKV projection with V written transposed for `attention_vt`.

    inputs: [B, S, K] float16; weight: [3D, K] float16; bias: [3D] float32 or
    None.  Returns (qkv, vt): qkv [B, S, 3D] with the Q and K columns of
    `linear(inputs, weight, bias)` (the V columns are left unwritten) and vt
    [B, H, head_dim, vt_row_stride(S)] holding V per head dimension, each
    32-token group in the attention's key order, zeros past S.  Needs S % 32
    == 0, K % 64 == 0 and K >= 256; the long-sequence attention reads it
    (head_dim 64).
    """
    _require_device(inputs, "linear_qkv_vt")
    if inputs.ndim != 3 or weight.ndim != 2:
        raise ValueError("inputs must be [B, S, K] and weight 2-D")
    if inputs.dtype != torch.float16 or weight.dtype != torch.float16:
        raise ValueError("linear_qkv_vt expects float16 inputs and weights")
    if not inputs.is_contiguous() or not weight.is_contiguous():
        raise ValueError("linear_qkv_vt expects contiguous inputs and weights")
    if bias is not None and (bias.dtype != torch.float32 or bias.numel() != weight.shape[0]):
        raise ValueError("bias must be float32 with one entry per output feature")
    batch, seq_len, k = inputs.shape
    n = weight.shape[0]
    if weight.shape[1] != k or n % (3 * num_heads) != 0:
        raise ValueError("weight must be [3 * num_heads * head_dim, K]")
    head_dim = n // (3 * num_heads)
    vt_shape = (batch, num_heads, head_dim, vt_row_stride(seq_len))
    if out is None:
        out = torch.empty((batch, seq_len, n), device=inputs.device, dtype=torch.float16)
    else:
        _check_buffer(out, (batch, seq_len, n), torch.float16, inputs.device, "out")
    if vt is None:
        vt = torch.empty(vt_shape, device=inputs.device, dtype=torch.float16)
    else:
        _check_buffer(vt, vt_shape, torch.float16, inputs.device, "vt")
    check(
        _launch(f"gemm_n{n}_k{k}_vt", lambda: lib().xb_linear_qkv_vt(
            inputs.data_ptr(), weight.data_ptr(), _ptr(bias), out.data_ptr(), vt.data_ptr(), batch, seq_len,
            num_heads, head_dim, k, int(variant), stream_handle(inputs.device),
        )),
        "xb_linear_qkv_vt",
    )
    return out, vt


def attention_vt(
    qkv: torch.Tensor,
    vt: torch.Tensor,
    num_heads: int,
    scale: Optional[float] = None,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Causal attention over (qkv, vt) from `linear_qkv_vt`: the same values as
    causal_attention over the full projection, bit for bit (head_dim 64)."""
    _require_device(qkv, "attention_vt")
    if qkv.ndim != 3 or qkv.shape[-1] % (3 * num_heads) != 0:
        raise ValueError("qkv must be [B, S, 3 * num_heads * head_dim]")
    batch, seq_len, width = qkv.shape
    d_model = width // 3
    head_dim = d_model // num_heads
    if qkv.dtype != torch.float16 or not qkv.is_contiguous():
        raise ValueError("qkv must be contiguous float16")
    _check_buffer(vt, (batch, num_heads, head_dim, vt_row_stride(seq_len)), torch.float16, qkv.device, "vt")
    if scale is None:
        scale = head_dim ** -0.5
    if out is None:
        out = torch.empty((batch, seq_len, d_model), device=qkv.device, dtype=torch.float16)
    else:
        _check_buffer(out, (batch, seq_len, d_model), torch.float16, qkv.device, "out")
    check(
        _launch(f"attention_hd{head_dim}_vt", lambda: lib().xb_attention_causal_vt(
            qkv.data_ptr(), vt.data_ptr(), out.data_ptr(), batch, seq_len, num_heads, head_dim, float(scale),
            stream_handle(qkv.device),
        )),
        "xb_attention_causal_vt",
    )
    return out


def _check_kv_cache(qkv: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, num_heads: int) -> Tuple[int, int, int, int]:
    if qkv.ndim != 3 or qkv.shape[-1] % (3 * num_heads) != 0:
        raise ValueError("qkv must be [B, chunk, 3 * num_heads * head_dim]")
    if qkv.dtype != torch.float16 or not qkv.is_contiguous():
        raise ValueError("qkv must be contiguous float16")
    batch, chunk, width = qkv.shape
    head_dim = width // 3 // num_heads
    for name, cache in (("k_cache", k_cache), ("v_cache", v_cache)):
        if cache.ndim != 4 or cache.shape[0] != batch or cache.shape[1] != num_heads or cache.shape[3] != head_dim:
            raise ValueError(f"{name} must be [B, heads, capacity, head_dim] = [{batch}, {num_heads}, *, {head_dim}]")
        if cache.dtype != torch.float16 or not cache.is_contiguous() or cache.device != qkv.device:
            raise ValueError(f"{name} must be contiguous float16 on the projection's device")
    if k_cache.shape != v_cache.shape:
        raise ValueError("k_cache and v_cache must have the same shape")
    return batch, chunk, head_dim, k_cache.shape[2]


def kv_cache_append(qkv: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, num_heads: int, start: int) -> None:
    """Write the chunk's keys and values into the caches at positions start.. (TTB:426-462)."""
    _require_device(qkv, "kv_cache_append")
    batch, chunk, head_dim, capacity = _check_kv_cache(qkv, k_cache, v_cache, num_heads)
    if start < 0 or start + chunk > capacity:
        raise ValueError(f"KV cache capacity exceeded ({start + chunk} > {capacity})")
    check(
        _launch(f"kv_append_hd{head_dim}", lambda: lib().xb_kv_cache_append(
            qkv.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), batch, chunk, num_heads, head_dim,
            int(start), capacity, stream_handle(qkv.device))),
        "xb_kv_cache_append",
    )


def attention_kv_cache(
    qkv: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    num_heads: int,
    start: int,
    scale: Optional[float] = None,
    out: Optional[torch.Tensor] = None,
    workspace: Optional[torch.Tensor] = None,
    no_alloc: bool = False,
) -> torch.Tensor:
    """Causal attention of a chunk at positions start.. over the cached keys 0..start+chunk-1.

    Call after kv_cache_append for the same chunk (TTB:747-765).  `workspace`
    (uint8, at least kv_cache_workspace_bytes) is allocated here when not
    given; decode chunks of up to 16 tokens need one.  no_alloc=True calls
    xb_attention_kv_cache_noalloc instead, whose partials live in the
    library's static per-GPU scratch (with `out` given, nothing is
    allocated); calls that overlap in time on one GPU must not use it.
    """
    _require_device(qkv, "attention_kv_cache")
    batch, chunk, head_dim, capacity = _check_kv_cache(qkv, k_cache, v_cache, num_heads)
    if start < 0 or start + chunk > capacity:
        raise ValueError(f"KV cache capacity exceeded ({start + chunk} > {capacity})")
    if scale is None:
        scale = head_dim ** -0.5
    d_model = num_heads * head_dim
    if out is None:
        out = torch.empty((batch, chunk, d_model), device=qkv.device, dtype=torch.float16)
    else:
        _check_buffer(out, (batch, chunk, d_model), torch.float16, qkv.device, "out")
    if no_alloc:
        with torch.cuda.device(qkv.device):
            check(
                _launch(f"attention_kv_hd{head_dim}_noalloc", lambda: lib().xb_attention_kv_cache_noalloc(
                    qkv.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), out.data_ptr(), batch, chunk, num_heads,
                    head_dim, int(start), capacity, float(scale), stream_handle(qkv.device))),
                "xb_attention_kv_cache_noalloc",
            )
        return out
    need = kv_cache_workspace_bytes(batch, chunk, num_heads, head_dim, start)
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty(need, device=qkv.device, dtype=torch.uint8)
    ws_ptr = workspace.data_ptr() if need else None
    ws_bytes = workspace.numel() * workspace.element_size() if need else 0
    check(
        _launch(f"attention_kv_hd{head_dim}{'_decode' if need else ''}", lambda: lib().xb_attention_kv_cache(
            qkv.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), out.data_ptr(), batch, chunk, num_heads,
            head_dim, int(start), capacity, float(scale), ws_ptr, ws_bytes, stream_handle(qkv.device))),
        "xb_attention_kv_cache",
    )
    return out


def kv_cache_workspace_bytes(batch: int, chunk: int, num_heads: int, head_dim: int, start: int) -> int:
    """Workspace bytes xb_attention_kv_cache needs (0 for chunks longer than 16 tokens)."""
    need = lib().xb_attention_kv_cache_workspace_bytes(batch, chunk, num_heads, head_dim, int(start))
    if need < 0:
        check(int(need), "xb_attention_kv_cache_workspace_bytes")
    return int(need)


def pack_linear_fragments(weight: torch.Tensor, natural: bool = False, scale: float = 1.0) -> torch.Tensor:
    """FP16 fragment-major copy of `scale * weight` (nn.Linear [n, k]) for the fused kernel.

    natural=False gives the permuted k order used against register-resident
    activations, natural=True the plain order used against LDS-resident ones.
    """
    _require_device(weight, "pack_linear_fragments")
    if weight.ndim != 2:
        raise ValueError("weight must be 2-D")
    w = weight.detach().float().contiguous()
    n, k = w.shape
    out = torch.empty(n * k, device=w.device, dtype=torch.float16)
    check(
        _launch("pack_fragments", lambda: lib().xb_pack_linear_fragments(
            w.data_ptr(), out.data_ptr(), n, k, _capi.XB_PACK_NATURAL if natural else _capi.XB_PACK_PERMUTED,
            float(scale), stream_handle(w.device))),
        "xb_pack_linear_fragments",
    )
    return out


FUSED_D128_HEAD_DIMS = (8, 16, 32, 64, 128)


def fused_forward_d128(
    x: torch.Tensor,
    wpack: torch.Tensor,
    ppack: torch.Tensor,
    num_heads: int,
    ffn_dim: int,
    num_layers: int,
    out: Optional[torch.Tensor] = None,
    affine_mask: int = -1,
    token_valid: Optional[torch.Tensor] = None,
    causal: bool = True,
    split: bool = True,
    strict: bool = False,
    spin_limit: int = _capi.XB_SPLIT_SPINS_DEFAULT,
    fault_flags: int = 0,
) -> torch.Tensor:
    """Whole-stack forward for d_model 128 / seq_len <= 128 (see xb_fused_forward_d128).

    wpack / ppack come from UserOptimizedTransformer._fused_stack_parameters
    (Wq and bq pre-multiplied by head_dim**-0.5 * log2(e)).  affine_mask bit
    2l / 2l+1 set = apply layer l's norm1 / norm2 gamma and beta (-1: all).
    token_valid ([B, S] bool/uint8) and causal=False give the padding and
    non-causal semantics of `attention` (padded rows come out zero).
    split=True lets a small causal batch run two workgroups per sequence
    (xb_fused_forward_d128_ws) with a workspace from `fused_split_workspace`;
    the results are the same bit for bit.  A hand-off that failed (its wait
    timed out, or it came from another XCD) turns the rows of the waiting
    workgroup into NaN and counts in the workspace; strict=True also
    synchronises after the call and raises RuntimeError if the count grew.
    spin_limit / fault_flags are passed through (tests force the failure
    paths with spin_limit=0 and fault_flags=XB_SPLIT_FAULT_NO_PUBLISH, or
    with XB_SPLIT_FAULT_FOREIGN_XCD).
    """
    _require_device(x, "fused_forward_d128")
    if x.ndim != 3 or x.shape[-1] != 128 or x.dtype != torch.float32 or not x.is_contiguous():
        raise ValueError("x must be contiguous float32 [B, S, 128]")
    batch, seq_len, _ = x.shape
    if out is None:
        out = torch.empty_like(x)
    else:
        _check_buffer(out, x.shape, torch.float32, x.device, "out")
    # the packed parameters of num_layers layers (UserOptimizedTransformer._fused_stack_parameters)
    _check_buffer(wpack, (num_layers * 128 * (4 * 128 + 2 * ffn_dim),), torch.float16, x.device, "wpack")
    _check_buffer(ppack, (num_layers * (9 * 128 + ffn_dim) + 2 * 128,), torch.float32, x.device, "ppack")
    valid = None if token_valid is None else _byte_mask(token_valid, batch * seq_len, x.device, "token_valid")
    ws = fused_split_workspace(x.device, batch, seq_len, num_heads, num_layers, causal) if split else None
    ws_bytes = 0 if ws is None else ws.numel()
    before = _split_timeouts_of(ws) if (strict and ws is not None) else 0
    check(
        _launch("fused_forward_d128_split" if ws is not None else "fused_forward_d128",
                lambda: lib().xb_fused_forward_d128_ws(
            x.data_ptr(), out.data_ptr(), wpack.data_ptr(), ppack.data_ptr(), batch, seq_len,
            num_heads, ffn_dim, num_layers, int(affine_mask), _ptr(valid), int(bool(causal)),
            _ptr(ws), ws_bytes, int(spin_limit), int(fault_flags), stream_handle(x.device))),
        "xb_fused_forward_d128_ws",
    )
    if strict and ws is not None:
        grown = _split_timeouts_of(ws) - before
        if grown:
            raise RuntimeError(f"fused_forward_d128: {grown} split-form K/V hand-off(s) failed (timed out, "
                               "or published from another XCD); the affected rows are NaN")
    return out


_SPLIT_MAX_BATCH = 128  # the largest batch the library splits (its workspace serves every smaller one)
_SPLIT_WORKSPACES: dict = {}        # eager calls: (device, stream, layers) -> workspace
_SPLIT_RETIRED: list = []
_POOL_SCOPES = threading.local()    # .stack: this thread's active SplitWorkspacePool scopes
_LIVE_POOLS: "weakref.WeakSet[SplitWorkspacePool]" = weakref.WeakSet()


def _pool_stack() -> list:
    stack = getattr(_POOL_SCOPES, "stack", None)
    if stack is None:
        stack = _POOL_SCOPES.stack = []
    return stack


class SplitWorkspacePool:
    """Split-form workspaces owned by one captured graph.

    A hipGraph replays on whatever stream is current at replay time, so a
    graph must not share a workspace with eager calls (or other graphs) that
    may run beside it.  While a pool is active (``with pool:``) in a thread,
    every split call of that thread on the pool's device -- and, when the
    pool was given a stream, only on that stream -- takes the pool's own
    workspace for its layer count, made on first use outside capture (the
    warm-up calls that precede a capture make it); the graph keeps the pool
    alive.  Calls from other threads, or on other streams, never see it.
    Replays of one graph must not overlap each other, as for any graph with
    static buffers.
    """

    def __init__(self, stream: Optional[torch.cuda.Stream] = None) -> None:
        self.workspaces: Dict[Tuple[int, int], torch.Tensor] = {}
        self.stream = stream
        _LIVE_POOLS.add(self)

    def __enter__(self) -> "SplitWorkspacePool":
        _pool_stack().append(self)
        return self

    def __exit__(self, *exc) -> None:
        _pool_stack().remove(self)

    def serves(self, index: int) -> bool:
        """Whether a split call on device `index`'s current stream takes this pool's workspace."""
        if self.stream is None:
            return True
        return self.stream.device.index == index and \
            torch.cuda.current_stream(index).cuda_stream == self.stream.cuda_stream

    def timeouts(self) -> int:
        return sum(_split_timeouts_of(ws) for ws in self.workspaces.values())


def _new_split_workspace(device: torch.device, seq_len: int, num_heads: int, num_layers: int, causal: bool,
                         need: int) -> torch.Tensor:
    size = int(lib().xb_fused_forward_d128_workspace_bytes(
        _SPLIT_MAX_BATCH, int(seq_len), int(num_heads), int(num_layers), int(bool(causal))))
    return torch.zeros(max(size, need), device=device, dtype=torch.uint8)


@lru_cache(maxsize=256)
def _split_workspace_bytes(batch: int, seq_len: int, num_heads: int, num_layers: int, causal: bool) -> int:
    """xb_fused_forward_d128_workspace_bytes, a function of the shape alone (0: one workgroup per sequence)."""
    return int(lib().xb_fused_forward_d128_workspace_bytes(batch, seq_len, num_heads, num_layers, int(causal)))


def fused_split_workspace(device, batch: int, seq_len: int, num_heads: int, num_layers: int,
                          causal: bool) -> Optional[torch.Tensor]:
    """The zero-filled uint8 workspace xb_fused_forward_d128_ws needs for this shape.

    None when the shape runs one workgroup per sequence.  The layout depends
    only on the layer count, so one tensor per (device, current stream,
    layers), sized for the largest split batch (a few MB), serves every batch
    and is kept for the process: each launch signals with its own epoch, so
    calls on one stream reuse it as it is, and calls on different streams,
    which may overlap in time, never share one.  Inside a
    `SplitWorkspacePool` scope the pool's workspace is used instead.  Under
    stream capture outside such a scope no workspace is used (its replays
    could overlap eager calls that share it): the call then runs the
    one-workgroup form, with the same results.
    """
    need = _split_workspace_bytes(int(batch), int(seq_len), int(num_heads), int(num_layers), bool(causal))
    if need <= 0:
        return None
    device = torch.device(device)
    index = device.index if device.index is not None else torch.cuda.current_device()
    capturing = torch.cuda.is_current_stream_capturing()
    stack = _pool_stack()
    if stack and stack[-1].serves(index):
        pool = stack[-1]
        key = (index, int(num_layers))
        ws = pool.workspaces.get(key)
        if ws is None or ws.numel() < need:
            if capturing:
                return None
            ws = _new_split_workspace(torch.device("cuda", index), seq_len, num_heads, num_layers, causal, need)
            pool.workspaces[key] = ws
        return ws
    if capturing:
        return None
    key = (index, stream_handle(torch.device("cuda", index)), int(num_layers))
    ws = _SPLIT_WORKSPACES.get(key)
    if ws is None:
        ws = _new_split_workspace(torch.device("cuda", index), seq_len, num_heads, num_layers, causal, need)
        _SPLIT_WORKSPACES[key] = ws
    if ws.numel() < need:  # only if the library splits larger batches than _SPLIT_MAX_BATCH
        _SPLIT_RETIRED.append(ws)  # a graph captured before may still use it: never freed
        ws = torch.zeros(need, device=device, dtype=torch.uint8)
        _SPLIT_WORKSPACES[key] = ws
    return ws


def _split_timeouts_of(ws: torch.Tensor) -> int:
    return int(ws[:4].view(torch.int32).item())


def split_launches_of(ws: torch.Tensor) -> int:
    """Completed split launches on a workspace (its launch generation, bytes 8..15)."""
    return int(ws[8:16].view(torch.int64).item())


def fused_split_timeouts(device=None) -> int:
    """Failed hand-offs (timed out, or from another XCD), summed over this process's eager split workspaces on `device`."""
    total = 0
    for (index, _, _), ws in _SPLIT_WORKSPACES.items():
        if device is None or torch.device(device).index in (None, index):
            total += _split_timeouts_of(ws)
    return total


def split_handoff_failures(device=None) -> int:
    """Failed split-form hand-offs in every workspace of this process: the
    eager ones on `device` (all devices for None) and those of every live
    graph's pool.  A count that grows across a call means that call wrote
    NaN rows; reading it synchronises with the device."""
    total = fused_split_timeouts(device)
    want = None if device is None else torch.device(device).index
    for pool in list(_LIVE_POOLS):
        for (index, _), ws in pool.workspaces.items():
            if want is None or index == want:
                total += _split_timeouts_of(ws)
    return total
