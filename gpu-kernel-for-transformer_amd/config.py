"""Model configuration, the official shape table and the per-shape execution plan.

`TransformerConfig` and `OFFICIAL_BENCHMARK_SHAPES` keep the reference's
field order, validation messages and table (torch_transformer_benchmark.py:47-95)
because they are the drop-in type: configs are positional, hashable dict keys.

`ShapeExecutionPlan` keeps the reference's fields and `describe()` format
(torch_transformer_benchmark.py:98-157), but its values name this build's
gfx950 kernel choices instead of Ampere/Triton strategies.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, Optional


@dataclass(frozen=True)
class TransformerConfig:
    """Causal pre-norm Transformer geometry (torch_transformer_benchmark.py:47-74)."""

    batch_size: int
    seq_len: int
    d_model: int
    num_heads: int
    ffn_dim: int
    num_layers: int
    causal: bool

    def validate(self) -> None:
        if self.batch_size <= 0:
            raise ValueError("batch_size must be positive")
        if self.seq_len <= 0:
            raise ValueError("seq_len must be positive")
        if self.d_model <= 0:
            raise ValueError("d_model must be positive")
        if self.num_heads <= 0:
            raise ValueError("num_heads must be positive")
        if self.d_model % self.num_heads != 0:
            raise ValueError(
                f"d_model ({self.d_model}) must be divisible by "
                f"num_heads ({self.num_heads})"
            )
        if self.ffn_dim <= 0:
            raise ValueError("ffn_dim must be positive")
        if self.num_layers <= 0:
            raise ValueError("num_layers must be positive")

    @property
    def head_dim(self) -> int:
        return self.d_model // self.num_heads


# The hackathon's official shapes (torch_transformer_benchmark.py:80-95);
# ``d_model`` is the table's QKV dimension.
OFFICIAL_BENCHMARK_SHAPES: Dict[int, TransformerConfig] = {
    1: TransformerConfig(64, 128, 128, 4, 128, 4, True),
    2: TransformerConfig(1, 128, 128, 4, 128, 4, True),
    3: TransformerConfig(4, 128, 128, 4, 128, 4, True),
    4: TransformerConfig(16, 128, 128, 4, 128, 4, True),
    5: TransformerConfig(128, 128, 128, 4, 128, 4, True),
    6: TransformerConfig(10000, 128, 128, 4, 128, 4, True),
    7: TransformerConfig(64, 128, 32, 4, 32, 4, True),
    8: TransformerConfig(64, 128, 1024, 4, 1024, 4, True),
    9: TransformerConfig(64, 128, 128, 1, 128, 4, True),
    10: TransformerConfig(64, 128, 128, 2, 128, 4, True),
    11: TransformerConfig(64, 128, 128, 16, 128, 4, True),
    12: TransformerConfig(64, 32, 128, 4, 128, 4, True),
    13: TransformerConfig(64, 1024, 128, 4, 128, 4, True),
    14: TransformerConfig(32, 100000, 1024, 16, 1024, 2, True),
}

# The five measured configurations, in the benchmark's order (cfg1 to cfg5), as official shape ids.
BENCHMARK_CONFIG_SHAPE_IDS = (1, 6, 8, 11, 14)

_OFFICIAL_SHAPE_IDS_BY_CONFIG = {
    config: shape_id for shape_id, config in OFFICIAL_BENCHMARK_SHAPES.items()
}


# One MI355X: 288 GB of HBM3E.  A batch whose forward working set exceeds
# this share of it runs in independent slices (batch elements are
# independent, README.md:260-263); every official batch fits whole.
HBM_BYTES = 288e9
CHUNK_BUDGET_FRACTION = 0.6


def forward_working_set_bytes(config: TransformerConfig, batch: int, seq_len: int, fused: bool = False) -> int:
    """Device bytes one forward of [batch, seq_len] keeps alive, input and output included.

    Per-op path: x and y (FP32), the FP32 residual stream, and the FP16
    intermediates (LayerNorm outputs, packed QKV, attention context, the two
    projection updates, FFN hidden), counted as if all were live at once.
    The whole-stack kernel keeps only x and y.
    """
    d, f = config.d_model, config.ffn_dim
    per_token = 8 * d if fused else 4 * d + 4 * d + 4 * d + 2 * (d + 3 * d + d + d + d + f + d)
    return int(batch) * int(seq_len) * per_token


@dataclass(frozen=True)
class ShapeExecutionPlan:
    """The kernels one forward runs on gfx950 (torch_transformer_benchmark.py:98-157).

    Built by `resolve_shape_execution_plan` from the library's own selection
    functions (xb_select_*), and read back by the model's forward, so
    `describe()` names what actually runs.  ffn / attention / projection
    strategies keep the reference's field names; `forward_strategy` is the
    whole-stack kernel form (`fused_stack_*`) or `per_op`, and the *_variant
    fields are the ids the model passes to the kernels (-1: not used).
    batch_chunk_size > 0 runs the batch in independent slices
    (torch_transformer_benchmark.py:1022-1049).
    """

    official_shape_id: Optional[int]
    ffn_strategy: str = "unresolved"
    attention_strategy: str = "unresolved"
    projection_strategy: str = "unresolved"
    batch_chunk_size: int = 0
    forward_strategy: str = "unresolved"
    arch: str = "gfx950"
    batch: int = 0
    seq_len: int = 0
    masked: bool = False
    fused_variant: int = -1
    qkv_variant: int = -1
    out_variant: int = -1
    ffn_in_variant: int = -1
    ffn_out_variant: int = -1
    attention_variant: int = -1

    @property
    def fused(self) -> bool:
        return self.fused_variant >= 0

    @property
    def runnable(self) -> bool:
        """Whether every step has a gfx950 kernel (else forward_strategy says why not)."""
        return self.fused or self.attention_variant >= 0

    def describe(self) -> str:
        shape = (
            f"official-{self.official_shape_id}"
            if self.official_shape_id is not None
            else "general"
        )
        chunk = (
            f", batch_chunk={self.batch_chunk_size}"
            if self.batch_chunk_size
            else ""
        )
        return (
            f"{shape}: ffn={self.ffn_strategy}, "
            f"attention={self.attention_strategy}, "
            f"projections={self.projection_strategy}{chunk}; "
            f"forward={self.forward_strategy} on {self.arch} "
            f"(B={self.batch}, S={self.seq_len}{', padded' if self.masked else ''})"
        )


def _variant_name(lib, op: int, variant: int) -> str:
    name = lib.xb_variant_name(op, variant)
    return name.decode() if name else f"variant-{variant}"


def resolve_shape_execution_plan(
    config: TransformerConfig,
    batch: Optional[int] = None,
    seq_len: Optional[int] = None,
    masked: bool = False,
    fused_allowed: bool = True,
    transposed_v_allowed: bool = True,
) -> ShapeExecutionPlan:
    """The gfx950 plan for a forward of [batch, seq_len] (default: the config's own shape).

    masked: a padding mask with at least one False (the key-masked kernel
    forms).  fused_allowed: the caller's whole-stack
    conditions beyond the shape (the toggle, LayerNorm eps 1e-5 with affine
    parameters).  transposed_v_allowed: the ping-pong attention may take V
    transposed from the QKV GEMM (xb_linear_qkv_vt / xb_attention_causal_vt;
    not for KV-cached steps, which attend through the cache).  The kernel choices are the library's (xb_select_*); only a
    batch whose working set exceeds CHUNK_BUDGET_FRACTION of HBM is chunked.
    Without the library the plan stays "unresolved" (the forward then raises).
    """
    from . import _capi

    b = config.batch_size if batch is None else int(batch)
    s = config.seq_len if seq_len is None else int(seq_len)
    shape_id = _OFFICIAL_SHAPE_IDS_BY_CONFIG.get(config) if (b, s) == (config.batch_size, config.seq_len) else None
    masked = bool(masked)
    if not _capi.XBLOCK_AVAILABLE:
        return ShapeExecutionPlan(official_shape_id=shape_id, batch=b, seq_len=s, masked=masked,
                                  forward_strategy=f"unresolved ({_capi.XBLOCK_LOAD_ERROR})")
    lib = _capi.lib()
    d, f, h = config.d_model, config.ffn_dim, config.num_heads
    fused = lib.xb_select_fused_d128(b, s, h, f, int(config.causal), int(masked)) if (fused_allowed and d == 128) else -1
    budget = CHUNK_BUDGET_FRACTION * HBM_BYTES
    per_seq = forward_working_set_bytes(config, 1, s, fused=fused >= 0)
    chunk = 0 if per_seq * b <= budget else max(1, int(budget // per_seq))
    if fused >= 0:
        name = _variant_name(lib, _capi.XB_OP_FUSED_D128, fused)
        return ShapeExecutionPlan(
            official_shape_id=shape_id, batch=b, seq_len=s, masked=masked, batch_chunk_size=chunk,
            forward_strategy=f"{name} (one launch for all layers)", fused_variant=fused,
            ffn_strategy=f"{name}: MFMA GEMMs + erf GELU in registers",
            attention_strategy=f"{name}: {'causal' if config.causal else 'full'} attention, K/V^T in LDS",
            projection_strategy=f"{name}: MFMA GEMMs, weights staged in LDS",
        )
    rows = (chunk or b) * s
    qkv = lib.xb_select_linear(rows, 3 * d, d, _capi.XB_EPI_BIAS)
    out = lib.xb_select_linear(rows, d, d, _capi.XB_EPI_BIAS)
    ffn_in = lib.xb_select_linear(rows, f, d, _capi.XB_EPI_BIAS_GELU)
    ffn_out = lib.xb_select_linear(rows, d, f, _capi.XB_EPI_BIAS)
    attn = lib.xb_select_attention(chunk or b, s, h, d // h, int(masked))
    missing = [f"{what}: {lib.xb_strerror(code).decode()}" for what, code in
               (("qkv", qkv), ("out", out), ("ffn_in", ffn_in), ("ffn_out", ffn_out), ("attention", attn)) if code < 0]
    if missing:
        return ShapeExecutionPlan(official_shape_id=shape_id, batch=b, seq_len=s, masked=masked, batch_chunk_size=chunk,
                                  forward_strategy="unsupported (" + "; ".join(missing) + ")")
    # The long-sequence (ping-pong) attention reads V transposed by the QKV
    # GEMM when the shape allows it: causal, 32 | S, and a QKV tile whose
    # width divides D, so every tile is all Q/K or all V.
    if (transposed_v_allowed and attn == _capi.XB_ATTN_PINGPONG and config.causal and s % 32 == 0
            and d % 128 == 0 and d >= 256):
        widths = {_capi.XB_LINEAR_DMA_256x256: 256, _capi.XB_LINEAR_DMA_128x256: 256, _capi.XB_LINEAR_DMA_128x128: 128}
        if d % widths.get(qkv, d + 1) != 0:
            qkv = _capi.XB_LINEAR_DMA_256x256 if d % 256 == 0 else _capi.XB_LINEAR_DMA_128x128
        attn = _capi.XB_ATTN_PINGPONG_VT
    lin = lambda v: _variant_name(lib, _capi.XB_OP_LINEAR, v)  # noqa: E731
    return ShapeExecutionPlan(
        official_shape_id=shape_id, batch=b, seq_len=s, masked=masked, batch_chunk_size=chunk,
        forward_strategy="per_op (LayerNorm, QKV GEMM, attention, out GEMM, residual LayerNorm, FFN GEMMs per layer)",
        ffn_strategy=f"{lin(ffn_in)}+gelu_erf / {lin(ffn_out)}",
        attention_strategy=_variant_name(lib, _capi.XB_OP_ATTENTION, attn),
        projection_strategy=f"qkv {lin(qkv)}, out {lin(out)}",
        qkv_variant=qkv, out_variant=out, ffn_in_variant=ffn_in, ffn_out_variant=ffn_out, attention_variant=attn,
    )
