"""MI355X (gfx950) causal pre-norm Transformer block inference path.

A drop-in for the reference's `UserOptimizedTransformer`
(torch_transformer_benchmark.py:320-1148): same `TransformerConfig`, same
`state_dict`, same `forward(x, valid_token_mask=None)`, with every device op a
hand-written HIP kernel in ``libxblock.so`` reached through the C-ABI declared
in include/xblock.h.

The directory name is not a Python identifier; import it with
``importlib.import_module("gpu-kernel-for-transformer_amd")`` after putting the
repository root on ``sys.path``.
"""

from ._capi import XBLOCK_AVAILABLE, XBLOCK_LOAD_ERROR, LIBRARY_PATH
from .config import (
    BENCHMARK_CONFIG_SHAPE_IDS,
    OFFICIAL_BENCHMARK_SHAPES,
    ShapeExecutionPlan,
    TransformerConfig,
    resolve_shape_execution_plan,
)
from .kernels import (
    attention,
    attention_kv_cache,
    attention_vt,
    causal_attention,
    ffn_gelu,
    fused_residual_layer_norm,
    kv_cache_append,
    layer_norm,
    linear,
    linear_qkv_vt,
    vt_row_stride,
)
from .model import (
    SelfAttentionParameters,
    TransformerBlockParameters,
    UserOptimizedTransformer,
    forward_bytes,
    forward_flops,
)

__all__ = [
    "BENCHMARK_CONFIG_SHAPE_IDS",
    "LIBRARY_PATH",
    "OFFICIAL_BENCHMARK_SHAPES",
    "SelfAttentionParameters",
    "ShapeExecutionPlan",
    "TransformerBlockParameters",
    "TransformerConfig",
    "UserOptimizedTransformer",
    "XBLOCK_AVAILABLE",
    "XBLOCK_LOAD_ERROR",
    "attention",
    "attention_kv_cache",
    "attention_vt",
    "causal_attention",
    "ffn_gelu",
    "forward_bytes",
    "forward_flops",
    "fused_residual_layer_norm",
    "kv_cache_append",
    "layer_norm",
    "linear",
    "linear_qkv_vt",
    "resolve_shape_execution_plan",
    "vt_row_stride",
]
