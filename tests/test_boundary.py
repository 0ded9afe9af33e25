"""CPU tests of the drop-in boundary: config type, state_dict compatibility,
the C-ABI library's exports and argument checks, and the no-fallback rule."""

from __future__ import annotations

import ctypes
import json
import re
from pathlib import Path

import pytest
import torch

from oracle.baseline import BaselineTransformer, copy_model_weights

REPO = Path(__file__).resolve().parents[1]


def test_config_validation_messages(pkg):
    TC = pkg.TransformerConfig
    TC(2, 4, 8, 2, 8, 1, True).validate()
    with pytest.raises(ValueError, match="batch_size must be positive"):
        TC(0, 4, 8, 2, 8, 1, True).validate()
    with pytest.raises(ValueError, match=r"d_model \(10\) must be divisible by num_heads \(4\)"):
        TC(1, 4, 10, 4, 8, 1, True).validate()
    with pytest.raises(ValueError, match="num_layers must be positive"):
        TC(1, 4, 8, 2, 8, 0, True).validate()
    assert hash(TC(1, 2, 8, 2, 8, 1, True)) == hash(TC(1, 2, 8, 2, 8, 1, True))


def test_benchmark_configs_match_baseline_json(pkg):
    """BASELINE.json's five configs are official shapes 1, 6, 8, 11, 14."""
    configs = json.loads((REPO / "BASELINE.json").read_text())["configs"]
    assert len(configs) == 5
    expected = [(64, 128, 128, 4, 128, 4), (10000, 128, 128, 4, 128, 4), (64, 128, 1024, 4, 1024, 4),
                (64, 128, 128, 16, 128, 4), (32, 100000, 1024, 16, 1024, 2)]
    for shape_id, geom in zip(pkg.BENCHMARK_CONFIG_SHAPE_IDS, expected):
        c = pkg.OFFICIAL_BENCHMARK_SHAPES[shape_id]
        assert (c.batch_size, c.seq_len, c.d_model, c.num_heads, c.ffn_dim, c.num_layers) == geom
        assert c.causal
    assert "B=10000" in configs[1] and "head_dim 8" in configs[3] and "S=100000" in configs[4]


def test_shape_plan(pkg, capi):
    """The plan is the library's selection (no GPU needed) and names what runs."""
    shapes = pkg.OFFICIAL_BENCHMARK_SHAPES
    plan = pkg.resolve_shape_execution_plan(shapes[6])
    assert plan.official_shape_id == 6
    assert plan.describe().startswith("official-6: ffn=")
    assert plan.fused and plan.fused_variant == capi.XB_FUSED_PAIRS and plan.batch_chunk_size == 0
    assert "fused_stack_1wg_8wave_pairs" in plan.describe()
    # small causal batches (up to 128 sequences) split each sequence over two workgroups
    for shape_id in (1, 5, 11):
        assert pkg.resolve_shape_execution_plan(shapes[shape_id]).fused_variant == capi.XB_FUSED_SPLIT
    # D=1024: per-op kernels; the QKV GEMM's tile is the cost model's (256 x 192 for N = 3072)
    cfg3 = pkg.resolve_shape_execution_plan(shapes[8])
    assert not cfg3.fused and cfg3.qkv_variant == 1 and "mfma_gemm_dma_256x192" in cfg3.projection_strategy
    assert cfg3.attention_strategy == "flash_8wave_128q"
    cfg5 = pkg.resolve_shape_execution_plan(shapes[14])
    assert cfg5.attention_strategy == "flash_pingpong_vt_8wave_512q" and cfg5.batch_chunk_size == 0
    assert cfg5.attention_variant == capi.XB_ATTN_PINGPONG_VT and cfg5.qkv_variant == capi.XB_LINEAR_DMA_256x256
    # V transposed by the QKV GEMM needs 32 | S and is not used for KV-cached steps
    odd = pkg.TransformerConfig(2, 100001, 1024, 16, 1024, 2, True)
    assert pkg.resolve_shape_execution_plan(odd).attention_strategy == "flash_pingpong_8wave_512q"
    assert pkg.resolve_shape_execution_plan(shapes[14], transposed_v_allowed=False).attention_variant == \
        capi.XB_ATTN_PINGPONG
    # a padded mask takes the key-masked forms: no ping-pong kernel
    assert pkg.resolve_shape_execution_plan(shapes[14], masked=True).attention_strategy == "flash_4wave_256q"
    # the whole-stack kernel off (toggle or LayerNorm contract): per-op
    assert not pkg.resolve_shape_execution_plan(shapes[6], fused_allowed=False).fused
    # a batch beyond the HBM budget runs in slices
    big = pkg.TransformerConfig(400, 100000, 1024, 16, 1024, 2, True)
    chunked = pkg.resolve_shape_execution_plan(big)
    assert 0 < chunked.batch_chunk_size < 400 and "batch_chunk=" in chunked.describe()
    general = pkg.resolve_shape_execution_plan(pkg.TransformerConfig(3, 5, 8, 2, 8, 1, True))
    assert general.official_shape_id is None and general.describe().startswith("general:")


def test_variant_selection_abi(capi):
    """xb_select_* and the *_v entry points' variant checks need no GPU."""
    lib = capi.lib()
    assert lib.xb_select_linear(8192, 3072, 1024, 0) == 1          # 256 x 192
    assert lib.xb_select_linear(8192, 384, 128, 0) in (4, 5)       # K = 128: the nt kernel
    assert lib.xb_select_linear(-1, 8, 8, 0) == -2
    assert lib.xb_select_attention(64, 128, 4, 256, 0) == 3          # cfg3: one 8-wave block per (batch, head)
    assert lib.xb_select_attention(8, 128, 4, 256, 0) == 0           # too few blocks for that
    assert lib.xb_select_attention(32, 100000, 16, 64, 0) == 4
    assert lib.xb_select_attention(32, 100000, 16, 64, 1) == 2
    assert lib.xb_select_attention(1, 8, 2, 24, 0) == -4
    assert lib.xb_select_fused_d128(64, 128, 4, 128, 1, 0) == 1
    assert lib.xb_select_fused_d128(10000, 128, 4, 128, 1, 0) == 0
    assert lib.xb_select_fused_d128(8, 128, 1, 128, 1, 1) == -4    # head_dim 128: causal, unmasked only
    assert lib.xb_select_fused_d128(8, 129, 4, 128, 1, 0) == -4
    # a variant not built for the shape is refused before any launch
    assert lib.xb_linear_v(16, 16, None, 16, 8192, 384, 128, 0, 0, None) == -10      # DMA tile needs K >= 256
    assert lib.xb_linear_v(16, 16, None, 16, 8192, 1024, 1024, 0, 1, None) == -10    # 256 x 192 needs N % 192
    assert lib.xb_attention_v(16, 16, None, 2, 64, 2, 32, 0.1, 1, 4, None) == -10     # ping-pong: head_dim 64 only
    assert lib.xb_attention_v(16, 16, 16, 2, 64, 2, 64, 0.1, 1, 4, None) == -10       # nor with a key mask
    names = {lib.xb_variant_name(op, v) for op, n in ((0, 6), (1, 5), (2, 3)) for v in range(n)}
    assert None not in names and len(names) == 14
    assert lib.xb_variant_name(0, 99) is None


@pytest.mark.parametrize("geom", [(2, 8, 32, 4, 48, 2), (1, 4, 128, 16, 128, 1)])
def test_state_dict_is_the_baselines(pkg, geom):
    cfg = pkg.TransformerConfig(*geom, True)
    torch.manual_seed(1234)
    baseline = BaselineTransformer(cfg)
    torch.manual_seed(1234)
    optimized = pkg.UserOptimizedTransformer(cfg)
    assert list(baseline.state_dict().keys()) == list(optimized.state_dict().keys())
    # Same construction order => the same seeded nn.Linear initialisation.
    for (k, a), (_, b) in zip(baseline.state_dict().items(), optimized.state_dict().items()):
        assert torch.equal(a, b), k
    other = pkg.UserOptimizedTransformer(cfg)
    copy_model_weights(baseline, other)  # strict load_state_dict (TTB:1151-1161)
    for (k, a), (_, b) in zip(baseline.state_dict().items(), other.state_dict().items()):
        assert torch.equal(a, b), k


def test_forward_has_no_cpu_fallback(pkg):
    cfg = pkg.TransformerConfig(1, 4, 32, 4, 32, 1, True)
    model = pkg.UserOptimizedTransformer(cfg).eval()
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        model(torch.randn(1, 4, 32))


def test_toggles(pkg):
    model = pkg.UserOptimizedTransformer(pkg.TransformerConfig(1, 4, 32, 4, 32, 1, True))
    with pytest.raises(ValueError):
        model.enable_mixed_precision(torch.float32)
    model.enable_mixed_precision(torch.float16)
    with pytest.raises(RuntimeError, match="eval"):
        model.enable_kv_cache(True)           # still in training mode (TTB:412-413)
    model.eval().enable_kv_cache(True)
    assert model.kv_cache_length == 0
    model.enable_kv_cache(False)
    assert model.kv_cache_length == 0
    with pytest.raises(ValueError, match="causal"):
        pkg.UserOptimizedTransformer(pkg.TransformerConfig(1, 4, 32, 4, 32, 1, False)).eval().enable_kv_cache(True)
    assert model.shape_execution_plan.official_shape_id is None
    # The reference's main() toggles (TTB:1765-1770) are accepted.
    model.enable_triton_fused_norm(False)
    model.enable_triton_fused_ffn(False)
    model.enable_attention_fp16_accumulation(False)
    with pytest.raises(ValueError, match="causal"):
        model.enable_attention_fp16_accumulation(True)
    pkg.UserOptimizedTransformer(pkg.TransformerConfig(1, 4, 32, 4, 32, 1, False)).enable_attention_fp16_accumulation(True)


def test_tree_cache_follows_registrations(pkg):
    """The cached parameter / LayerNorm walk is redone after any parameter or module assignment."""
    model = pkg.UserOptimizedTransformer(pkg.TransformerConfig(2, 8, 128, 4, 128, 2, True)).eval()
    x = torch.empty(2, 8, 128)
    params, norms = model._tree()
    assert list(params) == list(model.parameters()) and len(norms) == 2 * 2 + 1
    assert model._tree()[0] is params                      # no registration: the same walk
    assert model._fused_stack_eligible() and not model._single_launch_forward(x, None)  # CPU input
    fresh = torch.nn.Parameter(torch.zeros(128, 128))
    model.layers[1].ffn_in.weight = fresh
    assert any(p is fresh for p in model._tree()[0])
    model.final_norm = torch.nn.LayerNorm(128, eps=1e-6)
    assert model._tree()[1][-1] is model.final_norm
    assert not model._fused_stack_eligible()               # eps outside the kernel's contract
    assert not model.execution_plan(2, 8).fused


def test_fused_eligibility_checks_every_layer_norm_on_each_call(pkg):
    """The whole-stack kernel needs eps 1e-5, a weight and a bias on every LayerNorm, re-read per call."""
    model = pkg.UserOptimizedTransformer(pkg.TransformerConfig(2, 8, 128, 4, 128, 2, True)).eval()
    assert model._fused_stack_eligible() and model.execution_plan(2, 8).fused
    model.layers[0].norm2.eps = 1e-6                       # a plain attribute: no registration hook fires
    assert not model._fused_stack_eligible() and not model.execution_plan(2, 8).fused
    model.layers[0].norm2.eps = 1e-5
    assert model._fused_stack_eligible() and model.execution_plan(2, 8).fused
    for replacement in (torch.nn.LayerNorm(128, elementwise_affine=False), torch.nn.LayerNorm(128, bias=False)):
        model.layers[1].norm1 = replacement                # weight or bias registered as None
        assert not model._fused_stack_eligible()
    model.layers[1].norm1 = torch.nn.LayerNorm(128)
    assert model._fused_stack_eligible()
    model.enable_fused_stack(False)
    assert not model._fused_stack_eligible() and not model.execution_plan(2, 8).fused


def test_product_never_touches_the_oracle():
    for path in (REPO / "gpu-kernel-for-transformer_amd").rglob("*.py"):
        text = path.read_text()
        assert not re.search(r"^\s*(from|import)\s+oracle", text, re.M), path


# ----------------------------------------------------------------------------- C-ABI
def _declared_symbols():
    header = (REPO / "include" / "xblock.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(xb_\w+)\s*\(", header, re.M)))


def test_library_exports_every_declared_symbol(capi):
    assert capi.XBLOCK_AVAILABLE, capi.XBLOCK_LOAD_ERROR
    declared = _declared_symbols()
    assert declared == sorted(capi.EXPORTED_SYMBOLS)
    handle = ctypes.CDLL(str(capi.LIBRARY_PATH))
    for name in declared:
        assert hasattr(handle, name), name
    assert capi.lib().xb_abi_version() == capi.XB_ABI_VERSION


SCRATCH_BYTES = 32 << 20   # XB_DECODE_SCRATCH_BYTES


def _check_noalloc_scratch_rule(lib):
    """The no-allocation decode's documented limit, from the library's own sizing.

    A decode chunk's partials (batch*heads*n_splits*16*(4*head_dim+8) bytes)
    fit the static scratch whenever one split per (batch, head) does, at any
    cache length; beyond that the call is refused (-9) before any launch.
    Only the refusals are called here: an accepted call would launch.
    """
    limits = {8: 52428, 16: 29127, 32: 15420, 64: 7943, 128: 4032, 256: 2032}
    for head_dim, limit in limits.items():
        assert limit == SCRATCH_BYTES // (16 * (4 * head_dim + 8))
        for bh in (1, 13, 16, 33, 48, 512, 2000, limit):
            for cached in (31, 4000, 100000):
                need = lib.xb_attention_kv_cache_workspace_bytes(bh, 1, 1, head_dim, cached)
                assert 0 < need <= SCRATCH_BYTES, (head_dim, bh, cached, need)
        for cached in (31, 100000):
            need = lib.xb_attention_kv_cache_workspace_bytes(limit + 1, 1, 1, head_dim, cached)
            assert need == (limit + 1) * 16 * (4 * head_dim + 8) > SCRATCH_BYTES
            assert lib.xb_attention_kv_cache_noalloc(16, 16, 16, 16, limit + 1, 1, 1, head_dim, cached,
                                                     cached + 1, 0.1, None) == -9
    # the long caches still split over many key ranges (a workspace call and
    # a no-allocation call share this geometry)
    assert lib.xb_attention_kv_cache_workspace_bytes(1, 1, 16, 256, 100000) > 100 * 16 * 16 * 1032


def test_argument_errors_need_no_gpu(capi):
    lib = capi.lib()
    assert lib.xb_linear(None, None, None, None, 4, 8, 8, 0, None) == -1
    assert lib.xb_linear(None, None, None, None, 0, 8, 8, 0, None) == 0   # empty: NULL allowed
    assert lib.xb_layernorm(None, None, None, None, 1, 0, 128, 1e-5, 0, None) == 0
    assert lib.xb_linear(16, 16, None, 16, 4, 7, 8, 0, None) == -4      # N % 8
    assert lib.xb_linear(16, 16, None, 16, 4, 8, 8, 9, None) == -6      # epilogue
    assert lib.xb_linear(18, 16, None, 16, 4, 8, 8, 0, None) == -5      # alignment
    assert lib.xb_linear(16, 16, None, 16, 0, 8, 8, 0, None) == 0       # empty: no launch
    assert lib.xb_layernorm(16, None, None, 16, 7, 4, 128, 1e-5, 0, None) == -3
    assert lib.xb_layernorm(16, None, None, 16, 1, -1, 128, 1e-5, 0, None) == -2
    assert lib.xb_layernorm(16, None, None, 16, 1, 4, 128, 1e-5, 1, None) == -1  # affine w/o gamma
    assert lib.xb_residual_layernorm(16, 16, 1, None, None, None, 16, 1, 0, 128, 1e-5, 0, None) == 0
    assert lib.xb_attention_causal(16, 16, 1, 8, 2, 24, 0.1, None) == -4  # head_dim 24
    assert lib.xb_attention_causal(16, 16, 0, 8, 2, 8, 0.1, None) == 0
    assert lib.xb_attention(16, 16, None, 1, 8, 2, 24, 0.1, 0, None) == -4   # head_dim 24
    assert lib.xb_attention(None, None, None, 1, 8, 2, 64, 0.1, 1, None) == -1
    assert lib.xb_attention(16, 16, None, 0, 8, 2, 64, 0.1, 0, None) == 0    # empty: no launch
    # KV cache: capacity, head_dim, workspace sizing without a GPU
    assert lib.xb_kv_cache_append(16, 16, 16, 1, 5, 2, 64, 10, 12, None) == -2   # 10 + 5 > 12
    assert lib.xb_kv_cache_append(16, 16, 16, 1, 5, 2, 24, 0, 12, None) == -4
    assert lib.xb_kv_cache_append(None, None, None, 1, 5, 2, 64, 0, 12, None) == -1
    assert lib.xb_attention_kv_cache_workspace_bytes(1, 17, 2, 64, 100) == 0     # long chunk: none needed
    assert lib.xb_attention_kv_cache_workspace_bytes(1, 1, 16, 64, 20000) == 7096320
    assert lib.xb_attention_kv_cache_workspace_bytes(1, 1, 2, 24, 100) == -4
    assert lib.xb_attention_kv_cache(16, 16, 16, 16, 1, 1, 2, 64, 100, 101, 0.1, None, 0, None) == -1
    assert lib.xb_attention_kv_cache(16, 16, 16, 16, 1, 1, 2, 64, 100, 101, 0.1, 16, 64, None) == -7
    # mask_mode outside UPDATE|SUM|OUTPUT, and a mask mode without row_valid
    assert lib.xb_residual_layernorm_masked(16, 16, 1, None, None, None, 16, 1, 4, 128, 1e-5, 0, 16, 8, None) == -6
    assert lib.xb_residual_layernorm_masked(16, 16, 1, None, None, None, 16, 1, 4, 128, 1e-5, 0, None, 2, None) == -1
    assert lib.xb_residual_layernorm_masked(16, 16, 1, None, None, None, 16, 1, 0, 128, 1e-5, 0, None, 7, None) == 0
    # Fused d128 stack: which shapes split over two workgroups, and the workspace checks.
    # Layout: 256-byte header (timeout counter, finished blocks, generation), 64-bit flags of
    # 128 sequences x layers, K/V slots from a 256-byte boundary.
    slot = 2 * 64 * 128 * 2
    head = lambda layers: (256 + 8 * 128 * layers + 255) // 256 * 256
    assert lib.xb_fused_forward_d128_workspace_bytes(64, 128, 4, 4, 1) == head(4) + 64 * 4 * slot
    assert lib.xb_fused_forward_d128_workspace_bytes(80, 65, 4, 2, 1) == head(2) + 80 * 2 * slot
    for heads in (2, 4, 8, 16):  # up to 128 sequences (one workgroup per CU) at every head_dim <= 64
        assert lib.xb_fused_forward_d128_workspace_bytes(128, 128, heads, 4, 1) == head(4) + 128 * 4 * slot
        assert lib.xb_fused_forward_d128_workspace_bytes(129, 128, heads, 4, 1) == 0
    assert lib.xb_fused_forward_d128_workspace_bytes(64, 64, 4, 4, 1) == 0     # no second half
    assert lib.xb_fused_forward_d128_workspace_bytes(64, 128, 4, 4, 0) == 0    # non-causal
    assert lib.xb_fused_forward_d128_workspace_bytes(64, 128, 1, 4, 1) == 0    # head_dim 128
    need = head(4) + 64 * 4 * slot
    ws_args = (16, 16, 16, 16, 64, 128, 4, 128, 4, -1, None, 1)
    assert lib.xb_fused_forward_d128_ws(*ws_args, 16, need - 1, -1, 0, None) == -7
    assert lib.xb_fused_forward_d128_ws(*ws_args, 24, need, -1, 0, None) == -5
    assert lib.xb_fused_forward_d128_ws(*ws_args, 16, need, -1, 4, None) == -6    # unknown fault flag
    assert lib.xb_fused_forward_d128_ws(16, 16, 16, 16, 64, 129, 4, 128, 4, -1, None, 1, 16, 1 << 30, -1, 0, None) == -4
    assert lib.xb_fused_forward_d128_ws(16, 16, 16, 16, 0, 128, 4, 128, 4, -1, None, 1, None, 0, -1, 0, None) == 0
    # No-allocation decode: a call whose partials exceed the static scratch is refused before any launch
    assert lib.xb_attention_kv_cache_noalloc(16, 16, 16, 16, 20000, 1, 16, 64, 100, 101, 0.1, None) == -9
    assert lib.xb_attention_kv_cache_noalloc(None, 16, 16, 16, 1, 1, 2, 64, 100, 101, 0.1, None) == -1
    assert lib.xb_attention_kv_cache_noalloc(16, 16, 16, 16, 1, 1, 2, 64, 100, 100, 0.1, None) == -2
    _check_noalloc_scratch_rule(lib)
    for code in (0, -1, -2, -3, -4, -5, -6, -7, -8, -9):
        assert lib.xb_strerror(code)
    with pytest.raises(RuntimeError, match="xb_linear failed with code -4"):
        capi.check(-4, "xb_linear")


def test_captured_overlap_is_described(pkg):
    """The plan of a small per-op forward names what its hipGraph capture runs
    (two half-batches, each with its own out / FFN GEMM tiles); one-kernel,
    large and single-sequence forwards run as planned."""
    shapes = pkg.OFFICIAL_BENCHMARK_SHAPES
    cfg3 = pkg.UserOptimizedTransformer(shapes[8])
    note = cfg3.captured_overlap(64, 128)
    assert note.startswith("two half-batch streams under capture (32 sequences: out mfma_gemm_dma_128x128")
    assert cfg3.captured_overlap(1, 128) is None                                  # nothing to split
    assert cfg3.captured_overlap(512, 128) is None                                # 65536 tokens: long kernels
    for shape_id in (1, 6, 11):                                                   # one-kernel whole-stack forwards
        c = shapes[shape_id]
        assert pkg.UserOptimizedTransformer(c).captured_overlap(c.batch_size, c.seq_len) is None
    odd = pkg.UserOptimizedTransformer(pkg.TransformerConfig(7, 64, 1024, 4, 1024, 1, True))
    assert "4 sequences" in odd.captured_overlap(7, 64, padded=True) and "3 sequences" in odd.captured_overlap(7, 64)
