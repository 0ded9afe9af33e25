"""xb_attention_kv_cache_noalloc: the decode attention with its split partials
in the library's static per-GPU scratch, against xb_attention_kv_cache with a
caller workspace (the same kernels, so bit-for-bit equal), on two calls in a
row, the second with a smaller input.  Both go through the C-ABI (ctypes)."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def _decode_case(kernels, cuda, batch, heads, head_dim, start, capacity, seed):
    g = torch.Generator(device=cuda).manual_seed(seed)
    d = heads * head_dim
    prompt = torch.randn(batch, start, 3 * d, generator=g, device=cuda).half()
    step = torch.randn(batch, 1, 3 * d, generator=g, device=cuda).half()
    k_cache = torch.zeros(batch, heads, capacity, head_dim, device=cuda, dtype=torch.float16)
    v_cache = torch.zeros_like(k_cache)
    kernels.kv_cache_append(prompt, k_cache, v_cache, heads, 0)
    kernels.kv_cache_append(step, k_cache, v_cache, heads, start)
    return step, k_cache, v_cache


@pytest.mark.parametrize("head_dim", [64, 256])
def test_noalloc_decode_matches_workspace_call(pkg, cuda, head_dim):
    kernels = __import__(pkg.__name__ + ".kernels", fromlist=["attention_kv_cache"])
    heads = 1024 // head_dim
    # (batch, cached tokens): the second call is smaller than the first
    for call, (batch, start) in enumerate(((4, 4000), (2, 1000))):
        step, k_cache, v_cache = _decode_case(kernels, cuda, batch, heads, head_dim, start, start + 8, 500 + call)
        need = kernels.kv_cache_workspace_bytes(batch, 1, heads, head_dim, start)
        assert 0 < need <= 32 << 20
        with torch.inference_mode():
            ref = kernels.attention_kv_cache(step, k_cache, v_cache, heads, start)
            out = torch.full_like(ref, float("nan"))
            got = kernels.attention_kv_cache(step, k_cache, v_cache, heads, start, out=out, no_alloc=True)
            torch.cuda.synchronize()
        assert got is out
        print(f"no-alloc decode hd={head_dim} call {call}: B={batch} S_k={start + 1}, "
              f"max diff {(got.float() - ref.float()).abs().max().item()}", flush=True)
        assert torch.equal(got, ref), f"call {call}: no-alloc output differs from the workspace call"
