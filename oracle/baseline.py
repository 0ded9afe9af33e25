"""TEST INFRASTRUCTURE ONLY: restated BaselineTransformer (FP32, CPU) and harness helpers.

Restates, op for op and in the same order:
  BaselineSelfAttention      torch_transformer_benchmark.py:204-267
  BaselineTransformerBlock   torch_transformer_benchmark.py:270-290
  BaselineTransformer        torch_transformer_benchmark.py:293-317
  copy_model_weights         torch_transformer_benchmark.py:1151-1161
  generate_random_case       torch_transformer_benchmark.py:1182-1220
The module tree (and so the state_dict keys and the order in which nn.Linear
draws its initialisation from the global RNG) is the reference's.
"""

from __future__ import annotations

import copy
from typing import Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F


class BaselineSelfAttention(nn.Module):
    """Explicit multi-head self-attention (torch_transformer_benchmark.py:204-267)."""

    def __init__(self, d_model: int, num_heads: int) -> None:
        super().__init__()
        if d_model % num_heads != 0:
            raise ValueError("d_model must be divisible by num_heads")
        self.d_model = d_model
        self.num_heads = num_heads
        self.head_dim = d_model // num_heads
        self.scale = self.head_dim**-0.5
        self.q_proj = nn.Linear(d_model, d_model, bias=True)
        self.k_proj = nn.Linear(d_model, d_model, bias=True)
        self.v_proj = nn.Linear(d_model, d_model, bias=True)
        self.out_proj = nn.Linear(d_model, d_model, bias=True)

    def _heads(self, t: torch.Tensor) -> torch.Tensor:
        b, s, _ = t.shape
        return t.view(b, s, self.num_heads, self.head_dim).transpose(1, 2).contiguous()

    def forward(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor] = None, causal: bool = False) -> torch.Tensor:
        b, s, _ = x.shape
        q = self._heads(self.q_proj(x))
        k = self._heads(self.k_proj(x))
        v = self._heads(self.v_proj(x))
        scores = torch.matmul(q, k.transpose(-2, -1)) * self.scale
        if causal:
            upper = torch.ones((s, s), device=x.device, dtype=torch.bool).triu(diagonal=1)
            scores = scores.masked_fill(upper, float("-inf"))
        if valid_token_mask is not None:
            scores = scores.masked_fill(~valid_token_mask[:, None, None, :], float("-inf"))
        probs = torch.softmax(scores.float(), dim=-1).to(dtype=x.dtype)
        context = torch.matmul(probs, v).transpose(1, 2).contiguous().view(b, s, self.d_model)
        output = self.out_proj(context)
        if valid_token_mask is not None:
            output = output.masked_fill(~valid_token_mask[..., None], 0)
        return output


class BaselineTransformerBlock(nn.Module):
    """Pre-norm block: x + attn(LN1 x); x + ffn_out(gelu_erf(ffn_in(LN2 x))) (TTB:270-290)."""

    def __init__(self, d_model: int, num_heads: int, ffn_dim: int) -> None:
        super().__init__()
        self.norm1 = nn.LayerNorm(d_model)
        self.attention = BaselineSelfAttention(d_model, num_heads)
        self.norm2 = nn.LayerNorm(d_model)
        self.ffn_in = nn.Linear(d_model, ffn_dim)
        self.ffn_out = nn.Linear(ffn_dim, d_model)

    def forward(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor], causal: bool) -> torch.Tensor:
        x = x + self.attention(self.norm1(x), valid_token_mask, causal)
        x = x + self.ffn_out(F.gelu(self.ffn_in(self.norm2(x)), approximate="none"))
        if valid_token_mask is not None:
            x = x.masked_fill(~valid_token_mask[..., None], 0)
        return x


class BaselineTransformer(nn.Module):
    """Stack of blocks plus final LayerNorm (torch_transformer_benchmark.py:293-317)."""

    def __init__(self, config) -> None:
        super().__init__()
        self.config = config
        self.layers = nn.ModuleList(
            [BaselineTransformerBlock(config.d_model, config.num_heads, config.ffn_dim) for _ in range(config.num_layers)]
        )
        self.final_norm = nn.LayerNorm(config.d_model)

    def forward(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        for layer in self.layers:
            x = layer(x, valid_token_mask, self.config.causal)
        x = self.final_norm(x)
        if valid_token_mask is not None:
            x = x.masked_fill(~valid_token_mask[..., None], 0)
        return x


def copy_model_weights(baseline: nn.Module, optimized: nn.Module, strict: bool = True) -> None:
    """Strict state_dict copy into the optimized model (TTB:1151-1161)."""
    state_dict = copy.deepcopy(baseline.state_dict())
    incompatible = optimized.load_state_dict(state_dict, strict=strict)
    if not strict and (incompatible.missing_keys or incompatible.unexpected_keys):
        print(f"[warning] weight copy: missing={incompatible.missing_keys} unexpected={incompatible.unexpected_keys}")


def generate_random_case(
    config,
    device: torch.device,
    dtype: torch.dtype,
    seed: int,
    padding_ratio: float = 0.0,
    input_scale: float = 1.0,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Seeded x ~ N(0,1)*scale and validity mask (torch_transformer_benchmark.py:1182-1220)."""
    generator = torch.Generator(device=device)
    generator.manual_seed(seed)
    x = torch.randn(config.batch_size, config.seq_len, config.d_model, generator=generator, device=device, dtype=dtype)
    x = x * input_scale
    if padding_ratio <= 0:
        return x, torch.ones(config.batch_size, config.seq_len, device=device, dtype=torch.bool)
    min_valid = max(1, int(round(config.seq_len * (1.0 - padding_ratio))))
    lengths = torch.randint(low=min_valid, high=config.seq_len + 1, size=(config.batch_size,), generator=generator, device=device)
    positions = torch.arange(config.seq_len, device=device)[None, :]
    mask = positions < lengths[:, None]
    x = x.masked_fill(~mask[..., None], 0)
    return x, mask


def build_models(config, seed: int = 1234):
    """Seed the global RNG and construct the CPU FP32 baseline in eval mode (TTB:1724-1731).

    Callers copy its weights into the optimized model with `copy_model_weights`.
    """
    torch.manual_seed(seed)
    return BaselineTransformer(config).eval()
