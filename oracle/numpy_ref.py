"""TEST INFRASTRUCTURE ONLY: float64 NumPy brute force of the causal pre-norm forward.

Written from the formulas, independently of torch's modules, to pin the torch
restatement in baseline.py on tiny inputs:
  LayerNorm   y = (x - mean) / sqrt(var_biased + eps) * gamma + beta
  attention   per (batch, head, query): softmax over keys j <= i (causal) of
              q.k * head_dim**-0.5, explicit Python loops over queries
  GELU        0.5 * x * (1 + erf(x / sqrt 2)) via math.erf
  block       x += out_proj(attn(LN1 x));  x += W2 gelu(W1 LN2 x + b1) + b2
The step order is the reference's (torch_transformer_benchmark.py:230-317).
Only meant for B, S, D in the tens.
"""

from __future__ import annotations

import math
from typing import Dict

import numpy as np


def layer_norm(x: np.ndarray, gamma: np.ndarray, beta: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    mean = x.mean(axis=-1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=-1, keepdims=True)
    return (x - mean) / np.sqrt(var + eps) * gamma + beta


def gelu_erf(x: np.ndarray) -> np.ndarray:
    erf = np.vectorize(math.erf, otypes=[np.float64])
    return 0.5 * x * (1.0 + erf(x / math.sqrt(2.0)))


def linear(x: np.ndarray, weight: np.ndarray, bias: np.ndarray) -> np.ndarray:
    return x @ weight.T + bias


def causal_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, num_heads: int, causal: bool = True) -> np.ndarray:
    """q, k, v: [B, S, D] -> context [B, S, D], heads are contiguous D/H column groups."""
    batch, seq, d_model = q.shape
    hd = d_model // num_heads
    scale = hd**-0.5
    out = np.zeros_like(q)
    for b in range(batch):
        for h in range(num_heads):
            cols = slice(h * hd, (h + 1) * hd)
            for i in range(seq):
                last = i + 1 if causal else seq
                scores = np.array([float(np.dot(q[b, i, cols], k[b, j, cols])) * scale for j in range(last)])
                weights = np.exp(scores - scores.max())
                weights /= weights.sum()
                out[b, i, cols] = weights @ v[b, :last, cols]
    return out


def forward(state: Dict[str, np.ndarray], x: np.ndarray, num_layers: int, num_heads: int, causal: bool = True, eps: float = 1e-5) -> np.ndarray:
    """Forward of the whole stack from a state_dict converted to float64 arrays."""
    x = x.astype(np.float64)
    for i in range(num_layers):
        p = lambda name: state[f"layers.{i}.{name}"]  # noqa: E731
        n1 = layer_norm(x, p("norm1.weight"), p("norm1.bias"), eps)
        q = linear(n1, p("attention.q_proj.weight"), p("attention.q_proj.bias"))
        k = linear(n1, p("attention.k_proj.weight"), p("attention.k_proj.bias"))
        v = linear(n1, p("attention.v_proj.weight"), p("attention.v_proj.bias"))
        ctx = causal_attention(q, k, v, num_heads, causal)
        x = x + linear(ctx, p("attention.out_proj.weight"), p("attention.out_proj.bias"))
        n2 = layer_norm(x, p("norm2.weight"), p("norm2.bias"), eps)
        hidden = gelu_erf(linear(n2, p("ffn_in.weight"), p("ffn_in.bias")))
        x = x + linear(hidden, p("ffn_out.weight"), p("ffn_out.bias"))
    return layer_norm(x, state["final_norm.weight"], state["final_norm.bias"], eps)


def state_to_numpy(state_dict) -> Dict[str, np.ndarray]:
    return {k: v.detach().cpu().double().numpy() for k, v in state_dict.items()}
