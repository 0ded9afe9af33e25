"""TEST INFRASTRUCTURE ONLY: the reference's elementwise accuracy rule.

Restates AccuracyResult / compare_outputs (torch_transformer_benchmark.py:1223-1304):
an element passes iff both values are finite and
    |opt - ref| <= atol   OR   |opt - ref| <= rtol * |ref|
(not torch.isclose, whose atol + rtol*|ref| is more permissive).  Both tensors
are compared in FP32; the relative-error summary clamps |ref| at 1e-12.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List, Tuple

import torch

RTOL = 0.02
ATOL = 0.002


@dataclass
class AccuracyResult:
    passed: bool
    total_elements: int
    failed_elements: int
    max_abs_error: float
    max_relative_error: float
    mean_abs_error: float
    failed_feature_dims: List[int]
    worst_index: Tuple[int, ...]
    reference_at_worst: float
    optimized_at_worst: float

    def summary(self) -> str:
        return (
            f"{'PASS' if self.passed else 'FAIL'} | max_abs={self.max_abs_error:.6g} | "
            f"max_rel={self.max_relative_error:.6g} | failed={self.failed_elements}/{self.total_elements}"
        )


def compare_outputs(reference: torch.Tensor, optimized: torch.Tensor, rtol: float = RTOL, atol: float = ATOL) -> AccuracyResult:
    if reference.shape != optimized.shape:
        raise AssertionError(f"shape mismatch: baseline={tuple(reference.shape)}, optimized={tuple(optimized.shape)}")
    ref = reference.detach().float().cpu()
    opt = optimized.detach().float().cpu()
    finite = torch.isfinite(ref) & torch.isfinite(opt)
    abs_error = (opt - ref).abs()
    passed_mask = finite & ((abs_error <= atol) | (abs_error <= rtol * ref.abs()))
    failed_mask = ~passed_mask
    failed = int(failed_mask.sum().item())
    total = reference.numel()

    flat_worst = int(abs_error.reshape(-1).argmax().item()) if total else 0
    worst = []
    remaining = flat_worst
    for size in reversed(reference.shape):
        worst.append(remaining % size)
        remaining //= size
    worst_index = tuple(reversed(worst))
    relative = abs_error / ref.abs().clamp_min(1e-12)

    if reference.ndim == 0:
        dims = [0] if failed else []
    elif reference.ndim == 1:
        dims = torch.nonzero(failed_mask, as_tuple=False).flatten().tolist()
    else:
        dims = torch.nonzero(failed_mask.any(dim=tuple(range(reference.ndim - 1))), as_tuple=False).flatten().tolist()

    return AccuracyResult(
        passed=failed == 0,
        total_elements=total,
        failed_elements=failed,
        max_abs_error=float(abs_error.max().item()) if total else 0.0,
        max_relative_error=float(relative.max().item()) if total else 0.0,
        mean_abs_error=float(abs_error.mean().item()) if total else 0.0,
        failed_feature_dims=dims,
        worst_index=worst_index,
        reference_at_worst=float(ref[worst_index].item()) if total else 0.0,
        optimized_at_worst=float(opt[worst_index].item()) if total else 0.0,
    )
