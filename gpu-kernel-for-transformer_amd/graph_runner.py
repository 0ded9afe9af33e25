"""hipGraph capture and replay of a fixed-input forward.

Same contract as the reference's cuda_graph_runner.py:24-129 (the names are
kept for drop-in use; on ROCm `torch.cuda.CUDAGraph` captures a hipGraph):
  - capture after `warmup_iterations` eager calls on a side stream, so the
    mask and affine checks (the only host syncs) are cached before capture;
  - replay only when the input and mask are the captured objects at the
    captured `_version`, otherwise run eagerly;
  - return a clone of the static output (callers get independent tensors);
  - `maybe_cuda_graph` validates one replay bitwise against eager and falls
    back to eager on any capture error or mismatch.  A forward that is a
    single kernel launch (the whole-stack d_model 128 kernel) is not
    captured: its replay would be that one launch plus the output copy.
The kernels issue no hipMemsetAsync and allocate nothing themselves, so a
captured forward is a plain chain of kernel nodes.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn


def _tensor_version(tensor: Optional[torch.Tensor]) -> Optional[int]:
    if tensor is None:
        return -1
    try:
        return tensor._version
    except RuntimeError:
        return None


class FixedInputCUDAGraph(nn.Module):
    """Replay one eval-mode model for the exact captured input objects (CGR:24-93)."""

    def __init__(self, model: nn.Module, example_x: torch.Tensor, example_mask: Optional[torch.Tensor], warmup_iterations: int = 3) -> None:
        super().__init__()
        if not example_x.is_cuda or (example_mask is not None and not example_mask.is_cuda):
            raise ValueError("graph inputs must be GPU tensors")
        if model.training:
            raise ValueError("graph inference requires model.eval()")
        self.model = model
        self._captured_x = example_x
        self._captured_mask = example_mask
        self._captured_x_version = _tensor_version(example_x)
        self._captured_mask_version = _tensor_version(example_mask)
        if self._captured_x_version is None or self._captured_mask_version is None:
            raise ValueError("graph inputs must expose mutation version counters")
        device = example_x.device
        current = torch.cuda.current_stream(device)
        side = torch.cuda.Stream(device=device)
        side.wait_stream(current)
        with torch.inference_mode(), torch.cuda.stream(side):
            for _ in range(warmup_iterations):
                model(example_x, example_mask)
        current.wait_stream(side)
        torch.cuda.synchronize(device)
        self._graph = torch.cuda.CUDAGraph()
        with torch.inference_mode(), torch.cuda.graph(self._graph):
            self._captured_output = model(example_x, example_mask)
        torch.cuda.synchronize(device)

    def _matches_capture(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor]) -> bool:
        return (
            x is self._captured_x
            and valid_token_mask is self._captured_mask
            and _tensor_version(x) == self._captured_x_version
            and _tensor_version(valid_token_mask) == self._captured_mask_version
        )

    def replay(self) -> torch.Tensor:
        """Replay and return the static output buffer itself (no clone)."""
        self._graph.replay()
        return self._captured_output

    def forward(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        if not self._matches_capture(x, valid_token_mask):
            return self.model(x, valid_token_mask)
        self._graph.replay()
        return self._captured_output.clone()


def maybe_cuda_graph(model: nn.Module, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor], enabled: bool) -> Tuple[nn.Module, bool, str]:
    """Return a graphed model when capture and validation succeed (CGR:96-129)."""
    if not enabled:
        return model, False, "disabled"
    if not x.is_cuda:
        return model, False, "graphs require a GPU input"
    if bool(getattr(model, "_uses_internal_cuda_graphs", False)):
        return model, True, str(getattr(model, "graph_status", "internal graph replay"))
    if bool(getattr(model, "_kv_cache_enabled", False)):
        return model, False, "stateful KV-cache decoding uses the eager path"
    single_launch = getattr(model, "_single_launch_forward", None)
    if single_launch is not None and single_launch(x, valid_token_mask):
        return model, False, "one-kernel forward: launched eagerly (a replay adds only the output copy)"
    try:
        with torch.inference_mode():
            eager = model(x, valid_token_mask)
        wrapped = FixedInputCUDAGraph(model, x, valid_token_mask)
        with torch.inference_mode():
            replayed = wrapped(x, valid_token_mask)
    except (RuntimeError, ValueError) as error:
        return model, False, f"capture failed: {error}"
    if not torch.equal(eager, replayed):
        max_error = float((eager.float() - replayed.float()).abs().max().item())
        return model, False, f"replay validation failed (max_abs={max_error:.3g})"
    return wrapped, True, "fixed-input hipGraph replay"
