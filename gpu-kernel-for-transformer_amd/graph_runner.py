"""hipGraph capture of the forward's kernel sequence, and the graph-or-eager choice.

The public names and contracts are the reference's (cuda_graph_runner.py:24-129),
since benchmark callers use them: `FixedInputCUDAGraph(model, x, mask)` replays
only for the captured input objects at their captured versions and returns a
copy of the static output; `maybe_cuda_graph(model, x, mask, enabled)` returns
(module, graphed, reason) and only graphs a forward whose replay was checked
bit for bit against an eager run.  On ROCm `torch.cuda.CUDAGraph` is a hipGraph.

How capture works here:
  * `CapturedCall` captures any zero-argument callable that enqueues work on
    the current stream.  It first runs the callable eagerly on a private
    stream: that fills every host-side cache the forward keeps (packed
    weights, mask inspection, LayerNorm affine checks), whose first fill may
    synchronise and so must not happen inside a capture.  The captured call
    then records nothing but xb_* kernel launches; the tensors they write are
    carved from the graph's private memory pool once, at capture, so every
    replay reuses the same preallocated buffers.
  * The capture owns a `kernels.SplitWorkspacePool`, bound to its private
    stream: a replay runs on whatever stream is current at replay time, so
    the hand-off workspace of the split whole-stack kernel must belong to the
    graph, not be shared with eager calls that might run beside a replay.
    `maybe_cuda_graph` also refuses a graph whose check run counted a failed
    hand-off (`kernels.split_handoff_failures`).
  * A forward that is a single kernel launch (the whole-stack d_model 128
    kernel; `UserOptimizedTransformer._single_launch_forward`) is not
    captured: its replay would be that same launch plus the copy of the
    static output.
"""

from __future__ import annotations

from typing import Callable, Optional, Tuple

import torch
import torch.nn as nn

from . import kernels


class CapturedCall:
    """One hipGraph of `fn()`'s launches, captured after `warmups` eager calls.

    `output` is what the captured call returned; `replay()` re-runs the
    kernels into it and returns it (the same tensor every time).
    """

    def __init__(self, fn: Callable[[], torch.Tensor], device: torch.device, warmups: int = 2) -> None:
        if warmups < 1:
            raise ValueError("at least one eager call must precede the capture")
        self.stream = torch.cuda.Stream(device=device)
        self.pool = kernels.SplitWorkspacePool(self.stream)
        self.graph = torch.cuda.CUDAGraph()
        caller = torch.cuda.current_stream(device)
        self.stream.wait_stream(caller)
        with self.pool, torch.cuda.stream(self.stream):
            for _ in range(warmups):
                fn()
            with torch.cuda.graph(self.graph, stream=self.stream):
                self.output = fn()
        caller.wait_stream(self.stream)

    def replay(self) -> torch.Tensor:
        self.graph.replay()
        return self.output


class _InputKey:
    """Identity and mutation version of a forward's (x, mask) pair."""

    __slots__ = ("x", "mask", "versions")

    def __init__(self, x: torch.Tensor, mask: Optional[torch.Tensor]) -> None:
        self.x, self.mask = x, mask
        self.versions = self._versions(x, mask)
        if None in self.versions:
            raise ValueError("graph inputs must expose mutation version counters (not inference tensors)")

    @staticmethod
    def _versions(x: torch.Tensor, mask: Optional[torch.Tensor]) -> Tuple[Optional[int], Optional[int]]:
        def version(t):
            if t is None:
                return -1
            try:
                return t._version
            except RuntimeError:
                return None

        return version(x), version(mask)

    def matches(self, x: torch.Tensor, mask: Optional[torch.Tensor]) -> bool:
        return x is self.x and mask is self.mask and self._versions(x, mask) == self.versions


class FixedInputCUDAGraph(nn.Module):
    """Replays the model's forward for one fixed (x, mask) pair (CGR:24-93).

    Any other input, or the same tensors after an in-place change, runs the
    model eagerly.  A replay returns a clone of the static output, so the
    caller's tensor is not overwritten by the next replay.
    """

    def __init__(self, model: nn.Module, example_x: torch.Tensor, example_mask: Optional[torch.Tensor],
                 warmup_iterations: int = 3) -> None:
        super().__init__()
        if not example_x.is_cuda or (example_mask is not None and not example_mask.is_cuda):
            raise ValueError("graph inputs must be GPU tensors")
        if model.training:
            raise ValueError("graph inference requires model.eval()")
        self.model = model
        self._key = _InputKey(example_x, example_mask)
        with torch.inference_mode():
            self._call = CapturedCall(lambda: model(example_x, example_mask), example_x.device,
                                      max(1, warmup_iterations))

    def replay(self) -> torch.Tensor:
        """Replay and return the static output buffer itself (no clone)."""
        return self._call.replay()

    def forward(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        if self._key.matches(x, valid_token_mask):
            return self._call.replay().clone()
        return self.model(x, valid_token_mask)


def _why_not_graphed(model: nn.Module, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor],
                     enabled: bool) -> Optional[str]:
    """The reason this forward stays eager, or None when it should be captured."""
    if not enabled:
        return "disabled"
    if not x.is_cuda:
        return "graphs require a GPU input"
    if bool(getattr(model, "_kv_cache_enabled", False)):
        return "stateful KV-cache decoding uses the eager path"
    if x.numel() == 0:
        return "empty input: nothing to launch"
    single_launch = getattr(model, "_single_launch_forward", None)
    if single_launch is not None and single_launch(x, valid_token_mask):
        return "one-kernel forward: launched eagerly (a replay adds only the output copy)"
    return None


def maybe_cuda_graph(model: nn.Module, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor],
                     enabled: bool) -> Tuple[nn.Module, bool, str]:
    """(module, graphed, reason): a checked fixed-input graph, or the model itself (CGR:96-129)."""
    if enabled and bool(getattr(model, "_uses_internal_cuda_graphs", False)):
        return model, True, str(getattr(model, "graph_status", "internal graph replay"))
    reason = _why_not_graphed(model, x, valid_token_mask, enabled)
    if reason is not None:
        return model, False, reason
    try:
        failures = kernels.split_handoff_failures(x.device)
        graphed = FixedInputCUDAGraph(model, x, valid_token_mask)
        with torch.inference_mode():
            eager = model(x, valid_token_mask)
            replayed = graphed(x, valid_token_mask)
        failures = kernels.split_handoff_failures(x.device) - failures
    except (RuntimeError, ValueError) as error:
        return model, False, f"capture failed: {error}"
    if failures:
        return model, False, (f"{failures} split-form K/V hand-off(s) failed during the capture check "
                              "(their rows are NaN); staying eager")
    if not torch.equal(eager, replayed):
        worst = float((eager.float() - replayed.float()).abs().max().item())
        return model, False, f"replay differs from the eager forward (max_abs={worst:.3g}); staying eager"
    return graphed, True, "fixed-input hipGraph replay of the xb_* kernel sequence"
