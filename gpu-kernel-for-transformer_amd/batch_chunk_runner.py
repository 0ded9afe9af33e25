"""Exact batch slicing, optionally with one hipGraph per chunk shape.

Public name and constructor are the reference's `BatchChunkedTransformer`
(batch_chunk_runner.py:49-154, used for official shape 6 at chunk 1024,
torch_transformer_benchmark.py:1740, :1826-1846).  Batch elements are
independent (README.md:260-263), so the output equals the whole-batch
forward bit for bit.

Design:
  * Graphs (use_cuda_graphs, only for inputs whose mask is all True, as the
    caller asserts with all_tokens_valid) are keyed by the chunk's batch size:
    one for the full chunk, one for the remainder.  Each `_ChunkShapeGraph`
    owns a static input buffer of its shape and a `graph_runner.CapturedCall`
    of the model over it; a chunk is copied into the static input (device to
    device), the graph replayed, and the static output copied into the
    caller's output slice.  The copies are part of the contract: the captured
    kernels have their buffer addresses baked in, and callers pass a new
    input tensor on every call.
  * A chunk whose forward is one kernel (the whole-stack kernel,
    `UserOptimizedTransformer._single_launch_forward`) is not captured, as in
    `graph_runner.maybe_cuda_graph`: a replay would add only the two copies
    (at official shape 6, 1024-sequence chunks, 2.27 against 1.77 ms per
    batch on one MI355X).  It is launched eagerly and writes its slice of the
    output directly.
  * Without graphs each chunk is one eager forward written straight into the
    output slice (the model's `_forward_into`; a model without it returns
    its own output, which is copied).
  * `chunk_size_for_memory` sizes a chunk from a byte budget (default: a
    fraction of the GPU's free memory) with the model's own working-set
    estimate; one MI355X (288 GB) holds every official batch whole, so the
    model's execution plan only chunks batches beyond that.
"""

from __future__ import annotations

from typing import Dict, Optional

import torch
import torch.nn as nn

from .graph_runner import CapturedCall


class _ChunkShapeGraph:
    """A captured forward over a static [chunk, S, D] input buffer."""

    def __init__(self, model: nn.Module, like: torch.Tensor) -> None:
        self.static_input = like.detach().clone()
        with torch.inference_mode():
            self.call = CapturedCall(lambda: model(self.static_input, None), like.device)

    def run_into(self, chunk: torch.Tensor, destination: torch.Tensor) -> None:
        self.static_input.copy_(chunk)
        destination.copy_(self.call.replay())


def chunk_size_for_memory(model: nn.Module, x: torch.Tensor, budget_bytes: Optional[int] = None) -> int:
    """Largest batch slice whose forward working set fits `budget_bytes`.

    The default budget is 80% of the device's free memory.  Returns the
    whole batch when it fits, and at least 1.
    """
    per_sequence = model.activation_bytes(1, x.shape[1])
    if budget_bytes is None:
        free, _total = torch.cuda.mem_get_info(x.device)
        budget_bytes = int(0.8 * free)
    return max(1, min(x.shape[0], int(budget_bytes // max(1, per_sequence))))


class BatchChunkedTransformer(nn.Module):
    """Runs `model` over batch slices of `chunk_size` (BCR:49-154)."""

    def __init__(self, model: nn.Module, chunk_size: int, *, all_tokens_valid: bool, use_cuda_graphs: bool) -> None:
        super().__init__()
        if chunk_size <= 0:
            raise ValueError("chunk_size must be positive")
        if model.training:
            raise ValueError("batch chunking requires model.eval()")
        self.model = model
        self.chunk_size = int(chunk_size)
        self.all_tokens_valid = bool(all_tokens_valid)
        # Graph replays assume the mask the capture saw; only an all-valid batch qualifies.
        self.use_cuda_graphs = bool(use_cuda_graphs) and self.all_tokens_valid and torch.cuda.is_available()
        self._uses_internal_cuda_graphs = self.use_cuda_graphs
        self._graphs: Dict[tuple, _ChunkShapeGraph] = {}
        self._graph_errors: Dict[tuple, str] = {}
        self._one_launch_shapes: set = set()  # chunk batch sizes launched eagerly instead of captured
        self.eval()

    @property
    def graph_status(self) -> str:
        if not self.use_cuda_graphs:
            return "disabled"
        if self._graph_errors:
            failed = ", ".join(f"chunk {key[0]}: {err}" for key, err in sorted(self._graph_errors.items()))
            return f"eager for chunk shapes whose capture failed ({failed})"
        if self._one_launch_shapes and not self._graphs:
            return "one-kernel chunk forwards: launched eagerly into the output (a replay adds only the copies)"
        status = f"one hipGraph per chunk shape ({len(self._graphs)} captured)"
        if self._one_launch_shapes:
            status += "; one-kernel chunk shapes launched eagerly into the output"
        return status

    def _one_launch(self, chunk: torch.Tensor) -> bool:
        """Whether the chunk's forward is one kernel the model can write into an output slice."""
        probe = getattr(self.model, "_single_launch_forward", None)
        if probe is None or not hasattr(self.model, "_forward_into") or not probe(chunk, None):
            return False
        self._one_launch_shapes.add(chunk.shape[0])
        return True

    def _graph_for(self, chunk: torch.Tensor) -> Optional[_ChunkShapeGraph]:
        key = (chunk.shape[0], tuple(chunk.shape[1:]), chunk.dtype, chunk.device)
        if key in self._graph_errors:
            return None
        graph = self._graphs.get(key)
        if graph is None:
            try:
                graph = _ChunkShapeGraph(self.model, chunk)
            except (RuntimeError, ValueError) as error:
                self._graph_errors[key] = str(error)
                return None
            self._graphs[key] = graph
        return graph

    def forward(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        if x.ndim != 3:
            raise ValueError("batch-chunked Transformer input must be [B, S, D]")
        mask = None if self.all_tokens_valid else valid_token_mask
        output = torch.empty_like(x)
        write_into = getattr(self.model, "_forward_into", None)
        for start in range(0, x.shape[0], self.chunk_size):
            end = min(start + self.chunk_size, x.shape[0])
            chunk = x[start:end]
            chunk_mask = None if mask is None else mask[start:end]
            graph = None
            if self.use_cuda_graphs and chunk.numel() and not self._one_launch(chunk):
                graph = self._graph_for(chunk)
            if graph is not None:
                graph.run_into(chunk, output[start:end])
            elif write_into is not None:
                write_into(chunk, output[start:end], chunk_mask)
            else:
                output[start:end].copy_(self.model(chunk, chunk_mask))
        return output
