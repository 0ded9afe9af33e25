"""Graph capture and batch chunking on the GPU: FixedInputCUDAGraph,
maybe_cuda_graph and BatchChunkedTransformer (the reference's
cuda_graph_runner.py:24-129 and batch_chunk_runner.py:11-154 contracts).

Batch elements are independent (README.md:260-263), so every chunked or
replayed forward must equal the eager whole-batch forward bit for bit; the
official shape-6 configuration (chunk 1024 with per-chunk graphs,
torch_transformer_benchmark.py:1740, :1826-1846) is also checked against the
CPU oracle on slices."""

from __future__ import annotations

import pytest
import torch

from oracle.accuracy import compare_outputs
from oracle.baseline import BaselineTransformer, copy_model_weights

pytestmark = pytest.mark.gpu


def _models(pkg, config, device, seed=1234):
    torch.manual_seed(seed)
    baseline = BaselineTransformer(config).eval()
    optimized = pkg.UserOptimizedTransformer(config)
    copy_model_weights(baseline, optimized)
    return baseline, optimized.to(device).eval()


def _runners(pkg):
    graphs = __import__(pkg.__name__ + ".graph_runner", fromlist=["FixedInputCUDAGraph"])
    chunks = __import__(pkg.__name__ + ".batch_chunk_runner", fromlist=["BatchChunkedTransformer"])
    kernels = __import__(pkg.__name__ + ".kernels", fromlist=["fused_split_timeouts"])
    return graphs, chunks, kernels


@pytest.mark.parametrize("geom", [(2, 64, 256, 4, 512, 2), (16, 128, 128, 4, 128, 2), (3, 200, 1024, 16, 1024, 1),
                                  (1, 4128, 1024, 16, 1024, 1)])
def test_fixed_input_graph_replays_bitwise(pkg, cuda, geom):
    """Per-op, split whole-stack, D=1024 and long (transposed-V attention, its
    V^T buffer allocated inside the capture) forwards captured; replays with
    eager work (and eager forwards of the same model) between them equal
    eager; another input or an in-place change to the captured one runs
    eagerly."""
    graphs, _, kernels = _runners(pkg)
    config = pkg.TransformerConfig(*geom, True)
    _, optimized = _models(pkg, config, cuda)
    g = torch.Generator(device=cuda).manual_seed(5)
    x = torch.randn(config.batch_size, config.seq_len, config.d_model, generator=g, device=cuda)
    timeouts_before = kernels.fused_split_timeouts(cuda)  # earlier tests may force time-outs on purpose
    with torch.inference_mode():
        eager = optimized(x).clone()
    graphed = graphs.FixedInputCUDAGraph(optimized, x, None)
    with torch.inference_mode():
        for replay in range(3):
            out = graphed(x)
            torch.cuda.synchronize()
            assert torch.equal(out, eager), f"{geom} replay {replay}"
            assert torch.equal(optimized(x), eager)  # eager forward of the same model between replays
        other = torch.randn_like(x)
        assert torch.equal(graphed(other), optimized(other))
    x.mul_(2.0)  # the captured input changed in place: its version no longer matches
    with torch.inference_mode():
        assert torch.equal(graphed(x), optimized(x))
    assert graphed._call.pool.timeouts() == 0 and kernels.fused_split_timeouts(cuda) == timeouts_before


def test_maybe_cuda_graph_reasons(pkg, cuda):
    graphs, _, _ = _runners(pkg)
    single = pkg.TransformerConfig(4, 64, 128, 4, 128, 2, True)
    _, model = _models(pkg, single, cuda)
    x = torch.randn(4, 64, 128, device=cuda)
    assert graphs.maybe_cuda_graph(model, x, None, enabled=False)[1:] == (False, "disabled")
    runner, graphed, reason = graphs.maybe_cuda_graph(model, x, None, enabled=True)
    assert runner is model and not graphed and "one-kernel" in reason
    # the reference harness's all-True mask runs the unmasked one-kernel forward too
    all_valid = torch.ones(4, 64, dtype=torch.bool, device=cuda)
    runner, graphed, reason = graphs.maybe_cuda_graph(model, x, all_valid, enabled=True)
    assert runner is model and not graphed and "one-kernel" in reason
    with torch.inference_mode():
        assert torch.equal(model(x, all_valid), model(x))
    model.enable_kv_cache(True)
    assert "KV-cache" in graphs.maybe_cuda_graph(model, x, None, enabled=True)[2]
    model.enable_kv_cache(False)
    assert "GPU input" in graphs.maybe_cuda_graph(model, x.cpu(), None, enabled=True)[2]
    # with a padded mask the forward also converts the mask (two launches): captured
    mask = torch.ones(4, 64, dtype=torch.bool, device=cuda)
    mask[1, 50:] = False
    runner, graphed, reason = graphs.maybe_cuda_graph(model, x, mask, enabled=True)
    assert graphed and runner is not model, reason
    with torch.inference_mode():
        assert torch.equal(runner(x, mask), model(x, mask))


@pytest.mark.parametrize("geom,masked", [((5, 96, 256, 4, 512, 2), False), ((7, 64, 1024, 4, 1024, 1), True),
                                         ((2, 4096, 1024, 16, 1024, 1), False)])
def test_captured_per_op_forward_overlaps_half_batches(pkg, cuda, geom, masked):
    """A small per-op forward captured into a graph runs its two half-batches
    (odd batches: 3 + 2 and 4 + 3 sequences) on two side streams forked from
    the capturing stream; the replays equal the eager one-stream forward bit
    for bit, padded mask included, with eager forwards between them.  The
    side streams are made by the eager warm-up calls before the capture.
    The last geometry (8192 tokens of the long-sequence kind) checks the
    transposed-V attention inside the overlap."""
    graphs, _, _ = _runners(pkg)
    config = pkg.TransformerConfig(*geom, True)
    _, model = _models(pkg, config, cuda)
    g = torch.Generator(device=cuda).manual_seed(11)
    x = torch.randn(config.batch_size, config.seq_len, config.d_model, generator=g, device=cuda)
    mask = None
    if masked:
        mask = torch.ones(config.batch_size, config.seq_len, dtype=torch.bool, device=cuda)
        mask[1, 40:] = False
        mask[5, 3:] = False
    assert not model.execution_plan(config.batch_size, config.seq_len, padded=masked).fused
    with torch.inference_mode():
        eager = model(x, mask).clone()
    graphed = graphs.FixedInputCUDAGraph(model, x, mask)
    assert cuda.index in model.__dict__.get("_side_streams", {}), "the warm-up calls make the side streams"
    with torch.inference_mode():
        for replay in range(3):
            out = graphed(x, mask)
            torch.cuda.synchronize()
            assert torch.equal(out, eager), f"{geom} masked={masked} replay {replay}"
            assert torch.equal(model(x, mask), eager)


def test_maybe_cuda_graph_refuses_a_failed_handoff(pkg, cuda, monkeypatch):
    """A graph whose check run counted a failed split-form K/V hand-off (its
    rows would be NaN) is refused with the cause named, and the forward stays
    eager.  The failure count is faked from the host (a real failure is
    forced in test_fused_split_timeout_poisons_rows); every kernel runs
    normally."""
    graphs, _, kernels = _runners(pkg)
    config = pkg.TransformerConfig(2, 64, 256, 4, 512, 2, True)   # per-op forward: captured
    _, model = _models(pkg, config, cuda)
    x = torch.randn(2, 64, 256, device=cuda)
    counts = iter((0, 3))
    monkeypatch.setattr(kernels, "split_handoff_failures", lambda device=None: next(counts))
    runner, graphed, reason = graphs.maybe_cuda_graph(model, x, None, enabled=True)
    assert runner is model and not graphed
    assert "3 split-form K/V hand-off(s) failed" in reason


def test_batch_chunked_graphs_match_whole_batch(pkg, cuda):
    """Chunks of the split and one-workgroup whole-stack forms (one kernel each: launched
    eagerly into the output, no graph) and of a per-op geometry (per-chunk-shape graphs
    over static buffers, full chunk and remainder): bitwise equal to the whole-batch
    forward on two different inputs."""
    _, chunks, _ = _runners(pkg)
    for geom, chunk in (((45, 128, 128, 4, 128, 2), 16), ((300, 128, 128, 4, 128, 2), 128),
                        ((9, 96, 256, 4, 256, 2), 4)):
        config = pkg.TransformerConfig(*geom, True)
        _, optimized = _models(pkg, config, cuda)
        runner = chunks.BatchChunkedTransformer(optimized, chunk, all_tokens_valid=True, use_cuda_graphs=True)
        for seed in (1, 2):
            g = torch.Generator(device=cuda).manual_seed(seed)
            x = torch.randn(config.batch_size, config.seq_len, config.d_model, generator=g, device=cuda)
            with torch.inference_mode():
                whole = optimized(x)
                out = runner(x)
            torch.cuda.synchronize()
            assert torch.equal(out, whole), f"{geom} chunk {chunk} seed {seed}"
        if optimized.execution_plan(chunk, config.seq_len).fused:
            assert not runner._graphs, geom
            assert runner.graph_status.startswith("one-kernel chunk forwards: launched eagerly"), runner.graph_status
        else:
            expected_graphs = 1 + int(config.batch_size % chunk != 0)
            assert runner.graph_status == f"one hipGraph per chunk shape ({expected_graphs} captured)", runner.graph_status


def test_batch_chunked_padded_and_eager(pkg, cuda):
    """A padded mask is sliced per chunk and runs eagerly (graphs need all_tokens_valid)."""
    _, chunks, _ = _runners(pkg)
    config = pkg.TransformerConfig(20, 64, 128, 4, 128, 2, True)
    _, optimized = _models(pkg, config, cuda)
    x = torch.randn(20, 64, 128, device=cuda)
    mask = torch.rand(20, 64, device=cuda) > 0.3
    mask[:, 0] = True
    runner = chunks.BatchChunkedTransformer(optimized, 6, all_tokens_valid=False, use_cuda_graphs=True)
    assert not runner.use_cuda_graphs and runner.graph_status == "disabled"
    with torch.inference_mode():
        assert torch.equal(runner(x, mask), optimized(x, mask))


def test_forward_into_writes_the_given_buffer(pkg, cuda):
    """The chunk runner's direct path: _forward_into returns `out` itself, bitwise equal to
    forward, for a whole-stack, a per-op and a padded input; a wrong buffer is refused."""
    for geom in ((6, 128, 128, 4, 128, 2), (3, 96, 256, 4, 256, 2)):
        config = pkg.TransformerConfig(*geom, True)
        _, optimized = _models(pkg, config, cuda)
        x = torch.randn(config.batch_size, config.seq_len, config.d_model, device=cuda)
        mask = torch.ones(config.batch_size, config.seq_len, device=cuda, dtype=torch.bool)
        mask[1, config.seq_len // 2:] = False
        for m in (None, mask):
            out = torch.empty_like(x)
            with torch.inference_mode():
                got = optimized._forward_into(x, out, m)
                expected = optimized(x, m)
            assert got is out and torch.equal(out, expected), (geom, m is None)
        with pytest.raises(ValueError, match="out must be"):
            optimized._forward_into(x, torch.empty(x.shape, device=cuda, dtype=torch.float16))
        with pytest.raises(ValueError, match="out must be"):
            optimized._forward_into(x, torch.empty(x.shape[0] + 1, *x.shape[1:], device=cuda))


def test_shape6_chunk_1024_graphs_against_oracle(pkg, cuda):
    """The reference's shape-6 configuration: B=10000 in chunks of 1024 with graphs requested
    (each chunk is one whole-stack launch, so it writes its output slice eagerly), equal to
    the whole batch bitwise, and slices of it against the CPU oracle."""
    _, chunks, _ = _runners(pkg)
    config = pkg.OFFICIAL_BENCHMARK_SHAPES[6]
    baseline, optimized = _models(pkg, config, cuda)
    g = torch.Generator(device=cuda).manual_seed(1234)
    x = torch.randn(config.batch_size, config.seq_len, config.d_model, generator=g, device=cuda)
    runner = chunks.BatchChunkedTransformer(optimized, 1024, all_tokens_valid=True, use_cuda_graphs=True)
    with torch.inference_mode():
        out = runner(x)
        whole = optimized(x)
    assert torch.equal(out, whole)
    assert runner.graph_status.startswith("one-kernel chunk forwards"), runner.graph_status
    for start in (0, 9216, 9984):  # first chunk, the remainder chunk, its last rows
        rows = slice(start, start + 16)
        with torch.inference_mode():
            ref = baseline(x[rows].cpu())
        result = compare_outputs(ref, out[rows].cpu())
        print(f"shape 6 chunk-1024 graphs rows {start}..{start + 15}: {result.summary()}", flush=True)
        assert result.passed, result.summary()


def test_memory_budget_chunking(pkg, cuda):
    """chunk_size_for_memory sizes slices from a byte budget; the model's own chunk loop
    (the plan's batch_chunk_size, or _large_batch_chunk_size) is bitwise equal to one pass."""
    _, chunks, _ = _runners(pkg)
    config = pkg.TransformerConfig(6, 300, 256, 4, 512, 2, True)
    _, optimized = _models(pkg, config, cuda)
    x = torch.randn(6, 300, 256, device=cuda)
    per_seq = optimized.activation_bytes(1, 300)
    assert chunks.chunk_size_for_memory(optimized, x, budget_bytes=int(2.5 * per_seq)) == 2
    assert chunks.chunk_size_for_memory(optimized, x, budget_bytes=100 * per_seq) == 6
    assert chunks.chunk_size_for_memory(optimized, x, budget_bytes=1) == 1
    with torch.inference_mode():
        whole = optimized(x)
        optimized._large_batch_chunk_size = chunks.chunk_size_for_memory(optimized, x, budget_bytes=int(2.5 * per_seq))
        sliced = optimized(x)
        optimized._large_batch_chunk_size = 0
    assert torch.equal(whole, sliced)
