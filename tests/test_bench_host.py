"""Host logic of bench.py (no GPU): the long-sequence guards of the
reference's streamed_shape14.py (memory preflight SAFE_SKIP, SAFE_ABORT,
whole-output finiteness, streamed_shape14.py:167-169, :197-222), the
accuracy sample, the forward lower bound, and the kernel cost table."""

from __future__ import annotations

import pytest
import torch

import bench


def test_memory_preflight_skips_before_allocating(pkg):
    cfg5 = pkg.OFFICIAL_BENCHMARK_SHAPES[14]
    estimate = bench.device_estimate_bytes(pkg, cfg5)
    assert 50e9 < estimate < 200e9                    # fits one MI355X (288 GB) with room
    gib = 2**30
    assert bench.memory_preflight(estimate, 280 * gib, 288 * gib, 0.9) is None
    reason = bench.memory_preflight(estimate, 280 * gib, 288 * gib, 1e-3)   # forced by the fraction
    assert reason.startswith("SAFE_SKIP") and "no model or input was allocated" in reason
    assert bench.memory_preflight(estimate, 10 * gib, 288 * gib, 0.9).startswith("SAFE_SKIP")  # little free memory
    with pytest.raises(SystemExit):
        bench.parse_args(["--memory-fraction", "0"])
    assert bench.EXIT_SKIPPED == 3


def test_nonfinite_output_is_counted():
    out = torch.zeros(2, 5, 8)
    assert bench.nonfinite_count(out) == 0
    out[1, 3, 2] = float("nan")
    out[0, 0, 0] = float("inf")
    assert bench.nonfinite_count(out) == 2


def test_accuracy_rows_and_bounds(pkg):
    shapes = pkg.OFFICIAL_BENCHMARK_SHAPES
    assert bench.accuracy_rows(shapes[6], False) == list(range(10000))      # cfg2: whole batch
    assert bench.accuracy_rows(shapes[14], False) == [0, 16, 31]           # cfg5: first, middle, last
    assert bench.accuracy_rows(shapes[14], True) == list(range(32))
    # both are MFMA-bound against the fused lower bound (x read and y written once)
    bound, seconds = bench.forward_lower_bound(shapes[14], pkg.forward_flops(shapes[14]))
    assert bound == "mfma" and abs(seconds - pkg.forward_flops(shapes[14]) / bench.FP16_MFMA_FLOPS) < 1e-12
    bound2, _ = bench.forward_lower_bound(shapes[6], pkg.forward_flops(shapes[6]))
    assert bound2 == "mfma"


def test_kernel_costs_match_the_formulas(pkg):
    cfg3 = pkg.OFFICIAL_BENCHMARK_SHAPES[8]
    m = cfg3.batch_size * cfg3.seq_len
    by, fl = bench.kernel_costs("gemm_n3072_k1024", cfg3, m)
    assert fl == 2.0 * m * 3072 * 1024 and by == m * 2 * (3072 + 1024) + 2 * 3072 * 1024
    assert bench.kernel_costs("residual_layernorm_1024_final", cfg3, m)[0] == m * 10 * 1024
    cfg2 = pkg.OFFICIAL_BENCHMARK_SHAPES[6]
    m2 = cfg2.batch_size * cfg2.seq_len
    _, fused_flops = bench.kernel_costs("fused_forward_d128", cfg2, m2)
    assert fused_flops == pytest.approx(pkg.forward_flops(cfg2))
    assert bench.kernel_costs("kv_append_hd64", cfg2, m2) == (0.0, 0.0)


def test_trial_rows_follow_the_reference_trials(pkg):
    shapes = pkg.OFFICIAL_BENCHMARK_SHAPES
    for shape_id in (1, 8, 11):                       # small configs: every sequence of each trial
        assert bench.trial_rows(shapes[shape_id]) == list(range(shapes[shape_id].batch_size))
    rows = bench.trial_rows(shapes[6])                # cfg2: 1024 sequences from the start, middle and end
    assert len(rows) == 1024 and rows == sorted(set(rows)) and rows[0] == 0 and rows[-1] == 9999
    assert 5000 in rows
    assert bench.trial_rows(shapes[14]) == [0, 16, 31]
    args = bench.parse_args([])
    assert args.accuracy_trials == 5 and args.ref_repeats == 100 and args.ref_rounds == 3   # TTB:1618-1623
