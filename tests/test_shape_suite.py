"""Host logic of benchmark_shape_suite.py (no GPU): case grammar, memory
preflight, statuses, summary and exit codes, with the per-case process
replaced by a scripted launcher."""

from __future__ import annotations

import json

import pytest

import benchmark_shape_suite as suite

SHAPES = list(range(1, 15))
CONFIGS = (1, 6, 8, 11, 14)


def test_parse_case_ids_grammar():
    assert suite.parse_case_ids("all", SHAPES, CONFIGS) == SHAPES
    assert suite.parse_case_ids("configs", SHAPES, CONFIGS) == [1, 6, 8, 11, 14]
    assert suite.parse_case_ids("1-3, 12,2", SHAPES, CONFIGS) == [1, 2, 3, 12]
    with pytest.raises(ValueError, match="empty value"):
        suite.parse_case_ids("1,,2", SHAPES, CONFIGS)
    with pytest.raises(ValueError, match="descending"):
        suite.parse_case_ids("5-3", SHAPES, CONFIGS)
    with pytest.raises(ValueError, match=r"unknown benchmark shape IDs: \[15\]"):
        suite.parse_case_ids("14-15", SHAPES, CONFIGS)


def test_peak_estimate_scales_with_tokens(pkg):
    shapes = pkg.OFFICIAL_BENCHMARK_SHAPES
    cfg5 = shapes[14]
    full = suite.estimated_peak_bytes(cfg5)
    one = suite.estimated_peak_bytes(cfg5, batch=1)
    assert full > 30 * one / 1.01 and full < 33 * one
    # every official shape fits in 80% of one MI355X's 288 GB
    assert max(suite.estimated_peak_bytes(c) for c in shapes.values()) < 0.8 * 288e9


def _line(value=1e6, failed=0, passed=True):
    return json.dumps({"value": value, "ms_per_step": 1.5,
                       "roofline": {"kernel": "fused_forward_d128", "bound": "hbm", "frac": 0.25},
                       "forward_roofline": {"bound": "mfma", "frac": 0.04},
                       "accuracy": {"failed": failed, "total": 100, "passed": passed, "trials": 2},
                       "cpu_baseline": {"value": 1e3}})


class ScriptedLauncher:
    def __init__(self, outcomes):
        self.outcomes = outcomes
        self.commands = []

    def __call__(self, command, timeout):
        self.commands.append(command)
        shape_id = int(command[command.index("--workload") + 1])
        return self.outcomes[shape_id]


def test_statuses_summary_and_exit_codes(pkg):
    args = suite.parse_args(["--cases", "1,2,6,8,14", "--shape14-samples", "4", "--quick"])
    shapes = dict(pkg.OFFICIAL_BENCHMARK_SHAPES)
    launcher = ScriptedLauncher({
        1: (0, "log line\n" + _line()),
        2: (2, _line(failed=3, passed=False)),      # accuracy failure exits 2
        6: (124, ""),                               # killed at the time limit
        14: (0, _line(value=5e5)),
    })
    results = suite.run_suite([1, 2, 6, 14], shapes, args, None, launcher)
    # a device too small for shape 8 (estimate above 80% of it): skipped, never launched
    device_bytes = int(suite.estimated_peak_bytes(shapes[8]) / 0.8) - 1
    results += suite.run_suite([8], shapes, args, device_bytes, launcher)
    forced = suite.parse_args(["--quick", "--force-oversized"])
    launcher.outcomes[8] = (0, _line())
    assert suite.run_suite([8], shapes, forced, device_bytes, launcher)[0].status == "PASS"
    launcher.commands.pop()
    by_id = {r.shape_id: r for r in results}
    assert by_id[1].status == "PASS" and by_id[1].tokens_per_s == 1e6 and by_id[1].accuracy_trials == 2
    assert by_id[2].status == "FAIL" and by_id[2].reason == "accuracy check failed"
    assert by_id[6].status == "FAIL" and "timed out" in by_id[6].reason
    assert by_id[8].status == "SKIP"
    assert by_id[14].status == "PROXY" and "4/32" in by_id[14].reason
    assert 8 not in [int(c[c.index("--workload") + 1]) for c in launcher.commands]
    cmd14 = launcher.commands[3]
    assert cmd14[cmd14.index("--batch") + 1] == "4" and "--strict-accuracy" in cmd14
    # bench.py's own guard (SAFE_SKIP / SAFE_ABORT, status 3) is a SKIP with its reason
    launcher.outcomes[11] = (3, "SAFE_ABORT: out of device memory: HIP out of memory\n")
    skipped = suite.run_suite([11], shapes, args, None, launcher)[0]
    assert skipped.status == "SKIP" and skipped.reason.startswith("SAFE_ABORT")
    launcher.commands.pop()
    assert suite.exit_status(results, strict=False) == 1
    ok = [by_id[1], by_id[14]]
    assert suite.exit_status(ok, strict=False) == 0
    assert suite.exit_status(ok, strict=True) == 1          # PROXY counts as incomplete
    text = "\n".join(suite.summary_lines(results))
    assert "geometric-mean roofline fraction across completed cases: 25.0%" in text
    assert "geometric-mean fraction of the fused lower bound: 4.0%" in text
    assert "SKIP" in text and "PROXY" in text


def test_argument_validation():
    with pytest.raises(SystemExit):
        suite.parse_args(["--memory-fraction", "0"])
    with pytest.raises(SystemExit):
        suite.parse_args(["--shape14-samples", "33"])
    with pytest.raises(SystemExit):
        suite.parse_args(["--device", "cpu"])
    args = suite.parse_args([])
    assert args.cases == "configs" and args.accuracy_trials == 5 and args.benchmark_rounds == 3
