"""The shape-suite runner end to end on the GPU: two small official shapes,
each in its own bench.py process, must PASS with their accuracy checked."""

from __future__ import annotations

import json

import pytest

import benchmark_shape_suite as suite

pytestmark = pytest.mark.gpu


def test_suite_runs_cases_in_isolated_processes(tmp_path, cuda):
    out = tmp_path / "suite.json"
    status = suite.main(["--cases", "2,12", "--quick", "--cpu-seconds", "1", "--case-timeout", "300",
                         "--json", str(out)])
    payload = json.loads(out.read_text())
    cases = {c["shape_id"]: c for c in payload["cases"]}
    for shape_id in (2, 12):
        case = cases[shape_id]
        assert case["status"] == "PASS", case
        assert case["accuracy_failed"] == 0 and case["accuracy_total"] > 0
        assert case["tokens_per_s"] > 0 and 0 < case["roofline_frac"] < 1
    assert status == 0
