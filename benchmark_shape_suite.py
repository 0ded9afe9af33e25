#!/usr/bin/env python3
"""Run official benchmark shapes in isolated processes on one MI355X.

The counterpart of the reference's shape-suite runner
(benchmark_shape_suite.py:59-94, :176-333): each selected official shape runs
in a fresh `bench.py` process (a crash, hang or out-of-memory in one case
cannot touch the next), after a memory preflight that skips shapes whose
estimated device footprint exceeds --memory-fraction of the GPU.  Each case
ends as

  PASS   the case ran and every accuracy trial met the reference's rule
  PROXY  shape 14 on fewer than its 32 sequences (--shape14-samples); otherwise
         as PASS
  SKIP   the preflight estimate does not fit (--force-oversized runs it anyway),
         or bench.py itself skipped it (status 3: its own memory preflight or
         an out-of-memory error, the reference's SAFE_SKIP / SAFE_ABORT)
  FAIL   non-zero exit (an accuracy failure exits with 2), a time-out, or no
         result line

and the summary gives tokens/s, ms per forward, the dominant kernel's bound
(HBM or FP16 MFMA) and the fraction of that roofline it reached, the whole
forward's fraction of its lower bound, the accuracy counts, and geometric
means; --json writes the same as a file.  Exit status: 1 if a case
FAILed, or with --strict if one was SKIPped or PROXY; else 0.

Differences from the reference's runner: shape 14 runs at the real S=100000
in one process (the whole batch fits in 288 GB of HBM, so there is no
streamed proxy; --run-full-shape14 is accepted and changes nothing), and the
timing/accuracy worker is this repository's bench.py.
"""

from __future__ import annotations

import argparse
import json
import math
import statistics
import subprocess
import sys
import threading
from dataclasses import asdict, dataclass, field
from pathlib import Path
from typing import Callable, Dict, List, Optional, Sequence, Tuple

REPO = Path(__file__).resolve().parent
GIB = 1024**3
SHAPE14_BATCH = 32


def _package():
    sys.path.insert(0, str(REPO))
    import __graft_entry__ as entry

    return entry.load_package()


@dataclass
class CaseResult:
    shape_id: int
    status: str
    reason: str = ""
    tokens_per_s: Optional[float] = None
    ms: Optional[float] = None
    bound: Optional[str] = None
    roofline_frac: Optional[float] = None
    bound_min: Optional[str] = None
    kernel: Optional[str] = None
    roofline_frac_min: Optional[float] = None
    accuracy_failed: Optional[int] = None
    accuracy_total: Optional[int] = None
    accuracy_trials: Optional[int] = None
    cpu_tokens_per_s: Optional[float] = None
    estimated_peak_gib: Optional[float] = None
    line: Dict = field(default_factory=dict)


def parse_case_ids(specification: str, known: Sequence[int], configs: Sequence[int]) -> List[int]:
    """``all``, ``configs`` (the five benchmark configs), or values such as ``1,3,7`` / ``1-5,12``.

    Same grammar and errors as the reference (benchmark_shape_suite.py:34-56).
    """
    spec = specification.strip().lower()
    if spec == "all":
        return sorted(known)
    if spec == "configs":
        return sorted(configs)
    selected = set()
    for part in specification.split(","):
        token = part.strip()
        if not token:
            raise ValueError("empty value in --cases")
        if "-" in token:
            start_text, end_text = token.split("-", maxsplit=1)
            start, end = int(start_text), int(end_text)
            if start > end:
                raise ValueError(f"invalid descending case range: {token}")
            selected.update(range(start, end + 1))
        else:
            selected.add(int(token))
    unknown = sorted(selected.difference(known))
    if unknown:
        raise ValueError(f"unknown benchmark shape IDs: {unknown}")
    return sorted(selected)


def estimated_peak_bytes(config, batch: Optional[int] = None) -> int:
    """Conservative device footprint of one bench.py case on the per-op kernel path.

    Per token (M = B*S rows): input, output, its graph-replay clone and the
    FP32 residual stream (16 D bytes); FP16 LayerNorm outputs, packed QKV,
    context and updates (14 D); the FP16 FFN hidden row (2 F); doubled for the
    caching allocator's slack.  Weights: FP32 parameters plus FP16 and
    fragment-packed copies, 8 bytes per weight.  The fused d128 path needs
    less.  Unlike the reference's estimate (benchmark_shape_suite.py:59-94)
    there is no FP32 baseline on the device -- the oracle runs on the host.
    """
    b = config.batch_size if batch is None else batch
    m = b * config.seq_len
    d, f, layers = config.d_model, config.ffn_dim, config.num_layers
    activations = m * (16 * d + 14 * d + 2 * f) * 2
    weights = 8 * layers * (4 * d * d + 2 * d * f + 4 * d + f)
    return activations + weights


def case_command(shape_id: int, args: argparse.Namespace, batch: int) -> List[str]:
    quick = args.quick
    command = [
        sys.executable, "-u", str(REPO / "bench.py"),
        "--workload", str(shape_id), "--no-per-config", "--no-traffic", "--strict-accuracy",
        "--steps", str(10 if quick else args.repeats),
        "--warmup", str(3 if quick else args.warmup),
        "--rounds", str(1 if quick else args.benchmark_rounds),
        "--accuracy-trials", str(1 if quick else args.accuracy_trials),
        "--cpu-seconds", str(args.cpu_seconds),
    ]
    if batch:
        command += ["--batch", str(batch)]
    return command


Launcher = Callable[[List[str], float], Tuple[int, str]]


def launch_case(command: List[str], timeout: float) -> Tuple[int, str]:
    """Run one case in its own process; echo its output live; return (status, stdout).

    A time-out kills the child (status 124, as `timeout` reports it).
    """
    proc = subprocess.Popen(command, cwd=str(REPO), stdout=subprocess.PIPE, stderr=None, text=True, bufsize=1)
    lines: List[str] = []

    def pump() -> None:
        assert proc.stdout is not None
        for text in proc.stdout:
            lines.append(text)
            print(text, end="", flush=True)

    reader = threading.Thread(target=pump, daemon=True)
    reader.start()
    try:
        status = proc.wait(timeout=timeout)
    except subprocess.TimeoutExpired:
        proc.kill()
        proc.wait()
        status = 124
    reader.join(timeout=10)
    return status, "".join(lines)


def _result_line(stdout: str) -> Optional[Dict]:
    for text in reversed(stdout.strip().splitlines()):
        text = text.strip()
        if text.startswith("{") and text.endswith("}"):
            try:
                return json.loads(text)
            except json.JSONDecodeError:
                return None
    return None


def run_case(shape_id: int, config, args: argparse.Namespace, device_bytes: Optional[int],
             launcher: Launcher) -> CaseResult:
    batch = 0
    if shape_id == 14 and args.shape14_samples != SHAPE14_BATCH:
        batch = args.shape14_samples
    estimate = estimated_peak_bytes(config, batch or None)
    result = CaseResult(shape_id, "FAIL", estimated_peak_gib=estimate / GIB)
    print(f"config={config} | estimated_peak={estimate / GIB:.2f} GiB" + (f" | batch {batch}" if batch else ""),
          flush=True)
    if device_bytes is not None and estimate > device_bytes * args.memory_fraction and not args.force_oversized:
        result.status = "SKIP"
        result.reason = (f"estimated peak exceeds {args.memory_fraction:.0%} of "
                         f"{device_bytes / GIB:.2f} GiB device memory")
        print(f"SKIP: {result.reason}", flush=True)
        return result

    status, stdout = launcher(case_command(shape_id, args, batch), args.case_timeout)
    line = _result_line(stdout)
    if line is not None:
        result.line = line
        result.tokens_per_s = line.get("value")
        result.ms = line.get("ms_per_step")
        kernel = line.get("roofline") or {}
        forward = line.get("forward_roofline") or {}
        result.roofline_frac = kernel.get("frac")
        result.bound = kernel.get("bound")
        result.kernel = kernel.get("kernel")
        result.roofline_frac_min = forward.get("frac")
        result.bound_min = forward.get("bound")
        accuracy = line.get("accuracy") or {}
        result.accuracy_failed = accuracy.get("failed")
        result.accuracy_total = accuracy.get("total")
        result.accuracy_trials = accuracy.get("trials")
        result.cpu_tokens_per_s = (line.get("cpu_baseline") or {}).get("value")
    if status == 124:
        result.reason = f"timed out after {args.case_timeout:.0f} s"
    elif status == 3:  # bench.py's SAFE_SKIP (preflight) or SAFE_ABORT (out of memory)
        result.status = "SKIP"
        result.reason = next((t.strip() for t in stdout.splitlines() if t.startswith("SAFE_")),
                             "skipped by the benchmark (status 3)")
    elif status == 2 and line is not None:
        result.reason = "accuracy check failed"
    elif status != 0:
        result.reason = f"benchmark exited with status {status}"
    elif line is None:
        result.reason = "no result line"
    elif not (line.get("accuracy") or {}).get("passed", False):
        result.reason = "no passing accuracy result"
    elif batch:
        result.status = "PROXY"
        result.reason = f"real sequence completed for {batch}/{SHAPE14_BATCH} samples"
    else:
        result.status = "PASS"
    return result


def geometric_mean(values: Sequence[float]) -> Optional[float]:
    values = [v for v in values if v is not None and v > 0]
    if not values:
        return None
    return math.exp(statistics.fmean(math.log(v) for v in values))


def summary_lines(results: Sequence[CaseResult]) -> List[str]:
    out = ["=== Official shape-suite summary ===",
           "roofline: the dominant kernel's algorithmic bytes or FLOPs per launch / its HIP-event time,",
           "as a fraction of HBM or FP16 MFMA peak; fused: the whole forward against its lower bound",
           "max(FLOPs / MFMA peak, (x + y + weights) / HBM peak)",
           f"{'shape':>5}  {'status':6}  {'tokens/s':>11}  {'ms':>10}  {'bound':5}  {'roofline':>8}  "
           f"{'fused':>11}  accuracy"]
    for r in results:
        if r.tokens_per_s is None:
            out.append(f"{r.shape_id:5d}  {r.status:6}  {r.reason}")
            continue
        acc = (f"{r.accuracy_failed}/{r.accuracy_total} failed over {r.accuracy_trials} trial(s)"
               if r.accuracy_total is not None else "not checked")
        frac = f"{r.roofline_frac * 100:7.1f}%" if r.roofline_frac is not None else "     n/a"
        fmin = (f"{r.roofline_frac_min * 100:5.1f}% {r.bound_min or '-':4}" if r.roofline_frac_min is not None
                else "        n/a")
        out.append(f"{r.shape_id:5d}  {r.status:6}  {r.tokens_per_s:11.4g}  {r.ms:10.4f}  {r.bound or '-':5}  "
                   f"{frac}  {fmin}  {acc}" + (f"  ({r.reason})" if r.reason else ""))
    done = [r for r in results if r.status in ("PASS", "PROXY")]
    gm = geometric_mean([r.roofline_frac for r in done])
    if gm is not None:
        out.append(f"geometric-mean roofline fraction across completed cases: {gm * 100:.1f}%")
    gm_min = geometric_mean([r.roofline_frac_min for r in done])
    if gm_min is not None:
        out.append(f"geometric-mean fraction of the fused lower bound: {gm_min * 100:.1f}%")
    return out


def exit_status(results: Sequence[CaseResult], strict: bool) -> int:
    if any(r.status == "FAIL" for r in results):
        return 1
    if strict and any(r.status in ("SKIP", "PROXY") for r in results):
        return 1
    return 0


def run_suite(shape_ids: Sequence[int], shapes: Dict, args: argparse.Namespace, device_bytes: Optional[int],
              launcher: Launcher = launch_case) -> List[CaseResult]:
    results = []
    for position, shape_id in enumerate(shape_ids, start=1):
        print(f"\n=== [{position}/{len(shape_ids)}] official shape {shape_id} ===", flush=True)
        results.append(run_case(shape_id, shapes[shape_id], args, device_bytes, launcher))
    return results


def parse_args(argv: Optional[Sequence[str]] = None) -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--cases", default="configs",
                   help="all, configs (the five benchmark configs: shapes 1,6,8,11,14), or ids such as 1,3,7 or 1-5,12")
    p.add_argument("--list", action="store_true", help="list the official shapes and exit")
    p.add_argument("--device", default="auto", help="auto, cuda or cuda:0 (one MI355X)")
    p.add_argument("--quick", action="store_true", help="one accuracy trial and fewer timing samples")
    p.add_argument("--accuracy-trials", type=int, default=5)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--repeats", type=int, default=100, help="timed forwards per round")
    p.add_argument("--benchmark-rounds", type=int, default=3, help="timed rounds; the median is reported")
    p.add_argument("--memory-fraction", type=float, default=0.8,
                   help="maximum fraction of device memory allowed by the preflight estimate")
    p.add_argument("--force-oversized", action="store_true", help="run cases the preflight would skip")
    p.add_argument("--strict", action="store_true", help="exit 1 if any case is skipped or a proxy")
    p.add_argument("--run-full-shape14", action="store_true",
                   help="accepted for compatibility: shape 14 always runs the real 100000-token sequence")
    p.add_argument("--shape14-samples", type=int, default=SHAPE14_BATCH,
                   help="sequences of shape 14 to run (official batch 32; fewer gives PROXY)")
    p.add_argument("--cpu-seconds", type=float, default=5.0, help="bound on each case's CPU oracle timing")
    p.add_argument("--case-timeout", type=float, default=1200.0, help="seconds before a case is killed (FAIL)")
    p.add_argument("--json", type=Path, default=None, help="also write the results to this file")
    args = p.parse_args(argv)
    if not 0 < args.memory_fraction <= 1:
        p.error("--memory-fraction must be in (0, 1]")
    if args.accuracy_trials <= 0:
        p.error("--accuracy-trials must be positive")
    if args.warmup < 0 or args.repeats <= 0 or args.benchmark_rounds <= 0:
        p.error("warmup must be non-negative; repeats/rounds must be positive")
    if not 1 <= args.shape14_samples <= SHAPE14_BATCH:
        p.error(f"--shape14-samples must be between 1 and {SHAPE14_BATCH}")
    if args.device not in ("auto", "cuda", "cuda:0"):
        p.error("this suite runs on one MI355X: --device must be auto, cuda or cuda:0")
    return args


def device_memory_bytes() -> Optional[int]:
    import torch

    if not torch.cuda.is_available():
        return None
    return torch.cuda.get_device_properties(0).total_memory


def main(argv: Optional[Sequence[str]] = None) -> int:
    args = parse_args(argv)
    pkg = _package()
    shapes = pkg.OFFICIAL_BENCHMARK_SHAPES
    if args.list:
        for shape_id, config in shapes.items():
            tag = " (benchmark config)" if shape_id in pkg.BENCHMARK_CONFIG_SHAPE_IDS else ""
            print(f"shape {shape_id:02d}: {config}{tag}")
        return 0
    try:
        shape_ids = parse_case_ids(args.cases, list(shapes), pkg.BENCHMARK_CONFIG_SHAPE_IDS)
    except ValueError as error:
        print(f"error: {error}", file=sys.stderr)
        return 2
    device_bytes = device_memory_bytes()
    if device_bytes is None:
        print("error: no GPU visible; the suite measures the HIP path on one MI355X", file=sys.stderr)
        return 2
    results = run_suite(shape_ids, shapes, args, device_bytes)
    print()
    for text in summary_lines(results):
        print(text)
    if args.json is not None:
        payload = {
            "cases": [{k: v for k, v in asdict(r).items() if k != "line"} | {"bench": r.line} for r in results],
            "geomean_roofline_frac": geometric_mean(
                [r.roofline_frac for r in results if r.status in ("PASS", "PROXY")]),
            "geomean_roofline_frac_min": geometric_mean(
                [r.roofline_frac_min for r in results if r.status in ("PASS", "PROXY")]),
            "device_bytes": device_bytes,
        }
        args.json.parent.mkdir(parents=True, exist_ok=True)
        args.json.write_text(json.dumps(payload, indent=1))
    return exit_status(results, args.strict)


if __name__ == "__main__":
    raise SystemExit(main())
