#!/usr/bin/env python3
"""Throughput of the MI355X causal pre-norm block inference path.

Headline workload (the benchmark metric's configuration that fits one GPU):
benchmark config 2 = official shape 6, B=10000 S=128 D=128 H=4 F=128 L=4, one
"step" = one full forward of the whole batch with the input resident in HBM.
Weights: nn.Linear default init under torch.manual_seed(1234) (random, no
checkpoint); input: x ~ N(0,1) from seed 1234+100000 (synthetic), as the
reference's benchmark draws it (torch_transformer_benchmark.py:1478-1485).

Printed as ONE JSON line with, besides the driver's fields:
  roofline        the headline's dominant kernel (largest share of step time),
                  timed with HIP events around each of its launches inside
                  eager steps (on the launch stream), against its algorithmic
                  bytes or FLOPs; `traffic` from rocprofv3 FETCH/WRITE_SIZE
  forward_roofline  the whole forward against its own lower bound: max(FLOPs /
                  MFMA peak, (x read + y written + weights) / HBM peak)
  cpu_baseline    the CPU FP32 oracle (restated BaselineTransformer) on a
                  bounded sample of the same workload, on all of this host's
                  cores (len(os.sched_getaffinity(0)) threads)
  accuracy        the reference's rule (TTB:1237-1304) on the GPU output against
                  the oracle: the timed input's whole batch for every config
                  but cfg5, whose causal 4096-token prefix is checked on its
                  first, middle and last sequences (all 32 with
                  --full-accuracy), plus the reference's seeded trials
                  (inputs from seeds 1234+t, 5 by default; 2 on sampled
                  sequences for cfg2 and cfg5); every config's whole output
                  must also be finite (streamed_shape14.py:167-169) and no
                  split-form K/V hand-off may have failed
  per_config      all five benchmark configs: tokens/s, ms, execution plan,
                  dominant-kernel roofline, forward roofline, accuracy; cfg2
                  also times the reference's own shape-6 form (chunks of 1024
                  with graphs requested, TTB:1740, :1826-1846; each chunk is
                  one whole-stack launch, written into the output eagerly)
  decode          KV-cached single-token steps at cfg5's geometry
Timed call: forward(x, all-True mask), the reference harness's (TTB:1478-1491);
each config also reports the reference harness's per-call statistics
(median/mean/p90/min over 3 rounds of 100 calls, TTB:1426-1552) and its
measured peak device memory (streamed_shape14.py:174-175).
Timing: before the --warmup steps of every timed region, the step runs untimed
until --settle seconds of wall time have passed (default 0.1).  An MI355X
leaving idle needs about 30 ms of load before its clock settles: after 2 s
idle, cfg2's first forwards take 2.6, 2.5, 2.3, 2.2 ms and reach 1.9 ms only
from the 16th on, so 5 warm-up steps alone leave the ramp inside the timed
steps.  Then --warmup untimed steps and exactly --steps timed ones, with a
device synchronisation on both sides.  The default of 100 timed steps (about
0.19 s for cfg2) keeps one slow stretch of the clock from moving the
headline: single 20-step windows of the same code read 1.855 and 1.915 ms
in two runs.
A config whose device-memory estimate exceeds --memory-fraction of the GPU is
skipped before anything is allocated, and an out-of-memory error skips it
(the reference's SAFE_SKIP / SAFE_ABORT, streamed_shape14.py:197-222); for the
headline workload both exit with status 3.  Only one GPU is used; --gpus
above 1 exits with an explanation.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path
from typing import Optional

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

HBM_BYTES_PER_S = 8.0e12          # MI355X HBM3E peak
FP16_MFMA_FLOPS = 2.5166e15       # MI355X dense FP16 MFMA peak (256 CU x 2.4 GHz x 4096)
CONFIG_NAMES = {1: "cfg1", 6: "cfg2", 8: "cfg3", 11: "cfg4", 14: "cfg5"}
CPU_SAMPLE_ROWS = {1: 64, 6: 256, 8: 16, 11: 64, 14: 1}
LONG_PREFIX = 4096                # causal prefix checked for sequences longer than 8192
EXIT_SKIPPED = 3                  # streamed_shape14.py:214, :222
EXIT_ACCURACY = 2                 # torch_transformer_benchmark.py:1862-1865


def parse_args(argv=None):
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--workload", type=int, default=6, choices=range(1, 15), metavar="SHAPE_ID",
                   help="official shape id (1-14) of the headline line; default 6 = benchmark config 2")
    p.add_argument("--no-per-config", action="store_true", help="skip the other four configs")
    p.add_argument("--cpu-seconds", type=float, default=15.0, help="bound on the CPU baseline's timed work")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--profile-only", action="store_true", help="only the headline timed steps (for rocprofv3)")
    p.add_argument("--copy-calibration", action="store_true",
                   help="with --profile-only: also run a plain 1 GiB elementwise copy (HBM counter calibration)")
    p.add_argument("--no-traffic", action="store_true", help="skip the rocprofv3 FETCH_SIZE/WRITE_SIZE runs")
    p.add_argument("--no-decode", action="store_true", help="skip the KV-cache decode measurement")
    p.add_argument("--decode-only", action="store_true",
                   help="run only the KV-cache decode measurement and print its JSON object (for rocprofv3)")
    p.add_argument("--rounds", type=int, default=1, help="headline: median ms over this many timed rounds of --steps")
    p.add_argument("--settle", type=float, default=0.1,
                   help="seconds of untimed steps before the warm-up steps of each timed region (GPU clock ramp)")
    p.add_argument("--batch", type=int, default=0,
                   help="run the headline with this batch instead of the shape's (the line then says so)")
    p.add_argument("--accuracy-trials", type=int, default=5,
                   help="seeded accuracy trials per config, inputs seeded 1234+t, t < trials, as the reference's "
                        "harness (TTB:1307-1372, default 5, TTB:1618); the batch-heavy cfg2 and the long cfg5 run "
                        "min(trials, 2) of them on sampled sequences")
    p.add_argument("--ref-repeats", type=int, default=100,
                   help="reference-harness timing: per-call HIP-event samples per round (TTB:1426-1452, default "
                        "100 as TTB:1622); sequences longer than 8192 take 2")
    p.add_argument("--ref-rounds", type=int, default=3, help="reference-harness timing rounds (TTB:1623)")
    p.add_argument("--full-accuracy", action="store_true", help="cfg5: check all 32 sequences' prefixes")
    p.add_argument("--strict-accuracy", action="store_true", help="exit with status 2 when an accuracy check fails")
    p.add_argument("--memory-fraction", type=float, default=0.9,
                   help="skip a config whose device-memory estimate exceeds this fraction of the GPU")
    args = p.parse_args(argv)
    if (args.steps <= 0 or args.warmup < 0 or args.rounds <= 0 or args.accuracy_trials <= 0 or args.batch < 0
            or args.settle < 0 or args.ref_repeats <= 0 or args.ref_rounds <= 0):
        p.error("steps, rounds and accuracy trials must be positive; warmup, settle and batch non-negative")
    if not 0 < args.memory_fraction <= 1:
        p.error("--memory-fraction must be in (0, 1]")
    return args


def case_name(shape_id: int) -> str:
    return CONFIG_NAMES.get(shape_id, f"shape{shape_id}")


def sample_rows(shape_id: int, config) -> int:
    """Sequences per call of the bounded CPU-baseline timing sample."""
    if shape_id in CPU_SAMPLE_ROWS:
        return min(CPU_SAMPLE_ROWS[shape_id], config.batch_size)
    if config.seq_len > 8192:
        return 1
    budget = 8192 if config.d_model <= 256 else 2048  # tokens per oracle call
    return max(1, min(config.batch_size, budget // config.seq_len))


def accuracy_rows(config, full: bool):
    """Sequences whose output is checked against the oracle: all, or for long
    sequences (causal prefix only) the first, middle and last."""
    b = config.batch_size
    if config.seq_len <= 8192 or full:
        return list(range(b))
    return sorted({0, b // 2, b - 1})


def kernel_costs(name: str, config, rows: int):
    """Algorithmic (bytes, flops) of ONE launch of kernel `name` on `rows` tokens."""
    d, f, s = config.d_model, config.ffn_dim, config.seq_len
    b = rows // s
    if name.startswith("layernorm"):
        return rows * 6 * d, 0.0
    if name.startswith("residual_layernorm"):
        return rows * (10 if "_final" in name else 12) * d, 0.0
    if name.startswith("attention"):
        return rows * 8 * d, 2.0 * b * d * s * (s + 1)
    if name in ("fused_forward_d128", "fused_forward_d128_split"):
        layers = config.num_layers
        weights = 2 * layers * (4 * d * d + 2 * d * f)
        attn = 2.0 * b * layers * d * s * (s + 1)
        # split form: per sequence and layer, K and V of tokens 0..63 (FP16) written once and read once
        handoff = b * layers * 2 * (2 * 64 * d * 2) if name.endswith("_split") else 0
        return rows * 8 * d + weights + handoff, 2.0 * rows * layers * (4 * d * d + 2 * d * f) + attn
    if name.startswith("gemm_"):
        parts = name.split("_")
        n, k = int(parts[1][1:]), int(parts[2][1:])
        return rows * 2 * (n + k) + 2 * n * k, 2.0 * rows * n * k
    return 0.0, 0.0


def roofline_of(bytes_, flops, seconds):
    t_hbm, t_mfma = bytes_ / HBM_BYTES_PER_S, flops / FP16_MFMA_FLOPS
    if t_mfma > t_hbm:
        achieved = flops / seconds / 1e12
        return {"bound": "mfma", "achieved": achieved, "peak": FP16_MFMA_FLOPS / 1e12, "unit": "TFLOP/s",
                "frac": achieved * 1e12 / FP16_MFMA_FLOPS}
    achieved = bytes_ / seconds / 1e9
    return {"bound": "hbm", "achieved": achieved, "peak": HBM_BYTES_PER_S / 1e9, "unit": "GB/s",
            "frac": achieved * 1e9 / HBM_BYTES_PER_S}


def forward_lower_bound(config, flops: float):
    """(bound, seconds) of the whole forward read once / computed once: x in, y out, weights once."""
    tokens = config.batch_size * config.seq_len
    d, f, layers = config.d_model, config.ffn_dim, config.num_layers
    min_bytes = 8.0 * tokens * d + 2.0 * layers * (4 * d * d + 2 * d * f)
    t_mfma, t_hbm = flops / FP16_MFMA_FLOPS, min_bytes / HBM_BYTES_PER_S
    return ("mfma", t_mfma) if t_mfma >= t_hbm else ("hbm", t_hbm)


def device_estimate_bytes(pkg, config) -> int:
    """Device memory one config's leg needs: the forward working set (per-op
    path, the larger) plus FP32 and FP16 weights and the output's clone."""
    d, f, layers = config.d_model, config.ffn_dim, config.num_layers
    cfg_mod = __import__(pkg.__name__ + ".config", fromlist=["forward_working_set_bytes"])
    activations = cfg_mod.forward_working_set_bytes(config, config.batch_size, config.seq_len)
    clone = 4 * config.batch_size * config.seq_len * d
    weights = 8 * layers * (4 * d * d + 2 * d * f + 4 * d + f)
    return activations + clone + weights


def memory_preflight(estimate: int, free_bytes: int, total_bytes: int, fraction: float) -> Optional[str]:
    """None if `estimate` fits min(free, fraction * total), else the SAFE_SKIP reason."""
    budget = min(free_bytes, total_bytes * fraction)
    if estimate <= budget:
        return None
    return (f"SAFE_SKIP: device-memory estimate {estimate / 2**30:.2f} GiB exceeds the budget "
            f"{budget / 2**30:.2f} GiB (min of free memory and {fraction:.0%} of {total_bytes / 2**30:.2f} GiB); "
            "no model or input was allocated")


def nonfinite_count(out) -> int:
    """Elements of the (whole) output that are NaN or Inf, counted on its device."""
    import torch

    return int((~torch.isfinite(out)).sum().item())


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# Kernel symbol substring of each LaunchRecorder name (for counter CSVs).
KERNEL_SYMBOLS = (("fused_forward_d128_split", "fused_split"), ("fused_forward_d128", "fused_stack"),
                  ("attention", "attn_"),
                  ("gemm_", "gemm_"), ("residual_layernorm", "ln_"), ("layernorm", "ln_"))
CALIBRATION_BYTES = 1 << 30


def measure_traffic(workload: int, dominant: str, batch: int = 0):
    """HBM bytes per launch of `dominant` from two rocprofv3 --pmc runs of this script.

    Each run (FETCH_SIZE, then WRITE_SIZE) replays the headline workload with
    --profile-only plus a plain elementwise copy of CALIBRATION_BYTES; each
    counter is scaled by what it reads for that copy (expected: exactly
    CALIBRATION_BYTES read and written).  Returns (traffic_bytes, detail) or
    (None, reason).
    """
    import csv
    import shutil
    import subprocess
    import tempfile

    prof = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    if not Path(prof).exists():
        return None, "rocprofv3 not found"
    symbol = next((sym for prefix, sym in KERNEL_SYMBOLS if dominant.startswith(prefix)), None)
    if symbol is None:
        return None, f"no kernel symbol for {dominant}"
    detail = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        out_dir = tempfile.mkdtemp(prefix=f"xb_{counter.lower()}_", dir="/tmp")
        cmd = [prof, "--pmc", counter, "--output-format", "csv", "-d", out_dir, "-o", "run", "--",
               sys.executable, str(REPO / "bench.py"), "--profile-only", "--copy-calibration",
               "--workload", str(workload), "--steps", "2", "--warmup", "1", "--batch", str(batch)]
        try:
            proc = subprocess.run(cmd, cwd="/tmp", capture_output=True, text=True, timeout=240)
        except subprocess.TimeoutExpired:
            return None, f"rocprofv3 --pmc {counter} timed out"
        files = list(Path(out_dir).rglob("*counter_collection.csv"))
        if proc.returncode != 0 or not files:
            return None, f"rocprofv3 --pmc {counter} failed (rc {proc.returncode})"
        kernel_vals, copy_vals = [], []
        for row in csv.DictReader(open(files[0])):
            if row.get("Counter_Name") != counter:
                continue
            name, val = row["Kernel_Name"], float(row["Counter_Value"]) * 1024.0  # KiB -> bytes
            if symbol in name:
                kernel_vals.append(val)
            elif "elementwise" in name:
                copy_vals.append(val)
        shutil.rmtree(out_dir, ignore_errors=True)
        if not kernel_vals or not copy_vals or max(copy_vals) <= 0:
            return None, f"{counter}: kernel or calibration dispatch missing"
        factor = CALIBRATION_BYTES / max(copy_vals)
        detail[counter] = {"raw_bytes": statistics.median(kernel_vals), "calibration_factor": factor,
                           "bytes": statistics.median(kernel_vals) * factor, "dispatches": len(kernel_vals)}
    total = detail["FETCH_SIZE"]["bytes"] + detail["WRITE_SIZE"]["bytes"]
    return total, detail


DECODE_CONFIG = (32, 100000, 1024, 16, 1024, 2)   # cfg5's geometry; the cache holds seq_len tokens
DECODE_SPARE = 16                                  # cache slots left for the decode steps
DECODE_CHECK = (2, 4096)                           # (batch, cache capacity) of the oracle-checked decode


def decode_leg(pkg, kernels, device, time_steps, threads):
    """KV-cached decoding at cfg5's geometry: B=32 caches of 99,984 tokens, one new token per step.

    A step is one forward of [32, 1, 1024] with the cache enabled; its cost is
    dominated by the split-key attention reading each layer's K/V cache
    (4*B*S_k*D bytes per layer).  Correctness: the same decode path on a
    4095-token prompt plus one step (B=2), against the CPU oracle's forward
    over the 4096 tokens (the step's row); the oracle cannot run 100k-token
    attention.  The long run's first step is also compared with the model's
    own uncached forward (a consistency check, labelled as such).
    """
    import torch
    from oracle.accuracy import compare_outputs
    from oracle.baseline import BaselineTransformer, copy_model_weights

    cfg = pkg.TransformerConfig(*DECODE_CONFIG, True)
    torch.manual_seed(1234)
    baseline = BaselineTransformer(cfg).eval()
    model = pkg.UserOptimizedTransformer(cfg)
    copy_model_weights(baseline, model)
    model = model.to(device).eval()

    # Oracle check on a cache the CPU can attend over.
    b_chk, cap_chk = DECODE_CHECK
    small = pkg.UserOptimizedTransformer(pkg.TransformerConfig(b_chk, cap_chk, 1024, 16, 1024, 2, True))
    small.load_state_dict(model.state_dict())
    small = small.to(device).eval()
    g = torch.Generator(device=device).manual_seed(1234 + 300000)
    x_chk = torch.randn(b_chk, cap_chk, 1024, generator=g, device=device)
    small.enable_kv_cache(True)
    with torch.inference_mode():
        small(x_chk[:, : cap_chk - 1])
        step_out = small(x_chk[:, cap_chk - 1:]).cpu()
        ref = baseline(x_chk.cpu())[:, cap_chk - 1:]
    oracle_check = compare_outputs(ref, step_out)
    del small, x_chk

    prompt = cfg.seq_len - DECODE_SPARE
    g = torch.Generator(device=device).manual_seed(1234 + 200000)
    x_all = torch.randn(cfg.batch_size, prompt + 1, cfg.d_model, generator=g, device=device)
    log(f"[bench] decode: {cfg}, prompt {prompt} tokens in the cache, single-token steps")
    model.enable_kv_cache(True)
    with torch.inference_mode():
        model(x_all[:, :prompt])
        first = model(x_all[:, prompt:]).clone()
        token = x_all[:, prompt:].clone()
        ms, _ = time_steps(lambda: model(token), 8, 1, settle_first=False)  # each step appends to the cache
        steps = 4
        with kernels.LaunchRecorder() as rec:
            for _ in range(steps):
                model(token)
        torch.cuda.synchronize()
        length = model.kv_cache_length
        model.enable_kv_cache(False)
        full = model(x_all)[:, prompt:]
        torch.cuda.synchronize()
    consistency = compare_outputs(full.cpu(), first.cpu())
    per = {}
    for name, durs in rec.durations_ms().items():
        per[name] = {"avg_us": round(statistics.fmean(durs) * 1e3, 2), "per_step": len(durs) // steps}
    attn = next((k for k in per if k.startswith("attention_kv") and k.endswith("_decode")), None)
    out = {
        "workload": f"cfg5 geometry decode: B={cfg.batch_size}, cache {prompt}..{length} tokens, D={cfg.d_model}, "
                    f"H={cfg.num_heads}, L={cfg.num_layers}, one token per sequence per step",
        "ms_per_step": ms, "tokens_per_s": cfg.batch_size / (ms / 1e3),
        "check_vs_oracle": {"case": f"B={b_chk}, {cap_chk - 1}-token prompt + 1 decode step, CPU FP32 oracle "
                                    f"on {threads} threads", "passed": oracle_check.passed,
                            "failed": oracle_check.failed_elements, "total": oracle_check.total_elements,
                            "max_abs": oracle_check.max_abs_error},
        "consistency_vs_uncached_forward": {"failed": consistency.failed_elements, "total": consistency.total_elements,
                                            "max_abs": consistency.max_abs_error},
        "kernels": per,
    }
    if attn is not None:
        s_k = length - steps // 2  # mean cache length over the recorded steps
        by = 4.0 * cfg.batch_size * s_k * cfg.d_model  # K and V rows, FP16, read once
        sec = per[attn]["avg_us"] / 1e6
        out["roofline"] = {"kernel": attn, "bound": "hbm", "achieved": by / sec / 1e9, "peak": HBM_BYTES_PER_S / 1e9,
                           "unit": "GB/s", "frac": by / sec / HBM_BYTES_PER_S, "bytes_per_launch": by}
        log(f"[bench] decode: {ms:.3f} ms/step, {out['tokens_per_s']:.4g} tokens/s; {attn} {per[attn]['avg_us']:.1f} us "
            f"= {by / sec / 1e9:.0f} GB/s ({by / sec / HBM_BYTES_PER_S * 100:.1f}% of HBM); "
            f"oracle check {oracle_check.summary()}")
    del model, x_all, baseline
    torch.cuda.empty_cache()
    return out


def main(argv=None) -> int:
    args = parse_args(argv)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one MI355X only: this build has no multi-GPU path "
              "(sequences are independent, so the batch would shard across GPUs with no exchange step). "
              "Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch
    import __graft_entry__ as entry

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    pkg = entry.load_package()
    kernels = __import__(pkg.__name__ + ".kernels", fromlist=["LaunchRecorder"])
    graphs = __import__(pkg.__name__ + ".graph_runner", fromlist=["FixedInputCUDAGraph"])
    chunking = __import__(pkg.__name__ + ".batch_chunk_runner", fromlist=["BatchChunkedTransformer"])
    if not pkg.XBLOCK_AVAILABLE:
        raise RuntimeError(f"libxblock.so unavailable: {pkg.XBLOCK_LOAD_ERROR}")
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)

    def build(config):
        from oracle.baseline import BaselineTransformer, copy_model_weights

        torch.manual_seed(1234)
        baseline = BaselineTransformer(config).eval()
        model = pkg.UserOptimizedTransformer(config)
        copy_model_weights(baseline, model)
        return baseline, model.to(device).eval()

    def make_input(config, seed):
        g = torch.Generator(device=device).manual_seed(seed)
        return torch.randn(config.batch_size, config.seq_len, config.d_model, generator=g, device=device)

    def settle(run):
        """Untimed steps until args.settle seconds have passed (the clock ramp)."""
        t0 = time.perf_counter()
        batch = 1
        while time.perf_counter() - t0 < args.settle:
            t1 = time.perf_counter()
            for _ in range(batch):
                run()
            torch.cuda.synchronize()
            if time.perf_counter() - t1 < 0.01:
                batch *= 2

    def time_steps(run, steps, warmup, settle_first=True):
        if settle_first:
            settle(run)
        for _ in range(warmup):
            run()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(steps):
            run()
        end.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        return start.elapsed_time(end) / steps, wall

    def check_rows(baseline, config, out, x, rows):
        """The rule on the given sequences, in groups that bound host memory."""
        from oracle.accuracy import compare_outputs

        prefix = LONG_PREFIX if config.seq_len > 8192 else config.seq_len
        per_group = max(1, (1 << 21) // (prefix * config.d_model))
        results = []
        for i in range(0, len(rows), per_group):
            idx = torch.tensor(rows[i:i + per_group], device=out.device)
            with torch.inference_mode():
                ref = baseline(x[:, :prefix].index_select(0, idx).float().cpu().contiguous())
            results.append(compare_outputs(ref, out[:, :prefix].index_select(0, idx).cpu()))
        return results

    def seeded_trials(baseline, model, config, trials, rows):
        """The reference's accuracy trials (TTB:1307-1372): for t < trials, the
        full-size input generate_random_case draws on the GPU from seed 1234+t
        (x ~ N(0,1), all-True mask), one forward of the whole batch, checked
        against the oracle on `rows` sequences (causal prefix for long ones)."""
        from oracle.baseline import generate_random_case

        results = []
        for t in range(trials):
            xt, mt = generate_random_case(config, device, torch.float32, seed=1234 + t)
            with torch.inference_mode():
                out_t = model(xt, mt)
                torch.cuda.synchronize()
            results += check_rows(baseline, config, out_t, xt, rows)
            del xt, mt, out_t
        return results

    def reference_timing(run, repeats, rounds):
        """The reference harness's latency statistics (TTB:1426-1452, :1507-1552):
        per-call HIP events around each call, `repeats` calls per round."""
        samples = []
        for _ in range(rounds):
            starts = [torch.cuda.Event(enable_timing=True) for _ in range(repeats)]
            ends = [torch.cuda.Event(enable_timing=True) for _ in range(repeats)]
            torch.cuda.synchronize()
            for i in range(repeats):
                starts[i].record()
                run()
                ends[i].record()
            torch.cuda.synchronize()
            samples += [a.elapsed_time(b) for a, b in zip(starts, ends)]
        ordered = sorted(samples)
        pos = (len(ordered) - 1) * 0.9
        lo, hi = int(pos), min(int(pos) + 1, len(ordered) - 1)
        p90 = ordered[lo] * (1.0 - (pos - lo)) + ordered[hi] * (pos - lo)
        return {"median_ms": statistics.median(samples), "mean_ms": statistics.fmean(samples), "p90_ms": p90,
                "min_ms": ordered[0], "samples": len(samples), "rounds": rounds,
                "note": "per-call HIP events as the reference's benchmark_once (TTB:1426-1452); includes each "
                        "call's host issue time when the GPU is idle"}

    def cpu_leg(baseline, config, x_gpu, budget_s, rows_per_call):
        """The oracle on the host cores over a bounded slice: tokens/s."""
        x_cpu = x_gpu[:rows_per_call].float().cpu()
        prefix = None
        if config.seq_len > 8192:  # long context: causal prefix only
            prefix = LONG_PREFIX
            x_cpu = x_gpu[:rows_per_call, :prefix].float().cpu()
        with torch.inference_mode():
            t0 = time.perf_counter()
            baseline(x_cpu)
            first = time.perf_counter() - t0
            calls, elapsed = 1, first
            while elapsed < budget_s * 0.5 and elapsed + first < budget_s:
                t1 = time.perf_counter()
                baseline(x_cpu)
                elapsed += time.perf_counter() - t1
                calls += 1
        tokens = calls * x_cpu.shape[0] * x_cpu.shape[1]
        sample = f"{x_cpu.shape[0]} x {x_cpu.shape[1]} tokens per call, {calls} calls" + (
            f" (causal prefix {prefix} of S={config.seq_len})" if prefix else "")
        return {"value": tokens / elapsed, "unit": "tokens/s", "cores": threads, "kind": "port", "sample": sample}

    def kernel_profile(model, x, mask, config, tokens, reps, step_ms, lead=0):
        """Per-kernel average launch time from HIP events around each launch.

        A forward that is one launch has its kernel time bounded by the step
        time (back-to-back launches between two events, no per-launch event
        overhead); the events around a single tens-of-microseconds launch
        read several percent long, so such a kernel takes the smaller of the
        two and says which it used."""
        with torch.inference_mode():
            # `lead` unrecorded forwards first, with no synchronisation after them:
            # the host then runs ahead of the GPU, so the events around a short
            # kernel time the kernel and not the host's issue gaps.
            for _ in range(lead):
                model(x, mask)
            with kernels.LaunchRecorder() as rec:
                for _ in range(reps):
                    model(x, mask)
        torch.cuda.synchronize()
        durations = rec.durations_ms()
        one_launch = len(durations) == 1 and len(next(iter(durations.values()))) == reps
        per = {}
        for kname, durs in durations.items():
            avg = statistics.fmean(durs)
            source = "hip_events_per_launch"
            if one_launch and step_ms < avg:
                avg, source = step_ms, "step_time (one launch per forward)"
            b_, f_ = kernel_costs(kname, config, tokens)
            per[kname] = {"avg_ms": avg, "launches_per_step": len(durs) // reps, "time_source": source,
                          "share_ms": avg * len(durs) / reps, **roofline_of(max(b_, 1.0), f_, avg / 1e3),
                          "bytes_per_launch": b_, "flops_per_launch": f_}
        dominant = max(per, key=lambda k: per[k]["share_ms"])
        return per, dominant

    if args.decode_only:
        print(json.dumps({"decode": decode_leg(pkg, kernels, device, time_steps, threads)}), flush=True)
        return 0

    results = {}
    order = [args.workload] + ([] if (args.no_per_config or args.profile_only)
                               else [i for i in CONFIG_NAMES if i != args.workload])
    headline = None
    accuracy_failed = False
    free_bytes, total_bytes = torch.cuda.mem_get_info(device)
    for shape_id in order:
        config = pkg.OFFICIAL_BENCHMARK_SHAPES[shape_id]
        name = case_name(shape_id)
        is_head = shape_id == args.workload
        if is_head and args.batch and args.batch != config.batch_size:
            import dataclasses

            config = dataclasses.replace(config, batch_size=args.batch)
            name = f"{name}-b{args.batch}"
        log(f"[bench] {name} (official shape {shape_id}): {config}")
        estimate = device_estimate_bytes(pkg, config)
        free_bytes, _ = torch.cuda.mem_get_info(device)
        skip = memory_preflight(estimate, free_bytes, total_bytes, args.memory_fraction)
        if skip is not None:
            log(f"[bench] {name}: {skip}")
            if is_head:
                print(skip, flush=True)
                return EXIT_SKIPPED
            results[name] = {"workload": name, "official_shape": shape_id, "status": "SKIP", "reason": skip}
            continue
        try:
            entry_, head_extra = run_config(
                args, pkg, config, shape_id, name, is_head, build, make_input, time_steps, check_rows,
                seeded_trials, reference_timing, cpu_leg, kernel_profile, graphs, chunking, kernels, device)
        except torch.cuda.OutOfMemoryError as error:
            torch.cuda.empty_cache()
            reason = f"SAFE_ABORT: out of device memory: {str(error).splitlines()[0]}"
            log(f"[bench] {name}: {reason}")
            if is_head:
                print(reason, flush=True)
                return EXIT_SKIPPED
            results[name] = {"workload": name, "official_shape": shape_id, "status": "SKIP", "reason": reason}
            continue
        accuracy_failed |= not entry_.get("accuracy", {}).get("passed", True)
        results[name] = entry_
        if is_head:
            headline = dict(entry_, config=config, **head_extra)
        torch.cuda.empty_cache()

    decode = None
    if not (args.no_per_config or args.profile_only or args.no_decode):
        decode = decode_leg(pkg, kernels, device, time_steps, threads)
        accuracy_failed |= not decode["check_vs_oracle"]["passed"]

    if args.profile_only and args.copy_calibration:
        # A plain streaming copy of known size: reads and writes exactly
        # CALIBRATION_BYTES (the HBM counters' scale reference).
        src = torch.ones(CALIBRATION_BYTES // 4, device=device)
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.mul(src, 1.0, out=dst)
        torch.cuda.synchronize()
        del src, dst

    cfg = headline["config"]
    line = {
        "metric": "tokens/sec per config on 1 MI355X; % of FP16 MFMA / HBM roofline",
        "value": headline["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": headline["steps"],
        "warmup": args.warmup,
        "settle_s": args.settle,
        "rounds": args.rounds,
        "ms_per_step": headline["ms"],
        **({"rounds_ms": headline["rounds_ms"]} if "rounds_ms" in headline else {}),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (x ~ N(0,1) seeded; nn.Linear default init, seed 1234)",
        "config": {
            "workload": f"{case_name(args.workload)}: official shape {args.workload}, causal pre-norm block forward"
                        + (f" at batch {cfg.batch_size}" if args.batch else ""),
            "batch": cfg.batch_size, "seq_len": cfg.seq_len, "d_model": cfg.d_model, "heads": cfg.num_heads,
            "ffn_dim": cfg.ffn_dim, "layers": cfg.num_layers, "mode": headline["mode"],
            "plan": headline["plan"],
        },
    }
    if "roofline" in headline:
        line["roofline"] = dict(headline["roofline"], traffic=None)
        line["kernels"] = headline["kernels"]
    line["forward_roofline"] = headline["forward_roofline"]
    line["pipeline_bytes_frac"] = headline["pipeline_bytes_frac"]
    if "roofline" in headline and not args.no_traffic and not args.profile_only:
        dominant = headline["roofline"]["kernel"]
        log(f"[bench] HBM traffic of {dominant}: two rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE)")
        traffic, detail = measure_traffic(args.workload, dominant, args.batch)
        line["roofline"]["traffic"] = traffic
        line["roofline"]["traffic_detail"] = detail
        if traffic is not None:
            log(f"[bench] traffic {traffic / 1e9:.4f} GB per launch vs algorithmic "
                f"{line['roofline']['bytes_per_launch'] / 1e9:.4f} GB")
        else:
            log(f"[bench] traffic unavailable: {detail}")
    if "cpu_baseline" in headline:
        line["cpu_baseline"] = headline["cpu_baseline"]
    if "accuracy" in headline:
        line["accuracy"] = headline["accuracy"]
    if decode is not None:
        line["decode"] = decode
    if len(results) > 1:
        line["per_config"] = {n: {k: v for k, v in r.items() if k not in ("kernels",)} for n, r in results.items()}
    print(json.dumps(line), flush=True)
    if args.strict_accuracy and accuracy_failed:
        log("[bench] accuracy check FAILED")
        return EXIT_ACCURACY
    return 0


def trial_rows(config):
    """Sequences each seeded trial checks: every one for the small configs;
    1024 (first, middle and last ranges) for a batch of 10,000; the first,
    middle and last for long sequences (causal prefix)."""
    b = config.batch_size
    if config.seq_len > 8192:
        return sorted({0, b // 2, b - 1})
    if b * config.seq_len >= 1_000_000:
        third = 1024 // 3
        return sorted(set(range(third)) | set(range(b // 2, b // 2 + third)) | set(range(b - (1024 - 2 * third), b)))
    return list(range(b))


def run_config(args, pkg, config, shape_id, name, is_head, build, make_input, time_steps, check_rows,
               seeded_trials, reference_timing, cpu_leg, kernel_profile, graphs, chunking, kernels, device):
    """Time one config, profile its kernels, check it; returns (per-config entry, headline extras)."""
    import torch

    torch.cuda.reset_peak_memory_stats(device)
    baseline, model = build(config)
    x = make_input(config, 1234 + 100000)
    # The reference times its fixed input with the mask generate_random_case
    # gives at padding_ratio 0: all True (TTB:1478-1491, TTB:1615).
    mask = torch.ones(config.batch_size, config.seq_len, device=device, dtype=torch.bool)
    tokens = config.batch_size * config.seq_len
    big = config.seq_len > 8192
    if big:
        steps, warmup = (max(1, min(args.steps, 3)), 1) if is_head else (2, 1)
    else:
        # Non-headline small configs: 20 warmups, 3 rounds of 100, median
        # (the repeat counts the reference's harness suggests).
        steps, warmup = (args.steps, args.warmup) if is_head else (100, 20)
    plan = model.execution_plan(config.batch_size, config.seq_len)
    failures_before = kernels.split_handoff_failures(device)
    with torch.inference_mode():
        if big or tokens >= 1_000_000:
            run = lambda: model(x, mask)  # noqa: E731  (launch-overhead-free at this size)
            mode = "eager"
        else:
            # The reference harness's choice (cuda_graph_runner.maybe_cuda_graph):
            # replay with the output clone, or eager for a one-kernel forward.
            runner, graphed, status = graphs.maybe_cuda_graph(model, x, mask, enabled=True)
            run = lambda: runner(x, mask)  # noqa: E731
            mode = "hipGraph replay" if graphed else f"eager: {status}"
            overlap = model.captured_overlap(config.batch_size, config.seq_len) if graphed else None
            if overlap:
                mode += f"; {overlap}"
        rounds_ms = None
        if big or (is_head and args.rounds == 1):
            ms, wall = time_steps(run, steps, warmup)
        else:
            n_rounds = args.rounds if is_head else 3
            rounds = [time_steps(run, steps, warmup if r == 0 else 0) for r in range(n_rounds)]
            rounds_ms = [r[0] for r in rounds]
            ms, wall = statistics.median(rounds_ms), sum(r[1] for r in rounds)
        ref_stats = None
        if not args.profile_only:
            ref_stats = reference_timing(run, 2 if big else args.ref_repeats, 1 if big else args.ref_rounds)
        out = model(x, mask)
        torch.cuda.synchronize()
    entry_ = {"workload": name, "official_shape": shape_id, "status": "PASS", "tokens_per_s": tokens / (ms / 1e3),
              "ms": ms, "mode": mode, "steps": steps, "plan": plan.describe(),
              "timed_call": "forward(x, valid_token_mask=all True) as the reference harness (TTB:1478-1491)"}
    if rounds_ms is not None:
        entry_["rounds_ms"] = rounds_ms
    if ref_stats is not None:
        entry_["reference_harness_timing"] = ref_stats
    flops = pkg.forward_flops(config)
    bound, t_bound = forward_lower_bound(config, flops)
    entry_["forward_roofline"] = {"bound": bound, "frac": t_bound / (ms / 1e3),
                                  "note": "whole forward vs max(FLOPs/MFMA peak, (x+y+weights)/HBM peak)"}
    pipe = pkg.forward_bytes(config) / HBM_BYTES_PER_S
    entry_["pipeline_bytes_frac"] = {"frac": pipe / (ms / 1e3),
                                     "note": "unfused kernel pipeline's bytes / HBM peak / step time; "
                                             "not a roofline (a fused kernel moves fewer bytes, so it can exceed 1)"}
    head_extra = {}
    if not args.profile_only:
        reps = 1 if big else max(2, min(steps, 5))
        per, dominant = kernel_profile(model, x, mask, config, tokens, reps, ms, lead=0 if big else 20)
        k = per[dominant]
        entry_["roofline"] = {"kernel": dominant, "bound": k["bound"], "achieved": k["achieved"], "peak": k["peak"],
                              "unit": k["unit"], "frac": k["frac"], "avg_us": k["avg_ms"] * 1e3,
                              "time_source": k["time_source"],
                              "share_of_step": k["share_ms"] / ms, "bytes_per_launch": k["bytes_per_launch"],
                              "flops_per_launch": k["flops_per_launch"]}
        entry_["kernels"] = {n: {"avg_us": round(v["avg_ms"] * 1e3, 2), "per_step": v["launches_per_step"],
                                 "frac": round(v["frac"], 4), "bound": v["bound"]} for n, v in per.items()}
        head_extra["kernels"] = entry_["kernels"]
        for kname, v in sorted(per.items(), key=lambda kv: -kv[1]["share_ms"]):
            log(f"[bench]   {kname:28s} {v['avg_ms'] * 1e3:9.1f} us x{v['launches_per_step']} "
                f"{v['achieved']:9.1f} {v['unit']} ({v['frac'] * 100:5.1f}% {v['bound']})")
    # Device memory of the timed forward (streamed_shape14.py:174-175): model,
    # input, mask, the forward's working set and the replay's output clone.
    entry_["peak_memory"] = {"allocated_gib": torch.cuda.max_memory_allocated(device) / 2**30,
                             "reserved_gib": torch.cuda.max_memory_reserved(device) / 2**30,
                             "estimate_gib": device_estimate_bytes(pkg, config) / 2**30}
    log(f"[bench] {name}: {ms:.3f} ms/step, {entry_['tokens_per_s']:.4g} tokens/s ({mode}); plan {plan.describe()}; "
        f"forward {entry_['forward_roofline']['frac']:.3f} of its {bound} lower bound"
        + (f"; dominant {entry_['roofline']['kernel']} at {entry_['roofline']['frac']:.3f} of "
           f"{entry_['roofline']['bound']} peak" if "roofline" in entry_ else "")
        + (f"; reference harness median {ref_stats['median_ms']:.4f} ms" if ref_stats else "")
        + f"; peak allocated {entry_['peak_memory']['allocated_gib']:.2f} GiB")

    if not args.profile_only:
        bad = nonfinite_count(out)
        rows = accuracy_rows(config, args.full_accuracy)
        checks = check_rows(baseline, config, out, x, rows)
        del out
        small = not big and tokens < 1_000_000
        trials = args.accuracy_trials if small else min(args.accuracy_trials, 2)
        t_rows = trial_rows(config)
        checks += seeded_trials(baseline, model, config, trials, t_rows)
        handoff = kernels.split_handoff_failures(device) - failures_before
        passed = all(c.passed for c in checks) and bad == 0 and handoff == 0
        entry_["accuracy"] = {
            "passed": passed, "failed": sum(c.failed_elements for c in checks),
            "total": sum(c.total_elements for c in checks), "max_abs": max(c.max_abs_error for c in checks),
            "timed_input_sequences_checked": len(rows),
            "trials": 1 + trials, "seeded_trials": trials, "trial_seeds": f"1234+t, t < {trials}",
            "trial_sequences_checked": len(t_rows),
            "nonfinite_in_whole_output": bad, "split_handoff_failures": handoff,
            "prefix": LONG_PREFIX if config.seq_len > 8192 else None,
        }
        if not passed:
            entry_["status"] = "FAIL"
        log(f"[bench] {name}: accuracy: timed input on {len(rows)} sequences + {trials} seeded trials on "
            f"{len(t_rows)}: failed {entry_['accuracy']['failed']}/{entry_['accuracy']['total']}, max_abs "
            f"{entry_['accuracy']['max_abs']:.3g}; non-finite in the whole output: {bad}; failed hand-offs: {handoff}")
        if not args.no_cpu_baseline or is_head:
            budget = 0.0 if args.no_cpu_baseline else (args.cpu_seconds if is_head else min(args.cpu_seconds, 5.0))
            cpu = cpu_leg(baseline, config, x, budget, sample_rows(shape_id, config))
            entry_["cpu_baseline_tokens_per_s"] = cpu["value"]
            log(f"[bench] {name}: CPU FP32 oracle {cpu['value']:.4g} tokens/s on {cpu['cores']} threads "
                f"({cpu['sample']})")
            if is_head:
                head_extra["cpu_baseline"] = cpu
    else:
        del out
    if shape_id == 6 and not args.profile_only and not args.batch:
        # The reference's own shape-6 form: chunks of 1024 with graphs requested (a chunk whose
        # forward is one kernel is launched eagerly into its output slice instead of replayed).
        chunked = chunking.BatchChunkedTransformer(model, 1024, all_tokens_valid=True, use_cuda_graphs=True)
        with torch.inference_mode():
            c_ms, _ = time_steps(lambda: chunked(x), 10, 2)
            same = bool(torch.equal(chunked(x), model(x, mask)))
        entry_["reference_form_chunk1024_graphs"] = {
            "ms": c_ms, "tokens_per_s": tokens / (c_ms / 1e3), "equal_to_unchunked": same,
            "status": chunked.graph_status}
        log(f"[bench] {name}: chunk-1024 form {c_ms:.3f} ms ({chunked.graph_status}); bitwise equal: {same}")
        del chunked
    del baseline, model, x
    return entry_, head_extra


if __name__ == "__main__":
    raise SystemExit(main())
