"""Compile the gfx950 kernel library ``libxblock.so`` with hipcc.

Every ``*.hip`` file in this directory becomes one object; the objects are
linked into a single shared library next to the package (``../libxblock.so``)
so that it travels with the source tree.  Objects are rebuilt in parallel.
Run ``python build.py`` or call :func:`build`.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

CSRC = Path(__file__).resolve().parent
PACKAGE = CSRC.parent
REPO = PACKAGE.parent
LIBRARY = PACKAGE / "libxblock.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Keep the compiler from forming packed-FP32 VALU instructions.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", str(REPO / "include"),
    "-Wno-unused-result",
]


def _hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build")
    return found


# Per-file additions.  The attention kernels mask with -inf and never see
# NaN, so they drop IEEE NaN handling: max/min then compile to a single
# v_max/v_min instead of a canonicalising pair.  The GEMM keeps its MFMA
# accumulators in VGPRs: the AGPR form makes the register allocator copy
# accumulator tuples around the K loop.
EXTRA_FLAGS = {
    "fused_d128.hip": ["-fno-honor-nans"],
    "attention.hip": ["-fno-honor-nans"],
    "gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _compile(src: Path, obj: Path) -> None:
    cmd = [_hipcc(), *HIPCC_FLAGS, *EXTRA_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr}")


def build(verbose: bool = True) -> Path:
    """Compile all kernels for gfx950 and link ``libxblock.so``; return its path."""
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources in {CSRC}")
    out_dir = REPO / "_build" / "xblock"
    out_dir.mkdir(parents=True, exist_ok=True)
    objects = [out_dir / (src.stem + ".o") for src in sources]
    jobs = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        futures = [pool.submit(_compile, s, o) for s, o in zip(sources, objects)]
        for future in futures:
            future.result()
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY} from {len(sources)} HIP sources for {ARCH}")
    return LIBRARY


if __name__ == "__main__":
    build()
    sys.exit(0)
