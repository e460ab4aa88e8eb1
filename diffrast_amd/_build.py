"""Build libdiffrast_hip.so, the gfx950 kernels, in place with hipcc.

``python -m diffrast_amd._build`` (or :func:`build`) compiles every ``csrc/*.hip`` source to an
object file under ``_build/`` in parallel and links them into ``diffrast_amd/libdiffrast_hip.so``,
where the backend loads it from. No GPU is needed: hipcc cross-compiles for gfx950.

Flags that matter for correctness:

* ``-ffp-contract=off``: no multiply-add fusion anywhere. The visibility test, the resolve and
  the interpolation repeat the reference backend's float operations one by one, which a fused
  multiply-add (one rounding instead of two) would break.
* HIP's defaults are kept for ``/`` (correctly rounded) and for fp32 denormals (kept).
* ``-Xclang -target-feature -Xclang -packed-fp32-ops``: no packed fp32 instructions.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
SOURCES = PACKAGE / "csrc"
BUILD = PACKAGE / "_build"
LIBRARY = PACKAGE / "libdiffrast_hip.so"
ARCH = os.environ.get("DIFFRAST_HIP_ARCH", "gfx950")

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc was not found; install ROCm or set HIPCC.")


def _run(cmd: list[str]) -> None:
    result = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 target feature and says so; harmless.
    noise = "is not a recognized feature for this target"
    text = "\n".join(
        line for line in (result.stdout + result.stderr).splitlines() if noise not in line
    ).strip()
    if result.returncode != 0:
        raise RuntimeError(f"command failed ({result.returncode}): {' '.join(cmd)}\n{text}")
    if text:
        print(text, file=sys.stderr)


def build(verbose: bool = False) -> Path:
    """Compile and link the library; returns its path."""
    compiler = hipcc()
    BUILD.mkdir(exist_ok=True)
    sources = sorted(SOURCES.glob("*.hip"))
    objects = [BUILD / (src.stem + ".o") for src in sources]
    jobs = [[compiler, *FLAGS, "-c", str(src), "-o", str(obj)] for src, obj in zip(sources, objects)]
    with ThreadPoolExecutor(max_workers=min(8, len(jobs))) as pool:
        list(pool.map(_run, jobs))
    tmp = LIBRARY.with_suffix(".so.tmp")
    _run([compiler, f"--offload-arch={ARCH}", "-shared", "-o", str(tmp), *map(str, objects)])
    tmp.replace(LIBRARY)
    if verbose:
        print(f"built {LIBRARY}")
    return LIBRARY


if __name__ == "__main__":
    build(verbose=True)
