"""The row spans of the tile pass (diffrast_amd/csrc/coverage.h) against the coverage test
itself, on the CPU: tests/native/span_check.cpp draws triangles of many shapes at several image
sizes and checks that every pixel centre ``covers()`` accepts lies inside its row's span. A
span that misses a pixel would drop a covered pixel from the visibility pass."""

import shutil
import subprocess
from pathlib import Path

import pytest

NATIVE = Path(__file__).resolve().parent / "native"


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs a host C++ compiler")
def test_row_spans_contain_every_covered_centre(tmp_path):
    exe = tmp_path / "span_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-o", str(exe),
                    str(NATIVE / "span_check.cpp")], check=True)
    out = subprocess.run([str(exe), "150000"], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout
    _, checks, accepted, span_pixels, triangles = out.stdout.split()
    assert int(triangles) > 100000 and int(accepted) > 10**7
    # The spans are tight: a few percent more pixels than are covered.
    assert int(span_pixels) < 1.1 * int(accepted)
