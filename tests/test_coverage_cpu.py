"""The coverage test of the visibility kernels (``covers()`` in diffrast_amd/csrc/coverage.h,
compiled for the host from the same source) against the oracle's ``coverage``
(reference.py:293-365), decision for decision and depth bit for bit, on the CPU: random
triangles, centres lying exactly on edges and vertices (the fill rule's tie-breaks), degenerate
and camera-plane-crossing triangles."""

import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import reference as R

NATIVE = Path(__file__).resolve().parent / "native"


def _cases(seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    blocks = []
    # Random clip-space triangles and centres around them.
    n = 60000
    c = rng.uniform(-1, 1, (n, 1, 2))
    xy = c + rng.uniform(-0.3, 0.3, (n, 3, 2))
    w = rng.uniform(0.5, 3.0, (n, 3))
    z = rng.uniform(-1.2, 1.2, (n, 3)) * w
    p = c[:, 0] + rng.uniform(-0.3, 0.3, (n, 2))
    blocks.append(np.concatenate([xy[..., 0] * w, xy[..., 1] * w, z, w, p], axis=1))
    # Lattice triangles and centres (multiples of 1/8, w a power of two): edge values that are
    # exactly zero, so the tie-break by gradient x, then y, decides.
    n = 60000
    xy = rng.integers(-8, 9, (n, 3, 2)) / 8.0
    w = 2.0 ** rng.integers(-1, 3, (n, 3))
    z = rng.integers(-8, 9, (n, 3)) / 8.0 * w
    p = rng.integers(-8, 9, (n, 2)) / 8.0
    blocks.append(np.concatenate([xy[..., 0] * w, xy[..., 1] * w, z, w, p], axis=1))
    # Degenerate (collinear or repeated vertices) and camera-plane-crossing triangles.
    n = 20000
    a, b = rng.uniform(-1, 1, (n, 2)), rng.uniform(-1, 1, (n, 2))
    t = rng.uniform(-0.5, 1.5, (n, 1))
    xy = np.stack([a, b, a + t * (b - a)], axis=1)
    w = rng.uniform(-1.0, 2.0, (n, 3))
    z = rng.uniform(-1, 1, (n, 3)) * np.abs(w)
    p = rng.uniform(-1, 1, (n, 2))
    blocks.append(np.concatenate([xy[..., 0] * w, xy[..., 1] * w, z, w, p], axis=1))
    return np.concatenate(blocks).astype(np.float32)


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs a host C++ compiler")
def test_covers_matches_the_oracle_bit_for_bit(tmp_path):
    exe = tmp_path / "coverage_eval"
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-o", str(exe),
                    str(NATIVE / "coverage_eval.cpp")], check=True)
    cases = _cases(7)
    src, dst = tmp_path / "in.bin", tmp_path / "out.bin"
    with open(src, "wb") as f:
        f.write(np.int32(len(cases)).tobytes())
        f.write(cases.tobytes())
    subprocess.run([str(exe), str(src), str(dst)], check=True, timeout=120)
    got = np.fromfile(dst, dtype=np.float32).reshape(-1, 2)
    t = torch.from_numpy(cases)
    x, y, z, w = ([t[:, 3 * c + k] for k in range(3)] for c in range(4))
    ok, depth = R.coverage(x, y, z, w, t[:, 12], t[:, 13])
    hit = torch.from_numpy(got[:, 0] != 0)
    assert torch.equal(hit, ok), f"{(hit != ok).sum().item()} decisions differ"
    assert torch.equal(torch.from_numpy(got[:, 1])[ok], depth[ok])
    # The cases exercise every branch: hits, misses and exact ties on edges.
    e_zero = 0
    for k in range(3):
        i, j = (k + 1) % 3, (k + 2) % 3
        a_i, a_j = x[i] - t[:, 12] * w[i], x[j] - t[:, 12] * w[j]
        c_i, c_j = y[i] - t[:, 13] * w[i], y[j] - t[:, 13] * w[j]
        e_zero += int((a_i * c_j - a_j * c_i == 0).sum())
    assert ok.sum() > 5000 and (~ok).sum() > 10000 and e_zero > 1000
