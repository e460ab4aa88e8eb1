"""ctypes binding of the oracle's C restatements (oracle/visible.c, built by oracle/Makefile
into oracle/_build/liboracle.so): TEST INFRASTRUCTURE, never part of the product.

``visible_at`` is oracle.reference.visible_at (the reference's brute-force visibility,
reference.py:293-397, at listed pixels) in C with threads, for checking every triangle of the
large workloads at thousands of pixels. Same arguments and results.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent
LIBRARY = HERE / "_build" / "liboracle.so"
_lib = None


def build() -> Path:
    """Compiles the C restatements (make, gcc)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIBRARY


def load():
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            build()
        lib = ctypes.CDLL(str(LIBRARY))
        f = lib.oracle_visible_at
        f.restype = ctypes.c_int
        p = ctypes.c_void_p
        f.argtypes = [p, ctypes.c_int64, p, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                      ctypes.c_int64, p, p, p, p, p, p, p, ctypes.c_int]
        _lib = lib
    return _lib


def _threads() -> int:
    """The cores this process may run on, limited by OMP_NUM_THREADS where the environment sets
    it (a machine's share of cores for this job)."""
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    limit = os.environ.get("OMP_NUM_THREADS", "")
    return min(cores, int(limit)) if limit.isdigit() and int(limit) > 0 else cores


def visible_at(pos, tri, height, width, b, row, col, previous=None, threads=None):
    """(depth, id) of the nearest covering triangle at pixels (b, row, col), as
    oracle.reference.visible_at: depth +inf and id -1 where nothing covers; ``previous``
    ((depth, id) at the same pixels) keeps only triangles ordered after it."""
    lib = load()
    pos = pos.detach().to("cpu", torch.float32)
    if pos.ndim == 2:
        pos = pos[None]
    pos = pos.contiguous()
    stride = 0 if pos.shape[0] == 1 else pos.shape[1] * 4
    tri = tri.detach().to("cpu", torch.int32).contiguous()
    b = b.to(torch.int32)
    if pos.shape[0] == 1:
        b = torch.zeros_like(b)
    # Pixels of one image together, so that blocks share their triangle set-up.
    order = torch.argsort(b, stable=True)
    b, row, col = (t.to(torch.int32)[order].contiguous() for t in (b, row, col))
    n = b.numel()
    depth = torch.empty(n, dtype=torch.float32)
    ids = torch.empty(n, dtype=torch.int64)
    pd = pid = None
    if previous is not None:
        pd = previous[0].to(torch.float32)[order].contiguous()
        pid = previous[1].to(torch.int64)[order].contiguous()
    status = lib.oracle_visible_at(
        pos.data_ptr(), stride, tri.data_ptr(), tri.shape[0], int(height), int(width), n,
        b.data_ptr(), row.data_ptr(), col.data_ptr(),
        None if pd is None else pd.data_ptr(), None if pid is None else pid.data_ptr(),
        depth.data_ptr(), ids.data_ptr(), int(threads or _threads()))
    if status != 0:
        raise ValueError("oracle_visible_at: argument out of range")
    out_depth, out_ids = torch.empty_like(depth), torch.empty_like(ids)
    out_depth[order], out_ids[order] = depth, ids
    return out_depth, out_ids
