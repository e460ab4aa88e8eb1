"""The allocation-free visibility entry point (dr_raster_visibility_static), through the C ABI:
two calls in a row on one GPU, the second with a smaller geometry, each against the keys of
dr_raster_visibility (caller-allocated workspace and entry buffer), bit for bit; peeling from
the previous layer's keys; and the size limit."""

import ctypes

import pytest
import torch

from diffrast_amd.backends import _lib, hip
from helpers import mixed_mesh, random_mesh

pytestmark = pytest.mark.gpu


def _geometry(pos, tri, res):
    return hip._Geometry(pos, tri, res)


def _keys_allocated(pos, tri, res, prev=None):
    """dr_raster_visibility with a caller-allocated workspace and an entry buffer that fits the
    tile lists (their size from a first, waiting pass)."""
    geo = _geometry(pos, tri, res)
    keys = torch.empty(geo.shape, dtype=torch.int64, device=pos.device)
    size = ctypes.c_size_t()
    _lib.call("dr_raster_workspace_size", _lib.ref(geo.struct), ctypes.byref(size))
    workspace = torch.empty(max(size.value, 1), dtype=torch.uint8, device=pos.device)
    counts = (ctypes.c_uint32 * 4)()
    _lib.call("dr_raster_visibility_begin", _lib.ref(geo.struct), _lib.ptr(prev), _lib.ptr(keys),
              _lib.ptr(workspace), size.value, counts, _lib.stream(pos.device))
    capacity = max(counts[1], 1)
    entries = torch.empty(capacity, dtype=torch.int64, device=pos.device)
    _lib.call("dr_raster_visibility", _lib.ref(geo.struct), _lib.ptr(prev), _lib.ptr(keys),
              _lib.ptr(workspace), size.value, _lib.ptr(entries), capacity, 0, None,
              _lib.stream(pos.device))
    torch.cuda.synchronize()
    return keys, counts[1], size.value


def _keys_static(pos, tri, res, prev=None):
    geo = _geometry(pos, tri, res)
    keys = torch.empty(geo.shape, dtype=torch.int64, device=pos.device)
    _lib.call("dr_raster_visibility_static", _lib.ref(geo.struct), _lib.ptr(prev),
              _lib.ptr(keys), _lib.stream(pos.device))
    torch.cuda.synchronize()
    return keys


def test_two_calls_in_a_row_match_the_allocating_entry_point():
    gen = torch.Generator().manual_seed(21)
    big_pos, big_tri = mixed_mesh(gen, batch=3)
    small_pos, small_tri = random_mesh(300, gen, batch=2)
    cases = [(big_pos, big_tri, (120, 96)), (small_pos, small_tri, (40, 56))]
    for pos, tri, res in cases:
        pos, tri = pos.cuda().contiguous(), tri.cuda().int().contiguous()
        expected, _, _ = _keys_allocated(pos, tri, res)
        got = _keys_static(pos, tri, res)
        assert (expected != -1).any()
        assert torch.equal(got, expected), res
        # The next depth layer, peeled from these keys.
        assert torch.equal(_keys_static(pos, tri, res, got),
                           _keys_allocated(pos, tri, res, got)[0])


def test_tile_lists_beyond_the_buffer_go_through_the_overflow_pass():
    # A workspace that leaves less room for entries than the lists need: 600K instances of
    # large random triangles at 96 x 96 (tens of millions of tile entries).
    gen = torch.Generator().manual_seed(22)
    pos, tri = random_mesh(150_000, gen, batch=4)
    pos, tri = pos.cuda().contiguous(), tri.cuda().int().contiguous()
    res = (96, 96)
    expected, entries, workspace = _keys_allocated(pos, tri, res)
    assert entries > ((64 << 20) - workspace) // 4, "the lists should outgrow the buffer"
    assert torch.equal(_keys_static(pos, tri, res), expected)


def test_geometry_beyond_the_scratch_is_refused():
    gen = torch.Generator().manual_seed(23)
    pos, tri = random_mesh(500_000, gen, batch=2)  # 1M instances at 512^2: a 77 MB workspace
    pos, tri = pos.cuda().contiguous(), tri.cuda().int().contiguous()
    geo = _geometry(pos, tri, (512, 512))
    keys = torch.empty(geo.shape, dtype=torch.int64, device="cuda")
    with pytest.raises(RuntimeError, match="static scratch"):
        _lib.call("dr_raster_visibility_static", _lib.ref(geo.struct), None, _lib.ptr(keys),
                  _lib.stream(pos.device))
