"""bench.py's unique-byte model against the headline table it follows (icosphere(8) at
8 x 1024^2: 5.45 GB per forward+backward step, 0.681 ms at 8 TB/s), op by op, from the
arguments the backend passes to the C ABI."""

import ctypes
from types import SimpleNamespace

import pytest
import torch

import bench
from diffrast_amd.backends import _lib, hip

B, H, W = 8, 1024, 1024
V, T = 655_362, 1_310_720


def _model():
    tensors = {"pos": torch.empty(B, V, 4, device="meta"),
               "tri": torch.empty(T, 3, dtype=torch.int32, device="meta")}
    return bench.BytesModel(SimpleNamespace(tensors=tensors))


def _geometry():
    return _lib.RasterGeometry(pos=1, pos_batch_stride=V * 4, tri=1, num_tri=T, batch=B,
                               height=H, width=W, num_instances=B * T, num_vertices=V)


def _interp(channels, diff):
    return _lib.InterpolateArgs(attr=1, attr_batch_stride=0, num_vertices=V, channels=channels,
                                rast=1, rast_db=1 if diff else None, tri=1, num_tri=T,
                                batch=B, height=H, width=W, num_diff=diff)


def _texture():
    a = _lib.TextureArgs()
    a.texels, a.tex_batch, a.channels, a.num_texels = 1, 1, 4, 1_398_101
    a.uv, a.uv_da, a.batch, a.height, a.width = 1, 1, B, H, W
    a.boundary = hip.BOUNDARIES["wrap"]
    return a


def _aa():
    return _lib.AntialiasArgs(color=1, channels=4, batch=B, height=H, width=W, rast=1, pos=1,
                              pos_batch_stride=V * 4, tri=1, num_tri=T)


def test_headline_op_bytes():
    m = _model()
    g = ctypes.byref(_geometry())
    levels = (ctypes.c_int32 * 11)(*[1024 >> k for k in range(11)])
    calls = {
        "rast fwd": [("dr_resolve_forward", (g, None, None, 1))],
        "rast bwd": [("dr_resolve_backward", (g, None, None, 1))],
        "interp fwd": [("dr_interpolate_forward", (ctypes.byref(_interp(8, 0)),)),
                       ("dr_interpolate_forward", (ctypes.byref(_interp(2, 2)),))],
        "interp bwd": [("dr_interpolate_backward", (ctypes.byref(_interp(8, 0)),)),
                       ("dr_interpolate_backward", (ctypes.byref(_interp(2, 2)),))],
        "tex fwd": [("dr_texture_forward", (ctypes.byref(_texture()),)),
                    ("dr_mip_build", (None, None, 1, 4, 1_398_101, 1, 11, levels, levels))],
        "tex bwd": [("dr_texture_backward", (ctypes.byref(_texture()),)),
                    ("dr_mip_build_backward", (None, 1, 4, 1_398_101, 1, 11, levels, levels))],
        "aa fwd": [("dr_antialias_forward", (ctypes.byref(_aa()),))],
        "aa bwd": [("dr_antialias_backward", (ctypes.byref(_aa()),))],
    }
    # The per-op figures (MB) of the headline table.
    expected = {"rast fwd": 368.1, "rast bwd": 519.0, "interp fwd": 930.1,
                "interp bwd": 1359.0, "tex fwd": 380.3, "tex bwd": 604.0, "aa fwd": 533.7,
                "aa bwd": 751.8}
    total = 0
    for op, entries in calls.items():
        got = sum(m.op_bytes(name, args) for name, args in entries)
        total += got
        assert got / 1e6 == pytest.approx(expected[op], abs=0.15), op
    assert total / 1e9 == pytest.approx(5.45, abs=0.01)
    assert total / bench.HBM_PEAK * 1e3 == pytest.approx(0.681, abs=0.001)
    # The visibility passes carry no op bytes; the tile pass's kernel bytes are the whole
    # visibility's unique bytes (pos 83.9 MB, tri 15.7 MB, keys 67.1 MB).
    assert m.op_bytes("dr_raster_visibility_tiles", (g, None)) == 0
    assert m.kernel_bytes("dr_raster_visibility_tiles", (g, None)) / 1e6 == pytest.approx(
        166.7, abs=0.1)


def test_every_entry_point_belongs_to_an_op():
    # (a float64 twin belongs where its float32 entry point does)
    compute = {n.removesuffix("_f64") for n in _lib.EXPORTS if n not in (
        "dr_error_string", "dr_abi_version", "dr_struct_size") and "size" not in n}
    assert compute <= set(bench.OP_OF)
