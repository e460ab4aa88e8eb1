"""The C ABI of libdiffrast_hip.so, without a GPU: every symbol declared in
include/diffrast_hip.h is exported, struct layouts agree with the binding, and argument
checks that run before any launch reject bad input."""

import ctypes
import re
from pathlib import Path

import pytest

from diffrast_amd.backends import _lib

HEADER = Path(__file__).resolve().parent.parent / "include" / "diffrast_hip.h"


def declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const char\*|int)\s+(dr_[a-z0-9_]+)\(", text, re.M)))


def test_header_and_binding_agree():
    names = declared()
    assert len(names) >= 19
    assert set(names) == set(_lib.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared():
        assert hasattr(lib, name), name
    assert lib.dr_abi_version() == _lib.ABI_VERSION
    for index, struct in enumerate(_lib.STRUCTS):
        assert lib.dr_struct_size(index) == ctypes.sizeof(struct)
    assert lib.dr_struct_size(9) == -1
    assert lib.dr_error_string(1001).decode().startswith("invalid argument")


def test_argument_checks_before_launch():
    lib = _lib.load()
    g = _lib.RasterGeometry(num_tri=10, batch=1, height=0, width=8, num_instances=10)
    size = ctypes.c_size_t()
    assert lib.dr_raster_workspace_size(ctypes.byref(g), ctypes.byref(size)) == 1001
    g.height = 8
    g.pos = g.tri = 1  # not dereferenced by the size query
    assert lib.dr_raster_workspace_size(ctypes.byref(g), ctypes.byref(size)) == 0
    assert size.value > 10 * 16
    wide = _lib.RasterGeometry(num_tri=1, batch=1, height=8, width=(1 << 20) + 32, pos=1, tri=1,
                               num_instances=1)
    assert lib.dr_raster_workspace_size(ctypes.byref(wide), ctypes.byref(size)) == 1001
    counts = (ctypes.c_uint32 * 4)(0, 0, 0, 0)
    assert lib.dr_raster_visibility_bin(ctypes.byref(g), None, 0, None, counts, None) == 0
    assert lib.dr_raster_visibility_tiles(ctypes.byref(g), None, None, None, 0, None, counts,
                                          None) == 0
    counts[0], counts[1], counts[2] = 3, 5, 1
    assert lib.dr_raster_visibility_bin(ctypes.byref(g), None, 0, None, counts, None) == 1001
    assert lib.dr_raster_visibility_tiles(ctypes.byref(g), None, 1, None, 0, 1, counts,
                                          None) == 1002  # no workspace
    assert lib.dr_edge_hash_workspace_size(-1, ctypes.byref(size)) == 1001
    assert lib.dr_edge_hash_workspace_size(1000, ctypes.byref(size)) == 0
    a = _lib.InterpolateArgs(batch=0, height=4, width=4, channels=3)
    assert lib.dr_interpolate_forward(ctypes.byref(a), 1, None, None) == 0  # nothing to do
    a.num_diff = 2  # derivatives without rast_db
    assert lib.dr_interpolate_forward(ctypes.byref(a), 1, 1, None) == 1001
    t = _lib.TextureArgs(texels=1, uv=1, tex_batch=1, channels=3, num_levels=40, faces=1,
                         batch=1, height=4, width=4)
    assert lib.dr_texture_forward(ctypes.byref(t), 1, None) == 1001
    # Texel indices within an image's packed buffer are 32-bit: 2^32 - 1 texels is too many.
    t.num_levels, t.num_texels = 1, (1 << 32) - 1
    t.level_height[0] = t.level_width[0] = 4
    assert lib.dr_texture_forward(ctypes.byref(t), 1, None) == 1001
    assert lib.dr_texture_backward(ctypes.byref(t), 1, None, None, None, None, None) == 1001
    t.batch = 0  # in range, and nothing to do
    t.num_texels = 16
    assert lib.dr_texture_forward(ctypes.byref(t), 1, None) == 0
    heights = (ctypes.c_int32 * 2)(4, 3)  # 4 halves to 2, not 3
    widths = (ctypes.c_int32 * 2)(4, 2)
    offsets = (ctypes.c_int64 * 2)(0, 16)
    assert lib.dr_mip_build(1, None, 1, 3, 22, 1, 2, heights, widths, offsets, None) == 1001
    with pytest.raises(RuntimeError, match="invalid argument"):
        _lib.check(1001, "probe")
