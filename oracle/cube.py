"""CPU restatement of diffrast's cube-map geometry (test infrastructure only).

Follows ``src/diffrast/backends/_cube.py`` of the reference. Faces are ``+x, -x, +y, -y, +z,
-z`` oriented as in OpenGL: for a direction with major axis ``ma`` the face coordinates are
``s = (sc / |ma| + 1) / 2`` and ``t = (tc / |ma| + 1) / 2`` with (sc, tc) per face
``(-rz, -ry), (+rz, -ry), (+rx, +rz), (+rx, -rz), (+rx, -ry), (-rx, -ry)`` (_cube.py:7-16).
"""

from __future__ import annotations

import torch
from torch import Tensor

# _cube.py:31-33 -- per face: the major axis and the directions in which s and t grow.
MAJOR = ((1, 0, 0), (-1, 0, 0), (0, 1, 0), (0, -1, 0), (0, 0, 1), (0, 0, -1))
S_AXIS = ((0, 0, -1), (0, 0, 1), (1, 0, 0), (1, 0, 0), (1, 0, 0), (-1, 0, 0))
T_AXIS = ((0, -1, 0), (0, -1, 0), (0, 0, 1), (0, 0, -1), (0, -1, 0), (0, -1, 0))
# _cube.py:36 -- direction derivatives saturate at this multiple of the direction's length.
DERIVATIVE_LIMIT = 1e18


def _tables(dtype):
    return tuple(torch.tensor(t, dtype=dtype) for t in (MAJOR, S_AXIS, T_AXIS))


def project(dirs: Tensor, dirs_da: Tensor | None = None):
    """Face, face coordinates, their derivatives and validity (_cube.py:44-102)."""
    valid = torch.isfinite(dirs).all(-1) & (
        dirs.detach().abs().amax(-1) >= torch.finfo(dirs.dtype).tiny)
    dirs = torch.where(valid[..., None], dirs, dirs.new_tensor((0.0, 0.0, 1.0)))
    ax, ay, az = dirs.detach().abs().unbind(-1)
    x_major = (ax >= ay) & (ax >= az)
    y_major = ~x_major & (ay >= az)
    axis = 2 - 2 * x_major.long() - y_major.long()
    negative = dirs.detach().gather(-1, axis[..., None]).squeeze(-1) < 0
    face = 2 * axis + negative.long()

    length = dirs.detach().abs().amax(-1, keepdim=True)
    dirs = dirs / length
    major, s_axis, t_axis = (table[face] for table in _tables(dirs.dtype))
    ma = (dirs * major).sum(-1, keepdim=True)
    ratio = torch.stack([(dirs * s_axis).sum(-1), (dirs * t_axis).sum(-1)], -1) / ma
    st = 0.5 * (ratio + 1)
    if dirs_da is None:
        return face, st, None, valid
    undefined = valid & dirs_da.isnan().any(-1)
    da = torch.where((valid & ~undefined)[..., None], dirs_da, 0) / length
    da = da.clamp(-DERIVATIVE_LIMIT, DERIVATIVE_LIMIT).unflatten(-1, (3, 2))
    d_ma = (da * major[..., None]).sum(-2)
    d_sc = (da * s_axis[..., None]).sum(-2)
    d_tc = (da * t_axis[..., None]).sum(-2)
    ds = 0.5 * (d_sc - ratio[..., :1] * d_ma) / ma
    dt = 0.5 * (d_tc - ratio[..., 1:] * d_ma) / ma
    st_da = torch.where(undefined[..., None], torch.nan, torch.cat([ds, dt], -1))
    return face, st, st_da, valid


def fold(face: Tensor, row: Tensor, col: Tensor, size: Tensor):
    """Move texels one step outside a face onto the neighbouring face (_cube.py:105-143).

    In half-texel units texel centres are integer points on the cube ``[-size, size]^3``; a
    centre past an edge is clamped onto the cube and pulled one step back along the old major
    axis, then re-projected. Beyond a corner ``exists`` is false.
    """
    major, s_axis, t_axis = (table[face] for table in _tables(torch.long))
    over_col = (col < 0) | (col >= size)
    over_row = (row < 0) | (row >= size)
    extent = size[..., None]
    sc = (2 * col + 1 - size)[..., None]
    tc = (2 * row + 1 - size)[..., None]
    point = (extent * major + sc * s_axis + tc * t_axis).clamp(-extent, extent)
    point = point - (over_col | over_row)[..., None] * major
    axis = point.abs().argmax(-1)
    negative = point.gather(-1, axis[..., None]).squeeze(-1) < 0
    face = 2 * axis + negative.long()
    _, s_axis, t_axis = (table[face] for table in _tables(torch.long))
    col = ((point * s_axis).sum(-1) + size - 1) // 2
    row = ((point * t_axis).sum(-1) + size - 1) // 2
    return face, row.clamp(min=0), col.clamp(min=0), ~(over_col & over_row)
