"""CPU restatement of diffrast's pure-PyTorch reference backend (test infrastructure only).

This module is the oracle the HIP backend is checked against; see ``oracle/__init__.py`` for
who may import it and how each function is pinned. It follows
``src/diffrast/backends/reference.py`` of the reference; every function cites the lines it
restates. Gradients come from autograd, as in the reference.

Visibility (``coverage``, ``inside_edge``, ``visible_triangles``) evaluates exactly the
reference's floating-point operations in the reference's order, each rounded on its own (PyTorch
CPU kernels never fuse a multiply into an add), so that both decide every pixel alike. The HIP
kernels repeat the same sequence with floating-point contraction disabled.
"""

from __future__ import annotations

from collections.abc import Sequence

import torch
import torch.nn.functional as F
from torch import Tensor

# reference.py:24 -- bound on batch * triangles * pixels evaluated per visibility chunk.
CHUNK_ELEMENTS = 1 << 22
# reference.py:27 -- a pixel is not drawn where the area is within this many epsilons.
AREA_TOLERANCE = 2
# reference.py:32 -- edges within this relative margin of 45 degrees go to horizontal pairs.
AXIS_TIE = 1 + 1e-4
# reference.py:35 -- rounding allowance of an edge function, in epsilons of its terms.
EDGE_TIE = 4
# reference.py:402 -- texel footprints saturate here.
FOOTPRINT_LIMIT = 1e18


# --------------------------------------------------------------------------------------------
# Rasterize (reference.py:38-114, 268-397)
# --------------------------------------------------------------------------------------------


def pixel_centres(height: int, width: int, like: Tensor) -> tuple[Tensor, Tensor]:
    """NDC x of each column and y of each row (reference.py:268-271)."""
    cols = torch.arange(width, dtype=like.dtype, device=like.device)
    rows = torch.arange(height, dtype=like.dtype, device=like.device)
    return (cols * 2 + 1) / width - 1, (rows * 2 + 1) / height - 1


def inside_edge(e, ai, ci, wi, aj, cj, wj, positive):
    """Fill-rule test of one edge (reference.py:338-365).

    ``e = ai * cj - aj * ci``; where it is exactly zero the sign of the screen-space gradient
    ``(ci wj - cj wi, aj wi - ai wj)`` decides, x first.
    """
    grad_x = ci * wj - cj * wi
    grad_y = aj * wi - ai * wj
    decided = torch.where(e == 0, torch.where(grad_x == 0, grad_y, grad_x), e)
    return torch.where(positive, decided > 0, decided < 0)


def coverage(x: Sequence[Tensor], y, z, w, px: Tensor, py: Tensor) -> tuple[Tensor, Tensor]:
    """Coverage and depth of triangles at pixel centres (reference.py:293-335).

    ``x``, ``y``, ``z``, ``w`` are triples (one tensor per vertex) that broadcast against
    ``px`` and ``py``. Each operation below is one rounded float operation, in the reference's
    order.
    """
    x0, x1, x2 = x
    y0, y1, y2 = y
    z0, z1, z2 = z
    w0, w1, w2 = w
    a0 = x0 - px * w0
    a1 = x1 - px * w1
    a2 = x2 - px * w2
    c0 = y0 - py * w0
    c1 = y1 - py * w1
    c2 = y2 - py * w2
    e0 = a1 * c2 - a2 * c1
    e1 = a2 * c0 - a0 * c2
    e2 = a0 * c1 - a1 * c0
    area = e0 + e1 + e2
    ew = e0 * w0 + e1 * w1 + e2 * w2
    depth = (e0 * z0 + e1 * z1 + e2 * z2) / ew

    positive = area > 0
    ok = inside_edge(e0, a1, c1, w1, a2, c2, w2, positive)
    ok = ok & inside_edge(e1, a2, c2, w2, a0, c0, w0, positive)
    ok = ok & inside_edge(e2, a0, c0, w0, a1, c1, w1, positive)

    reach_x = torch.maximum(torch.maximum(x0.abs() + w0.abs(), x1.abs() + w1.abs()),
                            x2.abs() + w2.abs())
    reach_y = torch.maximum(torch.maximum(y0.abs() + w0.abs(), y1.abs() + w1.abs()),
                            y2.abs() + w2.abs())
    span_x = a0.abs() + a1.abs() + a2.abs()
    span_y = c0.abs() + c1.abs() + c2.abs()
    eps = torch.finfo(depth.dtype).eps
    ok = ok & (area.abs() > (reach_x * span_y + span_x * (reach_y + span_y)) * (AREA_TOLERANCE * eps))
    ok = ok & torch.where(positive, ew > 0, ew < 0)
    ok = ok & (depth >= -1) & (depth <= 1)
    finite = torch.ones_like(ok)
    for t in (x0, x1, x2, y0, y1, y2, z0, z1, z2, w0, w1, w2):
        finite = finite & t.isfinite()
    return ok & finite, depth


def _corner_values(verts: Tensor):
    """Split ``[..., 3, 4]`` vertices into per-coordinate triples of ``[...]`` tensors."""
    return [tuple(verts[..., k, c] for k in range(3)) for c in range(4)]


def visible_triangles(pos, tri, px, py, previous=None):
    """Nearest covering triangle per pixel by ``(depth, index)`` (reference.py:368-397).

    Returns ``(depth, index)`` of shape ``[batch, height, width]``; index -1 and depth +inf
    where nothing covers the pixel. With ``previous`` only triangles ordered after it count.
    """
    batch, height, width = pos.shape[0], py.shape[0], px.shape[0]
    best_depth = pos.new_full((batch, height, width), torch.inf)
    best_id = torch.full((batch, height, width), -1, dtype=torch.long, device=pos.device)
    step = max(1, CHUNK_ELEMENTS // max(1, batch * height * width))
    pxg, pyg = px.view(1, 1, 1, width), py.view(1, 1, height, 1)
    for start in range(0, tri.shape[0], step):
        idx = tri[start:start + step].long()
        verts = pos[:, idx][:, :, None, None]            # [B, n, 1, 1, 3, 4]
        x, y, z, w = _corner_values(verts)
        ok, depth = coverage(x, y, z, w, pxg, pyg)        # [B, n, H, W]
        if previous is not None:
            prev_depth, prev_id = (t[:, None] for t in previous)
            index = torch.arange(start, start + idx.shape[0]).view(1, -1, 1, 1)
            ok = ok & ((depth > prev_depth) | ((depth == prev_depth) & (index > prev_id)))
        depth = torch.where(ok, depth, torch.inf)
        chunk_depth, chunk_id = depth.min(dim=1)
        nearer = chunk_depth < best_depth
        best_depth = torch.where(nearer, chunk_depth, best_depth)
        best_id = torch.where(nearer, chunk_id + start, best_id)
    return best_depth, best_id


def visible_at(pos, tri, height, width, b, row, col, previous=None):
    """``visible_triangles`` at a list of pixels ``(b, row, col)`` only.

    Every (triangle, pixel) pair goes through the same elementwise arithmetic as the full-grid
    version, so the result is identical at those pixels; this makes brute-force checks of large
    images affordable.
    """
    px, py = pixel_centres(height, width, pos)
    px, py = px[col][None, :], py[row][None, :]            # [1, P]
    best_depth = pos.new_full(b.shape, torch.inf)
    best_id = torch.full(b.shape, -1, dtype=torch.long)
    step = max(1, CHUNK_ELEMENTS // max(1, b.numel()))
    for start in range(0, tri.shape[0], step):
        idx = tri[start:start + step].long()
        verts = pos[b[None, :, None], idx[:, None]]        # [n, P, 3, 4]
        x, y, z, w = _corner_values(verts)
        ok, depth = coverage(x, y, z, w, px, py)
        if previous is not None:
            prev_depth, prev_id = (t[None] for t in previous)
            index = torch.arange(start, start + idx.shape[0]).view(-1, 1)
            ok = ok & ((depth > prev_depth) | ((depth == prev_depth) & (index > prev_id)))
        depth = torch.where(ok, depth, torch.inf)
        chunk_depth, chunk_id = depth.min(dim=0)
        nearer = chunk_depth < best_depth
        best_depth = torch.where(nearer, chunk_depth, best_depth)
        best_id = torch.where(nearer, chunk_id + start, best_id)
    return best_depth, best_id


def edge_functions(x, y, w, px, py):
    """Homogeneous edge functions ``a x c`` stacked last (reference.py:274-278)."""
    a = x - px[..., None] * w
    c = y - py[..., None] * w
    return torch.stack([a[..., 1] * c[..., 2] - a[..., 2] * c[..., 1],
                        a[..., 2] * c[..., 0] - a[..., 0] * c[..., 2],
                        a[..., 0] * c[..., 1] - a[..., 1] * c[..., 0]], -1)


def edge_derivatives(x, y, w, px, py):
    """d/dpx and d/dpy of ``edge_functions``: ``c x w`` and ``w x a`` (reference.py:281-290)."""
    a = x - px[..., None] * w
    c = y - py[..., None] * w

    def cross(u, v):
        return torch.stack([u[..., 1] * v[..., 2] - u[..., 2] * v[..., 1],
                            u[..., 2] * v[..., 0] - u[..., 0] * v[..., 2],
                            u[..., 0] * v[..., 1] - u[..., 1] * v[..., 0]], -1)

    return cross(c, w), cross(w, a)


def rasterize_from_ids(pos, tri, tri_id, grad_db):
    """``rast`` and ``rast_db`` of the given visible triangles (reference.py:69-114)."""
    batch, height, width = tri_id.shape
    px, py = pixel_centres(height, width, pos)
    b_idx, r_idx, c_idx = (tri_id >= 0).nonzero(as_tuple=True)
    ids = tri_id[b_idx, r_idx, c_idx]
    verts = pos[b_idx[:, None], tri.long()[ids]]
    x, y, z, w = verts.unbind(-1)
    cx, cy = px[c_idx], py[r_idx]
    e = edge_functions(x, y, w, cx, cy)
    area = e.sum(-1, keepdim=True)
    bary = e / area
    depth = (bary * z).sum(-1) / (bary * w).sum(-1)
    de_dx, de_dy = edge_derivatives(x, y, w, cx, cy)
    db_dx = (de_dx - bary * de_dx.sum(-1, keepdim=True)) / area
    db_dy = (de_dy - bary * de_dy.sum(-1, keepdim=True)) / area
    if not grad_db:
        db_dx, db_dy = db_dx.detach(), db_dy.detach()
    values = torch.stack([bary[:, 0], bary[:, 1], depth, (ids + 1).to(pos.dtype)], -1)
    derivs = torch.stack([db_dx[:, 0] * (2 / width), db_dy[:, 0] * (2 / height),
                          db_dx[:, 1] * (2 / width), db_dy[:, 1] * (2 / height)], -1)
    where = (b_idx, r_idx, c_idx)
    rast = pos.new_zeros(batch, height, width, 4).index_put(where, values)
    rast_db = pos.new_zeros(batch, height, width, 4).index_put(where, derivs)
    return rast, rast_db


def rasterize_layer(pos, tri, resolution, grad_db, previous):
    """One depth layer and the state for the next (reference.py:45-66)."""
    height, width = resolution
    if tri.shape[0] == 0 or pos.shape[0] == 0:
        empty = pos.new_zeros(pos.shape[0], height, width, 4)
        none = torch.full((pos.shape[0], height, width), -1, dtype=torch.long)
        return empty, empty.clone(), (pos.new_full(none.shape, torch.inf), none)
    px, py = pixel_centres(height, width, pos)
    with torch.no_grad():
        depth, tri_id = visible_triangles(pos, tri, px, py, previous)
    rast, rast_db = rasterize_from_ids(pos, tri, tri_id, grad_db)
    return rast, rast_db, (depth, tri_id)


def rasterize(pos, tri, resolution, grad_db=True):
    """(reference.py:38-42)"""
    rast, rast_db, _ = rasterize_layer(pos, tri, resolution, grad_db, None)
    return rast, rast_db


def rasterize_ranges(pos, tri, resolution, ranges, grad_db=True):
    """Range mode as the reference's ops layer runs it: one call per item, ids shifted by the
    item's start (ops.py:69-74, 482-508)."""
    rasts, dbs = [pos.new_zeros(0, *resolution, 4)], [pos.new_zeros(0, *resolution, 4)]
    for start, count in ranges.tolist():
        rast, rast_db = rasterize(pos[None], tri[start:start + count], resolution, grad_db)
        ids = rast[..., 3:]
        rasts.append(torch.cat([rast[..., :3], torch.where(ids > 0, ids + start, ids)], -1))
        dbs.append(rast_db)
    return torch.cat(rasts), torch.cat(dbs)


# --------------------------------------------------------------------------------------------
# Interpolate (reference.py:117-146)
# --------------------------------------------------------------------------------------------


def interpolate(attr, rast, tri, rast_db, diff_attrs):
    batch, height, width, _ = rast.shape
    channels = attr.shape[-1]
    out = attr.new_zeros(batch, height, width, channels)
    out_da = attr.new_zeros(batch, height, width, 2 * len(diff_attrs))
    if tri.shape[0] == 0:
        return out, out_da
    tri_id = rast[..., 3].round().long() - 1
    where = ((tri_id >= 0) & (tri_id < tri.shape[0])).nonzero(as_tuple=True)
    table = attr[None] if attr.ndim == 2 else attr
    table = table.expand(batch, -1, -1)
    corners = table[where[0][:, None], tri.long()[tri_id[where]]]
    a0, a1, a2 = corners.unbind(-2)
    u = rast[where][:, 0:1]
    v = rast[where][:, 1:2]
    out = out.index_put(where, u * a0 + v * a1 + (1 - u - v) * a2)
    if not diff_attrs:
        return out, out_da
    sel = list(diff_attrs)
    da_du, da_dv = (a0 - a2)[:, sel], (a1 - a2)[:, sel]
    du_dx, du_dy, dv_dx, dv_dy = rast_db[where][:, :, None].unbind(1)
    d_dx = du_dx * da_du + dv_dx * da_dv
    d_dy = du_dy * da_du + dv_dy * da_dv
    return out, out_da.index_put(where, torch.stack([d_dx, d_dy], -1).flatten(-2))


# --------------------------------------------------------------------------------------------
# Texture (reference.py:149-199, 405-672)
# --------------------------------------------------------------------------------------------


def texture(tex, uv, uv_da, filter_mode, boundary_mode, max_mip_level,
            mip_level_bias=None, mip=None, packed=None):
    """(reference.py:149-194)"""
    mipmapped = "mipmap" in filter_mode
    face = valid = None
    if boundary_mode == "cube":
        from oracle import cube

        face, uv, uv_da, valid = cube.project(uv, uv_da if mipmapped else None)
    image = torch.arange(uv.shape[0])[:, None, None]
    if mipmapped:
        texels, heights, widths, offsets = pack_levels(tex, mip, max_mip_level, packed)
        lod = uv.new_zeros(uv.shape[:3])
        if uv_da is not None:
            lod = lod + level_of_detail(uv_da, tex.shape[-3], tex.shape[-2])
        if mip_level_bias is not None:
            lod = lod + mip_level_bias
        out, bad = sample_mipmapped(texels, (heights, widths, offsets), uv, lod,
                                    filter_mode == "linear-mipmap-linear", boundary_mode,
                                    image, face)
    else:
        texels, heights, widths, offsets = pack([tex])
        size = (heights[0], widths[0], offsets[0])
        sampler = sample_nearest if filter_mode == "nearest" else sample_linear
        out, bad = sampler(texels, size, uv, boundary_mode, image, face)
    out = torch.where(bad[..., None], torch.nan, out)
    return out if valid is None else torch.where(valid[..., None], out, 0)


def texture_construct_mip(tex, max_mip_level):
    """(reference.py:197-199)"""
    return mip_chain(tex, max_mip_level)[1:]


def mip_levels(tex, mip, max_mip_level):
    """(reference.py:405-412)"""
    if mip is None:
        return mip_chain(tex, max_mip_level)
    levels = [tex, *mip]
    return levels if max_mip_level is None else levels[:max_mip_level + 1]


def pack_levels(tex, mip, max_mip_level, packed=None):
    """(reference.py:415-430)"""
    if packed is None:
        return pack(mip_levels(tex, mip, max_mip_level))
    texels, *tables = packed
    count = None if max_mip_level is None else max_mip_level + 1
    return (texels, *(t[:count] for t in tables))


def mip_chain(tex, max_mip_level):
    """Halve (rounding up) until 1x1; cube faces one by one (reference.py:433-446)."""
    cube = tex.ndim == 5
    levels = [tex.flatten(0, 1) if cube else tex]
    while max(levels[-1].shape[1:3]) > 1 and (max_mip_level is None
                                              or len(levels) <= max_mip_level):
        levels.append(downsample(levels[-1]))
    if cube:
        levels = [tex, *(level.unflatten(0, tex.shape[:2]) for level in levels[1:])]
    return levels


def downsample(level):
    """Area-weighted halving of ``[batch, h, w, c]`` (reference.py:449-466)."""
    height, width = level.shape[1:3]
    image = level.permute(0, 3, 1, 2)
    kernel = (2 if height % 2 == 0 else 1, 2 if width % 2 == 0 else 1)
    if kernel != (1, 1):
        image = F.avg_pool2d(image, kernel)
    if height > 1 and height % 2 == 1:
        image = halve_odd(image, 2)
    if width > 1 and width % 2 == 1:
        image = halve_odd(image, 3)
    return image.permute(0, 2, 3, 1)


def halve_odd(image, dim):
    """``n`` (odd) texels into ``(n + 1) / 2`` equal bins, three taps each (reference.py:469-488)."""
    n = image.shape[dim]
    m = (n + 1) // 2
    j = torch.arange(m)
    first = j * n // m
    shape = [1] * image.ndim
    shape[dim] = m
    out = 0
    for tap in range(3):
        i = first + tap
        overlap = torch.minimum((j + 1) * n, (i + 1) * m) - torch.maximum(j * n, i * m)
        weight = (overlap.clamp(min=0).to(image.dtype) / n).view(shape)
        out = out + weight * image.index_select(dim, i.clamp(max=n - 1))
    return out


def level_of_detail(uv_da, height, width):
    """``0.5 log2`` of the longer footprint axis in texels (reference.py:491-501)."""
    limit = FOOTPRINT_LIMIT
    du_dx, du_dy, dv_dx, dv_dy = uv_da.unbind(-1)
    len_x = (du_dx * width).clamp(-limit, limit) ** 2 + (dv_dx * height).clamp(-limit, limit) ** 2
    len_y = (du_dy * width).clamp(-limit, limit) ** 2 + (dv_dy * height).clamp(-limit, limit) ** 2
    return 0.5 * torch.log2(torch.maximum(len_x, len_y).clamp_min(1e-30))


def pack(levels):
    """All levels in one ``[tex_batch, texels, channels]`` buffer plus size tables
    (reference.py:504-519)."""
    batch, channels = levels[0].shape[0], levels[0].shape[-1]
    sizes = [[*level.shape[-3:-1], level.shape[1:-1].numel()] for level in levels]
    parts = [level.expand(batch, *level.shape[1:]).reshape(batch, size[2], channels)
             for level, size in zip(levels, sizes)]
    texels = parts[0] if len(parts) == 1 else torch.cat(parts, 1)
    heights, widths, counts = torch.tensor(sizes).unbind(1)
    return texels, heights, widths, counts.cumsum(0) - counts


def sample_mipmapped(texels, sizes, uv, lod, blend, boundary_mode, image, face):
    """(reference.py:522-552)"""
    top = sizes[0].shape[0] - 1
    bad = lod.isnan()
    lod = torch.where(bad, 0, lod).clamp(0, top)
    lower = (lod.detach() + (0.0 if blend else 0.5)).floor().long()
    out, bad_lower = sample_linear(texels, [t[lower] for t in sizes], uv, boundary_mode,
                                   image, face)
    bad = bad | bad_lower
    if blend:
        upper = (lower + 1).clamp(max=top)
        frac = (lod - lower)[..., None]
        above, bad_upper = sample_linear(texels, [t[upper] for t in sizes], uv, boundary_mode,
                                         image, face)
        out = out * (1 - frac) + above * frac
        bad = bad | bad_upper
    return out, bad


def sample_nearest(texels, size, uv, boundary_mode, image, face=None):
    """(reference.py:555-573)"""
    height, width, _ = size
    x, bad_x = texel_coordinate(uv[..., 0], width, 0.0, boundary_mode)
    y, bad_y = texel_coordinate(uv[..., 1], height, 0.0, boundary_mode)
    col, row = x.detach().floor().long(), y.detach().floor().long()
    mode = "clamp" if boundary_mode == "cube" else boundary_mode
    return fetch(texels, size, image, row, col, mode, face), bad_x | bad_y


def sample_linear(texels, size, uv, boundary_mode, image, face=None):
    """(reference.py:576-612)"""
    height, width, _ = size
    x, bad_x = texel_coordinate(uv[..., 0], width, 0.5, boundary_mode)
    y, bad_y = texel_coordinate(uv[..., 1], height, 0.5, boundary_mode)
    x0, y0 = x.floor().detach(), y.floor().detach()
    fx, fy = (x - x0)[..., None], (y - y0)[..., None]
    col, row = x0.long(), y0.long()
    rows = torch.stack([row, row, row + 1, row + 1], -1)
    cols = torch.stack([col, col + 1, col, col + 1], -1)
    per_tap = [t[..., None] for t in size]
    tap_face = None if face is None else face[..., None]
    taps = fetch(texels, per_tap, image[..., None], rows, cols, boundary_mode, tap_face)
    t00, t01, t10, t11 = taps.unbind(-2)
    out = (1 - fy) * ((1 - fx) * t00 + fx * t01) + fy * ((1 - fx) * t10 + fx * t11)
    if boundary_mode == "cube":
        left, right = (col < 0)[..., None], (col + 1 >= width)[..., None]
        above, below = (row < 0)[..., None], (row + 1 >= height)[..., None]
        missing = (1 - fy) * ((1 - fx) * (left & above) + fx * (right & above)) + fy * (
            (1 - fx) * (left & below) + fx * (right & below))
        out = out + missing * taps.sum(-2) / 3
    return out, bad_x | bad_y


def texel_coordinate(coord, size, shift, boundary_mode):
    """(reference.py:615-633)"""
    if boundary_mode == "wrap":
        coord = coord - coord.detach().floor()
    x = coord * size - shift
    if boundary_mode in ("clamp", "zero"):
        x = x.clamp(min=-1).clamp(max=size)
    bad = ~torch.isfinite(x)
    return torch.where(bad, 0, x), bad


def fetch(texels, size, image, row, col, boundary_mode, face=None):
    """(reference.py:636-672)"""
    height, width, offset = size
    valid = None
    if boundary_mode == "cube":
        from oracle import cube

        face, row, col, valid = cube.fold(face, row, col, width)
    elif boundary_mode == "wrap":
        row, col = row % height, col % width
    else:
        if boundary_mode == "zero":
            valid = (row >= 0) & (row < height) & (col >= 0) & (col < width)
        row = row.clamp(min=0).clamp(max=height - 1)
        col = col.clamp(min=0).clamp(max=width - 1)
    if face is not None:
        row = row + face * height
    index = offset + row * width + col
    if texels.shape[0] > 1:
        index = index + image * texels.shape[1]
    out = texels.reshape(-1, texels.shape[-1])[index]
    return out if valid is None else out * valid[..., None]


# --------------------------------------------------------------------------------------------
# Antialias (reference.py:202-265, 675-814)
# --------------------------------------------------------------------------------------------


def antialias(color, rast, pos, tri, pos_gradient_boost=1.0, neighbours=None):
    """(reference.py:202-265)"""
    if tri.shape[0] == 0:
        return color.clone()
    batch, height, width = rast.shape[:3]
    tri = tri.long()
    if pos.ndim == 2:
        pos = pos[None]
    tri_id = rast[..., 3].detach().round().long() - 1
    tri_id = torch.where(tri_id < tri.shape[0], tri_id, -1)
    depth = rast[..., 2].detach()
    with torch.no_grad():
        silhouette = silhouette_edges(pos, tri, neighbours).expand(batch, -1, -1)
    pos = pos.expand(batch, -1, -1)
    px, py = pixel_centres(height, width, pos)
    out = color
    for d_row, d_col in ((0, 1), (1, 0)):
        id_p = tri_id[:, :height - d_row, :width - d_col]
        id_q = tri_id[:, d_row:, d_col:]
        b, row, col = (id_p != id_q).nonzero(as_tuple=True)
        row_q, col_q = row + d_row, col + d_col
        common = (pos, tri, silhouette, b, d_col == 1, width, height)
        from_p, t_p = edge_crossing(*common, id_p[b, row, col], px[col], py[row], px[col_q],
                                    py[row_q])
        from_q, t_q = edge_crossing(*common, id_q[b, row, col], px[col_q], py[row_q], px[col],
                                    py[row])
        use_p = from_p & (~from_q | (depth[b, row, col] <= depth[b, row_q, col_q]))
        use_q = from_q & ~use_p
        t = torch.where(use_p, t_p, 1 - t_q)
        t = t.detach() + pos_gradient_boost * (t - t.detach())
        active = (use_p | use_q)[:, None]
        c_p, c_q = color[b, row, col], color[b, row_q, col_q]
        delta_p = torch.where(active & (t < 0.5)[:, None], (0.5 - t)[:, None] * (c_q - c_p), 0.0)
        delta_q = torch.where(active & (t >= 0.5)[:, None], (t - 0.5)[:, None] * (c_p - c_q), 0.0)
        out = out.index_put((b, row, col), delta_p, accumulate=True)
        out = out.index_put((b, row_q, col_q), delta_q, accumulate=True)
    return out.contiguous()


def edge_crossing(pos, tri, silhouette, b, horizontal, width, height, tri_id, src_x, src_y,
                  dst_x, dst_y):
    """Exit of the triangle at ``src`` towards ``dst`` (reference.py:675-727)."""
    count = tri_id.shape[0]
    covered = (tri_id >= 0).nonzero().squeeze(1)
    b, tri_id = b[covered], tri_id[covered]
    src_x, src_y, dst_x, dst_y = (t[covered] for t in (src_x, src_y, dst_x, dst_y))
    x, y, _, w = pos[b[:, None], tri[tri_id]].unbind(-1)
    e_src = edge_functions(x, y, w, src_x, src_y)
    e_dst = edge_functions(x, y, w, dst_x, dst_y)
    sign = torch.where(e_src.sum(-1, keepdim=True) < 0, -1.0, 1.0)
    span = e_src - e_dst
    with torch.no_grad():
        slack = edge_slack(x, y, w, dst_x, dst_y)
        crossed = (e_dst * sign <= slack) & (span * sign > 2 * slack)
    t_edge = torch.where(crossed, e_src / torch.where(crossed, span, 1.0), torch.inf)
    t, edge = t_edge.min(-1)
    with torch.no_grad():
        found = crossed.any(-1) & silhouette[b, tri_id, edge] & along_axis(
            x, y, w, edge, horizontal, width, height)
    all_found = found.new_zeros(count).index_put((covered,), found)
    all_t = t.new_zeros(count).index_put((covered,), torch.where(found, t, 0.0))
    return all_found, all_t


def edge_slack(x, y, w, px, py):
    """Rounding bound of ``edge_functions`` at ``(px, py)`` (reference.py:730-746)."""
    a, c = x - px[..., None] * w, y - py[..., None] * w
    reach_x, reach_y = x.abs() + w.abs(), y.abs() + w.abs()
    i, j = [1, 2, 0], [2, 0, 1]
    terms = ((reach_x[:, i] + a[:, i].abs()) * c[:, j].abs()
             + (reach_x[:, j] + a[:, j].abs()) * c[:, i].abs()
             + reach_y[:, j] * a[:, i].abs()
             + reach_y[:, i] * a[:, j].abs())
    return terms * (EDGE_TIE * torch.finfo(x.dtype).eps)


def along_axis(x, y, w, edge, horizontal, width, height):
    """Whether pairs along this axis handle ``edge`` (reference.py:749-765)."""
    i, j = ((edge + 1) % 3)[:, None], ((edge + 2) % 3)[:, None]
    xi, yi, wi = (v.gather(-1, i).squeeze(-1) for v in (x, y, w))
    xj, yj, wj = (v.gather(-1, j).squeeze(-1) for v in (x, y, w))
    steep = (wj * yi - wi * yj).abs() * height * AXIS_TIE
    flat = (xj * wi - xi * wj).abs() * width
    return steep >= flat if horizontal else flat > steep


def edge_neighbours(tri):
    """Partner edge ``3 * t + k`` of each edge, or -1 (reference.py:768-787)."""
    tri = tri.long()
    start, end = tri[:, [1, 2, 0]].flatten(), tri[:, [2, 0, 1]].flatten()
    key = (torch.minimum(start, end) << 32) | torch.maximum(start, end)
    _, inverse, counts = torch.unique(key, return_inverse=True, return_counts=True)
    order = torch.argsort(inverse, stable=True)
    first = (counts.cumsum(0) - counts)[(counts == 2).nonzero().squeeze(1)]
    partner = torch.full_like(key, -1)
    partner[order[first]] = order[first + 1]
    partner[order[first + 1]] = order[first]
    return partner.view(-1, 3)


def silhouette_edges(pos, tri, neighbours=None):
    """Silhouette flag per ``[batch, triangle, edge]`` (reference.py:790-814)."""
    num_tri = tri.shape[0]
    partner = (edge_neighbours(tri) if neighbours is None else neighbours).flatten()
    start, end = tri[:, [1, 2, 0]].flatten(), tri[:, [2, 0, 1]].flatten()
    xyw = pos[..., [0, 1, 3]]
    line = torch.linalg.cross(xyw[:, start], xyw[:, end], dim=-1)

    def side(vertex):
        p = xyw[:, vertex]
        return torch.sign((line * p).sum(-1) * p[..., 2])

    opposite = tri.flatten()
    shared = partner >= 0
    fold = side(opposite) * side(opposite[partner.clamp(min=0)]) > 0
    return (~shared | fold).view(-1, num_tri, 3)
