"""Public differentiable rasterization ops: validation and dispatch (reference: ops.py:1-638).

Each op checks its inputs exactly as the reference does -- same exceptions, same messages, so
code and tests written against the reference see the same behaviour -- and hands the validated,
unexpanded tensors to the backend (``diffrast_amd.backends``). Range mode goes to the backend's
batched ``rasterize_ranges`` in one call instead of one call per item.
"""

from __future__ import annotations

import operator
from collections.abc import Sequence
from typing import Literal, SupportsFloat, get_args

import torch
from torch import Tensor

from diffrast_amd._cache import TensorCache
from diffrast_amd.backends import get_backend
from diffrast_amd.context import RasterizeContext
from diffrast_amd.topology import TopologyHash, neighbours_for

FilterMode = Literal["auto", "nearest", "linear", "linear-mipmap-nearest", "linear-mipmap-linear"]
BoundaryMode = Literal["wrap", "clamp", "zero", "cube"]

FILTER_MODES = get_args(FilterMode)
BOUNDARY_MODES = get_args(BoundaryMode)


def rasterize(glctx: RasterizeContext, pos: Tensor, tri: Tensor, resolution: tuple[int, int],
              ranges: Tensor | None = None, grad_db: bool = True) -> tuple[Tensor, Tensor]:
    """Rasterize triangles into per-pixel barycentrics, depth and triangle ids.

    ``pos`` of shape ``[batch, vertices, 4]`` draws every triangle in every image (instanced
    mode); ``[vertices, 4]`` with ``ranges`` (``(start, count)`` per image, int32 ``[batch,
    2]``) draws ``tri[start : start + count]`` in image ``i`` (range mode). A pixel is covered
    when its centre is inside a triangle; a centre exactly on an edge belongs to the triangle
    whose interior lies towards +x of it (+y for a horizontal edge). Zero-area triangles and
    triangles with a non-finite vertex are not drawn.

    Returns ``(rast, rast_db)``, ``[batch, height, width, 4]`` each: ``(u, v, z / w,
    triangle_id + 1)`` (zeros for background; the id is the row of ``tri`` in both modes) and
    ``(du/dx, du/dy, dv/dx, dv/dy)``. For a context with ``output_db`` false, ``rast_db`` is
    ``[batch, height, width, 0]`` and ``grad_db`` is ignored.
    """
    resolution = check_rasterize_inputs(glctx, pos, tri, resolution, ranges)
    backend = get_backend(pos.device, "rasterize")
    output_db = getattr(glctx, "output_db", True)
    grad_db = grad_db and output_db
    if pos.ndim == 2:
        rast, rast_db, _ = backend.rasterize_ranges(pos, tri, resolution, grad_db, ranges)
    else:
        rast, rast_db = backend.rasterize(pos, tri, resolution, grad_db)
    return rast, (rast_db if output_db else rast.new_zeros(*rast.shape[:3], 0))


def interpolate(attr: Tensor, rast: Tensor, tri: Tensor, rast_db: Tensor | None = None,
                diff_attrs: Sequence[int] | Literal["all"] | None = None
                ) -> tuple[Tensor, Tensor]:
    """Interpolate vertex attributes across the rasterized triangles.

    Args:
        attr: ``[batch, vertices, channels]`` or ``[vertices, channels]`` (shared), float32.
        rast: First output of :func:`rasterize`. Ids past the end of ``tri`` are background.
        tri: int32 ``[triangles, 3]`` indices into ``attr``; the index range is checked once
            per tensor object.
        rast_db: Second output of :func:`rasterize`; required with ``diff_attrs``. An empty
            ``[batch, height, width, 0]`` tensor counts as ``None``.
        diff_attrs: Channels to differentiate in screen space, or ``"all"``.

    Returns:
        ``(out, out_da)``: ``[batch, height, width, channels]`` and ``[batch, height, width,
        2 * len(diff_attrs)]`` with ``(d/dx, d/dy)`` per selected channel.
    """
    shared = isinstance(attr, Tensor) and attr.ndim == 2
    layout = "[batch, vertices, channels] or [vertices, channels]"
    _check(attr, "attr", ndim=2 if shared else 3, dtype=torch.float32, layout=layout)
    _check(rast, "rast", ndim=4, last=4, dtype=torch.float32)
    _check(tri, "tri", ndim=2, last=3, dtype=torch.int32)
    if attr.ndim == 3 and attr.shape[0] not in (1, rast.shape[0]):
        raise ValueError(
            f"attr batch size {attr.shape[0]} does not match rast batch size {rast.shape[0]}."
        )
    _check_devices(attr=attr, rast=rast, tri=tri, rast_db=rast_db)
    channels = _diff_channels(diff_attrs, attr.shape[-1])
    empty = rast_db is not None and rast_db.ndim == 4 and rast_db.shape[-1] == 0
    if rast_db is not None and not empty:
        _check(rast_db, "rast_db", ndim=4, last=4, dtype=torch.float32)
        if rast_db.shape != rast.shape:
            raise ValueError(
                f"rast_db must have the same shape as rast, got {tuple(rast_db.shape)} and "
                f"{tuple(rast.shape)}."
            )
    if not channels:
        rast_db = None
    elif rast_db is None or empty:
        given = ", but the one given is empty" if empty else ""
        raise ValueError(f"rast_db is required when diff_attrs is set{given}.")
    _check_indices(tri, attr.shape[-2])
    return get_backend(rast.device, "interpolate").interpolate(attr, rast, tri, rast_db, channels)


def texture(tex: Tensor, uv: Tensor, uv_da: Tensor | None = None,
            mip_level_bias: Tensor | None = None, mip: MipStack | Sequence[Tensor] | None = None,
            filter_mode: FilterMode = "auto", boundary_mode: BoundaryMode = "wrap",
            max_mip_level: int | None = None) -> Tensor:
    """Sample a 2D texture or a cube map at per-pixel texture coordinates.

    Args:
        tex: ``[batch, tex_height, tex_width, channels]``, or a cube map ``[batch, 6, size,
            size, channels]`` (faces ``+x, -x, +y, -y, +z, -z``, OpenGL orientation). A batch
            of one is shared by all images.
        uv: ``[batch, height, width, 2]``; for a cube map, directions ``[..., 3]``.
        uv_da: Screen-space derivatives ``(du/dx, du/dy, dv/dx, dv/dy)`` (six values, ``(d/dx,
            d/dy)`` per component, for a cube map). Mipmapped filters need it or
            ``mip_level_bias``.
        mip_level_bias: ``[batch, height, width]`` offset of the level of detail.
        mip: Levels 1 and up: a :func:`texture_construct_mip` result or a list of tensors.
        filter_mode: ``"auto"`` picks ``"linear-mipmap-linear"`` when a level of detail is
            given and ``"linear"`` otherwise.
        boundary_mode: ``"wrap"``, ``"clamp"``, ``"zero"``, or ``"cube"`` for a cube map.
        max_mip_level: Coarsest level to use, or ``None`` for all.

    Returns:
        ``[batch, height, width, channels]``; NaN (and no gradient) where coordinates or level
        of detail are undefined, zero for cube directions that select no point.
    """
    if filter_mode not in FILTER_MODES:
        raise ValueError(f"Unknown filter_mode {filter_mode!r}; expected one of {FILTER_MODES}.")
    if boundary_mode not in BOUNDARY_MODES:
        raise ValueError(
            f"Unknown boundary_mode {boundary_mode!r}; expected one of {BOUNDARY_MODES}."
        )
    cube = boundary_mode == "cube"
    _check_texture(tex, "tex", cube, 'boundary_mode="cube"')
    _check(uv, "uv", ndim=4, last=3 if cube else 2, dtype=torch.float32)
    if tex.shape[0] not in (1, uv.shape[0]):
        raise ValueError(
            f"tex batch size {tex.shape[0]} does not match uv batch size {uv.shape[0]}."
        )
    if isinstance(uv_da, Tensor) and uv_da.ndim == 4 and uv_da.shape[-1] == 0:
        uv_da = None
    has_lod = uv_da is not None or mip_level_bias is not None
    if filter_mode == "auto":
        filter_mode = "linear-mipmap-linear" if has_lod else "linear"
    if "mipmap" in filter_mode and not has_lod:
        raise ValueError(f"filter_mode {filter_mode!r} requires uv_da or mip_level_bias.")
    if uv_da is not None:
        _check(uv_da, "uv_da", ndim=4, last=6 if cube else 4, dtype=torch.float32)
        if uv_da.shape[:3] != uv.shape[:3]:
            raise ValueError("uv_da must match uv in batch, height and width.")
    if mip_level_bias is not None:
        _check(mip_level_bias, "mip_level_bias", ndim=3, dtype=torch.float32)
        if mip_level_bias.shape != uv.shape[:3]:
            raise ValueError("mip_level_bias must match uv in batch, height and width.")
    if max_mip_level is not None and max_mip_level < 0:
        raise ValueError(f"max_mip_level must be non-negative, got {max_mip_level}.")
    levels = None if mip is None else _check_mip(mip, tex, cube)
    stacked = isinstance(mip, MipStack) and "mipmap" in filter_mode
    _check_devices(tex=tex, uv=uv, uv_da=uv_da, mip_level_bias=mip_level_bias)
    backend = get_backend(uv.device, "texture")
    return backend.texture(
        tex, uv, uv_da, filter_mode, boundary_mode, max_mip_level,
        mip_level_bias=mip_level_bias, mip=levels,
        packed=mip.pack(tex) if stacked else None,
    )


def texture_construct_mip(tex: Tensor, max_mip_level: int | None = None,
                          cube_mode: bool = False) -> MipStack:
    """Build the mip levels of a texture once, for several :func:`texture` calls.

    Gradients flow through the levels to ``tex`` when it requires them (rebuild the stack
    whenever ``tex`` changes). For a ``tex`` that needs no gradient the stack also keeps the
    packed buffer the kernels sample between calls.

    Args:
        tex: ``[batch, tex_height, tex_width, channels]`` or a cube map.
        max_mip_level: Coarsest level to build, or ``None`` for all.
        cube_mode: Must be true for a cube map.

    Returns:
        An opaque object holding mip levels 1 and up.
    """
    _check_texture(tex, "tex", cube_mode, "cube_mode=True")
    if max_mip_level is not None and max_mip_level < 0:
        raise ValueError(f"max_mip_level must be non-negative, got {max_mip_level}.")
    levels = get_backend(tex.device, "texture").texture_construct_mip(tex, max_mip_level)
    return MipStack(levels, bool(cube_mode), tex.shape)


class MipStack:
    """Mip levels built by :func:`texture_construct_mip`; the contents are private."""

    __slots__ = ("_packed", "cube_mode", "levels", "shape")

    def __init__(self, levels: Sequence[Tensor], cube_mode: bool, shape: Sequence[int]) -> None:
        self.levels = tuple(levels)
        self.cube_mode = cube_mode
        self.shape = tuple(shape)
        self._packed = None

    def pack(self, tex: Tensor):
        """``tex`` and the levels in the one buffer the kernels sample, with its tables.

        Kept for later calls with the same, unmodified tensor while nothing involved takes part
        in autograd (reference ops.py:282-303).
        """
        constant = not (
            tex.requires_grad
            or tex.is_inference()
            or torch.is_inference_mode_enabled()
            or any(level.requires_grad for level in self.levels)
        )
        if constant and self._packed is not None:
            base, version, packed = self._packed
            if base is tex and version == tex._version:
                return packed
        packed = get_backend(tex.device, "texture").pack([tex, *self.levels])
        if constant:
            self._packed = (tex, tex._version, packed)
        return packed


def _check_texture(t: Tensor, name: str, cube: bool, cube_option: str) -> None:
    """Validate a texture or mip level; ``cube_option`` names what selects cube maps."""
    if isinstance(t, Tensor) and t.ndim == 5 and not cube:
        raise ValueError(
            f"{name} has the shape of a cube map, {tuple(t.shape)}, which needs {cube_option}."
        )
    if isinstance(t, Tensor) and t.ndim == 4 and cube:
        raise ValueError(
            f"{cube_option} needs {name} to be a cube map of shape "
            f"[batch, 6, size, size, channels], got {tuple(t.shape)}."
        )
    _check(t, name, ndim=5 if cube else 4, dtype=torch.float32)
    if cube and (t.shape[1] != 6 or t.shape[2] != t.shape[3]):
        raise ValueError(
            f"{name} must have six square faces, [batch, 6, size, size, channels], "
            f"got {tuple(t.shape)}."
        )
    if 0 in t.shape[1:]:
        raise ValueError(
            f"{name} must have at least one texel and one channel, got shape {tuple(t.shape)}."
        )


def _check_mip(mip: MipStack | Sequence[Tensor], tex: Tensor, cube: bool) -> list[Tensor]:
    """Validate ``mip`` against ``tex``; return the tensors of levels 1 and up."""
    if isinstance(mip, MipStack):
        if mip.cube_mode != cube:
            raise ValueError(
                f"mip was constructed with cube_mode={mip.cube_mode}, which does not match "
                f"{'a cube map' if cube else 'a 2D texture'}."
            )
        if mip.shape != tuple(tex.shape):
            raise ValueError(
                f"mip was constructed for a texture of shape {mip.shape}, but tex has shape "
                f"{tuple(tex.shape)}."
            )
        levels = list(mip.levels)
    elif isinstance(mip, Sequence):
        levels = list(mip)
    else:
        raise TypeError(
            "mip must be a list of tensors or the result of texture_construct_mip, "
            f"got {type(mip).__name__}."
        )
    for index, level in enumerate(levels, start=1):
        name = f"mip level {index}"
        _check_texture(level, name, cube, 'boundary_mode="cube"')
        if level.shape[-1] != tex.shape[-1]:
            raise ValueError(f"{name} has {level.shape[-1]} channels but tex has {tex.shape[-1]}.")
        if level.shape[0] not in (1, tex.shape[0]):
            raise ValueError(
                f"{name} has batch size {level.shape[0]}; expected 1 or that of tex, "
                f"{tex.shape[0]}."
            )
        if level.device != tex.device:
            raise ValueError(f"{name} is on {level.device} but tex is on {tex.device}.")
    return levels


def antialias(color: Tensor, rast: Tensor, pos: Tensor, tri: Tensor,
              topology_hash: TopologyHash | None = None,
              pos_gradient_boost: float = 1.0) -> Tensor:
    """Antialias silhouette edges, so that visibility changes give gradients to ``pos``.

    Args:
        color: ``[batch, height, width, channels]`` shaded image.
        rast: First output of :func:`rasterize` for the same geometry.
        pos: ``[batch, vertices, 4]`` or ``[vertices, 4]`` (shared) clip-space positions.
        tri: int32 ``[triangles, 3]``; silhouettes are found from edges shared by index.
        topology_hash: From :func:`antialias_construct_topology_hash`; otherwise the adjacency
            is built on first use and cached per ``tri`` tensor object.
        pos_gradient_boost: Multiplier of the gradient flowing into ``pos``.

    Returns:
        The antialiased image, shaped like ``color``.
    """
    _check(color, "color", ndim=4, dtype=torch.float32)
    _check(rast, "rast", ndim=4, last=4, dtype=torch.float32)
    shared = isinstance(pos, Tensor) and pos.ndim == 2
    layout = "[batch, vertices, 4] or [vertices, 4]"
    _check(pos, "pos", ndim=2 if shared else 3, last=4, dtype=torch.float32, layout=layout)
    _check(tri, "tri", ndim=2, last=3, dtype=torch.int32)
    if color.shape[:3] != rast.shape[:3]:
        raise ValueError(
            "color must match rast in batch, height and width, got "
            f"{tuple(color.shape)} and {tuple(rast.shape)}."
        )
    if not shared and pos.shape[0] != rast.shape[0]:
        raise ValueError(
            f"pos batch size {pos.shape[0]} does not match rast batch size {rast.shape[0]}."
        )
    if not isinstance(pos_gradient_boost, SupportsFloat):
        raise TypeError(f"pos_gradient_boost must be a number, got {pos_gradient_boost!r}.")
    _check_devices(color=color, rast=rast, pos=pos, tri=tri)
    _check_indices(tri, pos.shape[-2])
    # Without triangles there is no adjacency to find, but a topology_hash is still checked.
    neighbours = None
    if topology_hash is not None or tri.shape[0]:
        neighbours = neighbours_for(tri, topology_hash)
    return get_backend(color.device, "antialias").antialias(
        color, rast, pos, tri, float(pos_gradient_boost), neighbours
    )


def antialias_construct_topology_hash(tri: Tensor) -> TopologyHash:
    """Precompute the part of :func:`antialias` that depends only on the index buffer.

    Args:
        tri: int32 ``[triangles, 3]``.

    Returns:
        An opaque object for the ``topology_hash`` argument of :func:`antialias`, valid with
        ``tri`` or any tensor of the same shape and contents on the same device.
    """
    _check(tri, "tri", ndim=2, last=3, dtype=torch.int32)
    return TopologyHash(tri)


def check_rasterize_inputs(glctx: RasterizeContext, pos: Tensor, tri: Tensor,
                           resolution: Sequence[int], ranges: Tensor | None) -> tuple[int, int]:
    """Validate the arguments of :func:`rasterize`; return the resolution as two ints."""
    range_mode = isinstance(pos, Tensor) and pos.ndim == 2
    _check(pos, "pos", ndim=2 if range_mode else 3, last=4, dtype=torch.float32)
    _check(tri, "tri", ndim=2, last=3, dtype=torch.int32)
    # rast stores triangle_id + 1 as float32, exact for integers up to 2**24.
    if tri.shape[0] > 1 << 24:
        raise ValueError(
            f"tri has {tri.shape[0]} triangles, but at most 2**24 = {1 << 24} are supported: "
            "rast stores triangle ids as float32, which is exact only up to there."
        )
    _check_devices(pos=pos, tri=tri)
    _check_indices(tri, pos.shape[-2])
    if pos.device != glctx.device:
        raise ValueError(f"pos is on {pos.device} but the context is on {glctx.device}.")
    if range_mode:
        _check_ranges(ranges, tri.shape[0])
    return _check_resolution(resolution)


def _check_ranges(ranges: Tensor | None, num_tri: int) -> None:
    if ranges is None:
        raise ValueError(
            "ranges is required when pos has shape [vertices, 4] (range mode); give pos a "
            "leading batch dimension to draw all triangles (instanced mode)."
        )
    _check(ranges, "ranges", ndim=2, last=2, dtype=torch.int32)
    for item, (start, count) in enumerate(ranges.tolist()):
        if start < 0 or count < 0 or start + count > num_tri:
            raise ValueError(
                f"ranges[{item}] = (start {start}, count {count}) does not lie within the "
                f"{num_tri} triangles of tri."
            )


def split_ranges(tri: Tensor, ranges: Tensor) -> list[Tensor]:
    """The slice of ``tri`` each image draws in range mode (reference ops.py:482-487)."""
    return [tri[start:start + count] for start, count in ranges.tolist()]


def _check(t: Tensor, name: str, ndim: int, last: int | None = None,
           dtype: torch.dtype | None = None, layout: str | None = None) -> None:
    """Raise unless ``t`` is a tensor with ``ndim`` dimensions, the last of size ``last``."""
    if not isinstance(t, Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(t).__name__}.")
    if t.ndim != ndim or (last is not None and t.shape[-1] != last):
        if layout is None:
            layout = _LAYOUTS.get(name)
            fits = layout is not None and layout.count(",") + 1 == ndim
            if not fits or (last and not layout.endswith(f" {last}]")):
                layout = f"[{', '.join(['...'] * (ndim - 1) + [str(last) if last else '...'])}]"
        hint = ""
        unbatched = t.ndim == ndim - 1 and (last is None or t.shape[-1:] == (last,))
        if unbatched and layout.startswith("[batch") and " or " not in layout:
            hint = f"; add a batch dimension with {name}[None]"
        raise ValueError(f"{name} must have shape {layout}, got {tuple(t.shape)}{hint}.")
    if dtype is not None and t.dtype != dtype:
        cast = {torch.float32: "float", torch.int32: "int"}.get(dtype)
        hint = f"; convert it with {name}.{cast}()" if cast and name.isidentifier() else ""
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}{hint}.")


_LAYOUTS = {
    "pos": "[batch, vertices, 4]",
    "tri": "[triangles, 3]",
    "rast": "[batch, height, width, 4]",
    "rast_db": "[batch, height, width, 4]",
    "color": "[batch, height, width, channels]",
    "tex": "[batch, tex_height, tex_width, channels]",
    "uv": "[batch, height, width, 2]",
    "uv_da": "[batch, height, width, 4]",
    "mip_level_bias": "[batch, height, width]",
}


def _check_devices(**tensors: Tensor | None) -> None:
    devices = {}
    for name, t in tensors.items():
        if t is None:
            continue
        if not isinstance(t, Tensor):
            raise TypeError(f"{name} must be a torch.Tensor, got {type(t).__name__}.")
        devices[name] = t.device
    if len(set(devices.values())) > 1:
        listing = ", ".join(f"{name} on {device}" for name, device in devices.items())
        raise ValueError(f"All inputs must be on the same device; got {listing}.")


def _index_range(tri: Tensor) -> tuple[int, int]:
    low, high = torch.stack(tri.aminmax()).tolist()
    return low, high


_index_ranges: TensorCache[tuple[int, int]] = TensorCache(_index_range)


def _check_indices(tri: Tensor, num_vertices: int, name: str = "tri") -> None:
    """Raise ``ValueError`` if ``tri`` refers to a vertex outside ``[0, num_vertices)``.

    The smallest and largest index take a reduction and a device synchronisation, so they are
    remembered per tensor object until PyTorch records an in-place edit.
    """
    if tri.numel() == 0:
        return
    low, high = _index_ranges.get(tri)
    if low < 0 or high >= num_vertices:
        index = low if low < 0 else high
        valid = "there are no vertices"
        if num_vertices > 0:
            valid = f"valid indices are 0 to {num_vertices - 1} for {num_vertices} vertices"
        raise ValueError(f"{name} refers to vertex {index}, but {valid}.")


def _diff_channels(diff_attrs: Sequence[int] | str | None, num_channels: int) -> list[int]:
    """Channel indices selected by ``diff_attrs``."""
    if diff_attrs is None:
        return []
    expected = (
        f"diff_attrs must be a sequence of channel indices, 'all' or None, got {diff_attrs!r}."
    )
    if isinstance(diff_attrs, str):
        if diff_attrs != "all":
            raise ValueError(expected)
        return list(range(num_channels))
    try:
        channels = [operator.index(c) for c in diff_attrs]
    except TypeError:
        raise TypeError(expected) from None
    if any(c < 0 or c >= num_channels for c in channels):
        raise ValueError(f"diff_attrs {channels} out of range for {num_channels} channels.")
    return channels


def _check_resolution(resolution: Sequence[int]) -> tuple[int, int]:
    """``resolution`` as ``(height, width)``; a list, tuple, tensor or array of two ints."""
    values = resolution.tolist() if hasattr(resolution, "tolist") else resolution
    try:
        if not isinstance(values, (list, tuple)) or any(isinstance(r, bool) for r in values):
            raise TypeError
        height, width = (operator.index(r) for r in values)
    except (TypeError, ValueError):
        raise ValueError(
            f"resolution must be (height, width) as two ints, got {resolution!r}."
        ) from None
    if height <= 0 or width <= 0:
        raise ValueError(f"resolution must be positive, got {resolution!r}.")
    return height, width
