"""The differentiable render ops: rasterize, interpolate, texture, antialias.

The API is the reference's (src/diffrast/ops.py: the same functions, arguments, defaults, output
formats, exception types and messages, so code written for it runs unchanged). Each op checks its
arguments (``_validate``) and hands the checked, unexpanded tensors to the backend that runs on
their device (``diffrast_amd.backends``: the MI355X kernels). Range mode goes to the backend's
batched ``rasterize_ranges`` in one call rather than one call per item.
"""

from __future__ import annotations

from collections.abc import Sequence
from typing import Literal, SupportsFloat, get_args

import torch
from torch import Tensor

from diffrast_amd import _validate as V
from diffrast_amd._cache import TensorCache
from diffrast_amd.backends import get_backend
from diffrast_amd.context import RasterizeContext
from diffrast_amd.topology import TopologyHash, neighbours_for

FilterMode = Literal["auto", "nearest", "linear", "linear-mipmap-nearest", "linear-mipmap-linear"]
BoundaryMode = Literal["wrap", "clamp", "zero", "cube"]

FILTER_MODES = get_args(FilterMode)
BOUNDARY_MODES = get_args(BoundaryMode)

# rast carries triangle_id + 1 in float32, exact for integers up to 2**24.
MAX_TRIANGLES = 1 << 24

# ---- argument checks shared by the ops (also importable under these names) -------------------

_check = V.tensor
_check_devices = V.same_device
_check_resolution = V.resolution
_diff_channels = V.channels


def _index_range(tri: Tensor) -> tuple[int, int]:
    """Smallest and largest index of ``tri`` (one reduction, one device synchronisation)."""
    bounds = torch.stack(tri.aminmax()).cpu()  # one copy to the host
    return int(bounds[0]), int(bounds[1])


# Remembered per index-buffer object until PyTorch records an edit of it.
_index_ranges: TensorCache[tuple[int, int]] = TensorCache(_index_range)


def _check_indices(tri: Tensor, num_vertices: int, name: str = "tri") -> None:
    """``ValueError`` unless every index of ``tri`` is in ``[0, num_vertices)``. The range of an
    index buffer is found once per tensor object (until it is modified in place), whatever it is
    checked against."""
    V.indices_within(tri, num_vertices, name, lambda t: _index_ranges.get(t))


def _empty_derivatives(rast_db) -> bool:
    return isinstance(rast_db, Tensor) and rast_db.ndim == 4 and rast_db.shape[-1] == 0


def _no_db_like(rast: Tensor) -> Tensor:
    return rast.new_zeros(*rast.shape[:3], 0)


# ---- rasterize --------------------------------------------------------------------------------


def check_rasterize_inputs(glctx: RasterizeContext, pos: Tensor, tri: Tensor,
                           resolution: Sequence[int], ranges: Tensor | None) -> tuple[int, int]:
    """Check the arguments of :func:`rasterize` (and of ``DepthPeeler``); return the
    resolution as two ints."""
    range_mode = isinstance(pos, Tensor) and pos.ndim == 2
    _check(pos, "pos", ndim=2 if range_mode else 3, last=4, dtype=torch.float32)
    _check(tri, "tri", ndim=2, last=3, dtype=torch.int32)
    if tri.shape[0] > MAX_TRIANGLES:
        raise ValueError(
            f"tri has {tri.shape[0]} triangles, but at most 2**24 = {MAX_TRIANGLES} are "
            "supported: rast stores triangle ids as float32, which is exact only up to there."
        )
    _check_devices(pos=pos, tri=tri)
    _check_indices(tri, pos.shape[-2])
    if pos.device != glctx.device:
        raise ValueError(f"pos is on {pos.device} but the context is on {glctx.device}.")
    if range_mode:
        V.range_table(ranges, tri.shape[0])
    return _check_resolution(resolution)


def rasterize(glctx: RasterizeContext, pos: Tensor, tri: Tensor, resolution: tuple[int, int],
              ranges: Tensor | None = None, grad_db: bool = True) -> tuple[Tensor, Tensor]:
    """Rasterize triangles into per-pixel barycentrics, depth and triangle ids.

    ``pos`` of shape ``[batch, vertices, 4]`` draws every triangle in every image (instanced
    mode, ``ranges`` ignored); ``[vertices, 4]`` with ``ranges`` (int32 ``[batch, 2]`` of
    ``(start, count)``) draws ``tri[start : start + count]`` in image ``i`` (range mode). A pixel
    is covered when its centre is inside a triangle; a centre exactly on an edge belongs to the
    triangle whose interior lies towards +x of it (+y for a horizontal edge). Zero-area triangles
    and triangles with a non-finite vertex are not drawn. Where triangles overlap the nearest
    wins, and at equal depth the lower index.

    Returns ``(rast, rast_db)``, ``[batch, height, width, 4]`` each: ``(u, v, z / w,
    triangle_id + 1)`` (zeros where nothing is drawn; the id is the row of ``tri`` in both modes)
    and ``(du/dx, du/dy, dv/dx, dv/dy)``. For a context with ``output_db`` false, ``rast_db`` is
    ``[batch, height, width, 0]`` and ``grad_db`` is ignored.
    """
    size = check_rasterize_inputs(glctx, pos, tri, resolution, ranges)
    output_db = getattr(glctx, "output_db", True)
    backend = get_backend(pos.device, "rasterize")
    if pos.ndim == 2:
        rast, rast_db, _ = backend.rasterize_ranges(pos, tri, size, grad_db and output_db,
                                                    ranges)
    else:
        rast, rast_db = backend.rasterize(pos, tri, size, grad_db and output_db)
    return rast, rast_db if output_db else _no_db_like(rast)


# ---- interpolate ------------------------------------------------------------------------------


def interpolate(attr: Tensor, rast: Tensor, tri: Tensor, rast_db: Tensor | None = None,
                diff_attrs: Sequence[int] | Literal["all"] | None = None
                ) -> tuple[Tensor, Tensor]:
    """Interpolate vertex attributes across the rasterized triangles.

    Args:
        attr: ``[batch, vertices, channels]``, or ``[vertices, channels]`` shared by the batch
            (a batch of one is shared too), float32.
        rast: First output of :func:`rasterize`. Ids past the end of ``tri`` are background.
        tri: int32 ``[triangles, 3]`` indices into ``attr``; the index range is checked once per
            tensor object (pass the same tensor to every call).
        rast_db: Second output of :func:`rasterize`, required with ``diff_attrs``; an empty
            ``[batch, height, width, 0]`` tensor counts as ``None``.
        diff_attrs: Channels to differentiate in screen space, or ``"all"``.

    Returns:
        ``(out, out_da)``: ``[batch, height, width, channels]`` and ``[batch, height, width,
        2 * len(diff_attrs)]`` holding ``(d/dx, d/dy)`` of each selected channel in turn (empty
        without ``diff_attrs``).
    """
    shared = isinstance(attr, Tensor) and attr.ndim == 2
    _check(attr, "attr", ndim=2 if shared else 3, dtype=torch.float32,
           layout="[batch, vertices, channels] or [vertices, channels]")
    _check(rast, "rast", ndim=4, last=4, dtype=torch.float32)
    _check(tri, "tri", ndim=2, last=3, dtype=torch.int32)
    if not shared and attr.shape[0] not in (1, rast.shape[0]):
        raise ValueError(
            f"attr batch size {attr.shape[0]} does not match rast batch size {rast.shape[0]}."
        )
    _check_devices(attr=attr, rast=rast, tri=tri, rast_db=rast_db)
    picked = _diff_channels(diff_attrs, attr.shape[-1])
    empty = _empty_derivatives(rast_db)
    if rast_db is not None and not empty:
        _check(rast_db, "rast_db", ndim=4, last=4, dtype=torch.float32)
        if rast_db.shape != rast.shape:
            raise ValueError(
                f"rast_db must have the same shape as rast, got {tuple(rast_db.shape)} and "
                f"{tuple(rast.shape)}."
            )
    if picked and (rast_db is None or empty):
        raise ValueError("rast_db is required when diff_attrs is set"
                         + (", but the one given is empty." if empty else "."))
    _check_indices(tri, attr.shape[-2])
    return get_backend(rast.device, "interpolate").interpolate(
        attr, rast, tri, rast_db if picked else None, picked)


# ---- texture ----------------------------------------------------------------------------------


class MipStack:
    """Mip levels built by :func:`texture_construct_mip`, given to :func:`texture` as ``mip``.
    The contents are private."""

    __slots__ = ("_packed", "cube_mode", "levels", "shape")

    def __init__(self, levels: Sequence[Tensor], cube_mode: bool, shape: Sequence[int]) -> None:
        self.levels = tuple(levels)
        self.cube_mode = cube_mode
        self.shape = tuple(shape)
        self._packed = None  # (tex, its version, packed buffer and tables) while constant

    def _constant(self, tex: Tensor) -> bool:
        """Whether nothing involved takes part in autograd, so a packed buffer may be kept."""
        if tex.requires_grad or tex.is_inference() or torch.is_inference_mode_enabled():
            return False
        return not any(level.requires_grad for level in self.levels)

    def pack(self, tex: Tensor):
        """``tex`` and the levels in the one buffer the kernels sample, with its size tables;
        kept for later calls with the same, unmodified ``tex`` while everything is constant."""
        keep = self._constant(tex)
        if keep and self._packed is not None:
            source, version, packed = self._packed
            if source is tex and version == tex._version:
                return packed
        packed = get_backend(tex.device, "texture").pack([tex, *self.levels])
        self._packed = (tex, tex._version, packed) if keep else None
        return packed


def _mip_tensors(mip, tex: Tensor, cube: bool) -> list[Tensor]:
    if isinstance(mip, MipStack):
        if mip.cube_mode != cube:
            kind = "a cube map" if cube else "a 2D texture"
            raise ValueError(
                f"mip was constructed with cube_mode={mip.cube_mode}, which does not match "
                f"{kind}."
            )
        if mip.shape != tuple(tex.shape):
            raise ValueError(
                f"mip was constructed for a texture of shape {mip.shape}, but tex has shape "
                f"{tuple(tex.shape)}."
            )
        return V.mip_levels(mip.levels, tex, cube)
    if isinstance(mip, Sequence):
        return V.mip_levels(mip, tex, cube)
    raise TypeError(
        "mip must be a list of tensors or the result of texture_construct_mip, got "
        f"{type(mip).__name__}."
    )


def texture(tex: Tensor, uv: Tensor, uv_da: Tensor | None = None,
            mip_level_bias: Tensor | None = None, mip: MipStack | Sequence[Tensor] | None = None,
            filter_mode: FilterMode = "auto", boundary_mode: BoundaryMode = "wrap",
            max_mip_level: int | None = None) -> Tensor:
    """Sample a 2D texture or a cube map at per-pixel coordinates.

    Args:
        tex: ``[batch, tex_height, tex_width, channels]``, or a cube map ``[batch, 6, size,
            size, channels]`` (faces ``+x, -x, +y, -y, +z, -z``, OpenGL orientation); a batch of
            one is shared by all images.
        uv: ``[batch, height, width, 2]`` with ``(0, 0)`` and ``(1, 1)`` the outer corners of
            the first and last texel; for a cube map, directions ``[..., 3]`` (any length).
        uv_da: ``(du/dx, du/dy, dv/dx, dv/dy)`` per pixel (``(d/dx, d/dy)`` of each of the three
            components for a cube map). The mipmapped filters need it or ``mip_level_bias``.
        mip_level_bias: ``[batch, height, width]`` added to the level of detail.
        mip: Levels 1 and up: a :func:`texture_construct_mip` result for this ``tex``, or a list
            of tensors (gradients reach the listed tensors and stop there).
        filter_mode: ``"auto"`` is ``"linear-mipmap-linear"`` with a level of detail and
            ``"linear"`` without.
        boundary_mode: ``"wrap"``, ``"clamp"``, ``"zero"``, or ``"cube"`` (required by, and only
            for, a cube map: filtered across face edges; directions that select no point read 0).
        max_mip_level: Coarsest level to use (``0``: no mipmapping), or ``None`` for all.

    Returns:
        ``[batch, height, width, channels]``; NaN (with no gradient) where a coordinate or the
        level of detail is NaN or leaves no texel to read.
    """
    if filter_mode not in FILTER_MODES:
        raise ValueError(f"Unknown filter_mode {filter_mode!r}; expected one of {FILTER_MODES}.")
    if boundary_mode not in BOUNDARY_MODES:
        raise ValueError(
            f"Unknown boundary_mode {boundary_mode!r}; expected one of {BOUNDARY_MODES}."
        )
    cube = boundary_mode == "cube"
    V.texture_format(tex, "tex", cube, 'boundary_mode="cube"')
    _check(uv, "uv", ndim=4, last=3 if cube else 2, dtype=torch.float32)
    if tex.shape[0] not in (1, uv.shape[0]):
        raise ValueError(
            f"tex batch size {tex.shape[0]} does not match uv batch size {uv.shape[0]}."
        )
    if _empty_derivatives(uv_da):
        uv_da = None
    lod_given = uv_da is not None or mip_level_bias is not None
    if filter_mode == "auto":
        filter_mode = "linear-mipmap-linear" if lod_given else "linear"
    mipmapped = "mipmap" in filter_mode
    if mipmapped and not lod_given:
        raise ValueError(f"filter_mode {filter_mode!r} requires uv_da or mip_level_bias.")
    if uv_da is not None:
        _check(uv_da, "uv_da", ndim=4, last=6 if cube else 4, dtype=torch.float32)
        if uv_da.shape[:3] != uv.shape[:3]:
            raise ValueError("uv_da must match uv in batch, height and width.")
    if mip_level_bias is not None:
        _check(mip_level_bias, "mip_level_bias", ndim=3, dtype=torch.float32)
        if mip_level_bias.shape != uv.shape[:3]:
            raise ValueError("mip_level_bias must match uv in batch, height and width.")
    V.max_level(max_mip_level)
    levels = None if mip is None else _mip_tensors(mip, tex, cube)
    _check_devices(tex=tex, uv=uv, uv_da=uv_da, mip_level_bias=mip_level_bias)
    packed = mip.pack(tex) if isinstance(mip, MipStack) and mipmapped else None
    return get_backend(uv.device, "texture").texture(
        tex, uv, uv_da, filter_mode, boundary_mode, max_mip_level,
        mip_level_bias=mip_level_bias, mip=levels, packed=packed)


def texture_construct_mip(tex: Tensor, max_mip_level: int | None = None,
                          cube_mode: bool = False) -> MipStack:
    """Build the mip levels of ``tex`` once, for several :func:`texture` calls with it.

    Gradients flow through the levels to ``tex`` when it requires them (so rebuild the stack
    when ``tex`` changes). For a ``tex`` that needs no gradient the stack also keeps the packed
    buffer the kernels sample between calls.

    Args:
        tex: ``[batch, tex_height, tex_width, channels]``, or a cube map with ``cube_mode``.
        max_mip_level: Coarsest level to build, or ``None`` for all.
        cube_mode: Must be true for a cube map.
    """
    V.texture_format(tex, "tex", cube_mode, "cube_mode=True")
    V.max_level(max_mip_level)
    levels = get_backend(tex.device, "texture").texture_construct_mip(tex, max_mip_level)
    return MipStack(levels, bool(cube_mode), tex.shape)


# ---- antialias --------------------------------------------------------------------------------


def antialias(color: Tensor, rast: Tensor, pos: Tensor, tri: Tensor,
              topology_hash: TopologyHash | None = None,
              pos_gradient_boost: float = 1.0) -> Tensor:
    """Blend colours across silhouette edges, so that visibility changes give ``pos`` a
    gradient.

    Args:
        color: ``[batch, height, width, channels]`` shaded image.
        rast: First output of :func:`rasterize` for the same geometry.
        pos: ``[batch, vertices, 4]``, or ``[vertices, 4]`` shared by the batch.
        tri: int32 ``[triangles, 3]``; silhouettes come from edges shared by index, so pass
            position-only indices.
        topology_hash: From :func:`antialias_construct_topology_hash`; otherwise the adjacency
            is built on first use and kept per ``tri`` tensor object.
        pos_gradient_boost: Multiplier of the gradient flowing into ``pos``.

    Returns:
        The antialiased image, shaped like ``color``.
    """
    _check(color, "color", ndim=4, dtype=torch.float32)
    _check(rast, "rast", ndim=4, last=4, dtype=torch.float32)
    shared = isinstance(pos, Tensor) and pos.ndim == 2
    _check(pos, "pos", ndim=2 if shared else 3, last=4, dtype=torch.float32,
           layout="[batch, vertices, 4] or [vertices, 4]")
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
    # An empty tri has no adjacency to find, but a topology_hash given with it is still checked.
    neighbours = (neighbours_for(tri, topology_hash)
                  if topology_hash is not None or tri.shape[0] else None)
    return get_backend(color.device, "antialias").antialias(
        color, rast, pos, tri, float(pos_gradient_boost), neighbours)


def antialias_construct_topology_hash(tri: Tensor) -> TopologyHash:
    """The part of :func:`antialias` that depends on the index buffer alone, built now.

    Args:
        tri: int32 ``[triangles, 3]``.

    Returns:
        An opaque object for :func:`antialias`'s ``topology_hash``, valid with ``tri`` or any
        tensor of the same shape and contents on the same device.
    """
    _check(tri, "tri", ndim=2, last=3, dtype=torch.int32)
    return TopologyHash(tri)
