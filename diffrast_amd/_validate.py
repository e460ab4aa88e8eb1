"""Argument checks of the public API and the messages they raise.

The exception types and message texts are the reference's (src/diffrast/ops.py), which user code
and tests match on; the checks are organised here around named layouts: an argument's usual
shape is declared once as text such as ``"[batch, vertices, 4]"``, and that text is what a shape
error shows (with ``...`` placeholders where the usual layout does not describe the shape asked
for).
"""

from __future__ import annotations

import operator
from collections.abc import Callable, Sequence

import torch
from torch import Tensor


class Layout:
    """A shape described by dimension names, e.g. ``[batch, height, width, 4]``."""

    __slots__ = ("text", "ndim", "last")

    def __init__(self, text: str) -> None:
        self.text = text
        names = [d.strip() for d in text.strip("[]").split(",")]
        self.ndim = len(names)
        self.last = int(names[-1]) if names[-1].isdigit() else None

    @staticmethod
    def placeholder(ndim: int, last: int | None) -> str:
        return "[" + ", ".join(["..."] * (ndim - 1) + [str(last) if last else "..."]) + "]"


USUAL = {name: Layout(text) for name, text in {
    "pos": "[batch, vertices, 4]",
    "tri": "[triangles, 3]",
    "rast": "[batch, height, width, 4]",
    "rast_db": "[batch, height, width, 4]",
    "color": "[batch, height, width, channels]",
    "tex": "[batch, tex_height, tex_width, channels]",
    "uv": "[batch, height, width, 2]",
    "uv_da": "[batch, height, width, 4]",
    "mip_level_bias": "[batch, height, width]",
}.items()}

_CASTS = {torch.float32: "float", torch.int32: "int"}


def _shape_text(name: str, ndim: int, last: int | None, layout: str | None) -> str:
    if layout is not None:
        return layout
    usual = USUAL.get(name)
    if usual is None or usual.ndim != ndim or (last and usual.last != last):
        return Layout.placeholder(ndim, last)
    return usual.text


def tensor(t, name: str, ndim: int, last: int | None = None, dtype: torch.dtype | None = None,
           layout: str | None = None) -> None:
    """A tensor of ``ndim`` dimensions (the last of size ``last``) and type ``dtype``.

    ``layout`` names the dimensions for the message; by default the argument's usual layout,
    when it has one that fits."""
    if not isinstance(t, Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(t).__name__}.")
    if t.ndim != ndim or (last is not None and t.shape[-1] != last):
        text = _shape_text(name, ndim, last, layout)
        batchless = t.ndim == ndim - 1 and (last is None or t.shape[-1:] == (last,))
        hint = ""
        if batchless and text.startswith("[batch") and " or " not in text:
            hint = f"; add a batch dimension with {name}[None]"
        raise ValueError(f"{name} must have shape {text}, got {tuple(t.shape)}{hint}.")
    if dtype is not None and t.dtype != dtype:
        cast = _CASTS.get(dtype)
        hint = f"; convert it with {name}.{cast}()" if cast and name.isidentifier() else ""
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}{hint}.")


def same_device(**named: Tensor | None) -> None:
    """Every given tensor on one device (``None`` entries are skipped)."""
    seen: dict[str, torch.device] = {}
    for name, t in named.items():
        if t is None:
            continue
        if not isinstance(t, Tensor):
            raise TypeError(f"{name} must be a torch.Tensor, got {type(t).__name__}.")
        seen[name] = t.device
    if len(set(seen.values())) > 1:
        where = ", ".join(f"{name} on {device}" for name, device in seen.items())
        raise ValueError(f"All inputs must be on the same device; got {where}.")


def indices_within(tri: Tensor, num_vertices: int, name: str,
                   bounds: Callable[[Tensor], tuple[int, int]]) -> None:
    """Every index of ``tri`` in ``[0, num_vertices)``; ``bounds`` gives its (min, max)."""
    if tri.numel() == 0:
        return
    low, high = bounds(tri)
    if low >= 0 and high < num_vertices:
        return
    index = low if low < 0 else high
    if num_vertices > 0:
        valid = f"valid indices are 0 to {num_vertices - 1} for {num_vertices} vertices"
    else:
        valid = "there are no vertices"
    raise ValueError(f"{name} refers to vertex {index}, but {valid}.")


def resolution(value) -> tuple[int, int]:
    """``(height, width)`` as two positive ints, from a list, tuple, tensor or array of two
    integers (no bools; sets, mappings and iterators are refused: their order is not the
    caller's, or reading them consumes them)."""
    items = value.tolist() if hasattr(value, "tolist") else value

    def refuse():
        return ValueError(f"resolution must be (height, width) as two ints, got {value!r}.")

    if not isinstance(items, (list, tuple)) or len(items) != 2:
        raise refuse()
    try:
        if any(isinstance(v, bool) for v in items):
            raise TypeError
        height, width = (operator.index(v) for v in items)
    except TypeError:
        raise refuse() from None
    if min(height, width) <= 0:
        raise ValueError(f"resolution must be positive, got {value!r}.")
    return height, width


def channels(diff_attrs, count: int) -> list[int]:
    """The channel indices ``diff_attrs`` selects out of ``count`` (``"all"``, a sequence of
    integers, or ``None`` for none)."""
    if diff_attrs is None:
        return []
    wrong = f"diff_attrs must be a sequence of channel indices, 'all' or None, got {diff_attrs!r}."
    if isinstance(diff_attrs, str):
        if diff_attrs == "all":
            return list(range(count))
        raise ValueError(wrong)
    try:
        picked = [operator.index(c) for c in diff_attrs]
    except TypeError:
        raise TypeError(wrong) from None
    if not all(0 <= c < count for c in picked):
        raise ValueError(f"diff_attrs {picked} out of range for {count} channels.")
    return picked


def range_table(ranges, num_tri: int) -> None:
    """The ``ranges`` of range mode: int32 ``[batch, 2]`` of (start, count) inside ``tri``."""
    if ranges is None:
        raise ValueError(
            "ranges is required when pos has shape [vertices, 4] (range mode); give pos a "
            "leading batch dimension to draw all triangles (instanced mode)."
        )
    tensor(ranges, "ranges", ndim=2, last=2, dtype=torch.int32)
    for item, (start, count) in enumerate(ranges.tolist()):
        if not (start >= 0 and count >= 0 and start + count <= num_tri):
            raise ValueError(
                f"ranges[{item}] = (start {start}, count {count}) does not lie within the "
                f"{num_tri} triangles of tri."
            )


_CUBE_LAYOUT = "[batch, 6, size, size, channels]"


def texture_format(t, name: str, cube: bool, cube_option: str) -> None:
    """A 2D texture ``[batch, h, w, channels]`` or, with ``cube``, a cube map of six square
    faces; ``cube_option`` is how the caller asks for a cube map (named in messages)."""
    if isinstance(t, Tensor) and t.ndim == 5 and not cube:
        raise ValueError(
            f"{name} has the shape of a cube map, {tuple(t.shape)}, which needs {cube_option}."
        )
    if isinstance(t, Tensor) and t.ndim == 4 and cube:
        raise ValueError(
            f"{cube_option} needs {name} to be a cube map of shape {_CUBE_LAYOUT}, got "
            f"{tuple(t.shape)}."
        )
    tensor(t, name, ndim=5 if cube else 4, dtype=torch.float32)
    if cube and not (t.shape[1] == 6 and t.shape[2] == t.shape[3]):
        raise ValueError(
            f"{name} must have six square faces, {_CUBE_LAYOUT}, got {tuple(t.shape)}."
        )
    if 0 in t.shape[1:]:
        raise ValueError(
            f"{name} must have at least one texel and one channel, got shape {tuple(t.shape)}."
        )


def mip_levels(levels: Sequence[Tensor], tex: Tensor, cube: bool) -> list[Tensor]:
    """Mip levels 1 and up given as tensors: each a texture of ``tex``'s kind and channels,
    with a batch of one or ``tex``'s, on ``tex``'s device."""
    checked = list(levels)
    for number, level in enumerate(checked, start=1):
        name = f"mip level {number}"
        texture_format(level, name, cube, 'boundary_mode="cube"')
        if level.shape[-1] != tex.shape[-1]:
            raise ValueError(f"{name} has {level.shape[-1]} channels but tex has {tex.shape[-1]}.")
        if level.shape[0] not in (1, tex.shape[0]):
            raise ValueError(
                f"{name} has batch size {level.shape[0]}; expected 1 or that of tex, "
                f"{tex.shape[0]}."
            )
        if level.device != tex.device:
            raise ValueError(f"{name} is on {level.device} but tex is on {tex.device}.")
    return checked


def max_level(value: int | None) -> None:
    if value is not None and value < 0:
        raise ValueError(f"max_mip_level must be non-negative, got {value}.")
