"""Rasterization contexts: which device the ops run on (the reference's src/diffrast/context.py
API: RasterizeContext, its nvdiffrast alias RasterizeCudaContext, and RasterizeGLContext, which
rasterizes exactly like the others and only adds ``output_db``). They hold no GPU state."""

from __future__ import annotations

import operator

import torch


def _gpu_index(device) -> int:
    """A GPU given by number (any integer-like but bool)."""
    if isinstance(device, bool):
        raise TypeError
    return operator.index(device)


def _requested(device) -> torch.device:
    """The device asked for, before checking what this machine has."""
    if device is None:
        return torch.device("cuda" if torch.cuda.is_available() else "cpu")
    if isinstance(device, (torch.device, str)):
        return torch.device(device)
    try:
        index = _gpu_index(device)
    except TypeError:
        raise TypeError(
            f"device must be a torch.device, a string or a GPU index, got {device!r}."
        ) from None
    if index < 0:
        raise ValueError(f"device must not be a negative GPU index, got {device!r}.")
    return torch.device("cuda", index)


def _resolve_device(device) -> torch.device:
    """The device a context runs on: a GPU always with its index, checked to exist."""
    found = _requested(device)
    if found.type != "cuda":
        return found
    if not torch.cuda.is_available():
        raise RuntimeError(
            f"device {str(found)!r} was requested, but no CUDA or ROCm device is available."
        )
    count = torch.cuda.device_count()
    if found.index is None:
        return torch.device("cuda", torch.cuda.current_device())
    if found.index >= count:
        raise ValueError(
            f"device {str(found)!r} does not exist; {count} CUDA or ROCm devices are available."
        )
    return found


class RasterizeContext:
    """Device that :func:`diffrast_amd.rasterize` runs on.

    Args:
        device: A ``torch.device``, a string such as ``"cuda:0"`` or a GPU index. Defaults to
            the current ROCm device, or the CPU when there is none.

    Attributes:
        device: The resolved device, with an explicit index for a GPU.
        output_db: Whether :func:`diffrast_amd.rasterize` returns ``rast_db``; always true here.
    """

    output_db = True

    def __init__(self, device: torch.device | str | int | None = None) -> None:
        self.device = _resolve_device(device)

    def __repr__(self) -> str:
        return f"{type(self).__name__}(device={str(self.device)!r})"


#: nvdiffrast's name for the same context.
RasterizeCudaContext = RasterizeContext


class RasterizeGLContext(RasterizeContext):
    """Stand-in for nvdiffrast's OpenGL context: there is no OpenGL rasterizer, and this
    context rasterizes like :class:`RasterizeContext`.

    Args:
        output_db: With ``False``, :func:`diffrast_amd.rasterize` returns an empty
            ``[batch, height, width, 0]`` tensor in place of ``rast_db``.
        mode: Accepted and ignored.
        device: As for :class:`RasterizeContext`.
    """

    def __init__(self, output_db: bool = True, mode: str = "automatic",
                 device: torch.device | str | int | None = None) -> None:
        # The other contexts take the device first; here a device there would read as true.
        if isinstance(output_db, (str, torch.device)):
            raise TypeError(
                f"output_db must be a bool, got {output_db!r}; pass the device as device=..."
            )
        super().__init__(device)
        self.output_db = bool(output_db)
        self.mode = mode

    def __repr__(self) -> str:
        return f"RasterizeGLContext(output_db={self.output_db}, device={str(self.device)!r})"

    def set_context(self) -> None:
        """Nothing to make current."""

    def release_context(self) -> None:
        """Nothing to release."""
