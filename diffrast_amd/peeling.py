"""Depth peeling (the reference's src/diffrast/peeling.py API: ``DepthPeeler``).

A layer is one backend call that carries the previous layer's per-pixel state -- here the 64-bit
visibility keys -- and keeps keys strictly behind it. Range mode peels every item of the batch in
the same call.
"""

from __future__ import annotations

import weakref
from types import TracebackType

from torch import Tensor

from diffrast_amd.backends import get_backend
from diffrast_amd.context import RasterizeContext
from diffrast_amd.ops import check_rasterize_inputs

_CLOSED = ("This DepthPeeler was closed when its with block exited; create a new one to "
           "rasterize more layers.")


class DepthPeeler:
    """Successive depth layers of one geometry, nearest first.

    The first :meth:`rasterize_next_layer` is :func:`diffrast_amd.rasterize`'s result; each
    later one holds, per pixel, the nearest triangle behind the previous layer's, in order of
    depth and then of triangle index (equal depths come in index order), and stays empty where
    none is left. Layers have :func:`diffrast_amd.rasterize`'s format and pass gradients back to
    ``pos``. The arguments are :func:`diffrast_amd.rasterize`'s, range mode included. The peeler
    works on copies of ``pos``, ``tri`` and ``ranges`` taken when it is made, so later edits of
    those tensors do not reach it (gradients still reach the ``pos`` given). Used as a context
    manager, it refuses further layers after its block::

        with dr.DepthPeeler(glctx, pos, tri, (512, 512)) as peeler:
            for _ in range(num_layers):
                rast, rast_db = peeler.rasterize_next_layer()
    """

    def __init__(self, glctx: RasterizeContext, pos: Tensor, tri: Tensor,
                 resolution: tuple[int, int], ranges: Tensor | None = None,
                 grad_db: bool = True) -> None:
        self._resolution = check_rasterize_inputs(glctx, pos, tri, resolution, ranges)
        self._output_db = getattr(glctx, "output_db", True)
        self._grad_db = bool(grad_db) and self._output_db
        self._geometry = (pos.clone(), tri.clone(), ranges.clone() if pos.ndim == 2 else None)
        # The per-pixel state belongs to the backend that made it: the backend is fixed now.
        self._backend = get_backend(pos.device, "rasterize")
        self._state = None
        self._open = True
        # A backend that keeps per-tri state (the HIP backend's processing order of a large
        # mesh) may let the copy of tri use what it keeps for tri, and, once the first layer
        # has made it for the copy, give it back to tri while tri still holds the same values.
        self._share = getattr(self._backend, "share_order", None)
        self._source = None
        if self._share is not None and not tri.is_inference():
            if not self._share(tri, self._geometry[1]):
                self._source = (weakref.ref(tri), tri._version, tri.data_ptr())

    def __enter__(self) -> DepthPeeler:
        return self

    def __exit__(self, exc_type: type[BaseException] | None, exc_value: BaseException | None,
                 traceback: TracebackType | None) -> None:
        self._open = False
        self._state = None

    def rasterize_next_layer(self) -> tuple[Tensor, Tensor]:
        """``(rast, rast_db)`` of the next layer."""
        if not self._open:
            raise RuntimeError(_CLOSED)
        pos, tri, ranges = self._geometry
        if ranges is None:
            rast, rast_db, state = self._backend.rasterize_layer(
                pos, tri, self._resolution, self._grad_db, self._state)
        else:
            rast, rast_db, state = self._backend.rasterize_ranges(
                pos, tri, self._resolution, self._grad_db, ranges, self._state)
        self._state = state
        if self._source is not None:
            source, version, address = self._source
            self._source = None
            original = source()
            if original is not None and original._version == version and \
                    original.data_ptr() == address:
                self._share(tri, original)
        if not self._output_db:
            rast_db = rast.new_zeros(*rast.shape[:3], 0)
        return rast, rast_db
