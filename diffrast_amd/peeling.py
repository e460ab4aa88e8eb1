"""Depth peeling (reference: peeling.py:1-92).

Each layer is one backend call carrying the previous layer's 64-bit visibility keys. In range
mode all items are peeled together in one launch per layer, rather than one call per item.
"""

from __future__ import annotations

from types import TracebackType

from torch import Tensor

from diffrast_amd.backends import get_backend
from diffrast_amd.context import RasterizeContext
from diffrast_amd.ops import check_rasterize_inputs


class DepthPeeler:
    """Rasterize successive depth layers of the same geometry.

    The first :meth:`rasterize_next_layer` equals :func:`rasterize`; each later call gives, per
    pixel, the nearest triangle behind the previous one, ordered by depth and then by index, so
    triangles at exactly equal depth come in index order. Layers have the format of
    :func:`rasterize` and pass gradients to ``pos``. Arguments are as for :func:`rasterize`,
    including range mode. The peeler copies ``pos``, ``tri`` and ``ranges``, so later edits of
    those tensors do not mix geometries; gradients still reach the ``pos`` passed in. After its
    ``with`` block it raises::

        with dr.DepthPeeler(glctx, pos, tri, (512, 512)) as peeler:
            for _ in range(num_layers):
                rast, rast_db = peeler.rasterize_next_layer()
    """

    def __init__(self, glctx: RasterizeContext, pos: Tensor, tri: Tensor,
                 resolution: tuple[int, int], ranges: Tensor | None = None,
                 grad_db: bool = True) -> None:
        self._resolution = check_rasterize_inputs(glctx, pos, tri, resolution, ranges)
        self._output_db = getattr(glctx, "output_db", True)
        self._grad_db = grad_db and self._output_db
        self._pos, self._tri = pos.clone(), tri.clone()
        self._ranges = ranges.clone() if pos.ndim == 2 else None
        # The per-pixel state belongs to the backend that made it.
        self._backend = get_backend(pos.device, "rasterize")
        self._state = None
        self._closed = False

    def __enter__(self) -> DepthPeeler:
        return self

    def __exit__(self, exc_type: type[BaseException] | None, exc_value: BaseException | None,
                 traceback: TracebackType | None) -> None:
        self._state = None
        self._closed = True

    def rasterize_next_layer(self) -> tuple[Tensor, Tensor]:
        """``(rast, rast_db)`` of the next depth layer."""
        if self._closed:
            raise RuntimeError(
                "This DepthPeeler was closed when its with block exited; create a new one to "
                "rasterize more layers."
            )
        if self._ranges is None:
            rast, rast_db, self._state = self._backend.rasterize_layer(
                self._pos, self._tri, self._resolution, self._grad_db, self._state
            )
        else:
            rast, rast_db, self._state = self._backend.rasterize_ranges(
                self._pos, self._tri, self._resolution, self._grad_db, self._ranges, self._state
            )
        return rast, (rast_db if self._output_db else rast.new_zeros(*rast.shape[:3], 0))
