"""Edge adjacency of a mesh for antialias (reference: topology.py:1-72).

Built once per index buffer on the GPU (a hash table keyed on each edge's vertex pair; see
``csrc/antialias.hip``), either explicitly through ``antialias_construct_topology_hash`` or
through a cache keyed on the ``tri`` tensor object.
"""

from __future__ import annotations

import weakref

from torch import Tensor

from diffrast_amd._cache import TensorCache, stamp
from diffrast_amd.backends import get_backend


def _neighbours(tri: Tensor) -> Tensor:
    return get_backend(tri.device, "antialias").edge_neighbours(tri)


class TopologyHash:
    """Edge adjacency of an index buffer, from ``antialias_construct_topology_hash``.

    The contents are an implementation detail. Pass it to :func:`antialias` with the ``tri`` it
    was built from, or a tensor of the same contents.
    """

    def __init__(self, tri: Tensor) -> None:
        self._neighbours = _neighbours(tri)
        self._shape = tuple(tri.shape)
        self._device = tri.device
        self._source: weakref.ref[Tensor] | None = weakref.ref(tri)
        self._stamp = stamp(tri)

    def __repr__(self) -> str:
        return f"TopologyHash(triangles={self._shape[0]}, device={str(self._device)!r})"

    def __getstate__(self) -> dict:
        # Copies and pickles keep the adjacency but not the link to the source tensor, which
        # only serves to notice in-place edits.
        return {**self.__dict__, "_source": None, "_stamp": None}

    def neighbours(self, tri: Tensor) -> Tensor:
        """The adjacency, int32 ``[triangles, 3]``, if it can belong to ``tri``."""
        if tuple(tri.shape) != self._shape or tri.device != self._device:
            raise ValueError(
                f"topology_hash was built for a tri of shape {self._shape} on {self._device}, "
                f"got shape {tuple(tri.shape)} on {tri.device}."
            )
        if self._source is not None and self._source() is tri and stamp(tri) != self._stamp:
            raise ValueError(
                "tri was modified in place after topology_hash was built from it; build a new "
                "one with antialias_construct_topology_hash."
            )
        return self._neighbours


# An entry is as large as its index buffer, so only a few are kept.
_neighbour_cache: TensorCache[Tensor] = TensorCache(_neighbours, max_entries=16)


def neighbours_for(tri: Tensor, topology_hash: TopologyHash | None) -> Tensor:
    """Adjacency of ``tri``: from ``topology_hash`` if given, else from the cache."""
    if topology_hash is None:
        return _neighbour_cache.get(tri)
    if not isinstance(topology_hash, TopologyHash):
        raise TypeError(
            "topology_hash must come from antialias_construct_topology_hash, got "
            f"{type(topology_hash).__name__}."
        )
    return topology_hash.neighbours(tri)
